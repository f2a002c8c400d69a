"""Local safetensors checkpoints (lollm_amd/qwen3_5/checkpoint.py): config.json plus
shards read back tensor for tensor (the hf branch of src/loader.py:79-86), loaded
through the strict name map (src/qwen3_5/weights.py:27-70, mtp.py:171-189).  The
GPU cases build the model from the directory and compare it with the model built from
the same tensors in memory; a mis-shaped or missing tensor must raise."""

import json
import os

import pytest
import torch
from safetensors.torch import save_file

from lollm_amd.qwen3_5.checkpoint import load_checkpoint, read_checkpoint
from lollm_amd.qwen3_5.config import Qwen3_5Config, micro_config_dict
from lollm_amd.qwen3_5.random_init import random_weights


def write_checkpoint(path, raw, weights, shards=2):
    os.makedirs(path, exist_ok=True)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(raw, f)
    names = sorted(weights)
    for i in range(shards):
        part = {n: weights[n].contiguous() for n in names[i::shards]}
        save_file(part, os.path.join(path, f"model-{i + 1:05d}-of-{shards:05d}.safetensors"))


def micro_weights(seed=0):
    raw = micro_config_dict()
    W = random_weights(Qwen3_5Config.from_hf(raw), seed=seed)
    return raw, {k: v.to(torch.bfloat16) for k, v in W.items()}


def test_read_checkpoint_round_trip(tmp_path):
    raw, W = micro_weights()
    write_checkpoint(str(tmp_path), raw, W, shards=3)
    raw2, W2 = read_checkpoint(str(tmp_path))
    assert raw2 == raw
    assert sorted(W2) == sorted(W)
    for k in W:
        assert W2[k].dtype == torch.bfloat16 and torch.equal(W2[k], W[k]), k


def test_read_checkpoint_rejects_bad_directories(tmp_path):
    with pytest.raises(FileNotFoundError):
        read_checkpoint(str(tmp_path))                       # no config.json
    raw, W = micro_weights()
    with open(os.path.join(tmp_path, "config.json"), "w") as f:
        json.dump(raw, f)
    with pytest.raises(FileNotFoundError):
        read_checkpoint(str(tmp_path))                       # no shards
    name = sorted(W)[0]
    save_file({name: W[name]}, os.path.join(tmp_path, "a.safetensors"))
    save_file({name: W[name]}, os.path.join(tmp_path, "b.safetensors"))
    with pytest.raises(RuntimeError):
        read_checkpoint(str(tmp_path))                       # a tensor in two shards


@pytest.mark.gpu
def test_load_checkpoint_equals_in_memory_load(tmp_path):
    from lollm_amd.qwen3_5 import load, load_mtp
    raw, W = micro_weights(seed=3)
    write_checkpoint(str(tmp_path), raw, W)
    model, mtp, unused = load_checkpoint(str(tmp_path))
    assert mtp is not None and unused == []
    ref = load(raw, dict(W), "hf", device="cuda")
    ids = torch.randint(0, raw["vocab_size"], (2, 7), generator=torch.Generator().manual_seed(1))
    a, _ = model(ids.cuda(), model.new_cache(2, 32))
    b, _ = ref(ids.cuda(), ref.new_cache(2, 32))
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.gpu
def test_load_checkpoint_rejects_mis_shaped_and_missing(tmp_path):
    raw, W = micro_weights(seed=4)
    bad = dict(W)
    name = "model.language_model.layers.0.mlp.down_proj.weight"
    bad[name] = bad[name][:, :-8].contiguous()
    write_checkpoint(str(tmp_path / "shape"), raw, bad)
    with pytest.raises(RuntimeError, match="shape mismatch"):
        load_checkpoint(str(tmp_path / "shape"))
    miss = dict(W)
    del miss["model.language_model.norm.weight"]
    write_checkpoint(str(tmp_path / "miss"), raw, miss)
    with pytest.raises(RuntimeError, match="missing tensor"):
        load_checkpoint(str(tmp_path / "miss"))
