"""A local safetensors checkpoint -> the MI355X model and MTP head.

Reads a directory laid out like a Hugging Face snapshot -- `config.json` plus the
`*.safetensors` shards (the hf branch of src/loader.py:79-86, without the hub download
and the tokenizer) -- and hands the tensors to the strict family loaders: `load`
(the name map and shape checks of src/qwen3_5/weights.py:27-70) and `load_mtp`
(src/qwen3_5/mtp.py:171-189).  Tensors are read shard by shard on the host, popped
as they are moved to the device, and anything a loader does not consume is reported.
"""

from __future__ import annotations

import glob
import json
import os

from safetensors import safe_open

from .mtp import load_mtp
from .weights import load


def read_checkpoint(path: str):
    """(raw_config, weights): config.json and every tensor of the *.safetensors shards,
    keyed by checkpoint name, on the host in their stored dtype."""
    cfg_path = os.path.join(path, "config.json")
    if not os.path.isfile(cfg_path):
        raise FileNotFoundError(f"no config.json in {path}")
    with open(cfg_path) as f:
        raw_config = json.load(f)
    shards = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    if not shards:
        raise FileNotFoundError(f"no *.safetensors shards in {path}")
    weights = {}
    for shard in shards:
        with safe_open(shard, framework="pt", device="cpu") as f:
            for name in f.keys():
                if name in weights:
                    raise RuntimeError(f"tensor {name} appears in more than one shard")
                weights[name] = f.get_tensor(name)
    return raw_config, weights


def load_checkpoint(path: str, device="cuda", with_mtp=True, progress=None):
    """(model, mtp or None, unused tensor names).  The MTP head is built when asked for
    and the checkpoint carries `mtp.*` tensors; a missing or mis-shaped tensor raises
    (hard-fail, as the reference's loaders do)."""
    raw_config, weights = read_checkpoint(path)
    if raw_config.get("model_type") is None:
        raise ValueError("config.json has no 'model_type'; cannot route to a family")
    model = load(raw_config, weights, "hf", device=device, progress=progress)
    mtp = None
    if with_mtp and any(k.startswith("mtp.") for k in weights):
        mtp = load_mtp(model, weights, "hf", device=device)
    return model, mtp, sorted(weights)
