"""Checkpoint name map and strict streaming load (mirrors src/qwen3_5/weights.py:27-70).

`to_raw` maps the family's module names to checkpoint names (`model.` ->
`model.language_model.`; `lm_head.weight` stays top level and is absent when tied).
`load(raw_config, weights, fmt, device, dtype, progress)` pops every expected tensor
from `weights`, checks its shape, moves it to the device in `dtype` (bf16 by default)
and builds the MI355X model; a missing tensor or a shape mismatch raises, as in the
reference.  lm_head is tied to the embedding when the checkpoint has none.
"""

from __future__ import annotations

import torch

from .config import build_config
from .modeling_qwen3_5 import Qwen3_5Model
from .random_init import weight_shapes


def to_raw(canonical: str, fmt: str):
    if fmt == "hf":
        if canonical.startswith("model."):
            return "model.language_model." + canonical[len("model."):]
        return canonical
    raise NotImplementedError(f"qwen3_5 has no tensor-name map for the {fmt!r} format "
                              "(hf safetensors checkpoints only)")


def to_canonical(raw: str) -> str:
    if raw.startswith("model.language_model."):
        return "model." + raw[len("model.language_model."):]
    return raw


def take_weights(cfg, weights: dict, names, device, dtype, progress=None, who="qwen3_5"):
    """Pop, shape-check and move the named (raw name -> shape) tensors."""
    out = {}
    items = list(names.items())
    for i, (raw, (shape, _)) in enumerate(items):
        if progress is not None:
            progress(i, len(items))
        if raw not in weights:
            raise RuntimeError(f"{who}: missing tensor {raw}")
        t = weights.pop(raw)
        if tuple(t.shape) != tuple(shape):
            raise RuntimeError(f"{who}: shape mismatch {raw}: {tuple(t.shape)} vs {tuple(shape)}")
        out[to_canonical(raw)] = t.to(device=device, dtype=dtype)
    if progress is not None:
        progress(len(items), len(items))
    return out


def load(raw_config: dict, weights: dict, fmt: str, device="cuda", dtype=None,
         progress=None) -> Qwen3_5Model:
    cfg = build_config(raw_config, fmt)
    dev = torch.device(device)
    if dev.type != "cuda":
        raise RuntimeError("lollm_amd runs on the HIP device only (no CPU path)")
    dtype = dtype or torch.bfloat16
    if dtype != torch.bfloat16:
        raise NotImplementedError("lollm_amd kernels run the model in bf16")
    names = {k: v for k, v in weight_shapes(cfg, with_mtp=False).items() if k != "lm_head.weight"}
    tied = to_raw("lm_head.weight", fmt) not in weights
    if not tied:
        names[to_raw("lm_head.weight", fmt)] = ((cfg.vocab_size, cfg.hidden_size), "lin")
    W = take_weights(cfg, weights, names, dev, dtype, progress)
    if tied:
        W["lm_head.weight"] = W["model.embed_tokens.weight"]
    return Qwen3_5Model(cfg, W, dev)
