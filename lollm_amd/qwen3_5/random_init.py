"""Seeded random-init weights in the checkpoint's own tensor names.

The synthetic workloads have no real checkpoint, so weights are drawn from a seeded
generator and returned as the *raw* (checkpoint-named) dict that `weights.load` and
`mtp.load_mtp` consume -- the same `model.language_model.*` / `mtp.*` /
`lm_head.weight` naming the reference maps (src/qwen3_5/weights.py:27-37,
src/qwen3_5/mtp.py:165-168).  Shapes follow src/qwen3_5/blocks.py:196-342 and
src/qwen3_5/mtp.py:44-54.

Scales: linear weights and embeddings N(0, 0.02); "(1 + w)" RMSNorm weights
N(0, 0.1) so the +1 convention is exercised; gated-norm weights 1 + N(0, 0.1);
depthwise conv N(0, 0.3); A_log = log U(0.1, 2); dt_bias N(0, 0.5).
Tensors are generated in sorted-name order from one generator, so the dict is a
pure function of (config, seed, device).
"""

from __future__ import annotations

import torch

from .config import Qwen3_5Config


def _layer_shapes(cfg: Qwen3_5Config, prefix: str, layer_type: str) -> dict:
    H, D = cfg.hidden_size, cfg.head_dim
    s = {
        prefix + "input_layernorm.weight": ((H,), "norm1"),
        prefix + "post_attention_layernorm.weight": ((H,), "norm1"),
        prefix + "mlp.gate_proj.weight": ((cfg.intermediate_size, H), "lin"),
        prefix + "mlp.up_proj.weight": ((cfg.intermediate_size, H), "lin"),
        prefix + "mlp.down_proj.weight": ((H, cfg.intermediate_size), "lin"),
    }
    if layer_type == "full_attention":
        a = prefix + "self_attn."
        s.update({
            a + "q_proj.weight": ((cfg.num_attention_heads * D * 2, H), "lin"),
            a + "k_proj.weight": ((cfg.num_key_value_heads * D, H), "lin"),
            a + "v_proj.weight": ((cfg.num_key_value_heads * D, H), "lin"),
            a + "o_proj.weight": ((H, cfg.num_attention_heads * D), "lin"),
            a + "q_norm.weight": ((D,), "norm1"),
            a + "k_norm.weight": ((D,), "norm1"),
        })
    else:
        g = prefix + "linear_attn."
        s.update({
            g + "in_proj_qkv.weight": ((cfg.conv_dim, H), "lin"),
            g + "in_proj_z.weight": ((cfg.value_dim, H), "lin"),
            g + "in_proj_b.weight": ((cfg.linear_num_value_heads, H), "lin"),
            g + "in_proj_a.weight": ((cfg.linear_num_value_heads, H), "lin"),
            g + "conv1d.weight": ((cfg.conv_dim, 1, cfg.linear_conv_kernel_dim), "conv"),
            g + "dt_bias": ((cfg.linear_num_value_heads,), "dt"),
            g + "A_log": ((cfg.linear_num_value_heads,), "alog"),
            g + "norm.weight": ((cfg.linear_value_head_dim,), "gnorm"),
            g + "out_proj.weight": ((H, cfg.value_dim), "lin"),
        })
    return s


def weight_shapes(cfg: Qwen3_5Config, with_mtp: bool = True) -> dict:
    """Raw checkpoint name -> (shape, init kind)."""
    H, V = cfg.hidden_size, cfg.vocab_size
    s = {"model.language_model.embed_tokens.weight": ((V, H), "lin"),
         "model.language_model.norm.weight": ((H,), "norm1")}
    if not cfg.tie_word_embeddings:
        s["lm_head.weight"] = ((V, H), "lin")
    for i in range(cfg.num_hidden_layers):
        s.update(_layer_shapes(cfg, f"model.language_model.layers.{i}.", cfg.layer_type(i)))
    if with_mtp:
        s.update({
            "mtp.pre_fc_norm_embedding.weight": ((H,), "norm1"),
            "mtp.pre_fc_norm_hidden.weight": ((H,), "norm1"),
            "mtp.fc.weight": ((H, 2 * H), "lin"),
            "mtp.norm.weight": ((H,), "norm1"),
        })
        s.update(_layer_shapes(cfg, "mtp.layers.0.", "full_attention"))
    return s


@torch.no_grad()
def random_weights(cfg: Qwen3_5Config, seed: int, dtype=torch.float32, device="cpu",
                   with_mtp: bool = True) -> dict:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out = {}
    for name, (shape, kind) in sorted(weight_shapes(cfg, with_mtp).items()):
        if kind == "alog":
            t = torch.rand(shape, generator=gen, device=device) * 1.9 + 0.1
            t = t.log()
        else:
            t = torch.randn(shape, generator=gen, device=device)
            if kind == "lin":
                t = t * 0.02
            elif kind == "norm1":
                t = t * 0.1
            elif kind == "gnorm":
                t = 1.0 + t * 0.1
            elif kind == "conv":
                t = t * 0.3
            elif kind == "dt":
                t = t * 0.5
        out[name] = t.to(dtype)
    return out
