"""Writes the golden fixtures under tests/golden/ (run once in the build container).

Sources (none of them is the product or the oracle):
  * transformers 5.15.0 `models/qwen3_5/modeling_qwen3_5.py` -- the same Gated
    DeltaNet / gated attention lineage as the reference: `torch_recurrent_gated_delta_rule`,
    `torch_chunk_gated_delta_rule`, `l2norm`, `Qwen3_5RMSNormGated`, and the whole
    `Qwen3_5ForCausalLM` (prefill + cached decode + a 2-token cached chunk) built from a
    local config on the seeded random weights of `lollm_amd.qwen3_5.random_init`.
  * rocRAND's `rocrand_philox4x32_10.h` (Philox4x32-10 rounds), compiled here as a
    host program by `philox_kat.cpp`.

Usage:  python tests/golden/make_golden.py
Outputs: gdn_fns.safetensors, model_micro.safetensors, philox_kat.json
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
import tempfile

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from lollm_amd.qwen3_5.config import Qwen3_5Config, micro_config_dict  # noqa: E402
from lollm_amd.qwen3_5.random_init import random_weights  # noqa: E402


def gdn_functions():
    from transformers.models.qwen3_5 import modeling_qwen3_5 as M
    g = torch.Generator().manual_seed(11)
    out = {}
    B, T, H, D = 2, 7, 4, 32
    for tag, l2 in (("l2", True), ("raw", False)):
        q = torch.randn(B, T, H, D, generator=g)
        k = torch.randn(B, T, H, D, generator=g)
        if not l2:
            q = q / q.norm(dim=-1, keepdim=True)
            k = k / k.norm(dim=-1, keepdim=True)
        v = torch.randn(B, T, H, D, generator=g)
        beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
        gg = -torch.nn.functional.softplus(torch.randn(B, T, H, generator=g))
        s0 = torch.randn(B, H, D, D, generator=g) * 0.1
        o_r, s_r = M.torch_recurrent_gated_delta_rule(q, k, v, gg, beta, s0, True,
                                                      use_qk_l2norm_in_kernel=l2)
        o_c, s_c = M.torch_chunk_gated_delta_rule(q, k, v, gg, beta, chunk_size=4,
                                                  initial_state=s0, output_final_state=True,
                                                  use_qk_l2norm_in_kernel=l2)
        for n, t in dict(q=q, k=k, v=v, beta=beta, g=gg, s0=s0, o_rec=o_r, s_rec=s_r,
                         o_chunk=o_c, s_chunk=s_c).items():
            out[f"{tag}.{n}"] = t.contiguous()
    x = torch.randn(5, 64, generator=g)
    out["l2norm.x"] = x
    out["l2norm.y"] = M.l2norm(x)
    norm = M.Qwen3_5RMSNormGated(64, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.1 * torch.randn(64, generator=g))
        z = torch.randn(5, 64, generator=g)
        out["gnorm.x"], out["gnorm.z"], out["gnorm.w"] = x.clone(), z, norm.weight.detach().clone()
        out["gnorm.y"] = norm(x, z)
    save_file(out, os.path.join(HERE, "gdn_fns.safetensors"))


def model_micro():
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM
    raw = micro_config_dict()
    cfg = Qwen3_5Config.from_hf(raw)
    tc = Qwen3_5TextConfig(
        vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size,
        intermediate_size=cfg.intermediate_size, num_hidden_layers=cfg.num_hidden_layers,
        num_attention_heads=cfg.num_attention_heads,
        num_key_value_heads=cfg.num_key_value_heads, head_dim=cfg.head_dim,
        rms_norm_eps=cfg.rms_norm_eps,
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                         "partial_rotary_factor": cfg.partial_rotary_factor},
        tie_word_embeddings=True, hidden_act="silu", layer_types=cfg.layer_types,
        linear_num_key_heads=cfg.linear_num_key_heads,
        linear_num_value_heads=cfg.linear_num_value_heads,
        linear_key_head_dim=cfg.linear_key_head_dim,
        linear_value_head_dim=cfg.linear_value_head_dim,
        linear_conv_kernel_dim=cfg.linear_conv_kernel_dim, max_position_embeddings=4096)
    W = random_weights(cfg, seed=0, with_mtp=False)
    model = Qwen3_5ForCausalLM(tc).eval()
    sd = {}
    for name, t in W.items():
        sd[name.replace("model.language_model.", "model.")] = t
    missing, unexpected = model.load_state_dict(sd, strict=False)
    missing = [m for m in missing if m != "lm_head.weight"]
    assert not missing and not unexpected, (missing, unexpected)
    model.tie_weights()
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg.vocab_size, (2, 9), generator=g)
    steps = torch.randint(0, cfg.vocab_size, (2, 5), generator=g)
    with torch.no_grad():
        o = model(input_ids=prompt, use_cache=True)
        past = o.past_key_values
        res = {"prompt": prompt, "steps": steps, "logits_prefill": o.logits}
        for i in range(3):                     # three single-token cached decodes
            o = model(input_ids=steps[:, i:i + 1], past_key_values=past, use_cache=True)
            past = o.past_key_values
            res[f"logits_decode{i}"] = o.logits
        o = model(input_ids=steps[:, 3:5], past_key_values=past, use_cache=True)
        res["logits_chunk2"] = o.logits          # a 2-token cached chunk (verify shape)
        full = torch.cat([prompt, steps], 1)
        res["logits_full"] = model(input_ids=full, use_cache=False).logits
    save_file({k: v.contiguous() for k, v in res.items()},
              os.path.join(HERE, "model_micro.safetensors"))


def philox_kat():
    src = os.path.join(HERE, "philox_kat.cpp")
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "kat")
        subprocess.check_call(["hipcc", "-O1", "-x", "hip", "--offload-arch=gfx950", src,
                               "-o", exe])
        txt = subprocess.check_output([exe]).decode()
    cases = json.loads(txt)
    with open(os.path.join(HERE, "philox_kat.json"), "w") as f:
        json.dump({"source": "rocRAND rocrand_philox4x32_10.h ten_rounds (ROCm 7.2)",
                   "cases": cases}, f, indent=1)


if __name__ == "__main__":
    torch.manual_seed(0)
    gdn_functions()
    model_micro()
    philox_kat()
    print("golden fixtures written to", HERE)
