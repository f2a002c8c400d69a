"""The attention seam (reference: src/attention.py:84-91, `attention(q, k, v)`).

Same signature and offset-causal semantics (query i of q_len sits at absolute
total_k - q_len + i and sees keys at positions <= that; attention.py:43-51), computed
by the HIP verify-attention kernel.  The reference selects torch SDPA or a Triton
kernel with LOLLM_ATTN; this build has one path, so LOLLM_ATTN is not consulted.
"""

from __future__ import annotations

import torch

from . import ops


def attention(q, k, v):
    """q (B, H, q_len, D), k / v (B, H, total_k, D), bf16 -> (B, H, q_len, D)."""
    B, H, ql, D = q.shape
    tk = k.shape[2]
    if tk < ql:
        raise ValueError("total_k must be >= q_len")
    qq = q.transpose(1, 2).contiguous().to(torch.bfloat16)            # (B, q_len, H, D)
    kc = k.contiguous().to(torch.bfloat16)
    vc = v.contiguous().to(torch.bfloat16)
    kv_len = torch.full((B,), tk, dtype=torch.int32, device=q.device)
    o = ops.attn_verify(qq, kc, vc, kv_len, None)                      # (B, q_len, H*D)
    return o.view(B, ql, H, D).transpose(1, 2).to(q.dtype)
