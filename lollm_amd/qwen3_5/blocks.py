"""Qwen3.5 decoder blocks on the MI355X kernels.

Each block keeps the reference block's parameters (src/qwen3_5/blocks.py:186-342) but
stores them the way the verify step consumes them: projections that read the same
input are concatenated into one GEMM weight (GDN in_proj_qkv|z|b|a, attention
q|k|v, MLP gate|up), so a layer issues 4 GEMMs plus fused HIP kernels for everything
between them.  A GEMM over at most 64 rows (the verify and draft passes) streams a
tiled copy of its weight through lollm_gemm, with SiLU(gate) * up fused into the
gate|up GEMM; longer calls (the prefill) use hipBLASLt on the row-major weight.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import ops
from .config import Qwen3_5Config


def _cat_rows(*ws):
    return torch.cat([w.reshape(w.shape[0], -1) for w in ws], 0).contiguous()


# Fixed GEMM path and grid per projection shape, so a given (weights, inputs) gives the
# same bits in every process (a timing-based choice could differ between runs and
# change rounding).  Rows <= 64 take lollm_gemm, rows > 64 (the prefill) hipBLASLt.
# lollm_gemm deals 64-column groups x 128-k stages out to one workgroup per CU; when the
# groups number between 3/4 of the CUs and the CUs, one workgroup per group instead
# leaves no group cut between workgroups, so no merge launch follows (the GDN in_proj
# of the 4096-hidden model, 193 groups: 25.0 us against 30.2 us on 256 workgroups and
# 25.7 us on hipBLASLt, weights streaming from HBM).  When 96-column groups number so
# (and 64-column ones do not fit), one workgroup per 96-column group: lollm_gemm then
# takes 96-column groups, none cut (the MLP gate|up, 256 groups, 37 us in the step
# against 43 us + a 4.6 us merge; the attention q|gate|k|v, 192 groups).


def gemm_path(N, K, epilogue, rows, tiled=True):
    """'gemm' (lollm_gemm) or 'blas' (hipBLASLt) for a projection call; a pure function
    of the shape."""
    return "gemm" if tiled and rows <= ops.GEMM_MAX_ROWS else "blas"


def gemm_grid(N, cus, rows=ops.GEMM_MAX_ROWS):
    """Workgroups of a lollm_gemm call with N output columns and `rows` rows on a device
    with `cus` CUs: one per 64-column group when that covers 3/4 of the CUs or more; else
    one per 96-column group on the same condition (lollm_gemm then takes 96-column
    groups, none cut: the attention q|gate|k|v of the 4096-hidden model, 192 groups; its
    MLP gate|up, 256 = one per CU); else one per CU.  (`rows` is kept for shapes whose
    grid may come to depend on it; every rule is the same for 1..64 rows today.)"""
    groups = N // 64
    if 4 * groups >= 3 * cus and groups <= cus:
        return groups
    if N % 96 == 0:
        wide = N // 96
        if 4 * wide >= 3 * cus and wide <= cus:
            return wide
    return cus


class Projection:
    """y = x W^T (blocks.py's nn.Linear layers, no bias).  Keeps the row-major weight
    for hipBLASLt (F.linear) and a tiled copy for lollm_gemm (<= 64 rows).
    epilogue=GEMM_SWIGLU: W = [gate; up], y = silu(x gate^T) * x up^T (blocks.py:341-342).
    The path of each call is gemm_path() of its shape, the grid gemm_grid()."""

    def __init__(self, weight, epilogue=ops.GEMM_NONE):
        self.weight = weight.to(torch.bfloat16).contiguous()
        self.N, self.K = self.weight.shape
        self.epilogue = epilogue
        self.tiled = (ops.gemm_tile_weights(self.weight, epilogue)
                      if self.weight.is_cuda and ops.gemm_supported(self.N, self.K, epilogue)
                      else None)

    def workspace_bytes(self, rows=ops.GEMM_MAX_ROWS):
        if self.tiled is None:
            return 0
        return max(ops.gemm_workspace_bytes(rows, self.N, self.K, self.grid(rows)),
                   ops.gemm_workspace_bytes(rows, self.N, self.K, _cus()))

    def grid(self, rows=ops.GEMM_MAX_ROWS):
        return gemm_grid(self.N, _cus(), rows)

    def path(self, rows):
        return gemm_path(self.N, self.K, self.epilogue, rows, self.tiled is not None)

    def argmax_grid(self, rows):
        """Workgroups of the fused lm_head argmax (lollm_gemm_argmax): one per CU."""
        return _cus()

    def _blas(self, x):
        y = F.linear(x, self.weight)
        return ops.swiglu(y) if self.epilogue == ops.GEMM_SWIGLU else y

    def __call__(self, x):
        rows = x.numel() // self.K
        if self.path(rows) == "blas":
            return self._blas(x)
        return ops.gemm(x, self.tiled, self.N, self.K, self.epilogue, grid=self.grid(rows))

    def add_norm(self, x, residual, norm):
        """The projection feeding the residual stream with the add and the next RMSNorm
        (modeling_qwen3_5.py:59-60): x_out = residual + x W^T, y = norm(x_out); returns
        (y, x_out).  residual=None: x_out = x W^T (the MTP fc, which starts the MTP
        layer's residual stream).  lollm_gemm_rmsnorm (one GEMM call, the norm fused into its second
        kernel) when the path is lollm_gemm and the shape fits it, else the projection
        followed by lollm_rmsnorm."""
        rows = x.numel() // self.K
        g1 = self.grid(rows)
        if (self.path(rows) == "gemm" and self.epilogue == ops.GEMM_NONE
                and ops.gemm_rmsnorm_supported(rows, self.N, self.K, g1)):
            return ops.gemm_rmsnorm(x, self.tiled, self.N, self.K, residual, norm.weight, norm.eps,
                                    grid=g1)
        if residual is None:
            h = self(x)
            return norm(h), h
        return norm(self(x), residual=residual)


_CUS = {}


def _cus():
    """Compute units of the current device (the one-workgroup-per-CU GEMM grid)."""
    dev = torch.cuda.current_device()
    if dev not in _CUS:
        _CUS[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
    return _CUS[dev]


class RMSNorm:
    """(1 + w) RMSNorm in fp32 (blocks.py:23-35); optionally fused with the residual
    add that precedes it in the decoder (modeling_qwen3_5.py:59-60)."""

    def __init__(self, weight, eps):
        self.weight = weight.to(torch.bfloat16).contiguous()
        self.eps = eps

    def __call__(self, x, residual=None):
        x = x.contiguous()
        if residual is None:
            return ops.rmsnorm(x, self.weight, self.eps)
        return ops.rmsnorm(x, self.weight, self.eps, residual=residual.contiguous())


class MLP:
    """SwiGLU (blocks.py:332-342): gate|up as one GEMM with silu*up fused, down."""

    def __init__(self, gate, up, down):
        self.gate_up = Projection(_cat_rows(gate, up), ops.GEMM_SWIGLU)
        self.down = Projection(down)

    def projections(self):
        return [self.gate_up, self.down]

    def __call__(self, x):
        return self.down(self.gate_up(x))


class GatedDeltaNet:
    """GDN mixer (blocks.py:239-329): one in-projection GEMM, the fused conv / gating /
    scan / gated-norm kernel (lollm_gdn_layer), out_proj."""

    def __init__(self, cfg: Qwen3_5Config, W: dict, p: str):
        self.cfg = cfg
        Hv = cfg.linear_num_value_heads
        w = [W[p + "in_proj_qkv.weight"], W[p + "in_proj_z.weight"], W[p + "in_proj_b.weight"],
             W[p + "in_proj_a.weight"]]
        rows = cfg.conv_dim + cfg.value_dim + 2 * Hv
        pad = (-rows) % 64                     # whole 64-column GEMM groups (16-byte rows)
        if pad:
            w.append(torch.zeros(pad, cfg.hidden_size, dtype=w[0].dtype, device=w[0].device))
        self.in_proj = Projection(_cat_rows(*w))
        self.conv_w = W[p + "conv1d.weight"].reshape(cfg.conv_dim, -1).to(torch.bfloat16).contiguous()
        self.A_log = W[p + "A_log"].float().contiguous()
        self.dt_bias = W[p + "dt_bias"].float().contiguous()
        self.norm_w = W[p + "norm.weight"].to(torch.bfloat16).contiguous()
        self.out_proj = Projection(W[p + "out_proj.weight"])

    @property
    def w_in(self):
        return self.in_proj.weight

    def projections(self):
        return [self.in_proj, self.out_proj]

    def core(self, x, cache, layer):
        """Everything before out_proj (blocks.py:288-325)."""
        B, T, _ = x.shape
        cfg = self.cfg
        proj = self.in_proj(x)
        s = cache.layers[layer]
        return ops.gdn_layer(proj, self.conv_w, self.A_log, self.dt_bias, self.norm_w, s["win"],
                             cache.conv_off, s["rec"], cache.rec_half, s["rep"], cache.replay,
                             cache.fresh, B, T,
                             cfg.linear_num_key_heads, cfg.linear_num_value_heads,
                             cfg.linear_key_head_dim, cfg.linear_conv_kernel_dim,
                             cfg.rms_norm_eps)

    @property
    def out(self):
        return self.out_proj

    def __call__(self, x, cache, layer):
        return self.out_proj(self.core(x, cache, layer))


def rope_inv_freq(rotary_dim, theta, device):
    """blocks.py:166-168: inv_freq = 1 / theta^(arange(0, rd, 2) / rd) in fp32."""
    idx = torch.arange(0, rotary_dim, 2, dtype=torch.float32)
    return (1.0 / (theta ** (idx / rotary_dim))).to(device)


class GatedAttention:
    """Gated full attention (blocks.py:186-236): one q|k|v GEMM, the prologue kernel
    (gate split, QK-norm, partial RoPE, KV-cache append), the split-K verify
    attention kernel with the sigmoid gate fused, o_proj."""

    def __init__(self, cfg: Qwen3_5Config, W: dict, p: str, inv_freq):
        self.cfg = cfg
        self.qkv = Projection(_cat_rows(W[p + "q_proj.weight"], W[p + "k_proj.weight"],
                                        W[p + "v_proj.weight"]))
        self.q_norm = W[p + "q_norm.weight"].to(torch.bfloat16).contiguous()
        self.k_norm = W[p + "k_norm.weight"].to(torch.bfloat16).contiguous()
        self.o_proj = Projection(W[p + "o_proj.weight"])
        self.inv_freq = inv_freq

    def projections(self):
        return [self.qkv, self.o_proj]

    def core(self, x, k_cache, v_cache, lengths, kv_len, rope_pos=None, grid=0,
             workspace=None):
        """Everything before o_proj (blocks.py:208-235).  rope_pos: None (RoPE at the cache
        rows), (B,) int32 start positions, or (B, T) int32 per-token positions."""
        B, T, _ = x.shape
        cfg = self.cfg
        qkv = self.qkv(x)
        if T == 1 and k_cache.shape[2] <= ops.ATTN_SMALL_MAXL:
            # one token over a short cache (the MTP head's draft block): prologue fused
            return ops.attn_small(qkv, self.q_norm, self.k_norm, self.inv_freq, lengths, kv_len, B,
                                  cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim,
                                  cfg.rotary_dim, cfg.rms_norm_eps, k_cache, v_cache,
                                  rope_pos=None if rope_pos is None else rope_pos.reshape(B))
        q, gate = ops.attn_prologue(qkv, self.q_norm, self.k_norm, self.inv_freq, lengths, B, T,
                                    cfg.num_attention_heads, cfg.num_key_value_heads,
                                    cfg.head_dim, cfg.rotary_dim, cfg.rms_norm_eps, k_cache,
                                    v_cache, rope_pos=rope_pos)
        return ops.attn_verify(q, k_cache, v_cache, kv_len, gate, grid=grid, workspace=workspace)

    @property
    def out(self):
        return self.o_proj

    def __call__(self, x, k_cache, v_cache, lengths, kv_len, rope_pos=None, grid=0,
                 workspace=None):
        return self.o_proj(self.core(x, k_cache, v_cache, lengths, kv_len, rope_pos=rope_pos,
                                     grid=grid, workspace=workspace))
