"""Torch-tensor wrappers over the C ABI.  PyTorch supplies device memory and the
stream; every computation runs in the HIP kernels of `liblollm_amd.so`.

Each wrapper validates shapes/dtypes/devices on the host (so a bad call raises
instead of reaching a kernel), allocates outputs from torch's caching allocator,
and launches on `torch.cuda.current_stream()`.
"""

from __future__ import annotations

import torch

from . import _lib

BF16, F32 = 0, 1


def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.bfloat16:
        return BF16
    if t.dtype == torch.float32:
        return F32
    raise TypeError(f"unsupported dtype {t.dtype} (bf16 or fp32)")


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _need(t: torch.Tensor, name: str, dtype=None, shape=None):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a HIP device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if t.data_ptr() % 16:
        raise ValueError(f"{name} must be 16-byte aligned")


# ------------------------------------------------------------------------------------
# Gated DeltaNet
# ------------------------------------------------------------------------------------
def gdn_verify(q, k, v, g, beta, state=None, state_slot=None, *, snapshots=True,
               final_state=False, qk_l2norm=False, q_scale=None, out=None, snap_out=None,
               final_out=None):
    """Recurrent gated delta rule over T positions (blocks.py:116-144 math).

    q, k: (B, T, Hk, Dk); v: (B, T, Hv, Dv); g (fp32), beta: (B, T, Hv).
    state: fp32 (B * S, Hv, Dk, Dv) viewed as S slots per sequence (S = 1 for a
    plain (B, Hv, Dk, Dv) state, S = T_prev for a previous call's snapshots), or None.
    state_slot: int32 (B,) slot per sequence (O(1) rollback), or None.
    Returns (out, snapshots or None, final_state or None)."""
    B, T, Hk, Dk = q.shape
    Hv, Dv = v.shape[2], v.shape[3]
    dt = q.dtype
    _need(q, "q")
    _need(k, "k", dt, (B, T, Hk, Dk))
    _need(v, "v", dt, (B, T, Hv, Dv))
    _need(g, "g", torch.float32, (B, T, Hv))
    _need(beta, "beta", dt, (B, T, Hv))
    slots = 1
    if state is not None:
        _need(state, "state", torch.float32)
        if state.numel() % (B * Hv * Dk * Dv):
            raise ValueError("state size is not a whole number of per-sequence slots")
        slots = state.numel() // (B * Hv * Dk * Dv)
    if state_slot is not None:
        _need(state_slot, "state_slot", torch.int32, (B,))
        if state is None:
            raise ValueError("state_slot needs a state")
    elif slots != 1:
        raise ValueError("a multi-slot state needs state_slot")
    if out is None:
        out = torch.empty(B, T, Hv, Dv, dtype=dt, device=q.device)
    _need(out, "out", dt, (B, T, Hv, Dv))
    snaps = None
    if snapshots:
        snaps = snap_out if snap_out is not None else torch.empty(
            B, T, Hv, Dk, Dv, dtype=torch.float32, device=q.device)
        _need(snaps, "snapshots", torch.float32, (B, T, Hv, Dk, Dv))
    fin = None
    if final_state:
        fin = final_out if final_out is not None else torch.empty(
            B, Hv, Dk, Dv, dtype=torch.float32, device=q.device)
        _need(fin, "final_state", torch.float32, (B, Hv, Dk, Dv))
    if q_scale is None:
        q_scale = Dk ** -0.5
    rc = _lib.lib().lollm_gdn_verify(
        _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(state), _ptr(state_slot), slots,
        _ptr(out), _ptr(snaps), _ptr(fin), B, T, Hk, Hv, Dk, Dv, _dtype_code(q),
        int(bool(qk_l2norm)), float(q_scale), _stream())
    _lib.check(rc, "lollm_gdn_verify")
    return out, snaps, fin


def gdn_select_state(snapshots, slot, out=None):
    """Materialise the rolled-back state: out[b] = snapshots[b, slot[b]]."""
    B, T, Hv, Dk, Dv = snapshots.shape
    _need(snapshots, "snapshots", torch.float32)
    _need(slot, "slot", torch.int32, (B,))
    if out is None:
        out = torch.empty(B, Hv, Dk, Dv, dtype=torch.float32, device=snapshots.device)
    _need(out, "out", torch.float32, (B, Hv, Dk, Dv))
    rc = _lib.lib().lollm_gdn_select_state(_ptr(snapshots), _ptr(slot), _ptr(out), B, T, Hv,
                                           Dk, Dv, _stream())
    _lib.check(rc, "lollm_gdn_select_state")
    return out


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None,
                               use_qk_l2norm_in_kernel=False):
    """Drop-in for `torch_recurrent_gated_delta_rule(query, key, value, g, beta,
    initial_state=None, use_qk_l2norm_in_kernel=False) -> (out, final_state)`
    (src/qwen3_5/blocks.py:116-144): same argument meaning and outputs.  Unlike the
    reference, query/key may carry the qk-head count (Hk <= Hv); v-head h reads
    qk-head h // (Hv // Hk), which is what the reference's repeat_interleave
    (blocks.py:309-311) produces."""
    B, T, Hk, Dk = query.shape
    if beta.dtype != query.dtype:
        beta = beta.to(query.dtype)
    state = None if initial_state is None else initial_state.float().contiguous()
    out, _, fin = gdn_verify(query.contiguous(), key.contiguous(), value.contiguous(),
                             g.float().contiguous(), beta.contiguous(), state,
                             snapshots=False, final_state=True,
                             qk_l2norm=use_qk_l2norm_in_kernel)
    return out, fin
