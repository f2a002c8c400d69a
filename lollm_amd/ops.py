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


# ------------------------------------------------------------------------------------
# gated GQA attention over the KV cache
# ------------------------------------------------------------------------------------
def attn_workspace_bytes(B, T, Hq, Hkv, D, max_len, grid=0):
    """Bytes of the split-K partials buffer for `grid` workgroups (0: one per CU)."""
    n = _lib.lib().lollm_attn_workspace_bytes(B, T, Hq, Hkv, D, max_len, grid)
    if n < 0:
        raise ValueError("unsupported attention geometry")
    return n


def attn_verify(q, k_cache, v_cache, kv_len, gate=None, *, grid=0, scale=None,
                workspace=None, out=None):
    """q (B, T, Hq, D) bf16; k_cache / v_cache (B, Hkv, max_len, D) bf16 with the T
    new keys already written at positions kv_len-T .. kv_len-1; kv_len (B,) int32;
    gate (B, T, Hq*D) bf16 or None.  Returns (B, T, Hq*D) bf16.  The key blocks of
    all sequences are dealt out evenly to `grid` workgroups (0: one per CU)."""
    B, T, Hq, D = q.shape
    _need(q, "q", torch.bfloat16)
    if k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise ValueError("k_cache must be (B, Hkv, max_len, D)")
    Hkv, max_len = k_cache.shape[1], k_cache.shape[2]
    _need(k_cache, "k_cache", torch.bfloat16)
    _need(v_cache, "v_cache", torch.bfloat16, tuple(k_cache.shape))
    _need(kv_len, "kv_len", torch.int32, (B,))
    if gate is not None:
        _need(gate, "gate", torch.bfloat16, (B, T, Hq * D))
    if out is None:
        out = torch.empty(B, T, Hq * D, dtype=torch.bfloat16, device=q.device)
    _need(out, "out", torch.bfloat16, (B, T, Hq * D))
    if workspace is None:
        need = attn_workspace_bytes(B, T, Hq, Hkv, D, max_len, grid)
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    _need(workspace, "workspace")
    wbytes = workspace.numel() * workspace.element_size()
    if scale is None:
        scale = D ** -0.5
    rc = _lib.lib().lollm_attn_verify(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(kv_len), _ptr(gate), _ptr(out),
        _ptr(workspace), wbytes, B, T, Hq, Hkv, D, max_len, Hkv * max_len * D, max_len * D,
        grid, float(scale), _stream())
    _lib.check(rc, "lollm_attn_verify")
    return out


# ------------------------------------------------------------------------------------
# few-row weight-streaming GEMM
# ------------------------------------------------------------------------------------
GEMM_NONE, GEMM_SWIGLU = 0, 1
GEMM_MAX_ROWS = 64
# lollm_gemm_logits with extra penalised tokens: at most this many per row (n_extra0 + T - 1)
GEMM_LOGITS_MAX_EXTRA = 8
_gemm_ws = {}


def gemm_supported(N, K, epilogue=GEMM_NONE):
    return N % 64 == 0 and K % 128 == 0 and (epilogue == GEMM_NONE or (N // 2) % 32 == 0)


def gemm_tile_weights(weight, epilogue=GEMM_NONE):
    """The (N, K) bf16 weight re-laid in the 1 KB MFMA-operand blocks lollm_gemm streams
    (for GEMM_SWIGLU, weight = [gate; up] and gate/up rows are interleaved 8 by 8)."""
    N, K = weight.shape
    _need(weight, "weight", torch.bfloat16)
    out = torch.empty(N * K, dtype=torch.bfloat16, device=weight.device)
    rc = _lib.lib().lollm_gemm_tile_weights(_ptr(weight), _ptr(out), N, K, epilogue, _stream())
    _lib.check(rc, "lollm_gemm_tile_weights")
    return out


def gemm_workspace_bytes(M, N, K, grid=0):
    n = _lib.lib().lollm_gemm_workspace_bytes(M, N, K, grid)
    if n < 0:
        raise ValueError("unsupported GEMM shape")
    return n


_gemm_ws_retired = []


def gemm_workspace(nbytes, device):
    """The shared piece buffer of lollm_gemm (one per device, grown on demand; models
    reserve their largest size when they are built).  A buffer that is outgrown is kept
    alive, never freed: a HIP graph captured earlier may still write to its address."""
    key = torch.device(device)
    ws = _gemm_ws.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _gemm_ws_retired.append(ws)
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=key)
        _gemm_ws[key] = ws
    return ws


def gemm(x, tiled, N, K, epilogue=GEMM_NONE, out=None, grid=0):
    """y = x W^T for x (..., K) bf16 with at most 64 rows; `tiled` from
    gemm_tile_weights.  Returns (..., N), or (..., N / 2) = silu(gate) * up for
    GEMM_SWIGLU."""
    lead = x.shape[:-1]
    M = x.numel() // K
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} features, expected {K}")
    if M > GEMM_MAX_ROWS or M <= 0:
        raise ValueError(f"lollm_gemm takes 1..{GEMM_MAX_ROWS} rows, got {M}")
    x = x.contiguous()
    _need(x, "x", torch.bfloat16)
    _need(tiled, "tiled", torch.bfloat16, (N * K,))
    oc = N // 2 if epilogue == GEMM_SWIGLU else N
    if out is None:
        out = torch.empty(*lead, oc, dtype=torch.bfloat16, device=x.device)
    _need(out, "out", torch.bfloat16, (*lead, oc))
    ws = gemm_workspace(gemm_workspace_bytes(M, N, K, grid), x.device)
    rc = _lib.lib().lollm_gemm(_ptr(x), K, _ptr(tiled), _ptr(out), oc, M, N, K, epilogue, _ptr(ws),
                               ws.numel(), grid, _stream())
    _lib.check(rc, "lollm_gemm")
    return out


def gemm_argmax(x, tiled, N, K, out=None, grid=0):
    """argmax over the N columns of each row of x W^T (bf16-rounded products, ties to the
    lowest column) without writing the logits (lollm_gemm_argmax).  x (M, K) bf16 with
    M <= 64; `tiled` from gemm_tile_weights(W, GEMM_NONE).  out: (M,) int32, rows may be
    strided (e.g. one column of a (M, k) draft table)."""
    M = x.numel() // K
    if x.shape[-1] != K or M > GEMM_MAX_ROWS or M <= 0:
        raise ValueError(f"gemm_argmax takes 1..{GEMM_MAX_ROWS} rows of {K} features")
    x = x.contiguous()
    _need(x, "x", torch.bfloat16)
    _need(tiled, "tiled", torch.bfloat16, (N * K,))
    if out is None:
        out = torch.empty(M, dtype=torch.int32, device=x.device)
    if out.dtype != torch.int32 or out.dim() != 1 or out.numel() != M or not out.is_cuda:
        raise ValueError(f"out must be ({M},) int32 on the device")
    need = _lib.lib().lollm_gemm_argmax_workspace_bytes(M, N, K, grid)
    if need < 0:
        raise ValueError(f"gemm_argmax does not support M={M} N={N} K={K}")
    ws = gemm_workspace(need, x.device)
    rc = _lib.lib().lollm_gemm_argmax(_ptr(x), K, _ptr(tiled), M, N, K, _ptr(out), out.stride(0),
                                      _ptr(ws), ws.numel(), grid, _stream())
    _lib.check(rc, "lollm_gemm_argmax")
    return out


def gemm_rowmax_slots(grid=0):
    """Row-maximum slots per row that lollm_gemm_logits writes on `grid` workgroups."""
    n = _lib.lib().lollm_gemm_rowmax_slots(grid)
    if n < 0:
        raise ValueError(f"unsupported grid {grid}")
    return n


def gemm_logits(x, tiled, N, K, out=None, rowmax=None, *, seen=None, penalty=1.0, extra=None,
                n_extra0=0, T=1, grid=0):
    """Logits x W^T (bf16) with the repetition penalty applied in place to row m = (s, t)
    (s = m // T) for the tokens of seen[s] and extra[s, :n_extra0 + t] when seen is given
    (the bits of repetition_penalty on the stored logits), and the rows' maxima in
    `rowmax` (M, gemm_rowmax_slots(grid)) uint16 slots (lollm_gemm_logits; the input of
    spec_accept(..., target_rowmax=rowmax)).  Returns (out, rowmax)."""
    lead = x.shape[:-1]
    M = x.numel() // K
    if x.shape[-1] != K or M > GEMM_MAX_ROWS or M <= 0:
        raise ValueError(f"gemm_logits takes 1..{GEMM_MAX_ROWS} rows of {K} features")
    x = x.contiguous()
    _need(x, "x", torch.bfloat16)
    _need(tiled, "tiled", torch.bfloat16, (N * K,))
    if out is None:
        out = torch.empty(*lead, N, dtype=torch.bfloat16, device=x.device)
    _need(out, "out", torch.bfloat16, (*lead, N))
    slots = gemm_rowmax_slots(grid)
    if rowmax is None:
        rowmax = torch.empty(M, slots, dtype=torch.int16, device=x.device)
    if rowmax.dtype != torch.int16 or rowmax.dim() != 2 or rowmax.shape[0] != M or \
            rowmax.shape[1] != slots or rowmax.stride(1) != 1 or not rowmax.is_cuda:
        raise ValueError(f"rowmax must be ({M}, {slots}) int16 rows on the device")
    stride = 0
    if seen is not None:
        _need(seen, "seen", torch.int32)
        if M % T or seen.shape[0] != M // T or seen.shape[1] < seen_words(N):
            raise ValueError("seen must be (M / T, >= ceil(N / 32)) int32")
        if extra is not None:
            if extra.dtype != torch.int32 or extra.dim() != 2 or extra.shape[0] != M // T or \
                    extra.stride(1) != 1:
                raise ValueError("extra must be (M / T, n) int32 with unit column stride")
            stride = extra.stride(0)
    ws = gemm_workspace(gemm_workspace_bytes(M, N, K, grid), x.device)
    rc = _lib.lib().lollm_gemm_logits(
        _ptr(x), K, _ptr(tiled), M, N, K, _ptr(out), N, _ptr(rowmax), rowmax.stride(0),
        None if seen is None else _ptr(seen), 0 if seen is None else seen.shape[1],
        None if (seen is None or extra is None) else _ptr(extra), stride, int(n_extra0), int(T),
        float(penalty), _ptr(ws), ws.numel(), grid, _stream())
    _lib.check(rc, "lollm_gemm_logits")
    return out, rowmax


def gemm_rmsnorm_supported(M, N, K, grid=0):
    """Whether lollm_gemm_rmsnorm takes this shape (N <= 8192 and at least one
    (64-column, 128-k) unit per workgroup)."""
    if not gemm_supported(N, K) or N > 8192 or not 0 < M <= GEMM_MAX_ROWS:
        return False
    if grid <= 0:
        dev = torch.cuda.current_device()
        if dev not in _cu_count:
            _cu_count[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
        grid = 2 * _cu_count[dev]
    return (N // 64) * (K // 128) >= grid


_cu_count = {}


def gemm_rmsnorm(x, tiled, N, K, residual, w, eps, grid=0):
    """h = x W^T completed with the residual add and RMSNorm of the decoder layer:
    x_out = bf16(h + residual), y = RMSNorm_{1+w}(x_out).  Returns (y, x_out), the same
    bits as gemm() followed by rmsnorm(h, w, eps, residual=residual).  residual=None:
    x_out = h and y = rmsnorm(h, w, eps)."""
    lead = x.shape[:-1]
    M = x.numel() // K
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} features, expected {K}")
    if M > GEMM_MAX_ROWS or M <= 0:
        raise ValueError(f"lollm_gemm takes 1..{GEMM_MAX_ROWS} rows, got {M}")
    x = x.contiguous()
    _need(x, "x", torch.bfloat16)
    _need(tiled, "tiled", torch.bfloat16, (N * K,))
    if residual is not None:
        residual = residual.contiguous()
        _need(residual, "residual", torch.bfloat16, (*lead, N))
    _need(w, "w", torch.bfloat16, (N,))
    c = torch.empty(*lead, N, dtype=torch.bfloat16, device=x.device)
    x_out = torch.empty_like(c)
    y = torch.empty_like(c)
    ws = gemm_workspace(gemm_workspace_bytes(M, N, K, grid), x.device)
    rc = _lib.lib().lollm_gemm_rmsnorm(_ptr(x), K, _ptr(tiled), M, N, K,
                                       None if residual is None else _ptr(residual), _ptr(w),
                                       float(eps), _ptr(c), _ptr(x_out), _ptr(y), _ptr(ws),
                                       ws.numel(), grid, _stream())
    _lib.check(rc, "lollm_gemm_rmsnorm")
    return y, x_out


# ------------------------------------------------------------------------------------
# speculative sampling
# ------------------------------------------------------------------------------------
def inv_temperature(temperature: float) -> float:
    """1/T rounded to fp32 (0 selects greedy, the reference's T <= 0 branch)."""
    import numpy as np
    return float(np.float32(1.0 / temperature)) if temperature > 0 else 0.0


def spec_accept(target, draft, drafts, temperature, top_k=0, top_p=1.0, seed=0, offset=0, *,
                offset_dev=None, workspace=None, n_accepted=None, next_token=None,
                target_rowmax=None):
    """target (B, k+1, V) bf16; draft (B, k, V) bf16 or None (argmax drafts);
    drafts (B, k) int32.  target_rowmax: the (B (k+1), slots) row-maximum slots that
    gemm_logits wrote with the target logits (lollm_spec_accept_rowmax: each target row
    read once; same results).  Returns (n_accepted (B,), next_token (B,)) int32."""
    B, T, V = target.shape
    k = T - 1
    _need(target, "target", torch.bfloat16)
    if draft is not None:
        _need(draft, "draft", torch.bfloat16, (B, k, V))
    _need(drafts, "drafts", torch.int32, (B, k))
    if offset_dev is not None:
        _need(offset_dev, "offset_dev", torch.int64, (1,))
    need = _lib.lib().lollm_spec_workspace_bytes(B, k, int(draft is not None))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=target.device)
    _need(workspace, "workspace")
    if n_accepted is None:
        n_accepted = torch.empty(B, dtype=torch.int32, device=target.device)
    if next_token is None:
        next_token = torch.empty(B, dtype=torch.int32, device=target.device)
    args = (B, k, V, inv_temperature(temperature), int(top_k or 0),
            float(top_p if top_p is not None else 1.0), seed, offset, _ptr(offset_dev),
            _ptr(n_accepted), _ptr(next_token), _ptr(workspace), workspace.numel(), _stream())
    if target_rowmax is not None:
        rm = target_rowmax
        if rm.dtype != torch.int16 or rm.dim() != 2 or rm.shape[0] != B * T or rm.stride(1) != 1 \
                or not rm.is_cuda:
            raise ValueError(f"target_rowmax must be ({B * T}, slots) int16 rows on the device")
        rc = _lib.lib().lollm_spec_accept_rowmax(_ptr(target), _ptr(rm), rm.stride(0), rm.shape[1],
                                                 _ptr(draft), _ptr(drafts), *args)
        _lib.check(rc, "lollm_spec_accept_rowmax")
    else:
        rc = _lib.lib().lollm_spec_accept(_ptr(target), _ptr(draft), _ptr(drafts), *args)
        _lib.check(rc, "lollm_spec_accept")
    return n_accepted, next_token


def sample_workspace_bytes(rows):
    n = _lib.lib().lollm_sample_workspace_bytes(rows)
    if n < 0:
        raise ValueError("rows must be positive")
    return n


def sample_rows(logits, temperature, top_k=0, top_p=1.0, seed=0, offset=0, row_base=0, slot=0,
                *, offset_dev=None, workspace=None, out=None):
    """One token per row of logits (rows, V) bf16.  Returns (rows,) int32."""
    rows, V = logits.shape
    _need(logits, "logits", torch.bfloat16)
    if workspace is None:
        workspace = torch.empty(sample_workspace_bytes(rows), dtype=torch.uint8,
                                device=logits.device)
    _need(workspace, "workspace")
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    rc = _lib.lib().lollm_sample_rows(
        _ptr(logits), rows, V, inv_temperature(temperature), int(top_k or 0),
        float(top_p if top_p is not None else 1.0), seed, offset, _ptr(offset_dev), row_base,
        slot, _ptr(out), _ptr(workspace), workspace.numel(), _stream())
    _lib.check(rc, "lollm_sample_rows")
    return out


def philox_u24(seed, offset, rows, slots, device="cuda"):
    out = torch.empty(rows, slots, dtype=torch.int32, device=device)
    rc = _lib.lib().lollm_philox_uniform_u24(seed, offset, rows, slots, _ptr(out), _stream())
    _lib.check(rc, "lollm_philox_uniform_u24")
    return out


# ------------------------------------------------------------------------------------
# fused decoder-layer kernels
# ------------------------------------------------------------------------------------
def mtp_input(tok, hidden, table, w_emb, w_hidden, eps, out=None):
    """[RMSNorm_{1+w_emb}(table[tok]) | RMSNorm_{1+w_hidden}(hidden)] -> (B, 2H) bf16 in one
    kernel (lollm_mtp_input).  tok (B,) int32; hidden (B, H) bf16 (rows may be strided);
    table (V, H) bf16."""
    B = tok.numel()
    V, H = table.shape
    if tok.dtype != torch.int32 or tok.dim() != 1 or not tok.is_cuda:
        raise ValueError("tok must be a (B,) int32 device tensor (rows may be strided)")
    _need(table, "table", torch.bfloat16)
    _need(w_emb, "w_emb", torch.bfloat16, (H,))
    _need(w_hidden, "w_hidden", torch.bfloat16, (H,))
    if hidden.dtype != torch.bfloat16 or hidden.shape[-1] != H or hidden.numel() != B * H:
        raise ValueError(f"hidden must be ({B}, {H}) bf16, got {tuple(hidden.shape)} {hidden.dtype}")
    hidden = hidden.reshape(B, H)
    if hidden.stride(-1) != 1 or hidden.data_ptr() % 16 or hidden.stride(0) % 8:
        hidden = hidden.contiguous()
    if out is None:
        out = torch.empty(B, 2 * H, dtype=torch.bfloat16, device=table.device)
    _need(out, "out", torch.bfloat16, (B, 2 * H))
    rc = _lib.lib().lollm_mtp_input(_ptr(tok), tok.stride(0), _ptr(hidden), hidden.stride(0), _ptr(table), V,
                                    _ptr(w_emb), _ptr(w_hidden), _ptr(out), B, H, float(eps),
                                    _stream())
    _lib.check(rc, "lollm_mtp_input")
    return out


def verify_input(first, drafts, table, w, eps, lengths=None, *, ids=None, x=None, y=None,
                 kv_len=None):
    """The verify block's input in one kernel (lollm_verify_input): ids = [first | drafts]
    (B, 1 + k) int32, x = table[ids] and y = RMSNorm_{1+w}(x), both (B, 1 + k, H) bf16, and,
    with lengths, kv_len = lengths + 1 + k.  first (B,) int32, drafts (B, k) int32.
    Returns (ids, x, y, kv_len)."""
    B = first.numel()
    V, H = table.shape
    if first.dtype != torch.int32 or first.dim() != 1 or not first.is_cuda:
        raise ValueError("first must be a (B,) int32 device tensor")
    k = 0 if drafts is None else drafts.shape[1]
    if drafts is not None:
        _need(drafts, "drafts", torch.int32, (B, k))
    _need(table, "table", torch.bfloat16)
    _need(w, "w", torch.bfloat16, (H,))
    T = k + 1
    dev = table.device
    ids = torch.empty(B, T, dtype=torch.int32, device=dev) if ids is None else ids
    x = torch.empty(B, T, H, dtype=torch.bfloat16, device=dev) if x is None else x
    y = torch.empty(B, T, H, dtype=torch.bfloat16, device=dev) if y is None else y
    _need(ids, "ids", torch.int32, (B, T))
    _need(x, "x", torch.bfloat16, (B, T, H))
    _need(y, "y", torch.bfloat16, (B, T, H))
    if lengths is not None:
        _need(lengths, "lengths", torch.int32, (B,))
        kv_len = torch.empty(B, dtype=torch.int32, device=dev) if kv_len is None else kv_len
        _need(kv_len, "kv_len", torch.int32, (B,))
    else:
        kv_len = None
    rc = _lib.lib().lollm_verify_input(_ptr(first), _ptr(drafts), k, _ptr(table), V, _ptr(w),
                                       float(eps), _ptr(lengths), _ptr(ids), _ptr(x), _ptr(y),
                                       _ptr(kv_len), B, H, _stream())
    _lib.check(rc, "lollm_verify_input")
    return ids, x, y, kv_len


def rmsnorm(x, w, eps, residual=None, x_out=None, out=None):
    """y = RMSNorm_{1+w}(x) or, with residual, x_out = x + residual, y = norm(x_out).
    x: (..., H) bf16.  Returns y, or (y, x_out) when residual is given."""
    H = x.shape[-1]
    rows = x.numel() // H
    _need(x, "x", torch.bfloat16)
    _need(w, "w", torch.bfloat16, (H,))
    if residual is not None:
        _need(residual, "residual", torch.bfloat16, tuple(x.shape))
        if x_out is None:
            x_out = torch.empty_like(x)
    if out is None:
        out = torch.empty_like(x)
    rc = _lib.lib().lollm_rmsnorm(_ptr(x), _ptr(residual), _ptr(x_out), _ptr(w), _ptr(out), rows,
                                  H, float(eps), _stream())
    _lib.check(rc, "lollm_rmsnorm")
    return (out, x_out) if residual is not None else out


def swiglu(gate_up, out=None):
    """gate_up (..., 2F) bf16 -> (..., F)."""
    F2 = gate_up.shape[-1]
    rows = gate_up.numel() // F2
    _need(gate_up, "gate_up", torch.bfloat16)
    if out is None:
        out = torch.empty(*gate_up.shape[:-1], F2 // 2, dtype=torch.bfloat16, device=gate_up.device)
    rc = _lib.lib().lollm_swiglu(_ptr(gate_up), _ptr(out), rows, F2 // 2, _stream())
    _lib.check(rc, "lollm_swiglu")
    return out


def attn_prologue(qkv, q_norm_w, k_norm_w, inv_freq, lengths, B, T, Hq, Hkv, D, rotary_dim, eps,
                  k_cache, v_cache, q_out=None, gate_out=None, rope_pos=None):
    """rope_pos: None (RoPE at the cache rows lengths[b] + t), (B,) int32 (positions
    rope_pos[b] + t) or (B, T) int32 (each token's own position)."""
    _need(qkv, "qkv", torch.bfloat16)
    per_token = rope_pos is not None and rope_pos.dim() == 2
    if rope_pos is not None:
        _need(rope_pos, "rope_pos", torch.int32, (B, T) if per_token else (B,))
    if qkv.numel() != B * T * (Hq * 2 * D + 2 * Hkv * D):
        raise ValueError("qkv has the wrong size")
    _need(lengths, "lengths", torch.int32, (B,))
    _need(k_cache, "k_cache", torch.bfloat16)
    _need(v_cache, "v_cache", torch.bfloat16, tuple(k_cache.shape))
    max_len = k_cache.shape[2]
    if q_out is None:
        q_out = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=qkv.device)
    if gate_out is None:
        gate_out = torch.empty(B, T, Hq * D, dtype=torch.bfloat16, device=qkv.device)
    rc = _lib.lib().lollm_attn_prologue(
        _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(inv_freq), _ptr(lengths), _ptr(rope_pos),
        int(per_token), B, T, Hq, Hkv, D, rotary_dim, float(eps), _ptr(q_out), _ptr(gate_out), _ptr(k_cache), _ptr(v_cache),
        max_len, _stream())
    _lib.check(rc, "lollm_attn_prologue")
    return q_out, gate_out


ATTN_SMALL_MAXL = 16


def attn_small(qkv, q_norm_w, k_norm_w, inv_freq, lengths, kv_len, B, Hq, Hkv, D, rotary_dim, eps,
               k_cache, v_cache, rope_pos=None, scale=None, out=None):
    """One new token per sequence attending over a cache of at most ATTN_SMALL_MAXL rows,
    with the prologue fused (lollm_attn_small).  qkv (B, Hq*2D + 2*Hkv*D) bf16; caches
    (B, Hkv, max_len, D).  Returns (B, 1, Hq*D) bf16."""
    _need(qkv, "qkv", torch.bfloat16)
    if qkv.numel() != B * (Hq * 2 * D + 2 * Hkv * D):
        raise ValueError("qkv has the wrong size")
    _need(lengths, "lengths", torch.int32, (B,))
    _need(kv_len, "kv_len", torch.int32, (B,))
    _need(k_cache, "k_cache", torch.bfloat16)
    _need(v_cache, "v_cache", torch.bfloat16, tuple(k_cache.shape))
    max_len = k_cache.shape[2]
    if scale is None:
        scale = D ** -0.5
    if out is None:
        out = torch.empty(B, 1, Hq * D, dtype=torch.bfloat16, device=qkv.device)
    _need(out, "out", torch.bfloat16, (B, 1, Hq * D))
    rc = _lib.lib().lollm_attn_small(
        _ptr(qkv), _ptr(q_norm_w), _ptr(k_norm_w), _ptr(inv_freq), _ptr(lengths), _ptr(rope_pos),
        _ptr(kv_len), B, Hq, Hkv, D, rotary_dim, float(eps), float(scale), _ptr(k_cache),
        _ptr(v_cache), max_len, _ptr(out), _stream())
    _lib.check(rc, "lollm_attn_small")
    return out


GDN_CHUNK_MIN_T = 64


def gdn_chunked_ok(T, slots, win_rows, conv_kernel, proj_stride=0):
    """Whether a call can take the chunked long-call kernel (lollm_gdn_layer_chunked):
    a call longer than the replay-record slots and the conv window, and one sequence's
    projection rows addressable with 32-bit byte offsets."""
    return (conv_kernel == 4 and T > slots and conv_kernel - 1 + T > win_rows
            and T * proj_stride * 2 < 2 ** 31)


def gdn_record_bytes(D):
    """Bytes of one replay record of a GDN head with Dk = Dv = D: k and v (bf16), then
    exp(g), beta and 1/|k| (fp32) and a pad word."""
    return 4 * D + 16


def _check_gdn_state(rec, rec_half, rep, replay, B, Hv, D):
    _need(rec, "rec", torch.float32, (B, 2, Hv, D, D))
    _need(rec_half, "rec_half", torch.int32, (B,))
    _need(replay, "replay", torch.int32, (B,))
    _need(rep, "rep", torch.uint8)
    if (rep.dim() != 5 or tuple(rep.shape[:3]) != (B, 2, Hv)
            or rep.shape[4] != gdn_record_bytes(D) or rep.shape[3] < 1):
        raise ValueError(f"rep must be (B, 2, Hv, slots, {gdn_record_bytes(D)}) uint8")
    return rep.shape[3]


def gdn_layer(proj, conv_w, A_log, dt_bias, norm_w, win, conv_off, rec, rec_half, rep, replay,
              fresh, B, T, Hk, Hv, D, conv_kernel, eps, out=None, chunked=None):
    """Fused GDN mixer (include/lollm_amd.h).  proj (B, T, P) bf16; win (B, 2W,
    conv_dim) bf16; rec (B, 2, Hv, D, D) fp32 state halves; rep (B, 2, Hv, S,
    gdn_record_bytes(D)) uint8 replay records; conv_off / rec_half / replay (B,) int32.
    chunked: None = the chunked kernel for long calls of at least GDN_CHUNK_MIN_T tokens
    that it supports, the recurrent kernel otherwise; True / False force one."""
    P = proj.shape[-1]
    _need(proj, "proj", torch.bfloat16)
    _need(win, "win", torch.bfloat16)
    _need(conv_off, "conv_off", torch.int32, (B,))
    S = _check_gdn_state(rec, rec_half, rep, replay, B, Hv, D)
    if win.shape[0] != B or win.shape[1] % 2:
        raise ValueError("win must hold two halves per sequence")
    value_dim = Hv * D
    if out is None:
        out = torch.empty(B, T, value_dim, dtype=torch.bfloat16, device=proj.device)
    W = win.shape[1] // 2
    if chunked is None:
        chunked = T >= GDN_CHUNK_MIN_T and gdn_chunked_ok(T, S, W, conv_kernel, P)
    fn = "lollm_gdn_layer_chunked" if chunked else "lollm_gdn_layer"
    rc = getattr(_lib.lib(), fn)(
        _ptr(proj), P, _ptr(conv_w), _ptr(A_log), _ptr(dt_bias), _ptr(norm_w), _ptr(win),
        _ptr(conv_off), W, _ptr(rec), _ptr(rec_half), _ptr(rep), _ptr(replay), S,
        int(bool(fresh)), _ptr(out), B, T, Hk, Hv, D, D, conv_kernel, float(eps), _stream())
    _lib.check(rc, fn)
    return out


def gdn_state(rec, rec_half, rep, replay, out=None, to_other_half=False):
    """The committed recurrent state of one GDN layer (lollm_gdn_state): (B, Hv, D, D) fp32
    in `out` (allocated if None), or, with to_other_half, written into the other half of
    rec (returns None; the caller then flips rec_half and zeroes replay)."""
    B, _, Hv, D, _ = rec.shape
    S = _check_gdn_state(rec, rec_half, rep, replay, B, Hv, D)
    if to_other_half:
        out = None
    elif out is None:
        out = torch.empty(B, Hv, D, D, dtype=torch.float32, device=rec.device)
    else:
        _need(out, "out", torch.float32, (B, Hv, D, D))
    rc = _lib.lib().lollm_gdn_state(_ptr(rec), _ptr(rec_half), _ptr(rep), _ptr(replay), S, B, Hv,
                                    D, D, _ptr(out), _stream())
    _lib.check(rc, "lollm_gdn_state")
    return out


def greedy_accept(argmax, drafts, n_accepted, next_token):
    """Greedy acceptance from the verify rows' argmax tokens (lollm_greedy_accept):
    argmax (B, k + 1) int32, drafts (B, k) int32; writes n_accepted, next_token (B,)."""
    B, T = argmax.shape
    k = T - 1
    _need(argmax, "argmax", torch.int32)
    if k > 0:
        _need(drafts, "drafts", torch.int32, (B, k))
    _need(n_accepted, "n_accepted", torch.int32, (B,))
    _need(next_token, "next_token", torch.int32, (B,))
    rc = _lib.lib().lollm_greedy_accept(_ptr(argmax), _ptr(drafts) if k > 0 else None, B, k,
                                        _ptr(n_accepted), _ptr(next_token), _stream())
    _lib.check(rc, "lollm_greedy_accept")


def spec_commit(verify_ids, n_accepted, next_token, lengths, rec_half, replay, conv_off, pending,
                out_tokens, out_count, hidden, h_last, offset, slots, win_rows, accept_hist=None,
                seen=None):
    B, T = verify_ids.shape
    H = hidden.shape[-1]
    if seen is not None:
        _need(seen, "seen", torch.int32)
        if seen.dim() != 2 or seen.shape[0] != B:
            raise ValueError("seen must be (B, words) int32")
    rc = _lib.lib().lollm_spec_commit(
        _ptr(verify_ids), _ptr(n_accepted), _ptr(next_token), _ptr(lengths), _ptr(rec_half),
        _ptr(replay), _ptr(conv_off), _ptr(pending), _ptr(out_tokens), _ptr(out_count), out_tokens.shape[1],
        _ptr(hidden), _ptr(h_last), B, T, H, slots, win_rows, _ptr(offset), _ptr(accept_hist),
        _ptr(seen), 0 if seen is None else seen.shape[1], _stream())
    _lib.check(rc, "lollm_spec_commit")


# ------------------------------------------------------------------------------------
# repetition penalty (src/generate.py:18-22) on the device
# ------------------------------------------------------------------------------------
def seen_words(V):
    """32-bit words of one sequence's seen-token bitmap."""
    return (V + 31) // 32


def new_seen(B, V, device):
    """Empty (B, words) seen-token bitmaps (int32 storage of the uint32 words)."""
    return torch.zeros(B, seen_words(V), dtype=torch.int32, device=device)


def seen_mark(seen, tokens, V):
    """seen[b] |= set(tokens[b]) for tokens (B, n) or (B,) integer ids on the device."""
    _need(seen, "seen", torch.int32)
    B = seen.shape[0]
    t = tokens.reshape(B, -1)
    if t.dtype != torch.int32 or t.stride(-1) != 1:
        t = t.to(torch.int32).contiguous()
    n = t.shape[1]
    rc = _lib.lib().lollm_seen_mark(_ptr(seen), seen.shape[1], B, _ptr(t), t.stride(0), n, V,
                                    _stream())
    _lib.check(rc, "lollm_seen_mark")
    return seen


def repetition_penalty(logits, seen, penalty, extra=None, n_extra0=0):
    """In place on bf16 logits (B, T, V) (or (B, V) = T 1): row (b, t) penalises the tokens
    of seen[b] plus extra[b, :n_extra0 + t] (each once), the reference's
    where(x > 0, x / p, x * p) in bf16 arithmetic.  Returns logits."""
    if logits.dim() == 2:
        B, V = logits.shape
        T = 1
    else:
        B, T, V = logits.shape
    if logits.dtype != torch.bfloat16 or not logits.is_cuda or logits.stride(-1) != 1:
        raise ValueError("logits must be bf16 on the device with unit column stride")
    # the kernel addresses row (b, t) at (b * T + t) * ld: one row stride for all rows
    # (strides of size-1 dimensions are irrelevant)
    if T > 1:
        ld = logits.stride(-2)
        if B > 1 and logits.stride(0) != T * ld:
            raise ValueError("logits rows must be evenly strided")
    else:
        ld = logits.stride(0) if B > 1 else V
    if ld < V:
        raise ValueError("logits rows overlap")
    _need(seen, "seen", torch.int32)
    if seen.shape[0] != B or seen.shape[1] < seen_words(V):
        raise ValueError("seen must be (B, >= ceil(V / 32)) int32")
    stride = 0
    if extra is not None:
        if extra.dtype != torch.int32 or extra.dim() != 2 or extra.shape[0] != B or extra.stride(1) != 1:
            raise ValueError("extra must be (B, n) int32 with unit column stride")
        stride = extra.stride(0)
        if extra.shape[1] < n_extra0 + T - 1:
            raise ValueError("extra has fewer tokens than the rows need")
    rc = _lib.lib().lollm_repetition_penalty(_ptr(logits), ld, B, T, V, _ptr(seen), seen.shape[1],
                                             _ptr(extra), stride, int(n_extra0), float(penalty),
                                             _stream())
    _lib.check(rc, "lollm_repetition_penalty")
    return logits
