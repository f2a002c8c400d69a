"""lollm_spec_accept_noalloc (no workspace argument, no device allocation) against
lollm_spec_accept with a caller workspace, through the C ABI: bit-identical accept
counts and emitted tokens on two calls in a row, the second with a smaller input (the
fixed scratch array keeps the first call's contents), and a shape whose workspace
exceeds the array is refused before any launch."""

import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(B, k, V, seed, with_draft):
    g = torch.Generator().manual_seed(seed)
    tgt = (torch.randn(B, k + 1, V, generator=g) * 3).bfloat16().cuda()
    drf = (tgt[:, :k].float().cpu() + torch.randn(B, k, V, generator=g)).bfloat16().cuda()
    # drafts = the argmax of each draft row (some accepted, some rejected)
    drafts = drf.float().argmax(-1).to(torch.int32).contiguous()
    return tgt, (drf if with_draft else None), drafts


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _accept(fn, tgt, drf, drafts, temp, top_k, top_p, seed, offset, ws=None):
    from lollm_amd import _lib, ops
    B, T, V = tgt.shape
    k = T - 1
    na = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    nt = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    args = [_ptr(tgt), _ptr(drf), _ptr(drafts), B, k, V, ops.inv_temperature(temp), top_k, top_p,
            seed, offset, None, _ptr(na), _ptr(nt)]
    if fn == "lollm_spec_accept":
        rc = L.lollm_spec_accept(*args, _ptr(ws), ws.numel(), stream)
    else:
        rc = L.lollm_spec_accept_noalloc(*args, stream)
    assert rc == 0, (fn, rc, L.lollm_strerror(rc))
    torch.cuda.synchronize()
    return na.cpu().numpy(), nt.cpu().numpy()


@pytest.mark.parametrize("temp,top_k,top_p", [(0.7, 0, 0.95), (0.0, 0, 1.0)])
def test_spec_accept_noalloc_matches_workspace_entry_point(temp, top_k, top_p):
    from lollm_amd import _lib
    L = _lib.lib()
    print(f"case noalloc T={temp}", flush=True)
    # first call: the acceptance workload with sampled drafts; second: smaller, one-hot q
    for B, k, V, seed, with_draft in ((64, 3, 151936, 1, True), (8, 2, 4096, 2, False)):
        tgt, drf, drafts = _case(B, k, V, seed, with_draft)
        need = L.lollm_spec_workspace_bytes(B, k, int(with_draft))
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        for off in (0, 5):
            want = _accept("lollm_spec_accept", tgt, drf, drafts, temp, top_k, top_p, 9, off, ws)
            got = _accept("lollm_spec_accept_noalloc", tgt, drf, drafts, temp, top_k, top_p, 9, off)
            assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
            assert (got[0] >= 0).all() and (got[1] >= 0).all()


def test_spec_accept_noalloc_refuses_oversized_shapes():
    """B = 2048 rows with k = 8 sampled drafts need more than the 1 MiB array (the
    workspace does not depend on the vocabulary), so the call returns LOLLM_EUNSUPPORTED
    before any launch.  The buffers are real device tensors over a vocabulary of 8, so
    that even a launch past the guard would only read and write memory it owns."""
    from lollm_amd import _lib
    L = _lib.lib()
    B, k, V = 2048, 8, 8
    assert L.lollm_spec_workspace_bytes(B, k, 1) > (1 << 20)
    tgt = torch.zeros(B, k + 1, V, dtype=torch.bfloat16, device="cuda")
    drf = torch.zeros(B, k, V, dtype=torch.bfloat16, device="cuda")
    drafts = torch.zeros(B, k, dtype=torch.int32, device="cuda")
    na = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    nt = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    rc = L.lollm_spec_accept_noalloc(_ptr(tgt), _ptr(drf), _ptr(drafts), B, k, V, 1.0, 0, 1.0, 0, 0,
                                     None, _ptr(na), _ptr(nt),
                                     torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 2          # LOLLM_EUNSUPPORTED, before any launch
    assert bool((na == -1).all()) and bool((nt == -1).all())
