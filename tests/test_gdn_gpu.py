"""GDN verify kernel vs the oracle (src/qwen3_5/blocks.py:116-144 restated).

Tolerances (written here, as the brief states them): fp32 inputs rtol 1e-4; bf16
inputs rtol 2e-2 (outputs are bf16; the oracle normalises q,k in bf16 like the
reference while the kernel normalises in fp32).
"""

import pytest
import torch

from oracle import qwen3_5_ref as R

pytestmark = pytest.mark.gpu

FP32_TOL = dict(rtol=1e-4, atol=1e-5)
BF16_TOL = dict(rtol=2e-2, atol=2e-2)


def make_inputs(B, T, Hk, Hv, seed, dtype, l2=False, state=True):
    """The isolated verify workload's distributions: q,k ~ N(0,1) then L2-normalised
    (unless the kernel normalises), v ~ N(0,1), beta = sigmoid(N(0,1)),
    g = -softplus(N(0,1)), S0 ~ N(0, 0.02^2) fp32."""
    gen = torch.Generator().manual_seed(seed)
    D = 128
    q = torch.randn(B, T, Hk, D, generator=gen)
    k = torch.randn(B, T, Hk, D, generator=gen)
    if not l2:
        q = q / q.norm(dim=-1, keepdim=True).clamp_min(1e-6)
        k = k / k.norm(dim=-1, keepdim=True).clamp_min(1e-6)
    v = torch.randn(B, T, Hv, D, generator=gen)
    beta = torch.sigmoid(torch.randn(B, T, Hv, generator=gen))
    g = -torch.nn.functional.softplus(torch.randn(B, T, Hv, generator=gen))
    s0 = torch.randn(B, Hv, D, D, generator=gen) * 0.02 if state else None
    q, k, v, beta = (t.to(dtype) for t in (q, k, v, beta))
    return q, k, v, g, beta, s0


def oracle(q, k, v, g, beta, s0, l2):
    rep = v.shape[2] // q.shape[2]
    qq = q.repeat_interleave(rep, dim=2)
    kk = k.repeat_interleave(rep, dim=2)
    return R.gdn_scan_recurrent_snapshots(qq, kk, v, g, beta, s0, qk_l2=l2)


def to_dev(*ts):
    return [None if t is None else t.cuda() for t in ts]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
# the last two shapes are the isolated workload's head counts at B = 8 and 16
@pytest.mark.parametrize("B,T,Hk,Hv", [(1, 1, 2, 4), (3, 2, 2, 4), (2, 5, 16, 32), (1, 3, 4, 4),
                                       (8, 2, 16, 32), (16, 3, 16, 32)])
@pytest.mark.parametrize("l2", [False, True])
def test_gdn_verify_matches_oracle(dtype, B, T, Hk, Hv, l2):
    from lollm_amd import ops
    print(f"case dtype={dtype} B={B} T={T} Hk={Hk} Hv={Hv} l2={l2}", flush=True)
    q, k, v, g, beta, s0 = make_inputs(B, T, Hk, Hv, seed=B * 100 + T, dtype=dtype, l2=l2)
    o_ref, snaps_ref = oracle(q, k, v, g, beta, s0, l2)
    out, snaps, fin = ops.gdn_verify(*to_dev(q, k, v, g, beta, s0), snapshots=True,
                                     final_state=True, qk_l2norm=l2)
    torch.cuda.synchronize()
    tol = FP32_TOL if dtype == torch.float32 else BF16_TOL
    torch.testing.assert_close(out.cpu().float(), o_ref.float(), **tol)
    torch.testing.assert_close(snaps.cpu(), snaps_ref, **tol)
    torch.testing.assert_close(fin.cpu(), snaps_ref[:, -1], **tol)


def test_gdn_batch_invariant_bits():
    """The same (sequence, head) computed alone and inside batches of 8 and 16 gives
    identical bits: a workgroup's sums never depend on the batch around it."""
    from lollm_amd import ops
    T, Hk, Hv = 3, 16, 32
    q, k, v, g, beta, s0 = make_inputs(1, T, Hk, Hv, seed=31, dtype=torch.bfloat16)
    res = []
    for B in (1, 8, 16):
        print(f"batch-invariance case B={B}", flush=True)
        rep = lambda t: t.expand(B, *t.shape[1:]).contiguous()
        out, snaps, fin = ops.gdn_verify(*to_dev(*(rep(t) for t in (q, k, v, g, beta, s0))),
                                         snapshots=True, final_state=True)
        torch.cuda.synchronize()
        res.append((out[:1].cpu(), snaps[:1].cpu(), fin[:1].cpu()))
        assert torch.equal(out[0].cpu(), out[-1].cpu())
    for r in res[1:]:
        for a, b in zip(res[0], r):
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                               b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))


def test_gdn_zero_initial_state():
    from lollm_amd import ops
    q, k, v, g, beta, _ = make_inputs(2, 3, 2, 4, seed=7, dtype=torch.float32, state=False)
    o_ref, snaps_ref = oracle(q, k, v, g, beta, None, False)
    out, snaps, _ = ops.gdn_verify(*to_dev(q, k, v, g, beta), None)
    torch.testing.assert_close(out.cpu(), o_ref, **FP32_TOL)
    torch.testing.assert_close(snaps.cpu(), snaps_ref, **FP32_TOL)


def test_gdn_rollback_slots_and_select():
    """O(1) rollback: a second call reads snapshot slot a_b of the first call's
    snapshots; it must equal a fresh run over the accepted prefix then the new
    tokens.  select_state materialises the same slots."""
    from lollm_amd import ops
    B, T, Hk, Hv = 4, 4, 2, 4
    q, k, v, g, beta, s0 = make_inputs(B, T, Hk, Hv, seed=21, dtype=torch.float32)
    q2, k2, v2, g2, b2, _ = make_inputs(B, T, Hk, Hv, seed=22, dtype=torch.float32)
    acc = torch.tensor([0, 3, 1, 2], dtype=torch.int32)
    _, snaps, _ = ops.gdn_verify(*to_dev(q, k, v, g, beta, s0))
    out2, _, fin2 = ops.gdn_verify(*to_dev(q2, k2, v2, g2, b2), snaps, acc.cuda(),
                                   snapshots=False, final_state=True)
    sel = ops.gdn_select_state(snaps, acc.cuda())
    torch.cuda.synchronize()
    for b in range(B):
        a = int(acc[b]) + 1
        sl = slice(b, b + 1)
        _, sa = oracle(q[sl, :a], k[sl, :a], v[sl, :a], g[sl, :a], beta[sl, :a], s0[sl], False)
        torch.testing.assert_close(sel[b].cpu(), sa[0, -1], **FP32_TOL)
        o_ref, s_ref = oracle(q2[sl], k2[sl], v2[sl], g2[sl], b2[sl], sa[:, -1], False)
        torch.testing.assert_close(out2[b].cpu(), o_ref[0], **FP32_TOL)
        torch.testing.assert_close(fin2[b].cpu(), s_ref[0, -1], **FP32_TOL)


def test_gdn_in_place_final_state():
    from lollm_amd import ops
    q, k, v, g, beta, s0 = make_inputs(2, 2, 2, 4, seed=5, dtype=torch.float32)
    o_ref, snaps_ref = oracle(q, k, v, g, beta, s0, False)
    st = s0.cuda()
    ops.gdn_verify(*to_dev(q, k, v, g, beta), st, snapshots=False, final_state=True,
                   final_out=st)
    torch.testing.assert_close(st.cpu(), snaps_ref[:, -1], **FP32_TOL)


def test_gdn_reference_seam_signature():
    """recurrent_gated_delta_rule keeps the reference seam (already repeated heads)."""
    from lollm_amd import ops
    q, k, v, g, beta, s0 = make_inputs(2, 3, 4, 4, seed=9, dtype=torch.float32, l2=True)
    o_ref, s_ref = R.gdn_scan_recurrent(q, k, v, g, beta, s0, qk_l2=True)
    o, s = ops.recurrent_gated_delta_rule(*to_dev(q, k, v, g, beta), initial_state=s0.cuda(),
                                          use_qk_l2norm_in_kernel=True)
    torch.testing.assert_close(o.cpu(), o_ref, **FP32_TOL)
    torch.testing.assert_close(s.cpu(), s_ref, **FP32_TOL)


@pytest.mark.parametrize("k_draft", [1, 2, 4])
def test_gdn_full_size_properties(k_draft):
    """B=32, 32 v-heads / 16 qk-heads, dim 128, T = 1 + k: snapshot[-1] == final
    state, every rollback slot equals a fresh run of the accepted prefix (checked on
    the GPU itself for all sequences, and against the oracle on a sample)."""
    from lollm_amd import ops
    B, T, Hk, Hv = 32, 1 + k_draft, 16, 32
    print(f"full-size B={B} T={T}", flush=True)
    q, k, v, g, beta, s0 = make_inputs(B, T, Hk, Hv, seed=2, dtype=torch.bfloat16)
    dq, dk, dv, dg, db, ds = to_dev(q, k, v, g, beta, s0)
    out, snaps, fin = ops.gdn_verify(dq, dk, dv, dg, db, ds, final_state=True)
    assert torch.equal(snaps[:, -1], fin)
    acc = torch.randint(0, k_draft + 1, (B,), generator=torch.Generator().manual_seed(3),
                        dtype=torch.int32)
    sel = ops.gdn_select_state(snaps, acc.cuda())
    for a in range(T):
        idx = (acc == a).nonzero().flatten().cuda()
        if idx.numel() == 0:
            continue
        _, _, fa = ops.gdn_verify(dq[idx, :a + 1].contiguous(), dk[idx, :a + 1].contiguous(),
                                  dv[idx, :a + 1].contiguous(), dg[idx, :a + 1].contiguous(),
                                  db[idx, :a + 1].contiguous(), ds[idx].contiguous(),
                                  snapshots=False, final_state=True)
        torch.testing.assert_close(sel[idx], fa, rtol=1e-6, atol=1e-6)
    o_ref, snaps_ref = oracle(q[:2], k[:2], v[:2], g[:2], beta[:2], s0[:2], False)
    torch.testing.assert_close(out[:2].cpu().float(), o_ref.float(), **BF16_TOL)
    torch.testing.assert_close(snaps[:2].cpu(), snaps_ref, **BF16_TOL)
