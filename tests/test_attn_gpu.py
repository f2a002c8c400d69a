"""Gated GQA verify attention vs the oracle (src/attention.py:43-51 offset-causal SDPA
+ src/qwen3_5/blocks.py:229-235 GQA expansion and sigmoid gate), restated in
oracle/qwen3_5_ref.py.  The oracle runs in fp32 on the same bf16 inputs; the kernel
output is bf16, so the tolerance is bf16's (rtol 2e-2, atol 2e-2)."""

import pytest
import torch

from oracle import qwen3_5_ref as R

pytestmark = pytest.mark.gpu
TOL = dict(rtol=2e-2, atol=2e-2)
D = 256


def make_case(B, T, Hq, Hkv, lens, seed, max_len=None, nan_tail=True):
    gen = torch.Generator().manual_seed(seed)
    max_len = max_len or max(lens)
    q = torch.randn(B, T, Hq, D, generator=gen).bfloat16()
    kc = torch.randn(B, Hkv, max_len, D, generator=gen).bfloat16()
    vc = torch.randn(B, Hkv, max_len, D, generator=gen).bfloat16()
    if nan_tail:                        # junk beyond each sequence's length must not leak
        for b, L in enumerate(lens):
            kc[b, :, L:] = float("nan")
            vc[b, :, L:] = float("nan")
    gate = torch.randn(B, T, Hq * D, generator=gen).bfloat16()
    return q, kc, vc, torch.tensor(lens, dtype=torch.int32), gate


def oracle(q, kc, vc, lens, gate):
    B, T, Hq, _ = q.shape
    Hkv = kc.shape[1]
    rep = Hq // Hkv
    outs = []
    for b in range(B):
        L = int(lens[b])
        o = torch.empty(1, Hq, T, D)
        for g in range(Hkv):
            qq = q[b, :, g * rep:(g + 1) * rep].float().transpose(0, 1)[None]   # (1,rep,T,D)
            kk = kc[b, g, :L].float()[None, None].expand(1, rep, L, D)
            vv = vc[b, g, :L].float()[None, None].expand(1, rep, L, D)
            o[:, g * rep:(g + 1) * rep] = R.sdpa_offset_causal(qq, kk, vv)
        o = o.transpose(1, 2).reshape(T, Hq * D)
        if gate is not None:
            o = o * torch.sigmoid(gate[b].float())
        outs.append(o)
    return torch.stack(outs)


CASES = [
    # B, T, Hq, Hkv, lens, grid (workgroups of the balanced split; 0 = one per CU)
    (3, 4, 16, 2, [4, 37, 700], 0),            # plain causal, whole pairs and cut pairs
    (2, 1, 8, 2, [1, 1000], 5),                # decode, a long pair cut in many pieces
    (2, 2, 8, 2, [2, 129], 3),                 # k = 1 verify, n_rep = 4
    (2, 8, 16, 2, [8, 300], 4),                # two query blocks (n_rep 8 x 4 queries)
    (4, 1, 32, 4, [1, 2, 3, 4], 0),            # MTP draft block: tiny causal contexts
    (2, 4, 4, 2, [5, 64], 2),                  # n_rep 2
    (5, 3, 8, 2, [3, 64, 65, 190, 7], 7),      # ranges spanning several sequences
    (3, 4, 16, 2, [4, 600, 130], 1),           # one workgroup walks every pair
    (3, 4, 16, 2, [4, 600, 130], 1024),        # more workgroups than blocks
]


@pytest.mark.parametrize("B,T,Hq,Hkv,lens,grid", CASES)
@pytest.mark.parametrize("gated", [True, False])
def test_attn_verify_matches_oracle(B, T, Hq, Hkv, lens, grid, gated):
    from lollm_amd import ops
    print(f"case B={B} T={T} Hq={Hq} Hkv={Hkv} lens={lens} grid={grid} gated={gated}", flush=True)
    q, kc, vc, kl, gate = make_case(B, T, Hq, Hkv, lens, seed=sum(lens) + T)
    ref = oracle(q, kc, vc, kl, gate if gated else None)
    out = ops.attn_verify(q.cuda(), kc.cuda(), vc.cuda(), kl.cuda(),
                          gate.cuda() if gated else None, grid=grid)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.cpu().float(), ref, **TOL)


def test_attn_verify_long_ragged_contexts():
    """The isolated verify shape: 16 q / 2 kv heads, dim 256, 1 + k = 4 queries, ragged
    contexts drawn from U[1024, 32768] (4 sequences here to keep the CPU oracle fast;
    the full 16-sequence batch runs in the benchmark)."""
    from lollm_amd import ops
    gen = torch.Generator().manual_seed(3)
    lens = torch.randint(1024, 32769, (4,), generator=gen).tolist()
    q, kc, vc, kl, gate = make_case(4, 4, 16, 2, lens, seed=3, max_len=32768)
    ref = oracle(q, kc, vc, kl, gate)
    out = ops.attn_verify(q.cuda(), kc.cuda(), vc.cuda(), kl.cuda(), gate.cuda())
    torch.testing.assert_close(out.cpu().float(), ref, **TOL)


def test_attn_split_invariance():
    """The split-K combine must not change the answer: one workgroup per pair, pairs
    cut in a few pieces, and pairs cut in dozens of pieces agree."""
    from lollm_amd import ops
    q, kc, vc, kl, gate = make_case(2, 4, 16, 2, [900, 2000], seed=8)
    outs = [ops.attn_verify(q.cuda(), kc.cuda(), vc.cuda(), kl.cuda(), gate.cuda(), grid=g)
            for g in (4, 9, 64)]
    for o in outs[1:]:
        torch.testing.assert_close(o.float(), outs[0].float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("Hq,Hkv,base,grid", [(16, 2, [1000, 37, 700], 0), (32, 4, [2048, 2049, 130], 7),
                                            (8, 2, [1, 300, 129], 0)])
def test_attn_rows_do_not_depend_on_T(Hq, Hkv, base, grid):
    """Query i of a verify call over T = 4 positions and of a call over only the first
    t <= 4 positions (the history a rollback keeps) sees the same keys, and gets the same
    bits: every row keeps its own running maximum (the rescale decision is per row), so
    the other rows of its pair -- the later queries, or padding -- do not change it.
    Contexts are chosen so both calls deal the same key blocks out to the workgroups."""
    from lollm_amd import ops
    print(f"case attn rows Hq={Hq} Hkv={Hkv} base={base} grid={grid}", flush=True)
    B, T = len(base), 4
    q, kc, vc, kl, gate = make_case(B, T, Hq, Hkv, [b + T for b in base], seed=sum(base) + Hq)
    full = ops.attn_verify(q.cuda(), kc.cuda(), vc.cuda(), kl.cuda(), gate.cuda(), grid=grid)
    for t in (1, 2, 3):
        assert all((b + t + 127) // 128 == (b + T + 127) // 128 for b in base)
        part = ops.attn_verify(q[:, :t].contiguous().cuda(), kc.cuda(), vc.cuda(),
                               (kl - (T - t)).cuda(), gate[:, :t].contiguous().cuda(), grid=grid)
        assert torch.equal(part.cpu(), full[:, :t].cpu()), t


def test_attn_workspace_is_validated():
    """A workspace smaller than lollm_attn_workspace_bytes is refused, not overrun."""
    from lollm_amd import ops
    q, kc, vc, kl, gate = make_case(2, 4, 16, 2, [90, 200], seed=9)
    need = ops.attn_workspace_bytes(2, 4, 16, 2, D, 200, 8)
    small = torch.empty(need - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(RuntimeError):
        ops.attn_verify(q.cuda(), kc.cuda(), vc.cuda(), kl.cuda(), gate.cuda(), grid=8,
                        workspace=small)


@pytest.mark.parametrize("B,Hq,Hkv,rd,lens,rope", [(4, 32, 4, 64, [1, 2, 3, 3], False),
                                                  (3, 16, 2, 128, [1, 9, 16], True),
                                                  (2, 8, 8, 0, [5, 1], False)])
def test_attn_small_equals_prologue_then_verify(B, Hq, Hkv, rd, lens, rope):
    """lollm_attn_small (one token over a cache of at most 16 rows, prologue fused: the
    MTP head's draft block) against lollm_attn_prologue + lollm_attn_verify on the same
    qkv row and cache: the appended k / v rows bit for bit, the gated output within one
    bf16 rounding (the two differ only in the order of the dot-product sums), and both
    against the oracle's fp32 attention of the prologue's q."""
    from lollm_amd import ops
    print(f"case attn_small B={B} Hq={Hq} Hkv={Hkv} lens={lens}", flush=True)
    gen = torch.Generator().manual_seed(sum(lens) + Hq)
    max_len = 16
    qkv = torch.randn(B, 1, Hq * 2 * D + 2 * Hkv * D, generator=gen).bfloat16().cuda()
    qn = (0.1 * torch.randn(D, generator=gen)).bfloat16().cuda()
    kn = (0.1 * torch.randn(D, generator=gen)).bfloat16().cuda()
    inv_freq = (1.0 / (1e7 ** (torch.arange(0, max(rd, 2), 2).float() / max(rd, 2)))).cuda()
    kv_len = torch.tensor(lens, dtype=torch.int32).cuda()
    lengths = kv_len - 1                        # the new token goes to row kv_len - 1
    rope_pos = (kv_len + 3).int() if rope else None
    kc0 = torch.randn(B, Hkv, max_len, D, generator=gen).bfloat16().cuda()
    vc0 = torch.randn(B, Hkv, max_len, D, generator=gen).bfloat16().cuda()
    kc1, vc1 = kc0.clone(), vc0.clone()
    got = ops.attn_small(qkv, qn, kn, inv_freq, lengths, kv_len, B, Hq, Hkv, D, rd, 1e-6, kc1, vc1,
                         rope_pos=rope_pos)
    kc2, vc2 = kc0.clone(), vc0.clone()
    q, gate = ops.attn_prologue(qkv, qn, kn, inv_freq, lengths, B, 1, Hq, Hkv, D, rd, 1e-6, kc2, vc2,
                                rope_pos=rope_pos)
    ref = ops.attn_verify(q, kc2, vc2, kv_len, gate)
    torch.cuda.synchronize()
    assert torch.equal(kc1.cpu(), kc2.cpu()) and torch.equal(vc1.cpu(), vc2.cpu())
    g32, r32 = got.float().cpu(), ref.float().cpu()
    torch.testing.assert_close(g32, r32, rtol=1e-2, atol=1e-2)
    assert (g32 != r32).float().mean().item() <= 0.02
    o = oracle(q.cpu(), kc2.cpu(), vc2.cpu(), kv_len.cpu(), gate.cpu())
    torch.testing.assert_close(g32.view(B, -1), o.view(B, -1), **TOL)


def test_attn_verify_c3_full_batch():
    """The isolated verify workload at full size: B = 16, 1 + k = 4 queries, 16 q / 2 kv
    heads of 256, contexts U[1024, 32768] (seeded).  Four sequences spread over the batch
    against the oracle; all 16 through split invariance (the balanced split deals the
    blocks of all sequences out together, so a grid change moves every cut)."""
    from lollm_amd import ops
    gen = torch.Generator().manual_seed(33)
    lens = torch.randint(1024, 32769, (16,), generator=gen).tolist()
    q, kc, vc, kl, gate = make_case(16, 4, 16, 2, lens, seed=33, max_len=32768)
    qd, kd, vd, ld, gd = q.cuda(), kc.cuda(), vc.cuda(), kl.cuda(), gate.cuda()
    outs = [ops.attn_verify(qd, kd, vd, ld, gd, grid=g).float().cpu() for g in (0, 37, 1024)]
    for o in outs[1:]:
        torch.testing.assert_close(o, outs[0], rtol=1e-2, atol=1e-2)
    pick = [0, 5, 10, 15]
    ref = oracle(q[pick], kc[pick], vc[pick], kl[pick], gate[pick])
    torch.testing.assert_close(outs[0][pick], ref, **TOL)
