"""GPU speculative sampler vs the exact C oracle: accept counts, emitted tokens and
row draws must be bit-exact (identical logits and Philox uniforms)."""

import numpy as np
import pytest
import torch

from oracle import sampler_ref as S

pytestmark = pytest.mark.gpu


def acceptance_case(B, k, V, seed, noise=1.0, scale=3.0):
    """The isolated acceptance workload: target = bf16(N(0, scale^2)), draft =
    bf16(target[:, :k] + N(0, noise^2))."""
    gen = torch.Generator().manual_seed(seed)
    tgt = torch.randn(B, k + 1, V, generator=gen) * scale
    drf = tgt[:, :k] + torch.randn(B, k, V, generator=gen) * noise
    return tgt.bfloat16(), drf.bfloat16()


def test_philox_matches_oracle():
    from lollm_amd import ops
    seed, off = 0x0123_4567_89ab_cdef, 3 << 33 | 5
    u = ops.philox_u24(seed, off, 70, 9).cpu().numpy().astype(np.int64)
    for r in range(70):
        for s in range(9):
            assert u[r, s] == S.uniform_u24(seed, off, r, s)


@pytest.mark.parametrize("temp,top_k,top_p", [(0.7, 0, 0.95), (0.7, 20, 0.8), (1.0, 0, 1.0),
                                              (0.0, 0, 1.0), (1.7, 50, 0.5)])
def test_sample_rows_bit_exact(temp, top_k, top_p):
    from lollm_amd import ops
    print(f"case sample_rows T={temp} top_k={top_k} top_p={top_p}", flush=True)
    tgt, _ = acceptance_case(8, 3, 151936, seed=4)
    rows = tgt.reshape(-1, 151936).contiguous()
    inv = S.inv_temperature(temp)
    for off in (0, 1, 12345):
        ref = S.sample_rows(rows, inv, top_k, top_p, 99, off, row_base=2, slot=5)
        got = ops.sample_rows(rows.cuda(), temp, top_k, top_p, 99, off, row_base=2, slot=5)
        assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("with_draft", [True, False])
@pytest.mark.parametrize("temp,top_k,top_p", [(0.7, 0, 0.95), (0.7, 20, 0.8), (0.0, 0, 1.0)])
def test_spec_accept_bit_exact_full_vocab(with_draft, temp, top_k, top_p):
    """B=64, k=3, V=151936 (the isolated acceptance shape); drafts are drawn from the
    draft rows with the same Philox stream (slot k+1+i), as a sampling draft chain does."""
    from lollm_amd import ops
    print(f"case accept draft={with_draft} T={temp} top_k={top_k} top_p={top_p}", flush=True)
    B, k, V = 64, 3, 151936
    tgt, drf = acceptance_case(B, k, V, seed=4)
    inv = S.inv_temperature(temp)
    drafts = np.stack([S.sample_rows(drf[:, i].contiguous(), inv, top_k, top_p, 7, 0, 0, k + 1 + i)
                       for i in range(k)], 1).astype(np.int32)
    if not with_draft:
        drf = None
    for off in (0, 9):
        na_ref, nt_ref = S.spec_accept(tgt, drf, drafts, inv, top_k, top_p, 7, off)
        na, nt = ops.spec_accept(tgt.cuda(), None if drf is None else drf.cuda(),
                                 torch.from_numpy(drafts).cuda(), temp, top_k, top_p, 7, off)
        assert np.array_equal(na.cpu().numpy(), na_ref)
        assert np.array_equal(nt.cpu().numpy(), nt_ref)


def order_key_slots(x, slots=5, at=2):
    """The row-maximum slots lollm_gemm_logits writes, built on the host for rows x
    (rows, V) bf16: slot `at` holds each row's largest order key (bf16 bits b:
    b & 0x8000 ? ~b & 0xFFFF : b | 0x8000), the other slots lower keys (0 and the row's
    first key), so the consumer must take the maximum over all of them."""
    b = x.reshape(-1, x.shape[-1]).view(torch.int16).int() & 0xFFFF
    o = torch.where((b & 0x8000) != 0, (~b) & 0xFFFF, b | 0x8000)
    out = torch.zeros(o.shape[0], slots, dtype=torch.int32)
    out[:, at] = o.max(-1).values
    out[:, (at + 1) % slots] = o[:, 0]
    return torch.where(out >= 32768, out - 65536, out).to(torch.int16)


@pytest.mark.parametrize("with_draft", [True, False])
@pytest.mark.parametrize("temp,top_k,top_p", [(0.7, 0, 0.95), (0.7, 20, 0.8), (1.7, 50, 0.5)])
def test_spec_accept_rowmax_bit_exact(with_draft, temp, top_k, top_p):
    """lollm_spec_accept_rowmax (the target rows' maxima given, each row read once) on the
    full-vocabulary acceptance workload, and on rows whose logits are all negative (the
    order-key maximum), equals the C oracle bit for bit."""
    from lollm_amd import ops
    print(f"case accept rowmax draft={with_draft} T={temp} top_k={top_k} top_p={top_p}", flush=True)
    B, k, V = 64, 3, 151936
    tgt, drf = acceptance_case(B, k, V, seed=5)
    tgt[:3] = -(tgt[:3].float().abs() + 0.01).bfloat16()       # rows with no logit >= 0
    inv = S.inv_temperature(temp)
    drafts = np.stack([S.sample_rows(drf[:, i].contiguous(), inv, top_k, top_p, 7, 0, 0, k + 1 + i)
                       for i in range(k)], 1).astype(np.int32)
    if not with_draft:
        drf = None
    rm = order_key_slots(tgt).cuda()
    for off in (0, 9):
        na_ref, nt_ref = S.spec_accept(tgt, drf, drafts, inv, top_k, top_p, 7, off)
        na, nt = ops.spec_accept(tgt.cuda(), None if drf is None else drf.cuda(),
                                 torch.from_numpy(drafts).cuda(), temp, top_k, top_p, 7, off,
                                 target_rowmax=rm)
        assert np.array_equal(na.cpu().numpy(), na_ref)
        assert np.array_equal(nt.cpu().numpy(), nt_ref)


@pytest.mark.parametrize("with_draft", [True, False])
def test_spec_accept_rowmax_vocab_beyond_register_rows(with_draft):
    """A vocabulary larger than the rows the given-maxima statistics kernel holds in
    registers (20 x 1024 chunks of 8 = 163840 tokens): the rest of each row is counted
    from a second batch of loads.  Bit-exact against the C oracle."""
    from lollm_amd import ops
    print(f"case accept rowmax V=172032 draft={with_draft}", flush=True)
    B, k, V = 8, 2, 172032
    tgt, drf = acceptance_case(B, k, V, seed=6)
    tgt[1, :, 170000] = 30.0                                  # the maximum in the tail
    inv = S.inv_temperature(0.8)
    drafts = np.stack([S.sample_rows(drf[:, i].contiguous(), inv, 0, 0.9, 3, 0, 0, k + 1 + i)
                       for i in range(k)], 1).astype(np.int32)
    if not with_draft:
        drf = None
    rm = order_key_slots(tgt).cuda()
    for off in (0, 5):
        na_ref, nt_ref = S.spec_accept(tgt, drf, drafts, inv, 0, 0.9, 3, off)
        na, nt = ops.spec_accept(tgt.cuda(), None if drf is None else drf.cuda(),
                                 torch.from_numpy(drafts).cuda(), 0.8, 0, 0.9, 3, off,
                                 target_rowmax=rm)
        assert np.array_equal(na.cpu().numpy(), na_ref)
        assert np.array_equal(nt.cpu().numpy(), nt_ref)


def test_spec_accept_small_vocab_ties_and_edges():
    """Tiny vocabulary with heavy ties, flushed keys and argmax-drawn drafts; many
    offsets so accepts, residual draws and bonus draws all occur."""
    from lollm_amd import ops
    rng = np.random.default_rng(0)
    B, k, V = 16, 4, 64
    x = rng.normal(0, 1.0, (B, k + 1, V)).astype(np.float32)
    x[..., :8] = x[..., 8:9]
    x[..., 60:] = 1e-7
    tgt = torch.from_numpy(x).bfloat16()
    drf = (tgt[:, :k].float() + torch.from_numpy(rng.normal(0, 0.3, (B, k, V)).astype(np.float32))).bfloat16()
    drafts = drf.float().argmax(-1).int().numpy()
    seen = set()
    for off in range(12):
        for d in (drf, None):
            na_ref, nt_ref = S.spec_accept(tgt, d, drafts, S.inv_temperature(0.9), 0, 0.9, 3, off)
            na, nt = ops.spec_accept(tgt.cuda(), None if d is None else d.cuda(),
                                     torch.from_numpy(drafts).cuda(), 0.9, 0, 0.9, 3, off)
            assert np.array_equal(na.cpu().numpy(), na_ref)
            assert np.array_equal(nt.cpu().numpy(), nt_ref)
            seen.update(int(a) for a in na_ref)
    assert len(seen) >= 3                   # several acceptance lengths were exercised


def test_offset_from_device_memory():
    from lollm_amd import ops
    tgt, drf = acceptance_case(4, 3, 4096, seed=1)
    drafts = torch.randint(0, 4096, (4, 3), dtype=torch.int32)
    off = torch.tensor([41], dtype=torch.int64).cuda()
    a = ops.spec_accept(tgt.cuda(), drf.cuda(), drafts.cuda(), 0.7, 0, 0.95, 5, 41)
    b = ops.spec_accept(tgt.cuda(), drf.cuda(), drafts.cuda(), 0.7, 0, 0.95, 5, 0, offset_dev=off)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_spec_accept_full_vocab_late_rejections_and_bonus():
    """Full vocabulary with drafts at a dominant logit for the first j_b positions of
    sequence b and a flat row after: rejections at every position 0..k and all-accepted
    bonus draws both occur (the C4 workload itself rejects almost always at 0)."""
    from lollm_amd import ops
    B, k, V = 16, 3, 151936
    gen = torch.Generator().manual_seed(21)
    x = torch.randn(B, k + 1, V, generator=gen) * 3
    drafts = torch.randint(0, V, (B, k), generator=gen, dtype=torch.int32)
    for b in range(B):
        j = b % (k + 1)                       # positions < j are near-certain accepts
        for i in range(j):
            x[b, i, drafts[b, i]] = 60.0
    tgt = x.bfloat16()
    inv = S.inv_temperature(0.7)
    seen = set()
    for off in (0, 5):
        na_ref, nt_ref = S.spec_accept(tgt, None, drafts.numpy(), inv, 0, 0.95, 13, off)
        na, nt = ops.spec_accept(tgt.cuda(), None, drafts.cuda(), 0.7, 0, 0.95, 13, off)
        assert np.array_equal(na.cpu().numpy(), na_ref)
        assert np.array_equal(nt.cpu().numpy(), nt_ref)
        seen.update(int(a) for a in na_ref)
    assert seen == set(range(k + 1))


@pytest.mark.parametrize("temp", [0.0, 0.8])
def test_sample_rows_vocab_beyond_register_rows(temp):
    """A 200000-token vocabulary, larger than the test workloads elsewhere, with the
    maximum of one row far into the part the statistics kernel counts as it streams
    (past its first 8 chunks of 8 tokens per thread)."""
    from lollm_amd import ops
    V = 200000
    gen = torch.Generator().manual_seed(5)
    x = (torch.randn(3, V, generator=gen) * 3)
    x[1, 190000] = 40.0                      # the maximum in the tail
    rows = x.bfloat16()
    inv = S.inv_temperature(temp)
    for off in (0, 3):
        ref = S.sample_rows(rows, inv, 0, 0.9, 17, off, row_base=0, slot=1)
        got = ops.sample_rows(rows.cuda(), temp, 0, 0.9, 17, off, row_base=0, slot=1)
        assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("temp,top_k,top_p", [(0.7, 0, 0.95), (0.8, 0, 1.0), (1.3, 40, 0.9)])
def test_sample_rows_negative_and_extreme_rows(temp, top_k, top_p):
    """Rows the statistics kernel treats specially: every logit negative (the maximum is
    taken over order keys), only -0 and negatives, a +inf or NaN maximum (every weight
    zero), and a dominant logit far above the rest (without top-k most tokens fail the
    weight test and are not counted)."""
    from lollm_amd import ops
    print(f"case extreme rows T={temp} top_k={top_k} top_p={top_p}", flush=True)
    V = 151936
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(7, V, generator=gen) * 3
    x[0] = -x[0].abs() - 0.25                       # all negative
    x[1] = -x[1].abs()
    x[1, ::3] = -0.0                                # -0 is the maximum
    x[2, 777] = float("inf")
    x[3, 5] = float("nan")
    x[4, 123456] = 80.0                             # far above the rest
    x[5] = -x[5].abs() * 10 - 30.0
    x[5, 99] = -2.0                                 # negative maximum far above the rest
    x[6] = -1e-6                                    # every key flushed to 0: a flat row
    rows = x.bfloat16()
    inv = S.inv_temperature(temp)
    for off in (0, 4):
        ref = S.sample_rows(rows, inv, top_k, top_p, 23, off, row_base=1, slot=2)
        got = ops.sample_rows(rows.cuda(), temp, top_k, top_p, 23, off, row_base=1, slot=2)
        assert np.array_equal(got.cpu().numpy(), ref)


@pytest.mark.parametrize("temp,top_k,top_p", [(0.7, 0, 0.95), (1.3, 40, 0.9)])
def test_sample_rows_maximum_above_the_count_window(temp, top_k, top_p):
    """The statistics kernel counts keys in one pass over a window placed by the maximum
    of each thread's first 8 chunks (the first 65536 tokens); a row whose maximum lies
    more than 8192 keys above that is counted again: a far larger finite maximum, +inf
    and NaN past the first 65536 tokens, and a maximum exactly at the window's edge."""
    from lollm_amd import ops
    print(f"case window edge rows T={temp} top_k={top_k} top_p={top_p}", flush=True)
    V = 151936
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(5, V, generator=gen) * 3
    x[0, :65536] = -1.0e30                          # far below the rest: second pass
    x[1, 150000] = float("inf")
    x[2, 100000] = float("nan")
    # row 3: the first 65536 tokens at one key, a maximum exactly 8192 keys above it
    # (the last key the window holds), row 4 one key past it
    lo = 0x3F80                                     # bf16 1.0
    x[3, :65536] = 1.0
    x[4, :65536] = 1.0
    x[3, 65536:] = 0.5
    x[4, 65536:] = 0.5
    x[3, 70000] = torch.tensor([lo + 8192], dtype=torch.int16).view(torch.bfloat16).float()
    x[4, 70000] = torch.tensor([lo + 8193], dtype=torch.int16).view(torch.bfloat16).float()
    rows = x.bfloat16()
    inv = S.inv_temperature(temp)
    for off in (0, 2):
        ref = S.sample_rows(rows, inv, top_k, top_p, 29, off, row_base=0, slot=0)
        got = ops.sample_rows(rows.cuda(), temp, top_k, top_p, 29, off, row_base=0, slot=0)
        assert np.array_equal(got.cpu().numpy(), ref)
