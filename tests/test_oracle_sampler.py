"""Pins the exact sampler oracle (oracle/sampler_ref.c) on the CPU.

Checks: Philox4x32-10 against rocRAND's rounds (tests/golden/philox_kat.json) and the
published Random123 known-answer vectors; the exp2 polynomial against libm; the
top-k / top-p keep-set and kept mass against an independent brute force over sorted
keys in Python integers; greedy and q == p closed forms; and the defining property of
speculative sampling -- the emitted token is distributed as p whatever the draft q
(Leviathan et al. 2023, Theorem 1) -- by a chi-square test.
"""

import json
import math
import os

import numpy as np
import pytest

from oracle import sampler_ref as S


def test_philox_rocrand_kat(golden_dir):
    kat = json.load(open(os.path.join(golden_dir, "philox_kat.json")))
    for c in kat["cases"]:
        assert list(S.philox4x32_10(c["ctr"], c["key"])) == c["out"]


def test_philox_random123_published_vectors():
    # Random123 kat_vectors, philox4x32 R=10
    assert [hex(x) for x in S.philox4x32_10([0, 0, 0, 0], [0, 0])] == \
        ["0x6627e8d5", "0xe169c58d", "0xbc57ac4c", "0x9b00dbd8"]
    assert [hex(x) for x in S.philox4x32_10([0xffffffff] * 4, [0xffffffff] * 2)] == \
        ["0x408f276d", "0x41c83b0e", "0xa20bc7c6", "0x6d5451fd"]
    assert [hex(x) for x in S.philox4x32_10([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344],
                                            [0xa4093822, 0x299f31d0])] == \
        ["0xd16cfe09", "0x94fdcceb", "0x5001e420", "0x24126ea1"]


def test_uniform_u24_layout():
    seed, off = 0x1234_5678_9abc_def0, 77
    for row in (0, 5):
        for slot in range(6):
            words = S.philox4x32_10([row, off & 0xffffffff, off >> 32, slot >> 2],
                                    [seed & 0xffffffff, seed >> 32])
            assert S.uniform_u24(seed, off, row, slot) == int(words[slot & 3]) >> 8


def test_exp2_accuracy_and_exact_points():
    ts = np.linspace(-40.0, 0.0, 20001, dtype=np.float32)
    got = np.array([S.exp2(float(t)) for t in ts])
    rel = np.abs(got / np.exp2(ts.astype(np.float64)) - 1.0)
    assert rel.max() < 4e-7
    for n in range(0, 41):
        assert S.exp2(-float(n)) == 2.0 ** -n


def _bf16(vals):
    import torch
    return torch.tensor(vals, dtype=torch.float32).bfloat16()


def _brute_keep(x_bf16, inv_temp, top_k, top_p):
    """Independent restatement: sort distinct sampling keys descending, walk them."""
    import torch
    bits = x_bf16.view(torch.int16).numpy().astype(np.int64) & 0xFFFF
    mag = bits & 0x7FFF
    mc = np.where(mag > 0x3780, mag - 0x3780, 0)
    key = np.where(bits & 0x8000, -mc, mc)
    kmax = key.max()
    val = lambda k: 0.0 if k == 0 else float(np.array(
        [((abs(k) + 0x3780) | (0x8000 if k < 0 else 0)) << 16], dtype=np.uint32).view(np.float32)[0])
    c = float(np.float32(inv_temp) * np.float32(1.44269504088896341))
    w = {}
    for k in np.unique(key):
        if kmax - k >= 8192:
            w[k] = 0
        else:
            w[k] = S.weight(val(k), val(kmax), c)
    keys_desc = sorted(w, reverse=True)
    counts = {k: int((key == k).sum()) for k in keys_desc}
    kept = list(keys_desc)
    if top_k > 0:
        cum, kk = 0, []
        for k in keys_desc:
            kk.append(k)
            cum += counts[k]
            if cum >= top_k:
                break
        kept = kk
    W = sum(counts[k] * w[k] for k in kept)
    if 0 < top_p < 1:
        p24 = int(np.float32(top_p) * np.float32(16777216.0))
        tm = (W * p24) >> 24
        above, kk = 0, []
        for k in kept:
            if above <= tm:
                kk.append(k)
            above += counts[k] * w[k]
        kept = kk
    Z = sum(counts[k] * w[k] for k in kept)
    weights = np.array([w[k] if k in kept else 0 for k in key], dtype=np.uint64)
    return weights, Z


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("top_k,top_p", [(0, 1.0), (0, 0.95), (20, 0.8), (5, 1.0), (0, 0.3)])
def test_keep_set_matches_bruteforce(seed, top_k, top_p):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 3, size=512).astype(np.float32)
    x[rng.integers(0, 512, 60)] = x[3]                       # plenty of exact ties
    x[rng.integers(0, 512, 10)] = rng.normal(0, 1e-6, 10)    # flushed-to-zero keys
    xb = _bf16(x)
    for temp in (0.7, 1.3):
        inv = S.inv_temperature(temp)
        w_ref, Z_ref = _brute_keep(xb, inv, top_k, top_p)
        w = S.row_weights(xb, inv, top_k, top_p)
        st = S.row_stats(xb, inv, top_k, top_p)
        assert np.array_equal(w, w_ref)
        assert st["Z"] == Z_ref == int(w.sum())


def test_greedy_rules():
    x = _bf16([0.5, 2.0, -1.0, 2.0, 1.0])
    st = S.row_stats(x, 0.0)
    assert st["argmax"] == 1                                  # first maximum
    tgt = _bf16([[0.5, 2.0, -1.0, 2.0, 1.0, 0, 0, 0]] * 3).reshape(1, 3, 8)
    na, nt = S.spec_accept(tgt, None, [[1, 4]], 0.0, 0, 1.0, 1, 2)
    assert na[0] == 1 and nt[0] == 1                          # accept 1, reject 4, emit argmax
    na, nt = S.spec_accept(tgt, None, [[1, 1]], 0.0, 0, 1.0, 1, 2)
    assert na[0] == 2 and nt[0] == 1                          # all accepted, bonus = argmax


def test_q_equal_p_always_accepts():
    rng = np.random.default_rng(1)
    V, k = 256, 3
    tgt = _bf16(rng.normal(0, 2, (4, k + 1, V)))
    drafts = rng.integers(0, V, (4, k))
    inv = S.inv_temperature(0.9)
    for off in range(5):
        na, _ = S.spec_accept(tgt, tgt[:, :k].contiguous(), drafts, inv, 0, 0.9, 3, off)
        # drafts outside the keep-set have p = q = 0: u*0 < 0 is false -> rejected there
        w = [[S.row_weights(tgt[b, i], inv, 0, 0.9)[drafts[b, i]] for i in range(k)] for b in range(4)]
        for b in range(4):
            expect = 0
            while expect < k and w[b][expect] > 0:
                expect += 1
            assert na[b] == expect


def _chi2_ok(counts, probs, n):
    exp = probs * n
    m = exp > 5
    stat = (((counts[m] - exp[m]) ** 2) / exp[m]).sum()
    dof = max(int(m.sum()) - 1, 1)
    return stat < dof + 6 * math.sqrt(2 * dof)


@pytest.mark.parametrize("one_hot", [False, True])
def test_emitted_token_is_distributed_as_p(one_hot):
    """k = 1: draft d ~ q, then accept/residual; the first emitted token must follow p."""
    rng = np.random.default_rng(7)
    V = 16
    tgt = _bf16(rng.normal(0, 1.5, (1, 2, V)))
    drf = _bf16(rng.normal(0, 1.5, (1, 1, V)))
    inv = S.inv_temperature(1.0)
    p = S.row_weights(tgt[0, 0], inv, 0, 1.0).astype(np.float64)
    p /= p.sum()
    n = 6000
    counts = np.zeros(V)
    for off in range(n):
        if one_hot:
            d = int(S.sample_rows(drf[0], inv, 0, 1.0, 99, off, 0, 7)[0])
            na, nt = S.spec_accept(tgt, None, [[d]], inv, 0, 1.0, 5, off)
        else:
            d = int(S.sample_rows(drf[0], inv, 0, 1.0, 99, off, 0, 7)[0])
            na, nt = S.spec_accept(tgt, drf, [[d]], inv, 0, 1.0, 5, off)
        counts[d if na[0] == 1 else nt[0]] += 1
    assert _chi2_ok(counts, p, n)


def test_sample_rows_follows_weights():
    rng = np.random.default_rng(3)
    V = 12
    x = _bf16(rng.normal(0, 1.0, (1, V)))
    inv = S.inv_temperature(0.8)
    w = S.row_weights(x[0], inv, 0, 1.0).astype(np.float64)
    n = 5000
    counts = np.bincount([int(S.sample_rows(x, inv, 0, 1.0, 11, off)[0]) for off in range(n)],
                         minlength=V)
    assert _chi2_ok(counts, w / w.sum(), n)


def test_wrong_residual_rule_would_be_caught():
    """Planted mistake (CPU only): drawing the residual from max(0, q - p) instead of
    max(0, p - q) breaks the emitted-token distribution, so the chi-square test above
    has the power to catch it."""
    rng = np.random.default_rng(7)
    V = 16
    tgt = _bf16(rng.normal(0, 1.5, (1, 2, V)))
    drf = _bf16(rng.normal(0, 1.5, (1, 1, V)))
    inv = S.inv_temperature(1.0)
    p = S.row_weights(tgt[0, 0], inv, 0, 1.0).astype(np.float64)
    q = S.row_weights(drf[0, 0], inv, 0, 1.0).astype(np.float64)
    p, q = p / p.sum(), q / q.sum()
    wrong_resid = np.maximum(q - p, 0)
    wrong_resid /= wrong_resid.sum()
    emitted_wrong = np.minimum(p, q) + (1 - np.minimum(p, q).sum()) * wrong_resid
    n = 6000
    assert not _chi2_ok(emitted_wrong * n, p, n)
