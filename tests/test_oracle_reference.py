"""Pins the oracle to vectors written by the reference itself (CPU only).

tests/golden/make_golden_ref.py imports the giapnguyen74/lollm checkout in the build
container and records: MTP.forward at L = 1..4 and with explicit positions
(src/qwen3_5/mtp.py:61-73), speculate (mtp.py:76-89), sample_next's greedy pick under a
repetition penalty (src/generate.py:17-24), and the greedy generate_mtp / generate
trajectories (mtp.py:92-162, generate.py:40-62) on the tiny 1024-hidden model and, with
penalties 1.0 / 1.05 / 1.3, on the micro model.  Also here: the C sampler oracle's
repetition penalty against torch's own bf16 arithmetic, its top-k / top-p keep-sets
against the float rule of generate.py:26-36, and the host-side capacity checks.
"""

import os

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

from lollm_amd.qwen3_5.config import (Qwen3_5Config, micro_config_dict, tiny_config_dict)
from lollm_amd.qwen3_5.random_init import random_weights
from oracle import qwen3_5_ref as R
from oracle import sampler_ref as S


@pytest.fixture(scope="module")
def ref(golden_dir):
    return load_file(os.path.join(golden_dir, "ref_mtp.safetensors"))


def _model(raw):
    cfg = Qwen3_5Config.from_hf(raw)
    W = {k: v.to(torch.bfloat16).float() for k, v in random_weights(cfg, seed=0).items()}
    return R.canonical_weights(W), R.RefConfig.from_dict(raw)


@pytest.fixture(scope="module")
def micro():
    return _model(micro_config_dict())


@pytest.fixture(scope="module")
def tiny():
    return _model(tiny_config_dict())


@pytest.mark.parametrize("L", [1, 2, 3, 4])
@pytest.mark.parametrize("tag", ["micro", "tiny"])
def test_mtp_forward_matches_reference(ref, micro, tiny, tag, L):
    W, cfg = micro if tag == "micro" else tiny
    h, e = ref[f"{tag}.mtp{L}.hidden"], ref[f"{tag}.mtp{L}.next_emb"]
    torch.testing.assert_close(R.mtp_forward(W, cfg, h, e), ref[f"{tag}.mtp{L}.out"],
                               rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", ["mtp_pos", "mtp_pos_nc"])
@pytest.mark.parametrize("tag", ["micro", "tiny"])
def test_mtp_forward_positions_match_reference(ref, micro, tiny, tag, case):
    W, cfg = micro if tag == "micro" else tiny
    p = f"{tag}.{case}."
    got = R.mtp_forward(W, cfg, ref[p + "hidden"], ref[p + "next_emb"], ref[p + "positions"])
    torch.testing.assert_close(got, ref[p + "out"], rtol=1e-5, atol=1e-5)


def test_mtp_concat_order_is_pinned(ref, micro):
    """A swapped [hidden ; emb] concatenation (a plausible mistake) misses the fixture."""
    W, cfg = micro
    h, e = ref["micro.mtp2.hidden"], ref["micro.mtp2.next_emb"]
    W2 = dict(W)
    W2["mtp.pre_fc_norm_embedding.weight"], W2["mtp.pre_fc_norm_hidden.weight"] = (
        W["mtp.pre_fc_norm_hidden.weight"], W["mtp.pre_fc_norm_embedding.weight"])
    swapped = R.mtp_forward(W2, cfg, e, h)        # = fc([norm_h(hidden) ; norm_e(emb)])
    assert (swapped - ref["micro.mtp2.out"]).abs().max() > 1e-2


def test_speculate_matches_reference(ref, micro):
    W, cfg = micro
    torch.testing.assert_close(R.speculate(W, cfg, ref["micro.spec.ids"]), ref["micro.spec.logits"],
                               rtol=1e-4, atol=1e-4)


def test_sample_next_penalty_matches_reference(ref):
    rows, prev, picks = ref["penalty.logits"], ref["penalty.prev"], ref["penalty.pick_and_milli"]
    changed = 0
    for r in range(rows.shape[0]):
        ids = [int(t) for t in prev[r] if t >= 0]
        pen = int(picks[r, 1]) / 1000.0
        got = R.sample_next(rows[r], 0.0, 0, 1.0, pen, ids)
        assert got == int(picks[r, 0]), r
        changed += got != int(rows[r].float().argmax())
    assert changed >= 8          # the rows are built so the penalty decides the pick


@pytest.mark.parametrize("pen", [1.0, 1.05, 1.3])
def test_micro_trajectories_match_reference(ref, micro, pen):
    W, cfg = micro
    name = f"micro.pen{int(round(pen * 100))}"
    prompt = ref["micro.prompt"].tolist()
    want = ref[f"{name}.tokens"].tolist()
    spec, _ = R.generate_mtp_greedy(W, cfg, prompt, len(want), repetition_penalty=pen)
    assert spec == want
    assert R.generate_greedy(W, cfg, prompt, len(want), repetition_penalty=pen) == want
    if pen == 1.3:
        assert int(ref[f"{name}.changed_by_penalty"].sum()) > 0


def test_c1_trajectory_matches_reference(ref, tiny):
    """C1: the tiny model, 128-token prompt, 64 greedy tokens, k = 1 -- the oracle's
    speculative loop reproduces the reference's generate_mtp token for token (both fp32;
    the closest top-2 margin on the trajectory is 6e-4, far above fp32 rounding)."""
    W, cfg = tiny
    prompt = ref["c1.prompt"].tolist()
    want = ref["c1.pen100.tokens"].tolist()
    spec, acc = R.generate_mtp_greedy(W, cfg, prompt, len(want))
    assert spec == want


def test_penalty_oracle_matches_torch_bf16():
    """The C oracle's penalty is torch's bf16 arithmetic bit for bit: where(s > 0, s / p,
    s * p) on a bf16 tensor with a Python float p (generate.py:18-22)."""
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(50000, generator=g) * 5).to(torch.bfloat16)
    ids = torch.randint(0, 50000, (20000,), generator=g)
    idx = torch.tensor(sorted(set(ids.tolist())))
    for pen in (1.05, 1.1, 1.3, 0.9, 2.0, 0.77, 1.0):
        got = S.repetition_penalty(x, ids.numpy(), pen)
        want = x.clone()
        s = want[idx]
        want[idx] = torch.where(s > 0, s / pen, s * pen)
        np.testing.assert_array_equal(got, want.view(torch.int16).numpy().view(np.uint16))


def test_penalty_oracle_planted_mistake_fails():
    """Penalising each occurrence instead of each distinct token (a plausible mistake)
    changes tokens that occur twice."""
    x = torch.tensor([2.0, -1.0, 3.0, 0.5]).to(torch.bfloat16)
    once = S.repetition_penalty(x, [0, 0, 1], 1.3)
    twice = S.repetition_penalty(torch.from_numpy(once.view(np.int16)).view(torch.bfloat16),
                                 [0], 1.3)
    assert once[0] != twice[0] and once[2] == S._bits(x)[2]


def _float_keep(x, inv_temp, top_p):
    """generate.py:25-36 in float64 with ties kept together: keep a token iff the mass of
    the tokens with strictly larger logits is <= top_p; also returns that mass."""
    z = x.double() * inv_temp
    p = torch.softmax(z, 0)
    order = torch.argsort(z, descending=True, stable=True)
    ps, zs = p[order], z[order]
    above = torch.zeros_like(ps)
    # mass strictly above each sorted position: cumulative mass before its tie group
    cum = torch.cumsum(ps, 0) - ps
    first = torch.ones_like(zs, dtype=torch.bool)
    first[1:] = zs[1:] != zs[:-1]
    grp = torch.cumsum(first.long(), 0) - 1
    starts = cum[first]
    above = starts[grp]
    keep = torch.empty_like(above, dtype=torch.bool)
    keep[order] = above <= top_p
    mass = torch.empty_like(above)
    mass[order] = above
    return keep, mass


@pytest.mark.parametrize("top_p", [0.5, 0.8, 0.95])
def test_c_keep_set_matches_float_top_p_rule(top_p):
    """The exact integer keep-set of the C oracle equals the float top-p rule except for
    tokens whose mass-above lies within 1e-5 of top_p (exp2 polynomial and integer
    weights; the flushed |x| <= 2^-16 keys and tokens 8192 keys below the maximum carry
    less mass than that)."""
    g = torch.Generator().manual_seed(int(top_p * 100))
    inv_t = S.inv_temperature(0.7)
    kept = 0
    for r in range(6):
        x = (torch.randn(4096, generator=g) * (3.0 if r % 2 else 0.5)).to(torch.bfloat16)
        w = S.row_weights(x, inv_t, 0, top_p)
        keep_c = torch.from_numpy(w.astype(np.float64) > 0)
        keep_f, mass = _float_keep(x.float(), inv_t, top_p)
        diff = keep_c != keep_f
        assert not bool((diff & ((mass - top_p).abs() > 1e-5)).any()), r
        kept += int(keep_c.sum())
    assert kept > 100                    # the flat rows keep many tokens


def test_c_top_k_matches_float_rule():
    g = torch.Generator().manual_seed(8)
    for top_k in (1, 5, 40):
        x = (torch.randn(4096, generator=g) * 3).to(torch.bfloat16)
        x[7] = x[9]                                   # a tie
        w = S.row_weights(x, S.inv_temperature(1.0), top_k, 1.0)
        kth = torch.topk(x.float(), top_k).values[-1]
        np.testing.assert_array_equal(w > 0, (x.float() >= kth).numpy())


# ---------------------------------------------------------------------------------------
# capacity: the host raises before a kernel could drop rows
# ---------------------------------------------------------------------------------------
def _cpu_cache(max_len):
    from lollm_amd.qwen3_5.kv import Qwen3_5Cache
    cfg = Qwen3_5Config.from_hf(micro_config_dict())
    return Qwen3_5Cache(cfg, 2, max_len, spec_slots=4, device="cpu")


def test_cache_reserve_raises_past_max_len():
    c = _cpu_cache(8)
    c.reserve(8)
    c.lengths[:] = torch.tensor([6, 3], dtype=torch.int32)
    c.grew(6)
    c.reserve(2)
    with pytest.raises(RuntimeError, match="capacity"):
        c.reserve(3)
    with pytest.raises(RuntimeError, match="capacity"):
        c.advance(3)
    # a stale (too high) bound is refreshed from the device lengths before raising
    c.len_bound = 8
    c.reserve(2)
    assert c.len_bound == 6


def test_spec_step_capacity_raises():
    """SpecDecoder refuses a step whose k + 1 tokens might not fit the cache or the
    output buffer (the host bounds; exact device values are read before raising)."""
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    d = SpecDecoder.__new__(SpecDecoder)
    d.k, d.cache = 3, _cpu_cache(12)
    d.out_capacity, d.out_bound = 8, 0
    d.out_count = torch.zeros(2, dtype=torch.int32)
    d._reserve()
    d._grew()
    d._reserve()                                   # bounds 4 + 4 <= 8 and 4 + 4 <= 12
    d._grew()
    d._reserve()                                   # out bound 8 is refreshed to 0
    assert d.out_bound == 0
    d.out_count[:] = torch.tensor([6, 1], dtype=torch.int32)
    d.out_bound = 6
    with pytest.raises(RuntimeError, match="output capacity"):
        d._reserve()
    d.out_count.zero_()
    d.out_bound = 0
    d.cache.lengths[:] = torch.tensor([9, 2], dtype=torch.int32)
    d.cache.len_bound = 9
    with pytest.raises(RuntimeError, match="capacity"):
        d._reserve()


def test_sorted_acceptance_agrees_with_exact_oracle():
    """The float restatement of acceptance (the CPU baseline's algorithm, sort-based as
    generate.py:26-36) against the exact integer C oracle on the same rows and uniforms:
    identical at temperature 0; with sampling, identical except where a uniform falls
    within float rounding of a CDF boundary (a few rows at most)."""
    g = torch.Generator().manual_seed(40)
    B, k, V = 32, 3, 4096
    tgt = (torch.randn(B, k + 1, V, generator=g) * 3).bfloat16()
    drafts = tgt[:, :k].float().argmax(-1)
    drafts[::2, 1] = torch.randint(0, V, (B // 2,), generator=g)     # some rejections
    seed, off = 5, 2
    U = torch.tensor([[S.uniform_u24(seed, off, b, s) for s in range(k + 1)] for b in range(B)],
                     dtype=torch.float64) / 2 ** 24
    drf = (tgt[:, :k].float() + torch.randn(B, k, V, generator=g)).bfloat16()
    for temp, top_p, dl in ((0.0, 1.0, None), (0.7, 0.95, None), (1.0, 0.8, None), (0.7, 0.95, drf)):
        inv = S.inv_temperature(temp)
        na_c, nt_c = S.spec_accept(tgt, dl, drafts.numpy().astype(np.int32), inv, 0, top_p, seed, off)
        na_f, nt_f = R.spec_accept_sorted(tgt.float(), drafts, temp, 0, top_p, U,
                                          None if dl is None else dl.float())
        agree = (torch.from_numpy(na_c.astype(np.int64)) == na_f) & (torch.from_numpy(nt_c.astype(np.int64)) == nt_f)
        if temp == 0.0:
            assert bool(agree.all())
        else:
            assert int(agree.sum()) >= B - 2, (temp, int(agree.sum()))
