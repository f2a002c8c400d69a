"""The MI355X model, MTP head and speculative decoder vs the oracle.

Float outputs are held to the bf16 bar.  The oracle runs twice on the same
bf16-rounded weights: in fp32 (the truth) and in bf16 with the reference's dtype flow.
The build's bf16 logits must satisfy
    max |got - ref32| <= 2 * max |ref16 - ref32| + 1e-3 * max |ref32|
(no worse than twice the reference's own bf16 error; on these models that error is
about 2% of the logit range, i.e. the rtol 2e-2 bar) and, per row,
    1 - cos(got, ref32) <= max(2 * (1 - cos(ref16, ref32)), 1e-3)
(the reference's parity gate uses cosine > 0.9999 in fp32, compare_logits.py:130).  Token-level checks use greedy
decoding, where ties are the only legitimate source of disagreement.
"""

import pytest
import torch

from lollm_amd.qwen3_5.config import Qwen3_5Config, micro_config_dict
from lollm_amd.qwen3_5.random_init import random_weights
from oracle import qwen3_5_ref as R

pytestmark = pytest.mark.gpu


def close_logits(got, ref, ref16):
    got = got.float().cpu().reshape(-1, got.shape[-1])
    ref = ref.float().reshape(-1, ref.shape[-1])
    ref16 = ref16.float().reshape(-1, ref.shape[-1])
    scale = ref.abs().max().item()
    cs = torch.nn.functional.cosine_similarity
    deficit = (1 - cs(got, ref, dim=-1)).max().item()
    ref_deficit = (1 - cs(ref16, ref, dim=-1)).max().item()
    assert deficit <= max(2 * ref_deficit, 1e-3), f"1-cos {deficit:.3g} vs reference bf16 {ref_deficit:.3g}"
    err = (got - ref).abs().max().item()
    budget = 2 * (ref16 - ref).abs().max().item() + 1e-3 * scale
    assert err <= budget, f"max err {err:.4g} > budget {budget:.4g} (scale {scale:.3g})"


def build(raw, seed=0):
    from lollm_amd.qwen3_5 import load, load_mtp
    cfg = Qwen3_5Config.from_hf(raw)
    W = random_weights(cfg, seed=seed)
    Wb = {k: v.to(torch.bfloat16) for k, v in W.items()}       # both sides use bf16 weights
    ref_W = R.canonical_weights({k: v.float() for k, v in Wb.items()})
    ref_W16 = R.canonical_weights(dict(Wb))
    ref_cfg = R.RefConfig.from_dict(raw)
    weights = dict(Wb)
    model = load(raw, weights, "hf", device="cuda")
    mtp = load_mtp(model, weights, "hf", device="cuda")
    return model, mtp, (ref_W, ref_W16), ref_cfg


@pytest.fixture(scope="module")
def micro():
    return build(micro_config_dict())


def test_forward_prefill_decode_verify(micro):
    model, _, (W, W16), cfg = micro
    print("case micro forward", flush=True)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, cfg.vocab_size, (2, 9), generator=g)
    steps = torch.randint(0, cfg.vocab_size, (2, 6), generator=g)
    cache = model.new_cache(2, 64, spec_slots=4)
    lg, _ = model(prompt.cuda(), cache)
    ref, past = R.model_forward(W, cfg, prompt)
    r16, p16 = R.model_forward(W16, cfg, prompt)
    close_logits(lg, ref, r16)
    lg, _ = model(steps[:, :1].cuda(), cache)                  # decode T=1
    ref, past = R.model_forward(W, cfg, steps[:, :1], past)
    r16, p16 = R.model_forward(W16, cfg, steps[:, :1], p16)
    close_logits(lg, ref, r16)
    lg, _ = model(steps[:, 1:5].cuda(), cache)                 # verify-shaped T=4
    ref, past = R.model_forward(W, cfg, steps[:, 1:5], past)
    r16, p16 = R.model_forward(W16, cfg, steps[:, 1:5], p16)
    close_logits(lg, ref, r16)
    assert cache.seen_tokens == past.seen_tokens == 14


def test_rollback_equals_shorter_history(micro):
    """Verify 4 tokens, keep a+1 of them via rollback; the next step's logits must match
    a history that only ever saw those a+1 tokens."""
    model, _, (W, W16), cfg = micro
    g = torch.Generator().manual_seed(2)
    prompt = torch.randint(0, cfg.vocab_size, (3, 7), generator=g)
    blk = torch.randint(0, cfg.vocab_size, (3, 4), generator=g)
    nxt = torch.randint(0, cfg.vocab_size, (3, 1), generator=g)
    acc = torch.tensor([0, 2, 3], dtype=torch.int32)
    cache = model.new_cache(3, 64, spec_slots=4)
    model(prompt.cuda(), cache)
    model(blk.cuda(), cache)
    cache.rollback(acc.cuda())
    lg, _ = model(nxt.cuda(), cache)
    for b in range(3):
        a = int(acc[b]) + 1
        ids = torch.cat([prompt[b:b + 1], blk[b:b + 1, :a], nxt[b:b + 1]], 1)
        ref, _ = R.model_forward(W, cfg, ids)
        r16, _ = R.model_forward(W16, cfg, ids)
        close_logits(lg[b, -1], ref[0, -1], r16[0, -1])


def test_mtp_forward_and_chain(micro):
    model, mtp, (W, W16), cfg = micro
    g = torch.Generator().manual_seed(3)
    h = torch.randn(2, 3, cfg.hidden_size, generator=g).bfloat16()
    e = torch.randn(2, 3, cfg.hidden_size, generator=g).bfloat16()
    got = mtp(h.cuda(), e.cuda())
    ref = R.mtp_forward(W, cfg, h.float(), e.float())
    close_logits(got, ref, R.mtp_forward(W16, cfg, h, e))
    # the incremental draft chain == the no-cache recomputation of the draft block
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    prompt = torch.randint(0, cfg.vocab_size, (2, 8), generator=g)
    dec = SpecDecoder(model, mtp, 2, 64, k=3)
    dec.prefill(prompt.cuda())
    dec._draft_chain()
    got = dec.drafts.cpu().long()
    h_last = dec.h_last.cpu().float()[:, None]
    _, lg = R.mtp_chain_draft(W, cfg, h_last, dec.pending.cpu().long(), 3, forced=got)
    top2 = lg.float().topk(2, -1).values
    tie = (top2[..., 0] - top2[..., 1]) < 0.05
    assert bool(((lg.float().argmax(-1) == got) | tie).all())


def _oracle_trajectory(W, W16, cfg, prompt, n):
    """The oracle's greedy tokens (generate.py:40-62, fp32) and, along them, its top-16
    logits and the bf16 oracle's largest logit deviation (the near-tie tolerance)."""
    toks = R.generate_greedy(W, cfg, prompt, n)
    full = torch.tensor([prompt + toks])
    lg = R.model_forward(W, cfg, full)[0][0, len(prompt) - 1:-1].float()
    lg16 = R.model_forward(W16, cfg, full)[0][0, len(prompt) - 1:-1].float()
    v, i = lg.topk(16, -1)
    return toks, i, v, (lg16 - lg).abs().max().item()


def _agreed_prefix(got, want, top_idx, top_vals, tol):
    for i, (a, b) in enumerate(zip(got, want)):
        if a != b:
            idx = top_idx[i].tolist()
            assert a in idx and float(top_vals[i, 0] - top_vals[i, idx.index(a)]) <= tol, \
                f"step {i}: token {a} is not a near-tie of the oracle's {b}"
            return i
    return len(want)


@pytest.mark.parametrize("k", [1, 3])
def test_greedy_spec_decode_matches_oracle(micro, k):
    """Greedy speculative decoding (B = 4, k drafts) emits the oracle's greedy
    autoregressive tokens (mtp.py:101-103); a difference is allowed only at a near-tie of
    the oracle's own logits, where the comparison stops."""
    model, mtp, (W, W16), cfg = micro
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    print(f"case greedy spec k={k}", flush=True)
    g = torch.Generator().manual_seed(5)
    prompts = torch.randint(0, cfg.vocab_size, (4, 12), generator=g)
    n = 24
    dec = SpecDecoder(model, mtp, 4, 12 + n + 2 * k + 4, k=k, temperature=0.0)
    dec.prefill(prompts.cuda())
    while int(dec.out_count.min()) < n:
        dec.step()
    got = dec.tokens()
    agreed = 0
    for b in range(4):
        want, ti, tv, dev = _oracle_trajectory(W, W16, cfg, prompts[b].tolist(), n)
        agreed += _agreed_prefix(got[b][:n], want, ti, tv, 2 * dev)
    print(f"agreed {agreed} of {4 * n} steps", flush=True)
    assert agreed >= 2 * n              # near-ties are rare on this model


@pytest.mark.parametrize("use_graph", [False, True])
def test_greedy_verify_without_logits_matches_logits_path(micro, use_graph):
    """Temperature 0: verifying through the lm_head argmax (lollm_gemm_argmax +
    lollm_greedy_accept, no logits) emits exactly the tokens and accepted lengths of the
    logits path (lollm_gemm + lollm_spec_accept), eager and replayed from a graph."""
    model, mtp, _, cfg = micro
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    print(f"case greedy argmax verify graph={use_graph}", flush=True)
    g = torch.Generator().manual_seed(8)
    prompts = torch.randint(0, cfg.vocab_size, (4, 10), generator=g)
    res = []
    for fused in (True, False):
        dec = SpecDecoder(model, mtp, 4, 80, k=3, temperature=0.0)
        assert dec.greedy_argmax
        dec.greedy_argmax = fused
        dec.prefill(prompts.cuda())
        dec.step()
        if use_graph:
            dec.capture()
        for _ in range(8):
            dec.replay() if use_graph else dec.step()
        torch.cuda.synchronize()
        res.append((dec.tokens(), dec.accept_hist.cpu().tolist()))
    assert res[0] == res[1]
    assert sum(res[0][1]) == 9 * 4


@pytest.mark.parametrize("pen,draft", [(1.0, "argmax"), (1.05, "argmax"), (1.3, "sample")])
def test_graph_replay_matches_eager(micro, pen, draft):
    model, mtp, _, cfg = micro
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    print(f"case graph replay pen={pen} draft={draft}", flush=True)
    g = torch.Generator().manual_seed(6)
    prompts = torch.randint(0, cfg.vocab_size, (3, 10), generator=g)
    outs = []
    for use_graph in (False, True):
        dec = SpecDecoder(model, mtp, 3, 80, k=3, temperature=0.7, top_p=0.95, seed=9,
                          repetition_penalty=pen, draft=draft)
        dec.prefill(prompts.cuda())
        dec.step()
        if use_graph:
            dec.capture()
        for i in range(6):
            if use_graph:
                dec.replay()
                torch.cuda.synchronize()
                _ = dec.out_count.cpu()            # eager work between replays
            else:
                dec.step()
        outs.append(dec.tokens())
    assert outs[0] == outs[1]


def test_sampled_penalised_step_beyond_the_fused_extra_limit(micro):
    """k = 9 drafts with a repetition penalty: more penalised draft tokens per verify row
    than lollm_gemm_logits takes (8), so the decoder runs the lm_head, the penalty and the
    acceptance as separate passes; with k = 8 it fuses them.  Both run, and the k = 8
    decoder's tokens equal those of the same decoder forced onto the separate passes."""
    model, mtp, _, cfg = micro
    from lollm_amd import ops
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    print("case sampled penalised k=9 / k=8", flush=True)
    g = torch.Generator().manual_seed(12)
    prompts = torch.randint(0, cfg.vocab_size, (2, 10), generator=g)
    dec = SpecDecoder(model, mtp, 2, 120, k=9, temperature=0.7, top_p=0.95, seed=3,
                      repetition_penalty=1.2)
    assert not dec.fused_logits
    dec.prefill(prompts.cuda())
    for _ in range(3):
        dec.step()
    assert all(len(t) >= 3 for t in dec.tokens())
    outs = []
    for fused in (True, False):
        dec = SpecDecoder(model, mtp, 2, 120, k=ops.GEMM_LOGITS_MAX_EXTRA, temperature=0.7,
                          top_p=0.95, seed=3, repetition_penalty=1.2)
        assert dec.fused_logits
        dec.fused_logits = fused
        dec.prefill(prompts.cuda())
        for _ in range(3):
            dec.step()
        outs.append(dec.tokens())
    assert outs[0] == outs[1]


@pytest.mark.parametrize("B,k,temp,top_k,pen,draft", [
    (20, 3, 0.7, 0, 1.1, "argmax"),    # 80 verify rows: every verify projection on hipBLASLt
    (1, 1, 0.0, 0, 1.0, "argmax"),     # the reference's own shape (generate_mtp, k = 1)
    (5, 8, 1.0, 20, 1.3, "sample"),    # sampled drafts, top-k, the fused lm_head's limit
    (16, 3, 0.7, 0, 1.0, "argmax"),    # the benchmark's sampling, no penalty
])
def test_decoder_configurations_graph_equals_eager(micro, B, k, temp, top_k, pen, draft):
    """SpecDecoder across batch sizes (the GEMM and hipBLASLt paths of the verify pass),
    draft counts, sampling settings and draft modes: three graph replays give the tokens
    of three eager steps."""
    model, mtp, _, cfg = micro
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    print(f"case decoder B={B} k={k} T={temp} top_k={top_k} pen={pen} draft={draft}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + k)
    prompts = torch.randint(0, cfg.vocab_size, (B, 12), generator=g)
    outs = []
    for use_graph in (False, True):
        dec = SpecDecoder(model, mtp, B, 12 + 4 * (k + 1) + 8, k=k, temperature=temp,
                          top_k=top_k, top_p=0.95, seed=5, repetition_penalty=pen, draft=draft)
        dec.prefill(prompts.cuda())
        dec.step()
        if use_graph:
            dec.capture()
        for _ in range(3):
            if use_graph:
                dec.replay()
                torch.cuda.synchronize()
            else:
                dec.step()
        outs.append(dec.tokens())
    assert outs[0] == outs[1]
    assert all(len(t) >= 4 for t in outs[0])
