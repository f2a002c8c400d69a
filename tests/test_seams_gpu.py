"""The drop-in seams on the GPU, each against the oracle.

  * attention(q, k, v) (src/attention.py:84-91, offset-causal rule :43-51), the
    reference's one operator-plugin seam, on already-expanded heads;
  * sample_next (src/generate.py:17-37): greedy picks under a repetition penalty against
    the reference's own picks, and sampled draws bit-exact against the C oracle;
  * the cache methods (src/qwen3_5/kv.py:26-58) after a real forward, against the oracle's
    RefCache;
  * the repetition penalty kernel at the acceptance shape (B = 64, k = 3, V = 151936),
    bit-exact against the C oracle, and acceptance on penalised logits bit-exact;
  * run-to-run determinism: two freshly loaded models give identical bits.
"""

import os

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

from lollm_amd.qwen3_5.config import Qwen3_5Config, micro_config_dict
from lollm_amd.qwen3_5.random_init import random_weights
from oracle import qwen3_5_ref as R
from oracle import sampler_ref as S

pytestmark = pytest.mark.gpu


def build(raw, seed=0):
    from lollm_amd.qwen3_5 import load, load_mtp
    cfg = Qwen3_5Config.from_hf(raw)
    Wb = {k: v.to(torch.bfloat16) for k, v in random_weights(cfg, seed=seed).items()}
    weights = dict(Wb)
    model = load(raw, weights, "hf", device="cuda")
    mtp = load_mtp(model, weights, "hf", device="cuda")
    W = R.canonical_weights({k: v.float() for k, v in Wb.items()})
    W16 = R.canonical_weights(dict(Wb))
    return model, mtp, W, W16, R.RefConfig.from_dict(raw)


@pytest.fixture(scope="module")
def micro():
    return build(micro_config_dict())


# ----------------------------------------------------------------- attention seam
@pytest.mark.parametrize("B,H,ql,tk", [(2, 4, 1, 37), (2, 4, 4, 300), (1, 8, 37, 37),
                                       (3, 2, 4, 4), (2, 2, 64, 64)])
def test_attention_seam_matches_oracle(B, H, ql, tk):
    from lollm_amd.attention import attention
    print(f"case attention seam B={B} H={H} q_len={ql} total_k={tk}", flush=True)
    g = torch.Generator().manual_seed(B * 1000 + ql * 10 + tk)
    q = torch.randn(B, H, ql, 256, generator=g).bfloat16()
    k = torch.randn(B, H, tk, 256, generator=g).bfloat16()
    v = torch.randn(B, H, tk, 256, generator=g).bfloat16()
    got = attention(q.cuda(), k.cuda(), v.cuda())
    assert got.shape == (B, H, ql, 256) and got.dtype == torch.bfloat16
    ref = R.sdpa_offset_causal(q.float(), k.float(), v.float())
    torch.testing.assert_close(got.float().cpu(), ref, rtol=2e-2, atol=2e-2)


# ----------------------------------------------------------------- sample_next seam
def test_sample_next_penalty_matches_reference_picks(golden_dir):
    """The reference's own greedy picks (sample_next at temperature 0 with a penalty,
    written by tests/golden/make_golden_ref.py) through the drop-in."""
    from lollm_amd.generate import sample_next
    f = load_file(os.path.join(golden_dir, "ref_mtp.safetensors"))
    rows, prev, picks = f["penalty.logits"], f["penalty.prev"], f["penalty.pick_and_milli"]
    for r in range(rows.shape[0]):
        ids = [int(t) for t in prev[r] if t >= 0]
        pen = int(picks[r, 1]) / 1000.0
        x = rows[r].cuda()
        before = x.clone()
        assert sample_next(x, 0.0, 0, 1.0, pen, ids) == int(picks[r, 0]), r
        assert torch.equal(x, before)                  # the caller's logits are untouched


@pytest.mark.parametrize("temp,top_k,top_p,pen", [(0.7, 20, 0.8, 1.05), (1.0, 0, 0.95, 1.0),
                                                  (0.7, 0, 1.0, 1.3)])
def test_sample_next_draws_bit_exact(temp, top_k, top_p, pen):
    from lollm_amd.generate import sample_next
    g = torch.Generator().manual_seed(17)
    V = 151936
    x = (torch.randn(V, generator=g) * 3).bfloat16()
    prev = torch.randint(0, V, (3000,), generator=g).tolist()
    bits = S.repetition_penalty(x, prev, pen) if pen != 1.0 else S._bits(x)
    inv = S.inv_temperature(temp)
    for off in (1, 77):
        want = int(S.sample_rows(bits.reshape(1, V), inv, top_k, top_p, 5, off)[0])
        got = sample_next(x.cuda(), temp, top_k, top_p, pen, prev, seed=5, offset=off)
        assert got == want


# ----------------------------------------------------------------- cache methods
def test_linear_state_with_replay_records_matches_refcache(micro):
    """After a long forward (prefill: the state itself) and then a short one (T <= the
    replay slots: the committed state is the stored state plus T replay records),
    linear_state equals the oracle cache after the same 12 tokens (bf16 bar);
    set_linear_state on one layer folds every layer's records first and leaves the other
    layers' states bit for bit as they were."""
    model, _, W, W16, cfg = micro
    g = torch.Generator().manual_seed(14)
    ids = torch.randint(0, cfg.vocab_size, (2, 12), generator=g)
    cache = model.new_cache(2, 32, spec_slots=4)
    model(ids[:, :9].cuda(), cache)
    model(ids[:, 9:].cuda(), cache)
    assert int(cache.replay.min()) == 3
    _, past = R.model_forward(W, cfg, ids)
    _, p16 = R.model_forward(W16, cfg, ids)
    gdn = [i for i, lt in enumerate(cfg.layer_types) if lt != "full_attention"]
    before = {}
    for i in gdn:
        conv, rec = cache.linear_state(i)
        before[i] = (conv, rec)
        c_ref, r_ref = past.linear_state(i)
        c16, r16 = p16.linear_state(i)
        assert (conv.float().cpu() - c_ref).abs().max() <= 2 * (c16.float() - c_ref).abs().max() + 1e-3
        assert (rec.cpu() - r_ref).abs().max() <= 2 * (r16.float() - r_ref).abs().max() + 1e-3
    cache.set_linear_state(gdn[0], before[gdn[0]][0], before[gdn[0]][1] * 0 + 2)
    assert int(cache.replay.max()) == 0
    assert bool((cache.linear_state(gdn[0])[1] == 2).all())
    for i in gdn[1:]:
        conv, rec = cache.linear_state(i)
        assert torch.equal(conv, before[i][0]) and torch.equal(rec, before[i][1])


def test_cache_methods_match_refcache(micro):
    """read_kv / linear_state after a forward equal the oracle cache's contents (bf16
    bar); set_linear_state / append_kv / advance / clone / nbytes / seen_tokens behave as
    kv.py:26-58."""
    model, _, W, W16, cfg = micro
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (2, 9), generator=g)
    cache = model.new_cache(2, 32, spec_slots=4)
    model(ids.cuda(), cache)
    _, past = R.model_forward(W, cfg, ids)
    _, p16 = R.model_forward(W16, cfg, ids)
    assert cache.seen_tokens == past.seen_tokens == 9
    for i, lt in enumerate(cfg.layer_types):
        if lt == "full_attention":
            K, V = cache.read_kv(i)
            for got, want, w16 in ((K, past.read_kv(i)[0], p16.read_kv(i)[0]),
                                   (V, past.read_kv(i)[1], p16.read_kv(i)[1])):
                assert got.shape == want.shape
                err = (got.float().cpu() - want).abs().max().item()
                assert err <= 2 * (w16.float() - want).abs().max().item() + 1e-3
            assert cache.linear_state(i) == (None, None)
        else:
            conv, rec = cache.linear_state(i)
            c_ref, r_ref = past.linear_state(i)
            c16, r16 = p16.linear_state(i)
            assert conv.shape == c_ref.shape and rec.shape == r_ref.shape
            assert (conv.float().cpu() - c_ref).abs().max() <= 2 * (c16.float() - c_ref).abs().max() + 1e-3
            assert (rec.cpu() - r_ref).abs().max() <= 2 * (r16.float() - r_ref).abs().max() + 1e-3
    # set_linear_state round trip, clone independence, nbytes
    li = cfg.layer_types.index("linear_attention")
    conv, rec = cache.linear_state(li)
    twin = cache.clone()
    cache.set_linear_state(li, conv * 0 + 1, rec * 0 + 2)
    c2, r2 = cache.linear_state(li)
    assert bool((c2 == 1).all()) and bool((r2 == 2).all())
    c3, r3 = twin.linear_state(li)
    assert torch.equal(c3, conv) and torch.equal(r3, rec)
    assert cache.nbytes() == sum(t.numel() * t.element_size()
                                 for s in cache.layers if s for t in s.values())
    ai = cfg.layer_types.index("full_attention")
    kk = torch.randn(2, cfg.num_key_value_heads, 3, cfg.head_dim).bfloat16().cuda()
    K, V = twin.append_kv(ai, kk, kk)
    assert K.shape[2] == 12 and torch.equal(K[:, :, 9:], kk)
    twin.advance(3)
    assert twin.seen_tokens == 12 and cache.seen_tokens == 9
    with pytest.raises(RuntimeError, match="capacity"):
        twin.advance(30)


# ------------------------------------------------------- repetition penalty kernel
def test_repetition_penalty_bit_exact_acceptance_shape():
    """B = 64, k = 3, V = 151936 verify rows; each sequence's context is a 2048-token
    prompt plus committed tokens; row t also penalises drafts d_1..d_t (duplicates
    included).  Then acceptance on the penalised rows, penalty 1.05: bit-exact."""
    from lollm_amd import ops
    B, k, V = 64, 3, 151936
    g = torch.Generator().manual_seed(31)
    tgt = (torch.randn(B, k + 1, V, generator=g) * 3).bfloat16()
    ctx = torch.randint(0, V, (B, 2200), generator=g)
    drafts = torch.randint(0, V, (B, k), generator=g).to(torch.int32)
    drafts[::3, 1] = drafts[::3, 0]                     # a repeated draft
    drafts[::5, 0] = ctx[::5, 7].to(torch.int32)        # a draft already in the context
    seen = ops.new_seen(B, V, "cuda")
    ops.seen_mark(seen, ctx.cuda(), V)
    got = tgt.cuda()
    ops.repetition_penalty(got, seen, 1.05, extra=drafts.cuda())
    got = got.cpu().view(torch.int16).numpy().view(np.uint16)
    want = np.empty_like(got)
    for b in range(B):
        for t in range(k + 1):
            ids = ctx[b].tolist() + drafts[b, :t].tolist()
            want[b, t] = S.repetition_penalty(tgt[b, t], ids, 1.05)
    np.testing.assert_array_equal(got, want)
    # acceptance on the penalised logits: greedy drafts and sampled (one-hot q)
    pen = torch.from_numpy(want.view(np.int16)).view(torch.bfloat16)
    for temp in (0.7, 0.0):
        inv = S.inv_temperature(temp)
        na_ref, nt_ref = S.spec_accept(pen, None, drafts.numpy(), inv, 0, 0.95, 3, 11)
        na, nt = ops.spec_accept(pen.cuda(), None, drafts.cuda(), temp, 0, 0.95, 3, 11)
        assert np.array_equal(na.cpu().numpy(), na_ref) and np.array_equal(nt.cpu().numpy(), nt_ref)


def test_spec_commit_marks_context():
    """lollm_spec_commit adds the accepted drafts and the new pending token to the
    sequence's seen bitmap (mtp.py:129,150), nothing else; the GDN state moves to the
    half the verify wrote, with a + 1 of its replay records kept."""
    from lollm_amd import ops
    B, T, H, V = 3, 4, 64, 1000
    i32 = dict(dtype=torch.int32, device="cuda")
    ids = torch.tensor([[5, 6, 7, 8], [9, 10, 11, 12], [13, 14, 15, 16]], **i32)
    n_acc = torch.tensor([0, 2, 3], **i32)
    nxt = torch.tensor([100, 200, 300], **i32)
    z = lambda: torch.zeros(B, **i32)  # noqa: E731
    seen = ops.new_seen(B, V, "cuda")
    rec_half = torch.tensor([0, 1, 0], **i32)
    replay, conv_off = z(), torch.tensor([0, 7, 3], **i32)
    ops.spec_commit(ids, n_acc, nxt, z(), rec_half, replay, conv_off, z(),
                    torch.zeros(B, 16, **i32), z(),
                    torch.zeros(B, T, H, dtype=torch.bfloat16, device="cuda"),
                    torch.zeros(B, H, dtype=torch.bfloat16, device="cuda"),
                    torch.zeros(1, dtype=torch.int64, device="cuda"), 4, 7, seen=seen)
    assert rec_half.tolist() == [1, 0, 1]
    assert replay.tolist() == [1, 3, 4]
    assert conv_off.tolist() == [7 + 1, 0 + 3, 7 + 4]
    bits = seen.cpu().numpy().view(np.uint32)
    marked = [{t for t in range(V) if bits[b, t >> 5] >> (t & 31) & 1} for b in range(B)]
    assert marked == [{100}, {10, 11, 200}, {14, 15, 16, 300}]


# ----------------------------------------------------------------- determinism
def test_two_fresh_models_give_identical_bits():
    """Same weights loaded twice: identical verify logits and identical sampled
    speculative tokens (the GEMM path is a fixed function of the shape)."""
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    outs = []
    for _ in range(2):
        model, mtp, _, _, cfg = build(micro_config_dict(), seed=3)
        g = torch.Generator().manual_seed(8)
        prompts = torch.randint(0, cfg.vocab_size, (4, 12), generator=g)
        lg, _ = model(prompts.cuda(), model.new_cache(4, 40))
        dec = SpecDecoder(model, mtp, 4, 80, k=3, temperature=0.7, top_p=0.95, seed=4,
                          repetition_penalty=1.05)
        dec.prefill(prompts.cuda())
        for _ in range(5):
            dec.step()
        outs.append((lg.cpu(), dec.tokens()))
        del model, mtp, dec
    assert torch.equal(outs[0][0].view(torch.int16), outs[1][0].view(torch.int16))
    assert outs[0][1] == outs[1][1]
