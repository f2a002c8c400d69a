"""The end-to-end speculative workload at full size: a seeded random-init dense 8B-class
qwen3_5 (hidden 4096, 32 layers 3:1 GDN:attention, GDN 16 qk / 32 v heads of 128,
attention 32 q / 4 kv heads of 256, SwiGLU 12288, vocab 151936) with a 1-layer MTP head,
B = 16 sequences of 2048-token prompts, k = 3 drafts.

Checked here (the benchmark only times this workload):
  * one Gated DeltaNet layer and one gated-attention layer of the verify pass, on the
    prefilled cache (context 2048), against the CPU oracle at the bf16 bar;
  * graph replay == eager steps, token for token, with temperature 0.7 / top-p 0.95;
  * the fused verify lm_head (penalty and row maxima in the GEMM, one read per row in
    the acceptance) == the separate passes, token for token, with a repetition penalty;
  * the whole 32-layer verify pass against the oracle's model_forward (two sequences,
    fp32 and bf16 flows, from the GPU-prefilled cache) at the bf16 bar;
  * rollback == a shorter history, bit for bit: verify 4 tokens, keep a + 1 (a = 0..3
    over the batch), then the next token's logits equal those of a cache that only saw
    the kept tokens;
  * accepted drafts at this shape: drafts forced to the verify pass's own greedy fixed
    point are all accepted (the a = k commit, the bonus token, the last snapshot slot).
"""

import pytest
import torch

from oracle import qwen3_5_ref as R

pytestmark = pytest.mark.gpu
B, L, K = 16, 2048, 3


@pytest.fixture(scope="module")
def dense8b():
    from lollm_amd.qwen3_5 import load, load_mtp
    from lollm_amd.qwen3_5.config import Qwen3_5Config, dense_8b_config_dict
    from lollm_amd.qwen3_5.random_init import random_weights
    print("case C5 build dense 8B", flush=True)
    raw = dense_8b_config_dict()
    cfg = Qwen3_5Config.from_hf(raw)
    W = random_weights(cfg, seed=5, dtype=torch.bfloat16, device="cuda")
    # the oracle's layer tests need only layers 0 (GDN) and 3 (attention); the
    # whole-model test reads every weight back from the device
    keep = {k: v.float().cpu() for k, v in W.items()
            if ".layers.0." in k or ".layers.3." in k}
    every = {k.replace("model.language_model.", "model."): v for k, v in W.items()
             if not k.startswith("mtp.")}
    model = load(raw, W, "hf", device="cuda")
    mtp = load_mtp(model, W, "hf", device="cuda")
    del W
    g = torch.Generator(device="cuda").manual_seed(5)
    prompts = torch.randint(0, cfg.vocab_size, (B, L), device="cuda", generator=g)
    W_ref = {k.replace("model.language_model.", "model."): v for k, v in keep.items()}
    return model, mtp, W_ref, R.RefConfig.from_dict(raw), prompts, every


def _bf16_bar(got, ref32, ref16, what):
    got = got.float().cpu()
    err = (got - ref32).abs().max().item()
    budget = 2 * (ref16.float() - ref32).abs().max().item() + 1e-3 * ref32.abs().max().item()
    assert err <= budget, f"{what}: max err {err:.4g} > budget {budget:.4g}"


def test_c5_verify_layers_match_oracle(dense8b):
    model, _, W, cfg, prompts, _ = dense8b
    print("case C5 layers 0 and 3 vs oracle", flush=True)
    cache = model.new_cache(B, L + 8, spec_slots=K + 1)
    model(prompts, cache, logits="last")
    g = torch.Generator().manual_seed(50)
    x = torch.randn(B, K + 1, cfg.hidden_size, generator=g).bfloat16()
    W16 = {k: v.to(torch.bfloat16) for k, v in W.items()}
    # GDN layer 0: conv window + recurrent state from the prefilled cache
    conv, rec = cache.linear_state(0)
    gdn = model.model.layers[0].linear_attn
    got = gdn.out_proj(gdn.core(x.cuda(), cache, 0))
    p = "model.layers.0.linear_attn."
    r32, _, _ = R.gated_deltanet(W, p, cfg, x.float(), conv.float().cpu(), rec.cpu(), True)
    r16, _, _ = R.gated_deltanet(W16, p, cfg, x, conv.cpu(), rec.cpu(), True)
    _bf16_bar(got, r32, r16, "GDN layer 0")
    # attention layer 3: the cache's post-RoPE K / V rows, queries at positions L..L+3
    st = cache.layers[3]
    attn = model.model.layers[3].self_attn
    lengths = cache.lengths.clone()
    ref_k = st["k"][:, :, :L].float().cpu()
    ref_v = st["v"][:, :, :L].float().cpu()
    ws = model.attn_workspace(B, K + 1, cache.max_len)
    got = attn(x.cuda(), st["k"], st["v"], lengths, lengths + K + 1, workspace=ws)
    pos = torch.arange(L, L + K + 1)
    outs = []
    for Wd, dt in ((W, torch.float32), (W16, torch.bfloat16)):
        c = R.RefCache(cfg.num_hidden_layers)
        c.append_kv(3, ref_k.to(dt), ref_v.to(dt))
        cos, sin = R.rope_tables(pos, cfg.rotary_dim, cfg.rope_theta, dt)
        outs.append(R.gated_attention(Wd, "model.layers.3.self_attn.", cfg, x.to(dt), cos, sin,
                                      c, 3))
    _bf16_bar(got, outs[0], outs[1], "attention layer 3")


def test_c5_graph_replay_equals_eager(dense8b):
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    model, mtp, _, cfg, prompts, _ = dense8b
    print("case C5 graph vs eager", flush=True)
    toks = []
    for use_graph in (False, True):
        dec = SpecDecoder(model, mtp, B, L + 6 * (K + 1) + 8, k=K, temperature=0.7, top_p=0.95,
                          seed=5, out_capacity=6 * (K + 1) + 4)
        dec.prefill(prompts)
        dec.step()
        if use_graph:
            dec.capture()
        for _ in range(4):
            if use_graph:
                dec.replay()
                torch.cuda.synchronize()
            else:
                dec.step()
        toks.append(dec.tokens())
        del dec
    assert toks[0] == toks[1]
    assert all(len(t) == 5 for t in toks[0])       # random weights accept nothing here


def test_c5_fused_logits_equal_separate_passes(dense8b):
    """The sampled step (T = 0.7, top-p 0.95, repetition penalty 1.05) at full size, with
    the verify lm_head writing penalised logits and row maxima in one kernel and the
    acceptance reading each row once (lollm_gemm_logits + lollm_spec_accept_rowmax),
    emits exactly the tokens of the separate passes (lm_head, lollm_repetition_penalty,
    lollm_spec_accept), step after step."""
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    model, mtp, _, cfg, prompts, _ = dense8b
    print("case C5 fused logits vs separate passes", flush=True)
    toks = []
    for fused in (True, False):
        dec = SpecDecoder(model, mtp, B, L + 5 * (K + 1) + 8, k=K, temperature=0.7, top_p=0.95,
                          seed=5, out_capacity=5 * (K + 1) + 4, repetition_penalty=1.05)
        assert dec.fused_logits
        dec.fused_logits = fused
        dec.prefill(prompts)
        for _ in range(4):
            dec.step()
        toks.append((dec.tokens(), dec.accept_hist.cpu().tolist()))
        del dec
    assert toks[0] == toks[1]


class _AsFloat(dict):
    """The oracle's fp32 flow over bf16 weights held once: each tensor is widened when
    a layer reads it (the full fp32 copy of the 8B-class weights would be 32 GB)."""

    def __getitem__(self, k):
        return dict.__getitem__(self, k).float()


def _host_state(cache, cfg, rows, dtype):
    """The committed cache of sequences `rows` as the oracle's RefCache (kv.py:20-58)."""
    L = int(cache.lengths[rows[0]])
    past = R.RefCache(cfg.num_hidden_layers)
    for i in range(cfg.num_hidden_layers):
        if cfg.layer_types[i] == "full_attention":
            s = cache.layers[i]
            past.layers[i] = (s["k"][rows, :, :L].to(dtype).cpu(), s["v"][rows, :, :L].to(dtype).cpu())
        else:
            conv, rec = cache.linear_state(i)
            past.layers[i] = (conv[rows].to(dtype).cpu(), rec[rows].cpu())
    past.seen_tokens = L
    return past


def test_c5_verify_logits_match_oracle(dense8b):
    """The whole 32-layer verify pass at full size (B = 16, 1 + k = 4 positions after
    2048-token prompts) against the oracle's model_forward (modeling_qwen3_5.py:82-102)
    for two of the sequences, seeded with the GPU-prefilled cache read back to the host:
    the logits meet the model tests' bf16 bar (max error within twice the oracle's own
    bf16-vs-fp32 error plus 1e-3 of the scale, 1 - cosine within twice its deficit, the
    reference's parity gate being argmax equality and cosine > 0.9999,
    src/compare_logits.py:120-130), and every row's argmax is the oracle's or a near-tie
    of it (within twice the bf16 error)."""
    import time
    model, _, _, cfg, prompts, every = dense8b
    print("case C5 verify logits vs oracle", flush=True)
    cache = model.new_cache(B, L + 8, spec_slots=K + 1)
    model(prompts, cache, logits="last")
    rows = [0, 9]
    past32 = _host_state(cache, cfg, rows, torch.float32)
    past16 = _host_state(cache, cfg, rows, torch.bfloat16)
    g = torch.Generator().manual_seed(52)
    ids = torch.randint(0, cfg.vocab_size, (B, K + 1), generator=g)
    got, _ = model(ids.cuda(), cache)
    got = got[rows].float().cpu()
    t0 = time.time()
    W16 = R.canonical_weights({k: v.cpu() for k, v in every.items()})
    r16, _ = R.model_forward(W16, cfg, ids[rows], past16)
    print(f"oracle bf16 flow {time.time() - t0:.1f} s", flush=True)
    r32, _ = R.model_forward(_AsFloat(W16), cfg, ids[rows], past32)
    print(f"oracle fp32 flow {time.time() - t0:.1f} s", flush=True)
    r16 = r16.float()
    dev = (r16 - r32).abs().max().item()
    err = (got - r32).abs().max().item()
    scale = r32.abs().max().item()
    cs = torch.nn.functional.cosine_similarity
    flat = lambda t: t.reshape(-1, t.shape[-1])  # noqa: E731
    deficit = (1 - cs(flat(got), flat(r32), dim=-1)).max().item()
    ref_deficit = (1 - cs(flat(r16), flat(r32), dim=-1)).max().item()
    print(f"max err {err:.4g} (oracle bf16 {dev:.4g}, scale {scale:.3g}); 1-cos {deficit:.3g} "
          f"(oracle bf16 {ref_deficit:.3g})", flush=True)
    assert err <= 2 * dev + 1e-3 * scale
    assert deficit <= max(2 * ref_deficit, 1e-3)
    am, ref_am = flat(got).argmax(-1), flat(r32).argmax(-1)
    for i in range(am.numel()):
        a, b = int(am[i]), int(ref_am[i])
        assert a == b or float(flat(r32)[i, b] - flat(r32)[i, a]) <= 2 * dev, (i, a, b)


def test_c5_rollback_equals_shorter_history(dense8b):
    """Verify 4 tokens, keep a + 1 (a = 0..3 over the batch), then one more token: each
    sequence's logits equal, bit for bit, those of a cache that only ever saw its a + 1
    kept tokens.  Exact because nothing a sequence computes depends on how many rows
    share the call: the GEMMs add every output's k-steps in one order for 1..64 rows, the
    attention rows keep their own running maxima (and the contexts here deal the same key
    blocks to the workgroups), the GDN replay records rebuild the scanned state bit for
    bit, and every other kernel works row by row."""
    model, _, _, cfg, prompts, _ = dense8b
    print("case C5 rollback", flush=True)
    g = torch.Generator(device="cuda").manual_seed(51)
    blk = torch.randint(0, cfg.vocab_size, (B, K + 1), device="cuda", generator=g)
    nxt = torch.randint(0, cfg.vocab_size, (B, 1), device="cuda", generator=g)
    acc = (torch.arange(B, device="cuda") % (K + 1)).int()
    cache = model.new_cache(B, L + 16, spec_slots=K + 1)
    model(prompts, cache, logits="last")
    short = cache.clone()
    model(blk, cache)
    cache.rollback(acc)
    got, _ = model(nxt, cache)
    got = got.float().view(B, -1)
    hist = []
    for a in range(K + 1):
        c = short.clone()
        model(blk[:, :a + 1], c)
        lg, _ = model(nxt, c)
        hist.append(lg.float().view(B, -1))
        del c
    for b in range(B):
        a = int(acc[b])
        d = [(got[b] - h[b]).abs().max().item() for h in hist]
        print(f"b={b} a={a} max |diff| to each history: " + " ".join(f"{x:.3g}" for x in d),
              flush=True)
        assert torch.equal(got[b], hist[a][b])
        assert all(d[o] > 0 for o in range(K + 1) if o != a)


def test_c5_accepted_drafts_commit(dense8b):
    """Accepted drafts at full size (random weights accept nothing on their own): each
    step's drafts are forced to the verify pass's own greedy fixed point (k rounds of the
    verify forward, so position i's argmax already follows drafts 1..i), so at
    temperature 0 all k are accepted -- the a = k commit, the bonus token and the last
    snapshot slot -- and the emitted tokens are exactly those drafts."""
    from lollm_amd import ops
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    model, mtp, _, cfg, prompts, _ = dense8b
    print("case C5 accepted drafts", flush=True)
    steps = 3
    n = steps * (K + 1)
    dec = SpecDecoder(model, mtp, B, L + n + 8, k=K, temperature=0.0, out_capacity=n + 8)
    dec.prefill(prompts)
    expect = [[] for _ in range(B)]

    def fixed_point_chain():
        d = torch.zeros(B, K, dtype=torch.int32, device="cuda")
        for _ in range(K):
            ids = torch.cat([dec.pending.view(B, 1), d], 1)
            _, normed = model.hidden_states(ids, dec.cache)
            am = ops.sample_rows(model.lm_head(normed).view(B * (K + 1), -1), 0.0)
            d = am.view(B, K + 1)[:, :K].contiguous()
        dec.drafts.copy_(d)
        for b in range(B):
            expect[b] += [int(dec.pending[b])] + d[b].tolist()
    dec._draft_chain = fixed_point_chain
    for _ in range(steps):
        dec.step()
    hist = dec.accept_hist.cpu().tolist()
    print(f"accept histogram {hist}", flush=True)
    assert hist[K] == steps * B
    assert dec.tokens() == expect
