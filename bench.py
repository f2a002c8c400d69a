"""Benchmark of the qwen3_5 MTP speculative-decode step on one MI355X.

Workload (the headline metric's configuration): a seeded random-init dense 8B-class
qwen3_5 hybrid decoder (hidden 4096, 32 layers with 3:1 Gated DeltaNet : gated
attention, GDN 16 qk / 32 v heads of 128, attention 32 q / 4 kv heads of 256, SwiGLU
12288, vocab 151936, tied embeddings) plus a 1-layer MTP head; B = 16 sequences with
2048-token uniform-random prompts; k = 3 MTP drafts per step; temperature 0.7,
top-p 0.95; rejection-sampling acceptance.

A step = draft chain (3 MTP passes + lm_head + argmax) + one verify forward over the
1 + k positions of all 16 sequences + acceptance + commit, replayed from a HIP graph.
`value` = emitted tokens per second over the K timed steps (the pending token plus
the accepted drafts of every sequence; random weights accept almost nothing, so this
is close to B tokens per step).  `roofline` is the step itself: its algorithmic HBM
bytes (every weight the verify pass and the k draft passes stream, the GDN states and
replay records, the conv windows, the KV cache at the run's context, the logits) over
the HIP-event time of one graph replay, against the 8 TB/s HBM3E peak.  Also
reported: the accepted-length histogram, the verify-step time, a timed accepted path
(drafts forced to the verify pass's own greedy fixed point, so every step commits
k + 1 tokens per sequence), the hot kernels measured the way the step runs them (each
timed over every layer's own buffers in turn), the isolated-kernel workloads, and the
CPU restatement of the reference path timed on the host.

    python bench.py [--gpus 1] [--steps 256] [--warmup 8]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
METRIC = "accepted tok/s at B=16,k=3; verify-step µs; GDN/attn HBM GB/s vs peak"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def time_fn(fn, iters, warm=3, replays=5):
    """Average µs per call of fn(): `iters` calls captured into one HIP graph, replayed
    `replays` times between HIP events on torch's current stream (the stream the graph
    replays on).  Launching from Python costs 10-30 µs per call, more than many of
    these kernels take, so eager back-to-back calls would time the host instead."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) * 1000.0 / (iters * replays)


# ------------------------------------------------------------------------------------
# end-to-end speculative decoding
# ------------------------------------------------------------------------------------
def build_8b(seed=5):
    import torch
    from lollm_amd.qwen3_5 import load, load_mtp
    from lollm_amd.qwen3_5.config import Qwen3_5Config, dense_8b_config_dict
    from lollm_amd.qwen3_5.random_init import random_weights
    raw = dense_8b_config_dict()
    cfg = Qwen3_5Config.from_hf(raw)
    W = random_weights(cfg, seed=seed, dtype=torch.bfloat16, device="cuda")
    keep = dict(W)                       # the loader pops; keep references for the CPU leg
    model = load(raw, W, "hf", device="cuda")
    mtp = load_mtp(model, W, "hf", device="cuda")
    return raw, cfg, model, mtp, keep


def run_e2e(model, mtp, cfg, B, prompt_len, k, steps, warmup, temperature, top_p, seed):
    import torch
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    prompts = torch.randint(0, cfg.vocab_size, (B, prompt_len), device="cuda", generator=gen)
    max_len = prompt_len + (steps + warmup + 2) * (k + 1) + 8
    dec = SpecDecoder(model, mtp, B, max_len, k=k, temperature=temperature, top_p=top_p,
                      seed=seed, out_capacity=(steps + warmup + 2) * (k + 1) + 8)
    t0 = time.time()
    dec.prefill(prompts)
    torch.cuda.synchronize()
    log(f"prefill {B}x{prompt_len}: {time.time() - t0:.2f} s")
    n_eager = min(2, warmup)
    for _ in range(n_eager):
        dec.step()
    dec.capture()
    for _ in range(warmup - n_eager):
        dec.replay()
    torch.cuda.synchronize()
    # timed region: K graph replays; per-step accepted counts read after the region
    counts_before = dec.out_count.clone()
    hist_before = dec.accept_hist.clone()
    ctx_before = dec.cache.lengths.float().sum().item()
    marker()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dec.replay()
    e1.record()
    torch.cuda.synchronize()
    marker()
    wall = time.perf_counter() - t_start
    gpu_s = e0.elapsed_time(e1) / 1000.0
    emitted = int((dec.out_count - counts_before).sum())
    hist = (dec.accept_hist - hist_before).cpu().tolist()
    ctx_after = dec.cache.lengths.float().sum().item()
    return dec, {"emitted": emitted, "seconds": gpu_s, "wall_seconds": wall, "hist": hist,
                 "mean_accepted": sum(i * c for i, c in enumerate(hist)) / max(1, sum(hist)),
                 "final_context_mean": ctx_after / B,
                 # sum over the batch of the cache length a timed step starts from, averaged
                 "ctx_sum_mean": (ctx_before + ctx_after) / 2 - (ctx_after - ctx_before) / (2 * steps)}


MARKER_KERNEL = "scan"


def marker():
    """A small cumulative sum: its kernel (a scan, which the step never launches) marks
    the start and the end of the timed region in a rocprofv3 trace."""
    import torch
    torch.cumsum(torch.ones(4096, device="cuda"), 0)


def projection_paths(model, mtp, B, k):
    """The path of each projection shape of the step ("gemm grid g, c-col groups" =
    lollm_gemm on g workgroups with c-column groups -- 96 where those divide over the
    grid and 64-column ones would not, the library's rule -- "blas" = hipBLASLt; a fixed
    function of the shape), keyed "NxK M=rows"."""
    out = {}
    layers = list(model.model.layers) + list(mtp.layers)
    projs = [model.lm_head, mtp.fc]
    for layer in layers:
        mixer = layer.self_attn if layer.layer_type == "full_attention" else layer.linear_attn
        projs += mixer.projections() + layer.mlp.projections()
    for p in projs:
        for rows in (B, B * (k + 1)):
            tag = f"{p.N}x{p.K}{' swiglu' if p.epilogue else ''} M={rows}"
            path = p.path(rows)
            if path == "gemm":
                g = p.grid(rows)
                cols = 96 if p.N % 96 == 0 and (p.N // 96) % g == 0 and (p.N // 64) % g else 64
                out[tag] = f"gemm grid {g}, {cols}-col groups"
            else:
                out[tag] = path
    return dict(sorted(out.items()))


def verify_breakdown(dec, iters=20):
    """The step's parts (µs), each replayed alone from a graph: draft chain, verify
    forward, acceptance."""
    import torch
    from lollm_amd import ops
    B, k, model = dec.B, dec.k, dec.model
    st = {}
    st["draft_chain_us"] = time_fn(dec._draft_chain, iters)

    lm = model.lm_head

    def verify():
        # the verify pass over 1 + k positions (KV rows / GDN snapshots are written but
        # not committed, so repeating it is idempotent), ending in the step's lm_head:
        # logits with the penalty and row maxima fused when the step samples
        hidden, normed = dec.verify_hidden()
        if dec.fused_logits:
            lg, rm = ops.gemm_logits(normed.reshape(-1, lm.K), lm.tiled, lm.N, lm.K,
                                     out=dec.verify_logits.view(-1, lm.N), rowmax=dec.verify_rmax,
                                     seen=dec.seen, penalty=dec.penalty, extra=dec.drafts,
                                     T=k + 1, grid=lm.grid())
            return lg.view(B, k + 1, -1), rm
        return model.lm_head(normed), None
    st["verify_forward_us"] = time_fn(verify, iters)
    logits, rmax = verify()
    st["accept_us"] = time_fn(lambda: ops.spec_accept(
        logits, None, dec.drafts, dec.temperature, 0, dec.top_p, dec.seed, 0,
        offset_dev=dec.offset, workspace=dec.spec_ws, n_accepted=dec.n_acc,
        next_token=dec.next_tok, target_rowmax=rmax), iters)
    return st


# ------------------------------------------------------------------------------------
# the step's roofline and its hot kernels as the step runs them
# ------------------------------------------------------------------------------------
def step_bytes(cfg, B, k, ctx_sum, replayed, logits=True):
    """Algorithmic HBM bytes of one speculative step: what must cross HBM at least once.
    Weights (bf16): every decoder weight and the lm_head for the verify pass, and k times
    the MTP layer's weights plus the lm_head for the draft chain (each draft streams them
    again: 1.83 GB does not fit the 256 MB last-level cache).  GDN layers: the committed
    state read and its copy written to the other half (B Hv Dk Dv fp32 each), the replay
    records it applies (`replayed` positions over the batch) and the T it writes
    (Hv (4 Dk + 16) bytes per position), the conv window read (K-1 rows) and written
    (K-1+T rows).  Attention layers: the K and V rows of every sequence's context
    (ctx_sum = sum of the kv lengths) and the T new rows.  The (B, T, V) bf16 logits
    written and read once by the acceptance when the step samples (logits=True).
    Activations between kernels are left out (they could stay on chip)."""
    import math
    from lollm_amd.qwen3_5.random_init import weight_shapes
    T = k + 1
    H, V = cfg.hidden_size, cfg.vocab_size
    main = mtp = 0
    for name, (shape, _) in weight_shapes(cfg, with_mtp=True).items():
        if name.endswith("embed_tokens.weight") or name == "lm_head.weight":
            continue
        if name.startswith("mtp."):
            mtp += math.prod(shape) * 2
        else:
            main += math.prod(shape) * 2
    lm = V * H * 2
    Hv, D, K = cfg.linear_num_value_heads, cfg.linear_key_head_dim, cfg.linear_conv_kernel_dim
    n_gdn = sum(1 for i in range(cfg.num_hidden_layers) if cfg.layer_type(i) != "full_attention")
    n_attn = cfg.num_hidden_layers - n_gdn
    Hkv, Dh = cfg.num_key_value_heads, cfg.head_dim
    parts = {
        "verify_weights": main + lm,
        "draft_chain_weights": k * (mtp + lm),
        "gdn_state": n_gdn * 2 * B * Hv * D * D * 4,
        "gdn_records": n_gdn * (replayed + B * T) * Hv * (4 * D + 16),
        "conv_windows": n_gdn * B * (2 * (K - 1) + T) * cfg.conv_dim * 2,
        "kv_cache": n_attn * (int(ctx_sum) + B * T) * Hkv * Dh * 2 * 2,
        "logits": 2 * B * T * V * 2 if logits else 0,
    }
    parts["total"] = sum(parts.values())
    return parts


def gdn_layer_bytes(cfg, B, T, replayed=None):
    """Algorithmic HBM bytes of one short lollm_gdn_layer launch: read the committed
    half's state (B Hv Dk Dv fp32) and the records it replays (`replayed` positions over
    the batch, default B T; 4 Dk + 16 bytes per head), write the committed state to the
    other half and the T new records, read the projections (B T P bf16) and the conv
    window (K-1 rows), write the window (K-1+T rows) and the output (B T Hv Dv)."""
    D, Hv = cfg.linear_key_head_dim, cfg.linear_num_value_heads
    P = cfg.conv_dim + cfg.value_dim + 2 * Hv
    K = cfg.linear_conv_kernel_dim
    state = B * Hv * D * D * 4
    rec = Hv * (4 * D + 16)
    replayed = B * T if replayed is None else replayed
    return (2 * state + (replayed + B * T) * rec + B * T * P * 2 + B * (K - 1) * cfg.conv_dim * 2
            + B * (K - 1 + T) * cfg.conv_dim * 2 + B * T * cfg.value_dim * 2)


def _rate(name, launches, us_total, byt_total, extra=None):
    us = us_total / launches
    gbs = byt_total / us_total / 1e3
    row = {"kernel": name, "launches_per_step": launches, "avg_us": round(us, 2),
           "bytes_per_launch": int(byt_total // launches), "achieved": round(gbs, 1),
           "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4)}
    if extra:
        row.update(extra)
    return row


def in_step_kernels(model, mtp, dec, iters=2):
    """The verify pass's hot kernels as the step runs them: each kind is captured in one
    HIP graph that launches it once per layer of that kind, on that layer's own weights,
    cache state and KV rows in turn (so a launch never finds its data in the 256 MB
    last-level cache from the previous one, as in the step), and timed with HIP events
    over the replays.  Per launch: the average time, the algorithmic bytes and their
    rate against the 8 TB/s peak.  Attention is the (main + combine) pair; the
    residual-stream projections include their merge + residual + RMSNorm kernel."""
    import torch
    from lollm_amd import ops
    cfg, cache = model.cfg, dec.cache
    B, T = dec.B, dec.k + 1
    M = B * T
    layers = model.model.layers
    gdn_ids = [i for i, l in enumerate(layers) if l.layer_type != "full_attention"]
    att_ids = [i for i, l in enumerate(layers) if l.layer_type == "full_attention"]
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    rnd = lambda *shape: (0.5 * torch.randn(*shape, device="cuda", generator=g)).bfloat16()  # noqa: E731
    out = {}
    # fused GDN layer, one launch per GDN layer on its own state / records / window
    Hk, Hv, D = cfg.linear_num_key_heads, cfg.linear_num_value_heads, cfg.linear_key_head_dim
    projs = {i: rnd(B, T, layers[i].linear_attn.in_proj.N) for i in gdn_ids}
    o = torch.empty(B, T, cfg.value_dim, dtype=torch.bfloat16, device="cuda")

    def gdn_all():
        for i in gdn_ids:
            gdn, s = layers[i].linear_attn, cache.layers[i]
            ops.gdn_layer(projs[i], gdn.conv_w, gdn.A_log, gdn.dt_bias, gdn.norm_w, s["win"],
                          cache.conv_off, s["rec"], cache.rec_half, s["rep"], cache.replay, False,
                          B, T, Hk, Hv, D, cfg.linear_conv_kernel_dim, cfg.rms_norm_eps, out=o)
    replayed = int(cache.replay.clamp(0, cache.spec_slots).sum())
    us = time_fn(gdn_all, iters)
    out["gdn_layer"] = _rate("lollm::gdn_layer_verify_kernel", len(gdn_ids), us,
                             len(gdn_ids) * gdn_layer_bytes(cfg, B, T, replayed),
                             {"shape": f"B={B} T={T} Hv={Hv} Hk={Hk} D={D}, {replayed} records replayed"})
    del projs
    # gated attention (verify + combine), one launch per attention layer on its KV rows
    Hq, Hkv, Dh = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    q, gate = rnd(B, T, Hq, Dh), rnd(B, T, Hq * Dh)
    kv_len = (cache.lengths + T).contiguous()
    ws = model.attn_workspace(B, T, cache.max_len)
    ao = torch.empty(B, T, Hq * Dh, dtype=torch.bfloat16, device="cuda")

    def attn_all():
        for i in att_ids:
            s = cache.layers[i]
            ops.attn_verify(q, s["k"], s["v"], kv_len, gate, grid=model.attn_grid, workspace=ws, out=ao)
    us = time_fn(attn_all, iters)
    ctx = int(kv_len.sum())
    out["attention"] = _rate("lollm::attn_verify_kernel + attn_combine_kernel", len(att_ids), us,
                             len(att_ids) * (ctx * Hkv * Dh * 4 + 3 * M * Hq * Dh * 2),
                             {"shape": f"B={B} T={T} Hq={Hq} Hkv={Hkv} D={Dh}, mean context {ctx / B:.0f}"})
    # the verify pass's projections, one kind at a time over every layer that has it
    H, F = cfg.hidden_size, cfg.intermediate_size
    x, res = rnd(M, H), rnd(M, H)

    def gemm_kind(name, picks, fn):
        projs_ = [p for p in picks]
        us = time_fn(lambda: [fn(p) for p in projs_], iters)
        byt = sum(p.N * p.K * 2 + M * p.K * 2 + M * (p.N // (2 if p.epilogue else 1)) * 2 for p in projs_)
        out[name] = _rate(f"lollm_gemm {projs_[0].N}x{projs_[0].K}, M={M}", len(projs_), us, byt,
                          {"grid": projs_[0].grid(M)})
    gdn_layers = [layers[i] for i in gdn_ids]
    att_layers = [layers[i] for i in att_ids]
    norm = layers[0].input_layernorm
    core_v = rnd(M, cfg.value_dim)
    core_a = rnd(M, Hq * Dh)
    act = rnd(M, F)
    gemm_kind("gemm_gdn_in_proj", [l.linear_attn.in_proj for l in gdn_layers], lambda p: p(x))
    gemm_kind("gemm_attn_qkv", [l.self_attn.qkv for l in att_layers], lambda p: p(x))
    gemm_kind("gemm_gdn_out_proj_norm", [l.linear_attn.out_proj for l in gdn_layers],
              lambda p: p.add_norm(core_v, res, norm))
    gemm_kind("gemm_attn_o_proj_norm", [l.self_attn.o_proj for l in att_layers],
              lambda p: p.add_norm(core_a, res, norm))
    gemm_kind("gemm_mlp_gate_up", [l.mlp.gate_up for l in layers], lambda p: p(x))
    gemm_kind("gemm_mlp_down_norm", [l.mlp.down for l in layers], lambda p: p.add_norm(act, res, norm))
    gemm_kind("gemm_lm_head", [model.lm_head], lambda p: p(x))
    kinds = [v for key, v in out.items() if key.startswith("gemm_")]
    tot_us = sum(v["avg_us"] * v["launches_per_step"] for v in kinds)
    tot_b = sum(v["bytes_per_launch"] * v["launches_per_step"] for v in kinds)
    out["gemm_verify_all"] = {"us_per_step": round(tot_us, 1), "bytes_per_step": tot_b,
                              "achieved": round(tot_b / tot_us / 1e3, 1), "peak": PEAK_HBM_GBS,
                              "unit": "GB/s", "frac": round(tot_b / tot_us / 1e3 / PEAK_HBM_GBS, 4)}
    return out


def accepted_path(model, mtp, cfg, B, prompt_len, k, steps, seed):
    """The step when every draft is accepted: temperature 0, drafts forced to the verify
    pass's own greedy fixed point (k rounds of the verify forward, not committed, so the
    argmax at position i already follows drafts 1..i), computed before each step outside
    the timed region; the step itself is the graph-replayed draft chain (its own drafts
    then overwritten by the forced ones), verify, greedy acceptance and commit, timed
    with HIP events around each replay.  Every sequence commits k + 1 tokens per step."""
    import torch
    from lollm_amd import ops
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed + 1)
    prompts = torch.randint(0, cfg.vocab_size, (B, prompt_len), device="cuda", generator=gen)
    n = (steps + 4) * (k + 1)
    dec = SpecDecoder(model, mtp, B, prompt_len + n + 8, k=k, temperature=0.0, out_capacity=n + 8)
    dec.prefill(prompts)
    forced = torch.zeros(B, k, dtype=torch.int32, device="cuda")
    lm = model.lm_head
    am = torch.empty(B * (k + 1), dtype=torch.int32, device="cuda")

    def fixed_point():
        d = torch.zeros(B, k, dtype=torch.int32, device="cuda")
        for _ in range(k):
            ids = torch.cat([dec.pending.view(B, 1), d], 1)
            _, normed = model.hidden_states(ids, dec.cache)
            ops.gemm_argmax(normed.reshape(-1, lm.K), lm.tiled, lm.N, lm.K, out=am, grid=lm.grid())
            d = am.view(B, k + 1)[:, :k].contiguous()
        forced.copy_(d)
    chain = dec._draft_chain

    def forced_chain():
        chain()
        dec.drafts.copy_(forced)
    dec._draft_chain = forced_chain
    for _ in range(2):
        fixed_point()
        dec.step()
    dec.capture()
    hist0 = dec.accept_hist.clone()
    total = 0.0
    for _ in range(steps):
        fixed_point()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        dec.replay()
        e1.record()
        torch.cuda.synchronize()
        total += e0.elapsed_time(e1)
    hist = (dec.accept_hist - hist0).cpu().tolist()
    ms = total / steps
    emitted = sum((i + 1) * c for i, c in enumerate(hist))
    ctx = float(dec.cache.lengths.float().mean())
    byt = step_bytes(cfg, B, k, (ctx - steps * (k + 1) / 2) * B, B * (k + 1), logits=False)
    del dec
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 4), "tok_s": round(emitted / (total / 1e3), 1),
            "tokens_per_step": round(emitted / steps, 2), "accepted_length_hist": hist,
            "steps": steps, "temperature": 0.0,
            "roofline_frac": round(byt["total"] / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
            "note": "drafts forced to the verify pass's greedy fixed point (computed outside "
                    "the timed region); every draft accepted, k + 1 tokens per sequence per step"}


# ------------------------------------------------------------------------------------
# isolated kernel workloads
# ------------------------------------------------------------------------------------
def isolated_gdn(B, kd, cpu=False):
    import torch
    from lollm_amd import ops
    Hk, Hv, D, T = 16, 32, 128, 1 + kd
    g = torch.Generator(device="cuda")
    g.manual_seed(2)
    q = torch.nn.functional.normalize(torch.randn(B, T, Hk, D, device="cuda", generator=g), dim=-1).bfloat16()
    k = torch.nn.functional.normalize(torch.randn(B, T, Hk, D, device="cuda", generator=g), dim=-1).bfloat16()
    v = torch.randn(B, T, Hv, D, device="cuda", generator=g).bfloat16()
    beta = torch.sigmoid(torch.randn(B, T, Hv, device="cuda", generator=g)).bfloat16()
    gg = -torch.nn.functional.softplus(torch.randn(B, T, Hv, device="cuda", generator=g))
    s0 = torch.randn(B, Hv, D, D, device="cuda", generator=g) * 0.02
    out = torch.empty(B, T, Hv, D, dtype=torch.bfloat16, device="cuda")
    snaps = torch.empty(B, T, Hv, D, D, device="cuda")
    us = time_fn(lambda: ops.gdn_verify(q, k, v, gg, beta, s0, out=out, snap_out=snaps), 50)
    byt = B * Hv * (1 + T) * D * D * 4 + B * T * (2 * Hk * D * 2 + 2 * Hv * D * 2 + Hv * 6)
    row = {"B": B, "T": T, "us": round(us, 2), "MB": round(byt / 1e6, 1),
           "GBs": round(byt / us / 1e3, 1), "frac": round(byt / us / 1e3 / PEAK_HBM_GBS, 3)}
    if cpu:
        # the reference's T > 1 path: repeat_interleave to the v-heads, then the chunked
        # delta rule (blocks.py:309-322), bf16 inputs computed as the reference does
        from oracle import qwen3_5_ref as R
        qc, kc, vc = (t.cpu() for t in (q, k, v))
        gc, bc, sc = gg.cpu(), beta.cpu(), s0.cpu()
        rep = Hv // Hk
        row["_cpu"] = lambda: time_cpu(lambda: R.gdn_scan_chunked(
            qc.repeat_interleave(rep, 2), kc.repeat_interleave(rep, 2), vc, gc, bc, state=sc))
    return row


PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_BF16_MFMA_TFLOPS = 2500.0
# MFMA instructions the chunked prefill kernel issues per (sequence, v-head, 64-token
# chunk): bf16 16x16x32 (k.k^T, q.k^T tiles; W^T and Tm diag(beta) V with Tm as hi + lo;
# W S with both operands hi + lo (3 products); Q S, intra V', K^T V' with one operand
# hi + lo) and fp32 16x16x4 (the off-diagonal blocks of the triangular solve)
GDN_CHUNK_BF16_MFMA = 40 + 40 + 96 + 480 + 400 + 256
GDN_CHUNK_FP32_MFMA = 64


def isolated_gdn_prefill(B=16, T=2048):
    """The chunked GDN prefill layer (conv + gating + chunked delta rule + gated norm)
    at the e2e prompt shape.  Two rates: the algorithm's fp32 products per (sequence,
    v-head, 64-token chunk) -- k.k^T and q.k^T (2 x 64x64x128), W and Tm diag(beta) V
    (2 x 64x128x64), W S and Q S (2 x 64x128x128), intra V' (64x128x64), K^T V'
    (128x128x64), 2 flops per multiply-add -- per second; and the MFMA work the kernel
    issues for them (bf16 with hi/lo operand splits, plus the fp32 solve products) as a
    fraction of the bf16 dense matrix peak.  Neither bound is reached: the chunks of a
    (sequence, head) run in sequence and each is a chain of dependent phases."""
    import torch
    from lollm_amd import ops
    Hk, Hv, D, K, S = 16, 32, 128, 4, 4
    C = 2 * Hk * D + Hv * D
    P = -(-(C + Hv * D + 2 * Hv) // 8) * 8
    g = torch.Generator(device="cuda")
    g.manual_seed(6)
    proj = torch.randn(B, T, P, device="cuda", generator=g).bfloat16()
    conv_w = (torch.randn(C, K, device="cuda", generator=g) * 0.5).bfloat16()
    A_log = torch.randn(Hv, device="cuda", generator=g) * 0.5
    dt_bias = torch.randn(Hv, device="cuda", generator=g) * 0.5
    norm_w = (1 + 0.1 * torch.randn(D, device="cuda", generator=g)).bfloat16()
    win = torch.zeros(B, 2 * (K - 1 + S), C, device="cuda").bfloat16()
    rec = torch.zeros(B, 2, Hv, D, D, device="cuda")
    rep = torch.zeros(B, 2, Hv, S, ops.gdn_record_bytes(D), dtype=torch.uint8, device="cuda")
    zero = torch.zeros(B, dtype=torch.int32, device="cuda")
    out = torch.empty(B, T, Hv * D, dtype=torch.bfloat16, device="cuda")
    us = time_fn(lambda: ops.gdn_layer(proj, conv_w, A_log, dt_bias, norm_w, win, zero, rec, zero,
                                       rep, zero, True, B, T, Hk, Hv, D, K, 1e-6, out=out,
                                       chunked=True), 5)
    C64 = 64
    per_chunk = 2 * (2 * C64 * C64 * D + 2 * C64 * D * C64 + 2 * C64 * D * D + C64 * D * C64 + D * D * C64)
    flops = B * Hv * (-(-T // C64)) * per_chunk
    tf = flops / us / 1e6
    chunks = B * Hv * (-(-T // C64))
    issued = chunks * (GDN_CHUNK_BF16_MFMA * 16 * 16 * 32 * 2 + GDN_CHUNK_FP32_MFMA * 16 * 16 * 4 * 2)
    mf = issued / us / 1e6
    return {"B": B, "T": T, "us": round(us, 1), "algorithmic_GFLOP": round(flops / 1e9, 1),
            "algorithmic_TFLOPs": round(tf, 2), "mfma_issued_GFLOP": round(issued / 1e9, 1),
            "mfma_TFLOPs": round(mf, 2), "bound": "latency (serial chunks)",
            "peak": PEAK_BF16_MFMA_TFLOPS, "frac": round(mf / PEAK_BF16_MFMA_TFLOPS, 3)}


def isolated_attn(cpu=False, step_shape=False):
    """The gated-attention verify kernel alone: the isolated shape (16 q / 2 kv heads,
    contexts U[1024, 32768]) or, with step_shape, the shape the dense 8B-class step runs
    (32 q / 4 kv heads, contexts U[2052, 2308]: a 2048-token prompt plus up to 256
    decoded tokens)."""
    import torch
    from lollm_amd import ops
    g = torch.Generator().manual_seed(3)
    if step_shape:
        B, T, Hq, Hkv, D, max_len = 16, 4, 32, 4, 256, 2312
        lens = torch.randint(2052, 2309, (B,), generator=g)
    else:
        B, T, Hq, Hkv, D, max_len = 16, 4, 16, 2, 256, 32768
        lens = torch.randint(1024, 32769, (B,), generator=g)
    q = torch.randn(B, T, Hq, D, device="cuda").bfloat16()
    kc = torch.randn(B, Hkv, max_len, D, device="cuda").bfloat16()
    vc = torch.randn(B, Hkv, max_len, D, device="cuda").bfloat16()
    gate = torch.randn(B, T, Hq * D, device="cuda").bfloat16()
    kl = lens.int().cuda()
    ws = torch.empty(ops.attn_workspace_bytes(B, T, Hq, Hkv, D, max_len), dtype=torch.uint8, device="cuda")
    out = torch.empty(B, T, Hq * D, dtype=torch.bfloat16, device="cuda")
    us = time_fn(lambda: ops.attn_verify(q, kc, vc, kl, gate, workspace=ws, out=out), 20)
    byt = int(lens.sum()) * Hkv * D * 2 * 2 + 3 * B * T * Hq * D * 2
    row = {"B": B, "T": T, "sum_ctx": int(lens.sum()), "us": round(us, 2),
           "MB": round(byt / 1e6, 1), "GBs": round(byt / us / 1e3, 1),
           "frac": round(byt / us / 1e3 / PEAK_HBM_GBS, 3)}
    if cpu:
        # one sequence at a time, as the reference's cache holds one length:
        # repeat_kv (blocks.py:152-156), SDPA with the offset-causal bool mask
        # (attention.py:43-51), sigmoid gate (blocks.py:235); bf16
        from oracle import qwen3_5_ref as R
        qc, gc = q.cpu(), gate.cpu()
        ks = [kc[b, :, :int(lens[b])].cpu() for b in range(B)]
        vs = [vc[b, :, :int(lens[b])].cpu() for b in range(B)]

        def ref():
            for b in range(B):
                qq = qc[b].transpose(0, 1)[None]                          # (1, Hq, T, D)
                kk = R.repeat_kv(ks[b][None], Hq // Hkv)
                vv = R.repeat_kv(vs[b][None], Hq // Hkv)
                o = R.sdpa_offset_causal(qq, kk, vv).transpose(1, 2).reshape(T, Hq * D)
                o * torch.sigmoid(gc[b])
        row["_cpu"] = lambda: time_cpu(ref)
    del kc, vc
    return row


def isolated_sampler(cpu=False):
    import torch
    from lollm_amd import ops
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    B, k, V = 64, 3, 151936
    tgt = torch.randn(B, k + 1, V, device="cuda", generator=g) * 3
    drf = (tgt[:, :k] + torch.randn(B, k, V, device="cuda", generator=g)).bfloat16()
    tgt = tgt.bfloat16()
    drafts = torch.stack([ops.sample_rows(drf[:, i].contiguous(), 0.7, 0, 0.95, 7, 0, slot=k + 1 + i)
                          for i in range(k)], 1)
    ws = torch.empty(ops._lib.lib().lollm_spec_workspace_bytes(B, k, 1), dtype=torch.uint8, device="cuda")
    na = torch.empty(B, dtype=torch.int32, device="cuda")
    nt = torch.empty(B, dtype=torch.int32, device="cuda")
    us = time_fn(lambda: ops.spec_accept(tgt, drf, drafts, 0.7, 0, 0.95, 7, 0, workspace=ws,
                                         n_accepted=na, next_token=nt), 20)
    byt = B * (2 * k + 1) * V * 2
    row = {"B": B, "k": k, "V": V, "us": round(us, 2), "MB": round(byt / 1e6, 1),
           "GBs": round(byt / us / 1e3, 1), "frac": round(byt / us / 1e3 / PEAK_HBM_GBS, 3)}
    if cpu:
        # the reference's sampler arithmetic (generate.py:23-36: sort, softmax, cumsum)
        # with the rejection rule, on the same logits and Philox uniforms
        from oracle import qwen3_5_ref as R
        from oracle import sampler_ref as S
        tc, dc, dr = tgt.float().cpu(), drf.float().cpu(), drafts.long().cpu()
        U = torch.tensor([[S.uniform_u24(7, 0, b, i) for i in range(k + 1)] for b in range(B)],
                         dtype=torch.float64) / 2 ** 24
        row["_cpu"] = lambda: time_cpu(lambda: R.spec_accept_sorted(tc, dr, 0.7, 0, 0.95, U, draft=dc))
    return row


# ------------------------------------------------------------------------------------
# CPU baseline: the oracle (torch-on-CPU restatement of the reference path)
# ------------------------------------------------------------------------------------
def time_cpu(fn, warm=3, reps=20, budget_s=30.0):
    """Median ms of fn() on the host: `warm` untimed runs, then up to `reps` timed runs
    within about budget_s seconds (at least 3).  Returns (median ms, runs)."""
    for _ in range(warm):
        fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < reps and (len(ts) < 3 or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        ts.append((time.perf_counter() - t0) * 1e3)
    return sorted(ts)[len(ts) // 2], len(ts)


def cpu_info():
    import torch
    model_name = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model_name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model_name, "os_cpu_count": os.cpu_count(),
            "torch_threads": torch.get_num_threads()}


def tiny_e2e(n_new=64):
    """The tiny CPU-runnable config: hidden 1024, 8 layers, vocab 32768, 1 MTP layer,
    seeded weights; B = 1, a 128-token prompt (seed 1), 64 greedy tokens with k = 1,
    prefill included.  GPU: SpecDecoder on the kernels (bf16, eager steps).  CPU: the
    oracle's generate_mtp loop in fp32 (mtp.py:92-162 with the reference's chunked GDN,
    masked SDPA and deep-copy rollback)."""
    import torch
    from lollm_amd.qwen3_5 import load, load_mtp
    from lollm_amd.qwen3_5.config import Qwen3_5Config, tiny_config_dict
    from lollm_amd.qwen3_5.mtp import SpecDecoder
    from lollm_amd.qwen3_5.random_init import random_weights
    from oracle import qwen3_5_ref as R
    raw = tiny_config_dict()
    cfg = Qwen3_5Config.from_hf(raw)
    W = random_weights(cfg, seed=0)
    Wb = {n: t.to(torch.bfloat16) for n, t in W.items()}
    prompt = torch.randint(0, cfg.vocab_size, (128,), generator=torch.Generator().manual_seed(1))
    weights = dict(Wb)
    model = load(raw, weights, "hf", device="cuda")
    mtp = load_mtp(model, weights, "hf", device="cuda")

    def gpu_run():
        dec = SpecDecoder(model, mtp, 1, 128 + n_new + 8, k=1, temperature=0.0, out_capacity=n_new + 4)
        dec.prefill(prompt.view(1, -1).cuda())
        while True:
            for _ in range(8):
                dec.step()
            if int(dec.out_count[0]) >= n_new:
                return
    gpu_run()
    torch.cuda.synchronize()
    ts = []
    for _ in range(5):
        t0 = time.perf_counter()
        gpu_run()
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t0)
    g_s = sorted(ts)[2]
    Wr = R.canonical_weights({n: t.float() for n, t in Wb.items()})
    rcfg = R.RefConfig.from_dict(raw)
    t0 = time.perf_counter()
    R.generate_mtp_greedy(Wr, rcfg, prompt.tolist(), n_new)
    c_s = time.perf_counter() - t0
    return {"gpu_tok_s": round(n_new / g_s, 1), "gpu_s": round(g_s, 4),
            "cpu_tok_s": round(n_new / c_s, 2), "cpu_s": round(c_s, 2),
            "sample": f"{n_new} greedy tokens after a 128-token prompt, k=1, B=1, prefill included "
                      "(GPU bf16 eager steps; CPU the oracle in fp32, 1 run)"}


def cpu_baseline(raw, cfg, keep, dec, k, temperature, top_p, seed):
    """One speculative step of the reference algorithm on the host cores, from the GPU
    run's committed state: the k-step MTP draft chain, the deep-copy snapshot of the
    cache (kv.py:49-54), the verify forward over 1 + k positions (chunked GDN for T > 1,
    SDPA with a bool mask over repeat_kv'd K/V), the rejection test, and the re-run of
    the pending token from the snapshot (mtp.py:156-162; with random weights every
    sequence rejects at its first draft, so the re-run is the common case).  fp32, all
    host threads.  Extrapolated to tok/s as (accepted + 1) * B / step time."""
    import numpy as np
    import torch
    from oracle import qwen3_5_ref as R
    from oracle import sampler_ref as S
    torch.set_num_threads(os.cpu_count())
    t_setup = time.time()
    W = R.canonical_weights({n: t.float().cpu() for n, t in keep.items()})
    rcfg = R.RefConfig.from_dict(raw)
    cache = dec.cache
    L = int(cache.lengths.min())
    past = R.RefCache(cfg.num_hidden_layers)
    for i in range(cfg.num_hidden_layers):
        if cfg.layer_type(i) == "full_attention":
            s = cache.layers[i]
            past.layers[i] = (s["k"][:, :, :L].float().cpu(), s["v"][:, :, :L].float().cpu())
        else:
            conv, rec = cache.linear_state(i)
            past.layers[i] = (conv.float().cpu(), rec.float().cpu())
    past.seen_tokens = L
    pending = dec.pending.long().cpu()
    h_last = dec.h_last.float().cpu()[:, None]
    log(f"cpu baseline setup {time.time() - t_setup:.1f} s (threads {torch.get_num_threads()})")
    B = pending.shape[0]
    steps, toks = 2, 0
    inv = S.inv_temperature(temperature)
    t0 = time.perf_counter()
    with torch.no_grad():
        for step in range(steps):
            drafts, _ = R.mtp_chain_draft(W, rcfg, h_last, pending, k)
            snap = past.clone()
            ids = torch.cat([pending[:, None], drafts], 1)
            logits, past, hid = R.model_forward(W, rcfg, ids, past, return_hidden=True)
            na, nt = S.spec_accept(logits.bfloat16(), None, drafts.numpy().astype(np.int32), inv,
                                   0, top_p, seed, 1 + step)
            if int(na.min()) == k:                   # every draft accepted (not with random weights)
                h_last = hid[:, k:]
            else:
                # reject: restore the snapshot and re-run the pending token (mtp.py:156-162);
                # the batch re-runs together, as the reference does for its one sequence
                past = snap
                _, past, hid1 = R.model_forward(W, rcfg, pending[:, None], past, return_hidden=True)
                h_last = hid1[:, -1:]
            toks += int(na.sum()) + B
            pending = torch.from_numpy(nt.astype(np.int64))
    step_s = (time.perf_counter() - t0) / steps
    info = cpu_info()
    return {"value": round(toks / (step_s * steps), 3), "unit": "tok/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"{steps} speculative steps (k={k}, B={B}, context {L}) of the CPU "
                       f"restatement (oracle/) in fp32 on {info['os_cpu_count']} host CPUs "
                       f"({info['cpu_model']}): {step_s:.2f} s/step, {toks} tokens; "
                       "extrapolated to tok/s"),
            "step_seconds": round(step_s, 3)}



# ------------------------------------------------------------------------------------
# HBM traffic: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs over `python3 bench.py
# --pmc-probe` (the hot kernels one by one) and `--pmc-probe-step` (whole steps), each
# calibrated by a plain copy-like kernel of known size in the same process; the
# figures are committed under profiles/ (step_traffic.json is the bench line's traffic)
# ------------------------------------------------------------------------------------
PROBE_COPY_BYTES = 256 << 20


PROBE_ORDER = ("gdn_layer", "gemm_qkv", "gemm_gate_up", "gemm_down", "attn_step", "spec_accept_c4",
               "lm_head_logits_step", "spec_accept_rowmax_step")


def pmc_probe(B=16, T=4, launches=20):
    """Launch each hot kernel `launches` times at the dense 8B-class step's shapes, in
    the order of PROBE_ORDER, then torch.neg over 256 MiB (reads and writes
    PROBE_COPY_BYTES each) 5 times as the counter calibration:
      gdn_layer       the fused GDN layer, B=16, T=4, 32 v / 16 qk heads of 128
      gemm_qkv        lollm_gemm, 64 rows x q|gate|k|v (N=18432) x K=4096, 192 WGs
      gemm_gate_up    lollm_gemm with the SwiGLU epilogue, 64 rows x N=24576 x K=4096, 256
      gemm_down       lollm_gemm, 64 rows x N=4096 x K=12288, 256 WGs + the merge launch
                      (the step merges it in lollm_gemm_rmsnorm's second kernel)
      attn_step       lollm_attn_verify, B=16, T=4, 32 q / 4 kv heads, contexts U[2052, 2308]
      spec_accept_c4  lollm_spec_accept, B=64, k=3, V=151936 with sampled drafts
      lm_head_logits_step      lollm_gemm_logits, the step's verify lm_head: 64 rows x
                      N=151936 x K=4096 with the repetition penalty and the row maxima
      spec_accept_rowmax_step  lollm_spec_accept_rowmax on those (16, 4, 151936) logits with
                      argmax drafts (the step's acceptance: each target row read once)
    Each GEMM rotates over enough weight copies (> 512 MB) that every launch streams its
    weights from HBM, as a step that walks every layer does."""
    import torch
    from lollm_amd import ops
    Hk, Hv, D, K, S = 16, 32, 128, 4, 4
    C = 2 * Hk * D + Hv * D
    P = -(-(C + Hv * D + 2 * Hv) // 8) * 8
    W = K - 1 + S
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    proj = torch.randn(B, T, P, device="cuda", generator=g).bfloat16()
    conv_w = (0.5 * torch.randn(C, K, device="cuda", generator=g)).bfloat16()
    A_log = torch.randn(Hv, device="cuda", generator=g) * 0.5
    dt_bias = torch.randn(Hv, device="cuda", generator=g) * 0.5
    norm_w = torch.ones(D, device="cuda").bfloat16()
    win = torch.zeros(B, 2 * W, C, device="cuda").bfloat16()
    rec = 0.02 * torch.randn(B, 2, Hv, D, D, device="cuda", generator=g)
    rep = torch.zeros(B, 2, Hv, S, ops.gdn_record_bytes(D), dtype=torch.uint8, device="cuda")
    conv_off = torch.zeros(B, dtype=torch.int32, device="cuda")
    rec_half = torch.zeros(B, dtype=torch.int32, device="cuda")
    replay = torch.full((B,), T, dtype=torch.int32, device="cuda")   # replays T records
    out = torch.empty(B, T, Hv * D, dtype=torch.bfloat16, device="cuda")
    for _ in range(launches):
        ops.gdn_layer(proj, conv_w, A_log, dt_bias, norm_w, win, conv_off, rec, rec_half, rep,
                      replay, False, B, T, Hk, Hv, D, K, 1e-6, out=out)
    del rec, rep, win
    M = B * T
    from lollm_amd.qwen3_5.blocks import gemm_grid
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for N, Kd, epi in ((18432, 4096, ops.GEMM_NONE), (24576, 4096, ops.GEMM_SWIGLU),
                       (4096, 12288, ops.GEMM_NONE)):
        copies = max(2, -(-(512 << 20) // (N * Kd * 2)))
        Wts = [ops.gemm_tile_weights((0.02 * torch.randn(N, Kd, device="cuda", generator=g)).bfloat16(), epi)
               for _ in range(copies)]
        x = torch.randn(M, Kd, device="cuda", generator=g).bfloat16()
        for i in range(launches):   # the step's grid for the shape
            ops.gemm(x, Wts[i % copies], N, Kd, epi, grid=gemm_grid(N, cus, M))
        del Wts
        torch.cuda.empty_cache()
    kv_len = torch.randint(2052, 2309, (16,), generator=torch.Generator().manual_seed(3)).int().cuda()
    q = torch.randn(16, 4, 32, 256, device="cuda", generator=g).bfloat16()
    kc = torch.randn(16, 4, 2312, 256, device="cuda", generator=g).bfloat16()
    vc = torch.randn(16, 4, 2312, 256, device="cuda", generator=g).bfloat16()
    gate = torch.randn(16, 4, 32 * 256, device="cuda", generator=g).bfloat16()
    for _ in range(launches):
        ops.attn_verify(q, kc, vc, kv_len, gate)
    del kc, vc
    Bs, k, V = 64, 3, 151936
    tgt = torch.randn(Bs, k + 1, V, device="cuda", generator=g) * 3
    drf = (tgt[:, :k] + torch.randn(Bs, k, V, device="cuda", generator=g)).bfloat16()
    tgt = tgt.bfloat16()
    drafts = torch.stack([ops.sample_rows(drf[:, i].contiguous(), 0.7, 0, 0.95, 7, 0, slot=k + 1 + i)
                          for i in range(k)], 1)
    for _ in range(launches):
        ops.spec_accept(tgt, drf, drafts, 0.7, 0, 0.95, 7, 0)
    del tgt, drf
    Vs, Ks = 151936, 4096
    Wl = ops.gemm_tile_weights((0.02 * torch.randn(Vs, Ks, device="cuda", generator=g)).bfloat16())
    xl = torch.randn(M, Ks, device="cuda", generator=g).bfloat16()
    seen = ops.new_seen(B, Vs, "cuda")
    ops.seen_mark(seen, torch.randint(0, Vs, (B, 2048), device="cuda", generator=g).int(), Vs)
    dr = torch.randint(0, Vs, (B, T - 1), device="cuda", generator=g).int()
    for _ in range(launches):
        lg, rm = ops.gemm_logits(xl, Wl, Vs, Ks, seen=seen, penalty=1.05, extra=dr, T=T,
                                 grid=gemm_grid(Vs, cus, M))
    for _ in range(launches):
        ops.spec_accept(lg.view(B, T, Vs), None, dr, 0.7, 0, 0.95, 7, 0, target_rowmax=rm)
    del Wl
    x = torch.randn(PROBE_COPY_BYTES // 4, device="cuda", generator=g)
    y = torch.empty_like(x)
    for _ in range(5):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    log(f"pmc probe: {launches} launches each of {', '.join(PROBE_ORDER)}; "
        f"5 x neg over {PROBE_COPY_BYTES} bytes")


STEP_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "step_traffic.json")
STEP_PROBE_STEPS = 3


def pmc_probe_step(B=16, prompt_len=2048, k=3):
    """For the counter runs of the whole step: the headline workload (model, prefill, two
    eager steps, the graph capture and two warm replays), then STEP_PROBE_STEPS graph
    replays between two marker kernels, then torch.neg over 256 MiB 5 times (the counter
    calibration).  summarize_pmc_step() sums each counter over the dispatches between
    the markers."""
    import torch
    raw, cfg, model, mtp, keep = build_8b(5)
    del keep
    dec, _ = run_e2e(model, mtp, cfg, B, prompt_len, k, STEP_PROBE_STEPS, 4, 0.7, 0.95, 5)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    x = torch.randn(PROBE_COPY_BYTES // 4, device="cuda", generator=g)
    y = torch.empty_like(x)
    for _ in range(5):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    log(f"pmc step probe: {STEP_PROBE_STEPS} replays between markers; 5 x neg over "
        f"{PROBE_COPY_BYTES} bytes")


def _csv_rows(directory, suffix):
    import csv
    import glob
    files = sorted(glob.glob(os.path.join(directory, "**", "*" + suffix), recursive=True))
    if not files:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    with open(files[0]) as f:
        return list(csv.DictReader(f))


def _between_markers(rows, key):
    """Rows strictly between the first two markers, ordered by `key` (a marker may be
    more than one consecutive scan kernel)."""
    rows = sorted(rows, key=lambda r: int(r[key]))
    idx = [i for i, r in enumerate(rows) if MARKER_KERNEL in r["Kernel_Name"]]
    j = 1
    while j < len(idx) and idx[j] == idx[j - 1] + 1:
        j += 1
    if j >= len(idx):
        raise ValueError("the two timed-region markers are not in the trace")
    return rows[idx[j - 1] + 1:idx[j]]


def summarize_pmc_step(directory, out=STEP_TRAFFIC_FILE):
    """FETCH_SIZE and WRITE_SIZE (KiB per dispatch, rocprofv3 --pmc over
    `bench.py --pmc-probe-step`, in <directory>/pmc_FETCH_SIZE and pmc_WRITE_SIZE) summed
    over the dispatches of the probe's timed replays, per step, each counter scaled by
    what it reads for torch.neg over 256 MiB (which reads and writes 256 MiB)."""
    import statistics
    res = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        rows = _csv_rows(os.path.join(directory, f"pmc_{ctr}"), "counter_collection.csv")
        step = _between_markers(rows, "Dispatch_Id")
        neg = [float(r["Counter_Value"]) for r in rows if "neg" in r["Kernel_Name"]][-5:]
        scale = (PROBE_COPY_BYTES / 1024) / statistics.median(neg)
        total = sum(float(r["Counter_Value"]) for r in step)
        res[ctr] = {"kib_per_step": total / STEP_PROBE_STEPS, "dispatches_per_step":
                    len(step) / STEP_PROBE_STEPS, "copy_kib": statistics.median(neg),
                    "scale": round(scale, 6), "bytes_per_step": int(total / STEP_PROBE_STEPS * 1024 * scale)}
    t = {"workload": "dense 8B-class step, B=16, k=3, T=0.7, 2048-token prompts",
         "fetch": res["FETCH_SIZE"], "write": res["WRITE_SIZE"],
         "traffic_bytes_per_step": res["FETCH_SIZE"]["bytes_per_step"] + res["WRITE_SIZE"]["bytes_per_step"],
         "copy_kernel": "torch.neg over 256 MiB fp32 (reads and writes 268435456 bytes)",
         "commands": [f"cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc {c} --output-format csv "
                      f"-d <out>/pmc_{c} -o run -- python3 <repo>/bench.py --pmc-probe-step"
                      for c in ("FETCH_SIZE", "WRITE_SIZE")] +
                     ["python3 bench.py --summarize-pmc-step <out>"]}
    with open(out, "w") as f:
        json.dump(t, f, indent=1)
    print(json.dumps(t, indent=1))


def summarize_pmc_probe(directory):
    """The hot-kernel table of `bench.py --pmc-probe`: FETCH_SIZE / WRITE_SIZE (rocprofv3
    --pmc, in <directory>/pmc_FETCH_SIZE and pmc_WRITE_SIZE) and durations (a
    --kernel-trace run in <directory>/pmc_trace) per launch, medians over each item's
    launches, counters scaled by the torch.neg calibration, against each kernel's
    algorithmic bytes."""
    import statistics
    import torch
    from lollm_amd.qwen3_5.config import Qwen3_5Config, dense_8b_config_dict
    cfg = Qwen3_5Config.from_hf(dense_8b_config_dict())

    def by_kernel(rows, key, val):
        out = {}
        for r in sorted(rows, key=lambda r: int(r[key])):
            out.setdefault(r["Kernel_Name"].split("(")[0].replace("void ", ""), []).append(val(r))
        return out
    F = by_kernel(_csv_rows(os.path.join(directory, "pmc_FETCH_SIZE"), "counter_collection.csv"),
                  "Dispatch_Id", lambda r: float(r["Counter_Value"]))
    W = by_kernel(_csv_rows(os.path.join(directory, "pmc_WRITE_SIZE"), "counter_collection.csv"),
                  "Dispatch_Id", lambda r: float(r["Counter_Value"]))
    D = by_kernel(_csv_rows(os.path.join(directory, "pmc_trace"), "kernel_trace.csv"),
                  "Start_Timestamp",
                  lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    neg = next(n for n in F if "neg" in n)
    fs = PROBE_COPY_BYTES / 1024 / statistics.median(F[neg][-5:])
    ws = PROBE_COPY_BYTES / 1024 / statistics.median(W[neg][-5:])
    lens = torch.randint(2052, 2309, (16,), generator=torch.Generator().manual_seed(3))
    V, M = 151936, 64
    gm = lambda N, K, out: N * K * 2 + M * K * 2 + M * out * 2  # noqa: E731
    items = [  # label, kernel, which of its launches, algorithmic bytes
        ("gdn_layer B16 T4 (4 records replayed)", "lollm::gdn_layer_verify_kernel", slice(0, 20),
         gdn_layer_bytes(cfg, 16, 4, 64)),
        ("gemm q|gate|k|v 64x18432x4096", "lollm::gemm_stream_kernel<6>", slice(0, 20), gm(18432, 4096, 18432)),
        ("gemm gate|up 64x24576x4096 (SwiGLU)", "lollm::gemm_stream_kernel<6>", slice(20, 40), gm(24576, 4096, 12288)),
        ("gemm down 64x4096x12288", "lollm::gemm_stream_kernel<4>", slice(0, 20), gm(4096, 12288, 4096)),
        ("  its merge", "lollm::gemm_fixup_kernel", slice(0, 20), None),
        ("attention, the step's shape", "lollm::attn_verify_kernel", slice(0, 20),
         int(lens.sum()) * 4 * 256 * 4 + 3 * 16 * 4 * 32 * 256 * 2),
        ("  attn_combine", "lollm::attn_combine_kernel", slice(0, 20), None),
        ("C4 acceptance: row_stats (448 rows, max found by the kernel)", "lollm::row_stats_kernel",
         slice(0, 20), 64 * 7 * V * 2),
        ("  spec_partial", "lollm::spec_partial_kernel", slice(0, 20), None),
        ("  spec_final", "lollm::spec_final_kernel", slice(0, 20), None),
        ("step lm_head with penalty and row maxima 64x151936x4096", "lollm::gemm_stream_kernel<4>",
         slice(20, 40), gm(V, 4096, V)),
        ("  its merge", "lollm::gemm_fixup_kernel", slice(20, 40), None),
        ("step acceptance: row_stats (64 rows, maxima given)", "lollm::row_stats_known_kernel",
         slice(0, 20), 64 * V * 2),
        ("  spec_partial", "lollm::spec_partial_kernel", slice(20, 40), None),
        ("  spec_final", "lollm::spec_final_kernel", slice(20, 40), None),
    ]
    print(f"calibration: {neg[:50]}: FETCH_SIZE scale {fs:.5f}, WRITE_SIZE scale {ws:.5f}\n")
    print("| kernel | us | HBM bytes (fetch + write) | algorithmic bytes | traffic / algorithmic | frac of 8 TB/s |")
    print("|---|---:|---:|---:|---:|---:|")
    for label, k, sl, alg in items:
        if k not in F or not F[k][sl]:
            print(f"| {label} | (not in the runs) | | | | |")
            continue
        f = statistics.median(F[k][sl]) * 1024 * fs
        w = statistics.median(W[k][sl]) * 1024 * ws
        t = statistics.median(D[k][sl])
        if alg:
            print(f"| {label} | {t:.2f} | {int(f + w)} | {alg} | {(f + w) / alg:.3f} | "
                  f"{alg / t / 1e3 / PEAK_HBM_GBS:.3f} |")
        else:
            print(f"| {label} | {t:.2f} | {int(f + w)} | | | |")


def measured_step_traffic():
    try:
        with open(STEP_TRAFFIC_FILE) as f:
            return json.load(f).get("traffic_bytes_per_step")
    except (OSError, ValueError):
        return None


def summarize_trace(directory, steps=None):
    """Markdown table of one timed step from `rocprofv3 --kernel-trace` of bench.py (the
    csv under <directory>): every kernel between the two timed-region markers, per step
    (total, launches, average), the step's span, and the bench line's step time for
    comparison."""
    import collections
    rows = _between_markers(_csv_rows(directory, "kernel_trace.csv"), "Start_Timestamp")
    if steps is None:
        steps = sum(1 for r in rows if "spec_commit_kernel" in r["Kernel_Name"])
    span = (int(rows[-1]["End_Timestamp"]) - int(rows[0]["Start_Timestamp"])) / 1e3 / steps
    agg = collections.defaultdict(lambda: [0.0, 0])
    for r in rows:
        name = r["Kernel_Name"].split("(")[0].replace("void ", "")
        a = agg[name]
        a[0] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        a[1] += 1
    busy = sum(v[0] for v in agg.values()) / steps
    print(f"timed steps: {steps}; span per step {span:.1f} us; kernel time per step {busy:.1f} us; "
          f"launches per step {len(rows) / steps:.1f}\n")
    print("| us per step | launches per step | avg us | % of span | kernel |")
    print("|---:|---:|---:|---:|---|")
    for name, (us, n) in sorted(agg.items(), key=lambda kv: -kv[1][0]):
        print(f"| {us / steps:.1f} | {n / steps:.1f} | {us / n:.2f} | {100 * us / steps / span:.1f} | `{name[:80]}` |")


# ------------------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--prompt-len", type=int, default=2048)
    ap.add_argument("--k", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-isolated", action="store_true", help="skip the isolated kernels")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="only launch the hot kernels and a copy calibration (for rocprofv3 --pmc)")
    ap.add_argument("--pmc-probe-step", action="store_true",
                    help="only replay the step between markers and a copy calibration (for rocprofv3 --pmc)")
    ap.add_argument("--summarize-pmc-step", metavar="DIR",
                    help="write profiles/step_traffic.json from the two --pmc-probe-step counter runs")
    ap.add_argument("--summarize-pmc", metavar="DIR",
                    help="print the hot-kernel traffic table of the --pmc-probe counter and trace runs")
    ap.add_argument("--summarize-trace", metavar="DIR",
                    help="print the per-step kernel table of a rocprofv3 --kernel-trace of bench.py")
    ap.add_argument("--accepted-steps", type=int, default=32,
                    help="timed steps of the accepted path (0: skip it)")
    args = ap.parse_args()
    if args.summarize_pmc_step:
        summarize_pmc_step(args.summarize_pmc_step)
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace)
        return
    if args.summarize_pmc:
        summarize_pmc_probe(args.summarize_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU's share of the workload; --gpus {args.gpus} is not "
              "supported (this build runs on a single MI355X)", file=sys.stderr)
        sys.exit(2)
    import torch
    from lollm_amd import _lib
    _lib.lib()                                    # fail loudly if the kernels are not built
    if args.pmc_probe:
        pmc_probe()
        return
    if args.pmc_probe_step:
        pmc_probe_step(args.batch, args.prompt_len, args.k)
        return
    temperature, top_p, seed = 0.7, 0.95, 5
    t0 = time.time()
    raw, cfg, model, mtp, keep = build_8b(seed)
    log(f"model built in {time.time() - t0:.1f} s")
    dec, e2e = run_e2e(model, mtp, cfg, args.batch, args.prompt_len, args.k, args.steps,
                       args.warmup, temperature, top_p, seed)
    value = e2e["emitted"] / e2e["seconds"]
    ms_per_step = e2e["seconds"] * 1000.0 / args.steps
    log(f"e2e: {value:.1f} tok/s, {ms_per_step:.3f} ms/step, hist {e2e['hist']}")
    # the step's roofline: algorithmic bytes of one graph replay over its HIP-event time
    sb = step_bytes(cfg, args.batch, args.k, e2e["ctx_sum_mean"],
                    args.batch * (1 + e2e["mean_accepted"]), logits=not dec.greedy_argmax)
    gbs = sb["total"] / (ms_per_step * 1e-3) / 1e9
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": measured_step_traffic()}
    log(f"step: {sb['total'] / 1e9:.2f} GB algorithmic, {gbs:.0f} GB/s, frac {roof['frac']}")
    parts = verify_breakdown(dec)
    kernels = {"in_step": in_step_kernels(model, mtp, dec)}
    for key, v in kernels["in_step"].items():
        log(f"in step {key}: {v.get('avg_us', v.get('us_per_step'))} us, frac {v['frac']}")
    accepted = None
    if args.accepted_steps > 0:
        accepted = accepted_path(model, mtp, cfg, args.batch, args.prompt_len, args.k,
                                 args.accepted_steps, seed)
        log(f"accepted path: {accepted['ms_per_step']} ms/step, {accepted['tok_s']} tok/s")
    cpu_legs = not args.no_cpu
    if cpu_legs:
        torch.set_num_threads(os.cpu_count())
    if not args.no_isolated:
        kernels["gdn_verify_isolated"] = [isolated_gdn(B, kd, cpu=cpu_legs)
                                          for B in (1, 8, 32) for kd in (1, 2, 4)]
        kernels["attn_verify_isolated"] = isolated_attn(cpu=cpu_legs)
        kernels["attn_verify_step_shape"] = isolated_attn(step_shape=True)
        kernels["spec_accept_isolated"] = isolated_sampler(cpu=cpu_legs)
        kernels["gdn_prefill_chunked"] = isolated_gdn_prefill()
        kernels["tiny_e2e"] = tiny_e2e() if cpu_legs else None
        # the CPU legs of the isolated workloads, after every GPU timing (a GPU left idle
        # through seconds of host work clocks down and would time its next kernels slow)
        for row in kernels["gdn_verify_isolated"] + [kernels["attn_verify_isolated"],
                                                     kernels["spec_accept_isolated"]]:
            leg = row.pop("_cpu", None)
            if leg is not None:
                ms, n = leg()
                row.update(cpu_ms=round(ms, 2), cpu_runs=n,
                           gpu_speedup=round(ms * 1e3 / row["us"], 1))
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(raw, cfg, keep, dec, args.k, temperature, top_p, seed)
        except Exception as exc:                  # the CPU leg must not hide the GPU result
            log(f"cpu baseline failed: {exc!r}")
    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: seeded random-init weights, uniform random prompt ids",
        "config": {"workload": "qwen3_5 MTP speculative decode: dense 8B-class hybrid "
                               "(hidden 4096, 32 layers 3:1 GDN:attn, vocab 151936) + 1-layer "
                               f"MTP, B={args.batch}, {args.prompt_len}-token prompts, "
                               f"k={args.k}, T=0.7, top-p 0.95",
                   "global_batch": args.batch, "seq_len": args.prompt_len, "k": args.k,
                   "parallelism": "single GPU"},
        "accepted_length_hist": e2e["hist"], "mean_accepted": round(e2e["mean_accepted"], 4),
        "verify_step_us": round(parts["verify_forward_us"], 1), "step_parts_us":
            {k_: round(v, 1) for k_, v in parts.items()},
        "roofline": roof,
        "roofline_kernel": "the whole speculative step: one graph replay (draft chain, verify "
                           "forward, acceptance, commit)",
        "roofline_bytes": {k_: int(v) for k_, v in sb.items()},
        "accepted_path": accepted,
        "projection_paths": projection_paths(model, mtp, args.batch, args.k),
        "kernels": kernels,
        "cpu_baseline": cpu,
        "cpu_host": cpu_info() if cpu_legs else None,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
