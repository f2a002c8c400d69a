"""Torch-on-CPU restatement of the reference qwen3_5 float path -- TEST ORACLE ONLY.

Never imported by the product (`lollm_amd`).  Every function cites the reference
file:line it restates (paths relative to the giapnguyen74/lollm checkout).  The code
works on a flat dict of weights keyed by the reference's module names
(`model.layers.{i}.linear_attn.in_proj_qkv.weight`, `mtp.fc.weight`, ...), which is the
name space `src/qwen3_5/weights.py:27-37` maps checkpoint names into.

How each piece is pinned (see tests/test_oracle_*.py):
  * gdn_scan_recurrent / gdn_scan_chunked / l2_normalize / rmsnorm_gated /
    rope_apply / rmsnorm_plus1: golden vectors written by tests/golden/make_golden.py
    from the transformers 5.15.0 Qwen3_5 functions (same math lineage as the
    reference), plus closed forms (T=1 step, beta=0 pure decay, zero state with
    g=0,beta=1 => S = k v^T), chunked == recurrent, and an fp64 brute force.
  * sdpa_offset_causal: fp64 textbook softmax(QK^T/sqrt(D) + mask) V and the
    offset-causal rule; decode (q_len == 1) and plain-causal special cases.
  * model_forward (+ RefCache): transformers Qwen3_5ForCausalLM logits on the same
    random weights (prefill and cached decode), and prefill == incremental.
  * mtp_forward / speculate / generate_mtp_greedy / generate_greedy: vectors written by
    tests/golden/make_golden_ref.py from the reference itself (MTP.forward at L = 1..4 and
    explicit positions, speculate, and the greedy generate_mtp / generate trajectories
    with and without a repetition penalty on the tiny and micro models), plus the L=1
    closed form (softmax over one key => attention output = v).
  * sample_next: the reference's own greedy picks under a repetition penalty
    (tests/golden/ref_mtp.safetensors), temperature->0 == argmax, top_p/top_k keep-set
    rules on hand-built distributions.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------------
# config (reference: src/qwen3_5/config.py:15-101)
# ---------------------------------------------------------------------------------
@dataclass
class RefConfig:
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    partial_rotary_factor: float
    tie_word_embeddings: bool
    layer_types: list
    linear_num_key_heads: int
    linear_num_value_heads: int
    linear_key_head_dim: int
    linear_value_head_dim: int
    linear_conv_kernel_dim: int

    @classmethod
    def from_dict(cls, raw: dict) -> "RefConfig":
        """config.py:70-101: text sub-config, rope params, defaults."""
        t = raw.get("text_config", raw)
        nh = t["num_attention_heads"]
        rp = t.get("rope_parameters", {})
        return cls(
            vocab_size=t["vocab_size"], hidden_size=t["hidden_size"],
            intermediate_size=t["intermediate_size"],
            num_hidden_layers=t["num_hidden_layers"], num_attention_heads=nh,
            num_key_value_heads=t.get("num_key_value_heads", nh),
            head_dim=t.get("head_dim", t["hidden_size"] // nh),
            rms_norm_eps=t.get("rms_norm_eps", 1e-6),
            rope_theta=rp.get("rope_theta", t.get("rope_theta", 1e7)),
            partial_rotary_factor=rp.get("partial_rotary_factor",
                                         t.get("partial_rotary_factor", 1.0)),
            tie_word_embeddings=t.get("tie_word_embeddings",
                                      raw.get("tie_word_embeddings", False)),
            layer_types=list(t["layer_types"]),
            linear_num_key_heads=t["linear_num_key_heads"],
            linear_num_value_heads=t["linear_num_value_heads"],
            linear_key_head_dim=t["linear_key_head_dim"],
            linear_value_head_dim=t["linear_value_head_dim"],
            linear_conv_kernel_dim=t["linear_conv_kernel_dim"])

    # derived dims, config.py:42-65
    @property
    def n_rep(self):
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def rotary_dim(self):
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def key_dim(self):
        return self.linear_key_head_dim * self.linear_num_key_heads

    @property
    def value_dim(self):
        return self.linear_value_head_dim * self.linear_num_value_heads

    @property
    def conv_dim(self):
        return 2 * self.key_dim + self.value_dim

    @property
    def v_per_k(self):
        return self.linear_num_value_heads // self.linear_num_key_heads


def canonical_weights(raw_weights: dict) -> dict:
    """Inverse of weights.py:27-37 (`model.` <-> `model.language_model.`)."""
    out = {}
    for name, t in raw_weights.items():
        if name.startswith("model.language_model."):
            name = "model." + name[len("model.language_model."):]
        out[name] = t
    if "lm_head.weight" not in out:                       # weights.py:42,66-67 (tied)
        out["lm_head.weight"] = out["model.embed_tokens.weight"]
    return out


# ---------------------------------------------------------------------------------
# primitives (reference: src/qwen3_5/blocks.py)
# ---------------------------------------------------------------------------------
def linear(x, w):
    return x @ w.t()


def rmsnorm_plus1(x, w, eps):
    """blocks.py:23-35 -- fp32 mean-square norm, scaled by (1 + w), cast back."""
    xf = x.float()
    inv = torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)
    return (xf * inv * (1.0 + w.float())).to(x.dtype)


def rmsnorm_gated(x, z, w, eps):
    """blocks.py:38-51 -- normalise in fp32, cast to x.dtype, multiply by w (in the
    weight's dtype promotion), then by silu(z) in fp32, cast back."""
    dt = x.dtype
    xf = x.float()
    xn = (xf * torch.rsqrt(xf.square().mean(dim=-1, keepdim=True) + eps)).to(dt)
    h = w * xn
    return (h * F.silu(z.float())).to(dt)


def l2_normalize(x, eps=1e-6):
    """blocks.py:54-56 -- x / sqrt(sum x^2 + eps) over the last dim, in x.dtype."""
    return x * torch.rsqrt(x.square().sum(dim=-1, keepdim=True) + eps)


def gdn_scan_recurrent(q, k, v, g, beta, state=None, qk_l2=False):
    """blocks.py:116-144.  q,k,v: (B,T,H,D); g,beta: (B,T,H).  Per step t:
        S <- S * exp(g_t);  d = (v_t - S^T k_t) * beta_t;  S <- S + k_t d^T;
        o_t = S^T (q_t * Dk^-0.5)
    The scan runs in fp32; returns (o in q.dtype, final S fp32)."""
    dt = q.dtype
    if qk_l2:
        q, k = l2_normalize(q), l2_normalize(k)
    qf, kf, vf, bf, gf = (t.transpose(1, 2).float() for t in (q, k, v, beta, g))
    B, H, T, dk = kf.shape
    dv = vf.shape[-1]
    qf = qf * dk ** -0.5
    S = (torch.zeros(B, H, dk, dv) if state is None else state.float().clone())
    o = torch.empty(B, H, T, dv)
    for t in range(T):
        S = S * gf[:, :, t].exp()[..., None, None]
        kv = torch.einsum("bhij,bhi->bhj", S, kf[:, :, t])
        d = (vf[:, :, t] - kv) * bf[:, :, t][..., None]
        S = S + kf[:, :, t][..., :, None] * d[..., None, :]
        o[:, :, t] = torch.einsum("bhij,bhi->bhj", S, qf[:, :, t])
    return o.transpose(1, 2).contiguous().to(dt), S


def gdn_scan_recurrent_snapshots(q, k, v, g, beta, state=None, qk_l2=False):
    """The recurrent scan of blocks.py:116-144 with the state after every position
    kept: returns (o, snaps) with snaps (B, T, H, Dk, Dv) fp32, snaps[:, t] = state
    after positions 0..t.  (The build's verify contract; snaps[:, -1] is the final
    state the reference returns.)"""
    T = q.shape[1]
    snaps = []
    S = state
    outs = []
    for t in range(T):
        sl = slice(t, t + 1)
        o, S = gdn_scan_recurrent(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl],
                                  S, qk_l2)
        outs.append(o)
        snaps.append(S.clone())
    return torch.cat(outs, 1), torch.stack(snaps, 1)


def gdn_scan_chunked(q, k, v, g, beta, chunk=64, state=None, qk_l2=False):
    """blocks.py:59-113 -- the same recurrence in chunks of `chunk` positions:
    within a chunk, the delta-rule correction (I - A)^-1 is built row by row, the
    intra-chunk part is a masked matmul, and the state crosses chunk boundaries."""
    dt = q.dtype
    if qk_l2:
        q, k = l2_normalize(q), l2_normalize(k)
    qf, kf, vf, bf, gf = (t.transpose(1, 2).contiguous().float()
                          for t in (q, k, v, beta, g))
    B, H, T, dk = kf.shape
    dv = vf.shape[-1]
    pad = (-T) % chunk
    if pad:
        qf, kf, vf = (F.pad(t, (0, 0, 0, pad)) for t in (qf, kf, vf))
        bf, gf = F.pad(bf, (0, pad)), F.pad(gf, (0, pad))
    n = (T + pad) // chunk
    qf = qf * dk ** -0.5
    kb = kf * bf[..., None]
    vb = vf * bf[..., None]
    r = lambda t: t.reshape(B, H, n, chunk, t.shape[-1])
    qc, kc, vc, kbc, vbc = r(qf), r(kf), r(vf), r(kb), r(vb)
    gc = gf.reshape(B, H, n, chunk).cumsum(-1)
    # decay[i, j] = exp(G_i - G_j) for j <= i, 0 above the diagonal
    diff = gc[..., :, None] - gc[..., None, :]
    lower = torch.ones(chunk, chunk, dtype=torch.bool).tril()
    decay = torch.where(lower, diff, torch.zeros(())).exp() * lower
    A = -(kbc @ kc.transpose(-1, -2)) * decay
    A = A.masked_fill(~torch.ones(chunk, chunk, dtype=torch.bool).tril(-1), 0.0)
    for i in range(1, chunk):                   # forward substitution, row by row
        row = A[..., i, :i].clone()
        A[..., i, :i] = row + (row[..., :, None] * A[..., :i, :i]).sum(-2)
    A = A + torch.eye(chunk)
    u = A @ vbc
    w = A @ (kbc * gc.exp()[..., None])
    S = torch.zeros(B, H, dk, dv) if state is None else state.float().clone()
    o = torch.zeros(B, H, n, chunk, dv)
    strict_upper = torch.ones(chunk, chunk, dtype=torch.bool).triu(1)
    for c in range(n):
        qi, ki = qc[:, :, c], kc[:, :, c]
        intra = ((qi @ ki.transpose(-1, -2)) * decay[:, :, c]).masked_fill(strict_upper, 0)
        vnew = u[:, :, c] - w[:, :, c] @ S
        o[:, :, c] = (qi * gc[:, :, c, :, None].exp()) @ S + intra @ vnew
        glast = gc[:, :, c, -1]
        S = (S * glast.exp()[..., None, None]
             + (ki * (glast[..., None] - gc[:, :, c]).exp()[..., None]).transpose(-1, -2) @ vnew)
    o = o.reshape(B, H, n * chunk, dv)[:, :, :T]
    return o.transpose(1, 2).contiguous().to(dt), S


def rope_tables(positions, rotary_dim, theta, dtype):
    """blocks.py:159-173 -- inv_freq = theta^-(2i/rd); cos/sin of cat(freqs, freqs)."""
    idx = torch.arange(0, rotary_dim, 2, dtype=torch.float32)
    inv_freq = 1.0 / (theta ** (idx / rotary_dim))
    f = positions.float()[..., None] * inv_freq
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rope_apply(x, cos, sin):
    """blocks.py:175-183 -- rotate-half RoPE on the first rd = cos.shape[-1] dims of
    x (..., T, D); cos/sin broadcast as (T, rd)."""
    rd = cos.shape[-1]
    xr, xp = x[..., :rd], x[..., rd:]
    half = rd // 2
    rot = torch.cat([-xr[..., half:], xr[..., :half]], dim=-1)
    return torch.cat([xr * cos + rot * sin, xp], dim=-1)


def repeat_kv(x, n_rep):
    """blocks.py:152-156 -- head h of the output is KV head h // n_rep."""
    return x if n_rep == 1 else x.repeat_interleave(n_rep, dim=1)


def sdpa_offset_causal(q, k, v):
    """attention.py:43-51 -- query i of q_len sits at absolute total_k - q_len + i and
    sees keys at positions <= that; plain causal when q_len == total_k; no mask
    for q_len == 1.  Scale D^-0.5 (the SDPA default)."""
    q_len, total_k = q.shape[-2], k.shape[-2]
    if q_len > 1 and q_len != total_k:
        qpos = torch.arange(total_k - q_len, total_k)
        kpos = torch.arange(total_k)
        mask = (kpos[None, :] <= qpos[:, None])[None, None]
        return F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    return F.scaled_dot_product_attention(q, k, v, is_causal=q_len > 1)


# ---------------------------------------------------------------------------------
# cache (reference: src/qwen3_5/kv.py:20-58)
# ---------------------------------------------------------------------------------
class RefCache:
    """kv.py:20-58 -- per-layer (K, V) grown by concatenation, or (conv, rec);
    one scalar position counter; clone() deep-copies every tensor."""

    def __init__(self, n_layers):
        self.layers = [None] * n_layers
        self.seen_tokens = 0

    def append_kv(self, layer, k, v):
        cur = self.layers[layer]
        if cur is not None:
            k, v = torch.cat([cur[0], k], 2), torch.cat([cur[1], v], 2)
        self.layers[layer] = (k, v)
        return k, v

    def read_kv(self, layer):
        return self.layers[layer]

    def linear_state(self, layer):
        return self.layers[layer] or (None, None)

    def set_linear_state(self, layer, conv, rec):
        self.layers[layer] = (conv, rec)

    def advance(self, n):
        self.seen_tokens += n

    def clone(self):
        c = RefCache(len(self.layers))
        c.seen_tokens = self.seen_tokens
        c.layers = [None if s is None else tuple(t.clone() for t in s) for s in self.layers]
        return c


# ---------------------------------------------------------------------------------
# mixers, MLP, layers, model (blocks.py:186-342, modeling_qwen3_5.py:27-102)
# ---------------------------------------------------------------------------------
def gated_attention(W, p, cfg, x, cos, sin, cache=None, layer=0):
    """blocks.py:211-236.  q_proj packs [query | gate] per head; QK-norm; partial
    RoPE; cache append post-RoPE pre-GQA; offset-causal SDPA; o * sigmoid(gate)."""
    b, t, _ = x.shape
    H, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    qg = linear(x, W[p + "q_proj.weight"]).view(b, t, H, 2 * D)
    q, gate = qg[..., :D], qg[..., D:]
    gate = gate.reshape(b, t, H * D)
    q = rmsnorm_plus1(q, W[p + "q_norm.weight"], cfg.rms_norm_eps).transpose(1, 2)
    k = rmsnorm_plus1(linear(x, W[p + "k_proj.weight"]).view(b, t, Hkv, D),
                      W[p + "k_norm.weight"], cfg.rms_norm_eps).transpose(1, 2)
    v = linear(x, W[p + "v_proj.weight"]).view(b, t, Hkv, D).transpose(1, 2)
    q, k = rope_apply(q, cos, sin), rope_apply(k, cos, sin)
    if cache is not None:
        k, v = cache.append_kv(layer, k, v)
    o = sdpa_offset_causal(q, repeat_kv(k, cfg.n_rep), repeat_kv(v, cfg.n_rep))
    o = o.transpose(1, 2).reshape(b, t, H * D) * torch.sigmoid(gate)
    return linear(o, W[p + "o_proj.weight"])


def causal_conv(W, p, cfg, qkv, conv_state):
    """blocks.py:268-286.  qkv: (B, C, L) raw projections.  Depthwise causal conv
    (kernel K, no bias) over [conv_state | qkv] + SiLU; the new state is the last
    K-1 RAW input columns (left zero-padded when fewer exist)."""
    K = cfg.linear_conv_kernel_dim
    w = W[p + "conv1d.weight"]                             # (C, 1, K)
    L = qkv.shape[-1]
    xx = qkv if conv_state is None else torch.cat([conv_state, qkv], -1)
    padded = F.pad(xx, (K - 1, 0))
    out = F.silu(F.conv1d(padded, w, None, groups=xx.shape[1]))
    out = out[..., -L:]
    n = xx.shape[-1]
    new_state = xx[..., n - (K - 1):] if n >= K - 1 else F.pad(xx, (K - 1 - n, 0))
    return out, new_state


def gated_deltanet(W, p, cfg, x, conv_state=None, rec_state=None, use_cache=False):
    """blocks.py:288-329.  Projections -> causal conv -> split q,k,v -> heads
    (q,k repeated to the v-head count, v-head h uses qk-head h // v_per_k) ->
    beta = sigmoid(b) in x.dtype, g = -exp(A_log) softplus(a + dt_bias) in fp32 ->
    recurrent scan for cached T == 1, chunked otherwise (both with in-kernel l2norm)
    -> gated RMSNorm per v-head with gate z -> out_proj."""
    B, T, _ = x.shape
    Hk, Hv = cfg.linear_num_key_heads, cfg.linear_num_value_heads
    dk, dv = cfg.linear_key_head_dim, cfg.linear_value_head_dim
    cached = conv_state is not None
    qkv = linear(x, W[p + "in_proj_qkv.weight"]).transpose(1, 2)
    z = linear(x, W[p + "in_proj_z.weight"]).reshape(B, T, Hv, dv)
    bb = linear(x, W[p + "in_proj_b.weight"])
    aa = linear(x, W[p + "in_proj_a.weight"])
    act, new_conv = causal_conv(W, p, cfg, qkv, conv_state)
    act = act.transpose(1, 2)
    q = act[..., :cfg.key_dim].reshape(B, T, Hk, dk)
    k = act[..., cfg.key_dim:2 * cfg.key_dim].reshape(B, T, Hk, dk)
    v = act[..., 2 * cfg.key_dim:].reshape(B, T, Hv, dv)
    if cfg.v_per_k > 1:
        q = q.repeat_interleave(cfg.v_per_k, dim=2)
        k = k.repeat_interleave(cfg.v_per_k, dim=2)
    beta = torch.sigmoid(bb)
    g = -W[p + "A_log"].float().exp() * F.softplus(aa.float() + W[p + "dt_bias"].float())
    if cached and T == 1:
        core, new_rec = gdn_scan_recurrent(q, k, v, g, beta, rec_state, qk_l2=True)
    else:
        core, new_rec = gdn_scan_chunked(q, k, v, g, beta, state=rec_state if cached else None,
                                         qk_l2=True)
    core = rmsnorm_gated(core.reshape(-1, dv), z.reshape(-1, dv), W[p + "norm.weight"],
                         cfg.rms_norm_eps).reshape(B, T, cfg.value_dim)
    out = linear(core, W[p + "out_proj.weight"])
    if not use_cache:
        return out, None, None
    return out, new_conv, new_rec


def mlp(W, p, x):
    """blocks.py:332-342 -- SwiGLU."""
    return linear(F.silu(linear(x, W[p + "gate_proj.weight"])) * linear(x, W[p + "up_proj.weight"]),
                  W[p + "down_proj.weight"])


def decoder_layer(W, p, cfg, layer_type, x, cos, sin, cache, idx, use_cache=True):
    """modeling_qwen3_5.py:47-61 -- pre-norm residual mixer then MLP."""
    eps = cfg.rms_norm_eps
    h_in = rmsnorm_plus1(x, W[p + "input_layernorm.weight"], eps)
    if layer_type == "full_attention":
        h = gated_attention(W, p + "self_attn.", cfg, h_in, cos, sin, cache, idx)
    else:
        do_cache = use_cache and cache is not None
        cs, rs = cache.linear_state(idx) if cache is not None else (None, None)
        h, nc, nr = gated_deltanet(W, p + "linear_attn.", cfg, h_in, cs, rs, do_cache)
        if do_cache:
            cache.set_linear_state(idx, nc, nr)
    x = x + h
    return x + mlp(W, p + "mlp.", rmsnorm_plus1(x, W[p + "post_attention_layernorm.weight"], eps))


@torch.no_grad()
def model_forward(W, cfg, ids, past=None, return_hidden=False):
    """modeling_qwen3_5.py:82-102 -- embed; positions seen..seen+T; layer stack;
    advance; final norm; lm_head.  `hidden` is the pre-final-norm stream."""
    b, t = ids.shape
    x = W["model.embed_tokens.weight"][ids]
    cache = past if past is not None else RefCache(cfg.num_hidden_layers)
    pos = torch.arange(cache.seen_tokens, cache.seen_tokens + t)
    cos, sin = rope_tables(pos, cfg.rotary_dim, cfg.rope_theta, x.dtype)
    for i in range(cfg.num_hidden_layers):
        x = decoder_layer(W, f"model.layers.{i}.", cfg, cfg.layer_types[i], x, cos, sin, cache, i)
    cache.advance(t)
    logits = linear(rmsnorm_plus1(x, W["model.norm.weight"], cfg.rms_norm_eps), W["lm_head.weight"])
    return (logits, cache, x) if return_hidden else (logits, cache)


# ---------------------------------------------------------------------------------
# MTP head (reference: src/qwen3_5/mtp.py:40-89)
# ---------------------------------------------------------------------------------
def mtp_layer(W, cfg, hidden, next_emb, positions=None):
    """mtp.py:61-73 up to (not including) the final norm: returns the MTP decoder
    layer's output (B, L, H).  positions default to 1..L; no cache (attention only
    inside this call, causal)."""
    b, L, _ = hidden.shape
    if positions is None:
        positions = torch.arange(1, L + 1)
    cos, sin = rope_tables(positions, cfg.rotary_dim, cfg.rope_theta, hidden.dtype)
    eps = cfg.rms_norm_eps
    x = linear(torch.cat([rmsnorm_plus1(next_emb, W["mtp.pre_fc_norm_embedding.weight"], eps),
                          rmsnorm_plus1(hidden, W["mtp.pre_fc_norm_hidden.weight"], eps)], -1),
               W["mtp.fc.weight"])
    return decoder_layer(W, "mtp.layers.0.", cfg, "full_attention", x, cos, sin, None, 0,
                         use_cache=False)


@torch.no_grad()
def mtp_forward(W, cfg, hidden, next_emb, positions=None):
    """mtp.py:61-73 -- normalised MTP hidden (apply lm_head for logits)."""
    return rmsnorm_plus1(mtp_layer(W, cfg, hidden, next_emb, positions),
                         W["mtp.norm.weight"], cfg.rms_norm_eps)


@torch.no_grad()
def speculate(W, cfg, ids):
    """mtp.py:76-89 -- MTP logits (B, T-1, V): row i scores the token at i + 2 from the
    main model's hidden state at i and the embedding of token i + 1."""
    _, _, hidden = model_forward(W, cfg, ids, return_hidden=True)
    emb = W["model.embed_tokens.weight"][ids]
    return linear(mtp_forward(W, cfg, hidden[:, :-1], emb[:, 1:]), W["lm_head.weight"])


@torch.no_grad()
def mtp_chain_draft(W, cfg, hidden_last, pending, k, forced=None):
    """The build's k-step draft chain restated in the reference's own no-cache form
    (mtp.py:61-73 with cache=None): draft j runs the MTP block over the whole draft
    block so far -- hidden inputs [h_t, m_1..m_{j-1}], embeddings
    [emb(pending), emb(d_1)..emb(d_{j-1})], positions 1..j, causal -- and takes the
    argmax of the shared lm_head at the last position; m_j is the MTP layer output
    before its final norm.  For k == 1 this is exactly mtp.py:137-138.

    hidden_last: (B, 1, H); pending: (B,) long.  Returns drafts (B, k) long and the
    draft logits (B, k, V).  `forced` (B, k): feed these tokens forward instead of the
    argmax (teacher forcing, to score another implementation's drafts)."""
    emb_w = W["model.embed_tokens.weight"]
    hs = [hidden_last]
    toks = [pending]
    drafts, logits = [], []
    for j in range(k):
        h_in = torch.cat(hs, 1)
        e_in = emb_w[torch.stack(toks, 1)]
        m = mtp_layer(W, cfg, h_in, e_in)
        lg = linear(rmsnorm_plus1(m[:, -1:], W["mtp.norm.weight"], cfg.rms_norm_eps),
                    W["lm_head.weight"])[:, 0]
        d = lg.float().argmax(-1)
        drafts.append(d)
        logits.append(lg)
        hs.append(m[:, -1:])
        toks.append(d if forced is None else forced[:, j].long())
    return torch.stack(drafts, 1), torch.stack(logits, 1)


# ---------------------------------------------------------------------------------
# sampling and the loops (reference: src/generate.py:17-62, src/qwen3_5/mtp.py:92-162)
# ---------------------------------------------------------------------------------
def sample_next(logits, temperature, top_k, top_p, repetition_penalty=1.0, prev_ids=None,
                generator=None):
    """generate.py:17-37 -- repetition penalty, greedy at T<=0, temperature, top-k
    (keep >= k-th value), top-p (descending sort, drop where the cumulative mass
    BEFORE the token exceeds top_p), multinomial.  `generator` makes the draw
    reproducible for tests."""
    if repetition_penalty != 1.0 and prev_ids:
        idx = torch.tensor(sorted(set(prev_ids)), dtype=torch.long)
        logits = logits.clone()
        s = logits[idx]
        logits[idx] = torch.where(s > 0, s / repetition_penalty, s * repetition_penalty)
    if temperature <= 0.0:
        return int(torch.argmax(logits))
    logits = logits / temperature
    if top_k and top_k > 0:
        kth = torch.topk(logits, top_k).values[-1]
        logits = logits.masked_fill(logits < kth, float("-inf"))
    if top_p and 0.0 < top_p < 1.0:
        sl, si = torch.sort(logits, descending=True)
        cum = F.softmax(sl, dim=-1).cumsum(-1)
        drop = torch.zeros_like(cum, dtype=torch.bool)
        drop[1:] = cum[:-1] > top_p
        sl = sl.masked_fill(drop, float("-inf"))
        logits = torch.empty_like(logits).scatter_(0, si, sl)
    return int(torch.multinomial(F.softmax(logits, dim=-1), 1, generator=generator))


def _greedy_pick(logits, penalty=1.0, context=None):
    """generate.py:18-24 at temperature 0: argmax after the repetition penalty over
    set(context), in the logits' dtype."""
    return sample_next(logits, 0.0, 0, 1.0, penalty, context)


@torch.no_grad()
def generate_greedy(W, cfg, ids, n_new, repetition_penalty=1.0):
    """generate.py:40-62 at temperature 0 (token ids only, no text)."""
    context = list(ids)
    logits, past = model_forward(W, cfg, torch.tensor([ids]))
    out = []
    nxt = _greedy_pick(logits[0, -1], repetition_penalty, context)
    for _ in range(n_new):
        out.append(nxt)
        context.append(nxt)
        logits, past = model_forward(W, cfg, torch.tensor([[nxt]]), past)
        nxt = _greedy_pick(logits[0, -1], repetition_penalty, context)
    return out


@torch.no_grad()
def generate_mtp_greedy(W, cfg, ids, n_new, repetition_penalty=1.0):
    """mtp.py:92-162 at temperature 0 with k = 1: draft by MTP argmax (no penalty,
    mtp.py:138), snapshot, verify [pending, draft], accept iff draft == the penalised
    argmax of logits[0]; on reject restore the snapshot and re-run the pending token
    alone.  The penalty context is the prompt plus every emitted token
    (mtp.py:108,129,150).  Returns the token ids and the per-step accepted-draft counts."""
    context = list(ids)
    logits, past, hidden = model_forward(W, cfg, torch.tensor([ids]), return_hidden=True)
    h_last = hidden[:, -1:]
    pending = _greedy_pick(logits[0, -1], repetition_penalty, context)
    out, accepts = [], []
    emb_w = W["model.embed_tokens.weight"]
    while len(out) < n_new:
        out.append(pending)
        context.append(pending)
        if len(out) >= n_new:
            break
        x = mtp_forward(W, cfg, h_last, emb_w[torch.tensor([[pending]])])
        draft = int(linear(x, W["lm_head.weight"])[0, -1].argmax())
        snap = past.clone()
        lg2, past, hid2 = model_forward(W, cfg, torch.tensor([[pending, draft]]), past,
                                        return_hidden=True)
        true_next = _greedy_pick(lg2[0, 0], repetition_penalty, context)
        if draft == true_next:
            accepts.append(1)
            out.append(draft)
            context.append(draft)
            if len(out) >= n_new:
                break
            pending = _greedy_pick(lg2[0, 1], repetition_penalty, context)
            h_last = hid2[:, 1:2]
        else:
            accepts.append(0)
            past = snap
            _, past, hid1 = model_forward(W, cfg, torch.tensor([[pending]]), past,
                                          return_hidden=True)
            pending = true_next
            h_last = hid1[:, -1:]
    return out[:n_new], accepts


# ---------------------------------------------------------------------------------
# acceptance in the reference's own arithmetic (the CPU baseline of the sampler)
# ---------------------------------------------------------------------------------
def sample_next_probs(logits, temperature, top_k, top_p):
    """generate.py:23-36 batched over rows: the distribution sample_next draws from
    (temperature, top-k keeping logits >= the k-th, top-p by a descending sort with the
    cumulative mass shifted one place), in float32; greedy rows are one-hot at the first
    argmax.  logits (R, V) -> probabilities (R, V)."""
    x = logits.float()
    if temperature <= 0.0:
        return F.one_hot(x.argmax(-1), x.shape[-1]).float()
    x = x / temperature
    if top_k and top_k > 0:
        kth = torch.topk(x, top_k, dim=-1).values[:, -1:]
        x = x.masked_fill(x < kth, float("-inf"))
    if top_p and 0.0 < top_p < 1.0:
        sl, si = torch.sort(x, dim=-1, descending=True)
        cum = torch.softmax(sl, -1).cumsum(-1)
        drop = torch.zeros_like(cum, dtype=torch.bool)
        drop[:, 1:] = cum[:, :-1] > top_p
        sl = sl.masked_fill(drop, float("-inf"))
        x = torch.empty_like(x).scatter_(-1, si, sl)
    return torch.softmax(x, -1)


def spec_accept_sorted(target, drafts, temperature, top_k, top_p, uniforms, draft=None):
    """Speculative acceptance with the reference's sampler arithmetic: p_i =
    sample_next_probs(target[:, i]); q_i = sample_next_probs(draft[:, i]) for sampled
    drafts, or one-hot at the draft for argmax drafts (draft None, mtp.py:138); accept
    d_i iff u_i q_i(d_i) < p_i(d_i); at the first rejection draw from
    norm(max(0, p_i - q_i)), if all k are accepted draw the bonus from p_k, each by
    inverse CDF over token order with uniform u_k.  target (B, k+1, V); drafts (B, k)
    long; uniforms (B, k+1) in [0, 1).  Returns (n_accepted (B,), next_token (B,))."""
    B, T, V = target.shape
    k = T - 1
    p = sample_next_probs(target.reshape(B * T, V), temperature, top_k, top_p).view(B, T, V)
    q = None
    if draft is not None:
        q = sample_next_probs(draft.reshape(B * k, V), temperature, top_k, top_p).view(B, k, V)
    na = torch.zeros(B, dtype=torch.long)
    nt = torch.zeros(B, dtype=torch.long)
    for b in range(B):
        a = 0
        while a < k:
            d = drafts[b, a]
            qd = 1.0 if q is None else float(q[b, a, d])
            if not float(uniforms[b, a]) * qd < float(p[b, a, d]):
                break
            a += 1
        w = p[b, a].clone()
        if a < k:
            if q is None:
                w[drafts[b, a]] = max(0.0, float(w[drafts[b, a]]) - 1.0)
            else:
                w = (w - q[b, a]).clamp_min(0.0)
            if float(w.sum()) <= 0.0:
                w = p[b, a].clone()
        cdf = w.double().cumsum(0)
        tok = int(torch.searchsorted(cdf, uniforms[b, k].double() * cdf[-1], right=True))
        na[b], nt[b] = a, min(tok, V - 1)
    return na, nt
