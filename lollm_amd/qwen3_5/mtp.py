"""MTP draft head, the k-step draft chain and the on-device speculative step.

Reference: src/qwen3_5/mtp.py -- `MTP` (:40-73), `speculate` (:76-89), `generate_mtp`
(:92-162), `load_mtp` (:171-189).  The reference drafts one token (k = 1) for one
sequence, deep-copies the cache before the verify pass and re-runs on reject, with
three host syncs per step.  Here:

  * `MTP.forward(hidden, next_emb, positions=None)` keeps the reference signature and
    math: fc([RMSNorm(emb) ; RMSNorm(hidden)]) -> one forced full-attention decoder
    layer with no external cache (attention only inside the call, causal, positions
    1..L) -> RMSNorm.
  * The chain to k drafts (not defined by the reference): draft j runs the MTP layer
    on (hidden input, token) = (h_t, pending) for j = 1 and (m_{j-1}, d_{j-1}) after,
    where m is the MTP layer output before its final norm; position j; attention over
    the draft block so far through a small per-step KV cache (rows 0..j-1).  This is
    exactly the reference's no-cache form applied to the whole block [1..j] (the
    oracle's `mtp_chain_draft` recomputes it that way and the tests compare), and for
    k = 1 it is mtp.py:137-138.
  * `SpecDecoder.step()` runs draft chain -> one verify forward over [pending, d_1..d_k]
    -> `lollm_spec_accept` (rejection sampling, or argmax matching at temperature 0)
    -> `lollm_spec_commit` (O(1) rollback, token append, next pending, next hidden)
    entirely on the device; it can be captured in a HIP graph and replayed.
"""

from __future__ import annotations

import torch

from .. import ops
from .blocks import Projection, RMSNorm
from .kv import capturing
from .modeling_qwen3_5 import DecoderLayer, Qwen3_5Model
from .random_init import weight_shapes
from .weights import take_weights, to_raw


class MTP:
    def __init__(self, model: Qwen3_5Model, W: dict):
        cfg = model.cfg
        self.cfg, self.model = cfg, model
        eps = cfg.rms_norm_eps
        self.pre_fc_norm_embedding = RMSNorm(W["mtp.pre_fc_norm_embedding.weight"], eps)
        self.pre_fc_norm_hidden = RMSNorm(W["mtp.pre_fc_norm_hidden.weight"], eps)
        self.fc = Projection(W["mtp.fc.weight"])
        self.layers = [DecoderLayer(cfg, W, "mtp.layers.0.", "full_attention", model.inv_freq)]
        self.norm = RMSNorm(W["mtp.norm.weight"], eps)
        layer = self.layers[0]
        ops.gemm_workspace(max(p.workspace_bytes() for p in
                               [self.fc] + layer.self_attn.projections() + layer.mlp.projections()),
                           model.device)

    def _block(self, hidden, next_emb, k_cache, v_cache, lengths, kv_len, rope_pos, ws, tok=None):
        """Returns (MTP layer output before the final norm, normed output).  Given the
        next tokens' ids `tok` (B,) int32 instead of their embeddings, the lookup, both
        pre-fc norms and the concatenation run as one kernel (lollm_mtp_input)."""
        if tok is not None:
            B = tok.numel()
            fc_in = ops.mtp_input(tok, hidden, self.model.model.embed_tokens.weight,
                                  self.pre_fc_norm_embedding.weight, self.pre_fc_norm_hidden.weight,
                                  self.pre_fc_norm_embedding.eps).view(B, 1, -1)
        else:
            fc_in = torch.cat([self.pre_fc_norm_embedding(next_emb),
                               self.pre_fc_norm_hidden(hidden)], -1)
        layer = self.layers[0]
        # fc and the layer's input_layernorm (the fc output starts the residual stream)
        h_in, x = self.fc.add_norm(fc_in, None, layer.input_layernorm)
        core = layer.self_attn.core(h_in, k_cache, v_cache, lengths, kv_len, rope_pos=rope_pos,
                                    grid=self.model.attn_grid, workspace=ws)
        y, x = layer.self_attn.out.add_norm(core, x, layer.post_attention_layernorm)
        normed, x = layer.mlp.down.add_norm(layer.mlp.gate_up(y), x, self.norm)
        return x, normed

    def scratch_cache(self, B, L):
        cfg = self.cfg
        shape = (B, cfg.num_key_value_heads, L, cfg.head_dim)
        return (torch.zeros(shape, dtype=torch.bfloat16, device=self.model.device),
                torch.zeros(shape, dtype=torch.bfloat16, device=self.model.device))

    @torch.no_grad()
    def forward(self, hidden, next_emb, positions=None):
        """mtp.py:61-73: (B, L, H) -> normalised MTP hidden (B, L, H)."""
        B, L, _ = hidden.shape
        dev = self.model.device
        if positions is None:
            rope = torch.ones(B, dtype=torch.int32, device=dev)        # positions 1..L
        else:
            # any positions vector (L,) shared by the batch, as mtp.py:64-67, or (B, L)
            pos = torch.as_tensor(positions, device=dev).to(torch.int32)
            if pos.dim() == 1:
                pos = pos.view(1, -1).expand(B, -1)
            if tuple(pos.shape) != (B, L):
                raise ValueError(f"positions must be ({L},) or ({B}, {L}), got {tuple(positions.shape)}")
            rope = pos.contiguous()
        kc, vc = self.scratch_cache(B, L)
        zeros = torch.zeros(B, dtype=torch.int32, device=dev)
        kv_len = torch.full((B,), L, dtype=torch.int32, device=dev)
        _, normed = self._block(hidden.to(torch.bfloat16).contiguous(),
                                next_emb.to(torch.bfloat16).contiguous(), kc, vc, zeros, kv_len,
                                rope, None)
        return normed

    __call__ = forward


@torch.no_grad()
def speculate(model, mtp: MTP, input_ids):
    """mtp.py:76-89: MTP logits for position i + 2 given the context up to i + 1."""
    _, _, hidden = model(input_ids, return_hidden=True)
    emb = model.model.embed_tokens(input_ids.to(model.device))
    x = mtp(hidden[:, :-1], emb[:, 1:])
    return model.lm_head(x)


def load_mtp(model, weights: dict, fmt: str, device="cuda", dtype=None) -> MTP:
    """mtp.py:171-189: strict load of the `mtp.*` tensors; shares embed / lm_head."""
    cfg = model.cfg
    names = {k: v for k, v in weight_shapes(cfg, with_mtp=True).items() if k.startswith("mtp.")}
    names = {to_raw(k, fmt): v for k, v in names.items()}
    W = take_weights(cfg, weights, names, torch.device(device), dtype or torch.bfloat16,
                     who="qwen3_5 MTP")
    return MTP(model, W)


class SpecDecoder:
    """Batched MTP speculative decoding with k drafts per step, device-resident.

    temperature <= 0: greedy (argmax matching; the output equals greedy
    autoregressive decoding, the invariant of mtp.py:101-103).  temperature > 0:
    rejection sampling with p = sample_next's distribution (temperature, top-k,
    top-p) and q one-hot at the argmax draft (draft="argmax", the reference's
    drafting rule, mtp.py:138) or q = the MTP head's own distribution with sampled
    drafts (draft="sample").

    repetition_penalty != 1 applies sample_next's penalty (src/generate.py:18-22) to
    every verified position before acceptance, over each sequence's context as the
    reference keeps it (prompt, emitted tokens, the pending token, and the drafts
    verified before the position, mtp.py:108,129,150); argmax drafts are taken from the
    unpenalised MTP logits as in mtp.py:138, sampled drafts from penalised ones.

    Capacity: a step adds at most k + 1 tokens to a sequence; step() and replay() raise
    RuntimeError before a step whose tokens might not fit the cache (max_len) or the
    output buffer (out_capacity), from host-side upper bounds (exact values are read
    from the device only when a bound says the step might not fit)."""

    def __init__(self, model: Qwen3_5Model, mtp: MTP, batch: int, max_len: int, k: int = 3,
                 temperature: float = 0.0, top_k: int = 0, top_p: float = 1.0, seed: int = 0,
                 draft: str = "argmax", out_capacity: int = 4096, repetition_penalty: float = 1.0):
        if draft not in ("argmax", "sample"):
            raise ValueError("draft must be 'argmax' or 'sample'")
        if not repetition_penalty or repetition_penalty <= 0:
            raise ValueError("repetition_penalty must be positive")
        self.model, self.mtp, self.k = model, mtp, k
        self.B = batch
        self.temperature, self.top_k, self.top_p, self.seed = temperature, top_k, top_p, seed
        self.penalty = float(repetition_penalty)
        self.draft_mode = draft if temperature > 0 else "argmax"
        cfg, dev = model.cfg, model.device
        self.cache = model.new_cache(batch, max_len, spec_slots=k + 1)
        self.mkc, self.mvc = mtp.scratch_cache(batch, max(k, 1))
        i32 = dict(dtype=torch.int32, device=dev)
        self.pending = torch.zeros(batch, **i32)
        self.h_last = torch.zeros(batch, cfg.hidden_size, dtype=torch.bfloat16, device=dev)
        self.drafts = torch.zeros(batch, k, **i32)
        self.n_acc = torch.zeros(batch, **i32)
        self.next_tok = torch.zeros(batch, **i32)
        self.out_capacity = out_capacity
        self.out_tokens = torch.zeros(batch, out_capacity, **i32)
        self.out_count = torch.zeros(batch, **i32)
        self.out_bound = 0                                  # host upper bound of max(out_count)
        self.offset = torch.zeros(1, dtype=torch.int64, device=dev)
        self.accept_hist = torch.zeros(k + 1, **i32)       # accepted-length histogram
        self.seen = (ops.new_seen(batch, cfg.vocab_size, dev) if self.penalty != 1.0 else None)
        self.spec_ws = torch.empty(max(ops._lib.lib().lollm_spec_workspace_bytes(batch, k, 1), 16),
                                   dtype=torch.uint8, device=dev)
        self.row_ws = torch.empty(ops.sample_workspace_bytes(batch), dtype=torch.uint8, device=dev)
        self.mtp_ws = model.attn_workspace(batch, 1, max(k, 1))
        self.draft_logits = (torch.empty(batch, k, cfg.vocab_size, dtype=torch.bfloat16, device=dev)
                             if self.draft_mode == "sample" else None)
        # temperature 0 without a penalty: the verify rows need only their argmax, taken
        # from the lm_head GEMM without writing the (B, 1 + k, V) logits (same grid as the
        # logits path, so the same bits decide; set False to verify through the logits)
        lm = model.lm_head
        self.greedy_argmax = (temperature <= 0 and self.seen is None and lm.tiled is not None
                              and lm.path(batch * (k + 1)) == "gemm")
        self.verify_amax = torch.zeros(batch, k + 1, **i32)
        if self.greedy_argmax:   # reserve its workspace before any capture
            ops.gemm_workspace(ops._lib.lib().lollm_gemm_argmax_workspace_bytes(
                batch * (k + 1), lm.N, lm.K, lm.grid()), dev)
        # sampled verify: the lm_head writes the logits with the repetition penalty applied
        # and the rows' maxima (lollm_gemm_logits), so the acceptance reads each row once
        # (lollm_spec_accept_rowmax); set False to run lm_head, penalty and acceptance as
        # separate passes (same bits; taken by itself past lollm_gemm_logits' limit of
        # penalised draft tokens per row)
        self.fused_logits = (not self.greedy_argmax and temperature > 0 and lm.tiled is not None
                             and lm.path(batch * (k + 1)) == "gemm"
                             and (self.seen is None or k <= ops.GEMM_LOGITS_MAX_EXTRA))
        self.verify_logits = self.verify_rmax = None
        if self.fused_logits:
            self.verify_logits = torch.empty(batch, k + 1, cfg.vocab_size, dtype=torch.bfloat16,
                                             device=dev)
            self.verify_rmax = torch.empty(batch * (k + 1), ops.gemm_rowmax_slots(lm.grid()),
                                           dtype=torch.int16, device=dev)
        # the verify block's ids, embedding rows, layer 0 input norm and key counts, formed
        # by one kernel (lollm_verify_input)
        H = cfg.hidden_size
        self.verify_ids = torch.zeros(batch, k + 1, **i32)
        self.verify_x = torch.zeros(batch, k + 1, H, dtype=torch.bfloat16, device=dev)
        self.verify_y = torch.zeros(batch, k + 1, H, dtype=torch.bfloat16, device=dev)
        self.verify_kv_len = torch.zeros(batch, **i32)
        # per-draft-position index tensors (fixed across steps, so a graph can hold them)
        self.mtp_len = [torch.full((batch,), j, **i32) for j in range(k + 1)]
        self.graph = None
        self.steps_done = 0

    # ------------------------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompts):
        """prompts (B, L) long, equal lengths.  Runs the prompt through the model
        (mtp.py:120-122) and samples the first pending token (penalised by the prompt,
        mtp.py:122)."""
        V = self.model.cfg.vocab_size
        logits, _, hidden = self.model(prompts, self.cache, return_hidden=True, logits="last")
        last = logits[:, -1].contiguous()
        if self.seen is not None:
            self.seen.zero_()
            ops.seen_mark(self.seen, prompts.to(self.model.device), V)
            ops.repetition_penalty(last, self.seen, self.penalty)
        self.pending.copy_(ops.sample_rows(last, self.temperature, self.top_k, self.top_p,
                                           self.seed, 0, slot=2 * self.k + 2,
                                           workspace=self.row_ws))
        if self.seen is not None:
            ops.seen_mark(self.seen, self.pending, V)
        self.h_last.copy_(hidden[:, -1])
        self.out_count.zero_()
        self.out_bound = 0
        self.offset.fill_(1)

    def _draft_chain(self):
        B, k, model, mtp = self.B, self.k, self.model, self.mtp
        tok = self.pending
        h = self.h_last.view(B, 1, -1)
        for j in range(1, k + 1):
            m, normed = mtp._block(h, None, self.mkc, self.mvc, self.mtp_len[j - 1],
                                   self.mtp_len[j], self.mtp_len[j], self.mtp_ws, tok=tok)
            lm = model.lm_head
            if self.draft_mode == "sample":
                lg = lm(normed).view(B, -1)
                if self.seen is not None:
                    # the context of draft j holds the drafts before it
                    ops.repetition_penalty(lg, self.seen, self.penalty, extra=self.drafts,
                                           n_extra0=j - 1)
                self.draft_logits[:, j - 1].copy_(lg)
                d = ops.sample_rows(lg, self.temperature, self.top_k, self.top_p, self.seed, 0,
                                    slot=k + 1 + j, offset_dev=self.offset, workspace=self.row_ws)
                self.drafts[:, j - 1].copy_(d)
            elif lm.tiled is not None and B <= ops.GEMM_MAX_ROWS:
                # greedy draft straight from the lm_head GEMM (no logits), into its column
                x2 = normed.reshape(B, -1)
                col = self.drafts[:, j - 1]
                d = ops.gemm_argmax(x2, lm.tiled, lm.N, lm.K, out=col,
                                    grid=lm.argmax_grid(B))
            else:
                d = ops.sample_rows(lm(normed).view(B, -1), 0.0, workspace=self.row_ws)
                self.drafts[:, j - 1].copy_(d)
            tok, h = d, m

    def _reserve(self):
        """Raise before a step whose k + 1 tokens might not fit (see the class doc)."""
        T = self.k + 1
        self.cache.reserve(T)
        if self.out_bound + T > self.out_capacity:
            if capturing():
                raise RuntimeError("output capacity may be exceeded (cannot check under capture)")
            self.out_bound = int(self.out_count.max())
            if self.out_bound + T > self.out_capacity:
                raise RuntimeError(f"output capacity exceeded: a sequence holds {self.out_bound} "
                                   f"tokens, a step may add {T}, out_capacity {self.out_capacity}")

    def _grew(self):
        self.cache.grew(self.k + 1)
        self.out_bound += self.k + 1

    @torch.no_grad()
    def step(self):
        """One speculative step: k drafts, one verify pass over 1 + k positions, accept,
        commit.  Device-only (no host sync)."""
        live = not capturing()
        if live:
            self._reserve()
        self._step_kernels()
        if live:
            self._grew()

    def verify_hidden(self):
        """The verify pass over [pending | drafts] (mtp.py:141-142): the block's ids,
        embedding rows and layer 0 norm in one kernel, then the decoder stack; returns
        (pre-norm hidden, final-normed hidden) as Qwen3_5Model.hidden_states."""
        m = self.model
        ops.verify_input(self.pending, self.drafts, m.model.embed_tokens.weight,
                         m.model.layers[0].input_layernorm.weight,
                         m.model.layers[0].input_layernorm.eps, self.cache.lengths,
                         ids=self.verify_ids, x=self.verify_x, y=self.verify_y,
                         kv_len=self.verify_kv_len)
        return m.hidden_states(self.verify_ids, self.cache,
                               inputs=(self.verify_x, self.verify_y, self.verify_kv_len))

    def _step_kernels(self):
        B, k, model, cache = self.B, self.k, self.model, self.cache
        self._draft_chain()
        hidden, normed = self.verify_hidden()
        verify_ids = self.verify_ids
        if self.greedy_argmax:
            lm = model.lm_head
            ops.gemm_argmax(normed.reshape(-1, lm.K), lm.tiled, lm.N, lm.K,
                            out=self.verify_amax.view(-1), grid=lm.grid())
            ops.greedy_accept(self.verify_amax, self.drafts, self.n_acc, self.next_tok)
        else:
            rmax = None
            if self.fused_logits:
                lm = model.lm_head
                # position t's context holds the pending token and the drafts before t
                logits, rmax = ops.gemm_logits(normed.reshape(-1, lm.K), lm.tiled, lm.N, lm.K,
                                               out=self.verify_logits.view(-1, lm.N),
                                               rowmax=self.verify_rmax, seen=self.seen,
                                               penalty=self.penalty, extra=self.drafts,
                                               T=k + 1, grid=lm.grid())
                logits = logits.view(B, k + 1, -1)
            else:
                logits = model.lm_head(normed)
                if self.seen is not None:
                    ops.repetition_penalty(logits, self.seen, self.penalty, extra=self.drafts)
            ops.spec_accept(logits, self.draft_logits, self.drafts, self.temperature, self.top_k,
                            self.top_p, self.seed, 0, offset_dev=self.offset,
                            workspace=self.spec_ws, n_accepted=self.n_acc,
                            next_token=self.next_tok, target_rowmax=rmax)
        ops.spec_commit(verify_ids, self.n_acc, self.next_tok, cache.lengths, cache.rec_half,
                        cache.replay, cache.conv_off, self.pending, self.out_tokens, self.out_count,
                        hidden.contiguous(), self.h_last, self.offset, cache.spec_slots,
                        cache.win_rows, self.accept_hist, seen=self.seen)
        cache.fresh = False

    def capture(self):
        """Record step() in a HIP graph (after prefill and at least one eager step);
        replay with replay().  Capturing executes nothing."""
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._step_kernels()

    def replay(self):
        self._reserve()
        self.graph.replay()
        self._grew()

    @torch.no_grad()
    def generate(self, n_steps, use_graph=False):
        for _ in range(n_steps):
            if use_graph:
                self.replay()
            else:
                self.step()
            self.steps_done += 1

    def tokens(self):
        """Committed tokens per sequence (list of lists; host sync)."""
        cnt = self.out_count.cpu().tolist()
        out = self.out_tokens.cpu()
        return [out[b, :min(c, out.shape[1])].tolist() for b, c in enumerate(cnt)]


@torch.no_grad()
def generate_mtp(model, mtp: MTP, ids, decode, stop_ids, device="cuda", *, max_new_tokens=128,
                 temperature=0.7, top_k=20, top_p=0.8, repetition_penalty=1.1, k=1, seed=0):
    """Drop-in for the reference's generate_mtp (mtp.py:92-162): yields text pieces.
    Runs the batched decoder with B = 1 and k drafts (k = 1 by default, as the
    reference), with the reference's sampling arguments (run.py passes the family
    defaults, repetition_penalty 1.05 included)."""
    eos = set(stop_ids)
    pen = 1.0 if repetition_penalty is None else float(repetition_penalty)
    dec = SpecDecoder(model, mtp, 1, len(ids) + max_new_tokens + 2 * k + 8, k=k,
                      temperature=temperature, top_k=top_k, top_p=top_p, seed=seed,
                      out_capacity=max_new_tokens + 2 * k + 2, repetition_penalty=pen)
    dec.prefill(torch.tensor([ids], device=model.device))
    generated, prev = [], ""
    while True:
        # committed tokens, then the pending one (already final: it is the next
        # step's first verified position)
        stream = dec.tokens()[0] + [int(dec.pending[0])]
        while len(generated) < len(stream):
            tok = stream[len(generated)]
            if tok in eos or len(generated) >= max_new_tokens:
                return
            generated.append(tok)
            text = decode(generated)
            if len(text) > len(prev):
                yield text[len(prev):]
                prev = text
        dec.step()
