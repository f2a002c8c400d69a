"""Qwen3_5Model -- the hybrid decoder with the reference's forward contract.

`forward(input_ids (B, T), past=None, return_hidden=False) -> (logits (B, T, V),
past[, hidden (B, T, H)])` as in src/qwen3_5/modeling_qwen3_5.py:82-102: embed,
positions from the cache, the [GDN, GDN, GDN, attention] layer stack with pre-norm
residuals (modeling_qwen3_5.py:47-61), final norm, lm_head, `hidden` = the pre-final-
norm stream that the MTP head consumes.  Differences, all on purpose:
  * the batch may hold sequences of different lengths (per-sequence `cache.lengths`);
  * every residual add is fused into the following RMSNorm kernel;
  * `logits="last"` computes the lm_head only for the last position (prefill).
Runs only on the HIP device; there is no CPU path.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from .. import ops
from .blocks import MLP, GatedAttention, GatedDeltaNet, Projection, RMSNorm, rope_inv_freq
from .config import Qwen3_5Config
from .kv import Qwen3_5Cache

__all__ = ["DecoderLayer", "Qwen3_5Model", "Qwen3_5Cache"]


class DecoderLayer:
    """modeling_qwen3_5.py:27-61.  `layer_type` overrides the schedule (the MTP block
    is a forced full-attention layer, mtp.py:51-52)."""

    def __init__(self, cfg: Qwen3_5Config, W: dict, p: str, layer_type: str, inv_freq):
        self.layer_type = layer_type
        eps = cfg.rms_norm_eps
        self.input_layernorm = RMSNorm(W[p + "input_layernorm.weight"], eps)
        self.post_attention_layernorm = RMSNorm(W[p + "post_attention_layernorm.weight"], eps)
        if layer_type == "full_attention":
            self.self_attn = GatedAttention(cfg, W, p + "self_attn.", inv_freq)
        else:
            self.linear_attn = GatedDeltaNet(cfg, W, p + "linear_attn.")
        self.mlp = MLP(W[p + "mlp.gate_proj.weight"], W[p + "mlp.up_proj.weight"],
                       W[p + "mlp.down_proj.weight"])


class _Embedding:
    def __init__(self, weight):
        self.weight = weight

    def __call__(self, ids):
        return F.embedding(ids, self.weight)


class _Inner:
    pass


class Qwen3_5Model:
    def __init__(self, cfg: Qwen3_5Config, W: dict, device="cuda"):
        """W: canonical (`model.*`, `lm_head.weight`) bf16 tensors on the device."""
        self.cfg = cfg
        self.device = torch.device(device)
        self.inv_freq = rope_inv_freq(cfg.rotary_dim, cfg.rope_theta, device)
        self.model = _Inner()
        self.model.embed_tokens = _Embedding(W["model.embed_tokens.weight"])
        self.model.layers = [DecoderLayer(cfg, W, f"model.layers.{i}.", cfg.layer_type(i),
                                          self.inv_freq)
                             for i in range(cfg.num_hidden_layers)]
        self.model.norm = RMSNorm(W["model.norm.weight"], cfg.rms_norm_eps)
        self.lm_head = Projection(W["lm_head.weight"])
        self.attn_grid = 0          # attention workgroups (0: one per CU)
        ops.gemm_workspace(max(p.workspace_bytes() for p in self.projections()), self.device)
        self._ws = {}
        self.default_extra_capacity = 4096

    def projections(self):
        """Every weight GEMM of the decoder (for workspace sizing)."""
        out = [self.lm_head]
        for layer in self.model.layers:
            mixer = layer.self_attn if layer.layer_type == "full_attention" else layer.linear_attn
            out += mixer.projections() + layer.mlp.projections()
        return out

    # ---------------------------------------------------------------------------------
    def new_cache(self, batch, max_len, spec_slots=4):
        return Qwen3_5Cache(self.cfg, batch, max_len, spec_slots, self.device)

    def attn_workspace(self, B, T, max_len):
        """Split-K partials buffer of the attention layers (shared by all layers of a
        call; one per (B, T) shape, kept for graph replays)."""
        cfg = self.cfg
        key = (B, T, max_len, self.attn_grid)
        if key not in self._ws:
            n = ops.attn_workspace_bytes(B, T, cfg.num_attention_heads, cfg.num_key_value_heads,
                                         cfg.head_dim, max_len, self.attn_grid)
            self._ws[key] = torch.empty(max(n, 16), dtype=torch.uint8, device=self.device)
        return self._ws[key]

    @torch.no_grad()
    def forward(self, input_ids, past=None, return_hidden=False, logits="all"):
        B, T = input_ids.shape
        cache = past if past is not None else self.new_cache(B, T + self.default_extra_capacity)
        cache.reserve(T)                  # raise before any KV row could land past max_len
        x, normed = self.hidden_states(input_ids, cache)
        if logits == "last":
            out = self.lm_head(normed[:, -1:])
        else:
            out = self.lm_head(normed)
        cache.commit_all(T)
        return (out, cache, x) if return_hidden else (out, cache)

    __call__ = forward

    def hidden_states(self, input_ids, cache, inputs=None):
        """The decoder stack; returns (pre-norm hidden, final-normed hidden).  Writes
        the KV rows / GDN records of the T new tokens but does not commit them.  The
        caller has checked the capacity (cache.reserve(T)).  inputs: the block's
        (embedding rows, layer 0's input norm of them, lengths + T) when already formed
        (lollm_verify_input), else they are formed here."""
        B, T = input_ids.shape
        cfg = self.cfg
        lengths = cache.lengths
        if inputs is None:
            x = self.model.embed_tokens(input_ids.to(self.device))
            kv_len = lengths + T
            h_first = None
        else:
            x, h_first, kv_len = inputs
        ws = self.attn_workspace(B, T, cache.max_len)
        # each residual-stream projection (o_proj / out_proj / down_proj) is issued with
        # the residual add and the norm that follows it (modeling_qwen3_5.py:59-60)
        pending = None   # (down_proj, its input): opens the next layer
        for i, layer in enumerate(self.model.layers):
            if pending is None:
                h_in = layer.input_layernorm(x) if h_first is None else h_first
            else:
                h_in, x = pending[0].add_norm(pending[1], x, layer.input_layernorm)
            if layer.layer_type == "full_attention":
                s = cache.layers[i]
                mixer = layer.self_attn
                core = mixer.core(h_in, s["k"], s["v"], lengths, kv_len,
                                  grid=self.attn_grid, workspace=ws)
            else:
                mixer = layer.linear_attn
                core = mixer.core(h_in, cache, i)
            y, x = mixer.out.add_norm(core, x, layer.post_attention_layernorm)
            pending = (layer.mlp.down, layer.mlp.gate_up(y))
        normed, x = pending[0].add_norm(pending[1], x, self.model.norm)
        return x, normed
