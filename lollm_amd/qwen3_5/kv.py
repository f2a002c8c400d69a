"""Qwen3_5Cache -- the family cache, batched and device-resident, with O(1) rollback.

Keeps the method names of the reference cache (src/qwen3_5/kv.py:20-58:
append_kv / read_kv / linear_state / set_linear_state / advance / seen_tokens / clone
/ nbytes) so code written against that API keeps working, but the storage is laid out
for the MI355X kernels:

  * full-attention layers: preallocated K and V of shape (B, n_kv, max_len, head_dim)
    bf16, one contiguous slab per (sequence, KV head); `lengths` (B,) int32 on the
    device holds each sequence's committed length (the reference has one scalar
    `seen_tokens`, so it cannot hold ragged batches).
  * Gated DeltaNet layers: a conv-window buffer (B, 2W, conv_dim) bf16 with W = K-1+S
    rows per half, a recurrent-state buffer (B, 2, n_v, Dk, Dv) fp32 and a replay-record
    buffer (B, 2, n_v, S, 4 Dk + 16) bytes with S = 1 + k positions per half.
    `conv_off` (B,) int32 locates each sequence's committed conv state; `rec_half` and
    `replay` (B,) int32 say that its committed recurrent state is that half's state with
    the half's first `replay` records applied.  A forward reads the committed half and
    writes the other one (the kernel derives the halves on the device); a short forward
    (T <= S) writes the committed state plus one record per position instead of T
    states, so rolling back to `a` accepted drafts only rewrites four small integers per
    sequence (`lollm_spec_commit`) -- the reference instead deep-copies the whole cache
    before every verify (kv.py:49-54, mtp.py:141) and re-runs on reject (mtp.py:156-162).
"""

from __future__ import annotations

import torch

from .. import ops
from .config import Qwen3_5Config


def capturing() -> bool:
    """Whether the current stream is recording a HIP graph (False without a device)."""
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


class Qwen3_5Cache:
    def __init__(self, cfg: Qwen3_5Config, batch: int, max_len: int, spec_slots: int = 4,
                 device="cuda"):
        self.cfg = cfg
        self.batch, self.max_len, self.spec_slots = batch, max_len, spec_slots
        self.device = torch.device(device)
        n = cfg.num_hidden_layers
        self.layers = [None] * n
        K = cfg.linear_conv_kernel_dim
        for i in range(n):
            if cfg.layer_type(i) == "full_attention":
                shape = (batch, cfg.num_key_value_heads, max_len, cfg.head_dim)
                self.layers[i] = {"k": torch.zeros(shape, dtype=torch.bfloat16, device=device),
                                  "v": torch.zeros(shape, dtype=torch.bfloat16, device=device)}
            else:
                self.layers[i] = {
                    "win": torch.zeros(batch, 2 * self.win_rows, cfg.conv_dim,
                                       dtype=torch.bfloat16, device=device),
                    "rec": torch.zeros(batch, 2, cfg.linear_num_value_heads,
                                       cfg.linear_key_head_dim, cfg.linear_value_head_dim,
                                       dtype=torch.float32, device=device),
                    "rep": torch.zeros(batch, 2, cfg.linear_num_value_heads, spec_slots,
                                       4 * cfg.linear_key_head_dim + 16, dtype=torch.uint8,
                                       device=device),
                }
        self.fresh = True                 # no GDN state yet (zero initial state)
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=device)
        self.rec_half = torch.zeros(batch, dtype=torch.int32, device=device)
        self.replay = torch.zeros(batch, dtype=torch.int32, device=device)
        self.conv_off = torch.zeros(batch, dtype=torch.int32, device=device)
        self.last_T = 0
        # host-side upper bound of max(lengths): every forward or speculative step adds
        # its T, rollbacks leave it, so capacity is checked without reading the device
        self.len_bound = 0

    @property
    def win_rows(self):
        return self.cfg.linear_conv_kernel_dim - 1 + self.spec_slots

    # -- capacity ----------------------------------------------------------------------
    def reserve(self, T: int):
        """Raise RuntimeError unless T more rows fit every sequence (lengths + T <=
        max_len) -- the kernels would otherwise drop the KV rows past the end.  Reads the
        device lengths (a host sync) only when the host-side bound says they may not fit."""
        if self.len_bound + T <= self.max_len:
            return
        if capturing():
            raise RuntimeError(f"KV cache capacity: {self.len_bound} + {T} rows may exceed "
                               f"max_len {self.max_len} (cannot check exactly under capture)")
        self.len_bound = int(self.lengths.max()) if self.batch else 0
        if self.len_bound + T > self.max_len:
            raise RuntimeError(f"KV cache capacity exceeded: a sequence holds {self.len_bound} "
                               f"tokens, {T} more do not fit max_len {self.max_len}")

    def grew(self, T: int):
        """Record that a call may have added up to T tokens to every sequence."""
        self.len_bound += T

    # -- bookkeeping used by the model's forward -------------------------------------
    def commit_all(self, T: int):
        """After a forward over T tokens: every token is committed (the reference's
        forward + advance(T), modeling_qwen3_5.py:97).  The forward wrote the other half
        of every GDN buffer: a short forward its T records, a long one its final state."""
        S, W, K = self.spec_slots, self.win_rows, self.cfg.linear_conv_kernel_dim
        self.fresh = False
        self.last_T = T
        full = K - 1 + T <= W
        self.rec_half.bitwise_xor_(1)
        self.replay.fill_(T if T <= S else 0)
        self.conv_off.copy_(torch.where(self.conv_off >= W, 0, W) + (T if full else 0))
        self.lengths.add_(T)
        self.grew(T)

    def rollback(self, n_accepted: torch.Tensor):
        """After commit_all(T) with T <= spec_slots: keep n_accepted[b] + 1 tokens."""
        T = self.last_T
        if T > self.spec_slots:
            raise RuntimeError("rollback needs the last forward to have written replay records")
        a = n_accepted.to(torch.int32).clamp(0, T - 1)
        self.lengths.sub_(T - 1 - a)
        self.replay.sub_(T - 1 - a)
        self.conv_off.sub_(T - 1 - a)

    # -- the reference cache API (kv.py:26-58) ---------------------------------------
    def _uniform_length(self) -> int:
        L = self.lengths.cpu()
        if not bool((L == L[0]).all()):
            raise RuntimeError("sequences have different lengths; use .lengths")
        return int(L[0])

    @property
    def seen_tokens(self) -> int:
        return self._uniform_length()

    def advance(self, n):
        self.reserve(n)
        self.lengths.add_(n)
        self.grew(n)

    def append_kv(self, layer, k, v):
        """Write k, v (B, n_kv, t, D) at the current length; return the full (K, V)."""
        s = self.layers[layer]
        L = self._uniform_length()
        t = k.shape[2]
        if L + t > self.max_len:
            raise RuntimeError("KV cache capacity exceeded")
        s["k"][:, :, L:L + t] = k
        s["v"][:, :, L:L + t] = v
        return s["k"][:, :, :L + t], s["v"][:, :, :L + t]

    def read_kv(self, layer):
        s = self.layers[layer]
        if s is None or "k" not in s:
            return None
        L = self._uniform_length()
        return s["k"][:, :, :L], s["v"][:, :, :L]

    def linear_state(self, layer):
        """(conv_state (B, conv_dim, K-1), recurrent_state (B, n_v, Dk, Dv)) copies, or
        (None, None) before the first forward."""
        s = self.layers[layer]
        if s is None or "win" not in s or self.fresh:
            return None, None
        K = self.cfg.linear_conv_kernel_dim
        b = torch.arange(self.batch, device=self.device)
        rows = self.conv_off[:, None].long() + torch.arange(K - 1, device=self.device)[None]
        conv = s["win"][b[:, None], rows].transpose(1, 2).contiguous()
        rec = ops.gdn_state(s["rec"], self.rec_half, s["rep"], self.replay)
        return conv, rec

    def settle(self):
        """Fold every GDN layer's pending replay records into its state: each layer's
        committed state goes to the other half, which becomes the committed one with no
        records (the cache holds the same state afterwards)."""
        if self.fresh:
            return
        for s in self.layers:
            if s is not None and "rec" in s:
                ops.gdn_state(s["rec"], self.rec_half, s["rep"], self.replay, to_other_half=True)
        self.rec_half.bitwise_xor_(1)
        self.replay.zero_()

    def set_linear_state(self, layer, conv, rec):
        s = self.layers[layer]
        K = self.cfg.linear_conv_kernel_dim
        b = torch.arange(self.batch, device=self.device)
        self.settle()   # the other layers keep their states; this one's is replaced whole
        rows = self.conv_off[:, None].long() + torch.arange(K - 1, device=self.device)[None]
        s["win"][b[:, None], rows] = conv.transpose(1, 2).to(torch.bfloat16)
        s["rec"][b, self.rec_half.long()] = rec.float()
        self.fresh = False   # (a new cache's other layers hold zero states, as on a first call)

    def clone(self):
        new = Qwen3_5Cache.__new__(Qwen3_5Cache)
        new.__dict__.update(self.__dict__)
        new.layers = []
        for s in self.layers:
            if s is None:
                new.layers.append(None)
            else:
                new.layers.append({n: t.clone() for n, t in s.items()})
        for n in ("lengths", "rec_half", "replay", "conv_off"):
            setattr(new, n, getattr(self, n).clone())
        return new

    def nbytes(self):
        tot = 0
        for s in self.layers:
            if s is None:
                continue
            for t in s.values():
                tot += t.numel() * t.element_size()
        return tot
