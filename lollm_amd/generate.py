"""The shared generation loop and sampler (reference: src/generate.py:17-62).

`sample_next` keeps the reference signature and filter order (repetition penalty ->
greedy at T <= 0 -> temperature -> top-k -> top-p -> draw) but draws on the device
with `lollm_sample_rows` on explicit Philox uniforms instead of torch.multinomial, so a
draw is reproducible from (seed, offset).  `generate` is the plain autoregressive loop
over the family's `forward(ids, past) -> (logits, past)`.
"""

from __future__ import annotations

import itertools

import torch

from . import ops

_draws = itertools.count(1)
SEED = 0x5EED


def sample_next(logits, temperature, top_k, top_p, repetition_penalty=1.0, prev_ids=None,
                seed=None, offset=None):
    """(V,) logits on the device -> int token.  The repetition penalty runs in the
    lollm_repetition_penalty kernel over the bitmap of set(prev_ids) (generate.py:18-22,
    bf16 arithmetic as the reference's GPU logits have), on a copy of the row."""
    x = logits.reshape(1, -1)
    V = x.shape[1]
    x = x.to(torch.bfloat16)
    if x.data_ptr() == logits.data_ptr() or not x.is_contiguous():
        x = x.clone(memory_format=torch.contiguous_format)
    if repetition_penalty != 1.0 and prev_ids:
        seen = ops.new_seen(1, V, x.device)
        ops.seen_mark(seen, torch.tensor(list(prev_ids), dtype=torch.int32, device=x.device), V)
        ops.repetition_penalty(x, seen, repetition_penalty)
    off = next(_draws) if offset is None else offset
    tok = ops.sample_rows(x, temperature, top_k or 0, top_p if top_p else 1.0,
                          SEED if seed is None else seed, off)
    return int(tok[0])


@torch.no_grad()
def generate(model, ids, decode, stop_ids, device="cuda", *, max_new_tokens=128,
             temperature=0.7, top_k=20, top_p=0.8, repetition_penalty=1.1):
    """generate.py:40-62: prefill, then one token per forward; yields text pieces.  The
    cache holds the prompt plus max_new_tokens (the reference's grows without bound)."""
    input_ids = torch.tensor([ids], device=device)
    context = list(ids)
    eos = set(stop_ids)
    past = model.new_cache(1, len(ids) + max_new_tokens + 1)
    logits, past = model(input_ids, past)
    nxt = sample_next(logits[0, -1], temperature, top_k, top_p, repetition_penalty, context)
    generated, prev = [], ""
    for _ in range(max_new_tokens):
        if nxt in eos:
            break
        generated.append(nxt)
        context.append(nxt)
        text = decode(generated)
        if len(text) > len(prev):
            yield text[len(prev):]
            prev = text
        logits, past = model(torch.tensor([[nxt]], device=device), past)
        nxt = sample_next(logits[0, -1], temperature, top_k, top_p, repetition_penalty, context)


@torch.no_grad()
def greedy_tokens(model, prompts, n_new):
    """Batched greedy autoregressive decoding (temperature 0) returning token ids:
    the reference loop's semantics for B sequences of equal prompt length."""
    B, L = prompts.shape
    cache = model.new_cache(B, L + n_new + 1, spec_slots=4)
    logits, _ = model(prompts.to(model.device), cache, logits="last")
    out = []
    nxt = ops.sample_rows(logits[:, -1].contiguous(), 0.0)
    for _ in range(n_new):
        out.append(nxt.clone())
        logits, _ = model(nxt.view(B, 1).long(), cache)
        nxt = ops.sample_rows(logits[:, -1].contiguous(), 0.0)
    return torch.stack(out, 1).cpu()
