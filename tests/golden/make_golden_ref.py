"""Writes tests/golden/ref_mtp.safetensors from the reference implementation itself.

Runs only in the build container, where the giapnguyen74/lollm checkout is at
/root/reference; the reference never travels with the repository (only the vectors
written here do).  It is imported for the functions nothing else pins:

  * `MTP.forward` (src/qwen3_5/mtp.py:61-73) at L = 1..4 and with explicit positions
    (consecutive, and a vector that is neither consecutive nor increasing),
    on the micro and tiny seeded weights: the [emb ; hidden] concatenation order, the
    pre-fc norms, positions 1..L and the cache-less causal block;
  * `speculate` (mtp.py:76-89) on the micro weights;
  * `generate_mtp` (mtp.py:92-162) and `generate` (src/generate.py:40-62), greedy
    (temperature 0, so the trajectory is deterministic), B = 1, a 128-token
    uniform-random prompt (seed 1), 64 new tokens, k = 1: on the tiny 1024-hidden
    model without a penalty, and on the micro model (vocabulary 512, so the prompt
    covers a fifth of it and the penalty changes picks) with repetition_penalty 1.0,
    the family default 1.05 (src/qwen3_5/__init__.py:21) and 1.3;
  * `sample_next` (src/generate.py:17-37) at temperature 0 with a repetition penalty,
    on crafted rows where the penalty decides the argmax.

Weights: `lollm_amd.qwen3_5.random_init.random_weights(cfg, seed=0)` rounded to bf16
and held in fp32, the same bits the GPU tests load.  The reference runs in fp32 (the
truth) and, for the tie tolerance of the token checks, in bf16 (its GPU dtype,
src/run.py:34-39): per generated position the fixture stores the top-16 fp32 logits
(after the penalty where one applies) and the largest |bf16 - fp32| logit deviation
over the teacher-forced trajectory.

Usage:  python tests/golden/make_golden_ref.py
"""

from __future__ import annotations

import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF_SRC = "/root/reference/src"
sys.path.insert(0, ROOT)

from lollm_amd.qwen3_5.config import Qwen3_5Config, micro_config_dict, tiny_config_dict  # noqa: E402
from lollm_amd.qwen3_5.random_init import random_weights  # noqa: E402

TOPN = 16


def _ref_modules():
    sys.path.insert(0, REF_SRC)
    import generate as ref_generate
    from qwen3_5 import mtp as ref_mtp
    from qwen3_5 import weights as ref_weights
    return ref_generate, ref_mtp, ref_weights


def _weights(raw, seed=0):
    cfg = Qwen3_5Config.from_hf(raw)
    W = random_weights(cfg, seed=seed)
    return {k: v.to(torch.bfloat16).float() for k, v in W.items()}


def _load(ref_weights, ref_mtp, raw, dtype):
    W = _weights(raw)
    model = ref_weights.load(raw, dict(W), "hf", device="cpu", dtype=dtype)
    mtp = ref_mtp.load_mtp(model, dict(W), "hf", device="cpu", dtype=dtype)
    return model, mtp


def mtp_forward_cases(ref_mtp, ref_weights, tag, raw, out):
    model, mtp = _load(ref_weights, ref_mtp, raw, torch.float32)
    H = raw["hidden_size"]
    g = torch.Generator().manual_seed(21)
    for L in (1, 2, 3, 4):
        h = torch.randn(2, L, H, generator=g)
        e = torch.randn(2, L, H, generator=g) * 0.05
        with torch.no_grad():
            y = mtp(h, e)
        out[f"{tag}.mtp{L}.hidden"], out[f"{tag}.mtp{L}.next_emb"] = h, e
        out[f"{tag}.mtp{L}.out"] = y.contiguous()
    # explicit positions (the argument the default 1..L replaces)
    h = torch.randn(2, 3, H, generator=g)
    e = torch.randn(2, 3, H, generator=g) * 0.05
    pos = torch.arange(7, 10)
    with torch.no_grad():
        y = mtp(h, e, positions=pos)
    out[f"{tag}.mtp_pos.hidden"], out[f"{tag}.mtp_pos.next_emb"] = h, e
    out[f"{tag}.mtp_pos.positions"] = pos
    out[f"{tag}.mtp_pos.out"] = y.contiguous()
    # a positions vector that is neither consecutive nor increasing
    h = torch.randn(2, 4, H, generator=g)
    e = torch.randn(2, 4, H, generator=g) * 0.05
    pos = torch.tensor([5, 17, 18, 2])
    with torch.no_grad():
        y = mtp(h, e, positions=pos)
    out[f"{tag}.mtp_pos_nc.hidden"], out[f"{tag}.mtp_pos_nc.next_emb"] = h, e
    out[f"{tag}.mtp_pos_nc.positions"] = pos
    out[f"{tag}.mtp_pos_nc.out"] = y.contiguous()
    return model, mtp


def speculate_case(ref_mtp, model, mtp, raw, out):
    g = torch.Generator().manual_seed(22)
    ids = torch.randint(0, raw["vocab_size"], (2, 9), generator=g)
    with torch.no_grad():
        lg = ref_mtp.speculate(model, mtp, ids)
    out["micro.spec.ids"] = ids
    out["micro.spec.logits"] = lg.contiguous()


def _trajectory(gen_fn, model, *args, **kw):
    seen = []

    def decode(toks):
        seen[:] = list(toks)
        return " ".join(str(t) for t in toks)
    for _ in gen_fn(model, *args, decode=decode, **kw):
        pass
    return list(seen)


def _penalised(logits, prev, penalty):
    """src/generate.py:18-22 on one row (the reference's own code path is exercised by
    the trajectories; this only ranks the stored top-N the same way)."""
    if penalty == 1.0 or not prev:
        return logits
    idx = torch.tensor(sorted(set(prev)), dtype=torch.long)
    logits = logits.clone()
    s = logits[idx]
    logits[idx] = torch.where(s > 0, s / penalty, s * penalty)
    return logits


def trajectories(ref_generate, ref_mtp, ref_weights, out, tag, raw, penalties):
    """generate_mtp and generate at temperature 0 on a 128-token prompt (seed 1), 64 new
    tokens, for each repetition penalty; they must agree (mtp.py:101-103)."""
    model, mtp = _load(ref_weights, ref_mtp, raw, torch.float32)
    model16, _ = _load(ref_weights, ref_mtp, raw, torch.bfloat16)
    g = torch.Generator().manual_seed(1)
    prompt = torch.randint(0, raw["vocab_size"], (128,), generator=g).tolist()
    out[f"{tag}.prompt"] = torch.tensor(prompt, dtype=torch.int64)
    n_new = 64
    for pen in penalties:
        name = f"{tag}.pen{int(round(pen * 100))}"
        kw = dict(max_new_tokens=n_new, temperature=0.0, top_k=0, top_p=1.0,
                  repetition_penalty=pen)
        spec = _trajectory(lambda m, *a, **k: ref_mtp.generate_mtp(m, mtp, *a, **k), model,
                           prompt, stop_ids=[], device="cpu", **kw)
        ar = _trajectory(ref_generate.generate, model, prompt, stop_ids=[], device="cpu", **kw)
        assert len(spec) == n_new and spec == ar, (name, spec, ar)
        out[f"{name}.tokens"] = torch.tensor(spec, dtype=torch.int64)
        # teacher-forced logits along the trajectory: row i predicts token i
        full = torch.tensor([prompt + spec])
        with torch.no_grad():
            lg32 = model(full)[0][0, len(prompt) - 1:-1].float()
            lg16 = model16(full)[0][0, len(prompt) - 1:-1].float()
        vals, idxs, dev, changed = [], [], 0.0, []
        for i in range(n_new):
            prev = prompt + spec[:i]
            r32 = _penalised(lg32[i], prev, pen)
            r16 = _penalised(lg16[i].to(torch.bfloat16), prev, pen).float()
            v, ix = r32.topk(TOPN)
            vals.append(v)
            idxs.append(ix)
            dev = max(dev, (r16 - r32).abs().max().item())
            changed.append(int(int(lg32[i].argmax()) != spec[i]))
            # the incremental trajectory's pick is the teacher-forced argmax up to
            # chunked-vs-recurrent rounding
            assert r32[spec[i]] >= v[0] - 1e-3, (name, i)
        out[f"{name}.top_vals"] = torch.stack(vals)
        out[f"{name}.top_idx"] = torch.stack(idxs)
        out[f"{name}.bf16_dev"] = torch.tensor([dev])
        out[f"{name}.changed_by_penalty"] = torch.tensor(changed)


def sample_next_penalty_rows(ref_generate, out):
    """Rows where the penalty decides the greedy pick: the largest logit is a seen
    token, positive (divided) or, in a row of negatives, negative (multiplied)."""
    g = torch.Generator().manual_seed(23)
    V = 4096
    rows, prevs, picks = [], [], []
    for r in range(32):
        x = torch.randn(V, generator=g) * 3.0
        if r % 4 == 3:
            x = -x.abs() - 0.5                          # all negative: x * penalty
        x = x.to(torch.bfloat16)
        top = x.float().topk(4).indices.tolist()
        prev = top[: 1 + r % 3] + torch.randint(0, V, (50,), generator=g).tolist()
        pen = (1.05, 1.3, 0.9, 1.1)[r % 4]
        pick = ref_generate.sample_next(x, 0.0, 0, 1.0, pen, prev)
        rows.append(x)
        prevs.append(torch.tensor(prev[:53] + [-1] * (53 - len(prev[:53]))))
        picks.append([pick, int(pen * 1000)])
    out["penalty.logits"] = torch.stack(rows)
    out["penalty.prev"] = torch.stack(prevs).to(torch.int64)
    out["penalty.pick_and_milli"] = torch.tensor(picks, dtype=torch.int64)


def main():
    ref_generate, ref_mtp, ref_weights = _ref_modules()
    torch.manual_seed(0)
    out = {}
    model, mtp = mtp_forward_cases(ref_mtp, ref_weights, "micro", micro_config_dict(), out)
    speculate_case(ref_mtp, model, mtp, micro_config_dict(), out)
    mtp_forward_cases(ref_mtp, ref_weights, "tiny", tiny_config_dict(), out)
    sample_next_penalty_rows(ref_generate, out)
    trajectories(ref_generate, ref_mtp, ref_weights, out, "c1", tiny_config_dict(), [1.0])
    trajectories(ref_generate, ref_mtp, ref_weights, out, "micro", micro_config_dict(),
                 [1.0, 1.05, 1.3])
    save_file({k: v.contiguous() for k, v in out.items()},
              os.path.join(HERE, "ref_mtp.safetensors"))
    print("reference fixtures written to", os.path.join(HERE, "ref_mtp.safetensors"))


if __name__ == "__main__":
    main()
