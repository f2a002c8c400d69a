"""Pins the oracle's Gated DeltaNet math (CPU only).

Checks: transformers golden vectors (tests/golden/gdn_fns.safetensors), closed forms,
chunked == recurrent, an fp64 scalar-loop brute force, and the snapshot/rollback
contract.
"""

import os

import pytest
import torch
from safetensors.torch import load_file

from oracle import qwen3_5_ref as R


@pytest.fixture(scope="module")
def G(golden_dir):
    return load_file(os.path.join(golden_dir, "gdn_fns.safetensors"))


@pytest.mark.parametrize("tag,l2", [("l2", True), ("raw", False)])
def test_recurrent_matches_transformers(G, tag, l2):
    a = {n: G[f"{tag}.{n}"] for n in ("q", "k", "v", "g", "beta", "s0")}
    o, s = R.gdn_scan_recurrent(a["q"], a["k"], a["v"], a["g"], a["beta"], a["s0"], qk_l2=l2)
    torch.testing.assert_close(o, G[f"{tag}.o_rec"], rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(s, G[f"{tag}.s_rec"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("tag,l2", [("l2", True), ("raw", False)])
def test_chunked_matches_transformers(G, tag, l2):
    a = {n: G[f"{tag}.{n}"] for n in ("q", "k", "v", "g", "beta", "s0")}
    o, s = R.gdn_scan_chunked(a["q"], a["k"], a["v"], a["g"], a["beta"], chunk=4,
                              state=a["s0"], qk_l2=l2)
    torch.testing.assert_close(o, G[f"{tag}.o_chunk"], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(s, G[f"{tag}.s_chunk"], rtol=1e-5, atol=1e-5)


def _inputs(B=2, T=5, H=3, D=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g)
    k = torch.randn(B, T, H, D, generator=g)
    v = torch.randn(B, T, H, D, generator=g)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=g))
    gg = -torch.nn.functional.softplus(torch.randn(B, T, H, generator=g))
    s0 = torch.randn(B, H, D, D, generator=g) * 0.1
    return q, k, v, gg, beta, s0


@pytest.mark.parametrize("chunk", [4, 64])
def test_chunked_equals_recurrent(chunk):
    q, k, v, g, b, s0 = _inputs(T=11)
    o1, s1 = R.gdn_scan_recurrent(q, k, v, g, b, s0, qk_l2=True)
    o2, s2 = R.gdn_scan_chunked(q, k, v, g, b, chunk=chunk, state=s0, qk_l2=True)
    torch.testing.assert_close(o1, o2, rtol=1e-4, atol=1e-5)
    torch.testing.assert_close(s1, s2, rtol=1e-4, atol=1e-5)


def test_closed_form_single_step():
    q, k, v, g, b, s0 = _inputs(B=1, T=1, H=1, D=8)
    o, s = R.gdn_scan_recurrent(q, k, v, g, b, s0)
    S = s0[0, 0].double() * torch.exp(g[0, 0, 0].double())
    kk, qq, vv = k[0, 0, 0].double(), q[0, 0, 0].double(), v[0, 0, 0].double()
    d = (vv - S.t() @ kk) * b[0, 0, 0].double()
    S = S + torch.outer(kk, d)
    torch.testing.assert_close(s[0, 0].double(), S, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(o[0, 0, 0].double(), S.t() @ qq / 8 ** 0.5, rtol=1e-5, atol=1e-6)


def test_beta_zero_is_pure_decay():
    q, k, v, g, b, s0 = _inputs(T=4)
    o, s = R.gdn_scan_recurrent(q, k, v, g, torch.zeros_like(b), s0)
    expect = s0 * g.sum(1).exp()[..., None, None]
    torch.testing.assert_close(s, expect, rtol=1e-5, atol=1e-6)


def test_zero_state_unit_beta_gives_outer_product():
    q, k, v, g, b, s0 = _inputs(T=1)
    k = k / k.norm(dim=-1, keepdim=True)
    o, s = R.gdn_scan_recurrent(q, k, v, torch.zeros_like(g), torch.ones_like(b), None)
    expect = k[:, 0, :, :, None] * v[:, 0, :, None, :]
    torch.testing.assert_close(s, expect, rtol=1e-5, atol=1e-6)


def test_fp64_scalar_bruteforce():
    q, k, v, g, b, s0 = _inputs(B=1, T=3, H=2, D=4, seed=3)
    o, s = R.gdn_scan_recurrent(q.double(), k.double(), v.double(), g.double(), b.double(),
                                s0.double())
    D = 4
    for h in range(2):
        S = [[float(s0[0, h, i, j]) for j in range(D)] for i in range(D)]
        for t in range(3):
            dec = float(torch.exp(g[0, t, h].double()))
            S = [[S[i][j] * dec for j in range(D)] for i in range(D)]
            kv = [sum(S[i][j] * float(k[0, t, h, i]) for i in range(D)) for j in range(D)]
            dl = [(float(v[0, t, h, j]) - kv[j]) * float(b[0, t, h]) for j in range(D)]
            S = [[S[i][j] + float(k[0, t, h, i]) * dl[j] for j in range(D)] for i in range(D)]
            for j in range(D):
                oj = sum(S[i][j] * float(q[0, t, h, i]) for i in range(D)) / D ** 0.5
                assert abs(oj - float(o[0, t, h, j])) < 2e-6   # scan runs in fp32
        for i in range(D):
            for j in range(D):
                assert abs(S[i][j] - float(s[0, h, i, j])) < 2e-6


def test_snapshots_and_rollback():
    q, k, v, g, b, s0 = _inputs(T=5)
    o, snaps = R.gdn_scan_recurrent_snapshots(q, k, v, g, b, s0, qk_l2=True)
    o_ref, s_ref = R.gdn_scan_recurrent(q, k, v, g, b, s0, qk_l2=True)
    torch.testing.assert_close(o, o_ref)
    torch.testing.assert_close(snaps[:, -1], s_ref)
    for a in range(5):                       # rollback to a accepted => first a+1 tokens
        _, s_a = R.gdn_scan_recurrent(q[:, :a + 1], k[:, :a + 1], v[:, :a + 1],
                                      g[:, :a + 1], b[:, :a + 1], s0, qk_l2=True)
        torch.testing.assert_close(snaps[:, a], s_a)


def test_l2norm_and_gated_norm_match_transformers(G):
    torch.testing.assert_close(R.l2_normalize(G["l2norm.x"]), G["l2norm.y"])
    y = R.rmsnorm_gated(G["gnorm.x"], G["gnorm.z"], G["gnorm.w"], 1e-6)
    torch.testing.assert_close(y, G["gnorm.y"])


def test_planted_mistake_is_caught(G):
    """A wrong sign in the delta rule must fail the golden comparison."""
    a = {n: G[f"l2.{n}"] for n in ("q", "k", "v", "g", "beta", "s0")}
    o, _ = R.gdn_scan_recurrent(a["q"], a["k"], -a["v"], a["g"], a["beta"], a["s0"], qk_l2=True)
    assert not torch.allclose(o, G["l2.o_rec"], rtol=1e-3, atol=1e-3)
