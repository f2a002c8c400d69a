"""Fused inputs: the MTP head's (lollm_mtp_input: the embedding lookup of the draft
tokens, both pre-fc RMSNorms and their concatenation, src/qwen3_5/mtp.py:61-73) and the
verify block's (lollm_verify_input: the ids [pending | drafts], their embedding rows and
layer 0's input norm, mtp.py:141-142 + modeling_qwen3_5.py:86,48), each in one kernel.
Both share lollm_rmsnorm's row arithmetic, so they must equal the unfused ops bit for
bit, and sit within one bf16 rounding of the oracle's rmsnorm_plus1 (blocks.py:23-35) in
fp32."""

import pytest
import torch
import torch.nn.functional as F

from oracle import qwen3_5_ref as R

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,H,V,strided", [(16, 4096, 1000, False), (3, 512, 77, True),
                                           (1, 8192, 5, False)])
def test_mtp_input_equals_lookup_norms_cat(B, H, V, strided):
    from lollm_amd import ops
    print(f"case mtp_input B={B} H={H} V={V} strided={strided}", flush=True)
    g = torch.Generator().manual_seed(B * 131 + H)
    table = torch.randn(V, H, generator=g).bfloat16().cuda()
    w_e = (0.1 * torch.randn(H, generator=g)).bfloat16().cuda()
    w_h = (0.1 * torch.randn(H, generator=g)).bfloat16().cuda()
    tok = torch.randint(0, V, (B,), generator=g).int().cuda()
    base = torch.randn(B, 2 * H if strided else H, generator=g).bfloat16().cuda()
    hidden = base[:, :H]                      # row stride 2H when strided
    eps = 1e-6
    got = ops.mtp_input(tok, hidden, table, w_e, w_h, eps)
    torch.cuda.synchronize()
    emb = F.embedding(tok.long(), table)
    ref = torch.cat([ops.rmsnorm(emb.contiguous(), w_e, eps),
                     ops.rmsnorm(hidden.contiguous(), w_h, eps)], -1)
    assert torch.equal(got, ref)
    o = torch.cat([R.rmsnorm_plus1(emb.float().cpu(), w_e.float().cpu(), eps),
                   R.rmsnorm_plus1(hidden.float().cpu(), w_h.float().cpu(), eps)], -1)
    torch.testing.assert_close(got.float().cpu(), o, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("B,k,H,V", [(16, 3, 4096, 1000), (3, 1, 256, 50), (5, 0, 512, 70)])
def test_verify_input_equals_cat_lookup_norm(B, k, H, V):
    """lollm_verify_input against what it replaces: torch.cat of [pending | drafts], the
    embedding lookup, layer 0's input norm (lollm_rmsnorm) and lengths + 1 + k, bit for
    bit; the norm also against the oracle's fp32 RMSNorm."""
    from lollm_amd import ops
    print(f"case verify_input B={B} k={k} H={H} V={V}", flush=True)
    g = torch.Generator().manual_seed(B * 17 + k)
    table = torch.randn(V, H, generator=g).bfloat16().cuda()
    w = (0.1 * torch.randn(H, generator=g)).bfloat16().cuda()
    first = torch.randint(0, V, (B,), generator=g).int().cuda()
    drafts = torch.randint(0, V, (B, k), generator=g).int().cuda()
    lengths = torch.randint(0, 3000, (B,), generator=g).int().cuda()
    eps = 1e-6
    ids, x, y, kv_len = ops.verify_input(first, drafts, table, w, eps, lengths)
    torch.cuda.synchronize()
    ref_ids = torch.cat([first.view(B, 1), drafts], 1)
    assert torch.equal(ids, ref_ids)
    emb = F.embedding(ref_ids.long(), table)
    assert torch.equal(x, emb)
    assert torch.equal(y, ops.rmsnorm(emb.contiguous(), w, eps))
    assert torch.equal(kv_len, lengths + k + 1)
    o = R.rmsnorm_plus1(emb.float().cpu(), w.float().cpu(), eps)
    torch.testing.assert_close(y.float().cpu(), o, rtol=1e-2, atol=1e-2)


def test_verify_input_keeps_ids_and_clamps_lookup():
    """Ids outside the table are stored as given and clamped into it for the lookup."""
    from lollm_amd import ops
    H, V = 256, 9
    table = torch.randn(V, H).bfloat16().cuda()
    w = torch.zeros(H).bfloat16().cuda()
    first = torch.tensor([-5, 40], dtype=torch.int32).cuda()
    drafts = torch.tensor([[3], [11]], dtype=torch.int32).cuda()
    ids, x, y, kv_len = ops.verify_input(first, drafts, table, w, 1e-6)
    assert kv_len is None
    assert ids.cpu().tolist() == [[-5, 3], [40, 11]]
    _, x2, y2, _ = ops.verify_input(torch.tensor([0, V - 1], dtype=torch.int32).cuda(),
                                    torch.tensor([[3], [V - 1]], dtype=torch.int32).cuda(),
                                    table, w, 1e-6)
    assert torch.equal(x, x2) and torch.equal(y, y2)


def test_mtp_input_clamps_ids():
    """Ids outside the table are clamped into it (the kernel never reads out of range)."""
    from lollm_amd import ops
    H, V = 256, 9
    table = torch.randn(V, H).bfloat16().cuda()
    w = torch.zeros(H).bfloat16().cuda()
    hidden = torch.randn(2, H).bfloat16().cuda()
    got = ops.mtp_input(torch.tensor([-5, 40], dtype=torch.int32).cuda(), hidden, table, w, w, 1e-6)
    ref = ops.mtp_input(torch.tensor([0, V - 1], dtype=torch.int32).cuda(), hidden, table, w, w, 1e-6)
    assert torch.equal(got, ref)
