"""Fused input of the MTP head (lollm_mtp_input): the embedding lookup of the draft
tokens, both pre-fc RMSNorms and their concatenation (src/qwen3_5/mtp.py:61-73) in one
kernel.  It shares lollm_rmsnorm's row arithmetic, so it must equal the unfused
lookup + lollm_rmsnorm x 2 + cat bit for bit, and sit within one bf16 rounding of the
oracle's rmsnorm_plus1 (blocks.py:23-35) in fp32."""

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
