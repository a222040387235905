"""GPU: the [B, N, H*D] output layout of the attention epilogue.

JointAttention.forward (transformer.py:467-471 of sqcu/futudiffu) calls the
attention op and then copies its [B, H, N, D] output into [B, N, H*D] for the
out-projection.  The kernel can store rows in that layout directly
(out_layout "bnhd").  The arithmetic is the same, so the values must be
bit-identical to the transposed [B, H, N, D] output, LSE included, on every
kernel path: tile-masked, doc-id masked, unmasked whole items, and unmasked
split-tail items written by the merge of their pieces.  Rows past N must not
be stored: a guard region after the output keeps its fill value.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

FILL = -1536.0  # fill value of the guard region, exact in bf16 (-1.5 * 2^10)


def _bits16(t):
    return t.contiguous().cpu().view(torch.int16)


def _guarded(numel, guard, device):
    buf = torch.full((numel + guard,), FILL, dtype=torch.bfloat16, device=device)
    return buf, buf[:numel]


LAYOUT_CASES = [
    # (B, H, N, D, qk, pv, kind)
    (2, 3, 300, 128, "int8", "bf16", "tile"),    # production masked variant, ragged last query tile
    (2, 2, 700, 64, "fp8", "bf16", "doc"),       # exact document ids with key padding
    (2, 130, 200, 128, "int8", "fp8", "none"),   # 520 items: the last 8 split into pieces and merged
    (2, 130, 256, 64, "fp8", "bf16", "none"),    # split tail at D=64
    (1, 30, 4416, 128, "int8", "fp8", "none"),   # 1280x832 image tokens, 30 heads
]


@pytest.mark.parametrize("B,H,N,D,qk,pv,kind", LAYOUT_CASES)
def test_merged_heads_layout_bit_identical(cuda, B, H, N, D, qk, pv, kind):
    from futudiffu_amd import sage_attention as SA
    print(f"out layout {kind} B={B} H={H} N={N} D={D} {qk}/{pv}", flush=True)
    q, k, v = (t.to(cuda) for t in O.make_inputs(B, H, N, D, seed=61 + N + D))
    bm = doc = None
    if kind == "tile":
        bm = O.build_block_mask([120, 180], N).to(cuda)
    if kind == "doc":
        doc = torch.full((B, N), -1, dtype=torch.int32)
        for b in range(B):
            doc[b, :250 - 40 * b] = 0
            doc[b, 250 - 40 * b:550 - 40 * b] = 1
            doc[b, 20 + b:60 + b] = -1
        doc = doc.to(cuda)
    qz = SA.quantize_qkv(q, k, v, 1.0 / math.sqrt(D), qk=qk, pv=pv)
    numel, guard = B * H * N * D, 128 * H * D
    buf_a, flat_a = _guarded(numel, guard, cuda)
    buf_b, flat_b = _guarded(numel, guard, cuda)
    out_a, lse_a = SA.attn_from_quantized(qz, B, H, block_mask=bm, doc_ids=doc, out=flat_a.view(B, H, N, D))
    out_b, lse_b = SA.attn_from_quantized(qz, B, H, block_mask=bm, doc_ids=doc, out=flat_b.view(B, N, H * D),
                                          out_layout="bnhd")
    torch.cuda.synchronize()
    want = out_a.transpose(1, 2).reshape(B, N, H * D)
    bad = _bits16(out_b) != _bits16(want)
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} differ, first at {bad.nonzero()[0].tolist()}"
    assert torch.equal(lse_a.cpu().view(torch.int32), lse_b.cpu().view(torch.int32)), "LSE differs"
    for name, buf in (("bhnd", buf_a), ("bnhd", buf_b)):
        g = buf[numel:].float()
        assert torch.all(g == FILL), f"{name}: rows past N were stored into the guard region"


def test_merged_heads_op_matches_reference_call_site(cuda):
    """futudiffu_ii::sage_attn_masked_merged_heads against what the caller
    computes from futudiffu_ii::sage_attn_masked (transformer.py:467-471), and
    the result against the oracle."""
    import futudiffu_amd  # noqa: F401  (registers the ops)
    ops = torch.ops.futudiffu_ii
    B, H, N, D = 1, 4, 1023, 128
    q, k, v = O.make_inputs(B, H, N, D, seed=67)
    bm = O.build_block_mask([300, 500, 223], N)
    sm = 1.0 / math.sqrt(D)
    qc, kc, vc, mc = (t.to(cuda) for t in (q, k, v, bm))
    out, lse = ops.sage_attn_masked(qc, kc, vc, mc, sm)
    merged, lse_m = ops.sage_attn_masked_merged_heads(qc, kc, vc, mc, sm)
    torch.cuda.synchronize()
    reshaped = out.transpose(1, 2).reshape(B, -1, H * D)
    assert merged.shape == reshaped.shape == (B, N, H * D)
    assert torch.equal(_bits16(merged), _bits16(reshaped))
    assert torch.equal(lse.cpu(), lse_m.cpu())
    ref, _, _ = O.sage_forward(q, k, v, sm, "int8", "bf16", "token", True, bm, None)
    ref = ref.float().transpose(1, 2).reshape(B, N, H * D)
    assert (merged.float().cpu() - ref).abs().max().item() <= 2e-2
    assert O.cosine(merged.cpu(), ref) >= 0.999
