"""GPU parity of the reference's remaining entry points.

* ``sage_attn_forward`` / ``sage_attn_forward_masked`` (sage_attention.py:121-268):
  no LSE, bf16 P.V, QK quantization and smoothing from ``configure_sage``.
* ``futudiffu::sage_attn`` / ``futudiffu::sage_attn_masked`` (sage_attention.py:
  664-690, :740-769), as the legacy router calls them (attention.py:77-79,
  :101-103): transposed [B, H, N, D] views of [B, N, H*D] projections.

Each is compared with the oracle (max-abs <= 2e-2, cosine >= 0.999, LSE
within 2e-3), and the legacy ops' gradients with the backward they wrap.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

TOL_MAXABS = 2e-2
TOL_COS = 0.999
LSE_TOL = 2e-3
SEGMENTS = [300, 500, 223]


@pytest.fixture
def sa():
    from futudiffu_amd import sage_attention as SA
    yield SA
    SA.configure_sage()  # the reference's defaults: smoothing, fp8 QK, bf16 P.V


def _close(out, ref, what):
    out, ref = out.float().cpu(), ref.float()
    maxabs = (out - ref).abs().max().item()
    cos = O.cosine(out, ref)
    assert maxabs <= TOL_MAXABS and cos >= TOL_COS, f"{what}: max-abs {maxabs:.4g}, cosine {cos:.6f}"
    print(f"  {what}: max-abs {maxabs:.3e} cosine {cos:.7f}", flush=True)


def _lse_close(lse, ref_lse, what):
    lse = lse.cpu()
    fin = torch.isfinite(ref_lse)
    assert torch.equal(fin, torch.isfinite(lse)), f"{what}: LSE -inf pattern"
    err = (lse[fin] - ref_lse[fin]).abs().max().item()
    assert err <= LSE_TOL, f"{what}: LSE error {err:.3g}"


def _router_views(q, k, v, cuda):
    """[B, H, N, D] -> the legacy router's form: [B, N, H*D] projections viewed
    back as non-contiguous [B, H, N, D] (attention.py:67-70)."""
    B, H, N, D = q.shape
    return [t.transpose(1, 2).reshape(B, N, H * D).to(cuda).view(B, N, H, D).transpose(1, 2) for t in (q, k, v)]


@pytest.mark.parametrize("qk", ["int8", "fp8"])
def test_forward_without_lse_matches_oracle(cuda, sa, qk):
    B, H, N, D = 1, 2, 1023, 128
    q, k, v = O.make_inputs(B, H, N, D, seed=61)
    sm = 1.0 / math.sqrt(D)
    sa.configure_sage(qk_quant=qk, pv_quant="fp8")  # the no-LSE entry points still use bf16 P.V
    bm = O.build_block_mask(SEGMENTS, N)
    print(f"sage_attn_forward[_masked] {qk}", flush=True)
    out = sa.sage_attn_forward(q.to(cuda), k.to(cuda), v.to(cuda), sm)
    outm = sa.sage_attn_forward_masked(q.to(cuda), k.to(cuda), v.to(cuda), bm.to(cuda), sm)
    torch.cuda.synchronize()
    assert out.shape == (B, H, N, D) and out.dtype == torch.bfloat16
    ref, _, _ = O.sage_forward(q, k, v, sm, qk, "bf16", "token", True)
    _close(out, ref, f"sage_attn_forward {qk}")
    refm, _, _ = O.sage_forward(q, k, v, sm, qk, "bf16", "token", True, bm)
    _close(outm, refm, f"sage_attn_forward_masked {qk}")


def test_forward_without_lse_follows_smoothing_switch(cuda, sa):
    B, H, N, D = 1, 2, 300, 128
    q, k, v = O.make_inputs(B, H, N, D, seed=62)
    sa.configure_sage(smooth_k=False, qk_quant="int8")
    out = sa.sage_attn_forward(q.to(cuda), k.to(cuda), v.to(cuda))
    torch.cuda.synchronize()
    ref, _, _ = O.sage_forward(q, k, v, None, "int8", "bf16", "token", False)
    _close(out, ref, "sage_attn_forward without smoothing")


@pytest.mark.parametrize("qk,pv", [("int8", "fp8"), ("fp8", "bf16")])
def test_legacy_unmasked_op_matches_oracle(cuda, sa, qk, pv):
    """futudiffu::sage_attn with the configured variant, on the router's
    transposed views, and its gradients against the backward it wraps."""
    B, H, N, D = 1, 2, 700, 128
    q, k, v = O.make_inputs(B, H, N, D, seed=63)
    sm = 1.0 / math.sqrt(D)
    sa.configure_sage(qk_quant=qk, pv_quant=pv)
    qd, kd, vd = (t.requires_grad_() for t in _router_views(q, k, v, cuda))
    assert not qd.is_contiguous()
    print(f"futudiffu::sage_attn {qk}/{pv}", flush=True)
    out, lse = torch.ops.futudiffu.sage_attn(qd, kd, vd, sm)
    torch.cuda.synchronize()
    ref, ref_lse, _ = O.sage_forward(q, k, v, sm, qk, pv, "token", True)
    _close(out, ref, f"futudiffu::sage_attn {qk}/{pv}")
    _lse_close(lse, ref_lse, "futudiffu::sage_attn")
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(1)).bfloat16().to(cuda)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), g)
    want = sa.sage_backward(qd.detach(), kd.detach(), vd.detach(), out.detach(), lse, g, sm, qk=qk, smooth_k=True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert torch.equal(a.contiguous().view(torch.int16), b.view(torch.int16)), f"{name} differs"


def test_legacy_masked_op_matches_oracle(cuda, sa):
    """futudiffu::sage_attn_masked (int8 QK, bf16 P.V, the reference tile mask)
    through the module-level name the legacy router imports."""
    B, H, N, D = 1, 2, 1023, 128
    q, k, v = O.make_inputs(B, H, N, D, seed=64)
    sm = 1.0 / math.sqrt(D)
    bm = O.build_block_mask(SEGMENTS, N)
    qd, kd, vd = (t.requires_grad_() for t in _router_views(q, k, v, cuda))
    print("futudiffu::sage_attn_masked", flush=True)
    out, lse = sa.sage_attn_masked_op(qd, kd, vd, bm.to(cuda), sm)
    torch.cuda.synchronize()
    ref, ref_lse, _ = O.sage_forward(q, k, v, sm, "int8", "bf16", "token", True, bm)
    _close(out, ref, "futudiffu::sage_attn_masked")
    _lse_close(lse, ref_lse, "futudiffu::sage_attn_masked")
    g = torch.randn(out.shape, generator=torch.Generator().manual_seed(2)).bfloat16().to(cuda)
    dq, dk, dv = torch.autograd.grad(out, (qd, kd, vd), g)
    want = sa.sage_backward(qd.detach(), kd.detach(), vd.detach(), out.detach(), lse, g, sm,
                            block_mask=bm.to(cuda), qk="int8", smooth_k=True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv"), (dq, dk, dv), want):
        assert torch.equal(a.contiguous().view(torch.int16), b.view(torch.int16)), f"{name} differs"
