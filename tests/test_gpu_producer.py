"""GPU: the q/k/v producer (fused_qkv_postprocess, fused_kernels.py:271-390)
and the quantization fused into it.

* ``qkv_postprocess`` is bit-exact against the oracle's restatement.
* ``quantize_from_qkv`` (producer inside the quantization kernels) writes the
  same bytes as ``quantize_qkv`` of the producer's bf16 outputs, for every
  variant, at small shapes and at the 1x30x4416x128 shape.
* ``futudiffu_ii::sage_attn_qkv_masked`` (producer + quantization + masked
  attention + out-projection layout) matches the oracle's attention on the
  oracle's producer outputs.
* The producer's backward (fused_kernels.py:711-783) is within one bf16 step
  of the oracle's fp64 evaluation, v's gradient bit-exact; autograd through
  ``futudiffu::fused_qkv_postprocess`` and ``sage_attn_qkv_masked`` reaches
  ``qkv`` with the oracle's gradients.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu


def _inputs(b, n, h, d, seed):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(b, n, 3 * h * d, generator=g) * 2.0).bfloat16()
    qw = 1.0 + 0.3 * torch.randn(d, generator=g)
    kw = 1.0 + 0.3 * torch.randn(d, generator=g)
    ang = torch.rand(b, n, 1, d // 2, generator=g) * 6.283
    c, s = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2)
    return qkv, qw, kw, freqs


# head counts around the 8-head slab groups: one group of 1, 2 or 3, 8 + 1 and
# 8 + 4 heads per batch over several batches, and 8, 8, 8, 6 at full size;
# single-token and sub-pass sequences
@pytest.mark.parametrize("B,N,H,D", [(2, 300, 3, 128), (1, 77, 2, 64), (2, 300, 9, 128), (3, 129, 12, 64),
                                     (3, 1, 1, 64), (2, 17, 5, 128), (1, 4416, 30, 128)])
def test_qkv_postprocess_matches_oracle(cuda, B, N, H, D):
    from futudiffu_amd import sage_attention as SA
    qkv, qw, kw, freqs = _inputs(B, N, H, D, seed=N + D)
    print(f"producer B={B} N={N} H={H} D={D}", flush=True)
    got = SA.qkv_postprocess(qkv.to(cuda), qw.to(cuda), kw.to(cuda), freqs.to(cuda), H, D, 1e-5)
    torch.cuda.synchronize()
    want = O.qkv_postprocess(qkv, qw, kw, freqs, H, D, 1e-5)
    for name, g, w in zip("qkv", got, want):
        bad = g.cpu().view(torch.int16) != w.view(torch.int16)
        assert not bad.any(), f"{name}: {int(bad.sum())} of {bad.numel()} differ, first at {bad.nonzero()[0].tolist()}"


VARIANTS = [
    ("int8", "fp8", "token", True), ("int8", "bf16", "token", True), ("fp8", "bf16", "token", True),
    ("fp8", "fp8", "block64", True), ("int8", "bf16", "block64", False), ("fp8", "fp8", "token", False),
]


def _same_quantized(a, b):
    for f in ("q_codes", "q_scale", "k_codes", "k_scale", "v_op", "v_scale", "k_mean"):
        x, y = getattr(a, f), getattr(b, f)
        assert (x is None) == (y is None), f
        if x is not None:
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f"{f} differs"


@pytest.mark.parametrize("qk,pv,gran,smooth", VARIANTS)
@pytest.mark.parametrize("B,N,H,D", [(2, 300, 3, 128), (1, 700, 2, 64), (2, 300, 9, 128), (3, 129, 12, 64),
                                     (3, 1, 1, 64), (2, 17, 5, 128)])
def test_quantize_from_qkv_equals_two_steps(cuda, B, N, H, D, qk, pv, gran, smooth):
    from futudiffu_amd import sage_attention as SA
    qkv, qw, kw, freqs = (t.to(cuda) for t in _inputs(B, N, H, D, seed=11 + N))
    sm = 1.0 / math.sqrt(D)
    fused = SA.quantize_from_qkv(qkv, qw, kw, freqs, H, D, 1e-5, sm, qk=qk, pv=pv, granularity=gran,
                                 smooth_k=smooth)
    q, k, v = SA.qkv_postprocess(qkv, qw, kw, freqs, H, D, 1e-5)
    two = SA.quantize_qkv(q, k, v, sm, qk=qk, pv=pv, granularity=gran, smooth_k=smooth)
    torch.cuda.synchronize()
    _same_quantized(fused, two)


def test_quantize_from_qkv_equals_two_steps_at_full_size(cuda):
    from futudiffu_amd import sage_attention as SA
    B, N, H, D = 1, 4416, 30, 128
    qkv, qw, kw, freqs = (t.to(cuda) for t in _inputs(B, N, H, D, seed=5))
    print("fused producer quantize 1x30x4416x128", flush=True)
    fused = SA.quantize_from_qkv(qkv, qw, kw, freqs, H, D, qk="int8", pv="fp8")
    two = SA.quantize_qkv(*SA.qkv_postprocess(qkv, qw, kw, freqs, H, D), qk="int8", pv="fp8")
    torch.cuda.synchronize()
    _same_quantized(fused, two)


def test_qkv_masked_op_matches_oracle(cuda):
    import futudiffu_amd  # noqa: F401  (registers the ops)
    B, N, H, D = 1, 1023, 2, 128
    qkv, qw, kw, freqs = _inputs(B, N, H, D, seed=19)
    bm = O.build_block_mask([300, 500, 223], N)
    sm = 1.0 / math.sqrt(D)
    out, lse = torch.ops.futudiffu_ii.sage_attn_qkv_masked(qkv.to(cuda), qw.to(cuda), kw.to(cuda), freqs.to(cuda),
                                                           bm.to(cuda), H, D, 1e-5, sm)
    torch.cuda.synchronize()
    assert out.shape == (B, N, H * D) and lse.shape == (B * H, N)
    q, k, v = O.qkv_postprocess(qkv, qw, kw, freqs, H, D, 1e-5)
    ref, ref_lse, _ = O.sage_forward(q, k, v, sm, "int8", "bf16", "token", True, bm, None)
    ref = ref.float().transpose(1, 2).reshape(B, N, H * D)
    assert (out.float().cpu() - ref).abs().max().item() <= 2e-2
    assert O.cosine(out.cpu(), ref) >= 0.999
    fin = torch.isfinite(ref_lse)
    assert (lse.cpu()[fin] - ref_lse[fin]).abs().max().item() <= 2e-3


def _ulp_bf16(x):
    """Spacing of bf16 numbers at |x| (normal range)."""
    e = torch.floor(torch.log2(x.abs().clamp_min(2.0 ** -126)))
    return torch.exp2(e - 7)


@pytest.mark.parametrize("B,N,H,D", [(2, 300, 3, 128), (1, 77, 2, 64), (1, 4416, 30, 128)])
def test_producer_backward_matches_oracle(cuda, B, N, H, D):
    """HIP backward of the producer (fused_kernels.py:711-783) against the
    oracle's fp64 evaluation: within one bf16 step of the result (fp32
    arithmetic with fp64 row sums on the GPU), v's gradient bit-exact."""
    from futudiffu_amd import sage_attention as SA
    qkv, qw, kw, freqs = _inputs(B, N, H, D, seed=N + 3)
    g = torch.Generator().manual_seed(N)
    gq, gk, gv = (torch.randn(B, H, N, D, generator=g).bfloat16() for _ in range(3))
    print(f"producer bwd B={B} N={N} H={H} D={D}", flush=True)
    got = SA.qkv_postprocess_backward(*(t.to(cuda) for t in (qkv, qw, kw, freqs, gq, gk, gv)), H, D, 1e-5)
    torch.cuda.synchronize()
    got = got.cpu()
    want = O.qkv_postprocess_backward(qkv, qw, kw, freqs, gq, gk, gv, H, D, 1e-5)
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    hd = H * D
    assert torch.equal(got[..., 2 * hd:], want[..., 2 * hd:])
    w = want[..., :2 * hd].float()
    err = (got[..., :2 * hd].float() - w).abs()
    bound = 1.01 * _ulp_bf16(w) + 1e-6 * w.abs().max()
    bad = err > bound
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} beyond one bf16 step, worst {err.max().item():.3e}"


def test_autograd_through_fused_qkv_postprocess(cuda):
    import futudiffu_amd.fused_kernels  # noqa: F401  (registers futudiffu::fused_qkv_postprocess)
    B, N, H, D = 1, 200, 2, 128
    qkv, qw, kw, freqs = _inputs(B, N, H, D, seed=23)
    g = torch.Generator().manual_seed(24)
    gq, gk, gv = (torch.randn(B, H, N, D, generator=g).bfloat16() for _ in range(3))
    x = qkv.to(cuda).requires_grad_(True)
    q, k, v = torch.ops.futudiffu.fused_qkv_postprocess(x, qw.to(cuda), kw.to(cuda), freqs.to(cuda), H, D, 1e-5)
    (q.float() * gq.to(cuda).float() + k.float() * gk.to(cuda).float() + v.float() * gv.to(cuda).float()).sum() \
        .backward()
    torch.cuda.synchronize()
    want = O.qkv_postprocess_backward(qkv, qw, kw, freqs, gq, gk, gv, H, D, 1e-5)
    err = (x.grad.cpu().float() - want.float()).abs()
    assert (err <= 1.01 * _ulp_bf16(want.float()) + 1e-6 * want.float().abs().max()).all()


def test_autograd_through_qkv_masked_op(cuda):
    """futudiffu_ii::sage_attn_qkv_masked differentiated with respect to qkv:
    the oracle's attention backward (int8, smoothed, on the GPU forward's
    output and LSE) followed by the oracle's producer backward."""
    import futudiffu_amd  # noqa: F401  (registers the ops)
    B, N, H, D = 1, 700, 2, 128
    qkv, qw, kw, freqs = _inputs(B, N, H, D, seed=29)
    bm = O.build_block_mask([300, 400], N)
    sm = 1.0 / math.sqrt(D)
    dout = torch.randn(B, N, H * D, generator=torch.Generator().manual_seed(30)).bfloat16()
    x = qkv.to(cuda).requires_grad_(True)
    print("qkv masked autograd", flush=True)
    out, lse = torch.ops.futudiffu_ii.sage_attn_qkv_masked(x, qw.to(cuda), kw.to(cuda), freqs.to(cuda), bm.to(cuda),
                                                           H, D, 1e-5, sm)
    (out.float() * dout.to(cuda).float()).sum().backward()
    torch.cuda.synchronize()
    q, k, v = O.qkv_postprocess(qkv, qw, kw, freqs, H, D, 1e-5)
    o_bhnd = out.detach().cpu().view(B, N, H, D).transpose(1, 2).contiguous()
    do_bhnd = dout.view(B, N, H, D).transpose(1, 2).contiguous()
    dq, dk, dv = O.sage_backward(q, k, v, o_bhnd, lse.detach().cpu(), do_bhnd, sm, block_mask=bm)
    want = O.qkv_postprocess_backward(qkv, qw, kw, freqs, dq, dk, dv, H, D, 1e-5).float()
    got = x.grad.cpu().float()
    assert O.cosine(got, want) >= 0.9999
    assert (got - want).abs().max().item() <= 1e-2 * want.abs().max().item() + 1e-3
