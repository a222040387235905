"""Pins of the oracle's restatement of the q/k/v producer
(fused_qkv_postprocess, src/futudiffu/fused_kernels.py:271-390): closed forms
of the rotation, the RMS normalization against an fp64 evaluation, the layout
of the split and transpose, and the V pass-through."""

import math

import pytest
import torch

from oracle import sage_oracle as O


def _inputs(b=2, n=37, h=3, d=64, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    qkv = (scale * torch.randn(b, n, 3 * h * d, generator=g)).bfloat16()
    qw = 1.0 + 0.2 * torch.randn(d, generator=g)
    kw = 1.0 + 0.2 * torch.randn(d, generator=g)
    ang = torch.rand(b, n, 1, d // 2, generator=g) * 6.283
    c, s = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2)  # [b, n, 1, d/2, 2, 2]
    return qkv, qw, kw, freqs


def _rot(freqs, c, s):
    f = torch.empty_like(freqs)
    f[..., 0, 0], f[..., 0, 1], f[..., 1, 0], f[..., 1, 1] = c, -s, s, c
    return f


def _ulp_bf16(x):
    return torch.ldexp(torch.ones_like(x), torch.frexp(x.abs().clamp_min(1e-30))[1] - 8)


def test_split_transpose_and_v_pass_through():
    b, n, h, d = 2, 5, 3, 64
    qkv, qw, kw, freqs = _inputs(b, n, h, d)
    q, k, v = O.qkv_postprocess(qkv, qw, kw, _rot(freqs, 1.0, 0.0), h, d)
    assert q.shape == k.shape == v.shape == (b, h, n, d) and q.dtype == torch.bfloat16
    x = qkv.view(b, n, 3, h, d)
    assert torch.equal(v, x[:, :, 2].transpose(1, 2))
    # head hh of token t of q comes from columns [hh*d, (hh+1)*d) of the first third
    for hh in range(h):
        xq = x[:, :, 0, hh].float()
        rr = 1.0 / torch.sqrt((xq.double() ** 2).mean(-1, keepdim=True) + 1e-5)
        want = (xq.double() * rr * qw.double()).float()
        got = q[:, hh].float()
        assert ((got - want).abs() <= _ulp_bf16(want)).all()


def test_quarter_turn_is_an_exact_pair_swap():
    """cos = 0, sin = 1: even' = -odd, odd' = even, exactly (the products by 0
    and +-1 are exact), against the identity rotation of the same input."""
    qkv, qw, kw, freqs = _inputs(seed=1)
    q0, k0, _ = O.qkv_postprocess(qkv, qw, kw, _rot(freqs, 1.0, 0.0), 3, 64)
    q9, k9, _ = O.qkv_postprocess(qkv, qw, kw, _rot(freqs, 0.0, 1.0), 3, 64)
    for a0, a9 in ((q0, q9), (k0, k9)):
        assert torch.equal(a9[..., 0::2], -a0[..., 1::2])
        assert torch.equal(a9[..., 1::2], a0[..., 0::2])


def test_rotation_matches_fp64_complex_product():
    qkv, qw, kw, freqs = _inputs(seed=2)
    q, k, _ = O.qkv_postprocess(qkv, qw, kw, freqs, 3, 64)
    x = qkv.view(2, 37, 3, 3, 64)
    for j, (w, got) in enumerate(((qw, q), (kw, k))):
        xx = x[:, :, j].double()
        rr = 1.0 / torch.sqrt((xx ** 2).mean(-1, keepdim=True) + 1e-5)
        nn = xx * rr * w.double()
        z = torch.complex(nn[..., 0::2], nn[..., 1::2])
        ang = torch.complex(freqs[..., 0, 0].double(), freqs[..., 1, 0].double())  # cos + i sin
        r = z * ang
        want = torch.stack([r.real, r.imag], -1).flatten(-2).movedim(1, 2)
        err = (got.double() - want).abs()
        # bf16 output rounding plus fp32 rounding of the products and sums
        assert (err <= 1.01 * _ulp_bf16(want.float()).double() + 1e-6 * nn.abs().amax().item()).all()


def test_normalized_rows_have_unit_rms():
    qkv, _, _, freqs = _inputs(seed=3, scale=7.0)
    ones = torch.ones(64)
    q, _, _ = O.qkv_postprocess(qkv, ones, ones, freqs, 3, 64)
    rms = q.double().pow(2).mean(-1).sqrt()
    assert ((rms - 1.0).abs() < 1e-2).all()


def test_eps_dominates_tiny_rows():
    """x = 0 gives 0; a row far below sqrt(eps) is scaled by 1/sqrt(eps)."""
    qkv, qw, kw, freqs = _inputs(seed=4)
    qkv = qkv.clone()
    qkv[0, 0, :64] = 0
    qkv[0, 1, :64] = torch.tensor(1e-6).bfloat16()
    ones = torch.ones(64)
    q, _, _ = O.qkv_postprocess(qkv, ones, ones, _rot(freqs, 1.0, 0.0), 3, 64)
    assert torch.equal(q[0, 0, 0], torch.zeros(64, dtype=torch.bfloat16))
    want = float(torch.tensor(1e-6).bfloat16()) / math.sqrt(1e-12 + 1e-5)
    assert abs(float(q[0, 0, 1, 0]) - want) <= 2 * float(_ulp_bf16(torch.tensor(want)))


def test_five_dim_freqs_equal_six_dim():
    qkv, qw, kw, freqs = _inputs(seed=5)
    a = O.qkv_postprocess(qkv, qw, kw, freqs, 3, 64)
    b = O.qkv_postprocess(qkv, qw, kw, freqs.squeeze(2), 3, 64)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_sum_of_squares_order_is_runs_of_eight_then_pairwise():
    """The sum of squares is defined in a fixed fp64 order (8 channels left to
    right, then a pairwise tree over the runs).  With one square 2^60 and the
    others 9, a left-to-right sum over all channels loses every small term
    (ulp 256) while the tree keeps some of them; the oracle must give the tree's
    value, evaluated here with Python floats (IEEE fp64)."""
    d = 64
    vals = [3.0] * d
    vals[0] = 2.0 ** 30
    x = torch.tensor(vals).bfloat16().view(1, d)
    sq = [float(v) ** 2 for v in x.flatten().tolist()]
    runs = []
    for r in range(d // 8):
        acc = sq[8 * r]
        for e in range(1, 8):
            acc = acc + sq[8 * r + e]
        runs.append(acc)
    while len(runs) > 1:
        runs = [runs[i] + runs[i + 1] for i in range(0, len(runs), 2)]
    seq = 0.0
    for v in sq:
        seq = seq + v
    assert runs[0] == 2.0 ** 60 + 512 and seq == 2.0 ** 60
    assert O.sum_squares(x).item() == runs[0]


def _producer_fp64(qkv, qw, kw, freqs, h, d, eps=1e-5):
    """Differentiable fp64 producer: RMSNorm with weights, then the rotation."""
    b, n, _ = qkv.shape
    x = qkv.view(b, n, 3, h, d)
    f = freqs.squeeze(2).double()[:, :, None]  # [B, N, 1, D/2, 2, 2]

    def one(xr, w):
        rr = 1.0 / torch.sqrt((xr * xr).mean(-1, keepdim=True) + eps)
        nn = (xr * rr * w).reshape(b, n, h, d // 2, 2)
        e = f[..., 0, 0] * nn[..., 0] + f[..., 0, 1] * nn[..., 1]
        o = f[..., 1, 0] * nn[..., 0] + f[..., 1, 1] * nn[..., 1]
        return torch.stack([e, o], -1).reshape(b, n, h, d).movedim(1, 2)

    return one(x[:, :, 0], qw.double()), one(x[:, :, 1], kw.double()), x[:, :, 2].movedim(1, 2)


@pytest.mark.parametrize("d", [64, 128])
def test_producer_backward_matches_fp64_autograd(d):
    """The restated backward (fused_kernels.py:711-783) against autograd of the
    fp64 producer on the same bf16 input: differences are the bf16 rounding
    of the result only.  A dropped mean term, a wrong rotation sign or the
    wrong norm weight moves the result far outside the bound."""
    b, n, h = 2, 19, 3
    qkv, qw, kw, freqs = _inputs(b, n, h, d, seed=8, scale=1.5)
    g = torch.Generator().manual_seed(9)
    gq, gk, gv = (torch.randn(b, h, n, d, generator=g).bfloat16() for _ in range(3))
    x = qkv.double().requires_grad_(True)
    q, k, v = _producer_fp64(x, qw, kw, freqs, h, d)
    (q * gq.double()).sum().add_((k * gk.double()).sum()).add_((v * gv.double()).sum()).backward()
    want = x.grad
    got = O.qkv_postprocess_backward(qkv, qw, kw, freqs, gq, gk, gv, h, d)
    assert got.shape == qkv.shape and got.dtype == torch.bfloat16
    err = (got.double() - want).abs()
    assert (err <= 1.01 * _ulp_bf16(want.float()).double() + 1e-9).all(), err.max()
    # v's gradient is the incoming one, untransposed
    assert torch.equal(got[..., 2 * h * d:], gv.movedim(1, 2).reshape(b, n, h * d))
