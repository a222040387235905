"""Pins of the oracle's restatement of the Sage backward
(sage_attention.py:344-458 / :534-648, sage_kernels.py:321-349, :805-1030,
:1491-1722).

The reference has no golden vectors for the backward; its own test compares
against PyTorch SDPA gradients by cosine (test_sage_backward.py:49-93).  Here
the oracle is checked against fp64 autograd of exact attention on inputs whose
per-token int8 quantization is exact (every Q/K row is a power-of-two multiple
of integers in [-127, 127] with one entry at +-127), so the recomputed P equals
the exact softmax up to fp32 rounding and only the reference's bf16 roundings
of P, dS and the outputs remain.  A dropped sm_scale, a transposed product, a
missing D term or a wrong sign each moves the cosine far below the bound.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O


def _exact_rows(b, h, n, d, g, step):
    x = torch.randint(-127, 128, (b, h, n, d), generator=g).double()
    col = torch.randint(0, d, (b, h, n), generator=g)
    sign = torch.where(torch.rand(b, h, n, generator=g) < 0.5, -1.0, 1.0).double()
    x.scatter_(-1, col[..., None], (127.0 * sign)[..., None])
    return (x * step).bfloat16()


def _case(b=1, h=2, n=200, d=64, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = _exact_rows(b, h, n, d, g, 2.0 ** -6)
    k = _exact_rows(b, h, n, d, g, 2.0 ** -6)
    v = torch.randn(b, h, n, d, generator=g).bfloat16()
    dout = torch.randn(b, h, n, d, generator=g).bfloat16()
    return q, k, v, dout


def _autograd(q, k, v, dout, sm_scale, visible=None):
    """Exact gradients of sum(out * dout), out = softmax(q k^T sm_scale) v, in fp64."""
    b, h, n, d = q.shape
    qd, kd, vd = (t.double().requires_grad_(True) for t in (q, k, v))
    s = torch.matmul(qd, kd.transpose(-1, -2)) * sm_scale
    if visible is not None:
        s = s.masked_fill(~visible.view(b, h, n, n), -math.inf)
    lse = torch.logsumexp(s, -1)
    out = torch.matmul(torch.softmax(s, -1), vd)
    (out * dout.double()).sum().backward()
    return out.detach(), (lse.detach() * O.LOG2E).float().view(b * h, n), qd.grad, kd.grad, vd.grad


def _check(got, want, cos_min=0.9999, rel=2e-2):
    assert O.cosine(got, want) >= cos_min
    err = (got.double() - want).abs().max().item()
    assert err <= rel * want.abs().max().item(), err


@pytest.mark.parametrize("n,d", [(200, 64), (130, 128)])
def test_backward_matches_exact_autograd(n, d):
    q, k, v, dout = _case(n=n, d=d, seed=n + d)
    sm = 1.0 / math.sqrt(d)
    out, lse, gq, gk, gv = _autograd(q, k, v, dout, sm)
    dq, dk, dv = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, qk="int8", smooth=False)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        assert got.dtype == torch.bfloat16 and got.shape == q.shape
        _check(got, want)


def test_tile_masked_backward_matches_exact_autograd():
    n, d = 300, 64
    q, k, v, dout = _case(n=n, d=d, seed=7)
    sm = 1.0 / math.sqrt(d)
    bm = O.build_block_mask([150, 150], n)
    vis = O.tile_mask_visibility(bm, 2, n)
    out, lse, gq, gk, gv = _autograd(q, k, v, dout, sm, vis)
    dq, dk, dv = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, smooth=False, block_mask=bm)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        _check(got, want)
    # no gradient flows between documents: keys of tile 3 (tokens 192..255)
    # are hidden from query tile 0 (tokens 0..127), so perturbing dO there
    # leaves dK of those keys unchanged
    dout2 = dout.clone()
    dout2[:, :, 128:] = 0
    _, dk2, _ = O.sage_backward(q, k, v, out.bfloat16(), lse, dout2, sm, smooth=False, block_mask=bm)
    assert torch.equal(dk2[:, :, 192:256], torch.zeros_like(dk2[:, :, 192:256]))


def test_doc_masked_backward_matches_exact_autograd():
    n, d = 150, 64
    q, k, v, dout = _case(n=n, d=d, seed=9)
    sm = 1.0 / math.sqrt(d)
    doc = torch.tensor([[0] * 70 + [1] * 60 + [-1] * 20], dtype=torch.int32)
    vis = O.doc_visibility(doc.long()).expand(2, n, n)
    out, lse, gq, gk, gv = _autograd(q, k, v, dout, sm, vis)
    dq, dk, dv = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, smooth=False, doc_ids=doc)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        _check(got, want)
    # padded keys receive no gradient
    assert not dk[:, :, 130:].any() and not dv[:, :, 130:].any()


def test_fp8_recompute_close_to_exact_autograd():
    """fp8 codes are not exact; the gradients still follow the exact ones."""
    q, k, v, dout = _case(n=160, d=64, seed=3)
    sm = 1.0 / math.sqrt(64)
    out, lse, gq, gk, gv = _autograd(q, k, v, dout, sm)
    dq, dk, dv = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, qk="fp8", smooth=False)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        assert O.cosine(got, want) >= 0.99


def test_smoothing_leaves_gradients_unchanged():
    """Softmax is invariant to a per-channel shift of K, and sum_n dS[m, n] =
    dO_m . (P V)_m - D_m = 0 when O = P V: dQ = dS K~ equals dS K, and dK, dV
    do not depend on the shift.  With exactly quantized K rows whose mean is
    zero (rows come in +- pairs) smoothing changes nothing at all; with a
    general K it changes the gradients only at quantization level."""
    q, k, v, dout = _case(n=128, d=64, seed=5)
    k = torch.cat([k[:, :, :64], -k[:, :, :64]], dim=2)  # column means exactly 0
    sm = 0.125
    out, lse, *_ = _autograd(q, k, v, dout, sm)
    a = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, smooth=True)
    b = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, smooth=False)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    # the LSE is in the units of the scores the forward saw: smoothed scores
    # are shifted by q.mu per row, so each backward takes its own forward's LSE
    q2, k2, v2 = O.make_inputs(1, 2, 150, 64, seed=11)
    k2o = (k2.float() + 3.0).bfloat16()
    do2 = torch.randn(1, 2, 150, 64, generator=torch.Generator().manual_seed(2)).bfloat16()
    grads = []
    for smooth in (True, False):
        o2, l2, _ = O.sage_forward(q2, k2o, v2, sm, "int8", "bf16", "token", smooth)
        grads.append(O.sage_backward(q2, k2o, v2, o2, l2, do2, sm, smooth=smooth))
    for x, y in zip(*grads):
        assert O.cosine(x, y) >= 0.995


def test_delta_prepass_closed_form():
    out = torch.tensor([[[1.0, 2.0, 3.0], [0.5, -0.5, 4.0]]]).bfloat16()
    dout = torch.tensor([[[1.0, 1.0, 1.0], [2.0, 2.0, -1.0]]]).bfloat16()
    assert torch.equal(O.delta_prepass(dout, out), torch.tensor([[6.0, -4.0]]))


def test_rows_of_dv_sum_to_column_sums_of_dout():
    """Rows of P sum to 1, so sum_n dV[n] = sum_m dO[m] (up to bf16 rounding of P)."""
    q, k, v, dout = _case(n=96, d=64, seed=13)
    sm = 0.125
    out, lse, *_ = _autograd(q, k, v, dout, sm)
    _, _, dv = O.sage_backward(q, k, v, out.bfloat16(), lse, dout, sm, smooth=False)
    lhs = dv.double().sum(2)
    rhs = dout.double().sum(2)
    assert (lhs - rhs).abs().max().item() <= 0.02 * rhs.abs().max().item() + 0.05
