"""GPU: the Sage attention backward (sage_attention.py:344-458 / :534-648,
sage_kernels.py:321-349, :805-1030, :1491-1722) through the C ABI.

* The HIP dQ, dK, dV match the oracle's restatement given the same forward
  output and LSE, for int8 and fp8 QK, with and without smoothing, unmasked,
  tile-masked (2D and 3D masks) and with exact document ids, at ragged sizes
  and D in {64, 128}.  Differences come from exp2 rounding, fp32 (GPU) vs
  fp64 (oracle) accumulation and the bf16 roundings of P and dS that those
  move across a tie: the bound is cosine >= 0.9999 and a max-abs error within
  1% of the gradient's magnitude.
* The custom ops' autograd (futudiffu_ii::sage_attn_masked, ::sage_attn,
  ::sage_attn_ext) routes through the backward ops and matches the oracle.
* At 1x30x4416x128 two heads are checked against the oracle, and all heads
  against size-independent identities: the rows of P sum to 1, so
  sum_n dV[n] = sum_m dO[m]; softmax is shift-invariant, so sum_n dK[n] = 0.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu


def _close(got, want, name, cos_min=0.9999, rel=1e-2):
    got = got.float().cpu()
    want = want.float()
    cos = O.cosine(got, want)
    err = (got - want).abs().max().item()
    scale = want.abs().max().item()
    assert cos >= cos_min, f"{name}: cosine {cos:.6f}"
    assert err <= rel * scale + 1e-3, f"{name}: max-abs {err:.3e} vs scale {scale:.3e}"


def _inputs(b, h, n, d, seed):
    q, k, v = O.make_inputs(b, h, n, d, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    dout = torch.randn(b, h, n, d, generator=g).bfloat16()
    return q, k, v, dout


def _run(cuda, q, k, v, dout, qk, smooth, block_mask=None, doc_ids=None):
    from futudiffu_amd import sage_attention as SA
    d = q.shape[-1]
    sm = 1.0 / math.sqrt(d)
    qg, kg, vg, dog = (t.to(cuda) for t in (q, k, v, dout))
    bmg = None if block_mask is None else block_mask.to(cuda)
    dg = None if doc_ids is None else doc_ids.to(cuda)
    out, lse = SA.sage_forward(qg, kg, vg, sm, block_mask=bmg, doc_ids=dg, qk=qk, pv="bf16", smooth_k=smooth)
    dq, dk, dv = SA.sage_backward(qg, kg, vg, out, lse, dog, sm, block_mask=bmg, doc_ids=dg, qk=qk,
                                  smooth_k=smooth)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu(), dq.cpu(), dk.cpu(), dv.cpu()


@pytest.mark.parametrize("qk", ["int8", "fp8"])
@pytest.mark.parametrize("smooth", [True, False])
@pytest.mark.parametrize("B,H,N,D", [(1, 2, 200, 128), (2, 3, 300, 64), (1, 2, 1023, 128)])
def test_backward_matches_oracle(cuda, B, H, N, D, qk, smooth):
    q, k, v, dout = _inputs(B, H, N, D, seed=N + D)
    print(f"bwd B={B} H={H} N={N} D={D} qk={qk} smooth={smooth}", flush=True)
    out, lse, dq, dk, dv = _run(cuda, q, k, v, dout, qk, smooth)
    rq, rk, rv = O.sage_backward(q, k, v, out, lse, dout, 1.0 / math.sqrt(D), qk=qk, smooth=smooth)
    for name, g, w in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        assert g.shape == w.shape and g.dtype == torch.bfloat16
        assert torch.isfinite(g.float()).all(), name
        _close(g, w, name)


@pytest.mark.parametrize("three_d,qk", [(False, "int8"), (True, "int8"), (False, "fp8")])
def test_tile_masked_backward_matches_oracle(cuda, three_d, qk):
    B, H, N, D = 1, 2, 700, 128
    q, k, v, dout = _inputs(B, H, N, D, seed=3)
    bm = O.build_block_mask([300, 250, 150], N)
    if three_d:
        bm = bm.unsqueeze(0).repeat(B * H, 1, 1)
        bm[1, 0, 3] = 1  # a head-specific extra tile pair
    print(f"bwd tile mask 3d={three_d} qk={qk}", flush=True)
    out, lse, dq, dk, dv = _run(cuda, q, k, v, dout, qk, True, block_mask=bm)
    rq, rk, rv = O.sage_backward(q, k, v, out, lse, dout, 1.0 / math.sqrt(D), qk=qk, block_mask=bm)
    for name, g, w in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        _close(g, w, name)


@pytest.mark.parametrize("qk,D", [("int8", 64), ("int8", 128), ("fp8", 64)])
def test_doc_masked_backward_matches_oracle(cuda, qk, D):
    B, H, N = 2, 2, 520
    q, k, v, dout = _inputs(B, H, N, D, seed=5)
    doc = torch.full((B, N), -1, dtype=torch.int32)
    doc[0, :200], doc[0, 200:450] = 0, 1
    doc[1, 30:300], doc[1, 300:520] = 0, 1
    print(f"bwd doc ids qk={qk} D={D}", flush=True)
    out, lse, dq, dk, dv = _run(cuda, q, k, v, dout, qk, True, doc_ids=doc)
    rq, rk, rv = O.sage_backward(q, k, v, out, lse, dout, 1.0 / math.sqrt(D), qk=qk, doc_ids=doc)
    for name, g, w in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        _close(g, w, name)
    # padded keys get no gradient
    assert not dk[0, :, 450:].float().any() and not dv[1, :, :30].float().any()


def test_backward_close_to_exact_attention(cuda):
    """Against fp64 autograd of unquantized attention, as the reference's own
    test compares with SDPA (test_sage_backward.py:49-93, cosine > 0.95)."""
    B, H, N, D = 1, 2, 512, 128
    q, k, v, dout = _inputs(B, H, N, D, seed=8)
    out, lse, dq, dk, dv = _run(cuda, q, k, v, dout, "int8", True)
    qd, kd, vd = (t.double().requires_grad_(True) for t in (q, k, v))
    ref = torch.softmax(torch.matmul(qd, kd.transpose(-1, -2)) / math.sqrt(D), -1) @ vd
    (ref * dout.double()).sum().backward()
    for name, g, w in (("dq", dq, qd.grad), ("dk", dk, kd.grad), ("dv", dv, vd.grad)):
        assert O.cosine(g, w) >= 0.99, name


def test_autograd_through_custom_ops(cuda):
    import futudiffu_amd  # noqa: F401
    B, H, N, D = 1, 2, 333, 128
    q, k, v, dout = _inputs(B, H, N, D, seed=12)
    sm = 1.0 / math.sqrt(D)
    bm = O.build_block_mask([200, 133], N)
    print("bwd autograd ops", flush=True)
    for kind in ("masked", "plain", "ext_bnhd"):
        qg, kg, vg = (t.to(cuda).requires_grad_(True) for t in (q, k, v))
        if kind == "masked":
            out, lse = torch.ops.futudiffu_ii.sage_attn_masked(qg, kg, vg, bm.to(cuda), sm)
            go = dout.to(cuda)
            ref_kw = dict(block_mask=bm, qk="int8", smooth=True)
        elif kind == "plain":
            from futudiffu_amd import sage_attention as SA
            SA.configure_sage(smooth_k=True, qk_quant="int8", pv_quant="bf16")
            out, lse = torch.ops.futudiffu_ii.sage_attn(qg, kg, vg, sm)
            SA.configure_sage()
            go = dout.to(cuda)
            ref_kw = dict(qk="int8", smooth=True)
        else:
            out, lse = torch.ops.futudiffu_ii.sage_attn_ext(qg, kg, vg, None, None, sm, "fp8", "fp8", "token",
                                                             False, "bnhd")
            go = dout.transpose(1, 2).reshape(B, N, H * D).to(cuda)
            ref_kw = dict(qk="fp8", smooth=False)
        (out.float() * go.float()).sum().backward()
        torch.cuda.synchronize()
        o_bhnd = out.detach().cpu()
        if kind == "ext_bnhd":
            o_bhnd = o_bhnd.view(B, N, H, D).transpose(1, 2).contiguous()
        rq, rk, rv = O.sage_backward(q, k, v, o_bhnd, lse.detach().cpu(), dout, sm, **ref_kw)
        for name, g, w in (("dq", qg.grad, rq), ("dk", kg.grad, rk), ("dv", vg.grad, rv)):
            _close(g, w, f"{kind} {name}")


def test_backward_ops_by_reference_name(cuda):
    """futudiffu_ii::sage_bwd_masked / ::sage_bwd (attention_srcii.py:36-48,
    :91-103) called directly, with the module configuration."""
    import futudiffu_amd  # noqa: F401
    from futudiffu_amd import sage_attention as SA
    B, H, N, D = 1, 2, 257, 128
    q, k, v, dout = _inputs(B, H, N, D, seed=14)
    sm = 1.0 / math.sqrt(D)
    bm = O.build_block_mask([129, 128], N)
    qg, kg, vg, dog = (t.to(cuda) for t in (q, k, v, dout))
    out, lse = torch.ops.futudiffu_ii.sage_attn_masked(qg, kg, vg, bm.to(cuda), sm)
    got = torch.ops.futudiffu_ii.sage_bwd_masked(qg, kg, vg, out, lse, dog, bm.to(cuda), sm)
    want = O.sage_backward(q, k, v, out.cpu(), lse.cpu(), dout, sm, block_mask=bm)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        _close(g, w, f"sage_bwd_masked {name}")
    SA.configure_sage(smooth_k=False, qk_quant="fp8", pv_quant="bf16")
    try:
        out, lse = torch.ops.futudiffu_ii.sage_attn(qg, kg, vg, sm)
        got = torch.ops.futudiffu_ii.sage_bwd(qg, kg, vg, out, lse, dog, sm)
    finally:
        SA.configure_sage()
    want = O.sage_backward(q, k, v, out.cpu(), lse.cpu(), dout, sm, qk="fp8", smooth=False)
    for name, g, w in zip(("dq", "dk", "dv"), got, want):
        _close(g, w, f"sage_bwd {name}")


def test_backward_full_size(cuda):
    from futudiffu_amd import sage_attention as SA
    B, H, N, D = 1, 30, 4416, 128
    q, k, v, dout = _inputs(B, H, N, D, seed=21)
    sm = 1.0 / math.sqrt(D)
    print("bwd 1x30x4416x128", flush=True)
    qg, kg, vg, dog = (t.to(cuda) for t in (q, k, v, dout))
    out, lse = SA.sage_forward(qg, kg, vg, sm, qk="int8", pv="bf16", smooth_k=True)
    dq, dk, dv = SA.sage_backward(qg, kg, vg, out, lse, dog, sm, qk="int8", smooth_k=True)
    torch.cuda.synchronize()
    for g in (dq, dk, dv):
        assert torch.isfinite(g.float()).all()
    # identities over every head
    dvs, dos = dv.double().sum(2), dog.double().sum(2)
    assert (dvs - dos).abs().max().item() <= 0.02 * dos.abs().max().item() + 0.05
    dks = dk.double().sum(2).abs().max().item()
    assert dks <= 0.02 * dk.double().abs().sum(2).max().item()
    # two heads against the oracle
    out_c, lse_c = out.cpu(), lse.cpu()
    for hh in (0, H - 1):
        sl = slice(hh, hh + 1)
        rq, rk, rv = O.sage_backward(q[:, sl], k[:, sl], v[:, sl], out_c[:, sl], lse_c[hh:hh + 1], dout[:, sl],
                                     sm, head_chunk=1)
        for name, g, w in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
            _close(g[:, sl], w, f"head {hh} {name}")


def test_backward_dq_halves_match_whole_items(cuda, monkeypatch):
    """The last dQ items of a launch (up to 64) run as two key-tile halves
    whose fp32 partials the last half to finish adds (first + second): at
    1x8x1100x128, 64 of the 72 dQ items are cut.  dK and dV are the
    same bits as with whole items (SAGE_BWD_SPLIT=off), dQ agrees to fp32
    summation order, two runs give the same bits, and dQ matches the oracle."""
    from futudiffu_amd import sage_attention as SA
    B, H, N, D = 1, 8, 1100, 128
    q, k, v, dout = _inputs(B, H, N, D, seed=29)
    sm = 1.0 / math.sqrt(D)
    qg, kg, vg, dog = (t.to(cuda) for t in (q, k, v, dout))
    print("bwd dQ halves 1x8x1100x128", flush=True)
    out, lse = SA.sage_forward(qg, kg, vg, sm, qk="int8", pv="bf16", smooth_k=True)
    monkeypatch.delenv("SAGE_BWD_SPLIT", raising=False)
    g1 = SA.sage_backward(qg, kg, vg, out, lse, dog, sm, qk="int8", smooth_k=True)
    g2 = SA.sage_backward(qg, kg, vg, out, lse, dog, sm, qk="int8", smooth_k=True)
    monkeypatch.setenv("SAGE_BWD_SPLIT", "off")
    g0 = SA.sage_backward(qg, kg, vg, out, lse, dog, sm, qk="int8", smooth_k=True)
    torch.cuda.synchronize()
    for a, b_ in zip(g1, g2):
        assert torch.equal(a, b_), "the halves' merge must not depend on timing"
    assert torch.equal(g1[1], g0[1]) and torch.equal(g1[2], g0[2]), "dK and dV do not depend on the dQ cut"
    dq1, dq0 = g1[0].float(), g0[0].float()
    assert O.cosine(dq1.cpu(), dq0.cpu()) >= 0.99999
    assert (dq1 - dq0).abs().max().item() <= 1e-2 * dq0.abs().max().item()
    out_c, lse_c = out.cpu(), lse.cpu()
    for hh in (0, H - 1):
        sl = slice(hh, hh + 1)
        rq, _, _ = O.sage_backward(q[:, sl], k[:, sl], v[:, sl], out_c[:, sl], lse_c[hh:hh + 1], dout[:, sl], sm,
                                   head_chunk=1)
        _close(g1[0][:, sl], rq, f"head {hh} dq")
