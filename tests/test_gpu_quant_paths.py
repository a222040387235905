"""The quantization's launch forms give the same bits.

With smoothing, ``sage_quantize_qkv`` runs one kernel: its K workgroups wait
for their head's column sums through flags tagged with a per-call epoch, and
after a bounded wait they form the sums themselves.  Large launches whose heads
have 256-token chunks read K once (each K workgroup holds its chunk while it
waits, the single-read form); the others use the lagged form, whose K blocks
read K a second time.  Under stream capture it runs two kernels instead (a
captured epoch would repeat on every replay).  ``SAGE_QUANT_PATH`` forces a
form from the host: ``two`` (two kernels), ``lagged`` (the lagged one-kernel
form), ``fused`` (the single-read form wherever it applies) or ``fallback``
(the default one-kernel form with K workgroups that skip the wait and form the
sums themselves), so each form is checked against the others bit for bit, and
the default against the oracle.

Heads of 20000 tokens take 1024-token chunks at D = 128 (512 at D = 64), the
widening that keeps every head within 24 (48) chunk sums.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

PATHS = (None, "two", "fallback", "lagged", "fused")
FIELDS = ("q_codes", "q_scale", "k_codes", "k_scale", "v_op", "v_scale", "k_mean")

CASES = [
    # (B, H, N, D, qk, pv, gran)
    (1, 30, 4416, 128, "int8", "fp8", "token"),
    (4, 30, 4352, 128, "int8", "fp8", "token"),  # 2040 single-read K workgroups: more than stay resident
    (1, 2, 20000, 128, "int8", "fp8", "token"),
    (1, 2, 20000, 64, "fp8", "bf16", "token"),
    (2, 3, 1000, 128, "fp8", "fp8", "block64"),
    (1, 2, 77, 64, "int8", "bf16", "block64"),
]


def _sa():
    from futudiffu_amd import sage_attention as SA
    return SA


def _bits(t):
    if t is None:
        return None
    t = t.detach().cpu().contiguous()
    return t.view(torch.uint8) if t.dtype != torch.uint8 else t


def _outputs(qz):
    return {f: _bits(getattr(qz, f)) for f in FIELDS}


def _run_paths(monkeypatch, fn):
    res = {}
    for path in PATHS:
        if path is None:
            monkeypatch.delenv("SAGE_QUANT_PATH", raising=False)
        else:
            monkeypatch.setenv("SAGE_QUANT_PATH", path)
        res[path] = _outputs(fn())
        torch.cuda.synchronize()
    monkeypatch.delenv("SAGE_QUANT_PATH", raising=False)
    return res


def _assert_same(res, what):
    ref = res[None]
    for path in PATHS[1:]:
        for f in FIELDS:
            a, b = ref[f], res[path][f]
            if a is None:
                assert b is None
                continue
            bad = a != b
            assert not bad.any(), f"{what}: {f} of path {path!r} differs from the one-kernel path at {int(bad.sum())} bytes"


@pytest.mark.parametrize("B,H,N,D,qk,pv,gran", CASES)
def test_quantize_paths_bit_identical(cuda, monkeypatch, B, H, N, D, qk, pv, gran):
    from futudiffu_amd import layout
    SA = _sa()
    q, k, v = O.make_inputs(B, H, N, D, seed=N + 3 * D)
    qd, kd, vd = q.to(cuda), k.to(cuda), v.to(cuda)
    sm = 1.0 / math.sqrt(D)
    print(f"quantize paths {B}x{H}x{N}x{D} {qk}/{pv}/{gran}", flush=True)
    res = _run_paths(monkeypatch, lambda: SA.quantize_qkv(qd, kd, vd, sm, qk=qk, pv=pv, granularity=gran))
    _assert_same(res, f"{B}x{H}x{N}x{D}")
    # the default form against the oracle: the smoothing mean and the K codes
    oz = O.quantize_all(q, k, v, sm, qk, pv, gran, True)
    BH, Np = B * H, (N + 127) // 128 * 128
    assert torch.equal(res[None]["k_mean"].view(torch.int16).view(B, H, 1, D), oz.mu.view(torch.int16))
    rows = layout.unpack_rows(res[None]["k_codes"], BH, Np, D)
    assert torch.equal(rows[:, :N], oz.kc.contiguous().view(torch.uint8)), "k codes differ from the oracle"


def test_quantize_from_qkv_paths_bit_identical(cuda, monkeypatch):
    """The producer-fused form (projection output through RMSNorm + rotary)."""
    SA = _sa()
    B, N, H, D = 1, 1000, 3, 128
    g = torch.Generator().manual_seed(17)
    qkv = (torch.randn(B, N, 3 * H * D, generator=g) * 2.0).bfloat16().to(cuda)
    qw = (1.0 + 0.3 * torch.randn(D, generator=g)).to(cuda)
    kw = (1.0 + 0.3 * torch.randn(D, generator=g)).to(cuda)
    ang = torch.rand(B, N, 1, D // 2, generator=g) * 6.283
    c, s = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).to(cuda)
    for qk, pv in (("int8", "fp8"), ("fp8", "bf16")):
        print(f"quantize_from_qkv paths {qk}/{pv}", flush=True)
        res = _run_paths(monkeypatch, lambda: SA.quantize_from_qkv(qkv, qw, kw, freqs, H, D, 1e-5, qk=qk, pv=pv))
        _assert_same(res, f"from_qkv {qk}/{pv}")


def test_quantize_under_graph_capture(cuda):
    """A captured quantization (the two-kernel form) replayed on new inputs:
    every replay equals the eager call on the same inputs, with eager work and
    synchronization between the replays."""
    SA = _sa()
    B, H, N, D = 1, 4, 1000, 128
    sm = 1.0 / math.sqrt(D)
    q, k, v = (t.to(cuda) for t in O.make_inputs(B, H, N, D, seed=71))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            SA.quantize_qkv(q, k, v, sm, qk="int8", pv="fp8")
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        qz_g = SA.quantize_qkv(q, k, v, sm, qk="int8", pv="fp8")
    for rep in range(3):
        nq, nk, nv = O.make_inputs(B, H, N, D, seed=100 + rep)
        q.copy_(nq.to(cuda))
        k.copy_(nk.to(cuda))
        v.copy_(nv.to(cuda))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = _outputs(qz_g)
        want = _outputs(SA.quantize_qkv(q, k, v, sm, qk="int8", pv="fp8"))
        torch.cuda.synchronize()
        for f in FIELDS:
            if want[f] is None:
                continue
            assert torch.equal(got[f], want[f]), f"replay {rep}: {f} differs from the eager call"
        print(f"  replay {rep}: equal to eager", flush=True)
