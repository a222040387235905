"""The compile and graph-capture contract of the ops.

The reference registers its attention as custom ops so that AOT-autograd
tracing under gradient checkpointing and torch.compile work
(src_ii/attention_srcii.py:1-18); its model compiles every block
(src_ii/zimage_model.py:766-772) and the legacy generator captures CUDA graphs
(src/futudiffu/generate.py:250, mode "reduce-overhead").  Here:

* each forward op is captured in a HIP graph (torch.cuda.CUDAGraph) and
  replayed on three new inputs, with eager calls and synchronizations between
  the replays; every replay must equal the eager call bit for bit (the
  producer op too, whose quantization takes another form under capture);
* torch.library.opcheck runs on every forward and backward op (schema, fake
  tensor, autograd registration, AOT dispatch);
* a gradient-checkpointed block that calls futudiffu_ii::sage_attn_masked
  runs through torch.compile(backend="aot_eager", fullgraph=True), forward
  and backward, bit-identical to eager; and through torch's "cudagraphs"
  backend (AOT tracing plus CUDA graph trees, the part of "reduce-overhead"
  that does not generate kernels), forward only, as the generator uses it.
"""

import math

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


def _same(a, b, what):
    assert a.shape == b.shape and a.dtype == b.dtype, what
    bad = _bits(a) != _bits(b)
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} elements differ"


def _inputs(cuda, B, H, N, D, seed):
    return [t.to(cuda) for t in O.make_inputs(B, H, N, D, seed=seed)]


def _doc(cuda, B, N, segs):
    from futudiffu_amd import block_mask as BM
    return BM.build_doc_ids(segs, N, device="cpu", batch=B).to(cuda)


def _capture_and_replay(cuda, fn, make_args, what):
    """Capture fn(*static_args) in a graph; for three new inputs copy them into
    the static inputs, replay, and compare with the eager call of fn."""
    static = make_args(0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):  # warm-up off the capture (allocator, lazy loading)
            fn(*static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got = fn(*static)
    for i in range(1, 4):
        new = make_args(i)
        for s, n in zip(static, new):
            if isinstance(s, torch.Tensor):
                s.copy_(n)
        g.replay()
        torch.cuda.synchronize()
        want = fn(*new)  # eager, between replays
        torch.cuda.synchronize()
        for j, (a, b) in enumerate(zip(got, want)):
            _same(a, b, f"{what}: replay {i}, output {j}")
        print(f"  {what}: replay {i} bit-identical to eager", flush=True)


def test_graph_capture_sage_attn_masked(cuda):
    B, H, N, D = 1, 8, 1000, 128
    bm = O.build_block_mask([300, 500, 200], N).to(cuda)
    sc = 1.0 / math.sqrt(D)
    print("graph capture: futudiffu_ii::sage_attn_masked 1x8x1000x128 (tile mask)", flush=True)

    def make(i):
        q, k, v = _inputs(cuda, B, H, N, D, seed=200 + i)
        return q, k, v, bm

    def fn(q, k, v, m):
        return torch.ops.futudiffu_ii.sage_attn_masked(q, k, v, m, sc)

    _capture_and_replay(cuda, fn, make, "sage_attn_masked")


def test_graph_capture_sage_attn_split_tail(cuda):
    """futudiffu_ii::sage_attn with the int8-QK / fp8-PV configuration at
    1x30x1280x128: 300 query items, the 44 past one per CU cut into two key
    halves and merged by a second kernel; both kernels and the quantization's
    capture form are in the graph."""
    from futudiffu_amd import sage_attention as SA
    B, H, N, D = 1, 30, 1280, 128
    sc = 1.0 / math.sqrt(D)
    print("graph capture: futudiffu_ii::sage_attn int8/fp8 1x30x1280x128 (split items + merge)", flush=True)
    saved = (SA._SAGE_SMOOTH_K, SA._SAGE_QK_QUANT, SA._SAGE_PV_QUANT)
    SA.configure_sage(smooth_k=True, qk_quant="int8", pv_quant="fp8")
    try:
        def make(i):
            return tuple(_inputs(cuda, B, H, N, D, seed=210 + i))

        def fn(q, k, v):
            return torch.ops.futudiffu_ii.sage_attn(q, k, v, sc)

        _capture_and_replay(cuda, fn, make, "sage_attn")
    finally:
        SA.configure_sage(smooth_k=saved[0], qk_quant=saved[1], pv_quant=saved[2])


def test_graph_capture_sage_attn_ext_doc_ids(cuda):
    """futudiffu_ii::sage_attn_ext with exact document ids (key padding
    included): the summary and prefix kernels, the listed split query tiles
    and the attention in one graph; the ids change between replays too."""
    B, H, N, D = 2, 4, 1000, 128
    sc = 1.0 / math.sqrt(D)
    seg_sets = [[300, 500, 150], [640, 320], [128, 128, 700], [999]]
    print("graph capture: futudiffu_ii::sage_attn_ext 2x4x1000x128 int8/fp8 with document ids", flush=True)

    def make(i):
        q, k, v = _inputs(cuda, B, H, N, D, seed=220 + i)
        return q, k, v, _doc(cuda, B, N, seg_sets[i])

    def fn(q, k, v, doc):
        return torch.ops.futudiffu_ii.sage_attn_ext(q, k, v, None, doc, sc, "int8", "fp8", "token", True, "bhnd")

    _capture_and_replay(cuda, fn, make, "sage_attn_ext")


def test_graph_capture_sage_attn_qkv_masked(cuda):
    """futudiffu_ii::sage_attn_qkv_masked from the QKV projection output
    (1x1000x(3*12*128), tile mask): under capture the quantization takes its
    two-kernel form, eagerly the one-kernel slab form; every replay must equal
    the eager call bit for bit."""
    B, N, H, D = 1, 1000, 12, 128
    bm = O.build_block_mask([300, 500, 200], N).to(cuda)
    sc = 1.0 / math.sqrt(D)
    g = torch.Generator().manual_seed(270)
    qw = (1.0 + 0.3 * torch.randn(D, generator=g)).to(cuda)
    kw = (1.0 + 0.3 * torch.randn(D, generator=g)).to(cuda)
    ang = torch.rand(B, N, 1, D // 2, generator=g) * 6.283
    c, s = torch.cos(ang), torch.sin(ang)
    freqs = torch.stack([torch.stack([c, -s], -1), torch.stack([s, c], -1)], -2).to(cuda)
    print("graph capture: futudiffu_ii::sage_attn_qkv_masked 1x1000x12x128 (tile mask)", flush=True)

    def make(i):
        gi = torch.Generator().manual_seed(271 + i)
        return ((torch.randn(B, N, 3 * H * D, generator=gi) * 2.0).bfloat16().to(cuda),)

    def fn(qkv):
        return torch.ops.futudiffu_ii.sage_attn_qkv_masked(qkv, qw, kw, freqs, bm, H, D, 1e-6, sc)

    _capture_and_replay(cuda, fn, make, "sage_attn_qkv_masked")


def _opcheck(op, args, what):
    from torch.library import opcheck
    print(f"opcheck {what}", flush=True)
    res = opcheck(op, args)
    bad = {k: v for k, v in res.items() if v != "SUCCESS"}
    assert not bad, f"{what}: {bad}"


def test_opcheck_forward_ops(cuda):
    B, H, N, D = 1, 2, 320, 128
    sc = 1.0 / math.sqrt(D)
    q, k, v = (t.requires_grad_(True) for t in _inputs(cuda, B, H, N, D, seed=230))
    bm = O.build_block_mask([200, 120], N).to(cuda)
    doc = _doc(cuda, B, N, [200, 100])
    ops = torch.ops.futudiffu_ii
    _opcheck(ops.sage_attn_masked.default, (q, k, v, bm, sc), "sage_attn_masked")
    _opcheck(ops.sage_attn.default, (q, k, v, sc), "sage_attn")
    _opcheck(ops.sage_attn_masked_merged_heads.default, (q, k, v, bm, sc), "sage_attn_masked_merged_heads")
    _opcheck(ops.sage_attn_ext.default, (q, k, v, None, doc, sc, "int8", "fp8", "token", True, "bhnd"),
             "sage_attn_ext (doc ids)")
    _opcheck(ops.sage_attn_ext.default, (q, k, v, bm, None, sc, "int8", "bf16", "token", True, "bnhd"),
             "sage_attn_ext (tile mask, merged heads)")


def test_opcheck_backward_ops(cuda):
    B, H, N, D = 1, 2, 320, 128
    sc = 1.0 / math.sqrt(D)
    q, k, v = _inputs(cuda, B, H, N, D, seed=240)
    bm = O.build_block_mask([200, 120], N).to(cuda)
    doc = _doc(cuda, B, N, [200, 100])
    ops = torch.ops.futudiffu_ii
    out, lse = ops.sage_attn_masked(q, k, v, bm, sc)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(241)).bfloat16().to(cuda)
    _opcheck(ops.sage_bwd_masked.default, (q, k, v, out, lse, dout, bm, sc), "sage_bwd_masked")
    out2, lse2 = ops.sage_attn(q, k, v, sc)
    _opcheck(ops.sage_bwd.default, (q, k, v, out2, lse2, dout, sc), "sage_bwd")
    out3, lse3 = ops.sage_attn_ext(q, k, v, None, doc, sc, "int8", "bf16", "token", True, "bhnd")
    _opcheck(ops.sage_bwd_ext.default, (q, k, v, out3, lse3, dout, None, doc, sc, "int8", True), "sage_bwd_ext")


def _block(q, k, v, wq, wk, gate, bm, sc):
    """The attention part of a transformer block: per-channel scales on q and
    k (in place of the producer's norm), the production op, and a gate on
    its output."""
    out, _ = torch.ops.futudiffu_ii.sage_attn_masked(q * wq, k * wk, v, bm, sc)
    return out * gate


def _checkpointed(q, k, v, wq, wk, gate, bm, sc):
    return torch.utils.checkpoint.checkpoint(_block, q, k, v, wq, wk, gate, bm, sc, use_reentrant=False)


def test_compile_aot_eager_checkpointed_block(cuda):
    torch._dynamo.reset()
    B, H, N, D = 1, 4, 1000, 128
    sc = 1.0 / math.sqrt(D)
    bm = O.build_block_mask([300, 500, 200], N).to(cuda)
    q0, k0, v0 = _inputs(cuda, B, H, N, D, seed=250)
    g = torch.Generator().manual_seed(251)
    wq0 = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(cuda)
    wk0 = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(cuda)
    gate = torch.randn(B, H, N, D, generator=g).bfloat16().to(cuda)
    dout = torch.randn(B, H, N, D, generator=g).bfloat16().to(cuda)
    compiled = torch.compile(_checkpointed, backend="aot_eager", fullgraph=True)
    results = []
    for name, fn in (("eager", _checkpointed), ("aot_eager", compiled)):
        print(f"checkpointed block, {name}: forward and backward", flush=True)
        q, k, v, wq, wk = (t.clone().requires_grad_(True) for t in (q0, k0, v0, wq0, wk0))
        y = fn(q, k, v, wq, wk, gate, bm, sc)
        y.backward(dout)
        torch.cuda.synchronize()
        results.append([y.detach(), q.grad, k.grad, v.grad, wq.grad, wk.grad])
    for j, name in enumerate(("output", "dq", "dk", "dv", "dwq", "dwk")):
        _same(results[1][j], results[0][j], f"aot_eager {name}")
    print("  aot_eager outputs and gradients bit-identical to eager", flush=True)


def test_compile_cudagraphs_backend_forward(cuda):
    torch._dynamo.reset()
    B, H, N, D = 1, 4, 1000, 128
    sc = 1.0 / math.sqrt(D)
    bm = O.build_block_mask([300, 500, 200], N).to(cuda)
    g = torch.Generator().manual_seed(261)
    wq = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(cuda)
    wk = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(cuda)
    gate = torch.randn(B, H, N, D, generator=g).bfloat16().to(cuda)
    compiled = torch.compile(_block, backend="cudagraphs", fullgraph=True)
    with torch.no_grad():
        for i in range(4):  # the first calls warm up and record, later ones replay
            q, k, v = _inputs(cuda, B, H, N, D, seed=262 + i)
            got = compiled(q, k, v, wq, wk, gate, bm, sc).clone()
            torch.cuda.synchronize()
            want = _block(q, k, v, wq, wk, gate, bm, sc)
            torch.cuda.synchronize()
            _same(got, want, f"cudagraphs backend call {i}")
            print(f"  cudagraphs backend call {i} bit-identical to eager", flush=True)
