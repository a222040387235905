"""The C ABI (include/sage_mi355x.h) and the host-side mirror, without a GPU.

* libsage_mi355x.so loads and exports every function the header declares,
  with the ctypes prototypes the Python glue binds.
* Argument validation returns the documented status codes before any device
  work (so no GPU is touched), with a message in sage_last_error().
* The Python entry points raise the reference's exception types
  (sage_attention.py:54-57 ValueError for bad variants, :487-488
  AssertionError for head_dim/dtype).
"""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sage_mi355x.h")

# The validation tests below pass small fake device addresses (16, 32, ...).
# Each base argument set is itself invalid (no workspace, or a null output),
# so a call whose one override stops being rejected still returns a status
# instead of launching; and where a GPU is visible they do not run at all,
# so a check that regresses can never send a kernel to those addresses.
fake_addresses = pytest.mark.skipif(torch.cuda.device_count() > 0,
                                    reason="argument-validation calls with fake device addresses run without a GPU")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\s*\*?\s+(sage_\w+)\s*\(", text, re.M)))


def test_header_declarations_found():
    names = _declared()
    assert {"sage_quantize_qkv", "sage_attn_fwd", "sage_abi_version", "sage_last_error"} <= set(names)


def test_library_exports_every_declared_symbol():
    from futudiffu_amd import _lib
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes prototype"
    assert lib.sage_abi_version() == 6


def test_sizes_and_padding():
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert [lib.sage_padded_len(n) for n in (1, 128, 129, 4416)] == [128, 128, 256, 4480]
    # fp64 K column sums per head and chunk, then an 8-byte flag per chunk,
    # then per head an 8-byte mean flag and the fp32 mean; chunks of 256
    # tokens, widened by multiples of 256 so that a head has at most
    # 12 * (256 / D) of them
    def ws(bh, nch, d):
        return bh * nch * (d + 1) * 8 + bh * (8 + 4 * d)
    assert lib.sage_quant_workspace_bytes(30, 4416, 128) == ws(30, 18, 128)
    assert lib.sage_quant_workspace_bytes(2, 256, 64) == ws(2, 1, 64)
    assert lib.sage_quant_workspace_bytes(1, 257, 64) == ws(1, 2, 64)
    # 20000 tokens: 79 pieces of 256 -> 1024-token chunks (20) at D=128, 512-token (40) at D=64
    assert lib.sage_quant_workspace_bytes(1, 20000, 128) == ws(1, 20, 128)
    assert lib.sage_quant_workspace_bytes(1, 20000, 64) == ws(1, 40, 64)
    # per-batch summaries of every 64-key tile and 32- and 128-row query block
    # and the scheduled key-tile range of each 128-row query block (int4 each),
    # the list of split query tiles (a count and 2 entries, int4 each),
    # then (256-byte aligned) fp32 slots of 128 x D + 512 floats for the pieces
    # of the split tail, and an 8-byte arrival counter per split item: 26
    # items x 4 pieces (the cap) at the 1x30x4416x128 headline shape (1050
    # items = 2 rounds of 512 + 26); below one round, the items past one per
    # CU (256), when at most 128 of them, in min(4, 256 // spilled, nt // 2)
    # pieces, at least 2: 300 items at 1x30x1280 -> 44 x 4, 350 (1x35x1280)
    # -> 94 x 2, 260 items at 1x26x1280 -> 4 x 4, 260 items of 3 tiles
    # (1x130x160) -> 4 x 2, 400 items (1x40x1280) uncut
    for b, h, n, d, items, parts in ((2, 3, 200, 128, 0, 1), (1, 30, 4416, 128, 26, 4), (1, 1, 1, 64, 0, 1),
                                     (1, 30, 1280, 128, 44, 4), (1, 40, 1280, 128, 0, 1), (1, 26, 1280, 128, 4, 4),
                                     (1, 35, 1280, 128, 94, 2), (1, 130, 160, 64, 4, 2),
                                     (2, 30, 4416, 128, 52, 4)):
        np_, nt = (n + 127) // 128 * 128, (n + 63) // 64
        doc = ((b * (nt + np_ // 32 + 2 * (np_ // 128)) + 1 + 2) * 16 + 255) // 256 * 256
        assert lib.sage_attn_workspace_bytes(b, h, n, d) == doc + items * parts * (128 * d + 512) * 4 + items * 8
        # a masked launch splits no item: the summaries only
        assert lib.sage_attn_masked_workspace_bytes(b, h, n, d) == doc


def _quant_call(lib, **over):
    a = dict(q=16, k=32, v=48, bh=2, n=100, d=128, qk=0, pv=1, gran=0, smooth=1, fold=0.18,
             qc=64, qs=80, kc=96, ks=112, vo=128, vs=144, km=160, ws=None, wsb=0, stream=None)
    a.update(over)
    return lib.sage_quantize_qkv(a["q"], a["k"], a["v"], a["bh"], a["n"], a["d"], a["qk"], a["pv"], a["gran"],
                                 a["smooth"], a["fold"], a["qc"], a["qs"], a["kc"], a["ks"], a["vo"], a["vs"],
                                 a["km"], a["ws"], a["wsb"], a["stream"])


@pytest.mark.parametrize("over,status,msg", [
    (dict(d=96), 1, "head_dim"),
    (dict(n=0), 1, "positive"),
    (dict(qk=3), 1, "qk_kind"),
    (dict(pv=2), 1, "pv_kind"),
    (dict(gran=7), 1, "granularity"),
    (dict(q=None), 1, "null"),
    (dict(vs=None), 1, "v_scale"),
    (dict(k=33), 2, "aligned"),
    (dict(km=None), 1, "k_mean"),
    (dict(ws=176, wsb=8), 3, "workspace"),
    (dict(ws=184, wsb=1 << 20), 2, "workspace must be 16-byte aligned"),
    (dict(bh=70000), 1, "grid"),
    (dict(bh=65535, n=1 << 24), 1, "beyond one launch"),
])
@fake_addresses
def test_quantize_rejects_bad_arguments(over, status, msg):
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert _quant_call(lib, **over) == status
    assert msg in lib.sage_last_error().decode()


def _attn_call(lib, **over):
    a = dict(qc=16, qs=32, kc=48, ks=64, vi=80, vs=96, b=1, h=2, n=300, d=128, qk=0, pv=1, gran=0,
             mask=None, sz=0, nq=3, nkv=5, doc=None, ws=None, wsb=0, out=112, layout=0, lse=128, stream=None)
    a.update(over)
    return lib.sage_attn_fwd(a["qc"], a["qs"], a["kc"], a["ks"], a["vi"], a["vs"], a["b"], a["h"], a["n"], a["d"],
                             a["qk"], a["pv"], a["gran"], a["mask"], a["sz"], a["nq"], a["nkv"], a["doc"], a["ws"],
                             a["wsb"], a["out"], a["layout"], a["lse"], a["stream"])


@pytest.mark.parametrize("over,status,msg", [
    (dict(b=0), 1, "positive"),
    (dict(d=64 + 32), 1, "head_dim"),
    (dict(mask=256, nq=2), 1, "block_mask must be 3 x 5"),
    (dict(mask=256, sz=7), 1, "mask_stride_z"),
    (dict(ws=None), 3, "workspace"),
    (dict(doc=256, ws=None), 3, "workspace"),
    (dict(ws=256, wsb=100), 3, "workspace of"),
    (dict(doc=256, ws=264, wsb=1 << 24), 2, "workspace must be 16-byte aligned"),
    (dict(out=None), 1, "null"),
    (dict(pv=1, vs=None), 1, "v_scale"),
    (dict(layout=2), 1, "out_layout must be 0"),
    (dict(layout=-1), 1, "out_layout must be 0"),
    (dict(n=(1 << 22) + 1, nq=0, nkv=0), 1, "exceeds 4194304"),
])
@fake_addresses
def test_attn_rejects_bad_arguments(over, status, msg):
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert _attn_call(lib, **over) == status
    assert msg in lib.sage_last_error().decode()


def _prod_args(**over):
    a = dict(qkv=16, qw=32, kw=48, fr=64, b=1, h=2, n=100, d=128, eps=1e-5)
    a.update(over)
    return [a[x] for x in ("qkv", "qw", "kw", "fr", "b", "h", "n", "d", "eps")]


@pytest.mark.parametrize("over,status,msg", [
    (dict(b=0), 1, "positive"),
    (dict(h=70000), 1, "grid limit"),
    (dict(n=0), 1, "positive"),
    (dict(d=96), 1, "head_dim"),
    (dict(qkv=None), 1, "null"),
    (dict(fr=None), 1, "null"),
    (dict(qw=40), 2, "aligned"),
    (dict(eps=-1.0), 1, "norm_eps"),
    (dict(h=30000), 1, "too wide"),
])
@fake_addresses
def test_producer_entries_reject_bad_arguments(over, status, msg):
    from futudiffu_amd import _lib
    lib = _lib.load()
    # outputs null / workspace missing: rejected after the producer checks
    assert lib.sage_qkv_postprocess(*_prod_args(**over), 80, 96, None, None) == status
    assert msg in lib.sage_last_error().decode()
    assert lib.sage_quantize_from_qkv(*_prod_args(**over), 0, 1, 0, 1, 0.18, 128, 144, 160, 176, 192, 208, 224,
                                      None, 0, None) == status
    assert msg in lib.sage_last_error().decode()
    a = _prod_args(**over)
    assert lib.sage_qkv_postprocess_bwd(*a[:4], 80, 96, 112, *a[4:], None, None) == status
    assert msg in lib.sage_last_error().decode()


@fake_addresses
def test_producer_backward_checks_gradient_pointers():
    from futudiffu_amd import _lib
    lib = _lib.load()
    a = _prod_args()
    assert lib.sage_qkv_postprocess_bwd(*a[:4], 80, None, 112, *a[4:], 128, None) == 1
    assert "null" in lib.sage_last_error().decode()
    assert lib.sage_qkv_postprocess_bwd(*a[:4], 80, 96, 112, *a[4:], None, None) == 1
    assert lib.sage_qkv_postprocess_bwd(*a[:4], 80, 96, 120, *a[4:], 128, None) == 2
    assert "aligned" in lib.sage_last_error().decode()
    assert lib.sage_qkv_postprocess_bwd(*a[:4], 80, 96, 112, *a[4:], 136, None) == 2


def test_producer_backward_python_glue_checks():
    from futudiffu_amd import sage_attention as SA
    qkv = torch.zeros(1, 8, 3 * 2 * 64, dtype=torch.bfloat16)
    w = torch.ones(64)
    fr = torch.zeros(1, 8, 1, 32, 2, 2)
    g = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="grad_k must be"):
        SA.qkv_postprocess_backward(qkv, w, w, fr, g, g[:, :1], g, 2, 64)


def _bwd_call(lib, **over):
    a = dict(q=16, k=32, v=48, out=64, lse=80, do=96, b=1, h=2, n=300, d=128, qk=0, smooth=1, sm=0.088,
             sml=0.1275, mask=None, sz=0, nq=3, nkv=5, doc=None, ws=None, wsb=0, dq=112, dk=128, dv=144,
             stream=None)
    a.update(over)
    return lib.sage_attn_bwd(a["q"], a["k"], a["v"], a["out"], a["lse"], a["do"], a["b"], a["h"], a["n"], a["d"],
                             a["qk"], a["smooth"], a["sm"], a["sml"], a["mask"], a["sz"], a["nq"], a["nkv"],
                             a["doc"], a["ws"], a["wsb"], a["dq"], a["dk"], a["dv"], a["stream"])


@pytest.mark.parametrize("over,status,msg", [
    (dict(b=0), 1, "positive"),
    (dict(n=0), 1, "positive"),
    (dict(d=96), 1, "head_dim"),
    (dict(qk=2), 1, "qk_kind"),
    (dict(h=70000), 1, "grid"),
    (dict(dq=None), 1, "null"),
    (dict(lse=None), 1, "null"),
    (dict(do=40), 2, "aligned"),
    (dict(sm=0.0), 1, "sm_scale"),
    (dict(sml=-1.0), 1, "sm_scale"),
    (dict(mask=256, nkv=4), 1, "block_mask must be 3 x 5"),
    (dict(mask=256, sz=9), 1, "mask_stride_z"),
    (dict(ws=None), 3, "workspace"),
    (dict(ws=256, wsb=1000), 3, "workspace of"),
    (dict(ws=264, wsb=1 << 30), 2, "workspace must be 16-byte aligned"),
])
@fake_addresses
def test_backward_rejects_bad_arguments(over, status, msg):
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert _bwd_call(lib, **over) == status
    assert msg in lib.sage_last_error().decode()


def test_backward_workspace_size():
    """Codes (1 B), scales (4 B) of Q and K; the K mean; the column-sum
    partials; five bf16 operand images (dO, Q and K~ transposed, dO and V by
    row); D (4 B); the document-id summaries (16 B per 64-key tile and per
    32- and 128-row block of each batch); the fp32 partial dQ of up to 64
    items cut in two key halves (64 x 2 x 128 x D floats) and their 8-byte
    counters: each region 256-byte aligned."""
    from futudiffu_amd import _lib
    lib = _lib.load()
    for b, h, n, d in ((1, 30, 4416, 128), (2, 3, 300, 64), (1, 1, 1, 64)):
        rows = b * h * ((n + 127) // 128 * 128)
        up = lambda x: (x + 255) // 256 * 256  # noqa: E731
        want = (up(rows * d) * 2 + up(rows * 4) * 2 + up(b * h * d * 2) + up(lib.sage_quant_workspace_bytes(b * h, n, d))
                + up(rows * d * 2) * 5 + up(rows * 4))
        np_ = (n + 127) // 128 * 128
        want += up(b * ((n + 63) // 64 + np_ // 32 + np_ // 128) * 16)
        want += up(64 * 2 * 128 * d * 4) + up(64 * 8)
        assert lib.sage_attn_bwd_workspace_bytes(b, h, n, d) == want


def test_backward_python_glue_checks():
    from futudiffu_amd import sage_attention as SA
    q = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    lse = torch.zeros(2, 8)
    with pytest.raises(ValueError):
        SA.sage_backward(q, q, q, q, lse, q, qk="int4")
    with pytest.raises(AssertionError):
        SA.sage_backward(q.float(), q, q, q, lse, q)


@fake_addresses
def test_fused_quantize_entry_checks_outputs():
    from futudiffu_amd import _lib
    lib = _lib.load()
    # v_scale missing for fp8 PV; workspace too small for smoothing
    assert lib.sage_quantize_from_qkv(*_prod_args(), 0, 1, 0, 1, 0.18, 128, 144, 160, 176, 192, None, 224,
                                      None, 0, None) == 1
    assert "v_scale" in lib.sage_last_error().decode()
    assert lib.sage_quantize_from_qkv(*_prod_args(), 0, 1, 0, 1, 0.18, 128, 144, 160, 176, 192, 208, 224,
                                      240, 8, None) == 3


def test_python_glue_error_types():
    from futudiffu_amd import sage_attention as SA
    q = torch.zeros(1, 2, 8, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU tensor"):
        SA.sage_forward(q, q, q)
    with pytest.raises(AssertionError, match="head_dim"):
        x = torch.zeros(1, 2, 8, 96, dtype=torch.bfloat16)
        SA.sage_forward(x, x, x)
    with pytest.raises(AssertionError, match="BF16"):
        x = torch.zeros(1, 2, 8, 64, dtype=torch.float16)
        SA.sage_forward(x, x, x)
    with pytest.raises(ValueError, match="Unknown qk_quant"):
        SA.configure_sage(qk_quant="int4")
    with pytest.raises(ValueError, match="Unknown pv_quant"):
        SA.configure_sage(pv_quant="fp16")
    with pytest.raises(ValueError, match="must share one"):
        SA.sage_forward(q, q[:, :1], q)


def test_custom_op_schemas_and_fake_shapes():
    import futudiffu_amd  # noqa: F401
    from torch._subclasses.fake_tensor import FakeTensorMode
    ops = torch.ops.futudiffu_ii
    assert "block_mask" in str(ops.sage_attn_masked.default._schema)
    with FakeTensorMode():
        q = torch.empty(2, 3, 40, 128, dtype=torch.bfloat16)
        m = torch.empty(1, 1, dtype=torch.uint8)
        out, lse = ops.sage_attn_masked(q, q, q, m, 0.1)
        assert out.shape == (2, 3, 40, 128) and out.dtype == torch.bfloat16
        assert lse.shape == (6, 40) and lse.dtype == torch.float32
        out, lse = ops.sage_attn(q, q, q, 0.1)
        assert out.shape == (2, 3, 40, 128) and lse.shape == (6, 40)
        # [B, N, H*D] output for the out-projection (transformer.py:471)
        out, lse = ops.sage_attn_masked_merged_heads(q, q, q, m, 0.1)
        assert out.shape == (2, 40, 384) and out.dtype == torch.bfloat16 and lse.shape == (6, 40)
        out, lse = ops.sage_attn_ext(q, q, q, None, None, 0.1, "int8", "fp8", "token", True, "bnhd")
        assert out.shape == (2, 40, 384) and lse.shape == (6, 40)
        out, lse = ops.sage_attn_ext(q, q, q, None, None, 0.1, "int8", "fp8", "token", True)
        assert out.shape == (2, 3, 40, 128)
        # producer + attention from the QKV projection output
        qkv = torch.empty(2, 40, 3 * 3 * 128, dtype=torch.bfloat16)
        w = torch.empty(128)
        fr = torch.empty(2, 40, 1, 64, 2, 2)
        out, lse = ops.sage_attn_qkv_masked(qkv, w, w, fr, m, 3, 128, 1e-5, 0.1)
        assert out.shape == (2, 40, 384) and lse.shape == (6, 40)


def test_layout_round_trip():
    from futudiffu_amd import layout
    x = torch.randint(0, 255, (3, 256, 128), dtype=torch.uint8)
    assert torch.equal(layout.unpack_rows(layout.pack_rows(x), 3, 256, 128), x)
    # every index map is a permutation
    for fn in (layout._row_index, layout._v_fp8_index, layout._v_bf16_index):
        idx = fn(256, 64)
        assert torch.equal(idx.sort().values, torch.arange(256 * 64))


def test_doc_id_builders():
    from futudiffu_amd import block_mask as BM
    d = BM.build_doc_ids([3, 2], total_len=7, device="cpu", batch=2)
    assert d.tolist() == [[0, 0, 0, 1, 1, -1, -1]] * 2
    v = torch.tensor([[True, False, True]])
    assert BM.build_key_padding_doc_ids(v).tolist() == [[0, -1, 0]]


def test_legacy_op_schemas_and_fake_shapes():
    """futudiffu::sage_attn / ::sage_attn_masked (sage_attention.py:664-690,
    :740-769) and the module-level names the legacy router imports
    (attention.py:77-79, :101-103)."""
    from futudiffu_amd import sage_attention as SA
    from torch._subclasses.fake_tensor import FakeTensorMode
    ops = torch.ops.futudiffu
    assert str(ops.sage_attn.default._schema) == (
        "futudiffu::sage_attn(Tensor q, Tensor k, Tensor v, float sm_scale) -> (Tensor, Tensor)")
    assert str(ops.sage_attn_masked.default._schema) == (
        "futudiffu::sage_attn_masked(Tensor q, Tensor k, Tensor v, Tensor block_mask, float sm_scale) "
        "-> (Tensor, Tensor)")
    for name in ("sage_attn_op", "sage_attn_masked_op", "sage_attn_forward_masked", "sage_attn_forward"):
        assert callable(getattr(SA, name))
    with FakeTensorMode():
        # a transposed view, as the legacy router passes it (attention.py:69-70)
        q = torch.empty(2, 40, 3, 128, dtype=torch.bfloat16).transpose(1, 2)
        m = torch.empty(1, 1, dtype=torch.uint8)
        for out, lse in (SA.sage_attn_op(q, q, q, 0.1), SA.sage_attn_masked_op(q, q, q, m, 0.1)):
            assert out.shape == (2, 3, 40, 128) and out.is_contiguous() and out.dtype == torch.bfloat16
            assert lse.shape == (6, 40) and lse.dtype == torch.float32


def test_ext_backward_refuses_block_scales():
    """The backward recomputes P from per-token codes, so a forward run with
    per-64-token scales has no consistent gradient: refused before any work."""
    from futudiffu_amd import attention_srcii as A

    class Ctx:
        granularity = "block64"
        saved_tensors = ()
        args = (0.1, "int8", True, "bhnd")

    with pytest.raises(ValueError, match="granularity 'token' only"):
        A._ext_backward(Ctx(), None, None)


@fake_addresses
def test_noalloc_entry_rejects_shapes_beyond_its_scratch():
    """The allocation-free entry point keeps its workspace in a fixed 16 MiB
    device array: 1x32x4480x128 (96 tail items in 4 pieces, 25 MB of
    partials) is refused before any device call; argument checks match
    sage_attn_fwd's."""
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert lib.sage_attn_workspace_bytes(1, 32, 4480, 128) > 16 << 20
    assert lib.sage_attn_workspace_bytes(1, 30, 4416, 128) <= 16 << 20
    # masked launches need the summaries only (the packed 1x30x6912 batch: 7 KB)
    assert lib.sage_attn_masked_workspace_bytes(1, 30, 6912, 128) == 7168
    assert lib.sage_attn_masked_workspace_bytes(1, 32, 4480, 128) <= 16 << 20
    args = [16, 32, 48, 64, 80, 96, 1, 32, 4480, 128, 0, 1, 0, None, 0, 0, 0, None, 112, 0, 128, None]
    assert lib.sage_attn_fwd_noalloc(*args) == 3
    assert "beyond the 16777216-byte scratch" in lib.sage_last_error().decode()
    args[9] = 96
    assert lib.sage_attn_fwd_noalloc(*args) == 1
    assert "head_dim" in lib.sage_last_error().decode()
    args[9], args[6] = 128, 0
    assert lib.sage_attn_fwd_noalloc(*args) == 1
    assert "positive" in lib.sage_last_error().decode()
