"""sage_attn_fwd_noalloc (the allocation-free entry point) against sage_attn_fwd.

Both are called through the C ABI on the same quantized operands; the
allocation-free one keeps its workspace in the library's fixed device scratch.
Two calls in a row, the second smaller (and with document ids, so the scratch
then holds other data than the first call left there), must each give the
outputs and LSE of sage_attn_fwd bit for bit.  The packed 1x30x6912 batch
(1280 + 1216 + 4416 tokens) runs with its tile mask and with exact document
ids: masked launches need only the summaries, so it fits the scratch although
its unmasked workspace would not.  (A shape whose workspace exceeds the
scratch is rejected before any device call: tests/test_capi.py.)
"""


import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _noalloc(lib, qz, B, H, out, lse, block_mask=None, doc_ids=None, stream=None):
    from futudiffu_amd import sage_attention as SA
    bm, stride_z, nq, nkv = SA._norm_mask(block_mask, B * H, qz.n, qz.q_codes.device)
    return lib.sage_attn_fwd_noalloc(
        qz.q_codes.data_ptr(), qz.q_scale.data_ptr(), qz.k_codes.data_ptr(), qz.k_scale.data_ptr(),
        qz.v_op.data_ptr(), SA._ptr(qz.v_scale), B, H, qz.n, qz.d, SA._QK[qz.qk], SA._PV[qz.pv],
        SA._GRAN[qz.granularity], SA._ptr(bm), stride_z, nq, nkv, SA._ptr(doc_ids), out.data_ptr(), 0,
        lse.data_ptr(), torch.cuda.current_stream().cuda_stream if stream is None else stream)


def _case(cuda, lib, B, H, N, D, seed, pv, doc_segments=None, tile_segments=None):
    from futudiffu_amd import block_mask as BM
    from futudiffu_amd import sage_attention as SA
    masked = doc_segments is not None or tile_segments is not None
    need = (lib.sage_attn_masked_workspace_bytes if masked else lib.sage_attn_workspace_bytes)(B, H, N, D)
    assert need <= SCRATCH_BYTES
    q, k, v = (t.to(cuda) for t in O.make_inputs(B, H, N, D, seed=seed))
    doc = bm = None
    if doc_segments is not None:
        doc = BM.build_doc_ids(doc_segments, N, device="cpu", batch=B).to(cuda)
    if tile_segments is not None:
        bm = O.build_block_mask(tile_segments, N).to(cuda)
    qz = SA.quantize_qkv(q, k, v, qk="int8", pv=pv)
    want, want_lse = SA.attn_from_quantized(qz, B, H, block_mask=bm, doc_ids=doc)
    # fill values that a missing store would leave visible
    out = torch.full((B, H, N, D), float("nan"), dtype=torch.bfloat16, device=cuda)
    lse = torch.full((B * H, N), float("nan"), dtype=torch.float32, device=cuda)
    st = _noalloc(lib, qz, B, H, out, lse, block_mask=bm, doc_ids=doc)
    assert st == 0, lib.sage_last_error().decode()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16)), "outputs differ from sage_attn_fwd"
    assert torch.equal(lse.view(torch.int32), want_lse.view(torch.int32)), "LSE differs from sage_attn_fwd"


def test_noalloc_matches_workspace_entry_two_calls(cuda):
    from futudiffu_amd import _lib
    lib = _lib.load()
    # 1x30x4416x128: 26 tail items cut into 4 pieces, 6.9 MB of partials in scratch
    print("noalloc call 1: 1x30x4416x128 int8/fp8 (split tail in scratch)", flush=True)
    _case(cuda, lib, 1, 30, 4416, 128, seed=71, pv="fp8")
    # smaller, with document ids: the summaries now occupy the scratch's start
    print("noalloc call 2: 1x2x1000x128 int8/bf16 with document ids", flush=True)
    _case(cuda, lib, 1, 2, 1000, 128, seed=72, pv="bf16", doc_segments=[400, 350, 250])


def test_noalloc_packed_batch_masked(cuda):
    from futudiffu_amd import _lib
    lib = _lib.load()
    segs = [1280, 1216, 4416]
    print("noalloc packed 1x30x6912x128 int8/fp8 with document ids", flush=True)
    _case(cuda, lib, 1, 30, 6912, 128, seed=73, pv="fp8", doc_segments=segs)
    print("noalloc packed 1x30x6912x128 int8/fp8 with the tile mask", flush=True)
    _case(cuda, lib, 1, 30, 6912, 128, seed=74, pv="fp8", tile_segments=segs)
