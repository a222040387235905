"""GPU parity at the benchmark configurations' full sizes.

Every configuration the benchmark times runs here as one full launch of the
HIP path (all heads, the production schedule: the split tail items and their
merge at 1x30x4416x128, 256 whole and 44 split items at 512x512, the
masked schedules of the packed and k-tuple batches).  Heads taken out of those
launches are compared with the oracle on the same seeded inputs, with the
stated tolerance (max-abs <= 2e-2, cosine >= 0.999 against the emulation of
the reference scheme; LSE within 2e-3 log2 units).  The whole launch is also
checked through properties that hold at any size: finite outputs and LSE for
every row that sees a key, and, for the packed batch with exact document ids
and no smoothing, bit identity with each image run alone.

Smoothing, quantization and the visibility rules are per (batch, head), so the
oracle on the sliced head reproduces exactly what that head of the full launch
computes.
"""


import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu

TOL_MAXABS = 2e-2
TOL_COS = 0.999
LSE_TOL = 2e-3
# vs the emulation of the kernel's own P scheme (see test_gpu_parity.py)
TIGHT_COS = 0.99999
TIGHT_MAXABS = 8e-3

PACKED_SEGMENTS = [1280, 1216, 4416]   # 512x512, 640x384 and 1280x832 images
PACKED_N = sum(PACKED_SEGMENTS)        # 6912


def _sa():
    from futudiffu_amd import sage_attention as SA
    return SA


def _inputs(B, H, N, D, seed):
    return O.make_inputs(B, H, N, D, seed=seed)


def _check_head(out, lse, q, k, v, b, hh, qk, pv, block_mask=None, doc_ids=None, smooth=True):
    """Compare head (b, hh) of a full launch with the oracle on that head."""
    H = q.shape[1]
    sl_b, sl_h = slice(b, b + 1), slice(hh, hh + 1)
    doc1 = None if doc_ids is None else doc_ids[sl_b]
    ref, ref_lse, _ = O.sage_forward(q[sl_b, sl_h], k[sl_b, sl_h], v[sl_b, sl_h], None, qk, pv, "token", smooth,
                                     block_mask, doc1)
    got = out[b, hh].float().cpu()
    got_lse = lse[b * H + hh].cpu()
    ref = ref[0, 0].float()
    ref_lse = ref_lse[0]
    assert torch.isfinite(got).all(), f"head ({b}, {hh}): non-finite output"
    maxabs = (got - ref).abs().max().item()
    cos = O.cosine(got, ref)
    assert maxabs <= TOL_MAXABS, f"head ({b}, {hh}): max-abs {maxabs:.4g} > {TOL_MAXABS}"
    assert cos >= TOL_COS, f"head ({b}, {hh}): cosine {cos:.6f} < {TOL_COS}"
    fin = torch.isfinite(ref_lse)
    assert torch.equal(fin, torch.isfinite(got_lse)), f"head ({b}, {hh}): LSE -inf pattern differs"
    lerr = (got_lse[fin] - ref_lse[fin]).abs().max().item()
    assert lerr <= LSE_TOL, f"head ({b}, {hh}): LSE error {lerr:.3g}"
    if pv == "fp8":  # the kernel follows the reference's per-block P scaling: a tight bound as well
        assert cos >= TIGHT_COS and maxabs <= TIGHT_MAXABS, (
            f"head ({b}, {hh}): cosine {cos:.7f}, max-abs {maxabs:.4g} vs the reference scheme")
    print(f"  head ({b}, {hh}): max-abs {maxabs:.3e} cosine {cos:.7f} lse-err {lerr:.2e}", flush=True)
    return maxabs, cos


def _check_whole_launch(out, lse):
    assert torch.isfinite(out.float()).all(), "non-finite output"
    assert torch.isfinite(lse).all(), "every row of these workloads sees a key: LSE must be finite"


@pytest.mark.parametrize("qk,pv", [("int8", "fp8"), ("fp8", "bf16"), ("int8", "bf16")])
def test_headline_full_launch_matches_oracle(cuda, qk, pv):
    """1x30x4416x128: 1050 items, of which the last 26 (query tiles 9..34 of
    head 29, the 64-row light tile among them) run as 4 key-range pieces each
    and are merged by the second kernel.  Heads 0 and 29 against the oracle."""
    SA = _sa()
    B, H, N, D = 1, 30, 4416, 128
    q, k, v = _inputs(B, H, N, D, seed=5)
    print(f"headline 1x30x4416x128 {qk}/{pv}", flush=True)
    out, lse = SA.sage_forward(q.to(cuda), k.to(cuda), v.to(cuda), qk=qk, pv=pv)
    torch.cuda.synchronize()
    _check_whole_launch(out, lse)
    for hh in (0, 29):
        _check_head(out, lse, q, k, v, 0, hh, qk, pv)


def test_dit512_full_grid_matches_oracle(cuda):
    """512x512: 1x30x1280x128 int8/fp8, 300 items in less than one round:
    256 whole items, the other 44 in four key-tile pieces merged by the last
    of each to finish.  Every head against the oracle."""
    SA = _sa()
    B, H, N, D = 1, 30, 1280, 128
    q, k, v = _inputs(B, H, N, D, seed=21)
    print("dit512 1x30x1280x128 int8/fp8", flush=True)
    out, lse = SA.sage_forward(q.to(cuda), k.to(cuda), v.to(cuda), qk="int8", pv="fp8")
    torch.cuda.synchronize()
    _check_whole_launch(out, lse)
    for hh in range(H):
        _check_head(out, lse, q, k, v, 0, hh, "int8", "fp8")


@pytest.mark.parametrize("pv", ["fp8", "bf16"])
def test_packed_tile_mask_matches_oracle(cuda, pv):
    """Packed 1280 + 1216 + 4416 = 6912 tokens, H=30, the reference tile mask
    (block_mask.py:84-97).  Query tile 19 (rows 2432..2559) straddles images 2
    and 3: by the first-token rule all its rows see image 2's keys, the 64
    rows of image 3 included.  Heads 0 and 17 against the oracle, which
    expands the same mask."""
    from futudiffu_amd import block_mask as BM
    SA = _sa()
    B, H, N, D = 1, 30, PACKED_N, 128
    q, k, v = _inputs(B, H, N, D, seed=33)
    bm = BM.build_block_mask(PACKED_SEGMENTS, N, device="cpu")
    assert int(bm.sum()) == 2736 and bm.shape == (54, 108)
    assert bm[19, 20:39].all() and not bm[19, 39:].any()  # the straddling tile
    print(f"packed 6912 tile mask int8/{pv}", flush=True)
    out, lse = SA.sage_forward(q.to(cuda), k.to(cuda), v.to(cuda), qk="int8", pv=pv, block_mask=bm.to(cuda))
    torch.cuda.synchronize()
    _check_whole_launch(out, lse)
    for hh in (0, 17):
        _check_head(out, lse, q, k, v, 0, hh, "int8", pv, block_mask=bm)


def test_packed_doc_ids_matches_oracle(cuda):
    """The packed batch with exact per-token document ids: every query sees
    exactly its own image's keys (the straddling tile split at token 2496).
    Heads 0 and 29 against the oracle."""
    from futudiffu_amd import block_mask as BM
    SA = _sa()
    B, H, N, D = 1, 30, PACKED_N, 128
    q, k, v = _inputs(B, H, N, D, seed=34)
    doc = BM.build_doc_ids(PACKED_SEGMENTS, N, device="cpu", batch=B)
    print("packed 6912 doc ids int8/fp8", flush=True)
    out, lse = SA.sage_forward(q.to(cuda), k.to(cuda), v.to(cuda), qk="int8", pv="fp8", doc_ids=doc.to(cuda))
    torch.cuda.synchronize()
    _check_whole_launch(out, lse)
    for hh in (0, 29):
        _check_head(out, lse, q, k, v, 0, hh, "int8", "fp8", doc_ids=doc)


def test_packed_doc_ids_equal_serial_images_all_heads(cuda):
    """All 30 heads of the packed batch under exact document ids, without
    smoothing (every code then depends on its own token, or on its own
    64-token V block, and every image boundary is a multiple of 64): bit for
    bit the outputs and LSE of each image run alone.  The images run alone in
    groups of 6 heads (at most 210 items): an unmasked launch of more than 256
    items cuts some items into key-range pieces, whose merge sums in another
    order."""
    from futudiffu_amd import block_mask as BM
    SA = _sa()
    B, H, N, D = 1, 30, PACKED_N, 128
    q, k, v = (t.to(cuda) for t in _inputs(B, H, N, D, seed=35))
    doc = BM.build_doc_ids(PACKED_SEGMENTS, N, device="cpu", batch=B).to(cuda)
    print("packed 6912 doc ids vs serial images, all heads", flush=True)
    out, lse = SA.sage_forward(q, k, v, qk="int8", pv="fp8", doc_ids=doc, smooth_k=False)
    off = 0
    for seg in PACKED_SEGMENTS:
        sl = slice(off, off + seg)
        for h0 in range(0, H, 6):
            hs = slice(h0, h0 + 6)
            o1, l1 = SA.sage_forward(q[:, hs, sl].contiguous(), k[:, hs, sl].contiguous(),
                                     v[:, hs, sl].contiguous(), qk="int8", pv="fp8", smooth_k=False)
            torch.cuda.synchronize()
            got = out[:, hs, sl].contiguous()
            bad = got.view(torch.int16) != o1.view(torch.int16)
            assert not bad.any(), (f"image at {off}, heads {h0}..{h0 + 5}: {int(bad.sum())} outputs differ, "
                                   f"max {(got.float() - o1.float()).abs().max().item():.3g}")
            assert torch.equal(lse[hs, sl].contiguous().view(torch.int32), l1.view(torch.int32)), (
                f"image at {off}, heads {h0}..{h0 + 5}: LSE differs")
        off += seg


def test_ktuple_key_padding_matches_oracle(cuda):
    """k-tuple batch: B=4 samples of 4352 tokens (256 text slots first, then
    4096 image tokens), H=30; sample b keeps L_b ~ U[32, 256] text tokens and
    its text slots [L_b, 256) are padding keys (document id -1): no query
    attends them, and padded queries see every valid key of their sample.
    One head per sample against the oracle."""
    from futudiffu_amd import block_mask as BM
    SA = _sa()
    B, H, N, D = 4, 30, 4352, 128
    q, k, v = _inputs(B, H, N, D, seed=44)
    g = torch.Generator().manual_seed(45)
    lens = torch.randint(32, 257, (B,), generator=g)
    valid = torch.ones(B, N, dtype=torch.bool)
    for b in range(B):
        valid[b, int(lens[b]):256] = False
    doc = BM.build_key_padding_doc_ids(valid)
    print(f"k-tuple 4x30x4352x128 key padding, text lengths {lens.tolist()}", flush=True)
    out, lse = SA.sage_forward(q.to(cuda), k.to(cuda), v.to(cuda), qk="int8", pv="fp8", doc_ids=doc.to(cuda))
    torch.cuda.synchronize()
    _check_whole_launch(out, lse)
    for b, hh in ((0, 0), (1, 7), (2, 15), (3, 29)):
        _check_head(out, lse, q, k, v, b, hh, "int8", "fp8", doc_ids=doc)
