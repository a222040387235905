"""GPU: the device mask builders against the oracle (bit-exact), and the
packed plumbing end to end: a mask built on the device drives the attention
exactly like the host-built one, and exact document ids make a packed batch
equal to running each image alone."""

import math
import random

import pytest
import torch

from oracle import sage_oracle as O

pytestmark = pytest.mark.gpu


def _segments(rng, n_min=200):
    segs = [rng.choice([rng.randint(1, 700), 32 * rng.randint(1, 40), 64 * rng.randint(1, 20)])
            for _ in range(rng.randint(1, 5))]
    while sum(segs) < n_min:
        segs.append(rng.randint(1, 300))
    return segs


@pytest.mark.parametrize("seed", range(4))
def test_device_tile_mask_matches_oracle(cuda, seed):
    from futudiffu_amd import block_mask as BM
    rng = random.Random(100 + seed)
    rows, want = [], []
    for _ in range(3):
        segs = _segments(rng)
        total = sum(segs) + rng.choice([0, rng.randint(1, 200)])
        rows.append((segs, total))
    n = max(t for _, t in rows)
    docs = []
    for segs, total in rows:
        doc = O.packed_document_ids(segs, total) + [-1] * (n - total)
        docs.append(doc)
        want.append(O.tile_mask_from_doc(doc, pad_fill=0))
    print(f"tile mask seed={seed} n={n}", flush=True)
    d = torch.tensor(docs, dtype=torch.int32, device=cuda)
    got = BM.build_block_mask_device(d)
    one = BM.build_block_mask_device(d[0].contiguous())
    fill = BM.build_block_mask_device(d, pad_fill=7)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), torch.stack(want))
    assert torch.equal(one.cpu(), want[0])
    assert torch.equal(fill.cpu(), torch.stack([O.tile_mask_from_doc(x, pad_fill=7) for x in docs]))


@pytest.mark.parametrize("seed", range(4))
def test_device_doc_ids_from_cu_seqlens_match_oracle(cuda, seed):
    from futudiffu_amd import block_mask as BM
    rng = random.Random(200 + seed)
    nseg = rng.randint(1, 7)
    cus = []
    for _ in range(2):
        cu = [rng.choice([0, 0, rng.randint(1, 40)])]
        for _ in range(nseg):
            cu.append(cu[-1] + rng.choice([0, rng.randint(1, 500)]))
        cus.append(cu)
    n = max(c[-1] for c in cus) + rng.randint(0, 90)
    print(f"cu_seqlens seed={seed} n={n} segments={nseg}", flush=True)
    got = BM.doc_ids_from_cu_seqlens(torch.tensor(cus, dtype=torch.int32, device=cuda), n)
    one = BM.doc_ids_from_cu_seqlens(torch.tensor(cus[0], dtype=torch.int32, device=cuda), n)
    torch.cuda.synchronize()
    assert got.cpu().tolist() == [O.doc_ids_from_cu_seqlens(c, n) for c in cus]
    assert one.cpu().tolist() == [O.doc_ids_from_cu_seqlens(cus[0], n)]


def test_packing_info_device_mask_drives_attention_like_host_mask(cuda):
    """A padded packed plan (two images in 4288 tokens): the mask built on the
    device from document_id equals the host-built reference mask, so the
    attention outputs are bit-identical."""
    from types import SimpleNamespace

    from futudiffu_amd import block_mask as BM
    from futudiffu_amd import sage_attention as SA
    segs = [(0, 96, 96, 1184), (1280, 64, 1344, 1152)]
    lens = [96 + 1184, 64 + 1152]
    doc = torch.tensor(O.packed_document_ids(lens, 4288), dtype=torch.int32, device=cuda)
    info = SimpleNamespace(segments=segs, total_len=4288, document_id=doc)
    dev_mask = BM.build_block_mask_from_packing_info(info, device=cuda)
    host_mask = BM.build_block_mask(lens, 4288, device="cpu")
    assert torch.equal(dev_mask.cpu(), host_mask)
    B, H, N, D = 1, 2, 4288, 128
    q, k, v = (t.to(cuda) for t in O.make_inputs(B, H, N, D, seed=71))
    a, la = SA.sage_attn_forward_masked_with_lse(q, k, v, dev_mask, 1.0 / math.sqrt(D))
    b, lb = SA.sage_attn_forward_masked_with_lse(q, k, v, host_mask.to(cuda), 1.0 / math.sqrt(D))
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)) and torch.equal(la, lb)


@pytest.mark.parametrize("qk,pv", [("int8", "fp8"), ("fp8", "bf16"), ("int8", "bf16"), ("fp8", "fp8")])
def test_packed_exact_ids_equal_serial_images(cuda, qk, pv):
    """Three images of 64-aligned lengths packed into one sequence (plus 64
    padding tokens), masked by exact ids from device cu_seqlens.  Without K
    smoothing every code depends only on its own token (V scales on its own
    64-token block), and each image's rows see exactly its own key tiles in
    the same order, so the packed rows equal each image run alone, bit for
    bit, outputs and LSE."""
    from futudiffu_amd import block_mask as BM
    from futudiffu_amd import sage_attention as SA
    lens = [640, 1216, 1152]
    n = sum(lens) + 64
    B, H, D = 1, 2, 128
    q, k, v = (t.to(cuda) for t in O.make_inputs(B, H, n, D, seed=73))
    cu = torch.tensor([0, 640, 1856, 3008], dtype=torch.int32, device=cuda)
    doc = BM.doc_ids_from_cu_seqlens(cu, n)
    print(f"packed vs serial {qk}/{pv} lens={lens}", flush=True)
    out, lse = SA.sage_forward(q, k, v, qk=qk, pv=pv, smooth_k=False, doc_ids=doc)
    off = 0
    for s in lens:
        sl = slice(off, off + s)
        o1, l1 = SA.sage_forward(q[:, :, sl].contiguous(), k[:, :, sl].contiguous(), v[:, :, sl].contiguous(),
                                 qk=qk, pv=pv, smooth_k=False)
        torch.cuda.synchronize()
        got = out[:, :, sl].contiguous()
        bad = got.view(torch.int16) != o1.view(torch.int16)
        assert not bad.any(), (f"segment at {off}: {int(bad.sum())} outputs differ, "
                               f"max {(got.float() - o1.float()).abs().max().item():.3g}")
        assert torch.equal(lse.view(B * H, n)[:, sl].cpu(), l1.cpu()), f"segment at {off}: LSE differs"
        off += s


@pytest.mark.parametrize("qk,pv", [("int8", "fp8"), ("int8", "bf16"), ("fp8", "fp8")])
def test_packed_tile_mask_equal_serial_images(cuda, qk, pv):
    """Three images of 128-aligned lengths packed into one sequence, masked by
    the reference tile mask built on the device from their document ids; for
    aligned images that mask is exactly block diagonal.  Without K smoothing
    each image's rows see exactly their own key tiles, in the order of the
    image run alone, so outputs and LSE equal the serial runs bit for bit.
    The tile-mask loop starts its int8 score chains from zero like the
    unmasked one; the exact-id test above pins the document-id loop, which
    starts them from c0, to the same scores."""
    from futudiffu_amd import block_mask as BM
    from futudiffu_amd import sage_attention as SA
    lens = [640, 1152, 1280]
    n = sum(lens)
    B, H, D = 1, 2, 128
    q, k, v = (t.to(cuda) for t in O.make_inputs(B, H, n, D, seed=79))
    doc = torch.tensor(O.packed_document_ids(lens, n), dtype=torch.int32, device=cuda)
    mask = BM.build_block_mask_device(doc)
    print(f"packed tile mask vs serial {qk}/{pv} lens={lens}", flush=True)
    out, lse = SA.sage_forward(q, k, v, qk=qk, pv=pv, smooth_k=False, block_mask=mask)
    off = 0
    for s in lens:
        sl = slice(off, off + s)
        o1, l1 = SA.sage_forward(q[:, :, sl].contiguous(), k[:, :, sl].contiguous(), v[:, :, sl].contiguous(),
                                 qk=qk, pv=pv, smooth_k=False)
        torch.cuda.synchronize()
        got = out[:, :, sl].contiguous()
        bad = got.view(torch.int16) != o1.view(torch.int16)
        assert not bad.any(), (f"segment at {off}: {int(bad.sum())} outputs differ, "
                               f"max {(got.float() - o1.float()).abs().max().item():.3g}")
        assert torch.equal(lse.view(B * H, n)[:, sl].cpu(), l1.cpu()), f"segment at {off}: LSE differs"
        off += s
