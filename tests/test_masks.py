"""Mask and varlen plumbing on the CPU: the oracle's document-id forms pinned
against its segment-based restatement of src_ii/block_mask.py, the host-side
padding helper, and the C-ABI argument checks of the device builders (which
fail before any launch, so no GPU is needed)."""

import random

import pytest
import torch

from oracle import sage_oracle as O


def _layouts(seed, count=40):
    rng = random.Random(seed)
    out = []
    for _ in range(count):
        segs = [rng.choice([rng.randint(1, 400), 32 * rng.randint(1, 40), 64 * rng.randint(1, 20)])
                for _ in range(rng.randint(1, 5))]
        pad = rng.choice([0, 0, rng.randint(1, 300)])
        out.append((segs, sum(segs) + pad))
    return out


@pytest.mark.parametrize("segs,total", _layouts(3))
def test_tile_rule_on_document_ids_matches_segment_rule(segs, total):
    """block_mask.py builds the mask from segments (tokens past the last
    segment are document 0); the device kernel reads per-token ids padded with
    -1 and counts them as 0.  Both must give the same mask."""
    doc = O.packed_document_ids(segs, total)
    assert len(doc) == total and doc.count(-1) == total - sum(segs)
    assert torch.equal(O.tile_mask_from_doc(doc, pad_fill=0), O.build_block_mask(segs, total))


def test_packed_config_mask_known_answer():
    """Packed 1280 + 1216 + 4416 = 6912 tokens: a [54, 108] mask with 2736 of
    5832 tiles on (46.9 %), the figures the packed benchmark configuration is
    quoted with."""
    m = O.tile_mask_from_doc(O.packed_document_ids([1280, 1216, 4416]))
    assert m.shape == (54, 108) and int(m.sum()) == 2736
    # the 64 queries of Q tile 19 (rows 2432..2495 are image 2) follow its first token (image 1)
    assert m[19, 2496 // 64] == 0 and m[19, 1280 // 64] == 1


@pytest.mark.parametrize("seed", range(6))
def test_cu_seqlens_ids_match_packed_ids(seed):
    rng = random.Random(seed)
    segs = [rng.choice([0, rng.randint(1, 300)]) for _ in range(rng.randint(1, 6))]
    start = rng.choice([0, 0, rng.randint(1, 50)])
    cu = [start]
    for s in segs:
        cu.append(cu[-1] + s)
    n = cu[-1] + rng.randint(0, 100)
    got = O.doc_ids_from_cu_seqlens(cu, n)
    # brute force from the definition
    want = [-1] * n
    for s in range(len(segs)):
        for t in range(cu[s], cu[s + 1]):
            want[t] = s
    assert got == want
    if start == 0 and all(segs):
        assert got == O.packed_document_ids(segs, n)


def test_packed_document_ids_overflow_raises():
    with pytest.raises(ValueError):
        O.packed_document_ids([100, 200], 250)


def test_pad_document_ids_mirrors_fixed_length_padding():
    from futudiffu_amd import block_mask as BM
    d = torch.tensor([[0, 0, 1]], dtype=torch.int32)
    assert BM.pad_document_ids(d, 5).tolist() == [[0, 0, 1, -1, -1]]
    assert BM.pad_document_ids(d, 3) is d
    with pytest.raises(ValueError, match="exceeds"):
        BM.pad_document_ids(d, 2)


def test_packing_info_host_path_matches_reference_rule():
    from types import SimpleNamespace

    from futudiffu_amd import block_mask as BM
    segs = [(0, 96, 96, 1184), (1280, 64, 1344, 1152)]  # (text_start, text_len, img_start, img_len)
    info = SimpleNamespace(segments=segs, total_len=4288, document_id=None)
    want = O.build_block_mask([96 + 1184, 64 + 1152], 4288)
    assert torch.equal(BM.build_block_mask_from_packing_info(info, device="cpu"), want)


def test_device_builders_reject_host_tensors():
    from futudiffu_amd import block_mask as BM
    with pytest.raises(ValueError, match="GPU tensor"):
        BM.build_block_mask_device(torch.zeros(10, dtype=torch.int32))
    with pytest.raises(ValueError, match="GPU tensor"):
        BM.doc_ids_from_cu_seqlens(torch.zeros(3, dtype=torch.int32), 10)


@pytest.mark.parametrize("args,msg", [
    ((16, 0, 10, 0, 32, None), "positive"),
    ((16, 1, 0, 0, 32, None), "positive"),
    ((16, 70000, 10, 0, 32, None), "grid limit"),
    ((16, 1, (1 << 24) + 1, 0, 32, None), "2^24"),
    ((None, 1, 10, 0, 32, None), "null"),
    ((16, 1, 10, 0, None, None), "null"),
])
def test_tile_mask_entry_rejects_bad_arguments(args, msg):
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert lib.sage_build_tile_mask(*args) == 1
    assert msg in lib.sage_last_error().decode()


@pytest.mark.parametrize("args,msg", [
    ((16, 1, -1, 10, 32, None), "must not be negative"),
    ((16, 0, 2, 10, 32, None), "positive"),
    ((16, 1, 2, 0, 32, None), "positive"),
    ((None, 1, 2, 10, 32, None), "null"),
    ((16, 1, 2, 10, None, None), "null"),
])
def test_cu_seqlens_entry_rejects_bad_arguments(args, msg):
    from futudiffu_amd import _lib
    lib = _lib.load()
    assert lib.sage_doc_ids_from_cu_seqlens(*args) == 1
    assert msg in lib.sage_last_error().decode()
