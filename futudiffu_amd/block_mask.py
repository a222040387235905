"""uint8 block masks and document ids for packed multi-image sequences.

Mirrors ``src_ii/block_mask.py`` of sqcu/futudiffu (tile sizes BLOCK_M=128
query rows, BLOCK_N=64 keys, block_mask.py:27-28) and adds the exact
per-token form the MI355X kernel can also consume.

* :func:`build_block_mask` - reference semantics (block_mask.py:35-99): each
  tile takes the document id of its first token, tokens past the last segment
  keep id 0, and tile starts are clamped to ``N-1``.  Tiles that straddle a
  segment boundary therefore follow their first token.
* :func:`build_doc_ids` - exact per-token ids ``[B, N]`` int32 (-1 marks
  padding) for ``sage_forward(..., doc_ids=...)``: key n is visible to query
  m iff ``doc[n] >= 0`` and (``doc[m] == doc[n]`` or ``doc[m] < 0``).
"""

from __future__ import annotations

import torch

BLOCK_M: int = 128
BLOCK_N: int = 64


def _ceildiv(a: int, b: int) -> int:
    return (a + b - 1) // b


def _segment_doc_ids(segment_lengths: list[int], total_len: int, fill: int, device) -> torch.Tensor:
    doc = torch.full((total_len,), fill, dtype=torch.int32, device=device)
    off = 0
    for idx, seg in enumerate(segment_lengths):
        doc[off:off + seg] = idx
        off += seg
    return doc


def build_block_mask(segment_lengths: list[int], total_len: int | None = None,
                     device: torch.device | str = "cuda") -> torch.Tensor:
    """uint8 ``[ceil(N/128), ceil(N/64)]`` tile mask (block_mask.py:35-99)."""
    if total_len is None:
        total_len = sum(segment_lengths)
    n_q_blocks = _ceildiv(total_len, BLOCK_M)
    n_kv_blocks = _ceildiv(total_len, BLOCK_N)
    doc = _segment_doc_ids(segment_lengths, total_len, 0, device)
    q_starts = (torch.arange(n_q_blocks, device=device) * BLOCK_M).clamp(max=total_len - 1)
    kv_starts = (torch.arange(n_kv_blocks, device=device) * BLOCK_N).clamp(max=total_len - 1)
    return (doc[q_starts].unsqueeze(1) == doc[kv_starts].unsqueeze(0)).to(torch.uint8)


def build_block_mask_from_packing_info(packing_info, device: torch.device | str = "cuda") -> torch.Tensor:
    """Tile mask from a PackingInfo's ``segments``/``total_len`` (block_mask.py:102-129)."""
    segment_lengths = [text_len + img_len for (_ts, text_len, _is, img_len) in packing_info.segments]
    return build_block_mask(segment_lengths, total_len=packing_info.total_len, device=device)


def build_doc_ids(segment_lengths: list[int], total_len: int | None = None,
                  device: torch.device | str = "cuda", batch: int = 1) -> torch.Tensor:
    """Exact per-token document ids ``[batch, N]`` int32; tokens past the last
    segment are padding (-1)."""
    if total_len is None:
        total_len = sum(segment_lengths)
    doc = _segment_doc_ids(segment_lengths, total_len, -1, device)
    return doc.unsqueeze(0).expand(batch, -1).contiguous()


def build_key_padding_doc_ids(valid: torch.Tensor) -> torch.Tensor:
    """Doc ids ``[B, N]`` from a boolean validity mask: valid -> 0, padding -> -1."""
    return torch.where(valid, 0, -1).to(torch.int32)
