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

On-device forms (HIP kernels of ``libsage_mi355x.so``, no host loop and no
host synchronization, so they can run inside captured graphs):

* :func:`build_block_mask_device` - the reference tile rule evaluated on
  device document ids (padding ids count as document 0, like tokens past the
  last segment in block_mask.py:75-79).
* :func:`doc_ids_from_cu_seqlens` - exact ids from varlen segment offsets.
* :func:`pad_document_ids` - ``_pad_plan_to_fixed_len``'s document-id padding
  (forward_packed.py:27-73).
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
    """Tile mask from a PackingInfo (block_mask.py:102-129).

    When the plan carries its per-token ``document_id`` on a GPU (as
    build_packed_sequence and _pad_plan_to_fixed_len leave it,
    transformer.py:152, forward_packed.py:56-62), the mask is built there by
    the device kernel; otherwise from ``segments``/``total_len`` on the host.
    Both give the reference mask.
    """
    doc = getattr(packing_info, "document_id", None)
    if (isinstance(doc, torch.Tensor) and doc.is_cuda and doc.ndim == 1
            and doc.numel() == packing_info.total_len and torch.device(device).type == "cuda"):
        return build_block_mask_device(doc.to(torch.device(device)))
    segment_lengths = [text_len + img_len for (_ts, text_len, _is, img_len) in packing_info.segments]
    return build_block_mask(segment_lengths, total_len=packing_info.total_len, device=device)


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _device_int32(t: torch.Tensor, name: str) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != torch.int32:
        raise ValueError(f"{name} must be int32, got {t.dtype}")
    return t.contiguous()


def build_block_mask_device(doc_ids: torch.Tensor, pad_fill: int = 0) -> torch.Tensor:
    """Reference tile mask from device document ids (block_mask.py:84-97).

    ``doc_ids`` is int32 ``[N]`` or ``[B, N]`` on a GPU.  Returns uint8
    ``[ceil(N/128), ceil(N/64)]`` for 1D input (the 2D reference mask) or
    ``[B, ceil(N/128), ceil(N/64)]``; expand the latter with
    :func:`mask_per_head` for the ``[B*H, nq, nkv]`` form the op takes.
    Ids below zero count as ``pad_fill``.
    """
    from . import _lib
    doc = _device_int32(doc_ids, "doc_ids")
    if doc.ndim not in (1, 2):
        raise ValueError(f"doc_ids must be [N] or [B, N], got {tuple(doc.shape)}")
    b, n = (1, doc.shape[0]) if doc.ndim == 1 else doc.shape
    nq, nkv = _ceildiv(n, BLOCK_M), _ceildiv(n, BLOCK_N)
    mask = torch.empty(b, nq, nkv, dtype=torch.uint8, device=doc.device)
    lib = _lib.load()
    _lib.check(lib.sage_build_tile_mask(doc.data_ptr(), b, n, int(pad_fill), mask.data_ptr(), _stream(doc)))
    return mask[0] if doc.ndim == 1 else mask


def mask_per_head(mask: torch.Tensor, heads: int) -> torch.Tensor:
    """``[B, nq, nkv]`` per-sample tile masks -> the op's ``[B*H, nq, nkv]`` form
    (sage_attention.py:512-519: row z belongs to sample z // H)."""
    if mask.ndim != 3:
        raise ValueError(f"expected a [B, nq, nkv] mask, got {tuple(mask.shape)}")
    return mask.repeat_interleave(heads, dim=0)


def doc_ids_from_cu_seqlens(cu_seqlens: torch.Tensor, total_len: int) -> torch.Tensor:
    """Exact per-token document ids ``[B, total_len]`` int32 from varlen segment
    offsets ``[S+1]`` or ``[B, S+1]`` (int32, nondecreasing, on a GPU): token t
    of sample b gets the segment s with ``cu[b, s] <= t < cu[b, s+1]``, or -1."""
    from . import _lib
    cu = _device_int32(cu_seqlens, "cu_seqlens")
    if cu.ndim == 1:
        cu = cu.unsqueeze(0)
    if cu.ndim != 2 or cu.shape[1] < 1:
        raise ValueError(f"cu_seqlens must be [S+1] or [B, S+1], got {tuple(cu_seqlens.shape)}")
    b, nseg = cu.shape[0], cu.shape[1] - 1
    doc = torch.empty(b, total_len, dtype=torch.int32, device=cu.device)
    lib = _lib.load()
    _lib.check(lib.sage_doc_ids_from_cu_seqlens(cu.data_ptr(), b, nseg, total_len, doc.data_ptr(), _stream(cu)))
    return doc


def pad_document_ids(document_id: torch.Tensor, target_len: int) -> torch.Tensor:
    """Pad per-token ids (last dimension) to ``target_len`` with -1, as
    _pad_plan_to_fixed_len does for a packed plan (forward_packed.py:46-62);
    a longer plan raises ValueError like the reference."""
    n = document_id.shape[-1]
    if n > target_len:
        raise ValueError(f"Packed sequence length {n} exceeds REFERENCE_TOTAL_LEN {target_len}. "
                         "Content doesn't fit.")
    if n == target_len:
        return document_id
    return torch.nn.functional.pad(document_id, (0, target_len - n), value=-1)


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
