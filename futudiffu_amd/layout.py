"""Index maps of the MFMA-fragment storage orders used by libsage_mi355x.

The quantize kernel writes Q/K codes and V operands in the order the gfx950
attention kernel's MFMA operands consume them (see include/sage_mi355x.h).
These helpers turn that storage back into plain ``[BH, Np, D]`` tensors, for
inspection and for the bit-exact parity tests.
"""

from __future__ import annotations

import functools

import torch


def padded_len(n: int) -> int:
    return (n + 127) // 128 * 128


@functools.lru_cache(maxsize=32)
def _row_index(np_: int, d: int) -> torch.Tensor:
    tok = torch.arange(np_)[:, None]
    ch = torch.arange(d)[None, :]
    rb, r = tok // 32, tok % 32
    c, h, t = ch // 32, (ch // 16) % 2, ch % 16
    return (((rb * (d // 32) + c) * 64 + h * 32 + r) * 16 + t).reshape(-1)


@functools.lru_cache(maxsize=32)
def _v_fp8_index(np_: int, d: int) -> torch.Tensor:
    key = torch.arange(np_)[:, None]
    ch = torch.arange(d)[None, :]
    t, kk = key // 64, key % 64
    b, rem = kk // 32, kk % 32
    jj, hh, i = rem // 8, (rem % 8) // 4, rem % 4
    j, r = ch // 32, ch % 32
    return (((((t * (d // 32) + j) * 2 + b) * 64 + hh * 32 + r) * 16) + 4 * jj + i).reshape(-1)


@functools.lru_cache(maxsize=32)
def _v_bf16_index(np_: int, d: int) -> torch.Tensor:
    key = torch.arange(np_)[:, None]
    ch = torch.arange(d)[None, :]
    t, kk = key // 64, key % 64
    b, rem = kk // 32, kk % 32
    tt, rem2 = rem // 16, rem % 16
    jj, hh, i = rem2 // 8, (rem2 % 8) // 4, rem2 % 4
    j, r = ch // 32, ch % 32
    return ((((((t * (d // 32) + j) * 2 + b) * 2 + tt) * 64 + hh * 32 + r) * 8) + 4 * jj + i).reshape(-1)


def unpack_rows(codes: torch.Tensor, bh: int, np_: int, d: int) -> torch.Tensor:
    """Row-fragment Q/K codes (uint8 view, ``bh*np*d`` bytes) -> ``[bh, np, d]`` uint8."""
    flat = codes.reshape(bh, np_ * d)
    idx = _row_index(np_, d).to(flat.device)
    return flat[:, idx].reshape(bh, np_, d)


def unpack_v_fp8(vcodes: torch.Tensor, bh: int, np_: int, d: int) -> torch.Tensor:
    flat = vcodes.reshape(bh, np_ * d)
    idx = _v_fp8_index(np_, d).to(flat.device)
    return flat[:, idx].reshape(bh, np_, d)


def unpack_v_bf16(vfrag: torch.Tensor, bh: int, np_: int, d: int) -> torch.Tensor:
    flat = vfrag.reshape(bh, np_ * d)
    idx = _v_bf16_index(np_, d).to(flat.device)
    return flat[:, idx].reshape(bh, np_, d)


def pack_rows(x: torch.Tensor) -> torch.Tensor:
    """Inverse of unpack_rows: ``[bh, np, d]`` -> fragment order (same dtype)."""
    bh, np_, d = x.shape
    out = torch.empty(bh, np_ * d, dtype=x.dtype, device=x.device)
    out[:, _row_index(np_, d).to(x.device)] = x.reshape(bh, -1)
    return out
