"""ctypes binding of libsage_mi355x.so (the C ABI in include/sage_mi355x.h).

The library is built in-tree by ``futudiffu_amd/build.py``.  There is no
fallback: if the library is missing, or no GPU is visible, every compute entry
point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

# SAGE_MI355X_LIB selects another build of the same library (the measurement
# build, futudiffu_amd/build.py --phase-timing)
LIB_PATH = os.environ.get("SAGE_MI355X_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                             "libsage_mi355x.so")

# Every symbol include/sage_mi355x.h declares, with its ctypes signature.
_c = ctypes
_P = _c.c_void_p
_I64 = _c.c_int64
SIGNATURES = {
    "sage_abi_version": (_c.c_int, []),
    "sage_last_error": (_c.c_char_p, []),
    "sage_padded_len": (_I64, [_I64]),
    "sage_quant_workspace_bytes": (_c.c_size_t, [_I64, _I64, _I64]),
    "sage_quantize_qkv": (_c.c_int, [
        _P, _P, _P, _I64, _I64, _I64, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_float,
        _P, _P, _P, _P, _P, _P, _P, _P, _c.c_size_t, _P]),
    "sage_attn_workspace_bytes": (_c.c_size_t, [_I64, _I64, _I64, _I64]),
    "sage_attn_masked_workspace_bytes": (_c.c_size_t, [_I64, _I64, _I64, _I64]),
    "sage_attn_fwd": (_c.c_int, [
        _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_int, _c.c_int, _c.c_int,
        _P, _I64, _I64, _I64, _P, _P, _c.c_size_t, _P, _c.c_int, _P, _P]),
    "sage_attn_fwd_noalloc": (_c.c_int, [
        _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_int, _c.c_int, _c.c_int,
        _P, _I64, _I64, _I64, _P, _P, _c.c_int, _P, _P]),
    "sage_attn_qk_accumulators": (_c.c_int, [
        _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_int, _c.c_int, _P, _c.c_size_t, _P, _P, _P, _P]),
    "sage_build_tile_mask": (_c.c_int, [_P, _I64, _I64, _c.c_int32, _P, _P]),
    "sage_qkv_postprocess": (_c.c_int, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_float, _P, _P, _P, _P]),
    "sage_qkv_postprocess_bwd": (_c.c_int, [
        _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_float, _P, _P]),
    "sage_quantize_from_qkv": (_c.c_int, [
        _P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_float, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_float,
        _P, _P, _P, _P, _P, _P, _P, _P, _c.c_size_t, _P]),
    "sage_doc_ids_from_cu_seqlens": (_c.c_int, [_P, _I64, _I64, _I64, _P, _P]),
    "sage_attn_bwd_workspace_bytes": (_c.c_size_t, [_I64, _I64, _I64, _I64]),
    "sage_attn_bwd": (_c.c_int, [
        _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _c.c_int, _c.c_int, _c.c_float, _c.c_float,
        _P, _I64, _I64, _I64, _P, _P, _c.c_size_t, _P, _P, _P, _P]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load the library and attach prototypes (no GPU needed)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python futudiffu_amd/build.py` "
                    "(or __graft_entry__.build()) first")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.sage_abi_version() != 6:
                raise RuntimeError("libsage_mi355x.so ABI version mismatch")
            _lib = lib
        return _lib


class SageError(RuntimeError):
    """Non-zero status from the C ABI."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"sage status {status}: {msg}")
        self.status = status


def check(status: int) -> None:
    if status != 0:
        msg = load().sage_last_error().decode(errors="replace")
        if status == 1:
            raise ValueError(msg)
        raise SageError(status, msg)
