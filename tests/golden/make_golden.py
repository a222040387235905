"""Writes the committed golden fixtures of the Sage forward path.

The reference holds no golden vectors for this path and its Triton kernels
cannot run here, so the fixtures are produced by the CPU oracle
(oracle/sage_oracle.py, itself pinned by tests/test_oracle.py) and freeze its
results: inputs, K mean, Q/K/V codes and scales, int32 QK^T rows, outputs and
LSE.  Run from the repository root:

    python tests/golden/make_golden.py

Each case is one .npz (bf16 and fp8 stored as their bit patterns).
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import sage_oracle as O  # noqa: E402

# name: (B, H, N, D, qk, pv, granularity, mask kind)
CASES = {
    # CPU plumbing config: int8 QK with per-64-token block scales, bf16 PV, no mask
    "cfg1_int8_bf16_block64": (1, 4, 256, 64, "int8", "bf16", "block64", None),
    "cfg1_int8_bf16_token": (1, 2, 256, 64, "int8", "bf16", "token", None),
    "ragged_fp8_fp8_token": (1, 2, 77, 64, "fp8", "fp8", "token", None),
    "single_token_int8_fp8": (1, 1, 1, 128, "int8", "fp8", "token", None),
    "ragged_int8_fp8_d128": (1, 1, 130, 128, "int8", "fp8", "token", None),
    # two packed segments with the reference tile mask (second Q tile straddles)
    "packed_tilemask_int8_bf16": (1, 1, 320, 64, "int8", "bf16", "token", "tile"),
    # per-token doc ids: two batches, key padding in the middle and at the end
    "docids_int8_fp8": (2, 1, 200, 64, "int8", "fp8", "token", "doc"),
}

PACKED_SEGMENTS = [96, 160, 64]


def doc_ids_case(b: int, n: int) -> torch.Tensor:
    doc = torch.zeros(b, n, dtype=torch.int32)
    doc[0, 90:120] = -1          # padding keys mid-sequence
    doc[0, 120:] = 1
    doc[1, :150] = 0
    doc[1, 150:] = -1           # trailing padding
    return doc


def bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def make_case(name: str) -> dict:
    B, H, N, D, qk, pv, gran, mask = CASES[name]
    seed = sum(map(ord, name)) % 10007
    q, k, v = O.make_inputs(B, H, N, D, seed=seed)
    block_mask = O.build_block_mask(PACKED_SEGMENTS, N) if mask == "tile" else None
    doc_ids = doc_ids_case(B, N) if mask == "doc" else None
    sm = 1.0 / math.sqrt(D)
    out, lse, qz = O.sage_forward(q, k, v, sm, qk, pv, gran, True, block_mask, doc_ids)
    rows = min(N, 32)
    acc = O.qk_int32(qz.qc[:, :rows], qz.kc) if qk == "int8" else \
        O.qk_fp8(qz.qc[:, :rows], qz.kc).float()
    d = {
        "shape": np.array([B, H, N, D]), "qk": qk, "pv": pv, "granularity": gran,
        "sm_scale": np.float64(sm), "seed": seed,
        "q": bits(q), "k": bits(k), "v": bits(v),
        "k_mean": bits(qz.mu), "q_codes": bits(qz.qc), "q_scale": bits(qz.qs),
        "k_codes": bits(qz.kc), "k_scale": bits(qz.ks),
        "qk_rows": acc.numpy(), "out": bits(out), "lse": bits(lse),
    }
    if pv == "fp8":
        d["v_codes"] = bits(qz.vc)
        d["v_scale"] = bits(qz.vs)
    if block_mask is not None:
        d["block_mask"] = block_mask.numpy()
    if doc_ids is not None:
        d["doc_ids"] = doc_ids.numpy()
    return d


def load_inputs(fx) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, H, N, D = (int(x) for x in fx["shape"])
    return tuple(torch.from_numpy(fx[n].astype(np.int16)).view(torch.bfloat16).reshape(B, H, N, D)
                 for n in ("q", "k", "v"))


def main() -> None:
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    for name in CASES:
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **make_case(name))
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
