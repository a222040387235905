"""Committed golden fixtures (tests/golden/*.npz, written by make_golden.py).

CPU: the oracle reproduces every fixture bit for bit (codes, scales, K mean,
int32 QK^T rows, output bits, LSE bits), so any change to the oracle's
arithmetic shows up here.
GPU: the HIP path, called on the fixture inputs, reproduces the integer work
bit for bit and the outputs within the stated tolerance, without running the
oracle.
"""

import glob
import math
import os

import numpy as np
import pytest
import torch

from oracle import sage_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURES = sorted(glob.glob(os.path.join(HERE, "golden", "*.npz")))
IDS = [os.path.basename(p)[:-4] for p in FIXTURES]

TOL_MAXABS = 2e-2
TOL_COS = 0.999
LSE_TOL = 2e-3


def _load(path):
    fx = np.load(path, allow_pickle=False)
    B, H, N, D = (int(x) for x in fx["shape"])
    q, k, v = (torch.from_numpy(fx[n].astype(np.int16)).view(torch.bfloat16).reshape(B, H, N, D)
               for n in ("q", "k", "v"))
    mask = torch.from_numpy(fx["block_mask"]) if "block_mask" in fx else None
    doc = torch.from_numpy(fx["doc_ids"]) if "doc_ids" in fx else None
    return fx, (B, H, N, D), q, k, v, mask, doc


def _u(t):
    t = t.contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def test_fixtures_present():
    assert len(FIXTURES) >= 7


@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_oracle_reproduces_fixture(path):
    fx, (B, H, N, D), q, k, v, mask, doc = _load(path)
    qk, pv, gran = str(fx["qk"]), str(fx["pv"]), str(fx["granularity"])
    out, lse, qz = O.sage_forward(q, k, v, float(fx["sm_scale"]), qk, pv, gran, True, mask, doc)
    assert np.array_equal(_u(qz.mu), fx["k_mean"])
    for name, t in (("q_codes", qz.qc), ("k_codes", qz.kc), ("q_scale", qz.qs), ("k_scale", qz.ks)):
        assert np.array_equal(_u(t).view(np.uint8), fx[name].view(np.uint8)), name
    if pv == "fp8":
        assert np.array_equal(_u(qz.vc), fx["v_codes"])
        assert np.array_equal(_u(qz.vs).view(np.uint32), fx["v_scale"].view(np.uint32))
    rows = fx["qk_rows"].shape[1]
    acc = O.qk_int32(qz.qc[:, :rows], qz.kc) if qk == "int8" else O.qk_fp8(qz.qc[:, :rows], qz.kc).float()
    assert np.array_equal(acc.numpy(), fx["qk_rows"])
    assert np.array_equal(_u(out), fx["out"])
    assert np.array_equal(_u(lse).view(np.uint32), fx["lse"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=IDS)
def test_hip_matches_fixture(cuda, path):
    from futudiffu_amd import layout
    from futudiffu_amd import sage_attention as SA
    fx, (B, H, N, D), q, k, v, mask, doc = _load(path)
    qk, pv, gran = str(fx["qk"]), str(fx["pv"]), str(fx["granularity"])
    print(f"fixture {os.path.basename(path)} B={B} H={H} N={N} D={D} {qk}/{pv}/{gran}", flush=True)
    qz = SA.quantize_qkv(q.to(cuda), k.to(cuda), v.to(cuda), float(fx["sm_scale"]), qk=qk, pv=pv,
                         granularity=gran)
    out, lse = SA.attn_from_quantized(qz, B, H, block_mask=None if mask is None else mask.to(cuda),
                                      doc_ids=None if doc is None else doc.to(cuda))
    torch.cuda.synchronize()
    BH, Np = B * H, qz.np_
    assert np.array_equal(qz.k_mean.cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1),
                          fx["k_mean"].reshape(-1))
    for name, t in (("q_codes", qz.q_codes), ("k_codes", qz.k_codes)):
        rows = layout.unpack_rows(t.cpu(), BH, Np, D)[:, :N].numpy()
        assert np.array_equal(rows, fx[name].view(np.uint8)), name
    nsc = N if gran == "token" else (N + 63) // 64
    for name, t in (("q_scale", qz.q_scale), ("k_scale", qz.k_scale)):
        assert np.array_equal(t[:, :nsc].cpu().numpy().view(np.uint32), fx[name].view(np.uint32)), name
    if pv == "fp8":
        vrows = layout.unpack_v_fp8(qz.v_op.cpu(), BH, Np, D)[:, :N].numpy()
        assert np.array_equal(vrows, fx["v_codes"])
        assert np.array_equal(qz.v_scale[:, :(N + 63) // 64].cpu().numpy().view(np.uint32),
                              fx["v_scale"].view(np.uint32))
    if qk == "int8":
        s = SA.qk_accumulators(qz, B, H)[2].cpu()
        rows = fx["qk_rows"].shape[1]
        assert np.array_equal(s[:, :rows, :N].numpy(), fx["qk_rows"])
    ref = torch.from_numpy(fx["out"].astype(np.int16)).view(torch.bfloat16).reshape(B, H, N, D).float()
    got = out.float().cpu()
    maxabs = (got - ref).abs().max().item()
    cos = O.cosine(got, ref)
    assert maxabs <= TOL_MAXABS and cos >= TOL_COS, f"max-abs {maxabs:.4g}, cosine {cos:.6f}"
    rl = torch.from_numpy(fx["lse"])
    fin = torch.isfinite(rl)
    assert torch.equal(fin, torch.isfinite(lse.cpu()))
    if fin.any():
        assert (lse.cpu()[fin] - rl[fin]).abs().max().item() <= LSE_TOL
