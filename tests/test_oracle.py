"""Pins for the CPU oracle (oracle/sage_oracle.py), no GPU needed.

The reference holds no golden vectors or known-answer tests for this path
(its only attention checks are cosine thresholds on CUDA, e.g.
src/futudiffu/test_sage_backward.py:37, :93, :156), and its Triton kernels
cannot run here.  Every oracle function is therefore pinned by something the
mathematics fixes: the byte formats' definitions (re-derived independently in
oracle/np_codes.py), closed forms and special cases, invariants, and
brute force on tiny inputs.  Each check is chosen so that a plausible slip
(a dropped term, a wrong sign or index, a transposed operand, a wrong
rounding mode) fails it.
"""

import math
import random

import numpy as np
import pytest
import torch

from oracle import np_codes as NC
from oracle import sage_oracle as O

F8 = torch.float8_e4m3fn


# ---------------------------------------------------------------------------
# byte formats
# ---------------------------------------------------------------------------

def test_e4m3_table_matches_definition():
    table = NC.e4m3_decode_table()
    torch_vals = torch.arange(256, dtype=torch.uint8).view(F8).double().numpy()
    assert np.array_equal(np.isnan(table), np.isnan(torch_vals))
    fin = ~np.isnan(table)
    assert np.array_equal(table[fin], torch_vals[fin])
    # spot values fixed by the format: 1.0, max 448, min normal 2^-6, min subnormal 2^-9
    assert table[0x38] == 1.0 and table[0x7E] == 448.0 and table[0xFE] == -448.0
    assert table[0x08] == 2.0 ** -6 and table[0x01] == 2.0 ** -9
    assert np.isnan(table[0x7F]) and np.isnan(table[0xFF])
    assert int(fin.sum()) == 254


def _e4m3_probe_values():
    table = NC.e4m3_decode_table()
    pos = np.sort(table[(~np.isnan(table)) & (table >= 0)])
    mids = (pos[:-1] + pos[1:]) / 2.0  # exact ties (representable in fp32)
    f32 = np.float32
    near = np.concatenate([np.nextafter(mids.astype(f32), f32(0)), np.nextafter(mids.astype(f32), f32(500))])
    rng = np.random.default_rng(0)
    rnd = rng.uniform(-448, 448, 20000).astype(f32)
    small = (rng.standard_normal(5000) * 0.01).astype(f32)
    vals = np.concatenate([pos, mids, near, rnd, small, [448.00003, 463.99]]).astype(f32)
    return np.concatenate([vals, -vals])


def test_e4m3_encode_matches_torch_cast_including_ties():
    x = _e4m3_probe_values()
    mine = NC.e4m3_encode(x)
    theirs = torch.from_numpy(x).to(F8).view(torch.uint8).numpy()
    bad = np.nonzero(mine != theirs)[0]
    assert bad.size == 0, f"{bad.size} mismatches, e.g. x={x[bad[:5]]} mine={mine[bad[:5]]} torch={theirs[bad[:5]]}"


def test_e4m3_round_trip_and_ties_to_even():
    table = NC.e4m3_decode_table()
    codes = np.array([c for c in range(256) if not np.isnan(table[c])], dtype=np.uint8)
    assert np.array_equal(NC.e4m3_encode(table[codes].astype(np.float32)), codes)
    # 1.0625 lies halfway between 1.0 (mantissa 0) and 1.125 (mantissa 1): even wins
    assert NC.e4m3_encode(np.array([1.0625, 1.1875, 3 * 2.0 ** -10], np.float32)).tolist() == [0x38, 0x3A, 0x02]


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 3,
                        (np.arange(1, 2000, dtype=np.float32) * np.float32(2.0 ** -15) + 1).astype(np.float32)])
    mine = NC.bf16_round(x)
    theirs = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32))


# ---------------------------------------------------------------------------
# quantization
# ---------------------------------------------------------------------------

def _rows(bh=3, n=150, d=64, seed=0):
    q, k, v = O.make_inputs(1, bh, n, d, seed=seed)
    return q.reshape(bh, n, d), k.reshape(bh, n, d), v.reshape(bh, n, d)


@pytest.mark.parametrize("kind", ["int8", "fp8"])
def test_quantize_matches_numpy_restatement(kind):
    x, _, _ = _rows()
    codes, scale = O.quantize(x, kind, "token")
    xf = x.float().numpy()
    amax = np.abs(xf).max(axis=-1)
    if kind == "int8":
        ncodes, nscale = NC.quant_int8_rows(xf, amax)
        assert np.array_equal(codes.numpy(), ncodes)
    else:
        ncodes, nscale = NC.quant_fp8_rows(xf, amax)
        assert np.array_equal(codes.view(torch.uint8).numpy(), ncodes)
    assert np.array_equal(scale.numpy().view(np.uint32), nscale.view(np.uint32))


def test_int8_known_answers_truncate_toward_zero():
    # amax = 127 makes inv exactly 1, so the codes are trunc(x)
    row = torch.tensor([[[127.0, -1.5, 1.5, 0.99, -0.99, 126.5, -127.0, 0.0]]]).bfloat16()
    codes, scale = O.quantize(row, "int8", "token")
    assert codes.flatten().tolist() == [127, -1, 1, 0, 0, 126, -127, 0]
    assert scale.item() == 1.0


def test_fp8_known_answers_round_half_even():
    # amax = 448 makes inv exactly 1, so the codes are e4m3(x) at exact ties
    row = torch.tensor([[[448.0, 1.0625, 1.1875, -1.0625, 0.0029296875, 240.0, 0.5]]]).bfloat16()
    codes, scale = O.quantize(row, "fp8", "token")
    assert codes.view(torch.uint8).flatten().tolist() == [0x7E, 0x38, 0x3A, 0xB8, 0x02, 0x77, 0x30]
    assert scale.item() == 1.0


def test_int8_invariants():
    x, _, _ = _rows(seed=3)
    codes, scale = O.quantize(x, "int8", "token")
    c = codes.int()
    assert c.abs().max() <= 127
    # the amax element maps to 126 or 127 (truncation of 127*(1 +- eps))
    idx = x.float().abs().argmax(dim=-1, keepdim=True)
    top = c.gather(-1, idx).abs()
    assert ((top == 127) | (top == 126)).all()
    # dequantization error is below one step
    err = (x.float() - c.float() * scale[..., None]).abs()
    assert (err <= scale[..., None] * (1 + 1e-4)).all()  # fp32 rounding of x - c*s adds ~127 ulp of s
    # sign is preserved and truncation never overshoots
    assert ((c.float() * x.float()) >= 0).all()


def test_zero_rows_give_zero_codes_and_scales():
    x = torch.zeros(1, 4, 64).bfloat16()
    for kind in ("int8", "fp8"):
        codes, scale = O.quantize(x, kind, "token")
        assert not codes.view(torch.uint8).any() and not scale.any()


def test_block64_granularity():
    x, _, _ = _rows(bh=2, n=150, seed=4)
    codes, scale = O.quantize(x, "int8", "block64")
    assert scale.shape == (2, 3)
    xf = x.float().numpy()
    for b in range(3):
        seg = xf[:, 64 * b:64 * (b + 1)]
        amax = np.abs(seg).max(axis=(1, 2))
        ncodes, nscale = NC.quant_int8_rows(seg.reshape(2, -1), amax)
        assert np.array_equal(codes[:, 64 * b:64 * (b + 1)].reshape(2, -1).numpy(), ncodes)
        assert np.array_equal(scale[:, b].numpy(), nscale)


def test_q_scale_folds_softmax_scale():
    x, _, _ = _rows(seed=5)
    fold = O.sm_scale_log2e(1 / math.sqrt(64))
    _, plain = O.quantize(x, "int8", "token")
    _, folded = O.quantize(x, "int8", "token", fold=fold)
    assert torch.equal(folded, plain * torch.tensor(fold, dtype=torch.float32))
    # sm_scale * log2(e) in fp64, then handed over as fp32 (sage_attention.py:493-495)
    assert fold == float(np.float32(0.125 * 1.4426950408889634))


def test_v_fp8_per_block_channel():
    _, _, v = _rows(bh=2, n=130, seed=6)
    vc, vs = O.quantize_v_fp8(v)
    assert vc.shape == v.shape and vs.shape == (2, 3, 64)
    vf = v.float().numpy()
    for b in range(3):
        seg = vf[:, 64 * b:64 * (b + 1)]
        amax = np.abs(seg).max(axis=1)  # per channel
        # quantize columns: transpose so each channel is a row
        ncodes, nscale = NC.quant_fp8_rows(seg.transpose(0, 2, 1), amax)
        assert np.array_equal(vc[:, 64 * b:64 * (b + 1)].view(torch.uint8).numpy(), ncodes.transpose(0, 2, 1))
        assert np.array_equal(vs[:, b].numpy(), nscale)


# ---------------------------------------------------------------------------
# K smoothing
# ---------------------------------------------------------------------------

def test_k_mean_within_one_bf16_ulp_and_order_free():
    _, k, _ = O.make_inputs(2, 3, 300, 64, seed=8)
    mu = O.k_mean(k)
    exact = k.double().mean(dim=2, keepdim=True)
    ulp = torch.tensor(NC.bf16_round(np.abs(exact.float().numpy()) * np.float32(1 + 2 ** -7))).double() - \
        torch.tensor(NC.bf16_round(np.abs(exact.float().numpy()))).double()
    assert ((mu.double() - exact).abs() <= ulp.abs() + 1e-30).all()
    perm = torch.randperm(300, generator=torch.Generator().manual_seed(0))
    assert torch.equal(O.k_mean(k[:, :, perm]).view(torch.int16), mu.view(torch.int16))
    const = torch.full((1, 1, 77, 8), 1.5).bfloat16()
    assert (O.k_mean(const).float() == 1.5).all()


def test_smooth_k_matches_numpy():
    _, k, _ = O.make_inputs(1, 2, 100, 64, seed=9)
    ks, mu = O.smooth_k(k)
    want = NC.bf16_round(k.float().numpy() - mu.float().numpy())
    assert np.array_equal(ks.float().numpy().view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------------------
# integer QK^T
# ---------------------------------------------------------------------------

def test_qk_int32_brute_force():
    rng = random.Random(0)
    n, m, d = 5, 7, 8
    qc = torch.tensor([[[rng.randint(-127, 127) for _ in range(d)] for _ in range(n)]], dtype=torch.int8)
    kc = torch.tensor([[[rng.randint(-127, 127) for _ in range(d)] for _ in range(m)]], dtype=torch.int8)
    want = [[sum(int(qc[0, i, t]) * int(kc[0, j, t]) for t in range(d)) for j in range(m)] for i in range(n)]
    assert O.qk_int32(qc, kc)[0].tolist() == want


def test_qk_int32_extremes_and_numpy():
    d = 128
    ones = torch.full((1, 3, d), 127, dtype=torch.int8)
    neg = torch.full((1, 3, d), -127, dtype=torch.int8)
    assert (O.qk_int32(ones, ones) == 127 * 127 * d).all()
    assert (O.qk_int32(ones, neg) == -127 * 127 * d).all()
    x, y, _ = _rows(bh=2, n=200, d=128, seed=10)
    qc, _ = O.quantize(x, "int8")
    kc, _ = O.quantize(y, "int8")
    assert np.array_equal(O.qk_int32(qc, kc).numpy(), NC.qk_int32_bruteforce(qc.numpy(), kc.numpy()))


def test_qk_fp8_exact():
    x, y, _ = _rows(bh=1, n=40, d=64, seed=11)
    qc, _ = O.quantize(x, "fp8")
    kc, _ = O.quantize(y, "fp8")
    table = NC.e4m3_decode_table()
    qa = table[qc.view(torch.uint8).numpy()]
    ka = table[kc.view(torch.uint8).numpy()]
    # products of two e4m3 values and their sums over 64 terms are exact in fp64
    assert np.array_equal(O.qk_fp8(qc, kc).numpy(), qa @ ka.swapaxes(-1, -2))


# ---------------------------------------------------------------------------
# masks
# ---------------------------------------------------------------------------

def _ref_block_mask_bruteforce(segs, total):
    doc = [0] * total
    off = 0
    for i, s in enumerate(segs):
        for t in range(off, off + s):
            doc[t] = i
        off += s
    nq, nk = -(-total // 128), -(-total // 64)
    return [[int(doc[min(128 * i, total - 1)] == doc[min(64 * j, total - 1)]) for j in range(nk)]
            for i in range(nq)]


def test_block_mask_packed_config():
    segs = [1280, 1216, 4416]
    m = O.build_block_mask(segs)
    assert m.shape == (54, 108)
    assert int(m.sum()) == 2736  # 46.9 % of 5832 tiles on
    assert m.tolist() == _ref_block_mask_bruteforce(segs, 6912)
    # Q tile 19 starts at token 2432 (image 1) and straddles into image 2 at 2496
    assert m[19].nonzero().flatten().tolist() == list(range(20, 39))


def test_block_mask_trailing_pad_is_doc0():
    m = O.build_block_mask([64, 64], total_len=256)
    # tokens 128..255 are padding and keep document id 0
    assert m.tolist() == [[1, 0, 1, 1], [1, 0, 1, 1]]


def test_block_mask_host_builder_matches_oracle():
    from futudiffu_amd import block_mask as BM
    for segs, total in (([1280, 1216, 4416], None), ([64, 64], 256), ([1000], None), ([33, 95, 7], 200)):
        want = O.build_block_mask(segs, total)
        got = BM.build_block_mask(segs, total, device="cpu")
        assert torch.equal(got, want), segs


def test_doc_visibility_bruteforce():
    doc = torch.tensor([[0, 0, 1, -1, 1, 2]], dtype=torch.int32)
    vis = O.doc_visibility(doc)[0]
    d = doc[0].tolist()
    for i in range(6):
        for j in range(6):
            assert bool(vis[i, j]) == (d[j] >= 0 and (d[i] == d[j] or d[i] < 0))


def test_tile_mask_expansion():
    mask = torch.tensor([[1, 0, 1]], dtype=torch.uint8)  # N = 150 -> 2 q tiles? no: ceil(150/128)=2
    mask = torch.tensor([[1, 0, 1], [0, 1, 0]], dtype=torch.uint8)
    vis = O.tile_mask_visibility(mask, 2, 150)
    assert vis.shape == (2, 150, 150)
    assert vis[1, 0, 0] and not vis[0, 0, 64] and vis[0, 127, 149] and not vis[0, 128, 0] and vis[0, 149, 100]


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def _softmax_ref(s, v, visible=None):
    s = s.double()
    if visible is not None:
        s = s.masked_fill(~visible, -math.inf)
    m = s.amax(dim=-1, keepdim=True)
    p = torch.exp2(s - m)
    l = p.sum(dim=-1, keepdim=True)
    return (p @ v.double()) / l, (m + torch.log2(l)).squeeze(-1)


def test_attend_single_tile_equals_softmax():
    g = torch.Generator().manual_seed(0)
    s = torch.randn(2, 40, 40, generator=g) * 3
    v = torch.randn(2, 40, 32, generator=g).bfloat16()
    out, lse = O.attend(s, v, "bf16", None)
    m = s.amax(dim=-1, keepdim=True)
    p = torch.exp2(s - m)
    want = (p.bfloat16().double() @ v.double()) / p.double().sum(-1, keepdim=True)
    assert (out.double() - want).abs().max() <= 2 ** -8 * want.abs().max()
    assert (lse.double() - (m.squeeze(-1).double() + torch.log2(p.double().sum(-1)))).abs().max() < 1e-5


def test_attend_moving_max_across_tiles():
    # scores grow tile by tile, so every tile moves the running max (alpha != 1)
    n = 256
    g = torch.Generator().manual_seed(1)
    s = torch.randn(1, 8, n, generator=g) + torch.arange(n).float() / 16
    v = torch.randn(1, n, 16, generator=g).bfloat16()
    out, lse = O.attend(s, v, "bf16", None)
    want, wlse = _softmax_ref(s, v)
    assert (out.double() - want).abs().max() < 2e-2 * want.abs().max()
    assert (lse.double() - wlse).abs().max() < 1e-4
    out8, _ = O.attend(s, v, "fp8", None, *O.quantize_v_fp8(v))
    assert O.cosine(out8, want) > 0.998


def test_attend_uniform_scores_known_answer():
    # zero scores: p = 1 everywhere, l = N exactly, lse = log2(N), out = mean(V)
    n = 200
    s = torch.zeros(1, 3, n)
    v = torch.randn(1, n, 8, generator=torch.Generator().manual_seed(2)).bfloat16()
    out, lse = O.attend(s, v, "bf16", None)
    assert (lse == math.log2(n)).all()
    want = v.double().mean(dim=1, keepdim=True).expand(1, 3, 8)
    assert (out.double() - want).abs().max() <= 2 ** -8 * want.abs().max() + 1e-6


def test_attend_masked_rows_and_keys():
    g = torch.Generator().manual_seed(3)
    s = torch.randn(1, 70, 70, generator=g)
    v = torch.randn(1, 70, 8, generator=g).bfloat16()
    doc = torch.tensor([[0] * 30 + [1] * 30 + [-1] * 10], dtype=torch.int32)
    vis = O.doc_visibility(doc)
    vis[0, 5, :] = False  # a row that sees nothing
    out, lse = O.attend(s, v, "bf16", vis)
    assert (out[0, 5] == 0).all() and lse[0, 5] == -math.inf
    want, wlse = _softmax_ref(s, v, vis)
    rows = [r for r in range(70) if r != 5]
    assert (out[0, rows].double() - want[0, rows]).abs().max() < 2e-2
    assert (lse[0, rows].double() - wlse[0, rows]).abs().max() < 1e-4


@pytest.mark.parametrize("qk,pv,gran", [("int8", "bf16", "block64"), ("int8", "bf16", "token"),
                                        ("int8", "fp8", "token"), ("fp8", "bf16", "token"),
                                        ("fp8", "fp8", "token")])
def test_sage_forward_close_to_fp64(qk, pv, gran):
    q, k, v = O.make_inputs(1, 4, 256, 64, seed=12)
    out, lse, _ = O.sage_forward(q, k, v, None, qk, pv, gran, True)
    ref, _ = O.sdpa_fp64(q, k, v)
    assert O.cosine(out, ref) > (0.999 if pv == "bf16" else 0.998)
    # the LSE is that of the smoothed scores (a per-row shift of q.mu), as in the reference
    _, rlse = O.sdpa_fp64(q, O.smooth_k(k)[0], v)
    assert (lse.double() - rlse).abs().max() < 0.1


def test_smoothing_is_softmax_invariant():
    # unquantized: k and k - mean(k) give the same attention (per-row constant shift)
    q, k, v = O.make_inputs(1, 2, 128, 64, seed=13)
    ks, _ = O.smooth_k(k)
    sc = 1 / math.sqrt(64) * O.LOG2E
    a, _ = O.attend((q.float() @ k.float().transpose(-1, -2)).reshape(2, 128, 128) * sc, v.reshape(2, 128, 64), "bf16", None)
    b, _ = O.attend((q.float() @ ks.float().transpose(-1, -2)).reshape(2, 128, 128) * sc, v.reshape(2, 128, 64), "bf16", None)
    assert O.cosine(a, b) > 0.9999


def test_static_p_scheme_close_to_reference_scheme():
    q, k, v = O.make_inputs(1, 2, 512, 128, seed=14)
    a, la, _ = O.sage_forward(q, k, v, None, "int8", "fp8", "token", True)
    b, lb, _ = O.sage_forward(q, k, v, None, "int8", "fp8", "token", True, p_scheme="static", tau=2.0)
    assert O.cosine(a, b) > 0.999 and (a.float() - b.float()).abs().max() < 2e-2
    assert (la - lb).abs().max() < 1e-4


# ---------------------------------------------------------------------------
# fp8 P.V: one P scale per (row, 64-key block), known answers
# ---------------------------------------------------------------------------

def _fp8_pv_known_answer_case(offset):
    """One query row over two 64-key tiles whose live scores are exact
    integers (log2 units): s = -j for keys j = 0..15 of tile 0 and
    s = offset - j for keys 64 + j, j = 0..15, of tile 1; the other keys sit
    at -200 (p = 0 exactly in fp32).  V is the 128 x 128 identity, so output
    channel c is key c's share: out[c] = p_c / l with p_c = 2^(s_c - max s).

    Per (row, block) P scaling (sage_kernels.py:1137-1141) maps each tile's
    largest p to 448 and the rest to 448 * 2^-j, which e4m3 holds exactly for
    j <= 15 (7 * 2^(6 - j), subnormal below 2^-6), in both tiles.  One scale
    per row across tiles would instead give tile 1 the codes
    e4m3(448 * 2^(offset - j)): for offset = -12 those fall below e4m3's
    subnormal grid from j = 4 on (3.5 * 2^-9 rounds to 4 * 2^-9, ...)."""
    nk, d = 128, 128
    s = torch.full((1, 1, nk), -200.0)
    j = torch.arange(16, dtype=torch.float32)
    s[0, 0, :16] = -j
    s[0, 0, 64:80] = offset - j
    v = torch.eye(nk, d).bfloat16().unsqueeze(0)
    # V codes and scales from the definition (sage_kernels.py:1143-1148):
    # each channel's block max is 1, so its code is e4m3(448) = 448 and its
    # scale 1/448; channels with no key in a block have code 0 and scale 0
    vc = (torch.eye(nk, d) * 448.0).to(torch.float8_e4m3fn).unsqueeze(0)
    vs = torch.zeros(1, 2, d)
    vs[0, 0, :64] = torch.tensor(1.0 / 448.0, dtype=torch.float32)
    vs[0, 1, 64:] = torch.tensor(1.0 / 448.0, dtype=torch.float32)
    sd = s.double()
    p = torch.exp2(sd - sd.max())
    # keys at -200 have p = 0 in fp32, as the reference's exp2 gives them
    p = torch.where(sd > -100, p, torch.zeros(()))
    want = (p / p.sum())[0, 0]
    want_lse = float(sd.max() + torch.log2(p.sum()))
    return s, v, vc, vs, want, want_lse


def _rel_err(out, want):
    live = want > 0
    return ((out.double()[live] - want[live]).abs() / want[live]).max().item(), out.double()[~live].abs().max().item()


@pytest.mark.parametrize("offset", [-12.0, 12.0])
def test_attend_fp8_pv_per_block_p_scale_known_answer(offset):
    """The oracle's fp8 P.V against the closed form: every live key's output
    share within one bf16 rounding, dead keys exactly 0, LSE within fp32
    rounding.  offset = +12 moves the row max in tile 1 (alpha = 2^-12 on
    tile 0's products); offset = -12 leaves it in tile 0."""
    s, v, vc, vs, want, want_lse = _fp8_pv_known_answer_case(offset)
    out, lse = O.attend(s, v, "fp8", None, vc, vs)
    rel, dead = _rel_err(out[0, 0], want)
    assert rel <= 2.0 ** -8, rel
    assert dead == 0.0
    assert abs(float(lse[0, 0]) - want_lse) < 1e-6


def test_fp8_pv_known_answer_fails_one_scale_per_row():
    """The same closed form rejects one P scale per row across tiles (the
    running-max frame: pc = e4m3(448 * p) with p relative to the row's
    running max).  The oracle's "static" scheme with tau = 0 is exactly that
    mistake here: its reference point is set by tile 0 and never moves."""
    s, v, vc, vs, want, _ = _fp8_pv_known_answer_case(-12.0)
    out, _ = O.attend(s, v, "fp8", None, vc, vs, p_scheme="static", tau=0.0)
    rel, _ = _rel_err(out[0, 0], want)
    assert rel > 0.1, rel
