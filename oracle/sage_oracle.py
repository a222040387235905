"""CPU oracle for the Sage attention path (TEST INFRASTRUCTURE ONLY).

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``futudiffu_amd``) never calls into it and fails
loudly when the HIP library is missing.

It restates, in plain PyTorch CPU arithmetic, the reference's SageAttention
forward as implemented by the Triton kernels of sqcu/futudiffu
(``src/futudiffu/sage_kernels.py``) and their launcher
(``src/futudiffu/sage_attention.py``).  Each function cites the reference lines
it follows.  Every function here is pinned by a check in
``tests/test_oracle.py`` (closed forms, invariants, brute force on tiny
inputs; the packed-plan mask helpers in ``tests/test_masks.py``) and by the
committed fixtures in ``tests/golden/``; the reference has no golden vectors
or known-answer tests for this path.

Conventions (all follow the reference):
  * q, k, v are bf16 ``[B, H, N, D]``; internal math flattens to ``[BH, N, D]``.
  * Scores live in the log2 domain: ``s = q.k * sm_scale * log2(e)``; the
    softmax uses exp2 and the returned LSE is ``m + log2(l)`` in those units
    (sage_kernels.py:1468-1471).
  * Quantization ("per token", the reference's granularity):
      int8: ``inv = 127 / max(amax, 1e-12)`` (fp32 division),
            ``code = trunc(x * inv)``, ``scale = amax / 127``
            (sage_kernels.py:1415-1422 for Q, :1443-1449 for K).
      fp8 : ``inv = 448 / max(amax, 1e-12)``, ``code = e4m3fn_rne(x * inv)``,
            ``scale = amax / 448`` (sage_kernels.py:250-258, :272-280).
      The Q scale has ``sm_scale*log2(e)`` folded in (:1422, :258).
  * "block64" granularity (one scale per 64 tokens) is the CPU plumbing case's
    variant; it applies the same formulas with amax over a 64-token block.

Deviation that is a definition, not an approximation:
  * K-smoothing mean.  The reference computes ``k.mean(dim=2)`` in bf16 via
    torch (fp32 accumulation in an unspecified order, sage_attention.py:63-71),
    which can differ by one bf16 ulp between implementations.  The oracle and
    the HIP kernel both define ``mu = bf16_rne(fp32_rn(sum_fp64(k) / N))``;
    the fp64 sum of bf16 values is exact (hence order-independent) unless a
    channel mixes magnitudes more than ~2^40 apart.  ``tests/test_oracle.py``
    checks mu against the fp64 mean to within one bf16 ulp.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

LOG2E = math.log2(math.e)  # sage_attention.py:27
FP8_MAX = 448.0            # torch.finfo(float8_e4m3fn).max, sage_attention.py:149
INT8_MAX = 127.0           # sage_kernels.py:1420
EPS = 1e-12                # tl.maximum(amax, 1e-12), sage_kernels.py:1421
BLOCK_M = 128              # reference Q tile, block_mask.py:27
BLOCK_N = 64               # reference KV tile, block_mask.py:28
F8 = torch.float8_e4m3fn
_F32 = torch.float32


def _f32(x: float) -> torch.Tensor:
    return torch.tensor(x, dtype=_F32)


def sm_scale_log2e(sm_scale: float) -> float:
    """``sm_scale * log2(e)`` computed in fp64 and handed to the kernel as fp32.

    sage_attention.py:493-495 (Python float product, passed as a Triton fp32
    scalar argument).
    """
    return float(_f32(float(sm_scale) * LOG2E))


# ---------------------------------------------------------------------------
# Producer of q, k, v: QKV split + per-head RMSNorm + Flux RoPE + transpose
# (fused_qkv_postprocess, src/futudiffu/fused_kernels.py:271-390, op :613-643)
# ---------------------------------------------------------------------------

def sum_squares(x: torch.Tensor) -> torch.Tensor:
    """fp64 sum of squares over the last dimension in the producer's fixed
    order: each run of 8 channels left to right, then a pairwise tree over the
    runs in channel order.  Returns ``[..., 1]``."""
    d = x.shape[-1]
    sq = (x.double() ** 2).unflatten(-1, (d // 8, 8))
    runs = sq[..., 0]
    for e in range(1, 8):
        runs = runs + sq[..., e]
    while runs.shape[-1] > 1:
        runs = runs[..., 0::2] + runs[..., 1::2]
    return runs


def rms_rope(x: torch.Tensor, w: torch.Tensor, freqs: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm then rotary embedding of ``x`` (``[B, N, H, D]``, values of bf16),
    returned in fp32 before the bf16 store.

    fused_kernels.py:316-377: ``rrms = 1 / sqrt(mean(x^2) + eps)`` (:318-320),
    ``n = x * rrms * w`` (:357-360), and per pair p of channels (2p, 2p+1) with
    ``freqs[.., p] = [[cos, -sin], [sin, cos]]`` (:334-336):
    ``even' = cos*n_even + (-sin)*n_odd``, ``odd' = sin*n_even + cos*n_odd``
    (:363-366).  Definitions where the reference leaves the order open (as the
    K mean in the module docstring): the sum of squares is taken in fp64 over
    the bf16 squares in a fixed order -- each run of 8 channels left to right,
    then a pairwise tree over the D/8 runs in channel order -- and rounded once
    to fp32 with the division by D; every product and sum is a separately
    rounded fp32 operation (no fused multiply-add).
    """
    d = x.shape[-1]
    r32 = _round_f32
    ms = r32(sum_squares(x) / d)
    rrms = r32(1.0 / r32(torch.sqrt(r32(ms + float(_f32(eps))))))
    n = r32(r32(x.double() * rrms) * w.float().double())
    ne, no = n[..., 0::2], n[..., 1::2]
    f = freqs.float().double()            # [B, N, 1, D/2, 2, 2], broadcast over heads
    cos, nsin, sin = f[..., 0, 0], f[..., 0, 1], f[..., 1, 0]
    re = r32(r32(cos * ne) + r32(nsin * no))
    ro = r32(r32(sin * ne) + r32(cos * no))
    return torch.stack([re, ro], dim=-1).flatten(-2).float()


def _round_f32(t: torch.Tensor) -> torch.Tensor:
    """Round fp64 values to the nearest fp32 (kept as fp64).  Applied to the
    fp64 result of one +, -, *, / or sqrt of fp32 operands it gives exactly
    the correctly rounded fp32 operation (fp64 carries more than 2*24+2 bits,
    so the double rounding is innocuous), whatever the host's fp32 kernels do."""
    return t.float().double()


def qkv_postprocess(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor, freqs: torch.Tensor,
                    n_heads: int, head_dim: int, eps: float = 1e-5) -> tuple[torch.Tensor, ...]:
    """bf16 ``q, k, v`` ``[B, H, N, D]`` from the QKV projection output ``[B, N, 3*H*D]``
    (fused_kernels.py:271-390; torch form :517-541).  ``freqs`` is
    ``[B, N, 1, D/2, 2, 2]`` fp32."""
    b, n, _ = qkv.shape
    x = qkv.view(b, n, 3, n_heads, head_dim)
    if freqs.ndim == 5:
        freqs = freqs.unsqueeze(2)
    q = rms_rope(x[:, :, 0], q_norm_w, freqs, eps).to(torch.bfloat16)
    k = rms_rope(x[:, :, 1], k_norm_w, freqs, eps).to(torch.bfloat16)
    v = x[:, :, 2]
    return tuple(t.movedim(1, 2).contiguous() for t in (q, k, v))


def qkv_postprocess_backward(qkv: torch.Tensor, q_norm_w: torch.Tensor, k_norm_w: torch.Tensor,
                             freqs: torch.Tensor, grad_q: torch.Tensor, grad_k: torch.Tensor,
                             grad_v: torch.Tensor, n_heads: int, head_dim: int,
                             eps: float = 1e-5) -> torch.Tensor:
    """Gradient of the producer with respect to ``qkv``, bf16 ``[B, N, 3*H*D]``
    (fused_kernels.py:711-783; the norm weights and rotations get none, :783).

    Per head and token, with x the raw q (k) row, w its norm weights,
    rrms = 1/sqrt(mean(x^2) + eps) and g = the incoming gradient (:732-734):
      * the rotation's transpose, per pair (e, o) with (cos, sin) the matrix
        entries [0][0] and [1][0]: (cos*g_e + sin*g_o, -sin*g_e + cos*g_o)
        (:736-758);
      * the RMSNorm backward: gw = g' * w, c = sum(gw * x) / D,
        dx = rrms * (gw - x * rrms^2 * c) (:760-776), rounded to bf16;
      * v's gradient passes through; the three blocks are concatenated in the
        projection's layout (:778-783).
    Evaluated in fp64 from the bf16 inputs (the reference uses fp32 with
    unspecified reduction order: tolerance-level).
    """
    b, n, _ = qkv.shape
    h, d = n_heads, head_dim
    if freqs.ndim == 6:
        freqs = freqs.squeeze(2)
    cos = freqs[..., 0, 0].double()[:, :, None, :]  # [B, N, 1, D/2]
    sin = freqs[..., 1, 0].double()[:, :, None, :]
    x = qkv.view(b, n, 3, h, d)

    def one(grad, xr, w):
        g = grad.movedim(1, 2).double().reshape(b, n, h, d // 2, 2)
        ge, go = g[..., 0], g[..., 1]
        gp = torch.stack([cos * ge + sin * go, -sin * ge + cos * go], -1).reshape(b, n, h, d)
        xf = xr.double()
        rrms = 1.0 / torch.sqrt((xf * xf).mean(-1, keepdim=True) + eps)
        gw = gp * w.double()
        c = (gw * xf).sum(-1, keepdim=True) / d
        return (rrms * (gw - xf * rrms * rrms * c)).to(torch.bfloat16)

    dq = one(grad_q, x[:, :, 0], q_norm_w)
    dk = one(grad_k, x[:, :, 1], k_norm_w)
    dv = grad_v.movedim(1, 2)
    return torch.cat([dq.reshape(b, n, h * d), dk.reshape(b, n, h * d), dv.reshape(b, n, h * d)], -1).contiguous()


# ---------------------------------------------------------------------------
# K smoothing (sage_attention.py:63-71, called at :490-491)
# ---------------------------------------------------------------------------

def k_mean(k: torch.Tensor) -> torch.Tensor:
    """Per-(b, h, channel) mean of K over the sequence, bf16 ``[B, H, 1, D]``.

    Follows ``k.mean(dim=2, keepdim=True)`` (sage_attention.py:71) with the
    deterministic rounding chain fixed in the module docstring.
    """
    n = k.shape[2]
    s = k.double().sum(dim=2, keepdim=True)
    return (s / n).to(_F32).to(torch.bfloat16)


def smooth_k(k: torch.Tensor, mu: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """``k - mu`` in bf16 arithmetic (fp32 subtract, bf16 RNE), sage_attention.py:71."""
    if mu is None:
        mu = k_mean(k)
    return (k.float() - mu.float()).to(torch.bfloat16), mu


# ---------------------------------------------------------------------------
# Quantization (sage_kernels.py:1415-1422, :1443-1449, :250-258, :272-280)
# ---------------------------------------------------------------------------

def _amax(x: torch.Tensor, granularity: str) -> torch.Tensor:
    """|x| max per token ``[BH, N]`` or per 64-token block ``[BH, ceil(N/64)]``."""
    a = x.abs().amax(dim=-1)
    if granularity == "token":
        return a
    if granularity == "block64":
        bh, n = a.shape
        nb = (n + 63) // 64
        pad = torch.zeros(bh, nb * 64, dtype=a.dtype)
        pad[:, :n] = a
        return pad.view(bh, nb, 64).amax(dim=-1)
    raise ValueError(f"unknown granularity {granularity!r}")


def _expand(scale: torch.Tensor, n: int, granularity: str) -> torch.Tensor:
    if granularity == "token":
        return scale
    return scale.repeat_interleave(64, dim=-1)[:, :n]


def quantize(x: torch.Tensor, kind: str, granularity: str = "token",
             fold: float | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric int8 / fp8-e4m3fn quantization of ``x`` ``[BH, N, D]`` (bf16).

    Returns ``(codes, scale)``; ``scale`` is ``amax/127`` (int8) or
    ``amax/448`` (fp8), multiplied by ``fold`` when given (the Q path folds
    ``sm_scale*log2e`` there, sage_kernels.py:1422 / :258).  All arithmetic is
    IEEE fp32 with round-to-nearest; int8 codes truncate toward zero
    (Triton ``.to(tl.int8)`` lowers to fptosi), fp8 codes round to nearest even.
    """
    xf = x.float()
    n = xf.shape[1]
    amax = _amax(xf, granularity)
    qmax = INT8_MAX if kind == "int8" else FP8_MAX
    inv = _f32(qmax) / torch.clamp_min(amax, EPS)
    y = xf * _expand(inv, n, granularity)[..., None]
    if kind == "int8":
        codes = torch.trunc(y).to(torch.int8)
    elif kind == "fp8":
        codes = y.to(F8)
    else:
        raise ValueError(f"unknown quant kind {kind!r}")
    scale = amax / _f32(qmax)
    if fold is not None:
        scale = scale * _f32(fold)
    return codes, scale


def quantize_v_fp8(v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """V fp8 codes with one scale per (64-token block, channel).

    sage_kernels.py:1143-1148: ``vs_d = max_n |v|`` over the block's tokens,
    ``code = e4m3fn(v * 448 / max(vs_d, 1e-12))``, ``scale = vs_d / 448``.
    Returns codes ``[BH, N, D]`` and scales ``[BH, ceil(N/64), D]``.
    """
    vf = v.float()
    bh, n, d = vf.shape
    nb = (n + 63) // 64
    pad = torch.zeros(bh, nb * 64, d)
    pad[:, :n] = vf
    amax = pad.view(bh, nb, 64, d).abs().amax(dim=2)
    inv = _f32(FP8_MAX) / torch.clamp_min(amax, EPS)
    codes = (pad.view(bh, nb, 64, d) * inv[:, :, None, :]).to(F8).view(bh, nb * 64, d)[:, :n]
    return codes.contiguous(), amax / _f32(FP8_MAX)


def codes_to_float(codes: torch.Tensor) -> torch.Tensor:
    return codes.float()


def qk_int32(qc: torch.Tensor, kc: torch.Tensor) -> torch.Tensor:
    """Exact ``sum_d qc*kc`` as int32 ``[BH, N, N]`` (sage_kernels.py:1451).

    Evaluated in fp64: every partial sum is an integer below 2^53, so the
    result is exact (the Triton int8 dot returns int32).
    """
    return torch.matmul(qc.double(), kc.double().transpose(1, 2)).to(torch.int32)


def qk_fp8(qc: torch.Tensor, kc: torch.Tensor) -> torch.Tensor:
    """Exact fp64 value of the fp8 code dot products (sage_kernels.py:282)."""
    return torch.matmul(qc.double(), kc.double().transpose(1, 2))


# ---------------------------------------------------------------------------
# Masks
# ---------------------------------------------------------------------------

def build_block_mask(segment_lengths: list[int], total_len: int | None = None) -> torch.Tensor:
    """uint8 ``[ceil(N/128), ceil(N/64)]`` tile mask, block_mask.py:35-99.

    ``mask[i, j] = doc(first token of Q tile i) == doc(first token of KV tile j)``;
    tokens past the last segment keep doc 0 (block_mask.py:75-79); tile starts
    are clamped to ``N-1`` (:89, :93).
    """
    if total_len is None:
        total_len = sum(segment_lengths)
    doc = [0] * total_len
    off = 0
    for i, s in enumerate(segment_lengths):
        for t in range(off, min(off + s, total_len)):
            doc[t] = i
        off += s
    nq = (total_len + BLOCK_M - 1) // BLOCK_M
    nk = (total_len + BLOCK_N - 1) // BLOCK_N
    qd = [doc[min(i * BLOCK_M, total_len - 1)] for i in range(nq)]
    kd = [doc[min(j * BLOCK_N, total_len - 1)] for j in range(nk)]
    return torch.tensor([[1 if qd[i] == kd[j] else 0 for j in range(nk)] for i in range(nq)],
                        dtype=torch.uint8)


def packed_document_ids(segment_lengths: list[int], target_len: int | None = None) -> list[int]:
    """Per-token document ids of a packed plan, as ``build_packed_sequence``
    writes them (segment i -> id i, transformer.py:137-153) and
    ``_pad_plan_to_fixed_len`` pads them (-1 up to ``target_len``,
    forward_packed.py:56-62; longer plans raise ValueError, :47-51)."""
    doc = [i for i, s in enumerate(segment_lengths) for _ in range(s)]
    if target_len is not None:
        if len(doc) > target_len:
            raise ValueError(f"packed length {len(doc)} exceeds {target_len}")
        doc += [-1] * (target_len - len(doc))
    return doc


def tile_mask_from_doc(doc: list[int], pad_fill: int = 0) -> torch.Tensor:
    """The reference tile rule (block_mask.py:84-97) evaluated on per-token
    document ids: tile starts clamped to ``N-1``, mask = equality of the first
    tokens' ids.  Ids below zero (padding) count as ``pad_fill``: with 0 this is
    the reference's view of tokens past the last segment (block_mask.py:75-79)."""
    n = len(doc)
    d = [pad_fill if x < 0 else x for x in doc]
    nq = (n + BLOCK_M - 1) // BLOCK_M
    nk = (n + BLOCK_N - 1) // BLOCK_N
    qd = [d[min(i * BLOCK_M, n - 1)] for i in range(nq)]
    kd = [d[min(j * BLOCK_N, n - 1)] for j in range(nk)]
    return torch.tensor([[1 if qd[i] == kd[j] else 0 for j in range(nk)] for i in range(nq)],
                        dtype=torch.uint8)


def doc_ids_from_cu_seqlens(cu: list[int], n: int) -> list[int]:
    """Exact per-token ids from segment offsets ``cu`` (segment s covers tokens
    ``[cu[s], cu[s+1])``, the varlen form of build_packed_sequence's layout,
    transformer.py:137-153); tokens outside every segment are padding (-1).
    ``cu`` is nondecreasing, so the segments are disjoint."""
    doc = [-1] * n
    for t in range(n):
        for s in range(len(cu) - 1):
            if cu[s] <= t < cu[s + 1]:
                doc[t] = s
                break
    return doc


def doc_visibility(doc_ids: torch.Tensor) -> torch.Tensor:
    """Exact per-token visibility ``[B, N, N]`` from per-token document ids.

    Key n is visible to query m iff ``doc[n] >= 0`` and (``doc[m] == doc[n]``
    or ``doc[m] < 0``): a negative id marks padding; padded keys are never
    attended and padded queries see every valid key (key-padding semantics).
    This is the exact form of the reference's block-diagonal packing mask
    (block_mask.py:72-97 uses the first token of each tile instead).
    """
    dq = doc_ids[:, :, None]
    dk = doc_ids[:, None, :]
    return (dk >= 0) & ((dq == dk) | (dq < 0))


def tile_mask_visibility(mask: torch.Tensor, bh: int, n: int) -> torch.Tensor:
    """Dense ``[BH, N, N]`` expansion of a 2D/3D reference tile mask.

    A 2D mask broadcasts over B*H (``stride_bm_z = 0``, sage_attention.py:512-519);
    entry (i, j) governs queries ``[128i, 128i+128)`` x keys ``[64j, 64j+64)``
    (sage_kernels.py:1428-1436).
    """
    if mask.ndim == 2:
        mask = mask.unsqueeze(0).expand(bh, -1, -1)
    if mask.ndim != 3:
        raise ValueError(f"block_mask must be 2D or 3D, got {mask.ndim}D")
    full = mask.bool().repeat_interleave(BLOCK_M, dim=1).repeat_interleave(BLOCK_N, dim=2)
    return full[:, :n, :n]


# ---------------------------------------------------------------------------
# Attention (online softmax over 64-key tiles)
# ---------------------------------------------------------------------------

@dataclass
class Quantized:
    qc: torch.Tensor          # [BH, N, D] int8 / fp8
    qs: torch.Tensor          # [BH, N] or [BH, nb] fp32, sm_scale*log2e folded
    kc: torch.Tensor
    ks: torch.Tensor
    vc: torch.Tensor | None   # fp8 codes (pv="fp8") else None
    vs: torch.Tensor | None   # [BH, nb, D]
    mu: torch.Tensor | None   # [B, H, 1, D] bf16
    k_smoothed: torch.Tensor  # bf16 [BH, N, D]


def quantize_all(q, k, v, sm_scale, qk="int8", pv="bf16", granularity="token",
                 smooth=True) -> Quantized:
    """Smoothing + Q/K/V quantization exactly as the forward kernels see them."""
    b, h, n, d = q.shape
    mu = None
    if smooth:
        k, mu = smooth_k(k)
    qf = q.reshape(b * h, n, d)
    kf = k.reshape(b * h, n, d)
    vf = v.reshape(b * h, n, d)
    fold = sm_scale_log2e(sm_scale)
    qc, qs = quantize(qf, qk, granularity, fold=fold)
    kc, ks = quantize(kf, qk, granularity)
    vc = vs = None
    if pv == "fp8":
        vc, vs = quantize_v_fp8(vf)
    return Quantized(qc, qs, kc, ks, vc, vs, mu, kf)


def scores(qz: Quantized, qk: str, granularity: str, heads=None) -> torch.Tensor:
    """Dequantized log2-domain scores ``s = (acc*qd)*kd`` (sage_kernels.py:1451-1453)."""
    sel = slice(None) if heads is None else heads
    qc, kc = qz.qc[sel], qz.kc[sel]
    n = qc.shape[1]
    if qk == "int8":
        acc = qk_int32(qc, kc).float()
    else:
        acc = qk_fp8(qc, kc).float()
    qd = _expand(qz.qs[sel], n, granularity)
    kd = _expand(qz.ks[sel], n, granularity)
    return (acc * qd[:, :, None]) * kd[:, None, :]


def attend(s: torch.Tensor, v: torch.Tensor, pv: str, visible: torch.Tensor | None,
           vc: torch.Tensor | None = None, vs: torch.Tensor | None = None,
           p_scheme: str = "reference", tau: float = 8.0):
    """Online softmax over 64-key tiles in order, then normalize.

    ``s`` is ``[BH, N, N]`` fp32 log2-domain scores; ``v`` bf16 ``[BH, N, D]``.
    Per tile (sage_kernels.py:1455-1466):
        m' = max(m, rowmax s); alpha = 2^(m - m'); p = 2^(s - m')
        l = alpha*l + sum(p)   (unquantized fp32 p)
        o = alpha*o + PV
    bf16 PV: ``PV = bf16(p) @ v`` (:1462-1464).
    fp8 PV (the P/V stage of _sage_attn_fwd_fp8qk_fp8pv_lse, :1135-1154):
        ps = rowmax p; pc = e4m3(p * 448/max(ps,1e-12)); PV = (pc @ vc) * ps/448 * vs/448.
    Finally ``lse = m + log2(l)`` and ``o = o / l`` -> bf16 (:1468-1477).

    ``p_scheme="static"`` is the MI355X kernel's P quantization (a documented
    deviation, used only for a tight secondary check): the reference point
    ``m`` only moves when a tile's row max exceeds it by more than ``tau``;
    ``pc = e4m3(p * 448 / 2^tau)`` with ``p = 2^(s - m) <= 2^tau`` and one P
    scale for every tile.  V codes are the reference's in both schemes.

    Fully masked rows (no visible key) return 0 and ``lse = -inf`` (the
    reference would divide 0 by 0; its tile masks never produce such rows).
    """
    bh, n, nk = s.shape  # n queries, nk keys
    d = v.shape[-1]
    vfl = v.float()
    o = torch.zeros(bh, n, d)
    l = torch.zeros(bh, n, 1)
    m = torch.full((bh, n, 1), -math.inf)
    ninf = torch.tensor(-math.inf)
    for j0 in range(0, nk, BLOCK_N):
        j1 = min(j0 + BLOCK_N, nk)
        sj = s[:, :, j0:j1]
        if visible is not None:
            sj = torch.where(visible[:, :, j0:j1], sj, ninf)
        bm = sj.amax(dim=-1, keepdim=True)
        if p_scheme == "reference":
            m_new = torch.maximum(m, bm)
        else:
            move = (bm > m + tau) | torch.isinf(m)
            m_new = torch.where(move & torch.isfinite(bm), bm, m)
        dead = torch.isinf(m_new)  # nothing visible yet for this row
        alpha = torch.where(dead, torch.ones(()), torch.exp2(m - torch.where(dead, 0.0, m_new)))
        p = torch.where(dead, torch.zeros(()), torch.exp2(sj - torch.where(dead, 0.0, m_new)))
        l = alpha * l + p.sum(dim=-1, keepdim=True)
        o = o * alpha
        if pv == "bf16":
            o = o + torch.matmul(p.to(torch.bfloat16).float(), vfl[:, j0:j1])
        else:
            vcb = vc[:, j0:j1].float()
            vsb = vs[:, j0 // BLOCK_N][:, None, :]
            if p_scheme == "reference":
                ps = p.amax(dim=-1, keepdim=True)
                pc = (p * (_f32(FP8_MAX) / torch.clamp_min(ps, EPS))).to(F8).float()
                o = o + (torch.matmul(pc, vcb) * (ps / _f32(FP8_MAX))) * vsb
            else:
                sc = _f32(FP8_MAX / 2.0 ** tau)
                pc = (p * sc).to(F8).float()
                o = o + (torch.matmul(pc, vcb) / sc) * vsb
        m = m_new
    empty = l == 0
    lse = torch.where(empty, ninf, m + torch.log2(torch.where(empty, 1.0, l)))
    out = torch.where(empty, torch.zeros(()), o / torch.where(empty, 1.0, l))
    return out.to(torch.bfloat16), lse.squeeze(-1)


def sage_forward(q, k, v, sm_scale=None, qk="int8", pv="bf16", granularity="token",
                 smooth=True, block_mask=None, doc_ids=None, p_scheme="reference",
                 tau=8.0, head_chunk=4):
    """Full Sage forward emulation: returns ``(out [B,H,N,D] bf16, lse [BH,N] fp32, Quantized)``.

    Mirrors sage_attn_forward_masked_with_lse (sage_attention.py:461-531) with
    the variant chosen by arguments instead of module globals
    (sage_attention.py:32-60).  ``block_mask`` is the reference tile mask;
    ``doc_ids`` (``[B, N]`` int32) selects exact per-token masking.
    Processes ``head_chunk`` heads at a time to bound memory.
    """
    b, h, n, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    qz = quantize_all(q, k, v, sm_scale, qk, pv, granularity, smooth)
    vflat = v.reshape(b * h, n, d)
    outs, lses = [], []
    for h0 in range(0, b * h, head_chunk):
        sel = slice(h0, min(h0 + head_chunk, b * h))
        s = scores(qz, qk, granularity, sel)
        vis = None
        if block_mask is not None:
            vm = block_mask
            if vm.ndim == 3:
                vm = vm[sel]
            vis = tile_mask_visibility(vm, s.shape[0], n)
        if doc_ids is not None:
            bidx = torch.arange(sel.start, sel.stop) // h
            dv = doc_visibility(doc_ids.to(torch.int64))[bidx]
            vis = dv if vis is None else (vis & dv)
        o, lse = attend(s, vflat[sel], pv, vis,
                        None if qz.vc is None else qz.vc[sel],
                        None if qz.vs is None else qz.vs[sel], p_scheme, tau)
        outs.append(o)
        lses.append(lse)
    out = torch.cat(outs).view(b, h, n, d)
    return out, torch.cat(lses), qz


def sdpa_fp64(q, k, v, sm_scale=None, visible=None):
    """Unquantized attention in fp64 (sanity reference); returns (out, lse_log2)."""
    b, h, n, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    s = torch.matmul(q.double(), k.double().transpose(-1, -2)) * sm_scale
    if visible is not None:
        s = s.masked_fill(~visible.view(b, h, n, n) if visible.shape[0] == b * h
                          else ~visible[:, None], -math.inf)
    lse = torch.logsumexp(s, dim=-1) * LOG2E
    return torch.matmul(torch.softmax(s, dim=-1), v.double()), lse.view(b * h, n)


# ---------------------------------------------------------------------------
# Backward (sage_attention.py:344-458 unmasked, :534-648 masked;
# sage_kernels.py:321-349 D pre-pass, :805-1030 (int8) and :1491-1722 (int8,
# tile-masked) dK/dV and dQ, :356-590 (fp8))
# ---------------------------------------------------------------------------

def delta_prepass(dout: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``D_i = sum_d dO_id * O_id`` in fp32 ``[BH, N]`` (sage_kernels.py:321-349).

    The products are fp32; the sum is formed in fp64 and rounded once (the
    reference's ``tl.sum`` order is unspecified, so the sum is tolerance-level).
    """
    bh = dout.shape[0] * dout.shape[1] if dout.ndim == 4 else dout.shape[0]
    n, d = dout.shape[-2], dout.shape[-1]
    prod = dout.reshape(bh, n, d).float() * out.reshape(bh, n, d).float()
    return prod.double().sum(-1).float()


def sage_backward(q, k, v, out, lse, dout, sm_scale=None, qk="int8", smooth=True,
                  block_mask=None, doc_ids=None, head_chunk=4):
    """dQ, dK, dV (bf16 ``[B, H, N, D]``) of the Sage attention backward.

    Follows sage_attn_backward_masked (sage_attention.py:534-648) and the
    unmasked sage_attn_backward (:344-458); kernel lines below are those of
    the tile-masked int8 kernels in sage_kernels.py:
      * K is smoothed again (sage_attention.py:376 / :574) and Q, K quantized
        per token exactly as in the forward (:1564-1567 / :1655-1658; the fp8
        kernels the same formulas with 448, :415-418), Q's scale carrying
        ``sm_scale*log2(e)``.
      * ``s = (acc*qd)*kd`` with keys past N at -inf (:1571-1572);
        ``p = 2^(s - lse)`` from the forward's base-2 LSE (:1577); rows past N
        give p = 0 (:1578).  Tile-masked (query tile, key tile) pairs are
        skipped, so p = 0 there (:1553, :1679); ``doc_ids`` applies the exact
        per-token visibility instead (p = 0 where hidden).
      * ``D = rowsum(dO * O)`` (:321-349); ``dP = dO @ V^T`` (fp32 accumulation
        of bf16 operands, :1588); ``dS = P * (dP - D)`` (:1591).
      * ``dV = bf16(P)^T @ dO`` (:1595), ``dK = bf16(dS * sm_scale)^T @ Q``
        (:1592, :1599, Q the raw bf16 input), ``dQ = (bf16(dS) @ K~) * sm_scale``
        (:1717, :1720, K~ the smoothed bf16 K), each rounded once to bf16.
    Products are evaluated in fp64 from the bf16-rounded operands (fp32 in the
    kernels: the difference is accumulation order only).

    A row whose LSE is -inf (nothing visible in the forward) gets p = 0; the
    reference would produce NaN there, and its tile masks never make one.
    """
    b, h, n, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    qz = quantize_all(q, k, v, sm_scale, qk, "bf16", "token", smooth)
    bh = b * h
    qf = q.reshape(bh, n, d)
    vf = v.reshape(bh, n, d)
    dof = dout.reshape(bh, n, d)
    delta = delta_prepass(dout, out)
    sm = _f32(sm_scale)
    dqs, dks, dvs = [], [], []
    for h0 in range(0, bh, head_chunk):
        sel = slice(h0, min(h0 + head_chunk, bh))
        s = scores(qz, qk, "token", sel)
        vis = None
        if block_mask is not None:
            vm = block_mask
            if vm.ndim == 3:
                vm = vm[sel]
            vis = tile_mask_visibility(vm, s.shape[0], n)
        if doc_ids is not None:
            bidx = torch.arange(sel.start, sel.stop) // h
            dv_ = doc_visibility(doc_ids.to(torch.int64))[bidx]
            vis = dv_ if vis is None else (vis & dv_)
        ls = lse[sel][:, :, None]
        live = torch.isfinite(ls)
        p = torch.exp2(s - torch.where(live, ls, torch.zeros(())))
        p = torch.where(live, p, torch.zeros(()))
        if vis is not None:
            p = torch.where(vis, p, torch.zeros(()))
        do_ = dof[sel]
        dp = torch.matmul(do_.double(), vf[sel].double().transpose(1, 2)).float()
        ds = p * (dp - delta[sel][:, :, None])
        pb = p.to(torch.bfloat16).double()
        dvs.append(torch.matmul(pb.transpose(1, 2), do_.double()).to(torch.bfloat16))
        dsk = (ds * sm).to(torch.bfloat16).double()
        dks.append(torch.matmul(dsk.transpose(1, 2), qf[sel].double()).to(torch.bfloat16))
        dsq = ds.to(torch.bfloat16).double()
        dq = torch.matmul(dsq, qz.k_smoothed[sel].double()).float() * sm
        dqs.append(dq.to(torch.bfloat16))
    shape = (b, h, n, d)
    return torch.cat(dqs).view(shape), torch.cat(dks).view(shape), torch.cat(dvs).view(shape)


def make_inputs(b, h, n, d, seed=0, k_offset_std=2.0):
    """Seeded inputs of the benchmark distribution: q, k, v ~ N(0,1) bf16 and a
    per-(b, h, channel) K offset ~ N(0, std=k_offset_std) added before the bf16 cast."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, n, d, generator=g)
    k = torch.randn(b, h, n, d, generator=g) + k_offset_std * torch.randn(b, h, 1, d, generator=g)
    v = torch.randn(b, h, n, d, generator=g)
    return q.bfloat16(), k.bfloat16(), v.bfloat16()


def cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double().flatten()
    b = b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()).clamp_min(1e-300))
