"""SageAttention forward and backward on MI355X: host-side mirror of the reference API.

Mirrors ``src/futudiffu/sage_attention.py`` of sqcu/futudiffu (function names,
argument meaning and error behaviour) on top of the gfx950 HIP library
``libsage_mi355x.so``:

* ``configure_sage`` / module defaults     -> sage_attention.py:32-60
* ``sage_attn_forward``                    -> :121-180
* ``sage_attn_forward_masked``             -> :183-268
* ``sage_attn_forward_with_lse``           -> :271-341
* ``sage_attn_forward_masked_with_lse``    -> :461-531
* ``sage_attn_backward``                   -> :344-458
* ``sage_attn_backward_masked``            -> :534-648
* ``sage_attn_op`` (``futudiffu::sage_attn``) and ``sage_attn_masked_op``
  (``futudiffu::sage_attn_masked``), with autograd -> :664-690, :740-769

Each call runs two kernels on the current stream: ``sage_quantize_qkv``
(K smoothing + Q/K/V quantization) and ``sage_attn_fwd``.  All outputs and
temporaries are allocated through the PyTorch caching allocator; nothing
synchronizes the host.  Variant choice (qk int8/fp8, pv bf16/fp8, scale
granularity, smoothing, exact doc-id masking) is also available as explicit
keyword arguments of :func:`sage_forward`, which the module-level
configuration only supplies defaults for.

Differences from the reference, all deliberate:
* head_dim 64 is accepted as well as 128 (reference asserts 128,
  sage_attention.py:487);
* ``pv="fp8"`` honours ``qk`` (the reference's unmasked LSE path always uses
  fp8 QK with fp8 PV, sage_attention.py:316-323), so int8-QK/fp8-PV exists;
* rows that see no key return 0 and LSE = -inf instead of NaN.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _lib

_LOG2E = math.log2(math.e)

_SAGE_SMOOTH_K = True
_SAGE_QK_QUANT = "fp8"
_SAGE_PV_QUANT = "bf16"

_QK = {"int8": 0, "fp8": 1}
_PV = {"bf16": 0, "fp8": 1}
_GRAN = {"token": 0, "block64": 1}
# Output layouts: "bhnd" is the reference op's [B, H, N, D]; "bnhd" is
# [B, N, H*D], the out-projection input JointAttention builds with
# out.transpose(1, 2).reshape(b, -1, H*D) (transformer.py:471)
_LAYOUT = {"bhnd": 0, "bnhd": 1}


def configure_sage(*, smooth_k: bool = True, qk_quant: str = "fp8", pv_quant: str = "bf16") -> None:
    """Select the defaults used by the no-keyword entry points (sage_attention.py:37-60)."""
    global _SAGE_SMOOTH_K, _SAGE_QK_QUANT, _SAGE_PV_QUANT
    if qk_quant not in ("fp8", "int8"):
        raise ValueError(f"Unknown qk_quant: {qk_quant!r}")
    if pv_quant not in ("bf16", "fp8"):
        raise ValueError(f"Unknown pv_quant: {pv_quant!r}")
    _SAGE_SMOOTH_K = smooth_k
    _SAGE_QK_QUANT = qk_quant
    _SAGE_PV_QUANT = pv_quant


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_inputs(q: Tensor, k: Tensor, v: Tensor) -> tuple[int, int, int, int]:
    if q.ndim != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one [B, H, N, D] shape, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, H, N, D = q.shape
    assert D in (64, 128), f"SageAttention on MI355X requires head_dim 64 or 128, got {D}"
    for name, t in (("q", q), ("k", k), ("v", v)):
        assert t.dtype == torch.bfloat16, f"Expected BF16 input, got {t.dtype} for {name}"
        if not t.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor (device {t.device})")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on one device")
    return B, H, N, D


@dataclass
class SageQuantized:
    """Device tensors produced by ``sage_quantize_qkv`` (fragment storage order)."""
    q_codes: Tensor       # uint8 [BH, Np*D]
    q_scale: Tensor       # fp32 [BH, Np] or [BH, Np/64]
    k_codes: Tensor
    k_scale: Tensor
    v_op: Tensor          # fp8 codes (uint8 [BH, Np*D]) or bf16 fragments ([BH, Np*D])
    v_scale: Tensor | None
    k_mean: Tensor | None  # bf16 [BH, D]
    qk: str
    pv: str
    granularity: str
    n: int
    np_: int
    d: int


def _quant_outputs(BH: int, N: int, D: int, qk: str, pv: str, granularity: str, smooth_k: bool, dev):
    """Device buffers of one quantization call (codes in fragment order, scales, mean, workspace)."""
    if qk not in _QK or pv not in _PV or granularity not in _GRAN:
        raise ValueError(f"bad variant qk={qk!r} pv={pv!r} granularity={granularity!r}")
    lib = _lib.load()
    Np = int(lib.sage_padded_len(N))
    ns = Np if granularity == "token" else Np // 64
    qc = torch.empty(BH, Np * D, dtype=torch.uint8, device=dev)
    kc = torch.empty_like(qc)
    qs = torch.empty(BH, ns, dtype=torch.float32, device=dev)
    ks = torch.empty_like(qs)
    if pv == "fp8":
        vop = torch.empty(BH, Np * D, dtype=torch.uint8, device=dev)
        vs = torch.empty(BH, Np // 64, D, dtype=torch.float32, device=dev)
    else:
        vop = torch.empty(BH, Np * D, dtype=torch.bfloat16, device=dev)
        vs = None
    km = torch.empty(BH, D, dtype=torch.bfloat16, device=dev) if smooth_k else None
    wsb = int(lib.sage_quant_workspace_bytes(BH, N, D)) if smooth_k else 0
    ws = torch.empty(max(wsb, 16), dtype=torch.uint8, device=dev) if smooth_k else None
    qz = SageQuantized(qc, qs, kc, ks, vop, vs, km, qk, pv, granularity, N, Np, D)
    return qz, ws, wsb


def _fold(sm_scale: float) -> float:
    """``sm_scale*log2(e)`` as the fp32 the kernels receive (sage_attention.py:493-495)."""
    return float(torch.tensor(sm_scale * _LOG2E, dtype=torch.float32))


def quantize_qkv(q: Tensor, k: Tensor, v: Tensor, sm_scale: float | None = None, *,
                 qk: str = "int8", pv: str = "bf16", granularity: str = "token",
                 smooth_k: bool = True) -> SageQuantized:
    """Smoothing + quantization of q, k, v (``[B, H, N, D]`` bf16) on the GPU."""
    B, H, N, D = _check_inputs(q, k, v)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    BH = B * H
    dev = q.device
    qz, ws, wsb = _quant_outputs(BH, N, D, qk, pv, granularity, smooth_k, dev)
    q3, k3, v3 = (t.reshape(BH, N, D).contiguous() for t in (q, k, v))
    lib = _lib.load()
    _lib.check(lib.sage_quantize_qkv(
        q3.data_ptr(), k3.data_ptr(), v3.data_ptr(), BH, N, D,
        _QK[qk], _PV[pv], _GRAN[granularity], int(smooth_k), _fold(sm_scale),
        qz.q_codes.data_ptr(), qz.q_scale.data_ptr(), qz.k_codes.data_ptr(), qz.k_scale.data_ptr(),
        qz.v_op.data_ptr(), _ptr(qz.v_scale), _ptr(qz.k_mean), _ptr(ws), wsb, _stream_handle(dev)))
    return qz


def _check_producer(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                    n_heads: int, head_dim: int):
    """Validation of fused_qkv_postprocess's inputs (fused_kernels.py:415-440) and
    their device forms: fp32 weights, rotary matrices as ``[B*N, D/2, 2, 2]``."""
    assert qkv.ndim == 3, f"Expected qkv to be 3D (B, seq, 3*dim), got {qkv.ndim}D"
    assert qkv.is_contiguous(), "QKV must be contiguous"
    B, N, total = qkv.shape
    dim = n_heads * head_dim
    assert total == 3 * dim, f"QKV last dim {total} != 3 * {dim}"
    assert head_dim in (64, 128), f"SageAttention on MI355X requires head_dim 64 or 128, got {head_dim}"
    assert qkv.dtype == torch.bfloat16, f"Expected BF16 input, got {qkv.dtype} for qkv"
    if not qkv.is_cuda:
        raise ValueError(f"qkv must be a GPU tensor (device {qkv.device})")
    assert q_norm_weight.shape == (head_dim,), f"q_norm shape {q_norm_weight.shape} != ({head_dim},)"
    assert k_norm_weight.shape == (head_dim,), f"k_norm shape {k_norm_weight.shape} != ({head_dim},)"
    n_pairs = head_dim // 2
    if freqs_cis.ndim == 6:
        assert freqs_cis.shape[2] == 1, f"Expected freqs_cis dim 2 to be 1, got {freqs_cis.shape[2]}"
        freqs_cis = freqs_cis.squeeze(2)
    elif freqs_cis.ndim != 5:
        raise ValueError(f"Unexpected freqs_cis ndim: {freqs_cis.ndim}, shape: {tuple(freqs_cis.shape)}")
    fr = freqs_cis.reshape(B * N, n_pairs, 2, 2).to(device=qkv.device, dtype=torch.float32).contiguous()
    qw = q_norm_weight.to(device=qkv.device, dtype=torch.float32).contiguous()
    kw = k_norm_weight.to(device=qkv.device, dtype=torch.float32).contiguous()
    return B, N, qw, kw, fr


def qkv_postprocess(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                    n_heads: int, head_dim: int, norm_eps: float = 1e-5) -> tuple[Tensor, Tensor, Tensor]:
    """QKV split + per-head RMSNorm + Flux RoPE + transpose on the GPU: bf16
    ``q, k, v`` ``[B, H, N, D]`` from the projection output ``[B, N, 3*H*D]``
    (fused_qkv_postprocess, fused_kernels.py:271-390)."""
    B, N, qw, kw, fr = _check_producer(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim)
    out = [torch.empty(B, n_heads, N, head_dim, dtype=torch.bfloat16, device=qkv.device) for _ in range(3)]
    lib = _lib.load()
    _lib.check(lib.sage_qkv_postprocess(
        qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), fr.data_ptr(), B, n_heads, N, head_dim, float(norm_eps),
        out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), _stream_handle(qkv.device)))
    return out[0], out[1], out[2]


def qkv_postprocess_backward(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                             grad_q: Tensor, grad_k: Tensor, grad_v: Tensor, n_heads: int, head_dim: int,
                             norm_eps: float = 1e-5) -> Tensor:
    """Gradient of ``qkv_postprocess`` with respect to ``qkv`` (bf16
    ``[B, N, 3*H*D]``), given the gradients of its outputs ``[B, H, N, D]``:
    the reference's analytical backward (fused_kernels.py:711-783) on the GPU."""
    shape = (qkv.shape[0], n_heads, qkv.shape[1], head_dim)
    for name, g in (("grad_q", grad_q), ("grad_k", grad_k), ("grad_v", grad_v)):
        if tuple(g.shape) != shape:
            raise ValueError(f"{name} must be {list(shape)}, got {tuple(g.shape)}")
    B, N, qw, kw, fr = _check_producer(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim)
    gs = [g.to(device=qkv.device, dtype=torch.bfloat16).contiguous() for g in (grad_q, grad_k, grad_v)]
    dqkv = torch.empty_like(qkv)
    lib = _lib.load()
    _lib.check(lib.sage_qkv_postprocess_bwd(
        qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), fr.data_ptr(), gs[0].data_ptr(), gs[1].data_ptr(),
        gs[2].data_ptr(), B, n_heads, N, head_dim, float(norm_eps), dqkv.data_ptr(), _stream_handle(qkv.device)))
    return dqkv


def quantize_from_qkv(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                      n_heads: int, head_dim: int, norm_eps: float = 1e-5, sm_scale: float | None = None, *,
                      qk: str = "int8", pv: str = "bf16", granularity: str = "token",
                      smooth_k: bool = True) -> SageQuantized:
    """The quantized operands of ``qkv_postprocess``'s q, k, v, straight from the
    projection output: the producer (RMSNorm + RoPE) runs inside the
    quantization kernels, so the bf16 q, k, v never reach HBM.  Bit-identical
    to ``quantize_qkv(*qkv_postprocess(...))``."""
    B, N, qw, kw, fr = _check_producer(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim)
    D = head_dim
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    BH = B * n_heads
    dev = qkv.device
    qz, ws, wsb = _quant_outputs(BH, N, D, qk, pv, granularity, smooth_k, dev)
    lib = _lib.load()
    _lib.check(lib.sage_quantize_from_qkv(
        qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), fr.data_ptr(), B, n_heads, N, D, float(norm_eps),
        _QK[qk], _PV[pv], _GRAN[granularity], int(smooth_k), _fold(sm_scale),
        qz.q_codes.data_ptr(), qz.q_scale.data_ptr(), qz.k_codes.data_ptr(), qz.k_scale.data_ptr(),
        qz.v_op.data_ptr(), _ptr(qz.v_scale), _ptr(qz.k_mean), _ptr(ws), wsb, _stream_handle(dev)))
    return qz


def _norm_mask(block_mask: Tensor | None, BH: int, N: int, device) -> tuple[Tensor | None, int, int, int]:
    if block_mask is None:
        return None, 0, 0, 0
    bm = block_mask
    if bm.dtype != torch.uint8:
        bm = bm.to(torch.uint8)
    bm = bm.to(device).contiguous()
    if bm.ndim == 2:
        stride_z = 0
        nq, nkv = bm.shape
    elif bm.ndim == 3:
        if bm.shape[0] != BH:
            raise ValueError(f"3D block_mask must have B*H={BH} rows, got {bm.shape[0]}")
        nq, nkv = bm.shape[1], bm.shape[2]
        stride_z = nq * nkv
    else:
        raise ValueError(f"block_mask must be 2D or 3D, got {bm.ndim}D")
    return bm, stride_z, nq, nkv


def attn_from_quantized(qz: SageQuantized, B: int, H: int, *, block_mask: Tensor | None = None,
                        doc_ids: Tensor | None = None, out: Tensor | None = None,
                        lse: Tensor | None = None, out_layout: str = "bhnd") -> tuple[Tensor, Tensor]:
    """Run the fused attention kernel on quantized operands; returns (out, lse).

    ``out`` is ``[B, H, N, D]`` for ``out_layout="bhnd"`` and ``[B, N, H*D]``
    for ``"bnhd"`` (same values, written in the out-projection's layout).
    """
    if out_layout not in _LAYOUT:
        raise ValueError(f"out_layout must be one of {sorted(_LAYOUT)}, got {out_layout!r}")
    lib = _lib.load()
    BH, N, D = B * H, qz.n, qz.d
    dev = qz.q_codes.device
    out_shape = (B, H, N, D) if out_layout == "bhnd" else (B, N, H * D)
    bm, stride_z, nq, nkv = _norm_mask(block_mask, BH, N, dev)
    if doc_ids is not None:
        if doc_ids.shape != (B, N):
            raise ValueError(f"doc_ids must be [B, N] = [{B}, {N}], got {tuple(doc_ids.shape)}")
        doc_ids = doc_ids.to(device=dev, dtype=torch.int32).contiguous()
    if bm is None and doc_ids is None:
        wsb = int(lib.sage_attn_workspace_bytes(B, H, N, D))
    else:
        wsb = int(lib.sage_attn_masked_workspace_bytes(B, H, N, D))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    if out is None:
        out = torch.empty(out_shape, dtype=torch.bfloat16, device=dev)
    elif (tuple(out.shape) != out_shape or out.dtype != torch.bfloat16 or not out.is_contiguous()
          or out.device != dev):
        raise ValueError(f"out must be a contiguous bf16 {list(out_shape)} tensor on {dev}")
    if lse is None:
        lse = torch.empty(BH, N, dtype=torch.float32, device=dev)
    elif tuple(lse.shape) != (BH, N) or lse.dtype != torch.float32 or not lse.is_contiguous() or lse.device != dev:
        raise ValueError(f"lse must be a contiguous fp32 [{BH}, {N}] tensor on {dev}")
    _lib.check(lib.sage_attn_fwd(
        qz.q_codes.data_ptr(), qz.q_scale.data_ptr(), qz.k_codes.data_ptr(), qz.k_scale.data_ptr(),
        qz.v_op.data_ptr(), _ptr(qz.v_scale), B, H, N, D, _QK[qz.qk], _PV[qz.pv], _GRAN[qz.granularity],
        _ptr(bm), stride_z, nq, nkv, _ptr(doc_ids), _ptr(ws), wsb, out.data_ptr(), _LAYOUT[out_layout],
        lse.data_ptr(), _stream_handle(dev)))
    return out, lse


def sage_forward(q: Tensor, k: Tensor, v: Tensor, sm_scale: float | None = None, *,
                 block_mask: Tensor | None = None, doc_ids: Tensor | None = None,
                 qk: str | None = None, pv: str | None = None, granularity: str = "token",
                 smooth_k: bool | None = None, out_layout: str = "bhnd") -> tuple[Tensor, Tensor]:
    """Sage forward with explicit variant selection; returns ``(out, lse [B*H,N])``.

    ``out`` is ``[B, H, N, D]`` (``out_layout="bhnd"``, the reference op's
    output) or ``[B, N, H*D]`` (``"bnhd"``, the out-projection's input).
    """
    B, H, N, D = _check_inputs(q, k, v)
    qk = _SAGE_QK_QUANT if qk is None else qk
    pv = _SAGE_PV_QUANT if pv is None else pv
    smooth_k = _SAGE_SMOOTH_K if smooth_k is None else smooth_k
    if qk not in _QK:
        raise ValueError(f"Unknown qk_quant: {qk!r}")
    if pv not in _PV:
        raise ValueError(f"Unknown pv_quant: {pv!r}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    if out_layout not in _LAYOUT:
        raise ValueError(f"out_layout must be one of {sorted(_LAYOUT)}, got {out_layout!r}")
    qz = quantize_qkv(q, k, v, sm_scale, qk=qk, pv=pv, granularity=granularity, smooth_k=smooth_k)
    return attn_from_quantized(qz, B, H, block_mask=block_mask, doc_ids=doc_ids, out_layout=out_layout)


def sage_forward_from_qkv(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                          n_heads: int, head_dim: int, norm_eps: float = 1e-5, sm_scale: float | None = None, *,
                          block_mask: Tensor | None = None, doc_ids: Tensor | None = None, qk: str = "int8",
                          pv: str = "bf16", granularity: str = "token", smooth_k: bool = True,
                          out_layout: str = "bnhd") -> tuple[Tensor, Tensor]:
    """JointAttention's attention from the QKV projection output
    (transformer.py:459-471): producer, quantization and attention, returning
    ``out`` in ``[B, N, H*D]`` (``out_layout="bnhd"``, the out-projection input)
    or ``[B, H, N, D]``, and ``lse`` ``[B*H, N]``."""
    if out_layout not in _LAYOUT:
        raise ValueError(f"out_layout must be one of {sorted(_LAYOUT)}, got {out_layout!r}")
    qz = quantize_from_qkv(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim, norm_eps, sm_scale,
                           qk=qk, pv=pv, granularity=granularity, smooth_k=smooth_k)
    return attn_from_quantized(qz, qkv.shape[0], n_heads, block_mask=block_mask, doc_ids=doc_ids,
                               out_layout=out_layout)


def sage_attn_forward(q: Tensor, k: Tensor, v: Tensor, sm_scale: float | None = None) -> Tensor:
    """Forward without LSE using the configured QK quantization (sage_attention.py:121-180).

    Like the reference, this legacy entry point always uses bf16 PV.
    """
    return sage_forward(q, k, v, sm_scale, pv="bf16")[0]


def sage_attn_forward_masked(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                             sm_scale: float | None = None) -> Tensor:
    """Block-masked forward without LSE, bf16 PV (sage_attention.py:183-268)."""
    return sage_forward(q, k, v, sm_scale, block_mask=block_mask, pv="bf16")[0]


def sage_attn_forward_with_lse(q: Tensor, k: Tensor, v: Tensor,
                               sm_scale: float | None = None) -> tuple[Tensor, Tensor]:
    """Forward returning (out, lse) with the configured QK and PV (sage_attention.py:271-341)."""
    return sage_forward(q, k, v, sm_scale)


def sage_attn_forward_masked_with_lse(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                                      sm_scale: float | None = None, *, qk: str = "int8",
                                      pv: str = "bf16", granularity: str = "token",
                                      doc_ids: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """Masked forward with LSE; int8 QK / bf16 PV by default like the production kernel
    (sage_attention.py:461-531, hard-wired at :521-529)."""
    return sage_forward(q, k, v, sm_scale, block_mask=block_mask, doc_ids=doc_ids, qk=qk, pv=pv,
                        granularity=granularity)


def sage_attn_forward_masked_merged_heads(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                                          sm_scale: float | None = None, *, qk: str = "int8",
                                          pv: str = "bf16", granularity: str = "token",
                                          doc_ids: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """``sage_attn_forward_masked_with_lse`` with the output in ``[B, N, H*D]``.

    Bit-identical to ``out.transpose(1, 2).reshape(B, N, H*D)`` of the masked
    forward, which JointAttention.forward computes before its out-projection
    (transformer.py:467-471); the kernel writes that layout directly, so the
    transpose copy disappears.
    """
    return sage_forward(q, k, v, sm_scale, block_mask=block_mask, doc_ids=doc_ids, qk=qk, pv=pv,
                        granularity=granularity, out_layout="bnhd")


def sage_backward(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, dout: Tensor,
                  sm_scale: float | None = None, *, block_mask: Tensor | None = None,
                  doc_ids: Tensor | None = None, qk: str | None = None,
                  smooth_k: bool | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """dQ, dK, dV (bf16 ``[B, H, N, D]``) with explicit variant selection.

    P is recomputed from per-token Q / K codes (K smoothed again when
    ``smooth_k``) and the forward's base-2 ``lse``; ``smooth_k``, the mask and
    ``doc_ids`` must be the forward's.  Runs the quantization, the T-image and
    D pre-pass kernels, then the dK/dV and dQ kernels (sage_kernels.py:321-349,
    :805-1030, :1491-1722) on the current stream.
    """
    B, H, N, D = _check_inputs(q, k, v)
    qk = _SAGE_QK_QUANT if qk is None else qk
    smooth_k = _SAGE_SMOOTH_K if smooth_k is None else smooth_k
    if qk not in _QK:
        raise ValueError(f"Unknown qk_quant: {qk!r}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    dev = q.device
    for name, t in (("out", out), ("dout", dout)):
        if tuple(t.shape) != (B, H, N, D) or t.dtype != torch.bfloat16 or t.device != dev:
            raise ValueError(f"{name} must be a bf16 [{B}, {H}, {N}, {D}] tensor on {dev}")
    if tuple(lse.shape) != (B * H, N) or lse.dtype != torch.float32 or lse.device != dev:
        raise ValueError(f"lse must be an fp32 [{B * H}, {N}] tensor on {dev}")
    q, k, v, out, dout, lse = (t.contiguous() for t in (q, k, v, out, dout, lse))
    lib = _lib.load()
    BH = B * H
    bm, stride_z, nq, nkv = _norm_mask(block_mask, BH, N, dev)
    if doc_ids is not None:
        if doc_ids.shape != (B, N):
            raise ValueError(f"doc_ids must be [B, N] = [{B}, {N}], got {tuple(doc_ids.shape)}")
        doc_ids = doc_ids.to(device=dev, dtype=torch.int32).contiguous()
    wsb = int(lib.sage_attn_bwd_workspace_bytes(B, H, N, D))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    _lib.check(lib.sage_attn_bwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lse.data_ptr(), dout.data_ptr(),
        B, H, N, D, _QK[qk], int(bool(smooth_k)), float(sm_scale), _fold(sm_scale), _ptr(bm), stride_z, nq, nkv,
        _ptr(doc_ids), ws.data_ptr(), wsb, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), _stream_handle(dev)))
    return dq, dk, dv


def sage_attn_backward(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, dout: Tensor,
                       sm_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    """Backward of the unmasked forward with the configured QK quantization
    and smoothing (sage_attention.py:344-458: int8 kernels when qk_quant is
    "int8", the fp8 kernels otherwise)."""
    return sage_backward(q, k, v, out, lse, dout, sm_scale)


def sage_attn_backward_masked(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, dout: Tensor,
                              block_mask: Tensor, sm_scale: float, *,
                              doc_ids: Tensor | None = None) -> tuple[Tensor, Tensor, Tensor]:
    """Backward of the block-masked forward: int8 P recomputation whatever the
    configured QK quantization, configured smoothing (sage_attention.py:534-648)."""
    return sage_backward(q, k, v, out, lse, dout, sm_scale, block_mask=block_mask, doc_ids=doc_ids, qk="int8")


def qk_accumulators(qz: SageQuantized, B: int, H: int) -> tuple[Tensor, Tensor, Tensor]:
    """The attention forward (per-token scales, no mask) on quantized
    operands, plus the QK^T accumulators its own loop formed.

    Returns ``(out, lse, s)`` with ``s`` ``[B*H, Np, Np]`` (row = query,
    column = key): the result of ``tl.dot(q, k)`` before dequantization
    (int8 sage_kernels.py:1451, int32; fp8 :282, float32) as the kernel's
    pipelined loop consumed it, tile by tile.  Entries past ``32*ceil(N/32)``
    rows or ``64*ceil(N/64)`` keys stay zero.  Codes quantized with
    per-64-token scales run with those scales repeated per token (the
    accumulators depend on the codes only).
    """
    lib = _lib.load()
    BH, N, D = B * H, qz.n, qz.d
    dev = qz.q_codes.device
    qs, ks = qz.q_scale, qz.k_scale
    if qz.granularity == "block64":
        qs, ks = (t.repeat_interleave(64, dim=1).contiguous() for t in (qs, ks))
    wsb = int(lib.sage_attn_workspace_bytes(B, H, N, D))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    out = torch.empty(B, H, N, D, dtype=torch.bfloat16, device=dev)
    lse = torch.empty(BH, N, dtype=torch.float32, device=dev)
    s = torch.zeros(BH, qz.np_, qz.np_, dtype=torch.int32, device=dev)
    _lib.check(lib.sage_attn_qk_accumulators(
        qz.q_codes.data_ptr(), qs.data_ptr(), qz.k_codes.data_ptr(), ks.data_ptr(),
        qz.v_op.data_ptr(), _ptr(qz.v_scale), B, H, N, D, _QK[qz.qk], _PV[qz.pv], ws.data_ptr(), wsb,
        out.data_ptr(), lse.data_ptr(), s.data_ptr(), _stream_handle(dev)))
    return out, lse, (s if qz.qk == "int8" else s.view(torch.float32))


# ---- legacy ops (sage_attention.py:664-690, :740-769) ----------------------------------
#
# The reference registers these two ops in this module, and its legacy router
# imports them from here: attention.py:101-103 calls sage_attn_op for
# unmasked attention, :77-79 calls sage_attn_forward_masked for a uint8 block
# mask.  Same names, schemas, fake implementations (contiguous [B, H, N, D]
# output, [B*H, N] fp32 LSE) and autograd formulas.  The backward runs with
# the variant the forward ran with (the reference reads the module
# configuration again when its backward runs, :374-376, :413).

@torch.library.custom_op("futudiffu::sage_attn", mutates_args=())
def sage_attn_op(q: Tensor, k: Tensor, v: Tensor, sm_scale: float) -> tuple[Tensor, Tensor]:
    """SageAttention forward with the configured variant: returns (out, lse)."""
    return sage_attn_forward_with_lse(q, k, v, sm_scale)


@sage_attn_op.register_fake
def _sage_attn_op_fake(q, k, v, sm_scale):
    B, H, N, D = q.shape
    return q.new_empty(B, H, N, D), q.new_empty(B * H, N, dtype=torch.float32)


def _legacy_setup_context(ctx, inputs, output):
    q, k, v, sm_scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse)
    ctx.sm_scale = sm_scale
    ctx.qk = _SAGE_QK_QUANT
    ctx.smooth_k = _SAGE_SMOOTH_K


def _legacy_backward(ctx, grad_out, grad_lse):
    q, k, v, out, lse = ctx.saved_tensors
    dq, dk, dv = sage_backward(q, k, v, out, lse, grad_out.contiguous(), ctx.sm_scale, qk=ctx.qk,
                               smooth_k=ctx.smooth_k)
    return dq, dk, dv, None


sage_attn_op.register_autograd(_legacy_backward, setup_context=_legacy_setup_context)


@torch.library.custom_op("futudiffu::sage_attn_masked", mutates_args=())
def sage_attn_masked_op(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                        sm_scale: float) -> tuple[Tensor, Tensor]:
    """Block-masked SageAttention forward (int8 QK, bf16 PV): returns (out, lse)."""
    return sage_attn_forward_masked_with_lse(q, k, v, block_mask, sm_scale)


@sage_attn_masked_op.register_fake
def _sage_attn_masked_op_fake(q, k, v, block_mask, sm_scale):
    B, H, N, D = q.shape
    return q.new_empty(B, H, N, D), q.new_empty(B * H, N, dtype=torch.float32)


def _legacy_masked_setup_context(ctx, inputs, output):
    q, k, v, block_mask, sm_scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, block_mask)
    ctx.sm_scale = sm_scale
    ctx.smooth_k = _SAGE_SMOOTH_K


def _legacy_masked_backward(ctx, grad_out, grad_lse):
    q, k, v, out, lse, block_mask = ctx.saved_tensors
    dq, dk, dv = sage_backward(q, k, v, out, lse, grad_out.contiguous(), ctx.sm_scale, block_mask=block_mask,
                               qk="int8", smooth_k=ctx.smooth_k)
    return dq, dk, dv, None, None


sage_attn_masked_op.register_autograd(_legacy_masked_backward, setup_context=_legacy_masked_setup_context)
