"""torch.library custom ops: drop-in for src_ii/attention_srcii.py of sqcu/futudiffu.

Registers the same op names and schemas the reference registers
(src_ii/attention_srcii.py:36-48, :54-64, :91-103 and :109-119):

    futudiffu_ii::sage_attn_masked(q, k, v, block_mask, sm_scale) -> (out, lse)
    futudiffu_ii::sage_attn(q, k, v, sm_scale)                    -> (out, lse)
    futudiffu_ii::sage_bwd_masked(q, k, v, out, lse, grad_out, block_mask, sm_scale) -> (dq, dk, dv)
    futudiffu_ii::sage_bwd(q, k, v, out, lse, grad_out, sm_scale)                    -> (dq, dk, dv)

with identical fake (meta) implementations: contiguous ``[B, H, N, D]`` output
and ``[B*H, N]`` fp32 LSE, gradients shaped like their inputs.  The masked op
is int8-QK / bf16-PV like the production kernel it replaces
(sage_attention.py:521-529); the unmasked op uses the ``configure_sage``
selection (sage_attention.py:271-341).  Both forward ops carry the reference's
autograd formula (attention_srcii.py:67-84, :122-133): save q, k, v, out, lse
(and the mask) and run the backward; the LSE gradient is ignored.  The
variant the forward ran with is recorded at that time and the backward uses
it (the reference reads the module configuration again when the backward
runs).

``futudiffu_ii::sage_attn_ext`` exposes every variant as op arguments
(qk, pv, granularity, smoothing, optional tile mask, optional exact doc ids,
output layout).  ``futudiffu_ii::sage_attn_masked_merged_heads`` is
``sage_attn_masked`` with the output already in the ``[B, N, H*D]`` layout of
the out-projection that follows it (transformer.py:471).
``futudiffu_ii::sage_attn_qkv_masked`` also takes over the q/k/v producer
(fused_qkv_postprocess, transformer.py:459-463): it reads the QKV projection
output and quantizes inside the producer, so bf16 q, k, v never reach HBM.
The extension ops differentiate through ``futudiffu_ii::sage_bwd_ext``, with
the forward's variant; ``sage_attn_qkv_masked`` differentiates with respect to
``qkv`` through the attention backward and the producer's analytical backward
(fused_kernels.py:711-783).
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import sage_attention as _sa
from .sage_attention import (
    sage_attn_backward,
    sage_attn_backward_masked,
    sage_attn_forward_masked_merged_heads,
    sage_forward_from_qkv,
    sage_attn_forward_masked_with_lse,
    sage_attn_forward_with_lse,
    sage_backward,
    sage_forward,
)


def _fake_out(q: Tensor) -> tuple[Tensor, Tensor]:
    B, H, N, D = q.shape
    return q.new_empty(B, H, N, D), q.new_empty(B * H, N, dtype=torch.float32)


def _fake_grads(q: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _fake_merged_heads(q: Tensor) -> tuple[Tensor, Tensor]:
    B, H, N, D = q.shape
    return q.new_empty(B, N, H * D), q.new_empty(B * H, N, dtype=torch.float32)


def _to_bhnd(x: Tensor, shape) -> Tensor:
    """[B, N, H*D] -> contiguous [B, H, N, D]."""
    B, H, N, D = shape
    return x.view(B, N, H, D).transpose(1, 2).contiguous()


# ---- backward ops (attention_srcii.py:36-48, :91-103) -------------------------------

@torch.library.custom_op("futudiffu_ii::sage_bwd_masked", mutates_args=())
def sage_bwd_masked_op(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, grad_out: Tensor,
                       block_mask: Tensor, sm_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    return sage_attn_backward_masked(q, k, v, out, lse, grad_out, block_mask, sm_scale)


@sage_bwd_masked_op.register_fake
def _fake_bwd_masked(q, k, v, out, lse, grad_out, block_mask, sm_scale):
    return _fake_grads(q, k, v)


@torch.library.custom_op("futudiffu_ii::sage_bwd", mutates_args=())
def sage_bwd_op(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, grad_out: Tensor,
                sm_scale: float) -> tuple[Tensor, Tensor, Tensor]:
    return sage_attn_backward(q, k, v, out, lse, grad_out, sm_scale)


@sage_bwd_op.register_fake
def _fake_bwd(q, k, v, out, lse, grad_out, sm_scale):
    return _fake_grads(q, k, v)


@torch.library.custom_op("futudiffu_ii::sage_bwd_ext", mutates_args=())
def sage_bwd_ext_op(q: Tensor, k: Tensor, v: Tensor, out: Tensor, lse: Tensor, grad_out: Tensor,
                    block_mask: Tensor | None, doc_ids: Tensor | None, sm_scale: float, qk: str,
                    smooth_k: bool) -> tuple[Tensor, Tensor, Tensor]:
    return sage_backward(q, k, v, out, lse, grad_out, sm_scale, block_mask=block_mask, doc_ids=doc_ids, qk=qk,
                         smooth_k=smooth_k)


@sage_bwd_ext_op.register_fake
def _fake_bwd_ext(q, k, v, out, lse, grad_out, block_mask, doc_ids, sm_scale, qk, smooth_k):
    return _fake_grads(q, k, v)


# ---- forward ops and their autograd formulas ------------------------------------------

@torch.library.custom_op("futudiffu_ii::sage_attn_masked", mutates_args=())
def sage_attn_masked_op(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                        sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_attn_forward_masked_with_lse(q, k, v, block_mask, sm_scale)
    return out, lse


@sage_attn_masked_op.register_fake
def _fake_fwd_masked(q, k, v, block_mask, sm_scale):
    return _fake_out(q)


# The autograd formulas record the smoothing (and, unmasked, the QK
# quantization) in effect when the forward ran, and differentiate with that
# variant: the reference's backward reads the module configuration when it
# runs (sage_attention.py:374-376, :413), so a configure_sage() between forward
# and backward would recompute P with other codes than the forward used.
def _masked_setup_context(ctx, inputs, output):
    q, k, v, block_mask, sm_scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, block_mask)
    ctx.sm_scale = sm_scale
    ctx.smooth_k = _sa._SAGE_SMOOTH_K


def _masked_backward(ctx, grad_out, grad_lse):
    q, k, v, out, lse, block_mask = ctx.saved_tensors
    dq, dk, dv = sage_bwd_ext_op(q, k, v, out, lse, grad_out.contiguous(), block_mask, None, ctx.sm_scale, "int8",
                                 ctx.smooth_k)
    return dq, dk, dv, None, None


sage_attn_masked_op.register_autograd(_masked_backward, setup_context=_masked_setup_context)


@torch.library.custom_op("futudiffu_ii::sage_attn", mutates_args=())
def sage_attn_op(q: Tensor, k: Tensor, v: Tensor, sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_attn_forward_with_lse(q, k, v, sm_scale)
    return out, lse


@sage_attn_op.register_fake
def _fake_fwd(q, k, v, sm_scale):
    return _fake_out(q)


def _setup_context(ctx, inputs, output):
    q, k, v, sm_scale = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse)
    ctx.sm_scale = sm_scale
    ctx.qk = _sa._SAGE_QK_QUANT
    ctx.smooth_k = _sa._SAGE_SMOOTH_K


def _backward(ctx, grad_out, grad_lse):
    q, k, v, out, lse = ctx.saved_tensors
    dq, dk, dv = sage_bwd_ext_op(q, k, v, out, lse, grad_out.contiguous(), None, None, ctx.sm_scale, ctx.qk,
                                 ctx.smooth_k)
    return dq, dk, dv, None


sage_attn_op.register_autograd(_backward, setup_context=_setup_context)


@torch.library.custom_op("futudiffu_ii::sage_attn_ext", mutates_args=())
def sage_attn_ext_op(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor | None, doc_ids: Tensor | None,
                     sm_scale: float, qk: str, pv: str, granularity: str,
                     smooth_k: bool, out_layout: str = "bhnd") -> tuple[Tensor, Tensor]:
    out, lse = sage_forward(q, k, v, sm_scale, block_mask=block_mask, doc_ids=doc_ids, qk=qk, pv=pv,
                            granularity=granularity, smooth_k=smooth_k, out_layout=out_layout)
    return out, lse


@sage_attn_ext_op.register_fake
def _fake_ext(q, k, v, block_mask, doc_ids, sm_scale, qk, pv, granularity, smooth_k, out_layout="bhnd"):
    if out_layout == "bnhd":
        return _fake_merged_heads(q)
    return _fake_out(q)


def _ext_setup_context(ctx, inputs, output):
    q, k, v, block_mask, doc_ids, sm_scale, qk, pv, granularity, smooth_k, *rest = inputs
    out, lse = output
    ctx.save_for_backward(q, k, v, out, lse, block_mask, doc_ids)
    ctx.args = (sm_scale, qk, smooth_k, rest[0] if rest else "bhnd")
    ctx.granularity = granularity


def _ext_backward(ctx, grad_out, grad_lse):
    """The backward recomputes P from per-token Q / K codes (as the
    reference's backward kernels do, sage_kernels.py:1526-1577), which is
    the forward's P only for granularity "token": a forward with per-64-token
    scales has an LSE of other scores, so its gradient is refused."""
    if ctx.granularity != "token":
        raise ValueError(f"sage_attn_ext backward supports granularity 'token' only, the forward ran with "
                         f"{ctx.granularity!r}")
    q, k, v, out, lse, block_mask, doc_ids = ctx.saved_tensors
    sm_scale, qk, smooth_k, layout = ctx.args
    if layout == "bnhd":
        out, grad_out = _to_bhnd(out, q.shape), _to_bhnd(grad_out, q.shape)
    dq, dk, dv = sage_bwd_ext_op(q, k, v, out, lse, grad_out.contiguous(), block_mask, doc_ids, sm_scale, qk,
                                 smooth_k)
    return dq, dk, dv, None, None, None, None, None, None, None, None


sage_attn_ext_op.register_autograd(_ext_backward, setup_context=_ext_setup_context)


# JointAttention.forward (transformer.py:467-471) calls sage_attn_masked and
# then out.transpose(1, 2).reshape(b, -1, H*D) for its out-projection.  This op
# returns that [B, N, H*D] tensor directly (the kernel stores rows in that
# layout), bit-identical to the transposed output of sage_attn_masked.
@torch.library.custom_op("futudiffu_ii::sage_attn_masked_merged_heads", mutates_args=())
def sage_attn_masked_merged_heads_op(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                                     sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_attn_forward_masked_merged_heads(q, k, v, block_mask, sm_scale)
    return out, lse


@sage_attn_masked_merged_heads_op.register_fake
def _fake_fwd_merged(q, k, v, block_mask, sm_scale):
    return _fake_merged_heads(q)


def _merged_backward(ctx, grad_out, grad_lse):
    q, k, v, out, lse, block_mask = ctx.saved_tensors
    dq, dk, dv = sage_bwd_ext_op(q, k, v, _to_bhnd(out, q.shape), lse, _to_bhnd(grad_out, q.shape), block_mask,
                                 None, ctx.sm_scale, "int8", ctx.smooth_k)
    return dq, dk, dv, None, None


sage_attn_masked_merged_heads_op.register_autograd(_merged_backward, setup_context=_masked_setup_context)


# JointAttention.forward (transformer.py:459-471): fused_qkv_postprocess, then
# sage_attn_masked, then the transpose into the out-projection layout.  This
# op does all three from the QKV projection output, with the production
# kernel's variant (int8 QK, bf16 PV, sage_attention.py:521-529).
@torch.library.custom_op("futudiffu_ii::sage_attn_qkv_masked", mutates_args=())
def sage_attn_qkv_masked_op(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                            block_mask: Tensor, n_heads: int, head_dim: int, norm_eps: float,
                            sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_forward_from_qkv(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim, norm_eps,
                                     sm_scale, block_mask=block_mask, qk="int8", pv="bf16",
                                     smooth_k=_sa._SAGE_SMOOTH_K, out_layout="bnhd")
    return out, lse


@sage_attn_qkv_masked_op.register_fake
def _fake_qkv_masked(qkv, q_norm_weight, k_norm_weight, freqs_cis, block_mask, n_heads, head_dim, norm_eps,
                     sm_scale):
    B, N = qkv.shape[0], qkv.shape[1]
    return qkv.new_empty(B, N, n_heads * head_dim), qkv.new_empty(B * n_heads, N, dtype=torch.float32)


def _qkv_masked_setup(ctx, inputs, output):
    qkv, q_norm_weight, k_norm_weight, freqs_cis, block_mask, n_heads, head_dim, norm_eps, sm_scale = inputs
    out, lse = output
    ctx.save_for_backward(qkv, q_norm_weight, k_norm_weight, freqs_cis, block_mask, out, lse)
    ctx.args = (n_heads, head_dim, norm_eps, sm_scale)
    ctx.smooth_k = _sa._SAGE_SMOOTH_K


def _qkv_masked_backward(ctx, grad_out, grad_lse):
    """The producer's outputs are recomputed (bit-identical to the ones the
    fused forward quantized), then the attention backward (int8 P
    recomputation, as the forward) and the producer's backward."""
    qkv, qw, kw, freqs, block_mask, out, lse = ctx.saved_tensors
    n_heads, head_dim, norm_eps, sm_scale = ctx.args
    q, k, v = _sa.qkv_postprocess(qkv, qw, kw, freqs, n_heads, head_dim, norm_eps)
    shape = q.shape
    dq, dk, dv = sage_bwd_ext_op(q, k, v, _to_bhnd(out, shape), lse, _to_bhnd(grad_out, shape), block_mask, None,
                                 sm_scale, "int8", ctx.smooth_k)
    dqkv = _sa.qkv_postprocess_backward(qkv, qw, kw, freqs, dq, dk, dv, n_heads, head_dim, norm_eps)
    return dqkv, None, None, None, None, None, None, None, None


sage_attn_qkv_masked_op.register_autograd(_qkv_masked_backward, setup_context=_qkv_masked_setup)
