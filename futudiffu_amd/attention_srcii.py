"""torch.library custom ops: drop-in for src_ii/attention_srcii.py of sqcu/futudiffu.

Registers the same op names and schemas the reference registers
(src_ii/attention_srcii.py:54-64 and :109-119):

    futudiffu_ii::sage_attn_masked(q, k, v, block_mask, sm_scale) -> (out, lse)
    futudiffu_ii::sage_attn(q, k, v, sm_scale)                    -> (out, lse)

with identical fake (meta) implementations: contiguous ``[B, H, N, D]`` output
and ``[B*H, N]`` fp32 LSE.  The masked op is int8-QK / bf16-PV like the
production kernel it replaces (sage_attention.py:521-529); the unmasked op uses
the ``configure_sage`` selection (sage_attention.py:271-341).

``futudiffu_ii::sage_attn_ext`` exposes every variant as op arguments
(qk, pv, granularity, smoothing, optional tile mask, optional exact doc ids,
output layout).  ``futudiffu_ii::sage_attn_masked_merged_heads`` is
``sage_attn_masked`` with the output already in the ``[B, N, H*D]`` layout of
the out-projection that follows it (transformer.py:471).
``futudiffu_ii::sage_attn_qkv_masked`` also takes over the q/k/v producer
(fused_qkv_postprocess, transformer.py:459-463): it reads the QKV projection
output and quantizes inside the producer, so bf16 q, k, v never reach HBM.

Backward is not part of this forward-only build: the ops register an autograd
formula that raises, so a training graph fails loudly instead of silently
dropping gradients (the reference wires Triton backward kernels here,
attention_srcii.py:36-84).
"""

from __future__ import annotations

import torch
from torch import Tensor

from .sage_attention import (
    sage_attn_forward_masked_merged_heads,
    sage_forward_from_qkv,
    sage_attn_forward_masked_with_lse,
    sage_attn_forward_with_lse,
    sage_forward,
)


def _fake_out(q: Tensor) -> tuple[Tensor, Tensor]:
    B, H, N, D = q.shape
    return q.new_empty(B, H, N, D), q.new_empty(B * H, N, dtype=torch.float32)


def _no_backward(ctx, grad_out, grad_lse):
    raise NotImplementedError("Sage attention backward is not implemented in the MI355X build "
                              "(forward-only); run training with the reference backward kernels")


def _setup_context(ctx, inputs, output):
    pass


@torch.library.custom_op("futudiffu_ii::sage_attn_masked", mutates_args=())
def sage_attn_masked_op(q: Tensor, k: Tensor, v: Tensor, block_mask: Tensor,
                        sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_attn_forward_masked_with_lse(q, k, v, block_mask, sm_scale)
    return out, lse


@sage_attn_masked_op.register_fake
def _fake_fwd_masked(q, k, v, block_mask, sm_scale):
    return _fake_out(q)


sage_attn_masked_op.register_autograd(_no_backward, setup_context=_setup_context)


@torch.library.custom_op("futudiffu_ii::sage_attn", mutates_args=())
def sage_attn_op(q: Tensor, k: Tensor, v: Tensor, sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_attn_forward_with_lse(q, k, v, sm_scale)
    return out, lse


@sage_attn_op.register_fake
def _fake_fwd(q, k, v, sm_scale):
    return _fake_out(q)


sage_attn_op.register_autograd(_no_backward, setup_context=_setup_context)


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


sage_attn_ext_op.register_autograd(_no_backward, setup_context=_setup_context)


def _fake_merged_heads(q: Tensor) -> tuple[Tensor, Tensor]:
    B, H, N, D = q.shape
    return q.new_empty(B, N, H * D), q.new_empty(B * H, N, dtype=torch.float32)


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


sage_attn_masked_merged_heads_op.register_autograd(_no_backward, setup_context=_setup_context)


# JointAttention.forward (transformer.py:459-471): fused_qkv_postprocess, then
# sage_attn_masked, then the transpose into the out-projection layout.  This
# op does all three from the QKV projection output, with the production
# kernel's variant (int8 QK, bf16 PV, sage_attention.py:521-529).
@torch.library.custom_op("futudiffu_ii::sage_attn_qkv_masked", mutates_args=())
def sage_attn_qkv_masked_op(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                            block_mask: Tensor, n_heads: int, head_dim: int, norm_eps: float,
                            sm_scale: float) -> tuple[Tensor, Tensor]:
    out, lse = sage_forward_from_qkv(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim, norm_eps,
                                     sm_scale, block_mask=block_mask, qk="int8", pv="bf16", out_layout="bnhd")
    return out, lse


@sage_attn_qkv_masked_op.register_fake
def _fake_qkv_masked(qkv, q_norm_weight, k_norm_weight, freqs_cis, block_mask, n_heads, head_dim, norm_eps,
                     sm_scale):
    B, N = qkv.shape[0], qkv.shape[1]
    return qkv.new_empty(B, N, n_heads * head_dim), qkv.new_empty(B * n_heads, N, dtype=torch.float32)


sage_attn_qkv_masked_op.register_autograd(_no_backward, setup_context=_setup_context)
