"""Drop-in registration of ``futudiffu::fused_qkv_postprocess`` on MI355X.

Registers the op name, schema and fake implementation of
``src/futudiffu/fused_kernels.py:613-643`` (sqcu/futudiffu) over the gfx950
producer kernel (``sage_qkv_postprocess``): QKV split + per-head RMSNorm +
Flux RoPE + transpose, bf16 ``q, k, v`` ``[B, H, N, D]``.  Import this module
instead of the reference's ``futudiffu.fused_kernels`` (both register the same
name).  Its autograd formula is the reference's analytical backward
(:711-783) on the GPU: the gradient with respect to ``qkv`` only.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .sage_attention import qkv_postprocess, qkv_postprocess_backward


@torch.library.custom_op("futudiffu::fused_qkv_postprocess", mutates_args=())
def fused_qkv_postprocess(qkv: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, freqs_cis: Tensor,
                          n_heads: int, head_dim: int, norm_eps: float = 1e-5) -> tuple[Tensor, Tensor, Tensor]:
    q, k, v = qkv_postprocess(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim, norm_eps)
    return q, k, v


@fused_qkv_postprocess.register_fake
def _fake(qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim, norm_eps=1e-5):
    B, seq_len = qkv.shape[0], qkv.shape[1]
    return tuple(qkv.new_empty(B, n_heads, seq_len, head_dim) for _ in range(3))


def _setup(ctx, inputs, output):
    qkv, q_norm_weight, k_norm_weight, freqs_cis, n_heads, head_dim, norm_eps = inputs
    ctx.save_for_backward(qkv, q_norm_weight, k_norm_weight, freqs_cis)
    ctx.args = (n_heads, head_dim, norm_eps)


def _backward(ctx, grad_q, grad_k, grad_v):
    qkv, qw, kw, freqs = ctx.saved_tensors
    n_heads, head_dim, norm_eps = ctx.args
    dqkv = qkv_postprocess_backward(qkv, qw, kw, freqs, grad_q, grad_k, grad_v, n_heads, head_dim, norm_eps)
    return dqkv, None, None, None, None, None, None


fused_qkv_postprocess.register_autograd(_backward, setup_context=_setup)
