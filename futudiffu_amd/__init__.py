"""MI355X-native (gfx950) SageAttention forward and backward for sqcu/futudiffu.

Importing this package registers the ``futudiffu_ii::sage_attn_masked``,
``futudiffu_ii::sage_attn``, ``futudiffu_ii::sage_attn_ext``,
``futudiffu_ii::sage_attn_masked_merged_heads`` and
``futudiffu_ii::sage_attn_qkv_masked`` custom ops, and the backward ops
``futudiffu_ii::sage_bwd_masked``, ``futudiffu_ii::sage_bwd`` and
``futudiffu_ii::sage_bwd_ext`` their autograd formulas call.  ``futudiffu_amd.fused_kernels``
(imported separately) registers ``futudiffu::fused_qkv_postprocess``.
The compute lives in ``libsage_mi355x.so`` (HIP, built by ``build.py``).
"""

from . import attention_srcii  # noqa: F401  (registers the custom ops)
from .attention_srcii import (  # noqa: F401
    sage_attn_ext_op,
    sage_attn_masked_merged_heads_op,
    sage_attn_masked_op,
    sage_attn_qkv_masked_op,
    sage_attn_op,
    sage_bwd_ext_op,
    sage_bwd_masked_op,
    sage_bwd_op,
)
from .block_mask import build_block_mask, build_doc_ids  # noqa: F401
from .sage_attention import (  # noqa: F401
    configure_sage,
    sage_attn_backward,
    sage_attn_backward_masked,
    sage_backward,
    qkv_postprocess,
    quantize_from_qkv,
    quantize_qkv,
    sage_attn_forward,
    sage_attn_forward_masked,
    sage_attn_forward_masked_merged_heads,
    sage_attn_forward_masked_with_lse,
    sage_attn_forward_with_lse,
    sage_forward,
    sage_forward_from_qkv,
)
