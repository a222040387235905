"""MI355X-native (gfx950) SageAttention forward for sqcu/futudiffu.

Importing this package registers the ``futudiffu_ii::sage_attn_masked``,
``futudiffu_ii::sage_attn`` and ``futudiffu_ii::sage_attn_ext`` custom ops.
The compute lives in ``libsage_mi355x.so`` (HIP, built by ``build.py``).
"""

from . import attention_srcii  # noqa: F401  (registers the custom ops)
from .attention_srcii import sage_attn_ext_op, sage_attn_masked_op, sage_attn_op  # noqa: F401
from .block_mask import build_block_mask, build_doc_ids  # noqa: F401
from .sage_attention import (  # noqa: F401
    configure_sage,
    quantize_qkv,
    sage_attn_forward,
    sage_attn_forward_masked,
    sage_attn_forward_masked_with_lse,
    sage_attn_forward_with_lse,
    sage_forward,
)
