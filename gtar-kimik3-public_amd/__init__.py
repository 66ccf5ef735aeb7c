"""MI355X-native chunkwise gated delta-rule attention (KDA, Gated DeltaNet, GLA, DeltaNet).

The export surface mirrors the reference's op package for this family (src/ops/__init__.py:1-6): a
`chunk_*` (prefill) and a `recurrent_*` (decode) function per variant, backed by the hand-written gfx950 HIP
kernels of libgdr.so.  `RecurrentCache` mirrors the decode-state owner of src/cache.py:48-86.  A `verify_*`
function per variant serves speculative decoding (the verify / accept cycle of src/speculative.py:344-449), and
`chunk_kimi_delta_attention_fused` takes the KDA layer's pre-op tensors (src/layers/kimi_delta_attention.py:45-49).
For the hybrid stack around the op, `flash_attention` (causal grouped-query attention, src/ops/flash_attention_2.py)
and `short_convolution` (src/layers/short_convolution.py) take packed sequences through `cu_seqlens`.
"""

from ._common import set_chunk_backward_workspace
from .attention import flash_attention
from .cache import RecurrentCache
from .conv import short_convolution
from .epilogue import output_norm_gate
from .deltanet import chunk_deltanet, recurrent_deltanet, verify_deltanet
from .fused import chunk_gated_linear_attention_fused, chunk_kimi_delta_attention_fused
from .gated_deltanet import chunk_gated_deltanet, recurrent_gated_deltanet, verify_gated_deltanet
from .gated_linear_attention import (chunk_gated_linear_attention, recurrent_gated_linear_attention,
                                     verify_gated_linear_attention)
from .kimi_delta_attention import chunk_kimi_delta_attention, recurrent_kimi_delta_attention, verify_kimi_delta_attention
from .verify import VerifiedBlock

__all__ = [
    "RecurrentCache",
    "chunk_deltanet",
    "chunk_gated_deltanet",
    "chunk_gated_linear_attention",
    "chunk_gated_linear_attention_fused",
    "chunk_kimi_delta_attention",
    "chunk_kimi_delta_attention_fused",
    "flash_attention",
    "output_norm_gate",
    "recurrent_deltanet",
    "recurrent_gated_deltanet",
    "recurrent_gated_linear_attention",
    "recurrent_kimi_delta_attention",
    "set_chunk_backward_workspace",
    "short_convolution",
    "VerifiedBlock",
    "verify_deltanet",
    "verify_gated_deltanet",
    "verify_gated_linear_attention",
    "verify_kimi_delta_attention",
]
