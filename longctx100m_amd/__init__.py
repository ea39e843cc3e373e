"""MI355X-native exact causal ring attention (one rank's share of longctx100m).

The compute lives in liblongctx100m_attn.so (hand-written gfx950 HIP kernels
behind the C ABI in include/longctx100m_attn.h).  ``ring_attention`` mirrors
the reference's ring-attention functions on torch GPU tensors; ``build``
compiles the library.
"""

__all__ = ["ring_attention", "build"]
