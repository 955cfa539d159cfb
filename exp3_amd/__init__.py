"""MI355X-native sparse-prefill attention (exp3's FlashPrefill-V1 / mean-corrected path).

Modules mirror the reference's Python entry points:
  exp3_amd.attention                          AttentionBackend, METHODS
  exp3_amd.kernels                            descriptors, selectors, mean tail, merge
  exp3_amd.upstream.flashprefill_native_forward   block_mean_k, v1_scores,
                                              deal_output_score, exact_attention
All tensor work runs in gfx950 HIP kernels (exp3_amd/_C/libexp3_amd.so).
"""

from . import _lib  # noqa: F401

__all__ = ["attention", "kernels", "upstream", "synthetic"]
