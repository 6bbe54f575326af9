"""MI355X operator surface of Selective Attention Freezing (mixed-head prefill).

Same import surface as the reference's ``kernel`` package
(/root/reference/kernel/__init__.py:14-22), so a caller such as
``nanogpt/model.py`` switches with no code change:

    from kernel import (frozen_pv, frozen_pv_usable, linear_rows, linear_rows2,
                        linear_permuted_cols, fused_mixed_attn, fused_attn_usable,
                        decomposed_logz, decomp_logits, make_rho_band, BAND_ROWS)

The attention operators run hand-written gfx950 HIP kernels from
libsafattn.so (see include/saf_attn.h); there is no Triton and no CPU path.
"""
from .frozen_attn import frozen_pv, frozen_pv_usable, HAVE_TRITON
from .indexed_linear import linear_rows, linear_rows2, linear_permuted_cols
from .rope import rope_qk_, qk_rmsnorm_rope_
from .layernorm import add_layernorm_, add_rmsnorm_
from .projection import (gelu_, gelu_usable, linear_gelu, linear_gelu_usable, linear_rope, linear_rope_usable, linear_swiglu,
                         linear_swiglu_usable, swiglu_weight)
from .fused_attn import (fused_mixed_attn, fused_attn_usable, decomposed_logz,
                         decomp_log_normalizers, decomp_log_normalizers_fft,
                         decomp_logits, make_rho_band, BAND_ROWS,
                         classify_closed_form, CLOSED_NONE, CLOSED_MEAN,
                         CLOSED_DECAY, CLOSED_WINDOW, KernelTimer, set_kernel_timer)

__all__ = ["frozen_pv", "frozen_pv_usable", "HAVE_TRITON",
           "linear_rows", "linear_rows2", "linear_permuted_cols",
           "fused_mixed_attn", "fused_attn_usable", "decomposed_logz",
           "decomp_log_normalizers", "decomp_log_normalizers_fft",
           "decomp_logits", "make_rho_band", "BAND_ROWS",
           "classify_closed_form", "CLOSED_NONE", "CLOSED_MEAN",
           "CLOSED_DECAY", "CLOSED_WINDOW", "KernelTimer", "set_kernel_timer",
           "rope_qk_", "qk_rmsnorm_rope_", "add_layernorm_", "add_rmsnorm_", "gelu_", "gelu_usable", "linear_gelu", "linear_gelu_usable",
           "linear_rope", "linear_rope_usable", "linear_swiglu", "linear_swiglu_usable", "swiglu_weight"]
