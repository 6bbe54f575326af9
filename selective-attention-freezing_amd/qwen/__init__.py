"""Qwen3 / Qwen3.5 GQA caller of the mixed-head prefill operators (Hugging Face adapter)."""
from .hybrid_attention import (HybridAttentionBase, HeadRouting, FamilySpec, make_qwen3_hybrid_class,
                               make_qwen35_hybrid_class, get_hybrid_class_for,
                               convert_targets_to_hybrid, restore_originals,
                               discover_softmax_attention, iter_blocks, SoftmaxAttentionTarget,
                               fused_dispatch_count)
from .model import (qwen_config, build_model, nested_head_masks, n_frozen_for,
                    uniform_causal_prior, convert_with_rate, backbone_forward)

__all__ = ["HybridAttentionBase", "HeadRouting", "FamilySpec", "make_qwen3_hybrid_class",
           "make_qwen35_hybrid_class", "get_hybrid_class_for",
           "convert_targets_to_hybrid", "restore_originals", "discover_softmax_attention",
           "iter_blocks", "SoftmaxAttentionTarget", "fused_dispatch_count",
           "qwen_config", "build_model", "nested_head_masks", "n_frozen_for",
           "uniform_causal_prior", "convert_with_rate", "backbone_forward"]
