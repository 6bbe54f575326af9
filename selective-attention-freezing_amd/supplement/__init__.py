"""Opt-in trainable decomposed patterns over the SAF operators (the parameter
gradients of frozen heads' alpha / rho); the frozen prefill path is unchanged."""
from .trainable_pattern_kernels import normalisers, PatternGradient, pattern_gradients
from .trainable_patterns import (dense_reference, enable, attach_optimizer, patch_fused_dispatch,
                                 TrainablePatterns)

__all__ = ["normalisers", "PatternGradient", "pattern_gradients", "dense_reference", "enable",
           "attach_optimizer", "patch_fused_dispatch", "TrainablePatterns"]
