"""Rotary position embedding of the live-head Q/K, fused into one HIP kernel.

The reference applies ``apply_rotary_pos_emb`` (/root/reference/nanogpt/model.py:63-68)
to the compact live-head q/k of the fused path (:1007-1008) as a chain of
elementwise torch ops.  ``rope_qk_`` does the same rotation in place, in one
pass over the projection output (libsafattn.so ``saf_rope_qk_inplace``):
fp32 arithmetic with the model's cos/sin cache, one rounding to the activation
dtype.  ``qk_rmsnorm_rope_`` adds the per-head q/k RMSNorm of the Qwen3 fused
branch (/root/reference/qwen/nanogpt/hybrid_prior_attention.py:543-572) in the
same pass (``saf_qk_rmsnorm_rope_inplace``).  Forward only (the operators of
this build have no backward).
"""
import torch

from . import _ext


def rope_qk_(q, k, cos, sin):
    """Rotate q (B, Uq, T, hd) and k (B, Uk, T, hd) in place; cos/sin are the
    (T', hd) caches (any leading singleton dims are squeezed).  Returns (q, k)."""
    if not q.is_cuda:
        raise RuntimeError("rope_qk_ runs on HIP devices only (got a CPU tensor)")
    cos2 = cos.reshape(-1, cos.size(-1))
    sin2 = sin.reshape(-1, sin.size(-1))
    L = _ext.lib()
    rc = L.saf_rope_qk_inplace(_ext.tensor_desc(q), _ext.tensor_desc(k), _ext.tensor_desc(cos2),
                               _ext.tensor_desc(sin2), _ext.current_stream_ptr(q.device))
    _ext.check(rc)
    return q, k


def qk_rmsnorm_rope_(q, k, q_weight, k_weight, eps, cos, sin):
    """Qwen3 prologue in place: q <- rope(q_norm(q)), k <- rope(k_norm(k)) for
    q (B, Uq, T, hd) and k (B, HKV, T, hd); the norms are Qwen3RMSNorm over hd
    with (hd,) weights.  Returns (q, k)."""
    if not q.is_cuda:
        raise RuntimeError("qk_rmsnorm_rope_ runs on HIP devices only (got a CPU tensor)")
    cos2 = cos.reshape(-1, cos.size(-1))
    sin2 = sin.reshape(-1, sin.size(-1))
    L = _ext.lib()
    rc = L.saf_qk_rmsnorm_rope_inplace(
        _ext.tensor_desc(q), _ext.tensor_desc(k), _ext.tensor_desc(q_weight.detach()),
        _ext.tensor_desc(k_weight.detach()), float(eps), _ext.tensor_desc(cos2), _ext.tensor_desc(sin2),
        _ext.current_stream_ptr(q.device))
    _ext.check(rc)
    return q, k
