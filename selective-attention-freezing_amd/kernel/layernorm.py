"""Residual add + LayerNorm of the GPT block, fused into one HIP kernel.

The reference's block runs ``x = x + attn(ln_1(x)); x = x + mlp(ln_2(x))``
(/root/reference/nanogpt/model.py:1214-1240) with ``LayerNorm`` = F.layer_norm,
eps 1e-5, optional bias (:45-54): a residual add and a normalisation pass per
sub-layer.  ``add_layernorm_`` does both in one pass over the residual
(libsafattn.so ``saf_add_layernorm``): ``x += delta`` in place with one rounding
to the activation dtype, then the LayerNorm of the rounded x in fp32, one
rounding of the output.  Forward only.

``add_rmsnorm_`` is the same pass with transformers' Qwen3RMSNorm in place of
the LayerNorm (the Qwen caller's decoder-block norms, ``saf_add_rmsnorm``).
"""
import torch

from . import _ext


def add_layernorm_(x, delta, weight, bias=None, eps=1e-5):
    """x (..., C) residual, updated in place to x + delta (delta None: left
    as is); returns LayerNorm(x) * weight + bias as a new tensor of x's shape."""
    if not x.is_cuda:
        raise RuntimeError("add_layernorm_ runs on HIP devices only (got a CPU tensor)")
    C = x.size(-1)
    x2 = x.view(-1, C)
    d2 = None if delta is None else delta.reshape(-1, C)
    out = torch.empty_like(x2)
    L = _ext.lib()
    rc = L.saf_add_layernorm(_ext.tensor_desc(x2), _ext.tensor_desc(d2), _ext.tensor_desc(weight.detach()),
                             _ext.tensor_desc(None if bias is None else bias.detach()), float(eps),
                             _ext.tensor_desc(out), _ext.current_stream_ptr(x.device))
    _ext.check(rc)
    return out.view(x.shape)


def add_rmsnorm_(x, delta, weight, eps=1e-6):
    """x (..., C) residual, updated in place to x + delta (delta None: left
    as is); returns weight * round(x * rsqrt(mean(x^2) + eps)) as a new
    tensor of x's shape (Qwen3RMSNorm's rounding)."""
    if not x.is_cuda:
        raise RuntimeError("add_rmsnorm_ runs on HIP devices only (got a CPU tensor)")
    C = x.size(-1)
    x2 = x.view(-1, C)
    d2 = None if delta is None else delta.reshape(-1, C)
    out = torch.empty_like(x2)
    L = _ext.lib()
    rc = L.saf_add_rmsnorm(_ext.tensor_desc(x2), _ext.tensor_desc(d2), _ext.tensor_desc(weight.detach()),
                           float(eps), _ext.tensor_desc(out), _ext.current_stream_ptr(x.device))
    _ext.check(rc)
    return out.view(x.shape)
