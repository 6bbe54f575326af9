"""Opt-in learnable decomposed patterns for the nanoGPT caller.

Restates /root/reference/supplement/trainable_patterns.py over this build's
model: enable() turns each layer's fitted alpha / rho buffers into fp32
parameters (optionally in their own optimizer group, no weight decay),
state_dict() exports the current normalisers into dyn_z, and the model's
attention dispatch is wrapped so that, for trainable alpha, z is recomputed
when the parameters change (cached per parameter version once an optimizer
is attached), closed-form scans are not used (a trained pattern need not
stay a mean / decay / window) and PatternGradient adds the parameter
gradients.  Dense patterns and live heads are untouched."""
import torch
from torch import nn

from .trainable_pattern_kernels import normalisers, PatternGradient


def dense_reference(value, alpha, rho):
    """softmax_j(alpha_j + rho_{i-j}) over j <= i, applied to value (B, H, T, D)
    (supplement/trainable_patterns.py:7-13), plain torch."""
    T = value.shape[-2]
    pos = torch.arange(T, device=value.device)
    dist = pos[:, None] - pos[None, :]
    logits = alpha[:, None, :T] + rho[:, dist.clamp_min(0)]
    p = logits.masked_fill(dist < 0, float("-inf")).softmax(-1)
    return p.to(value.dtype) @ value


def _attn_modules(model):
    if hasattr(model, "attn_modules"):
        return model.attn_modules()
    return [b.attn for b in model.transformer.h]


def enable(model, optimizer=None):
    """Make every decomposed-pattern layer's alpha / rho trainable; returns
    the new parameters (supplement/trainable_patterns.py:16-41)."""
    params = []
    for attn in _attn_modules(model):
        dec = getattr(attn, "dyn_decomp", None)
        if dec is None or getattr(attn, "dyn_alpha", None) is None or not bool(dec.any()):
            continue
        for name in ("dyn_alpha", "dyn_rho"):
            old = getattr(attn, name)
            if isinstance(old, nn.Parameter):
                raise RuntimeError("Pattern parameters were already enabled")
            delattr(attn, name)
            p = nn.Parameter(old.detach().clone().float())
            attn.register_parameter(name, p)
            params.append(p)
        attn._fz_dirty = True
        attn.register_state_dict_pre_hook(_export_current_buffers)
    if not params:
        raise RuntimeError("No fitted patterns to train")
    if optimizer is not None:
        optimizer.add_param_group(dict(params=params, weight_decay=0.0))
    patch_fused_dispatch()
    if optimizer is not None:
        attach_optimizer(model, optimizer)
    return params


def attach_optimizer(model, optimizer):
    """Cache z per parameter version; the optimizer's step clears the cache
    (a fused step need not bump Tensor._version)."""
    from nanogpt import model as module
    patch_fused_dispatch()
    for name, p in model.named_parameters():
        if name.endswith(("dyn_alpha", "dyn_rho")):
            p._pattern_cache_enabled = True
    optimizer.register_step_post_hook(lambda *args: module.fused_mixed_attn.clear_pattern_cache())


@torch.no_grad()
def _export_current_buffers(attn, prefix, keep_vars):
    if attn.dyn_alpha.is_cuda:
        attn.dyn_z.copy_(normalisers(attn.dyn_alpha, attn.dyn_rho, attn.dyn_alpha.shape[1]))
    else:
        from kernel.fused_attn import decomposed_logz
        attn.dyn_z.copy_(decomposed_logz(attn.dyn_alpha.float(), attn.dyn_rho.float()))


def patch_fused_dispatch():
    """Wrap nanogpt.model.fused_mixed_attn once (idempotent)."""
    from nanogpt import model as module
    if getattr(module.fused_mixed_attn, "_trainable_patterns", False):
        return
    original = module.fused_mixed_attn
    cache = {}

    def dispatch(q, k, v, patt, frozen, hidx=None, pidx=None, **kwargs):
        alpha, rho = kwargs.get("alpha"), kwargs.get("rho")
        if alpha is None or not alpha.requires_grad:
            return original(q, k, v, patt, frozen, hidx, pidx, **kwargs)
        T = v.shape[-2]
        key = id(alpha)
        sig = (alpha._version, rho._version, T, alpha.device)
        hit = cache.get(key)
        if (not getattr(alpha, "_pattern_cache_enabled", False)
                or hit is None or hit[0] is not alpha or hit[1] != sig):
            z = normalisers(alpha, rho, T)
            cache[key] = (alpha, sig, z)
        else:
            z = hit[2]
        kwargs.update(alpha=alpha.detach(), rho=rho.detach(), z=z, closed_form=None)
        out = original(q, k, v, patt, frozen, hidx, pidx, **kwargs)
        if torch.is_grad_enabled():
            out = PatternGradient.apply(out, v, alpha, rho, z, frozen)
        return out

    dispatch._trainable_patterns = True
    dispatch._original = original
    dispatch.clear_pattern_cache = cache.clear
    module.fused_mixed_attn = dispatch
