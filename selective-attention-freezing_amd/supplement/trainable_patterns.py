"""Opt-in learnable decomposed patterns for the nanoGPT caller.

The reference's supplement (/root/reference/supplement/trainable_patterns.py)
turns the fitted alpha / rho of every decomposed-frozen layer into parameters
and trains them through the frozen path.  This module keeps its entry points
(``enable``, ``attach_optimizer``, ``patch_fused_dispatch``,
``dense_reference``) and their contract, over a design of its own:

* one ``TrainablePatterns`` object per model owns the parameters.  Each
  attention module that has decomposed heads holds a reference to it
  (``attn._patterns``) and asks it, per forward, for the kernel inputs
  (detached alpha / rho, the row normalisers z, no closed-form scan: a trained
  pattern need not stay a mean / decay / window) and for the gradient hook on
  its output (``PatternGradient``, whose backward runs the HIP dalpha / drho
  kernel);
* z is cached per layer and sequence length.  A cached z is valid while the
  model's pattern generation is unchanged and the two parameters' version
  counters are the ones it was computed from; the optimizer's step hook
  (``attach_optimizer``) advances the generation, since a fused step need not
  bump version counters;
* ``state_dict()`` of a trainable layer reports the normalisers of the current
  parameters under ``dyn_z`` (a state-dict post-hook rewrites that entry; the
  module's own buffer is left alone);
* ``patch_fused_dispatch`` serves callers outside the model that pass a
  parameter requiring grad straight to ``nanogpt.model.fused_mixed_attn``: the
  module global becomes a ``PatternAwareDispatch`` object that derives z (from
  the owner's cache when the parameter belongs to a ``TrainablePatterns``) and
  adds the gradient hook.  Calls from the model pass detached tensors and go
  straight through.

Dense patterns and live heads are untouched."""
import weakref

import torch
from torch import nn

from .trainable_pattern_kernels import normalisers, PatternGradient

_PARAM_NAMES = ("dyn_alpha", "dyn_rho")


def dense_reference(value, alpha, rho):
    """softmax_j(alpha_j + rho_{i-j}) over j <= i, applied to value (B, H, T, D)
    (supplement/trainable_patterns.py:7-13), plain torch."""
    T = value.shape[-2]
    pos = torch.arange(T, device=value.device)
    dist = pos[:, None] - pos[None, :]
    logits = alpha[:, None, :T] + rho[:, dist.clamp_min(0)]
    p = logits.masked_fill(dist < 0, float("-inf")).softmax(-1)
    return p.to(value.dtype) @ value


def _host_states(attn):
    from kernel.fused_attn import _host_table
    return _host_table(attn._fz_mask_i32)


class TrainablePatterns:
    """The trainable alpha / rho of one model and the normalisers derived
    from them."""

    # parameter -> owning TrainablePatterns, for the module-global dispatch
    _owners = weakref.WeakKeyDictionary()

    def __init__(self, model):
        self.layers = []           # attention modules with trainable patterns
        self.generation = 0        # advanced by the optimizer step hook
        self._z = {}               # attn -> (T, stamp, z)
        for attn in _attn_modules(model):
            dec = getattr(attn, "dyn_decomp", None)
            if dec is None or getattr(attn, "dyn_alpha", None) is None:
                continue
            if any(isinstance(getattr(attn, n), nn.Parameter) for n in _PARAM_NAMES):
                raise RuntimeError("Pattern parameters were already enabled")
            if bool(dec.any()):
                self.layers.append(attn)
        if not self.layers:
            raise RuntimeError("No fitted patterns to train")
        self.parameters = []
        for attn in self.layers:
            for n in _PARAM_NAMES:
                buf = attn._buffers.pop(n)
                p = nn.Parameter(buf.detach().float().clone())
                attn.register_parameter(n, p)
                self.parameters.append(p)
                TrainablePatterns._owners[p] = self
            attn._patterns = self
            attn._register_state_dict_hook(_report_current_normalisers)
            attn._fz_dirty = True

    def invalidate(self):
        """Forget every cached z (the parameters changed)."""
        self.generation += 1
        self._z.clear()

    def _stamp(self, alpha, rho):
        return (self.generation, alpha._version, rho._version)

    def z_for(self, attn, T):
        """Row normalisers of attn's current parameters for sequence length T."""
        alpha, rho = attn.dyn_alpha, attn.dyn_rho
        hit = self._z.get(attn)
        stamp = self._stamp(alpha, rho)
        if hit is not None and hit[0] == T and hit[1] == stamp and hit[2].device == alpha.device:
            return hit[2]
        z = normalisers(alpha, rho, T)
        self._z[attn] = (T, stamp, z)
        return z

    def kernel_inputs(self, attn, T):
        """fused_mixed_attn keyword arguments of a trainable layer."""
        return dict(alpha=attn.dyn_alpha.detach(), rho=attn.dyn_rho.detach(), z=self.z_for(attn, T),
                    closed_form=None)

    def attach_gradient(self, attn, out, v, z):
        """out, with the pattern-parameter gradients of attn's decomposed
        heads added in the backward."""
        if not torch.is_grad_enabled():
            return out
        return PatternGradient.apply(out, v, attn.dyn_alpha, attn.dyn_rho, z, _host_states(attn))


def _attn_modules(model):
    if hasattr(model, "attn_modules"):
        return model.attn_modules()
    return [b.attn for b in model.transformer.h]


@torch.no_grad()
def _report_current_normalisers(attn, state_dict, prefix, local_metadata):
    """state_dict post-hook of a trainable layer: dyn_z holds the normalisers
    of the current alpha / rho over the whole block."""
    key = prefix + "dyn_z"
    if key not in state_dict:
        return
    alpha, rho = attn.dyn_alpha, attn.dyn_rho
    if alpha.is_cuda:
        z = normalisers(alpha, rho, alpha.shape[1])
    else:
        from kernel.fused_attn import decomposed_logz
        z = decomposed_logz(alpha.float(), rho.float())
    state_dict[key] = z.to(state_dict[key].dtype)


def enable(model, optimizer=None):
    """Make every decomposed-pattern layer's alpha / rho trainable (fp32
    parameters, in their own optimizer group without weight decay when an
    optimizer is given) and return the new parameters
    (supplement/trainable_patterns.py:16-41)."""
    patterns = TrainablePatterns(model)
    model._saf_patterns = patterns
    if optimizer is not None:
        optimizer.add_param_group(dict(params=list(patterns.parameters), weight_decay=0.0))
    patch_fused_dispatch()
    if optimizer is not None:
        attach_optimizer(model, optimizer)
    return list(patterns.parameters)


def attach_optimizer(model, optimizer):
    """The optimizer's step invalidates the model's cached normalisers (a
    fused step need not bump Tensor._version)
    (supplement/trainable_patterns.py:44-51)."""
    patterns = getattr(model, "_saf_patterns", None)
    if patterns is None:
        raise RuntimeError("enable() the pattern parameters before attaching an optimizer")
    patch_fused_dispatch()
    optimizer.register_step_post_hook(lambda opt, args, kwargs: patterns.invalidate())


class PatternAwareDispatch:
    """``nanogpt.model.fused_mixed_attn`` after patch_fused_dispatch: calls
    whose alpha requires grad get their z (the owner's cached one when alpha
    belongs to a TrainablePatterns), detached pattern inputs, no closed-form
    scan and the pattern gradient; every other call goes straight to the
    operator."""

    _trainable_patterns = True

    def __init__(self, original):
        self._original = original

    def __call__(self, q, k, v, patt, frozen, hidx=None, pidx=None, **kwargs):
        alpha, rho = kwargs.get("alpha"), kwargs.get("rho")
        if alpha is None or not alpha.requires_grad:
            return self._original(q, k, v, patt, frozen, hidx, pidx, **kwargs)
        T = v.shape[-2]
        owner = TrainablePatterns._owners.get(alpha)
        attn = None
        if owner is not None:
            attn = next((a for a in owner.layers if a.dyn_alpha is alpha and a.dyn_rho is rho), None)
        z = owner.z_for(attn, T) if attn is not None else normalisers(alpha, rho, T)
        kwargs.update(alpha=alpha.detach(), rho=rho.detach(), z=z, closed_form=None)
        out = self._original(q, k, v, patt, frozen, hidx, pidx, **kwargs)
        if torch.is_grad_enabled():
            from kernel.fused_attn import _host_table
            out = PatternGradient.apply(out, v, alpha, rho, z, _host_table(frozen))
        return out

    def clear_pattern_cache(self):
        """Invalidate the normalisers of every model with trainable patterns."""
        for owner in set(TrainablePatterns._owners.values()):
            owner.invalidate()


def patch_fused_dispatch():
    """Install PatternAwareDispatch as nanogpt.model.fused_mixed_attn (once)."""
    from nanogpt import model as module
    if not getattr(module.fused_mixed_attn, "_trainable_patterns", False):
        module.fused_mixed_attn = PatternAwareDispatch(module.fused_mixed_attn)
