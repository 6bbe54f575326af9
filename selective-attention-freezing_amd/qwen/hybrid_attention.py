"""Hybrid (live + frozen head) attention for Hugging Face Qwen3 models.

The GQA caller of the mixed-head prefill path.  It keeps the API of
/root/reference/qwen/nanogpt/hybrid_prior_attention.py:
  HybridAttentionBase._hybrid_init (:74-171)   shrunken q_proj, prior buffers,
                                               head routing tables
  make_qwen3_hybrid_class (:477-642)           the Qwen3 forward: fused branch
                                               (:530-584), split fallback (:586-640)
  get_hybrid_class_for / convert_targets_to_hybrid / restore_originals (:645-729)
and the target discovery of /root/reference/qwen/nanogpt/test_prior_pretrained.py
(:181-240).  ``use_triton`` keeps the reference's keyword; here it selects the
fused HIP path (libsafattn.so), which is the only fused path this build has.

Differences that follow from the MI355X design (fused branch, no grad):
  * one projection GEMM for [Wq of the live heads; Wk; Wv] (weights gathered
    once per weight version), instead of three;
  * q_norm / k_norm and the rotary embedding of live q and raw k run as one
    in-place HIP kernel (``qk_rmsnorm_rope_``) on the projection output;
  * decomposed priors keep alpha, rho and z in fp32 (as the reference) and are
    classified once at conversion: causal mean, exponential decay and sliding
    window heads run the closed-form scan kernel; the (H, 64, S) rho band is
    not materialised (the HIP rebuild kernel reads rho directly);
  * the attention output is allocated T-major, so the head merge before o_proj
    is a view.
With gradients enabled the fused branch keeps torch's q/k norm and RoPE (the
operators have no backward, as the reference's GQA kernel).  The Qwen3.5
gated-attention family is not covered.
"""
from __future__ import annotations

import importlib
from dataclasses import dataclass
from typing import List, Optional, Type

import torch
import torch.nn as nn
import torch.nn.functional as F

import kernel as _kernel_mod
from kernel import fused_attn_usable, classify_closed_form  # noqa: F401
from kernel.fused_attn import decomposed_logz, decomp_logits

_FUSED_DISPATCH_COUNT = 0


def fused_dispatch_count():
    """Number of fused mixed-head dispatches made by hybrid Qwen modules."""
    return _FUSED_DISPATCH_COUNT


def fused_mixed_attn(*args, **kwargs):
    """Module-global hook (looked up at call time, like the reference's
    import of ``fused_mixed_attn`` into the adapter module) so harnesses can
    wrap or count the operator calls."""
    return _kernel_mod.fused_mixed_attn(*args, **kwargs)


class HybridAttentionBase:
    """Shrunken q_proj, frozen-prior buffers and head routing shared by the
    hybrid attention classes (hybrid_prior_attention.py:60-198)."""

    ORIGINAL_CLASS: Optional[type] = None

    def _hybrid_init(self, original: nn.Module, pattern, head_mask: torch.Tensor,
                     n_q: int, head_dim: int, device, dtype,
                     q_per_head_dim: int = None, decomp=None):
        """pattern: (n_q, T, T) dense priors (rows of live heads unused) or None
        with ``decomp`` = (alpha, rho), each (n_q, S) fp32."""
        if q_per_head_dim is None:
            q_per_head_dim = head_dim
        head_mask = head_mask.to(torch.bool).cpu()
        n_pattern = int(head_mask.sum().item())
        n_standard = n_q - n_pattern
        self.decomposed = decomp is not None
        self.n_q_heads = n_q
        self.n_pattern_heads = n_pattern
        self.n_standard_heads = n_standard
        self.head_dim_hybrid = head_dim

        if n_standard > 0:
            row_keep = (~head_mask).repeat_interleave(q_per_head_dim)
            q_orig = original.q_proj
            q_small = nn.Linear(q_orig.in_features, n_standard * q_per_head_dim,
                                bias=q_orig.bias is not None, device=device, dtype=dtype)
            with torch.no_grad():
                q_small.weight.copy_(q_orig.weight[row_keep.to(q_orig.weight.device)])
                if q_orig.bias is not None:
                    q_small.bias.copy_(q_orig.bias[row_keep.to(q_orig.bias.device)])
            self.q_proj_std = q_small
        else:
            self.q_proj_std = None

        pat_idx = torch.nonzero(head_mask, as_tuple=True)[0]
        std_idx = torch.nonzero(~head_mask, as_tuple=True)[0]
        self.register_buffer("pattern_head_idx", pat_idx.to(device))
        self.register_buffer("standard_head_idx", std_idx.to(device))
        self._closed = None
        if self.decomposed:
            alpha, rho = decomp
            alpha = alpha.detach().to(device=device, dtype=torch.float32).contiguous()
            rho = rho.detach().to(device=device, dtype=torch.float32).contiguous()
            z = decomposed_logz(alpha, rho)
            self.register_buffer("dec_alpha", alpha)
            self.register_buffer("dec_rho", rho)
            self.register_buffer("dec_z", z.contiguous())
            self.register_buffer("prior_pattern", torch.empty(0, device=device, dtype=dtype))
            if n_pattern:
                self._closed = classify_closed_form(alpha, rho, z, heads=pat_idx.tolist())
        elif n_pattern > 0:
            subset = pattern[pat_idx].to(device=device, dtype=dtype)
            # lower-triangular, row-normalised in the model dtype (:146-152)
            subset = subset.tril()
            subset = subset / subset.sum(dim=-1, keepdim=True).clamp_min(torch.finfo(dtype).tiny)
            self.register_buffer("prior_pattern", subset.contiguous())
        else:
            self.register_buffer("prior_pattern", torch.empty(0, device=device, dtype=dtype))

        # head states 0 live / 1 dense / 2 decomposed; compact Q and P slots
        frozen_i32 = head_mask.to(device=device, dtype=torch.int32)
        if self.decomposed:
            frozen_i32 = frozen_i32 * 2
        hidx_i32 = torch.zeros(n_q, device=device, dtype=torch.int32)
        pidx_i32 = torch.zeros(n_q, device=device, dtype=torch.int32)
        if n_standard:
            hidx_i32[std_idx.to(device)] = torch.arange(n_standard, device=device, dtype=torch.int32)
        if n_pattern:
            pidx_i32[pat_idx.to(device)] = torch.arange(n_pattern, device=device, dtype=torch.int32)
        self.register_buffer("frozen_mask_i32", frozen_i32)
        self.register_buffer("hidx_i32", hidx_i32)
        self.register_buffer("pidx_i32", pidx_i32)
        self._wc_key = None
        self.hybrid_calls = 0
        self.triton_calls = 0  # fused-path calls (the reference's counter name)

    def _fused_prior_kwargs(self):
        if self.n_pattern_heads == 0:
            return dict(patt=None)
        if self.decomposed:
            return dict(patt=None, alpha=self.dec_alpha, rho=self.dec_rho, z=self.dec_z,
                        closed_form=self._closed)
        return dict(patt=self.prior_pattern)

    def _fused_prior_ready(self, T):
        if self.n_pattern_heads == 0:
            return True
        if self.decomposed:
            return self.dec_alpha.size(-1) >= T
        return self.prior_pattern.ndim == 3 and self.prior_pattern.size(-1) >= T

    def _split_patterns(self, T, dtype):
        """(n_pattern, T, T) dense priors for the torch split path (:187-194)."""
        if not self.decomposed:
            return self.prior_pattern[:, :T, :T].to(dtype)
        idx = self.pattern_head_idx
        lg = decomp_logits(self.dec_alpha[idx, :T], self.dec_rho[idx, :T])
        return torch.exp(lg - self.dec_z[idx, :T][:, :, None]).to(dtype)

    def _qkv_weight_cache(self):
        """[Wq(live); Wk; Wv] (and biases), rebuilt when a weight changes."""
        ws = [m.weight for m in (self.q_proj_std, self.k_proj, self.v_proj) if m is not None]
        key = tuple((w._version, w.data_ptr()) for w in ws)
        if self._wc_key != key:
            with torch.no_grad():
                self._wc_w = torch.cat([w.detach() for w in ws])
                mods = [m for m in (self.q_proj_std, self.k_proj, self.v_proj) if m is not None]
                self._wc_b = None if mods[0].bias is None else torch.cat([m.bias.detach() for m in mods])
            self._wc_key = key
        return self._wc_w, self._wc_b


def make_qwen3_hybrid_class():
    """Hybrid subclass of transformers' Qwen3Attention (:477-642)."""
    qwen3 = importlib.import_module("transformers.models.qwen3.modeling_qwen3")
    OriginalAttention = qwen3.Qwen3Attention
    eager_attention_forward = qwen3.eager_attention_forward
    repeat_kv = qwen3.repeat_kv
    apply_rotary_pos_emb = qwen3.apply_rotary_pos_emb

    class HybridQwen3Attention(HybridAttentionBase, OriginalAttention):
        ORIGINAL_CLASS = OriginalAttention

        def __init__(self, original, pattern, head_mask, device, dtype, use_triton=True,
                     assume_causal_prefill=False, decomp=None):
            nn.Module.__init__(self)
            cfg = original.config
            self.config = cfg
            self.layer_idx = original.layer_idx
            self.layer_type = getattr(original, "layer_type", None)
            self.attention_dropout = original.attention_dropout
            self.num_attention_heads = cfg.num_attention_heads
            self.num_key_value_heads = cfg.num_key_value_heads
            self._real_num_kv_groups = original.num_key_value_groups
            # K/V are broadcast by hand on the split path
            self.num_key_value_groups = 1
            self.head_dim = original.head_dim
            self.scaling = original.scaling
            self.is_causal = original.is_causal
            self.sliding_window = getattr(original, "sliding_window", None)
            self.use_triton_kernel = use_triton
            self.assume_causal_prefill = assume_causal_prefill
            # with no frozen head the reference leaves the module unconverted;
            # set (convert_targets_to_hybrid(fuse_live_only=True)) to run an
            # all-live layer through the HIP flash kernel instead of SDPA
            self.fuse_live_only = False
            self.k_proj = original.k_proj
            self.v_proj = original.v_proj
            self.o_proj = original.o_proj
            self.q_norm = original.q_norm
            self.k_norm = original.k_norm
            self._hybrid_init(original, pattern, head_mask, n_q=self.num_attention_heads,
                              head_dim=self.head_dim, device=device, dtype=dtype,
                              q_per_head_dim=self.head_dim, decomp=decomp)
            # query head h reads KV head h // groups of the raw K/V (:526-528)
            self.register_buffer("kvidx_i32", (
                torch.arange(self.num_attention_heads, device=device)
                // self._real_num_kv_groups).to(torch.int32))

        def _fused_forward(self, hidden_states, cos, sin):
            global _FUSED_DISPATCH_COUNT
            B, T, _ = hidden_states.shape
            n_std, hd = self.n_standard_heads, self.head_dim
            hkv, n_q = self.num_key_value_heads, self.num_attention_heads
            if torch.is_grad_enabled():
                k = self.k_norm(self.k_proj(hidden_states).view(B, T, hkv, hd)).transpose(1, 2)
                v = self.v_proj(hidden_states).view(B, T, hkv, hd).transpose(1, 2)
                if n_std > 0:
                    q = self.q_norm(self.q_proj_std(hidden_states).view(B, T, n_std, hd)).transpose(1, 2)
                    q, k = apply_rotary_pos_emb(q, k, cos, sin)
                else:
                    q = v[:, :0]
            else:
                w, wb = self._qkv_weight_cache()
                qkv = F.linear(hidden_states, w, wb).view(B, T, n_std + 2 * hkv, hd)
                q = qkv[:, :, :n_std].transpose(1, 2)
                k = qkv[:, :, n_std:n_std + hkv].transpose(1, 2)
                v = qkv[:, :, n_std + hkv:].transpose(1, 2)
                if n_std > 0:
                    if cos.dim() == 3 and cos.size(0) != 1:
                        # per-sequence positions: torch prologue
                        q = self.q_norm(q.transpose(1, 2)).transpose(1, 2)
                        k = self.k_norm(k.transpose(1, 2)).transpose(1, 2)
                        q, k = apply_rotary_pos_emb(q, k, cos, sin)
                    else:
                        _kernel_mod.qk_rmsnorm_rope_(q, k, self.q_norm.weight, self.k_norm.weight,
                                                     self.q_norm.variance_epsilon, cos, sin)
            _FUSED_DISPATCH_COUNT += 1
            out_heads = fused_mixed_attn(
                q, k, v, frozen=self.frozen_mask_i32, hidx=self.hidx_i32, pidx=self.pidx_i32,
                kvidx=self.kvidx_i32, sm_scale=self.scaling, validate=False,
                **self._fused_prior_kwargs())
            self.triton_calls += 1
            out = out_heads.transpose(1, 2).reshape(B, T, n_q * hd)
            return self.o_proj(out), None

        def forward(self, hidden_states, position_embeddings, attention_mask=None,
                    past_key_values=None, cache_position=None, **kwargs):
            self.hybrid_calls += 1
            B, T, _ = hidden_states.shape
            n_std, n_pat = self.n_standard_heads, self.n_pattern_heads
            head_dim, n_q = self.head_dim, self.num_attention_heads
            cos, sin = position_embeddings

            mask_is_supported = attention_mask is None
            if self.assume_causal_prefill and isinstance(attention_mask, torch.Tensor):
                mask_is_supported = (attention_mask.ndim == 4
                                     and attention_mask.shape[-2:] == (T, T)
                                     and attention_mask.shape[0] in (1, B))
            can_fuse = (self.use_triton_kernel and (n_pat > 0 or self.fuse_live_only)
                        and not self.training
                        and fused_attn_usable(hidden_states) and mask_is_supported
                        and past_key_values is None and self.sliding_window is None
                        and self._fused_prior_ready(T))
            if can_fuse:
                return self._fused_forward(hidden_states, cos, sin)

            # split path (also the correctness reference): SDPA / eager for the
            # standard heads, dense P @ V for the pattern heads (:586-640)
            k = self.k_norm(self.k_proj(hidden_states).view(
                B, T, self.num_key_value_heads, head_dim)).transpose(1, 2)
            v = self.v_proj(hidden_states).view(B, T, self.num_key_value_heads, head_dim).transpose(1, 2)
            k_full = repeat_kv(k, self._real_num_kv_groups)
            v_full = repeat_kv(v, self._real_num_kv_groups)
            if n_std > 0:
                q_std = self.q_norm(self.q_proj_std(hidden_states).view(
                    B, T, n_std, head_dim)).transpose(1, 2)
                k_std = k_full[:, self.standard_head_idx]
                q_std, k_std = apply_rotary_pos_emb(q_std, k_std, cos, sin)
                v_std = v_full[:, self.standard_head_idx]
                impl_name = getattr(self.config, "_attn_implementation", "eager")
                if impl_name in ("sdpa", "flash_attention_2") and T > 1:
                    out_std = F.scaled_dot_product_attention(
                        q_std, k_std, v_std, attn_mask=attention_mask,
                        is_causal=attention_mask is None, scale=self.scaling).transpose(1, 2).contiguous()
                else:
                    out_std, _ = eager_attention_forward(
                        self, q_std, k_std, v_std, attention_mask,
                        dropout=0.0 if not self.training else self.attention_dropout,
                        scaling=self.scaling)
                out_std = out_std.view(B, T, n_std, head_dim)
            if n_pat > 0:
                v_pat = v_full[:, self.pattern_head_idx]
                pat = self._split_patterns(T, v_pat.dtype)
                out_pat = torch.matmul(pat.unsqueeze(0), v_pat).transpose(1, 2).contiguous()
            out = hidden_states.new_empty(B, T, n_q, head_dim)
            if n_std > 0:
                out[:, :, self.standard_head_idx] = out_std
            if n_pat > 0:
                out[:, :, self.pattern_head_idx] = out_pat
            return self.o_proj(out.reshape(B, T, n_q * head_dim)), None

    return HybridQwen3Attention


_REGISTRY_BUILDERS = {"Qwen3Attention": make_qwen3_hybrid_class}
_BUILT_CACHE: dict = {}


def get_hybrid_class_for(original_module: nn.Module) -> Optional[Type]:
    """Hybrid class for an attention module's class name (:659-665)."""
    name = type(original_module).__name__
    if name not in _REGISTRY_BUILDERS:
        return None
    if name not in _BUILT_CACHE:
        _BUILT_CACHE[name] = _REGISTRY_BUILDERS[name]()
    return _BUILT_CACHE[name]


@dataclass
class SoftmaxAttentionTarget:
    layer_idx: int
    module: nn.Module
    attr_name: str


_ATTN_ATTR_CANDIDATES = ("self_attn", "attention", "attn", "full_attn")


def iter_blocks(model: nn.Module):
    """The transformer blocks of a causal LM (test_prior_pretrained.py:199-212)."""
    for path in (lambda m: m.model.layers, lambda m: m.transformer.h,
                 lambda m: m.model.decoder.layers, lambda m: m.gpt_neox.layers):
        try:
            blocks = path(model)
        except AttributeError:
            continue
        if blocks is not None:
            return list(blocks)
    raise ValueError(f"cannot find the transformer blocks of {type(model).__name__}")


def _is_softmax_attention(m: nn.Module) -> bool:
    return all(hasattr(m, n) for n in ("q_proj", "k_proj", "v_proj")) and \
        any(hasattr(m, n) for n in ("o_proj", "c_proj"))


def discover_softmax_attention(model: nn.Module) -> List[SoftmaxAttentionTarget]:
    """Every standard softmax-attention module, one per block (:215-240)."""
    targets = []
    for li, block in enumerate(iter_blocks(model)):
        found = None
        for name in _ATTN_ATTR_CANDIDATES:
            m = getattr(block, name, None)
            if m is not None and _is_softmax_attention(m):
                found = (m, name)
                break
        if found is None:
            for name, m in block.named_children():
                if _is_softmax_attention(m):
                    found = (m, name)
                    break
        if found is not None:
            targets.append(SoftmaxAttentionTarget(li, found[0], found[1]))
    return targets


def convert_targets_to_hybrid(model, targets, mean_attn, head_masks, device, dtype,
                              use_triton=True, assume_causal_prefill=False, decomp=None,
                              fuse_live_only=False):
    """Swap each target's attention module for its hybrid counterpart (:671-722).

    mean_attn: per-target (n_heads, T, T) dense priors, or None with ``decomp``
    = per-target (alpha, rho) pairs of (n_heads, S) fp32 tensors (None entries
    for targets with no frozen head).  Returns the list restore_originals takes.
    fuse_live_only (an extension) also converts targets with no frozen head, so
    their attention runs the HIP flash kernel rather than the model's SDPA.
    """
    if mean_attn is None:
        if decomp is None:
            raise ValueError("need mean_attn or decomp")
        priors = [None] * len(targets)
    else:
        priors = list(mean_attn)
    if not len(targets) == len(priors) == len(head_masks):
        raise ValueError("targets, priors and head_masks must have one entry per target")
    if decomp is not None and len(decomp) != len(targets):
        raise ValueError("decomp must have one entry per target")
    blocks = iter_blocks(model)
    saved = []
    for ti, (t, prior, mask) in enumerate(zip(targets, priors, head_masks)):
        if not bool(mask.any()) and not fuse_live_only:
            saved.append((blocks[t.layer_idx], t.attr_name, None))
            continue
        original = getattr(blocks[t.layer_idx], t.attr_name)
        cls = get_hybrid_class_for(original)
        if cls is None:
            raise RuntimeError(f"No hybrid class registered for {type(original).__name__}")
        hybrid = cls(original, prior, mask, device, dtype, use_triton=use_triton,
                     assume_causal_prefill=assume_causal_prefill,
                     decomp=None if decomp is None else decomp[ti])
        hybrid.fuse_live_only = bool(fuse_live_only)
        hybrid.train(original.training)
        setattr(blocks[t.layer_idx], t.attr_name, hybrid)
        saved.append((blocks[t.layer_idx], t.attr_name, original))
    return saved


def restore_originals(saved):
    """Undo convert_targets_to_hybrid (:725-729)."""
    for block, attr_name, original in saved:
        if original is not None:
            setattr(block, attr_name, original)
