"""Live + frozen head attention for Hugging Face Qwen3 and Qwen3.5 models.

The GQA caller of the mixed-head prefill path.  Entry points keep the names
and signatures of the reference adapter
(/root/reference/qwen/nanogpt/hybrid_prior_attention.py): the hybrid classes
(``make_qwen3_hybrid_class`` :477-642, ``make_qwen35_hybrid_class``
:205-470), ``get_hybrid_class_for`` (:659-665), ``convert_targets_to_hybrid``
(:671-722), ``restore_originals`` (:725-729), the module-global
``fused_mixed_attn`` (the reference's bench wraps it, bench_qwen_prefill_triton.py:136-138)
and the per-module ``hybrid_calls`` / ``triton_calls`` counters it reads
(:169-170); plus the target discovery of
/root/reference/qwen/nanogpt/test_prior_pretrained.py:181-240.  The layer's
function is the reference's: query heads in ``head_mask`` skip their query
projection and QK^T and apply a fixed causal prior to their KV group's V;
the others are causal softmax heads; Qwen3.5's per-head sigmoid gate
multiplies every head's output.

Design of this build:
  * ``FamilySpec`` describes a model family: where its attention class lives,
    whether q_proj emits a (query, gate) pair per head, and whether this
    build's fused q/k RMSNorm + RoPE kernel matches the family's prologue
    (Qwen3: yes; Qwen3.5 with its (1 + w) norm and partial rotation: its own
    modules run instead).
  * ``HeadRouting`` holds one layer's routing and prior: live and frozen head
    lists, the operator's device tables (head state, live slot, prior slot,
    KV head) and the frozen heads' prior (compact dense rows, or fp32
    alpha / rho / z with their closed-form classification).
  * ``HybridAttentionBase`` is one nn.Module for every family: it adopts the
    original's k / v / o projections and norms, keeps the live heads' query
    rows (and every head's gate rows) as its own projection, and, on the fused
    no-grad path, runs ONE gathered GEMM [Wq(live); Wk; Wv; Wgate] whose
    output feeds the operator as strided views; the attention output comes
    back T-major, so the head merge before o_proj is a view.
  * The split path (gradients, attention masks, caches, sliding windows, CPU
    tensors) computes the same function in torch: SDPA (or an eager softmax)
    for the live heads over their KV group, P @ V for the frozen heads.
"""
from __future__ import annotations

import importlib
from dataclasses import dataclass
from typing import Dict, List, Optional, Type

import torch
import torch.nn as nn
import torch.nn.functional as F

import kernel as _kernel_mod
from kernel import classify_closed_form, fused_attn_usable
from kernel.fused_attn import decomp_logits, decomposed_logz

_FUSED_DISPATCH_COUNT = 0

# head dims the HIP operator runs (include/saf_attn.h)
_FUSED_HEAD_DIMS = (32, 64, 96, 128, 256)
# head dims of the fused q/k RMSNorm + RoPE kernel (larger heads use torch's)
_PROLOGUE_HEAD_DIMS = (32, 64, 96, 128)


def fused_dispatch_count():
    """Number of fused mixed-head dispatches made by hybrid Qwen modules."""
    return _FUSED_DISPATCH_COUNT


def fused_mixed_attn(*args, **kwargs):
    """Module-global hook, looked up at call time (harnesses wrap or count it)."""
    return _kernel_mod.fused_mixed_attn(*args, **kwargs)


@dataclass(frozen=True)
class FamilySpec:
    class_name: str        # transformers attention class
    module: str            # where it lives
    gated: bool            # q_proj rows per head: query (hd), then gate (hd)
    hip_prologue: bool     # the family's q/k norm + RoPE is saf_qk_rmsnorm_rope_inplace's


QWEN3 = FamilySpec("Qwen3Attention", "transformers.models.qwen3.modeling_qwen3", gated=False, hip_prologue=True)
QWEN35 = FamilySpec("Qwen3_5Attention", "transformers.models.qwen3_5.modeling_qwen3_5", gated=True,
                    hip_prologue=False)
FAMILIES: Dict[str, FamilySpec] = {f.class_name: f for f in (QWEN3, QWEN35)}


class HeadRouting:
    """One layer's split of query heads into live and frozen, the operator's
    routing tables and the frozen heads' prior.

    head_mask (H,) bool: True = frozen.  The prior is ``pattern`` ((H, T, T)
    dense rows, those of live heads unused) or ``decomp`` = (alpha, rho),
    (H, S) logit vectors of softmax(alpha[j] + rho[i - j])."""

    def __init__(self, head_mask, n_kv_heads, device, dtype, pattern=None, decomp=None):
        mask = torch.as_tensor(head_mask).to(torch.bool).cpu().reshape(-1)
        H = mask.numel()
        if H % n_kv_heads:
            raise ValueError(f"{H} query heads do not split into {n_kv_heads} KV groups")
        self.n_heads = H
        self.frozen = mask.nonzero().flatten().tolist()
        self.live = (~mask).nonzero().flatten().tolist()
        self.decomposed = decomp is not None
        group = H // n_kv_heads
        kv = torch.arange(H) // group
        live_slot = torch.zeros(H, dtype=torch.int32)
        live_slot[self.live] = torch.arange(len(self.live), dtype=torch.int32)
        prior_slot = torch.zeros(H, dtype=torch.int32)
        prior_slot[self.frozen] = torch.arange(len(self.frozen), dtype=torch.int32)
        state = mask.to(torch.int32) * (2 if self.decomposed else 1)
        # the operator's int32 device tables (state 0 / 1 / 2, hidx, pidx, kvidx)
        self.state = state.to(device)
        self.live_slot = live_slot.to(device)
        self.prior_slot = prior_slot.to(device)
        self.kv_head = kv.to(torch.int32).to(device)
        self.live_kv = kv[self.live].to(device)
        self.frozen_kv = kv[self.frozen].to(device)
        self.frozen_idx = torch.as_tensor(self.frozen, dtype=torch.long, device=device)
        self.closed = None
        self.patterns = self.alpha = self.rho = self.z = None
        if self.decomposed:
            a, r = decomp
            self.alpha = a.detach().to(device=device, dtype=torch.float32).contiguous()
            self.rho = r.detach().to(device=device, dtype=torch.float32).contiguous()
            self.z = decomposed_logz(self.alpha, self.rho).contiguous()
            if self.frozen:
                self.closed = classify_closed_form(self.alpha, self.rho, self.z, heads=self.frozen)
        elif self.frozen:
            if pattern is None:
                raise ValueError("frozen heads need a dense prior or decomp=(alpha, rho)")
            rows = pattern[self.frozen].to(device=device, dtype=dtype).tril()
            # causal, row-stochastic in the model dtype (the prior definition of
            # hybrid_prior_attention.py:146-152)
            self.patterns = (rows / rows.sum(-1, keepdim=True).clamp_min(torch.finfo(dtype).tiny)).contiguous()

    def covers(self, T):
        """True if the stored prior reaches sequence length T."""
        if not self.frozen:
            return True
        ref = self.alpha if self.decomposed else self.patterns
        return ref.size(-1) >= T

    def operator_kwargs(self):
        """The prior arguments of fused_mixed_attn for this layer."""
        if not self.frozen:
            return {"patt": None}
        if self.decomposed:
            return {"patt": None, "alpha": self.alpha, "rho": self.rho, "z": self.z,
                    "closed_form": self.closed}
        return {"patt": self.patterns}

    def dense_priors(self, T, dtype):
        """(n_frozen, T, T) prior matrices for the split path."""
        if not self.decomposed:
            return self.patterns[:, :T, :T].to(dtype)
        idx = self.frozen_idx
        lg = decomp_logits(self.alpha[idx, :T], self.rho[idx, :T])
        return torch.exp(lg - self.z[idx, :T, None]).to(dtype)


def _rows_of_heads(heads, head_dim, stride, offset=0):
    """Row indices of `head_dim` rows per head in a weight whose head h starts
    at row h * stride + offset."""
    return [h * stride + offset + d for h in heads for d in range(head_dim)]


def _sub_linear(src: nn.Linear, rows, device, dtype):
    """nn.Linear holding rows `rows` of src (weights copied)."""
    lin = nn.Linear(src.in_features, len(rows), bias=src.bias is not None, device=device, dtype=dtype)
    idx = torch.as_tensor(rows, dtype=torch.long, device=src.weight.device)
    with torch.no_grad():
        lin.weight.copy_(src.weight.index_select(0, idx))
        if src.bias is not None:
            lin.bias.copy_(src.bias.index_select(0, idx))
    return lin


def _eager_attention(q, k, v, mask, scale, dropout, training):
    """softmax(q k^T scale + mask) v with the weights in fp32, then cast (the
    eager attention of the Hugging Face modules)."""
    w = torch.matmul(q, k.transpose(-1, -2)) * scale
    if mask is not None:
        w = w + mask[..., :k.size(-2)]
    else:
        T, S = q.size(-2), k.size(-2)
        causal = torch.ones(T, S, dtype=torch.bool, device=q.device).tril(S - T)
        w = w.masked_fill(~causal, float("-inf"))
    w = torch.softmax(w, dim=-1, dtype=torch.float32).to(q.dtype)
    w = F.dropout(w, p=dropout, training=training)
    return torch.matmul(w, v)


class HybridAttentionBase(nn.Module):
    """Hybrid attention layer for one model family (SPEC), built from the
    original attention module it replaces."""

    SPEC: Optional[FamilySpec] = None
    ORIGINAL_CLASS: Optional[type] = None

    def __init__(self, original, pattern, head_mask, device, dtype, use_triton=True,
                 assume_causal_prefill=False, decomp=None):
        super().__init__()
        spec = self.SPEC
        cfg = original.config
        self.config = cfg
        self.layer_idx = original.layer_idx
        self.layer_type = getattr(original, "layer_type", None)
        self.num_attention_heads = cfg.num_attention_heads
        self.num_key_value_heads = cfg.num_key_value_heads
        self.head_dim = original.head_dim
        self.scaling = original.scaling
        self.attention_dropout = original.attention_dropout
        self.is_causal = True
        self.sliding_window = getattr(original, "sliding_window", None)
        self.use_triton_kernel = use_triton
        # opt-in: a square (B or 1, 1, T, T) mask passed for unpadded prefill
        # is taken to be the causal mask the kernel applies itself
        self.assume_causal_prefill = assume_causal_prefill
        # run an all-live layer through the HIP flash kernel (the reference
        # leaves such layers unconverted)
        self.fuse_live_only = False
        for name in ("k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
            setattr(self, name, getattr(original, name))
        self.routing = HeadRouting(head_mask, self.num_key_value_heads, device, dtype, pattern, decomp)
        r, hd, H = self.routing, self.head_dim, self.num_attention_heads
        per_head = 2 * hd if spec.gated else hd
        # live heads' query rows; gated families: every head's gate rows
        self.q_live = _sub_linear(original.q_proj, _rows_of_heads(r.live, hd, per_head), device, dtype) \
            if r.live else None
        self.gate = _sub_linear(original.q_proj, _rows_of_heads(range(H), hd, per_head, hd), device, dtype) \
            if spec.gated else None
        self._cache_key = None
        self.hybrid_calls = 0
        self.triton_calls = 0
        self.train(original.training)   # a new module would start in training mode

    # -- the single gathered projection of the fused path ------------------
    def _projection_weights(self):
        """[Wq[live]; Wk; Wv (; gates)] gathered once per weight version, its
        rows padded with zeros to a multiple of 256 when the padding is whole
        heads: hipBLASLt's bf16 kernels for an odd multiple of 128 output
        columns run about 1.5x as long as for the next multiple of 256 (the
        columns past the heads are never read)."""
        mods = [m for m in (self.q_live, self.k_proj, self.v_proj, self.gate) if m is not None]
        key = tuple((m.weight._version, m.weight.data_ptr()) for m in mods)
        if self._cache_key != key:
            with torch.no_grad():
                ws = [m.weight.detach() for m in mods]
                bs = None if mods[0].bias is None else [m.bias.detach() for m in mods]
                rows = sum(w.size(0) for w in ws)
                pad = -rows % 256
                if pad and pad % self.head_dim == 0:
                    ws.append(ws[0].new_zeros(pad, ws[0].size(1)))
                    if bs is not None:
                        bs.append(bs[0].new_zeros(pad))
                self._w_cat = torch.cat(ws)
                self._b_cat = None if bs is None else torch.cat(bs)
            self._cache_key = key
        return self._w_cat, self._b_cat

    def _rope(self):
        return importlib.import_module(self.SPEC.module).apply_rotary_pos_emb

    def _fusable(self, x, attention_mask, past_key_values, T):
        mask_ok = attention_mask is None
        if self.assume_causal_prefill and isinstance(attention_mask, torch.Tensor):
            mask_ok = (attention_mask.ndim == 4 and attention_mask.shape[-2:] == (T, T)
                       and attention_mask.shape[0] in (1, x.size(0)))
        return (self.use_triton_kernel and (bool(self.routing.frozen) or self.fuse_live_only)
                and not self.training and not self._builds_graph(x)
                and fused_attn_usable(x) and mask_ok and past_key_values is None
                and self.sliding_window is None and self.head_dim in _FUSED_HEAD_DIMS
                and self.routing.covers(T))

    def _builds_graph(self, x):
        """True when autograd records this call: the fused path (gathered
        weights, in-place prologue, GQA operator without a backward) is then
        not used and the split path computes the same function."""
        return torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters()))

    def _fused_forward(self, x, cos, sin):
        global _FUSED_DISPATCH_COUNT
        B, T, _ = x.shape
        r, hd, H, HKV = self.routing, self.head_dim, self.num_attention_heads, self.num_key_value_heads
        U = len(r.live)
        w, b = self._projection_weights()
        y = F.linear(x, w, b).view(B, T, -1, hd)
        q = y[:, :, :U].transpose(1, 2)
        k = y[:, :, U:U + HKV].transpose(1, 2)
        v = y[:, :, U + HKV:U + 2 * HKV].transpose(1, 2)
        gate = y[:, :, U + 2 * HKV:U + 2 * HKV + H] if self.SPEC.gated else None
        if U:
            if (self.SPEC.hip_prologue and hd in _PROLOGUE_HEAD_DIMS and q.dtype != torch.float32
                    and (cos.dim() == 2 or cos.size(0) == 1)):
                _kernel_mod.qk_rmsnorm_rope_(q, k, self.q_norm.weight, self.k_norm.weight,
                                             self.q_norm.variance_epsilon, cos, sin)
            else:
                q = self.q_norm(q.transpose(1, 2)).transpose(1, 2)
                k = self.k_norm(k.transpose(1, 2)).transpose(1, 2)
                q, k = self._rope()(q, k, cos, sin)
        _FUSED_DISPATCH_COUNT += 1
        out = fused_mixed_attn(q, k, v, frozen=r.state, hidx=r.live_slot, pidx=r.prior_slot,
                               kvidx=r.kv_head, sm_scale=self.scaling, validate=False, **r.operator_kwargs())
        self.triton_calls += 1
        out = out.transpose(1, 2)                     # (B, T, H, hd), a view of the T-major output
        if gate is not None:
            out = out * torch.sigmoid(gate)
        return self.o_proj(out.reshape(B, T, H * hd)), None

    def _split_forward(self, x, cos, sin, attention_mask):
        B, T, _ = x.shape
        r, hd, H, HKV = self.routing, self.head_dim, self.num_attention_heads, self.num_key_value_heads
        k = self.k_norm(self.k_proj(x).view(B, T, HKV, hd)).transpose(1, 2)
        v = self.v_proj(x).view(B, T, HKV, hd).transpose(1, 2)
        out = x.new_empty(B, T, H, hd)
        if r.live:
            q = self.q_norm(self.q_live(x).view(B, T, len(r.live), hd)).transpose(1, 2)
            q, k = self._rope()(q, k, cos, sin)
            kg = k.index_select(1, r.live_kv)
            vg = v.index_select(1, r.live_kv)
            impl = getattr(self.config, "_attn_implementation", "eager")
            if impl in ("sdpa", "flash_attention_2") and T > 1:
                o = F.scaled_dot_product_attention(q, kg, vg, attn_mask=attention_mask,
                                                   is_causal=attention_mask is None, scale=self.scaling)
            else:
                o = _eager_attention(q, kg, vg, attention_mask, self.scaling,
                                     self.attention_dropout, self.training)
            out[:, :, r.live] = o.transpose(1, 2)
        if r.frozen:
            vp = v.index_select(1, r.frozen_kv)
            out[:, :, r.frozen] = torch.matmul(r.dense_priors(T, vp.dtype).unsqueeze(0), vp).transpose(1, 2)
        if self.gate is not None:
            out = out * torch.sigmoid(self.gate(x).view(B, T, H, hd))
        return self.o_proj(out.reshape(B, T, H * hd)), None

    def forward(self, hidden_states, position_embeddings, attention_mask=None, past_key_values=None,
                cache_position=None, **kwargs):
        self.hybrid_calls += 1
        cos, sin = position_embeddings
        T = hidden_states.size(1)
        if self._fusable(hidden_states, attention_mask, past_key_values, T):
            return self._fused_forward(hidden_states, cos, sin)
        return self._split_forward(hidden_states, cos, sin, attention_mask)


_CLASS_CACHE: Dict[str, type] = {}


def _hybrid_class(spec: FamilySpec, name: str) -> type:
    if spec.class_name not in _CLASS_CACHE:
        original = getattr(importlib.import_module(spec.module), spec.class_name)
        _CLASS_CACHE[spec.class_name] = type(name, (HybridAttentionBase,),
                                             {"SPEC": spec, "ORIGINAL_CLASS": original})
    return _CLASS_CACHE[spec.class_name]


def make_qwen3_hybrid_class():
    """Hybrid class for transformers' Qwen3Attention (plain GQA + q/k norm)."""
    return _hybrid_class(QWEN3, "HybridQwen3Attention")


def make_qwen35_hybrid_class():
    """Hybrid class for transformers' Qwen3_5Attention (gated attention)."""
    return _hybrid_class(QWEN35, "HybridQwen3_5Attention")


_MAKERS = {"Qwen3Attention": make_qwen3_hybrid_class, "Qwen3_5Attention": make_qwen35_hybrid_class}


def get_hybrid_class_for(original_module: nn.Module) -> Optional[Type]:
    """The hybrid class for an attention module, or None for an unsupported family."""
    maker = _MAKERS.get(type(original_module).__name__)
    return None if maker is None else maker()


# ---------------------------------------------------------------------------
# Target discovery and conversion
# ---------------------------------------------------------------------------

@dataclass
class SoftmaxAttentionTarget:
    layer_idx: int
    module: nn.Module
    attr_name: str
    parent: Optional[nn.Module] = None


def _is_softmax_attention(m: nn.Module) -> bool:
    return all(hasattr(m, n) for n in ("q_proj", "k_proj", "v_proj")) and \
        any(hasattr(m, n) for n in ("o_proj", "c_proj"))


def _block_lists(model: nn.Module):
    """(path, ModuleList) of the model's stacks of transformer blocks."""
    for path, mod in model.named_modules():
        if isinstance(mod, nn.ModuleList) and len(mod) and \
                any(_is_softmax_attention(c) for b in mod for c in b.children()):
            yield path, mod


def iter_blocks(model: nn.Module):
    """The decoder blocks of a causal LM (the first stack holding softmax
    attention modules)."""
    for _, blocks in _block_lists(model):
        return list(blocks)
    raise ValueError(f"cannot find the transformer blocks of {type(model).__name__}")


def discover_softmax_attention(model: nn.Module) -> List[SoftmaxAttentionTarget]:
    """Every softmax attention module that is a direct child of a decoder
    block, in block order (blocks without one, e.g. linear-attention layers,
    are skipped)."""
    for _, blocks in _block_lists(model):
        targets = []
        for li, block in enumerate(blocks):
            for attr, child in block.named_children():
                if _is_softmax_attention(child):
                    targets.append(SoftmaxAttentionTarget(li, child, attr, block))
                    break
        return targets
    return []


# ---------------------------------------------------------------------------
# gated MLP of the decoder blocks (transformers' Qwen3MLP:
# down_proj(act_fn(gate_proj(x)) * up_proj(x)), SiLU)
# ---------------------------------------------------------------------------

# K (hidden size) up to which the gate / up half runs as one HIP kernel
# (kernel.linear_swiglu), measured against two library GEMMs plus torch's SiLU
# and product at the C4 shape
FUSED_SWIGLU_MAX_K = 1024
_PLAIN_FORWARD = object()  # restore marker: drop the instance's fused forward


def _is_silu(fn):
    return isinstance(fn, nn.SiLU) or type(fn).__name__ in ("SiLUActivation", "SiLU")


def _gated_mlp_fusable(mlp):
    return (all(isinstance(getattr(mlp, n, None), nn.Linear) for n in ("gate_proj", "up_proj", "down_proj"))
            and mlp.gate_proj.bias is None and mlp.up_proj.bias is None and _is_silu(getattr(mlp, "act_fn", None))
            and mlp.gate_proj.weight.shape == mlp.up_proj.weight.shape)


def _swiglu_weight_cache(mlp):
    """The interleaved [gate; up] weight of kernel.linear_swiglu, rebuilt when
    either weight changes (version, storage, dtype or device)."""
    wg, wu = mlp.gate_proj.weight, mlp.up_proj.weight
    key = (wg._version, wu._version, wg.data_ptr(), wu.data_ptr(), wg.dtype, wg.device)
    cache = mlp.__dict__.get("_swiglu_cache")
    if cache is None or cache[0] != key:
        with torch.no_grad():
            cache = (key, _kernel_mod.swiglu_weight(wg.detach(), wu.detach()))
        mlp.__dict__["_swiglu_cache"] = cache
    return cache[1]


def _gated_mlp_act(mlp, x):
    """act_fn(gate_proj(x)) * up_proj(x) of a Qwen3MLP: one HIP kernel (the
    SiLU and the product on the GEMM's fp32 accumulators) on the no-grad
    device path, torch's modules otherwise."""
    if (not torch.is_grad_enabled() and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)
            and x.size(-1) <= FUSED_SWIGLU_MAX_K and mlp.gate_proj.weight.size(0) % 128 == 0):
        w = _swiglu_weight_cache(mlp)
        if _kernel_mod.linear_swiglu_usable(x, w):
            return _kernel_mod.linear_swiglu(x, w)
    return mlp.act_fn(mlp.gate_proj(x)) * mlp.up_proj(x)


def _fused_gated_mlp_forward(mlp, x):
    """Qwen3MLP.forward with its gate / up half from _gated_mlp_act."""
    return mlp.down_proj(_gated_mlp_act(mlp, x))


def _fuse_block_mlp(block, saved):
    mlp = getattr(block, "mlp", None)
    if mlp is None or "forward" in mlp.__dict__ or not _gated_mlp_fusable(mlp):
        return
    mlp.forward = lambda x, _m=mlp: _fused_gated_mlp_forward(_m, x)
    saved.append((mlp, "forward", _PLAIN_FORWARD))


# transformers' RMSNorm classes with Qwen3RMSNorm's function
# (weight * round(x * rsqrt(mean(x^2) + eps))); Qwen3.5's (1 + w) norm is not one
_RMSNORM_CLASSES = ("Qwen3RMSNorm", "Qwen2RMSNorm", "LlamaRMSNorm")


def _rmsnorm_fusable(mod):
    w = getattr(mod, "weight", None)
    return (type(mod).__name__ in _RMSNORM_CLASSES and isinstance(w, torch.Tensor) and w.dim() == 1
            and hasattr(mod, "variance_epsilon"))


def _fused_rmsnorm_forward(mod, x):
    """Qwen3RMSNorm.forward as one HIP kernel (fp32 statistics, the same two
    roundings) on the no-grad device path; torch's ops otherwise."""
    C = x.size(-1)
    if (not torch.is_grad_enabled() and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)
            and mod.weight.dtype == x.dtype and C % 2 == 0 and C <= 2048 and x.is_contiguous()):
        return _kernel_mod.add_rmsnorm_(x, None, mod.weight, mod.variance_epsilon)
    input_dtype = x.dtype
    h = x.to(torch.float32)
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + mod.variance_epsilon)
    return mod.weight * h.to(input_dtype)


def _fuse_norm(mod, saved):
    if mod is None or "forward" in mod.__dict__ or not _rmsnorm_fusable(mod):
        return
    mod.forward = lambda x, _m=mod: _fused_rmsnorm_forward(_m, x)
    saved.append((mod, "forward", _PLAIN_FORWARD))


def _fused_decoder_forward(layer, hidden_states, attention_mask=None, position_ids=None, past_key_values=None,
                           use_cache=False, position_embeddings=None, **kwargs):
    """Qwen3DecoderLayer.forward with both residual additions fused, on the
    no-grad device path (the original forward otherwise): the post-attention
    one inside the post-attention RMSNorm's kernel (saf_add_rmsnorm: the
    attention output, a fresh tensor, becomes residual + attention in place,
    one rounding as torch's add, and the norm reads it), the last one inside
    the down projection's GEMM (that sum += act W_down^T, beta = 1).  The
    layer's input is not written."""
    norm = layer.post_attention_layernorm
    x = hidden_states
    if not (not torch.is_grad_enabled() and x.is_cuda and x.dtype in (torch.bfloat16, torch.float16)
            and x.is_contiguous() and norm.weight.dtype == x.dtype and x.size(-1) % 2 == 0 and x.size(-1) <= 2048):
        return type(layer).forward(layer, hidden_states, attention_mask=attention_mask, position_ids=position_ids,
                                   past_key_values=past_key_values, use_cache=use_cache,
                                   position_embeddings=position_embeddings, **kwargs)
    h = layer.input_layernorm(x)
    h, _ = layer.self_attn(hidden_states=h, attention_mask=attention_mask, position_ids=position_ids,
                           past_key_values=past_key_values, use_cache=use_cache,
                           position_embeddings=position_embeddings, **kwargs)
    if not h.is_contiguous() or h.shape != x.shape:
        h = h + x
        return h + layer.mlp(layer.post_attention_layernorm(h))
    normed = _kernel_mod.add_rmsnorm_(h, x, norm.weight, norm.variance_epsilon)
    mlp = layer.mlp
    if _gated_mlp_fusable(mlp) and mlp.down_proj.bias is None and mlp.down_proj.weight.dtype == h.dtype:
        # the block's last residual addition inside the down projection's GEMM
        # (h += act W_down^T: beta = 1, one rounding), h being the fresh sum
        act = _gated_mlp_act(mlp, normed)
        C = h.size(-1)
        h.view(-1, C).addmm_(act.reshape(-1, act.size(-1)), mlp.down_proj.weight.t())
        return h
    out = mlp(normed)
    out += h
    return out


def _fuse_decoder_layer(block, saved):
    if (type(block).__name__ != "Qwen3DecoderLayer" or "forward" in block.__dict__
            or not _rmsnorm_fusable(getattr(block, "post_attention_layernorm", None))
            or not hasattr(block, "input_layernorm") or not hasattr(block, "mlp")):
        return
    block.forward = lambda *a, _b=block, **k: _fused_decoder_forward(_b, *a, **k)
    saved.append((block, "forward", _PLAIN_FORWARD))


def convert_targets_to_hybrid(model, targets, mean_attn, head_masks, device, dtype,
                              use_triton=True, assume_causal_prefill=False, decomp=None,
                              fuse_live_only=False):
    """Replace each target's attention module by its hybrid counterpart.

    mean_attn: per-target (n_heads, T, T) dense priors, or None with ``decomp``
    = per-target (alpha, rho) pairs of (n_heads, S) fp32 tensors (None entries
    for targets with no frozen head).  Targets with no frozen head stay as
    they are unless fuse_live_only (an extension) asks for the HIP flash path
    there too.  Returns the list restore_originals takes."""
    n = len(targets)
    if mean_attn is None and decomp is None:
        raise ValueError("need mean_attn or decomp")
    priors = [None] * n if mean_attn is None else list(mean_attn)
    if len(priors) != n or len(head_masks) != n or (decomp is not None and len(decomp) != n):
        raise ValueError("targets, priors, head_masks (and decomp) must have one entry per target")
    blocks = None
    saved = []
    for i, (t, mask) in enumerate(zip(targets, head_masks)):
        parent = t.parent
        if parent is None:
            blocks = blocks or iter_blocks(model)
            parent = blocks[t.layer_idx]
        original = getattr(parent, t.attr_name)
        # the block's gated MLP and RMSNorms (same functions, one HIP kernel
        # each on the prefill path) whatever its heads
        _fuse_block_mlp(parent, saved)
        _fuse_norm(getattr(parent, "input_layernorm", None), saved)
        _fuse_norm(getattr(parent, "post_attention_layernorm", None), saved)
        _fuse_decoder_layer(parent, saved)
        if not bool(torch.as_tensor(mask).any()) and not fuse_live_only:
            saved.append((parent, t.attr_name, None))
            continue
        cls = get_hybrid_class_for(original)
        if cls is None:
            raise RuntimeError(f"No hybrid class registered for {type(original).__name__}")
        hybrid = cls(original, priors[i], mask, device, dtype, use_triton=use_triton,
                     assume_causal_prefill=assume_causal_prefill,
                     decomp=None if decomp is None else decomp[i])
        hybrid.fuse_live_only = bool(fuse_live_only)
        hybrid.train(original.training)
        setattr(parent, t.attr_name, hybrid)
        saved.append((parent, t.attr_name, original))
    # the backbone's final norm
    backbone = getattr(model, "model", model)
    _fuse_norm(getattr(backbone, "norm", None), saved)
    return saved


def restore_originals(saved):
    """Undo convert_targets_to_hybrid."""
    for parent, attr_name, original in saved:
        if original is _PLAIN_FORWARD:
            parent.__dict__.pop(attr_name, None)
            parent.__dict__.pop("_swiglu_cache", None)
        elif original is not None:
            setattr(parent, attr_name, original)
