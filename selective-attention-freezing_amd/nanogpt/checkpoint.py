"""Load the reference's nanoGPT checkpoints (the released SAF exports) into
this build's GPT.

Follows /root/reference/nanogpt/eval_nanogpt_logprobs.py:51-104
(``build_config_from_ckpt``, ``load_model``) and the lazy-buffer handling of
/root/reference/nanogpt/model.py:900-911, with four differences that follow
from this build:

* the file is read with ``torch.load(weights_only=True)``: tensors, dicts,
  lists, strings and numbers load; a checkpoint that pickles other objects
  is refused by torch with an error rather than executed;
* dense frozen patterns are stored compactly here: the reference's
  ``dyn_pattern`` is (n_head, S, S) with zero rows for live heads (or absent
  in decomposed mode until a dense freeze); this build keeps one (S, S) slot
  per dense-frozen head (``dyn_pattern`` (n_slots, S, S) + ``dyn_pattern_slot``),
  so the loader moves each dense-frozen head's matrix, bit for bit, into its
  slot, in head order;
* ``dyn_rho_band`` (the reference's (n_head, 64, S) derived band) is dropped:
  the HIP kernels read rho directly;
* the reference's Block names its attention ``main_block``
  (/root/reference/nanogpt/model.py:1219), so its export keys are
  ``transformer.h.{i}.main_block.*``; this build's Block calls the module
  ``attn``, and the loader renames the keys.

Only the architecture this build implements loads: standard softmax heads
with dynamic per-head freezing (any fraction frozen, dense or decomposed
priors).  Checkpoints of the reference's randomisation ablations (random
heads or layers, projection masks, attention masks, packed prune / uniform
layouts, state blocks) raise NotImplementedError naming the field.
"""
from __future__ import annotations

import dataclasses

import torch

from .model import GPT, GPTConfig

# GPTConfig defaults of the reference (/root/reference/nanogpt/model.py:1248-1285)
# for the fields this build reads; a checkpoint's model_args override them.
REFERENCE_DEFAULTS = {
    "block_size": 1024, "vocab_size": 50304, "n_layer": 12, "n_head": 12, "n_embd": 768,
    "dropout": 0.0, "bias": True, "position_encoding": "learned_absolute", "rope_base": 10000.0,
    "rand_attn_dynamic": False, "rand_attn_prior_repr": "dense", "freeze_pattern_dtype": "float32",
    "rand_seed": 42,
}

# Reference fields whose non-default values select architectures outside the
# prefill hot path (randomisation ablations A-G, state blocks); the value
# listed is the one this build implements.
_REQUIRED = {
    "state_size": 0, "shared_weights": False, "rand_head_rate": 0.0, "rand_layer_rate": 0.0,
    "rand_components": "none", "rand_attn_mask_rate": 0.0, "rand_attn_head_rate": 0.0,
    "rand_attn_pattern": "none", "random_proj": False, "block_type": "selfattention",
}

_PREFIX = "_orig_mod."
# The reference's Block holds its attention as ``main_block``
# (/root/reference/nanogpt/model.py:1219); this build's Block calls it ``attn``.
_REF_ATTN, _ATTN = ".main_block.", ".attn."


def build_config_from_ckpt(ckpt) -> GPTConfig:
    """GPTConfig from a checkpoint's ``model_args`` (or ``model_config``),
    tolerant of the reference's renamed fields, with the reference's defaults
    for absent ones (eval_nanogpt_logprobs.py:51-74)."""
    ma = dict(ckpt.get("model_args", ckpt.get("model_config", {})) or {})
    if not ma:
        raise ValueError("Checkpoint has neither model_args nor model_config")
    if "rand_mask_rate" in ma:  # renamed field of older exports
        ma["rand_proj_mask_rate"] = ma.pop("rand_mask_rate")
    cfg_dict = ckpt.get("config", {}) or {}
    # fields some exports persist only in the full config dict
    # (eval_nanogpt_logprobs.py:66-70)
    for k in ("rand_attn_prior_path", "rand_attn_pattern_sharing", "rand_attn_pattern",
              "rand_attn_head_rate", "rand_attn_head_rate_per_layer"):
        if k not in ma and cfg_dict.get(k) is not None:
            ma[k] = cfg_dict[k]
    if ma.get("rand_attn_pattern") == "":   # the reference treats "" as "none" (model.py:457)
        ma["rand_attn_pattern"] = "none"
    if ma.get("rand_attn_head_rate_per_layer"):
        raise NotImplementedError(
            f"checkpoint field rand_attn_head_rate_per_layer={ma['rand_attn_head_rate_per_layer']!r} "
            "selects per-layer random attention heads (Method H), which this build does not implement")
    for k, want in _REQUIRED.items():
        if k in ma and ma[k] is not None and ma[k] != want:
            raise NotImplementedError(f"checkpoint field {k}={ma[k]!r} selects an architecture this build "
                                      f"does not implement (needs {want!r})")
    if ma.get("rand_components", "none") != "none" and ma.get("rand_proj_mask_rate", 1.0) != 0.0:
        raise NotImplementedError("checkpoints with randomised projections are not supported")
    fields = {f.name for f in dataclasses.fields(GPTConfig)}
    args = dict(REFERENCE_DEFAULTS)
    args.update({k: v for k, v in ma.items() if k in fields})
    # a non-dynamic reference model has no freeze buffers; this build always
    # carries them (all heads live), in the cheaper decomposed layout
    if not args.pop("rand_attn_dynamic"):
        args["rand_attn_prior_repr"] = "decomposed" if args["block_size"] % 64 == 0 else "dense"
    return GPTConfig(**args)


def _layout_check(ckpt):
    layout = ckpt.get("attention_layout")
    if layout is None and ckpt.get("intervention"):
        iv = ckpt["intervention"]
        mode = iv.get("physical_mode", iv.get("mode"))
        layout = {"mode": {"prune_gate_taylor": "prune", "random_mean": "mean"}.get(mode, mode)}
    if layout is not None and layout.get("mode") not in ("ordinary", "mean"):
        raise NotImplementedError(f"attention layout {layout.get('mode')!r} (packed heads) is not supported")


def _attn_key(name):
    """This build's key for a reference state-dict key: the compile prefix
    stripped and the block's ``main_block.`` renamed ``attn.``."""
    if name.startswith(_PREFIX):
        name = name[len(_PREFIX):]
    if name.startswith("transformer.h.") and _REF_ATTN in name:
        name = name.replace(_REF_ATTN, _ATTN, 1)
    return name


@torch.no_grad()
def convert_state_dict(state_dict, model: GPT):
    """Reference state dict (keys ``transformer.h.{i}.main_block.*``, with or
    without torch.compile's ``_orig_mod.``) -> this build's, in place on
    ``model``'s pattern slots.  Returns the dict to pass to
    ``model.load_state_dict(..., strict=True)``."""
    sd = {}
    for k, v in state_dict.items():
        name = _attn_key(k)
        if name.startswith("transformer.h.") and ".attn.dyn_pattern_slot" in name:
            raise ValueError(f"{k}: not a reference export (this build's own pattern-slot table)")
        sd[name] = v
    out = {}
    for name, v in sd.items():
        if name.endswith(".attn.dyn_rho_band") or name.endswith(".attn.bias"):
            continue
        if not name.endswith(".attn.dyn_pattern"):
            out[name] = v
    for i, blk in enumerate(model.transformer.h):
        a = blk.attn
        pre = f"transformer.h.{i}.attn."
        H, S = a.n_head, a.block_size
        frozen = sd.get(pre + "dyn_frozen")
        if frozen is None:  # non-dynamic reference model: every head live
            out[pre + "dyn_frozen"] = torch.zeros(H, dtype=torch.bool)
            out[pre + "dyn_decomp"] = torch.zeros(H, dtype=torch.bool)
            if a.dyn_alpha is not None:
                for n in ("dyn_alpha", "dyn_rho", "dyn_z"):
                    out[pre + n] = torch.zeros(H, S)
            out[pre + "dyn_pattern_slot"] = torch.full((H,), -1, dtype=torch.int32)
            a.dyn_pattern = None
            continue
        # the dense representation registers no dyn_decomp (model.py:659-672)
        decomp = sd.get(pre + "dyn_decomp", torch.zeros(H, dtype=torch.bool))
        out[pre + "dyn_decomp"] = decomp
        if a.dyn_alpha is not None and pre + "dyn_alpha" not in sd:
            for n in ("dyn_alpha", "dyn_rho", "dyn_z"):
                out[pre + n] = torch.zeros(H, S)
        dense = [h for h in range(H) if bool(frozen[h]) and not bool(decomp[h])]
        slot = torch.full((H,), -1, dtype=torch.int32)
        if dense:
            full = sd.get(pre + "dyn_pattern")
            if full is None or full.dim() != 3 or full.size(0) != H:
                raise ValueError(f"layer {i}: dense-frozen heads {dense} need a (n_head, S, S) dyn_pattern")
            # padded slots on the model's device; load_state_dict copies the
            # compact matrices into them, so the layout survives the load
            a.dyn_pattern = a._alloc_patterns(len(dense), a._pattern_dtype, a.dyn_frozen.device)
            compact = torch.empty(len(dense), S, S, dtype=a._pattern_dtype)
            for s, h in enumerate(dense):
                compact[s] = full[h]
                slot[h] = s
            out[pre + "dyn_pattern"] = compact
        else:
            a.dyn_pattern = None
        out[pre + "dyn_pattern_slot"] = slot
        a._fz_dirty = True
    return out


def reference_state_dict(model: GPT, compile_prefix: bool = False):
    """This build's GPT state in the reference's export layout, the inverse
    of convert_state_dict.  Attention keys are ``transformer.h.{i}.main_block.*``
    and each layer carries exactly the buffers the reference's dynamic
    CausalSelfAttention saves (nanogpt/model.py:647-672, :735-764):
      * ``dyn_frozen``;
      * dense representation: ``dyn_pattern`` (n_head, S, S), always, with
        zero rows for heads that are not dense-frozen;
      * decomposed representation: ``dyn_decomp``, ``dyn_alpha``, ``dyn_rho``,
        ``dyn_z``; the lazily created ``dyn_rho_band`` (n_head, 64, S) (rows
        rho[r - u + S - 64], -inf outside [0, S): kernel/fused_attn.py:65-80)
        when a decomposed head is frozen, and ``dyn_pattern`` when a dense one
        is.
    No pattern-slot table.  compile_prefix adds torch.compile's ``_orig_mod.``."""
    from kernel.fused_attn import make_rho_band
    decomposed = model.config.rand_attn_prior_repr == "decomposed"
    own = {"dyn_pattern", "dyn_pattern_slot", "dyn_decomp", "dyn_alpha", "dyn_rho", "dyn_z"}
    out = {}
    for k, v in model.state_dict().items():
        if k.startswith("transformer.h.") and _ATTN in k:
            if k.rsplit(".", 1)[1] in own:
                continue
            k = k.replace(_ATTN, _REF_ATTN, 1)
        out[k] = v.detach().cpu().clone()
    for i, blk in enumerate(model.transformer.h):
        a = blk.attn
        pre = f"transformer.h.{i}.main_block."
        H, S = a.n_head, a.block_size
        frozen = a.dyn_frozen.cpu()
        dec = a.dyn_decomp.cpu() & frozen
        if decomposed:
            out[pre + "dyn_decomp"] = a.dyn_decomp.detach().cpu().clone()
            for n in ("dyn_alpha", "dyn_rho", "dyn_z"):
                out[pre + n] = getattr(a, n).detach().cpu().clone()
            if bool(dec.any()):
                # zero rows except the decomposed-frozen heads' (model.py:757-763)
                band = torch.zeros(H, 64, S, dtype=a.dyn_rho.dtype)
                idx = dec.nonzero(as_tuple=True)[0]
                band[idx] = make_rho_band(a.dyn_rho.detach().cpu()[idx])
                out[pre + "dyn_rho_band"] = band
        dense = frozen & ~dec
        if not decomposed or bool(dense.any()):
            dtype = a._pattern_dtype if a.dyn_pattern is None else a.dyn_pattern.dtype
            full = torch.zeros(H, S, S, dtype=dtype)
            for h in range(H):
                slot = int(a.dyn_pattern_slot[h])
                if slot >= 0 and bool(dense[h]):
                    full[h] = a.dyn_pattern[slot].cpu()
            out[pre + "dyn_pattern"] = full
    if compile_prefix:
        out = {_PREFIX + k: v for k, v in out.items()}
    return out


def save_reference_checkpoint(model: GPT, path, **extra):
    """Write ``model`` as a checkpoint file in the reference's layout
    (``model`` + ``model_args``, as nanogpt/train.py saves it), loadable by
    load_model here and, for the fields the reference reads, by
    eval_nanogpt_logprobs.py:load_model there.  ``extra`` entries (e.g.
    iter_num) are stored beside them."""
    cfg = model.config
    model_args = {f.name: getattr(cfg, f.name) for f in dataclasses.fields(GPTConfig)}
    ck = {"model": reference_state_dict(model, compile_prefix=True), "model_args": model_args}
    ck.update(extra)
    torch.save(ck, path)
    return path


def load_model(ckpt_path, device, dtype=None):
    """(model, cfg, ckpt) for a reference checkpoint file, in eval mode on
    ``device`` (and ``dtype`` if given; alpha / rho / z stay fp32)
    (eval_nanogpt_logprobs.py:77-104)."""
    ckpt = torch.load(ckpt_path, map_location="cpu", weights_only=True)
    _layout_check(ckpt)
    cfg = build_config_from_ckpt(ckpt)
    model = GPT(cfg)
    model.load_state_dict(convert_state_dict(ckpt["model"], model), strict=True)
    model.eval()
    model.to(device)
    if dtype is not None:
        model.to(dtype=dtype)
    return model, cfg, ckpt
