"""Qwen-style GQA prefill workload with frozen query heads.

Builds a random-init Hugging Face Qwen3 model locally (nothing is
downloaded) and converts its attention layers with the hybrid adapter, as
/root/reference/qwen/nanogpt/bench_qwen_prefill_triton.py does for a
pretrained checkpoint:
  _nested_head_masks (:143-159)       per-layer frozen sets, nested in the rate
  _uniform_causal_priors (:121-140)   the causal-mean prior (dense) or, with
                                      repr="decomposed", alpha = rho = 0
  _backbone_forward (:168-177)        prefill to the backbone's last hidden
                                      state (no vocabulary projection)
The architecture defaults to the Qwen2.5-0.5B-sized GQA shape (24 layers,
hidden 896, 14 query / 2 KV heads, head_dim 64, MLP 4864) in the Qwen3
module family, i.e. with the per-head q/k RMSNorm, RoPE theta 1e6.
"""
from __future__ import annotations

import torch

from .hybrid_attention import convert_targets_to_hybrid, discover_softmax_attention


def qwen_config(n_layers=24, hidden=896, n_heads=14, n_kv_heads=2, head_dim=64,
                intermediate=4864, vocab=151936, rope_theta=1e6, max_positions=32768,
                attn_implementation="sdpa"):
    from transformers import Qwen3Config
    cfg = Qwen3Config(hidden_size=hidden, num_attention_heads=n_heads,
                      num_key_value_heads=n_kv_heads, head_dim=head_dim,
                      num_hidden_layers=n_layers, intermediate_size=intermediate,
                      vocab_size=vocab, rope_theta=rope_theta,
                      max_position_embeddings=max_positions, use_cache=False,
                      attn_implementation=attn_implementation)
    return cfg


def build_model(cfg, device="cuda", dtype=torch.bfloat16, seed=1337):
    """Random-init Qwen3ForCausalLM (transformers' own N(0, 0.02) init),
    drawn on the CPU from `seed` and then moved, so the host reproduces the
    device's weights exactly."""
    from transformers import Qwen3ForCausalLM
    torch.manual_seed(seed)
    with torch.device("cpu"):
        model = Qwen3ForCausalLM(cfg)
    model = model.to(device=device, dtype=dtype).eval()
    model.config.use_cache = False
    return model


def n_frozen_for(rate, n_heads):
    """round(rate * H) with Python's rounding (bench_qwen_prefill_triton.py:150).
    The reference clamps to [1, H-1]; rate 0 is kept here as an all-live run."""
    f = int(round(rate * n_heads))
    return 0 if rate == 0 else min(max(f, 1), n_heads - 1)


def nested_head_masks(rate, n_layers, n_heads, seed=1337):
    """Per-layer frozen masks: randperm(H, seed + 104729 * layer)[:f] (:143-159)."""
    f = n_frozen_for(rate, n_heads)
    masks = []
    for layer in range(n_layers):
        g = torch.Generator(device="cpu")
        g.manual_seed(seed + 104729 * layer)
        order = torch.randperm(n_heads, generator=g)
        m = torch.zeros(n_heads, dtype=torch.bool)
        m[order[:f]] = True
        masks.append(m)
    return masks


def uniform_causal_prior(T, device, dtype):
    """(T, T) row-stochastic causal mean pattern (:121-140)."""
    p = torch.ones((T, T), device=device, dtype=dtype).tril_()
    p.div_(torch.arange(1, T + 1, device=device, dtype=torch.float32).to(dtype)[:, None])
    return p


def convert_with_rate(model, rate, T, repr="decomposed", seed=1337, use_triton=True,
                      fuse_live_only=False):
    """Freeze round(rate * H) query heads per layer to the causal mean.

    repr "dense" stores the (T, T) prior per frozen head (state 1, dense P.V);
    "decomposed" passes alpha = rho = 0 (state 2), which the adapter
    classifies as the causal mean and runs through the closed-form scan."""
    cfg = model.config
    H, L = cfg.num_attention_heads, cfg.num_hidden_layers
    dev = next(model.parameters()).device
    dtype = next(model.parameters()).dtype
    targets = discover_softmax_attention(model)
    masks = nested_head_masks(rate, L, H, seed)[:len(targets)]
    if repr == "dense":
        prior = uniform_causal_prior(T, dev, dtype).view(1, T, T).expand(H, T, T)
        priors, decomp = [prior] * len(targets), None
    elif repr == "decomposed":
        zeros = torch.zeros(H, T, device=dev, dtype=torch.float32)
        priors, decomp = None, [(zeros, zeros)] * len(targets)
    else:
        raise ValueError(f"unknown prior representation {repr!r}")
    saved = convert_targets_to_hybrid(model, targets, priors, masks, dev, dtype,
                                      use_triton=use_triton, decomp=decomp,
                                      fuse_live_only=fuse_live_only)
    return saved, masks


def backbone_forward(backbone, input_ids):
    """Prefill without cache or mask; returns the last hidden state."""
    out = backbone(input_ids=input_ids, attention_mask=None, use_cache=False,
                   output_attentions=False, output_hidden_states=False, return_dict=True)
    return out.last_hidden_state
