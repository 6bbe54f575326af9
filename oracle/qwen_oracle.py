"""CPU restatement of the hybrid Qwen3 backbone forward (torch fp32).

TEST INFRASTRUCTURE ONLY: the model-level checker of the HIP path for the
GQA caller.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may use it.

Works on a plain state dict with transformers' Qwen3 parameter names and
restates, without importing any model class:
  transformers modeling_qwen3 (the installed 5.15.0; the reference pins
  5.2.0, /root/reference/requirements.txt:7): RMSNorm in fp32 with eps,
  per-head q_norm / k_norm before RoPE, default RoPE (inv_freq =
  theta^(-2i/hd), cos/sin of cat(freqs, freqs)), GQA by repeating KV heads,
  SiLU-gated MLP, pre-norm residual blocks, final norm -> last hidden state;
  the split path of the reference's hybrid Qwen3 attention
  (/root/reference/qwen/nanogpt/hybrid_prior_attention.py:586-640): live heads
  through causal softmax attention with scale hd^-0.5, frozen query heads as
  P @ V of their KV group, P the dense prior tril'ed and row-renormalised
  (:146-152) or exp(alpha[j] + rho[i-j] - z[i]) for decomposed priors
  (:128-140, :187-194).
Pinned by tests/golden/qwen_forward_small.npz, written by the reference's own
adapter on CPU (tests/golden/make_golden_qwen.py).

qwen35_attention restates one Qwen3.5 gated attention layer with frozen
query heads (the reference's Qwen3.5 adapter,
/root/reference/qwen/nanogpt/hybrid_prior_attention.py:205-470, over
transformers' Qwen3_5Attention): q_proj emits (query, gate) per head, q/k
RMSNorm with (1 + w) weights in fp32, RoPE on the first rotary_dim features
only, live heads as causal softmax attention, frozen heads as P @ V of their
KV group, every head's output times sigmoid(gate), then o_proj.  Pinned in
tests/test_qwen.py against transformers' own module with no head frozen and
by the invariant that a frozen head whose prior is its own softmax matrix
changes nothing.
"""
import math

import numpy as np
import torch
import torch.nn.functional as F

from . import saf_oracle as orc


def rms_norm(x, w, eps):
    x = x.float()
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def rope_cache(hd, T, theta, inv_freq=None):
    """cos, sin (T, hd) of the default RoPE; inv_freq overrides the
    frequencies theta^(-2i/hd) (e.g. with those of a model cast to bf16,
    whose inv_freq buffer transformers rounds along with the weights)."""
    inv = 1.0 / (theta ** (torch.arange(0, hd, 2, dtype=torch.int64).float() / hd)) if inv_freq is None \
        else inv_freq.float()
    freqs = torch.outer(torch.arange(T, dtype=torch.float32), inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos(), emb.sin()


def _rot(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(x, cos, sin):
    return x * cos + _rot(x) * sin


def dense_prior(p, dtype=torch.float32):
    """tril + row renormalisation of a dense prior (:146-152)."""
    p = p.to(dtype).tril()
    return p / p.sum(-1, keepdim=True).clamp_min(torch.finfo(dtype).tiny)


def frozen_patterns(fr, T):
    """(n_pattern, T, T) fp32 priors of a layer's frozen heads in ascending
    head order.  fr: {"mask": (H,) bool, "dense": (H, S, S)} or
    {"mask": ..., "alpha": (H, S), "rho": (H, S)}."""
    heads = [h for h in range(len(fr["mask"])) if fr["mask"][h]]
    if "dense" in fr:
        return dense_prior(torch.from_numpy(np.asarray(fr["dense"])[heads]).float())[:, :T, :T]
    a = np.asarray(fr["alpha"], dtype=np.float64)[heads]
    r = np.asarray(fr["rho"], dtype=np.float64)[heads]
    z = orc.decomposed_logz(a, r)
    return torch.from_numpy(np.nan_to_num(orc.decomp_pattern(a, r, z, T), nan=0.0)).float()


def attention(x, sd, p, cfg, fr, cos, sin):
    B, T, _ = x.shape
    H, HKV, hd, eps = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["eps"]
    lin = lambda name, t: F.linear(t, sd[p + name + ".weight"], sd.get(p + name + ".bias"))
    q = rms_norm(lin("q_proj", x).view(B, T, H, hd), sd[p + "q_norm.weight"], eps).transpose(1, 2)
    k = rms_norm(lin("k_proj", x).view(B, T, HKV, hd), sd[p + "k_norm.weight"], eps).transpose(1, 2)
    v = lin("v_proj", x).view(B, T, HKV, hd).transpose(1, 2)
    q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    g = H // HKV
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    att = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(hd))
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    att = att.masked_fill(~causal, float("-inf")).softmax(-1)
    if fr is not None and bool(np.any(fr["mask"])):
        heads = [h for h in range(H) if fr["mask"][h]]
        att[:, heads] = frozen_patterns(fr, T).unsqueeze(0).expand(B, -1, -1, -1)
    y = (att @ v).transpose(1, 2).reshape(B, T, H * hd)
    return lin("o_proj", y)


@torch.no_grad()
def qwen_forward(sd, cfg, freeze, idx, layers=None, inv_freq=None):
    """Last hidden state (B, T, hidden) of the hybrid Qwen3 backbone.

    sd: float32 state dict (transformers names); cfg: dict with n_layers,
    n_heads, n_kv_heads, head_dim, eps, rope_theta; freeze: per-layer records
    for frozen_patterns() or None; layers: run only these layer indices;
    inv_freq: the model's RoPE frequencies if they are not theta's exact ones
    (transformers' rotary inv_freq buffer is cast with the model, so a bf16
    model rotates with bf16-rounded frequencies, computed in fp32)."""
    x = sd["model.embed_tokens.weight"][idx].float()
    T = idx.size(1)
    cos, sin = rope_cache(cfg["head_dim"], T, cfg["rope_theta"], inv_freq)
    for l in (range(cfg["n_layers"]) if layers is None else layers):
        p = f"model.layers.{l}."
        h = rms_norm(x, sd[p + "input_layernorm.weight"], cfg["eps"])
        x = x + attention(h, sd, p + "self_attn.", cfg, None if freeze is None else freeze[l], cos, sin)
        h = rms_norm(x, sd[p + "post_attention_layernorm.weight"], cfg["eps"])
        m = F.silu(F.linear(h, sd[p + "mlp.gate_proj.weight"])) * F.linear(h, sd[p + "mlp.up_proj.weight"])
        x = x + F.linear(m, sd[p + "mlp.down_proj.weight"])
    return rms_norm(x, sd["model.norm.weight"], cfg["eps"])


def rms_norm_offset(x, w, eps):
    """Qwen3.5 RMSNorm: x / rms(x) * (1 + w) in fp32."""
    x = x.float()
    return (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)) * (1.0 + w.float())


def apply_partial_rope(x, cos, sin):
    """Half rotation on the first cos.shape[-1] features, the rest passed through."""
    r = cos.shape[-1]
    return torch.cat([apply_rope(x[..., :r], cos, sin), x[..., r:]], dim=-1)


def qwen35_attention(x, sd, p, cfg, fr, cos, sin, return_probs=False):
    """One Qwen3.5 gated attention layer (B, T, hidden) -> (B, T, hidden),
    fp32.  sd: state dict with the layer's q_proj / k_proj / v_proj / o_proj
    and q_norm / k_norm weights under prefix p; cfg: n_heads, n_kv_heads,
    head_dim, eps; fr: None or {"mask": (H,) bool, "dense"/"alpha"+"rho"} as
    for frozen_patterns; cos / sin: (T, rotary_dim)."""
    B, T, _ = x.shape
    H, HKV, hd, eps = cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["eps"]
    lin = lambda name, t: F.linear(t, sd[p + name + ".weight"], sd.get(p + name + ".bias"))
    qg = lin("q_proj", x.float()).view(B, T, H, 2 * hd)
    q, gate = qg[..., :hd], qg[..., hd:]
    q = rms_norm_offset(q, sd[p + "q_norm.weight"], eps).transpose(1, 2)
    k = rms_norm_offset(lin("k_proj", x.float()).view(B, T, HKV, hd), sd[p + "k_norm.weight"], eps).transpose(1, 2)
    v = lin("v_proj", x.float()).view(B, T, HKV, hd).transpose(1, 2)
    q, k = apply_partial_rope(q, cos, sin), apply_partial_rope(k, cos, sin)
    g = H // HKV
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    att = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(hd))
    causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
    att = att.masked_fill(~causal, float("-inf")).softmax(-1)
    probs = att.clone()
    if fr is not None and bool(np.any(fr["mask"])):
        heads = [h for h in range(H) if fr["mask"][h]]
        att[:, heads] = frozen_patterns(fr, T).unsqueeze(0).expand(B, -1, -1, -1)
    y = (att @ v).transpose(1, 2) * torch.sigmoid(gate)
    out = lin("o_proj", y.reshape(B, T, H * hd))
    return (out, probs) if return_probs else out
