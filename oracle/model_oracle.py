"""CPU restatement of the reference GPT forward with frozen heads (torch fp32).

TEST INFRASTRUCTURE ONLY: the model-level checker of the HIP path and the
CPU baseline that bench.py times on the host cores.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may use it.

It works on a plain state dict (no model classes shared with the product
package) and restates /root/reference/nanogpt/model.py:
  LayerNorm eps 1e-5 (:45-54), RoPE half rotation (:57-99), MLP with exact
  GELU (:1193-1207), pre-LN Block (:1237-1240), tied lm_head and last-position
  logits (:1337, :1401-1417), and two attention paths:
  path="eager"  _attend_dynamic (:824-844): full softmax, frozen heads
                overridden by their pattern, att @ v, then c_proj
  path="split"  the CPU branch of _attend_cheap (:1017-1061): V for all heads,
                frozen heads as (materialised pattern) @ V, live heads through
                causal SDPA, heads concatenated [live..., frozen...] and
                c_proj applied to the matching column permutation.
Decomposed patterns are materialised as exp(alpha[j] + rho[i-j] - z[i])
(:796-803); only the frozen heads' patterns are built.
"""
import math

import torch
import torch.nn.functional as F


def layer_norm(x, w, b):
    return F.layer_norm(x, w.shape, w, b, 1e-5)


def rope_cache(dim, T, base=10000.0, dtype=torch.float32):
    inv = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    freqs = torch.outer(torch.arange(T, dtype=torch.float32), inv)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype).view(1, 1, T, dim), emb.sin().to(dtype).view(1, 1, T, dim)


def _rot(x):
    x1, x2 = x.chunk(2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


def apply_rope(q, k, cos, sin):
    return q * cos + _rot(q) * sin, k * cos + _rot(k) * sin


def head_patterns(fr, heads, T):
    """(len(heads), T, T) fp32 patterns of frozen heads from a layer's freeze
    record {"patterns": {h: (T', T') tensor}, "decomp": {h: (alpha, rho, z)}}."""
    out = torch.zeros(len(heads), T, T)
    ar = torch.arange(T)
    dist = ar[:, None] - ar[None, :]
    for n, h in enumerate(heads):
        if h in fr.get("decomp", {}):
            a, r, z = (t.float() for t in fr["decomp"][h])
            lg = a[None, :T] + r[dist.clamp(min=0)] - z[:T, None]
            out[n] = torch.exp(lg.masked_fill(dist < 0, float("-inf")))
        else:
            out[n] = fr["patterns"][h][:T, :T].float()
    return out


def attention(x, sd, p, fr, cos, sin, n_head, path):
    B, T, C = x.shape
    hd = C // n_head
    lin = lambda name, t: F.linear(t, sd[p + name + ".weight"], sd.get(p + name + ".bias"))
    frozen = [bool(b) for b in fr["frozen"]]
    fz = [h for h in range(n_head) if frozen[h]]
    uf = [h for h in range(n_head) if not frozen[h]]
    v = lin("v_proj", x).view(B, T, n_head, hd).transpose(1, 2)
    if path == "eager" or not fz:
        q = lin("q_proj", x).view(B, T, n_head, hd).transpose(1, 2)
        k = lin("k_proj", x).view(B, T, n_head, hd).transpose(1, 2)
        if cos is not None:
            q, k = apply_rope(q, k, cos, sin)
        if not fz:
            y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        else:
            att = (q @ k.transpose(-2, -1)) * (1.0 / math.sqrt(hd))
            causal = torch.tril(torch.ones(T, T, dtype=torch.bool))
            att = att.masked_fill(~causal, float("-inf")).softmax(-1)
            att[:, fz] = head_patterns(fr, fz, T).to(att.dtype).unsqueeze(0).expand(B, -1, -1, -1)
            y = att @ v
        return lin("c_proj", y.transpose(1, 2).reshape(B, T, C))
    # split fallback: [live..., frozen...] head order, permuted c_proj columns
    yf = head_patterns(fr, fz, T).to(v.dtype).unsqueeze(0) @ v[:, fz]
    parts = []
    if uf:
        cols = torch.tensor([h * hd + d for h in uf for d in range(hd)])
        # linear_rows2: the live heads' rows of Wq / Wk and of their biases
        # (kernel/indexed_linear.py:131-135)
        rows = lambda n: None if sd.get(p + n) is None else sd[p + n][cols]
        q = F.linear(x, sd[p + "q_proj.weight"][cols], rows("q_proj.bias")).view(B, T, len(uf), hd).transpose(1, 2)
        k = F.linear(x, sd[p + "k_proj.weight"][cols], rows("k_proj.bias")).view(B, T, len(uf), hd).transpose(1, 2)
        if cos is not None:
            q, k = apply_rope(q, k, cos, sin)
        parts.append(F.scaled_dot_product_attention(q, k, v[:, uf], is_causal=True).transpose(1, 2))
    parts.append(yf.transpose(1, 2))
    y = torch.cat(parts, dim=2).reshape(B, T, C)
    perm = torch.tensor([h * hd + d for h in uf + fz for d in range(hd)])
    return F.linear(y, sd[p + "c_proj.weight"][:, perm], sd.get(p + "c_proj.bias"))


def block(x, sd, l, fr, cos, sin, n_head, path):
    p = f"transformer.h.{l}."
    h = layer_norm(x, sd[p + "ln_1.weight"], sd.get(p + "ln_1.bias"))
    x = x + attention(h, sd, p + "attn.", fr, cos, sin, n_head, path)
    h = layer_norm(x, sd[p + "ln_2.weight"], sd.get(p + "ln_2.bias"))
    h = F.gelu(F.linear(h, sd[p + "mlp.c_fc.weight"], sd.get(p + "mlp.c_fc.bias")))
    return x + F.linear(h, sd[p + "mlp.c_proj.weight"], sd.get(p + "mlp.c_proj.bias"))


@torch.no_grad()
def gpt_forward(sd, cfg, freeze, idx, path="split", all_positions=False, layers=None, positions=None,
                head=True):
    """Logits of the reference GPT on CPU fp32 (head=False: the final
    LayerNorm's output at the same positions instead).

    sd: float32 state dict; cfg: dict with n_layer, n_head, n_embd,
    position_encoding, rope_base; freeze: per-layer records
    {"frozen": (H,) bool, "patterns": {...}, "decomp": {...}}; layers: run
    only these layer indices (a bounded sample for timing); positions: the
    logits of these positions only (B, len(positions), vocab), for long
    sequences whose all-position logits would not fit; otherwise the last
    position (the reference's prefill output) or, with all_positions, all."""
    x = sd["transformer.wte.weight"][idx]
    T = idx.size(1)
    cos = sin = None
    if cfg.get("position_encoding", "rope") == "rope":
        cos, sin = rope_cache(cfg["n_embd"] // cfg["n_head"], T, cfg.get("rope_base", 10000.0))
    else:
        x = x + sd["transformer.wpe.weight"][:T]
    for l in (range(cfg["n_layer"]) if layers is None else layers):
        x = block(x, sd, l, freeze[l], cos, sin, cfg["n_head"], path)
    x = layer_norm(x, sd["transformer.ln_f.weight"], sd.get("transformer.ln_f.bias"))
    if positions is not None:
        x = x[:, torch.as_tensor(positions), :]
    elif not all_positions:
        x = x[:, -1:, :]
    return F.linear(x, sd["lm_head.weight"]) if head else x
