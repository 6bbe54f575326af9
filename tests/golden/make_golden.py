"""Writes golden vectors for the composed GPT forward from the reference's own
CPU code (waylonli/Selective-Attention-Freezing, nanogpt/model.py).

What only an import of the reference pins: the composition of its GPT forward
on the frozen-head path -- LayerNorm eps, exact GELU, weight tying, RoPE cast
points, the split fallback of _attend_cheap (nanogpt/model.py:1017-1061) and
the eager override path (:824-844), and the storage of decomposed freezes
(:735-764).  The attention arithmetic itself is pinned without the reference
(tests/test_oracle.py).

Run in the container where the reference is mounted (never on the GPU box):
    python tests/golden/make_golden.py
It writes tests/golden/gpt_forward_small.npz: fp16-representable weights,
tokens, the freeze state and both paths' fp32 logits.
"""
import os
import sys

import numpy as np

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gpt_forward_small.npz")


def main():
    sys.path[:0] = [os.path.join(REF, "nanogpt"), REF]
    import torch
    import model as ref_model  # the reference's nanogpt/model.py

    torch.manual_seed(20240)
    cfg = ref_model.GPTConfig(block_size=64, vocab_size=128, n_layer=3, n_head=2, n_embd=64,
                              dropout=0.0, bias=False, position_encoding="rope",
                              rand_attn_dynamic=True, rand_attn_prior_repr="decomposed")
    m = ref_model.GPT(cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(p.half().float())          # fp16-representable weights (small fixture)

    g = torch.Generator().manual_seed(7)
    T = 64
    attn = [blk.main_block for blk in m.transformer.h]
    dense = torch.rand(1, T, T, generator=g)
    attn[0].freeze_heads([1], dense)
    a1 = (torch.randn(1, T, generator=g) * 0.5)
    r1 = (torch.randn(1, T, generator=g) * 0.5)
    attn[1].freeze_heads_decomposed([0], a1, r1)
    zeros = torch.zeros(1, T)
    attn[2].freeze_heads_decomposed([1], zeros, zeros)     # causal mean
    x = torch.randint(0, cfg.vocab_size, (2, T), generator=g)

    with torch.no_grad():
        logits_split = m.forward_all_positions(x).float().numpy()
        for a in attn:
            a.set_capture(True, capture_logits=False, retain_attention=False)
        logits_eager = m.forward_all_positions(x).float().numpy()
        for a in attn:
            a.set_capture(False)

    out = {"tokens": x.numpy().astype(np.int64),
           "logits_split": logits_split, "logits_eager": logits_eager,
           "cfg": np.array([cfg.n_layer, cfg.n_head, cfg.n_embd, cfg.vocab_size, cfg.block_size])}
    sd = m.state_dict()
    for k, v in sd.items():
        if not v.is_floating_point() or k.endswith("wpe.weight"):
            continue
        name = k.replace(".main_block.", ".attn.")
        if any(s in name for s in ("dyn_", "_dyn_", "rotary")):
            continue
        out["w:" + name] = v.half().numpy()
    for l, a in enumerate(attn):
        out[f"frozen:{l}"] = a.dyn_frozen.numpy()
        out[f"decomp:{l}"] = a.dyn_decomp.numpy()
        out[f"alpha:{l}"] = a.dyn_alpha.numpy()
        out[f"rho:{l}"] = a.dyn_rho.numpy()
        out[f"z:{l}"] = a.dyn_z.numpy()
        if a.dyn_pattern is not None:
            out[f"pattern:{l}"] = a.dyn_pattern.numpy()
        if a.dyn_rho_band is not None:
            out[f"rho_band:{l}"] = a.dyn_rho_band.numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
