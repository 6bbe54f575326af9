"""Writes golden vectors for the composed GPT forward from the reference's own
CPU code (waylonli/Selective-Attention-Freezing, nanogpt/model.py).

What only an import of the reference pins: the composition of its GPT forward
on the frozen-head path -- LayerNorm eps, exact GELU, weight tying, RoPE cast
points, the split fallback of _attend_cheap (nanogpt/model.py:1017-1061) and
the eager override path (:824-844), and the storage of decomposed freezes
(:735-764).  The attention arithmetic itself is pinned without the reference
(tests/test_oracle.py).

Run in the container where the reference is mounted (never on the GPU box):
    python tests/golden/make_golden.py            # both fixtures
    python tests/golden/make_golden.py export     # the export fixture only
It writes
  * tests/golden/gpt_forward_small.npz: fp16-representable weights, tokens,
    the freeze state and both paths' fp32 logits;
  * tests/golden/gpt_export_small.npz: the reference's own state dicts, key
    names unrenamed (transformer.h.{i}.main_block.*, every buffer the
    reference registers and saves: dyn_frozen, dyn_decomp, dyn_alpha, dyn_rho,
    dyn_z, the lazily created dyn_rho_band and dyn_pattern, and the dense
    representation's (n_head, S, S) dyn_pattern), the GPTConfig fields as
    JSON (what nanogpt/train.py stores as model_args), tokens and the split
    path's fp32 logits, for a decomposed-representation model (a dense, a
    generic decomposed and a causal-mean freeze) and a dense-representation
    model (one dense freeze, one layer with none).
"""
import dataclasses
import json
import os
import sys

import numpy as np

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "gpt_forward_small.npz")
OUT_EXPORT = os.path.join(HERE, "gpt_export_small.npz")


def _ref_model():
    sys.path[:0] = [os.path.join(REF, "nanogpt"), REF]
    import model as ref_model  # the reference's nanogpt/model.py
    return ref_model


def _export_entries(tag, m, cfg, x):
    """Fixture entries of one reference model: its state dict under
    '<tag>/sd/<key>' (floating tensors stored as float16 when exactly
    representable, flagged in '<tag>/f16keys'), model_args JSON, tokens and
    the split path's all-position logits."""
    import torch
    with torch.no_grad():
        logits = m.forward_all_positions(x).float().numpy()
    out = {f"{tag}/model_args": np.array(json.dumps(dataclasses.asdict(cfg))),
           f"{tag}/tokens": x.numpy().astype(np.int64), f"{tag}/logits_split": logits}
    f16 = []
    for k, v in m.state_dict().items():
        v = v.detach().cpu()
        if v.is_floating_point() and torch.equal(v.half().float(), v):
            out[f"{tag}/sd/{k}"] = v.half().numpy()
            f16.append(k)
        else:
            out[f"{tag}/sd/{k}"] = v.numpy()
    out[f"{tag}/f16keys"] = np.array(json.dumps(f16))
    return out


def export_fixture():
    import torch
    ref_model = _ref_model()
    out = {}
    # decomposed representation: dense freeze (layer 0, lazily creates that
    # layer's (n_head, S, S) dyn_pattern), generic decomposed (layer 1) and
    # causal-mean (layer 2) freezes (each creates its layer's dyn_rho_band)
    torch.manual_seed(31337)
    cfg = ref_model.GPTConfig(block_size=64, vocab_size=96, n_layer=3, n_head=2, n_embd=64,
                              dropout=0.0, bias=False, position_encoding="rope",
                              rand_attn_dynamic=True, rand_attn_prior_repr="decomposed")
    m = ref_model.GPT(cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(p.half().float())
    g = torch.Generator().manual_seed(11)
    T = 64
    attn = [blk.main_block for blk in m.transformer.h]
    attn[0].freeze_heads([0], torch.rand(1, T, T, generator=g))
    attn[1].freeze_heads_decomposed([1], torch.randn(1, T, generator=g) * 0.5,
                                    torch.randn(1, T, generator=g) * 0.5)
    zeros = torch.zeros(1, T)
    attn[2].freeze_heads_decomposed([0], zeros, zeros)
    x = torch.randint(0, cfg.vocab_size, (2, T), generator=g)
    out.update(_export_entries("decomposed", m, cfg, x))

    # dense representation: every layer registers its (n_head, S, S)
    # dyn_pattern at construction; layer 1 stays unfrozen (zero buffer)
    torch.manual_seed(4242)
    cfg = ref_model.GPTConfig(block_size=64, vocab_size=96, n_layer=2, n_head=2, n_embd=64,
                              dropout=0.0, bias=True, position_encoding="rope",
                              rand_attn_dynamic=True, rand_attn_prior_repr="dense")
    m = ref_model.GPT(cfg).eval()
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(p.half().float())
            if p.dim() == 1 and not torch.count_nonzero(p):   # biases: non-zero, fp16 values
                p.copy_((torch.randn(p.shape, generator=g) * 0.02).half().float())
    m.transformer.h[0].main_block.freeze_heads([1], torch.rand(1, T, T, generator=g))
    x = torch.randint(0, cfg.vocab_size, (2, T), generator=g)
    out.update(_export_entries("dense", m, cfg, x))
    np.savez_compressed(OUT_EXPORT, **out)
    print(f"wrote {OUT_EXPORT} ({os.path.getsize(OUT_EXPORT)} bytes)")


def main():
    import torch
    ref_model = _ref_model()

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
    if sys.argv[1:] != ["export"]:
        main()
    export_fixture()
