"""Writes golden vectors for the hybrid Qwen3 forward from the reference's own
CPU code (waylonli/Selective-Attention-Freezing,
qwen/nanogpt/hybrid_prior_attention.py with transformers' Qwen3 model).

What only an import of the reference pins: the composition of its Qwen3
hybrid forward on the split path (:586-640) -- the shrunken q_proj, q/k
RMSNorm before RoPE, GQA broadcast of raw K/V to the frozen query heads,
the dense prior's tril + renormalisation in the model dtype (:146-152), the
decomposed prior's z (:128-140) -- and its head routing tables (:154-171,
:526-528).  The attention arithmetic itself is pinned without the reference
(tests/test_oracle.py).

transformers is the installed 5.15.0; the reference pins 5.2.0
(requirements.txt:7).  The Qwen3 modules used here (RMSNorm, rotary
embedding, MLP, decoder layer) have the same arithmetic in both.

Run in the container where the reference is mounted (never on the GPU box):
    python tests/golden/make_golden_qwen.py
It writes tests/golden/qwen_forward_small.npz: fp16-representable weights,
tokens, the frozen masks and priors, the routing tables and the fp32 last
hidden states of the unconverted model, the dense-prior and the
decomposed-prior hybrid models.
"""
import os
import sys

import numpy as np

REF = "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qwen_forward_small.npz")

CFG = dict(hidden_size=64, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
           num_hidden_layers=2, intermediate_size=96, vocab_size=128, rope_theta=1e6,
           rms_norm_eps=1e-6)


def main():
    sys.path[:0] = [os.path.join(REF, "qwen", "nanogpt"), os.path.join(REF, "qwen")]
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM
    import hybrid_prior_attention as hpa   # the reference's adapter
    import test_prior_pretrained as tpp     # its target discovery

    torch.manual_seed(4242)
    cfg = Qwen3Config(**CFG, attn_implementation="sdpa", use_cache=False)
    model = Qwen3ForCausalLM(cfg).eval()
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(p.half().float())
            if p.dim() == 1:                 # norm weights: away from 1.0
                p.copy_((1.0 + 0.25 * torch.randn_like(p)).half().float())

    g = torch.Generator().manual_seed(11)
    B, T = 2, 64
    H = CFG["num_attention_heads"]
    ids = torch.randint(0, CFG["vocab_size"], (B, T), generator=g)
    masks = [torch.tensor([False, True, True, False]), torch.tensor([False, False, False, True])]
    dense = torch.rand(len(masks), H, T, T, generator=g).half().float()   # arbitrary priors
    alpha = (torch.randn(len(masks), H, T, generator=g) * 0.5)
    rho = (torch.randn(len(masks), H, T, generator=g) * 0.5)

    out = {"tokens": ids.numpy().astype(np.int64), "cfg_json": np.array(repr(CFG))}
    with torch.inference_mode():
        out["hidden_base"] = model.model(input_ids=ids, use_cache=False).last_hidden_state.numpy()
    targets = tpp.discover_softmax_attention(model)
    for name, kw in (("dense", dict(mean_attn=dense)),
                     ("decomp", dict(mean_attn=None, decomp=[(alpha[i], rho[i]) for i in range(len(masks))]))):
        saved = hpa.convert_targets_to_hybrid(model, targets, head_masks=masks, device="cpu",
                                              dtype=torch.float32, use_triton=True, **kw)
        with torch.inference_mode():
            out[f"hidden_{name}"] = model.model(input_ids=ids, use_cache=False).last_hidden_state.numpy()
        for l, blk in enumerate(model.model.layers):
            a = blk.self_attn
            out[f"{name}:frozen:{l}"] = a.frozen_mask_i32.numpy()
            out[f"{name}:hidx:{l}"] = a.hidx_i32.numpy()
            out[f"{name}:pidx:{l}"] = a.pidx_i32.numpy()
            out[f"{name}:kvidx:{l}"] = a.kvidx_i32.numpy()
            if name == "dense":
                out[f"dense:prior:{l}"] = a.prior_pattern.numpy()
            else:
                out[f"decomp:z:{l}"] = a.dec_z.numpy()
        hpa.restore_originals(saved)
    for l, m in enumerate(masks):
        out[f"mask:{l}"] = m.numpy()
    out["dense_in"] = dense.half().numpy()
    out["alpha"] = alpha.numpy()
    out["rho"] = rho.numpy()
    for k, v in model.state_dict().items():
        if k == "lm_head.weight":
            continue
        out["w:" + k] = v.half().numpy()
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
