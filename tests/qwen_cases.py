"""Shared builders for the Qwen3 GQA caller tests (fixture model and oracle inputs)."""
import ast
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qwen_forward_small.npz")


def load_golden():
    return np.load(GOLDEN)


def golden_cfg(z):
    C = ast.literal_eval(str(z["cfg_json"]))
    ocfg = dict(n_layers=C["num_hidden_layers"], n_heads=C["num_attention_heads"],
                n_kv_heads=C["num_key_value_heads"], head_dim=C["head_dim"],
                eps=C["rms_norm_eps"], rope_theta=C["rope_theta"])
    return C, ocfg


def golden_state_dict(z):
    return {k[2:]: torch.from_numpy(z[k]).float() for k in z.files if k.startswith("w:")}


def golden_model(z, device="cpu", dtype=torch.float32):
    """transformers Qwen3ForCausalLM holding the fixture's weights."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    C, _ = golden_cfg(z)
    cfg = Qwen3Config(**C, attn_implementation="sdpa", use_cache=False)
    with torch.device("cpu"):
        m = Qwen3ForCausalLM(cfg)
    sd = golden_state_dict(z)
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and set(missing) <= {"lm_head.weight"}, (missing, unexpected)
    return m.to(device=device, dtype=dtype).eval()


def golden_freeze(z, repr):
    """Per-layer oracle freeze records and the adapter's conversion inputs."""
    n = sum(1 for k in z.files if k.startswith("mask:"))
    masks = [torch.from_numpy(z[f"mask:{l}"]) for l in range(n)]
    if repr == "dense":
        dense = z["dense_in"].astype(np.float32)
        fr = [dict(mask=z[f"mask:{l}"], dense=dense[l]) for l in range(n)]
        conv = dict(mean_attn=[torch.from_numpy(dense[l]) for l in range(n)], decomp=None)
    else:
        fr = [dict(mask=z[f"mask:{l}"], alpha=z["alpha"][l], rho=z["rho"][l]) for l in range(n)]
        conv = dict(mean_attn=None, decomp=[(torch.from_numpy(z["alpha"][l]), torch.from_numpy(z["rho"][l]))
                                            for l in range(n)])
    return masks, fr, conv


def convert_golden(model, z, repr, device, dtype):
    import qwen
    masks, fr, conv = golden_freeze(z, repr)
    mean_attn = conv["mean_attn"]
    if mean_attn is not None:
        mean_attn = [p.to(device) for p in mean_attn]
    decomp = conv["decomp"]
    if decomp is not None:
        decomp = [(a.to(device), r.to(device)) for a, r in decomp]
    targets = qwen.discover_softmax_attention(model)
    saved = qwen.convert_targets_to_hybrid(model, targets, mean_attn, masks, device, dtype,
                                           use_triton=True, decomp=decomp)
    return saved, fr
