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


def qwen35_layer(hd=64, H=8, HKV=2, hidden=256, seed=0, impl="sdpa"):
    """A random-init transformers Qwen3_5Attention (fp32, CPU) with non-trivial
    norm weights, its text rotary embedding (partial rotation, factor 0.25)
    and the layer's state dict (keys relative to the module)."""
    from transformers.models.qwen3_5 import modeling_qwen3_5 as m
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(hidden_size=hidden, num_attention_heads=H, num_key_value_heads=HKV, head_dim=hd,
                            num_hidden_layers=1, layer_types=["full_attention"], intermediate_size=2 * hidden,
                            vocab_size=128, rope_parameters={"rope_type": "default", "rope_theta": 10000.0,
                                                             "partial_rotary_factor": 0.25})
    cfg._attn_implementation = impl
    torch.manual_seed(seed)
    attn = m.Qwen3_5Attention(cfg, layer_idx=0).eval()
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in attn.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(0.3 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(torch.randn(p.shape, generator=g) * (p.shape[-1] ** -0.5))
    rot = m.Qwen3_5TextRotaryEmbedding(cfg)
    return attn, rot, cfg


def qwen35_position_embeddings(rot, T, device="cpu", dtype=torch.float32, B=1):
    x = torch.zeros(1, device=device, dtype=dtype)
    pos = torch.arange(T, device=device)[None].expand(B, T)
    return rot.to(device)(x, pos)
