"""GPU parity of the Qwen3 GQA caller and its HIP prologue kernel.

* saf_qk_rmsnorm_rope_inplace vs fp32 arithmetic of Qwen3RMSNorm (with its two
  roundings) + the half rotation, on strided views of one projection output;
  max-abs <= 2e-2, relative L2 <= 4e-3, bytes outside q/k untouched; and vs
  transformers' own bf16 modules (max-abs <= 2^-6 of the largest value,
  relative L2 <= 4e-3).
* The reference-pinned fixture model (tests/golden/qwen_forward_small.npz) in
  bf16 through the fused HIP path (dense and decomposed priors): last hidden
  state vs the reference's fp32 values, cosine >= 0.9999, relative L2 <= 1e-2.
* C4-shaped heads (14 query / 2 KV heads, head_dim 64) with causal-mean
  frozen sets at each rate of the sweep (closed-form scan, and dense priors
  at 50%), ragged T: hidden state vs the fp32 oracle, same bar; every layer
  takes the fused path.
"""
import numpy as np
import pytest
import torch

import qwen_cases as qc
from oracle import qwen_oracle as qo

DEV = "cuda"
pytestmark = pytest.mark.gpu


def _cos(a, b):
    a = a.double().flatten()
    b = b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()))


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm())


def _prologue_ref(x, w, eps, cos, sin):
    """fp32 arithmetic of the kernel's contract on (B, U, T, hd) bf16 x."""
    xf = x.float()
    r = torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    n = (w.float() * (xf * r).to(torch.bfloat16).float()).to(torch.bfloat16).float()
    x1, x2 = n.chunk(2, dim=-1)
    rot = torch.cat((-x2, x1), dim=-1)
    return n * cos.float() + rot * sin.float()


@pytest.mark.parametrize("hd", [32, 64, 96, 128])
@pytest.mark.parametrize("cs_dtype", [torch.bfloat16, torch.float32])
def test_qk_rmsnorm_rope_matches_fp32(hd, cs_dtype):
    import kernel
    g = torch.Generator().manual_seed(hd)
    B, T, Uq, HKV = 2, 77, 5, 2
    proj = (torch.randn(B, T, Uq + 2 * HKV, hd, generator=g) * 2).to(torch.bfloat16).to(DEV)
    before = proj.clone()
    q = proj[:, :, :Uq].transpose(1, 2)
    k = proj[:, :, Uq:Uq + HKV].transpose(1, 2)
    qw = (1 + 0.3 * torch.randn(hd, generator=g)).to(torch.bfloat16).to(DEV)
    kw = (1 + 0.3 * torch.randn(hd, generator=g)).to(torch.bfloat16).to(DEV)
    cos_f, sin_f = qo.rope_cache(hd, T + 5, 1e6)
    cos, sin = cos_f.to(cs_dtype).to(DEV), sin_f.to(cs_dtype).to(DEV)
    ref_q = _prologue_ref(q, qw, 1e-6, cos[:T], sin[:T])
    ref_k = _prologue_ref(k, kw, 1e-6, cos[:T], sin[:T])
    kernel.qk_rmsnorm_rope_(q, k, qw, kw, 1e-6, cos.unsqueeze(0), sin.unsqueeze(0))
    torch.cuda.synchronize()
    for got, ref in ((q, ref_q), (k, ref_k)):
        assert (got.float() - ref).abs().max().item() <= 2e-2
        assert _rel(got.float(), ref) <= 4e-3
    assert torch.equal(proj[:, :, Uq + HKV:], before[:, :, Uq + HKV:])


def test_qk_rmsnorm_rope_matches_transformers_modules():
    import kernel
    from transformers.models.qwen3 import modeling_qwen3 as m
    g = torch.Generator().manual_seed(5)
    B, T, Uq, HKV, hd = 2, 130, 3, 2, 64
    proj = torch.randn(B, T, Uq + HKV, hd, generator=g).to(torch.bfloat16).to(DEV)
    qn, kn = m.Qwen3RMSNorm(hd, eps=1e-6).to(DEV, torch.bfloat16), m.Qwen3RMSNorm(hd, eps=1e-6).to(DEV, torch.bfloat16)
    with torch.no_grad():
        qn.weight.copy_(1 + 0.3 * torch.randn(hd, generator=g))
        kn.weight.copy_(1 + 0.3 * torch.randn(hd, generator=g))
    cos_f, sin_f = qo.rope_cache(hd, T, 1e6)
    cos, sin = cos_f.to(torch.bfloat16).to(DEV)[None], sin_f.to(torch.bfloat16).to(DEV)[None]
    with torch.no_grad():
        rq, rk = m.apply_rotary_pos_emb(qn(proj[:, :, :Uq]).transpose(1, 2),
                                        kn(proj[:, :, Uq:]).transpose(1, 2), cos, sin)
    q = proj[:, :, :Uq].transpose(1, 2)
    k = proj[:, :, Uq:].transpose(1, 2)
    kernel.qk_rmsnorm_rope_(q, k, qn.weight, kn.weight, 1e-6, cos, sin)
    torch.cuda.synchronize()
    # transformers rounds both rotation products to bf16 before their sum, the
    # kernel rounds once: the gap scales with the products (up to the tensor's
    # largest magnitude), not with a small cancelled result
    for got, ref in ((q, rq), (k, rk)):
        ref = ref.float()
        assert (got.float() - ref).abs().max().item() <= 2 ** -6 * ref.abs().max().item()
        assert _rel(got.float(), ref) <= 4e-3


@pytest.mark.parametrize("repr", ["dense", "decomp"])
def test_golden_model_fused_path(repr):
    import qwen
    z = qc.load_golden()
    m = qc.golden_model(z, device=DEV, dtype=torch.bfloat16)
    qc.convert_golden(m, z, repr, DEV, torch.bfloat16)
    n0 = qwen.fused_dispatch_count()
    with torch.inference_mode():
        y = qwen.backbone_forward(m.model, torch.from_numpy(z["tokens"]).to(DEV))
    torch.cuda.synchronize()
    assert qwen.fused_dispatch_count() - n0 == len(m.model.layers)
    ref = torch.from_numpy(z[f"hidden_{repr}"])
    y = y.float().cpu()
    assert _cos(y, ref) >= 0.9999
    assert _rel(y, ref) <= 1e-2


@pytest.mark.parametrize("rate,repr", [(0.0, "decomposed"), (0.25, "decomposed"), (0.5, "decomposed"),
                                       (0.75, "decomposed"), (0.5, "dense")])
def test_c4_heads_model_vs_oracle(rate, repr):
    import qwen
    T = 333
    cfg = qwen.qwen_config(n_layers=3, hidden=256, n_heads=14, n_kv_heads=2, head_dim=64,
                           intermediate=512, vocab=1024)
    m = qwen.build_model(cfg, device=DEV, dtype=torch.bfloat16, seed=7)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n.endswith("norm.weight"):
                p.copy_(1 + 0.2 * torch.randn_like(p))
    sd = {k: v.detach().float().cpu() for k, v in m.state_dict().items()}
    saved, masks = qwen.convert_with_rate(m, rate, T, repr=repr, fuse_live_only=rate == 0.0)
    # one attention entry per layer, plus each block's fused gated MLP, two
    # RMSNorms and its own forward (the post-attention residual add in the
    # norm's kernel), and the final norm
    assert sum(1 for e in saved if e[1] != "forward") == cfg.num_hidden_layers
    assert sum(1 for e in saved if e[1] == "forward") == 4 * cfg.num_hidden_layers + 1
    g = torch.Generator().manual_seed(9)
    ids = torch.randint(0, 1024, (2, T), generator=g)
    n0 = qwen.fused_dispatch_count()
    with torch.inference_mode():
        y = qwen.backbone_forward(m.model, ids.to(DEV))
    torch.cuda.synchronize()
    assert qwen.fused_dispatch_count() - n0 == cfg.num_hidden_layers
    if repr == "decomposed" and rate > 0:
        assert all((blk.self_attn.routing.closed[0][mk.numpy()] == 1).all() for blk, mk in zip(m.model.layers, masks))
    mean = np.tril(np.ones((T, T), dtype=np.float32))
    fr = [dict(mask=mk.numpy(), dense=np.broadcast_to(mean, (14, T, T))) for mk in masks]
    ocfg = dict(n_layers=cfg.num_hidden_layers, n_heads=14, n_kv_heads=2, head_dim=64,
                eps=cfg.rms_norm_eps, rope_theta=1e6)
    ref = qo.qwen_forward(sd, ocfg, fr, ids)
    y = y.float().cpu()
    assert _cos(y, ref) >= 0.9999
    assert _rel(y, ref) <= 1e-2


@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("prior", ["dense", "decomp"])
def test_qwen35_gated_fused_path_vs_oracle(hd, prior):
    """The Qwen3.5 gated-attention hybrid (qwen/nanogpt/hybrid_prior_attention.py:205-470)
    on its fused path: one gathered projection [q(live); k; v; gate(all)],
    the module's own (1 + w) q/k norms and partial RoPE, the HIP operator with
    the GQA map, sigmoid gate, o_proj; against the fp32 oracle with the
    module's bf16-rounded weights (cosine >= 0.9999, relative L2 <= 1e-2)."""
    import qwen
    attn, rot, cfg = qc.qwen35_layer(hd=hd, H=8, HKV=2, hidden=512, seed=hd)
    attn = attn.to(DEV, torch.bfloat16)
    T, H = 300, 8
    sd = {k: v.detach().float().cpu() for k, v in attn.state_dict().items()}
    mask = torch.zeros(H, dtype=torch.bool)
    mask[[1, 2, 6]] = True
    g = torch.Generator().manual_seed(hd + 1)
    cls = qwen.make_qwen35_hybrid_class()
    if prior == "dense":
        dense = torch.rand(H, T, T, generator=g)
        hyb = cls(attn, dense.to(DEV), mask, DEV, torch.bfloat16)
        fr = {"mask": mask.numpy(), "dense": hyb.routing.patterns.float().cpu().numpy()}
        full = np.zeros((H, T, T), dtype=np.float32)
        full[[1, 2, 6]] = fr["dense"]
        fr["dense"] = full
    else:
        a, r = torch.randn(H, 320, generator=g) * 0.5, torch.randn(H, 320, generator=g) * 0.5
        a[2], r[2] = 0.0, -0.05 * torch.arange(320.0)   # a closed-form decay head
        hyb = cls(attn, None, mask, DEV, torch.bfloat16, decomp=(a.to(DEV), r.to(DEV)))
        assert int(hyb.routing.closed[0][2]) == 2
        fr = {"mask": mask.numpy(), "alpha": a.numpy(), "rho": r.numpy()}
    x = torch.randn(2, T, cfg.hidden_size, generator=torch.Generator().manual_seed(3))
    cos, sin = qc.qwen35_position_embeddings(rot, T, device=DEV, dtype=torch.bfloat16, B=2)
    n0 = qwen.fused_dispatch_count()
    with torch.inference_mode():
        y, _ = hyb(x.to(DEV, torch.bfloat16), (cos, sin))
    torch.cuda.synchronize()
    assert qwen.fused_dispatch_count() - n0 == 1 and hyb.triton_calls == 1
    xr = x.to(torch.bfloat16).float()
    ref = qo.qwen35_attention(xr, sd, "", dict(n_heads=H, n_kv_heads=2, head_dim=hd, eps=cfg.rms_norm_eps),
                              fr, cos[0].float().cpu(), sin[0].float().cpu())
    y = y.float().cpu()
    assert _cos(y, ref) >= 0.9999
    assert _rel(y, ref) <= 1e-2
