"""GPU parity of the trainable-pattern gradients against the float64 oracle.

  * decomp_log_normalizers backward (saf_decomposed_logz_bwd) vs
    oracle.saf_oracle.logz_grads; fp32 sums of up to S terms in [0, |gz|]:
    |err| <= 1e-4 (1 + |ref|).
  * dalpha / drho of decomposed heads (saf_decomp_param_bwd through
    supplement.PatternGradient after fused_mixed_attn) vs
    oracle.saf_oracle.pattern_grads (both pinned in tests/test_oracle.py by
    torch float64 autograd of the reference's dense definition,
    supplement/trainable_patterns.py:7-13, and finite differences); the
    oracle sees the same bf16/fp16-rounded V and upstream gradient, and
    takes delta from the kernel's rounded forward output, as the reference's
    kernel does (supplement/trainable_pattern_kernels.py:44; with sharp
    logits dP - delta nearly cancels, so the forward's own rounding, checked
    by the forward tests, would otherwise dominate): relative L2 <= 1e-2 and
    max-abs <= 2e-2 max(1, max|ref|).
  * one training step of the bf16 nanoGPT caller with enable(): the
    pattern-parameter gradients against the fp32 CPU model oracle's autograd
    (z as a differentiable logsumexp), cosine >= 0.999 per layer; after an
    optimizer step the exported dyn_z and the inference logits follow the
    updated parameters."""
import numpy as np
import pytest
import torch

from oracle import model_oracle, saf_oracle as orc
from saf_cases import f64, make_decomp, make_pattern, qkv, routing

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel_ok(got, ref, what, rel_tol=1e-2, abs_frac=2e-2):
    got = got.detach().double().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite gradient"
    err = np.abs(got - ref)
    rel = float(np.linalg.norm(got - ref)) / (float(np.linalg.norm(ref)) or 1.0)
    bound = abs_frac * max(1.0, float(np.abs(ref).max()))
    print(f"{what}: max_abs={err.max():.3e} rel_l2={rel:.3e}", flush=True)
    assert rel <= rel_tol and err.max() <= bound, f"{what}: max_abs={err.max():.3e} rel_l2={rel:.3e}"


@pytest.mark.parametrize("H,S,scale,window", [(1, 1, 1.0, 0), (3, 37, 1.0, 0), (4, 700, 1.5, 0),
                                              (2, 1024, 0.5, 100), (2, 4096, 1.0, 0)])
def test_normaliser_backward_matches_oracle(H, S, scale, window):
    import kernel
    g = torch.Generator().manual_seed(H * 97 + S)
    alpha = torch.randn(H, S, generator=g) * scale
    rho = torch.randn(H, S, generator=g) * scale
    if window:
        rho[0, window:] = float("-inf")
    gz = torch.randn(H, S, generator=g)
    a = alpha.to(DEV).requires_grad_(True)
    r = rho.to(DEV).requires_grad_(True)
    z = kernel.decomp_log_normalizers(a, r)
    (z * gz.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    da, dr = orc.logz_grads(alpha.double().numpy(), rho.double().numpy(), gz.double().numpy())
    for got, ref, name in ((a.grad, da, "dalpha"), (r.grad, dr, "drho")):
        got = got.double().cpu().numpy()
        assert np.isfinite(got).all(), name
        err = np.abs(got - ref)
        assert (err <= 1e-4 * (1 + np.abs(ref))).all(), f"{name} H{H} S{S}: max err {err.max():.3e}"


def _pattern_case(B, H, T, hd, S, dec, dense=(), dtype=torch.bfloat16, scale=0.8):
    import kernel
    import supplement
    states = {h: 2 for h in dec}
    states.update({h: 1 for h in dense})
    frozen, hidx, live = routing(H, states)
    alpha, rho, _ = make_decomp(H, S, seed=7 * H + T + hd, scale=scale)
    patt = make_pattern(H, S, seed=H + S + T)
    q, k, v = qkv(B, H, T, hd, seed=T + 3 * hd + B, dtype=dtype)
    a_p = alpha.to(DEV).requires_grad_(True)
    r_p = rho.to(DEV).requires_grad_(True)
    z = supplement.normalisers(a_p, r_p, T)
    tv = v.to(DEV).requires_grad_(True)
    tq = q[:, live].contiguous().to(DEV).requires_grad_(True)
    tk = k[:, live].contiguous().to(DEV).requires_grad_(True)
    fr = frozen.to(DEV)
    y = kernel.fused_mixed_attn(tq, tk, tv, patt.to(DEV), fr, hidx.to(DEV), alpha=a_p.detach(),
                                rho=r_p.detach(), z=z)
    y_fwd = f64(y)
    y = supplement.PatternGradient.apply(y, tv, a_p, r_p, z, fr)
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(T + hd)).to(DEV)
    (y.float() * w).sum().backward()
    torch.cuda.synchronize()
    dout = f64(w.to(dtype))
    da, dr = orc.pattern_grads(f64(v), dout, frozen.numpy(), alpha.double().numpy(), rho.double().numpy(),
                               out=y_fwd)
    what = f"B{B} H{H} T{T} hd{hd} dec={list(dec)} dense={list(dense)} {dtype}"
    _rel_ok(a_p.grad, da, "dalpha " + what)
    _rel_ok(r_p.grad, dr, "drho " + what)
    nd = [h for h in range(H) if h not in dec]
    assert (a_p.grad[nd] == 0).all() and (r_p.grad[nd] == 0).all(), "gradient on a non-decomposed head"
    assert (a_p.grad[:, T:] == 0).all() and (r_p.grad[:, T:] == 0).all(), "gradient beyond T"
    return tv.grad


@pytest.mark.parametrize("case", [
    (2, 8, 700, 64, 1024, [0, 3, 5], [1]),
    (2, 12, 1024, 64, 1024, list(range(12)), []),
    (1, 4, 1, 64, 64, [1, 2], []),
    (2, 4, 37, 64, 64, [0], [3]),
    (1, 16, 1000, 96, 1024, [0, 15], [7]),
    (1, 6, 333, 128, 512, [0, 2], []),
    (2, 4, 517, 32, 1024, [1, 3], [0]),
], ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}d{c[3]}")
def test_pattern_gradients_match_oracle(case):
    B, H, T, hd, S, dec, dense = case
    _pattern_case(B, H, T, hd, S, dec, dense)


def test_pattern_gradients_fp16_and_sharp_logits():
    _pattern_case(2, 4, 300, 64, 512, [0, 2], dtype=torch.float16)
    _pattern_case(1, 4, 640, 64, 1024, [1, 3], scale=6.0)


def test_pattern_gradients_need_decomposed_heads_only():
    """No decomposed head: zero gradients, no launch failure."""
    import supplement
    v = torch.randn(1, 2, 64, 64, device=DEV, dtype=torch.bfloat16)
    a = torch.zeros(2, 64, device=DEV)
    da, dr = supplement.pattern_gradients(v, v, a, a, a, torch.tensor([0, 1]), v)
    assert (da == 0).all() and (dr == 0).all()


# ---------------------------------------------------------------------------
# nanoGPT caller
# ---------------------------------------------------------------------------

@pytest.fixture
def restore_dispatch():
    from nanogpt import model as module
    yield
    fn = module.fused_mixed_attn
    if getattr(fn, "_trainable_patterns", False):
        module.fused_mixed_attn = fn._original


def test_patched_dispatch_adds_pattern_gradients(restore_dispatch):
    """A direct caller handing trainable alpha / rho to the patched
    nanogpt.model.fused_mixed_attn gets z derived and the pattern gradients
    added: the same dalpha / drho as the explicit PatternGradient route."""
    import supplement
    from nanogpt import model as module
    supplement.patch_fused_dispatch()
    B, H, T, hd, S, dec = 2, 6, 300, 64, 512, [1, 4]
    frozen, hidx, live = routing(H, {h: 2 for h in dec})
    alpha, rho, _ = make_decomp(H, S, seed=5, scale=0.8)
    q, k, v = qkv(B, H, T, hd, seed=17, dtype=torch.bfloat16)
    a_p = alpha.to(DEV).requires_grad_(True)
    r_p = rho.to(DEV).requires_grad_(True)
    y = module.fused_mixed_attn(q[:, live].contiguous().to(DEV), k[:, live].contiguous().to(DEV), v.to(DEV),
                                None, frozen.to(DEV), hidx.to(DEV), alpha=a_p, rho=r_p)
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(23)).to(DEV)
    (y.float() * w).sum().backward()
    torch.cuda.synchronize()
    da, dr = orc.pattern_grads(f64(v), f64(w.bfloat16()), frozen.numpy(), alpha.double().numpy(),
                               rho.double().numpy(), out=f64(y))
    _rel_ok(a_p.grad, da, "dalpha via dispatch")
    _rel_ok(r_p.grad, dr, "drho via dispatch")


def _freeze_records(m, req):
    """Model-oracle freeze records whose decomposed rows are the trainable
    (alpha, rho) of `req` and z their differentiable logsumexp."""
    recs = []
    T = m.config.block_size
    ar = torch.arange(T)
    dist = ar[:, None] - ar[None, :]
    for l, blk in enumerate(m.transformer.h):
        a = blk.attn
        rec = {"frozen": a.dyn_frozen.cpu().tolist(), "patterns": {}, "decomp": {}}
        al, rh = req.get(l, (None, None))
        for h in range(m.config.n_head):
            if not rec["frozen"][h]:
                continue
            if bool(a.dyn_decomp[h]):
                lg = (al[h][None, :] + rh[h][dist.clamp(min=0)]).masked_fill(dist < 0, float("-inf"))
                rec["decomp"][h] = (al[h], rh[h], lg.logsumexp(-1))
            else:
                rec["patterns"][h] = a.dyn_pattern[int(a.dyn_pattern_slot[h])].float().cpu()
        recs.append(rec)
    return recs


def _cos(a, b):
    a, b = a.double().flatten(), b.double().flatten()
    return float((a @ b) / (a.norm() * b.norm()).clamp_min(1e-30))


def test_model_trainable_patterns_match_oracle(restore_dispatch):
    import supplement
    from test_model import _oracle_inputs, _small_model
    T = 128
    m, x = _small_model(T=T, layers=2, device=DEV, dtype=torch.bfloat16)
    m.train()
    opt = torch.optim.SGD([p for p in m.parameters() if p.requires_grad], lr=0.0)
    params = supplement.enable(m, opt)
    assert len(params) == 4
    sd, ocfg, _ = _oracle_inputs(m)
    w = torch.randn(1, T, m.config.vocab_size, generator=torch.Generator().manual_seed(9))
    m.zero_grad(set_to_none=True)
    (m.forward_all_positions(x).float() * w.to(DEV)).sum().backward()
    torch.cuda.synchronize()

    ref_sd = {k: v.clone().requires_grad_(True) for k, v in sd.items()}
    req = {}
    for l in range(2):
        req[l] = (ref_sd[f"transformer.h.{l}.attn.dyn_alpha"], ref_sd[f"transformer.h.{l}.attn.dyn_rho"])
    forward = getattr(model_oracle.gpt_forward, "__wrapped__", model_oracle.gpt_forward)
    ref = forward(ref_sd, ocfg, _freeze_records(m, req), x.cpu(), path="split", all_positions=True)
    (ref * w).sum().backward()
    for l, blk in enumerate(m.transformer.h):
        a = blk.attn
        for name in ("dyn_alpha", "dyn_rho"):
            got = getattr(a, name).grad
            want = ref_sd[f"transformer.h.{l}.attn.{name}"].grad
            assert got is not None and torch.isfinite(got).all(), f"layer {l} {name}"
            dec = a.dyn_decomp.cpu()
            c = _cos(got[dec].cpu(), want[dec])
            print(f"layer {l} {name}: cosine {c:.6f}", flush=True)
            assert c >= 0.999, f"layer {l} {name}: gradient cosine {c:.6f}"
            assert (got[~dec.to(DEV)] == 0).all()

    # a step that moves the patterns: exported z and inference logits follow
    with torch.no_grad():
        for p in params:
            p.add_(0.05 * torch.randn(p.shape, generator=torch.Generator().manual_seed(11)).to(DEV))
    opt.step()   # clears the dispatch's z cache
    a0 = m.transformer.h[0].attn
    z_new = m.state_dict()["transformer.h.0.attn.dyn_z"]
    want_z = orc.decomposed_logz(a0.dyn_alpha.detach().double().cpu().numpy(),
                                 a0.dyn_rho.detach().double().cpu().numpy())
    fin = np.isfinite(want_z)
    np.testing.assert_allclose(z_new.cpu().numpy()[fin], want_z[fin], rtol=1e-5, atol=1e-4)
    m.eval()
    with torch.no_grad():
        got = m(x).float().cpu()
    sd2, _, fr2 = _oracle_inputs(m)
    want = model_oracle.gpt_forward(sd2, ocfg, fr2, x.cpu())
    c = _cos(got, want)
    assert c >= 0.999, f"logits after the update: cosine {c:.6f}"
