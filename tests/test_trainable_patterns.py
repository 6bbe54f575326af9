"""Host-side checks of the trainable-pattern supplement (the reference's
supplement/trainable_patterns.py): enable() semantics, the optimizer group,
the dispatch wrapper, fp32 parameters across dtype casts, and the host
path of decomp_log_normalizers against the oracle's gradients (which
tests/test_oracle.py pins by torch float64 autograd and finite
differences)."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc


def _model(T=64, layers=2, decomposed=True):
    from nanogpt.model import GPT, GPTConfig
    torch.manual_seed(0)
    cfg = GPTConfig(block_size=T, vocab_size=256, n_layer=layers, n_head=4, n_embd=128, bias=False,
                    rand_attn_prior_repr="decomposed")
    m = GPT(cfg)
    if decomposed:
        g = torch.Generator().manual_seed(1)
        m.transformer.h[0].attn.freeze_heads_decomposed([1, 2], torch.randn(2, T, generator=g),
                                                        torch.randn(2, T, generator=g))
    return m


@pytest.fixture
def restore_dispatch():
    from nanogpt import model as module
    yield
    fn = module.fused_mixed_attn
    if getattr(fn, "_trainable_patterns", False):
        module.fused_mixed_attn = fn._original


def test_enable_turns_fitted_buffers_into_parameters(restore_dispatch):
    import supplement
    from nanogpt import model as module
    m = _model()
    opt = torch.optim.AdamW(m.parameters(), lr=1e-3, weight_decay=0.1)
    params = supplement.enable(m, opt)
    a0 = m.transformer.h[0].attn
    assert len(params) == 2 and params[0] is a0.dyn_alpha and params[1] is a0.dyn_rho
    assert all(isinstance(p, torch.nn.Parameter) and p.dtype == torch.float32 for p in params)
    # layer 1 has nothing decomposed: its buffers stay buffers
    assert "dyn_alpha" in dict(m.transformer.h[1].attn.named_buffers())
    assert opt.param_groups[-1]["weight_decay"] == 0.0 and len(opt.param_groups[-1]["params"]) == 2
    assert getattr(module.fused_mixed_attn, "_trainable_patterns", False)
    assert a0._patterns is m._saf_patterns and m.transformer.h[1].attn._patterns is None
    with pytest.raises(RuntimeError, match="already enabled"):
        supplement.enable(m)
    # patching twice keeps one wrapper
    fn = module.fused_mixed_attn
    supplement.patch_fused_dispatch()
    assert module.fused_mixed_attn is fn


def test_enable_without_fitted_patterns_raises(restore_dispatch):
    import supplement
    with pytest.raises(RuntimeError, match="No fitted patterns"):
        supplement.enable(_model(decomposed=False))


def test_state_dict_exports_current_normalisers_and_bf16_cast_keeps_fp32(restore_dispatch):
    import supplement
    m = _model()
    supplement.enable(m)
    a0 = m.transformer.h[0].attn
    with torch.no_grad():
        a0.dyn_alpha[1, :10] += 0.5
    sd = m.state_dict()
    want = orc.decomposed_logz(a0.dyn_alpha.detach().double().numpy(), a0.dyn_rho.detach().double().numpy())
    np.testing.assert_allclose(sd["transformer.h.0.attn.dyn_z"].numpy(), want, rtol=1e-5, atol=1e-5)
    alpha32 = a0.dyn_alpha.detach().clone()
    m.to(torch.bfloat16)
    assert isinstance(a0.dyn_alpha, torch.nn.Parameter)
    assert a0.dyn_alpha.dtype == torch.float32 and torch.equal(a0.dyn_alpha.detach(), alpha32)


def test_dense_reference_matches_oracle_output():
    import supplement
    g = torch.Generator().manual_seed(3)
    H, T, S, hd = 3, 19, 24, 4
    v = torch.randn(2, H, T, hd, generator=g, dtype=torch.float64)
    a = torch.randn(H, S, generator=g, dtype=torch.float64)
    r = torch.randn(H, S, generator=g, dtype=torch.float64)
    want = orc.eager_mixed_attention(None, None, v.numpy(), np.full(H, 2), alpha=a.numpy(), rho=r.numpy(),
                                     z=orc.decomposed_logz(a.numpy(), r.numpy()))
    np.testing.assert_allclose(supplement.dense_reference(v, a, r).numpy(), want, atol=1e-12)


def test_host_normalisers_gradient_matches_oracle():
    import kernel
    g = torch.Generator().manual_seed(4)
    a = (torch.randn(3, 40, generator=g, dtype=torch.float64)).requires_grad_(True)
    r = (torch.randn(3, 40, generator=g, dtype=torch.float64)).requires_grad_(True)
    gz = torch.randn(3, 40, generator=g, dtype=torch.float64)
    z = kernel.decomp_log_normalizers(a, r)
    np.testing.assert_allclose(z.detach().numpy(), orc.decomposed_logz(a.detach().numpy(), r.detach().numpy()),
                               atol=1e-12)
    (z * gz).sum().backward()
    da, dr = orc.logz_grads(a.detach().numpy(), r.detach().numpy(), gz.numpy())
    np.testing.assert_allclose(a.grad.numpy(), da, atol=1e-10)
    np.testing.assert_allclose(r.grad.numpy(), dr, atol=1e-10)
    assert kernel.decomp_log_normalizers_fft is kernel.decomp_log_normalizers


def test_normaliser_cache_follows_parameters_and_optimizer_steps(restore_dispatch, monkeypatch):
    """z is computed once per (layer, length) while the parameters stay put;
    an in-place edit (version counter), another length, the optimizer's step
    (generation) or clear_pattern_cache recompute it.  The HIP normalisers are
    replaced by a counting host stand-in (the cache logic is host code)."""
    import supplement
    import supplement.trainable_patterns as tp
    from kernel.fused_attn import decomposed_logz
    from nanogpt import model as module
    calls = []

    def fake(alpha, rho, length):
        calls.append(int(length))
        z = torch.zeros(alpha.shape)
        z[:, :length] = decomposed_logz(alpha[:, :length].detach().float(), rho[:, :length].detach().float())
        return z
    monkeypatch.setattr(tp, "normalisers", fake)
    m = _model()
    opt = torch.optim.SGD(m.parameters(), lr=0.0)
    supplement.enable(m, opt)
    pats, a0 = m._saf_patterns, m.transformer.h[0].attn
    z1 = pats.z_for(a0, 48)
    assert pats.z_for(a0, 48) is z1 and calls == [48]
    np.testing.assert_allclose(z1[:, :48].numpy(), orc.decomposed_logz(
        a0.dyn_alpha.detach()[:, :48].double().numpy(), a0.dyn_rho.detach()[:, :48].double().numpy()),
        rtol=1e-5, atol=1e-5)
    pats.z_for(a0, 64)
    assert calls == [48, 64]
    with torch.no_grad():
        a0.dyn_rho[0, 3] += 1.0
    pats.z_for(a0, 64)
    assert calls == [48, 64, 64]
    pats.z_for(a0, 64)
    opt.step()
    pats.z_for(a0, 64)
    assert calls == [48, 64, 64, 64]
    module.fused_mixed_attn.clear_pattern_cache()
    pats.z_for(a0, 64)
    assert calls == [48, 64, 64, 64, 64]
    kw = pats.kernel_inputs(a0, 64)
    assert kw["closed_form"] is None and not kw["alpha"].requires_grad and kw["z"] is pats.z_for(a0, 64)
