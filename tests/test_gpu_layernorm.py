"""GPU parity of the fused residual add + LayerNorm (saf_add_layernorm)
against the oracle's restatement of the reference's LayerNorm and residual
update (nanogpt/model.py:45-54, :1214-1240): the updated residual is bit-exact
with torch's bf16/fp16 add, the normalised output within half-precision
rounding of the float64 result."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc

pytestmark = pytest.mark.gpu


def _round(dtype):
    return lambda a: torch.from_numpy(a).to(dtype).double().numpy()


@pytest.mark.parametrize("C", [64, 130, 256, 768, 896, 1152, 2048])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_delta,with_bias,wdtype",
                         [(True, False, "act"), (False, False, "act"), (True, True, "f32"), (True, True, "act")])
def test_add_layernorm_matches_oracle(C, dtype, with_delta, with_bias, wdtype):
    import kernel
    g = torch.Generator().manual_seed(C + (7 if with_delta else 0))
    rows = 37 if C > 1000 else 1000
    x = (torch.randn(rows, C, generator=g) * 2 + 0.5).to(dtype)
    d = torch.randn(rows, C, generator=g).to(dtype) if with_delta else None
    wt = torch.float32 if wdtype == "f32" else dtype
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(wt)
    b = (0.1 * torch.randn(C, generator=g)).to(wt) if with_bias else None
    xd = x.cuda()
    y = kernel.add_layernorm_(xd, None if d is None else d.cuda(), w.cuda(), None if b is None else b.cuda())
    torch.cuda.synchronize()
    ref_x = (x.cuda() + d.cuda()).cpu() if with_delta else x
    assert torch.equal(xd.cpu(), ref_x), "residual update must be bit-exact with torch's add"
    xn, yr = orc.add_layernorm(x.double().numpy(), None if d is None else d.double().numpy(), w.double().numpy(),
                               None if b is None else b.double().numpy(), round_fn=_round(dtype))
    err = np.abs(y.double().cpu().numpy() - yr).max()
    tol = 3e-2 if dtype == torch.bfloat16 else 4e-3   # one rounding of O(1) values
    assert err <= tol, f"C={C} {dtype}: max-abs {err:.3e} > {tol}"


def test_add_layernorm_3d_view_and_rejections():
    import kernel
    x = torch.randn(2, 50, 768, dtype=torch.bfloat16, device="cuda")
    d = torch.randn(2, 50, 768, dtype=torch.bfloat16, device="cuda")
    w = torch.ones(768, dtype=torch.bfloat16, device="cuda")
    ref = torch.nn.functional.layer_norm((x + d).float(), (768,), w.float(), None, 1e-5)
    y = kernel.add_layernorm_(x, d, w)
    assert y.shape == (2, 50, 768)
    assert (y.float() - ref).abs().max().item() < 3e-2
    with pytest.raises(NotImplementedError, match="not supported"):
        kernel.add_layernorm_(torch.zeros(4, 2050, dtype=torch.bfloat16, device="cuda"), None,
                              torch.ones(2050, device="cuda"))
    with pytest.raises(NotImplementedError, match="bf16 / fp16"):
        kernel.add_layernorm_(torch.zeros(4, 768, device="cuda"), None, torch.ones(768, device="cuda"))
    with pytest.raises(ValueError, match="weight and bias"):
        kernel.add_layernorm_(torch.zeros(4, 768, dtype=torch.bfloat16, device="cuda"), None,
                              torch.ones(767, device="cuda"))


@pytest.mark.parametrize("C,rows,offset", [(768, 1001, 0), (768, 999, 4), (2048, 7, 0), (256, 3, 4)])
def test_add_layernorm_alignment_paths(C, rows, offset):
    """Rows 16-byte aligned (half-wave rows, 16-byte pieces; odd row counts
    leave half a wave idle) and rows only 8-byte aligned (a view offset by
    four channels: the one-wave-per-row kernel) give the same results."""
    import kernel
    g = torch.Generator().manual_seed(C + rows + offset)
    base = (torch.randn(rows, C + offset, generator=g) * 2 + 0.5).bfloat16()
    dbase = torch.randn(rows, C + offset, generator=g).bfloat16()
    x, d = base[:, offset:], dbase[:, offset:]
    w = (1 + 0.1 * torch.randn(C, generator=g)).bfloat16()
    b = (0.1 * torch.randn(C, generator=g)).bfloat16()
    xb = base.cuda()
    y = kernel.add_layernorm_(xb[:, offset:], dbase.cuda()[:, offset:], w.cuda(), b.cuda())
    torch.cuda.synchronize()
    ref_x = (x.cuda() + d.cuda()).cpu()
    assert torch.equal(xb[:, offset:].cpu(), ref_x)
    if offset:
        assert torch.equal(xb[:, :offset].cpu(), base[:, :offset]), "channels outside the view changed"
    _, yr = orc.add_layernorm(x.double().numpy(), d.double().numpy(), w.double().numpy(), b.double().numpy(),
                              round_fn=_round(torch.bfloat16))
    err = np.abs(y.double().cpu().numpy() - yr).max()
    assert err <= 3e-2, f"C={C} rows={rows} offset={offset}: max-abs {err:.3e}"


@pytest.mark.parametrize("C", [64, 130, 768, 896, 1024, 2048])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("with_delta", [True, False])
def test_add_rmsnorm_matches_oracle(C, dtype, with_delta):
    """saf_add_rmsnorm against the oracle's restatement of transformers'
    Qwen3RMSNorm (with its intermediate rounding) and the residual update."""
    import kernel
    g = torch.Generator().manual_seed(C + (3 if with_delta else 0))
    rows = 37 if C > 1000 else 1000
    x = (torch.randn(rows, C, generator=g) * 2 + 0.5).to(dtype)
    d = torch.randn(rows, C, generator=g).to(dtype) if with_delta else None
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(dtype)
    xd = x.cuda()
    y = kernel.add_rmsnorm_(xd, None if d is None else d.cuda(), w.cuda(), 1e-6)
    torch.cuda.synchronize()
    ref_x = (x.cuda() + d.cuda()).cpu() if with_delta else x
    assert torch.equal(xd.cpu(), ref_x), "residual update must be bit-exact with torch's add"
    _, yr = orc.add_rmsnorm(x.double().numpy(), None if d is None else d.double().numpy(), w.double().numpy(), 1e-6,
                            round_fn=_round(dtype))
    err = np.abs(y.double().cpu().numpy() - yr).max()
    tol = 3e-2 if dtype == torch.bfloat16 else 4e-3   # the final rounding (and a flip of the intermediate one)
    assert err <= tol, f"C={C} {dtype}: max-abs {err:.3e} > {tol}"


def test_add_rmsnorm_is_transformers_qwen3_rmsnorm_on_device():
    """Against transformers' Qwen3RMSNorm module run by torch on the GPU in
    bf16 (the C4 model's norms: C = 896)."""
    import kernel
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    norm = Qwen3RMSNorm(896, eps=1e-6).cuda().to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(1 + 0.2 * torch.randn(896, device="cuda"))
        x = torch.randn(4, 4096, 896, device="cuda").to(torch.bfloat16)
        ref = norm(x)
    y = kernel.add_rmsnorm_(x.clone(), None, norm.weight, 1e-6)
    diff = (y.float() - ref.float()).abs()
    assert diff.max().item() <= 2 * 2.0 ** -8 * ref.float().abs().max().item()
    assert (diff == 0).float().mean().item() > 0.99, "nearly every output equals torch's to the bit"
