"""GPU parity of the fused SwiGLU projection (saf_linear_swiglu) against the
oracle's restatement of transformers' Qwen3MLP front half (the Qwen caller's
act_fn(gate_proj(x)) * up_proj(x), SiLU), and at the C4 shape against the
same products and activation computed by torch in fp32.  The kernel keeps
both products and the activation in fp32 and rounds once, so each output is
within half an ulp of the output dtype (plus the fp32 accumulation-order
error) of the exact value."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc

pytestmark = pytest.mark.gpu

_RTOL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
_ATOL = 2e-5


def _check(y, ref, dtype, what):
    y = y.double().cpu().numpy()
    err = np.abs(y - ref)
    bound = _RTOL[dtype] * np.abs(ref) + _ATOL
    worst = int(np.argmax(err - bound))
    assert (err <= bound).all(), (f"{what}: {int((err > bound).sum())} outputs off; worst at "
                                  f"{np.unravel_index(worst, err.shape)} got {y.flat[worst]:.6e} "
                                  f"want {ref.flat[worst]:.6e}")


@pytest.mark.parametrize("M,I,K", [(1, 128, 128), (255, 128, 256), (300, 384, 896), (1000, 256, 128),
                                   (513, 640, 384)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_swiglu_matches_oracle(M, I, K, dtype):
    import kernel
    g = torch.Generator().manual_seed(M + 3 * I + K)
    x = torch.randn(M, K, generator=g).to(dtype)
    wg = (0.08 * torch.randn(I, K, generator=g)).to(dtype)
    wu = (0.08 * torch.randn(I, K, generator=g)).to(dtype)
    w = kernel.swiglu_weight(wg, wu)
    y = kernel.linear_swiglu(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    assert y.shape == (M, I) and y.dtype == dtype
    ref = orc.linear_swiglu(x.double().numpy(), wg.double().numpy(), wu.double().numpy())
    _check(y, ref, dtype, f"M={M} I={I} K={K} {dtype}")


def test_linear_swiglu_wide_range_and_views():
    """Gate products beyond +-30 (silu's tails: -0 and the identity) and a
    3-D activation view."""
    import kernel
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(9)
    x = torch.randn(3, 100, 256, generator=g).to(dtype)
    wg = (torch.randn(256, 256, generator=g) * torch.linspace(0.01, 8.0, 256)[:, None] / 16).to(dtype)
    wu = (0.1 * torch.randn(256, 256, generator=g)).to(dtype)
    y = kernel.linear_swiglu(x.cuda(), kernel.swiglu_weight(wg, wu).cuda())
    assert y.shape == (3, 100, 256)
    gate = x.reshape(300, 256).double().numpy() @ wg.double().numpy().T
    assert np.abs(gate).max() > 30
    ref = orc.linear_swiglu(x.reshape(300, 256).double().numpy(), wg.double().numpy(), wu.double().numpy())
    assert torch.isfinite(y).all()
    _check(y.reshape(300, 256), ref, dtype, "wide range")


def test_linear_swiglu_c4_shape_against_torch_fp32():
    """The C4 model's MLP (hidden 896, intermediate 4864, B = 4, T = 4096)
    against torch's fp32 products and SiLU, and torch's own bf16 path."""
    import kernel
    dtype = torch.bfloat16
    M, K, I = 16384, 896, 4864
    g = torch.Generator(device="cuda").manual_seed(4)
    x = torch.randn(M, K, device="cuda", generator=g).to(dtype)
    wg = (0.02 * torch.randn(I, K, device="cuda", generator=g)).to(dtype)
    wu = (0.02 * torch.randn(I, K, device="cuda", generator=g)).to(dtype)
    y = kernel.linear_swiglu(x, kernel.swiglu_weight(wg, wu))
    xf = x.float()
    ref = torch.nn.functional.silu(xf @ wg.float().t()) * (xf @ wu.float().t())
    err = (y.float() - ref).abs()
    bound = _RTOL[dtype] * ref.abs() + 1e-4
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item():.3e}"
    F = torch.nn.functional
    y2 = F.silu(F.linear(x, wg)) * F.linear(x, wu)
    assert bool(((y.float() - y2.float()).abs() <= 4 * _RTOL[dtype] * ref.abs() + 1e-3 * ref.abs().max()).all())


def test_linear_swiglu_rejections():
    import kernel
    bf = dict(dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="do not chain"):
        kernel._ext.check(kernel._ext.lib().saf_linear_swiglu(
            kernel._ext.tensor_desc(torch.zeros(4, 128, **bf)), kernel._ext.tensor_desc(torch.zeros(256, 128, **bf)),
            kernel._ext.tensor_desc(torch.zeros(4, 256, **bf)), None))
    with pytest.raises(NotImplementedError, match="multiple of 256"):
        kernel.linear_swiglu(torch.zeros(4, 128, **bf), torch.zeros(192, 128, **bf))
    with pytest.raises(ValueError, match="multiple of 64"):
        kernel.swiglu_weight(torch.zeros(100, 8), torch.zeros(100, 8))
    assert kernel.linear_swiglu(torch.zeros(0, 128, **bf), torch.zeros(256, 128, **bf)).shape == (0, 128)
    assert kernel.linear_swiglu_usable(torch.zeros(4, 896, **bf), torch.zeros(9728, 896, **bf))
