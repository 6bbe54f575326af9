"""GPU parity of the fused MLP up-projection + GELU (saf_linear_gelu) against
the oracle's restatement of the reference's MLP front half
(nanogpt/model.py:1193-1207: bias-free c_fc, then nn.GELU()), and at the
full prefill shapes against the same product and GELU computed by torch in
fp32.  The kernel rounds once, so each output is within half an ulp of the
output dtype (plus the fp32 accumulation-order error) of the exact value."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc

pytestmark = pytest.mark.gpu

# one rounding of the output: half an ulp is 2^-8 (bf16) / 2^-11 (fp16) of
# the value; the small absolute term covers the fp32 accumulation order
_RTOL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
_ATOL = 2e-5


def _inputs(M, N, K, dtype, seed, wscale=0.05):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (wscale * torch.randn(N, K, generator=g)).to(dtype)
    return x, w


def _check(y, ref, dtype, what):
    y = y.double().cpu().numpy()
    err = np.abs(y - ref)
    bound = _RTOL[dtype] * np.abs(ref) + _ATOL
    worst = int(np.argmax(err - bound))
    assert (err <= bound).all(), (f"{what}: {int((err > bound).sum())} outputs off; worst at "
                                  f"{np.unravel_index(worst, err.shape)} got {y.flat[worst]:.6e} "
                                  f"want {ref.flat[worst]:.6e}")


@pytest.mark.parametrize("M,N,K", [(1, 256, 128), (255, 256, 256), (257, 512, 128), (1000, 768, 384),
                                   (512, 3072, 768), (300, 256, 2048)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_gelu_matches_oracle(M, N, K, dtype):
    import kernel
    x, w = _inputs(M, N, K, dtype, seed=M * 7 + N + K)
    y = kernel.linear_gelu(x.cuda(), w.cuda())
    torch.cuda.synchronize()
    assert y.shape == (M, N) and y.dtype == dtype
    _check(y, orc.linear_gelu(x.double().numpy(), w.double().numpy()), dtype, f"M={M} N={N} K={K} {dtype}")


def test_linear_gelu_wide_range_and_strided_rows():
    """Products beyond +-20 (the GELU's tails: -0 and the identity) and
    x rows that are a column slice of a wider tensor (row stride > K)."""
    import kernel
    dtype = torch.bfloat16
    M, N, K = 384, 512, 256
    g = torch.Generator().manual_seed(5)
    big = torch.randn(M, K + 128, generator=g).to(dtype)
    x = big[:, 64:64 + K]
    w = (torch.randn(N, K, generator=g) * torch.linspace(0.01, 8.0, N)[:, None] / 16).to(dtype)
    xd = big.cuda()[:, 64:64 + K]
    assert xd.stride(0) == K + 128
    y = kernel.linear_gelu(xd, w.cuda())
    ref = orc.linear_gelu(x.double().numpy(), w.double().numpy())
    assert np.abs(x.double().numpy() @ w.double().numpy().T).max() > 20
    assert torch.isfinite(y).all()
    _check(y, ref, dtype, "wide range")


@pytest.mark.parametrize("M,N,K", [(16384, 3072, 768), (16384, 8192, 2048)])
def test_linear_gelu_full_shapes_against_torch_fp32(M, N, K):
    """The 124M model's MLP at T = 16384 and the 1B-class model's at B = 2,
    T = 8192, against torch's fp32 product and exact GELU on the GPU."""
    import kernel
    dtype = torch.bfloat16
    g = torch.Generator(device="cuda").manual_seed(M + N)
    x = torch.randn(M, K, device="cuda", generator=g).to(dtype)
    w = (0.02 * torch.randn(N, K, device="cuda", generator=g)).to(dtype)
    y = kernel.linear_gelu(x, w)
    ref = torch.nn.functional.gelu(x.float() @ w.float().t(), approximate="none")
    err = (y.float() - ref).abs()
    bound = _RTOL[dtype] * ref.abs() + 1e-4
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item():.3e}"
    # against torch's own bf16 path (product rounded, then GELU rounded):
    # at most two roundings apart
    y2 = torch.nn.functional.gelu(torch.nn.functional.linear(x, w))
    assert bool(((y.float() - y2.float()).abs() <= 2 * _RTOL[dtype] * ref.abs() + 2e-3 * ref.abs().max()).all())


def test_linear_gelu_repeated_calls_and_views():
    """Two calls in a row (the second smaller), a 3-D activation view."""
    import kernel
    x, w = _inputs(2 * 300, 768, 256, torch.bfloat16, seed=3)
    xd, wd = x.cuda(), w.cuda()
    y1 = kernel.linear_gelu(xd.view(2, 300, 256), wd)
    assert y1.shape == (2, 300, 768)
    y2 = kernel.linear_gelu(xd[:17], wd)
    torch.cuda.synchronize()
    ref = orc.linear_gelu(x.double().numpy(), w.double().numpy())
    _check(y1.view(600, 768), ref, torch.bfloat16, "first call")
    _check(y2, ref[:17], torch.bfloat16, "second call")


def test_linear_gelu_rejections():
    import kernel
    bf = dict(dtype=torch.bfloat16, device="cuda")
    with pytest.raises(NotImplementedError, match="multiple of 256"):
        kernel.linear_gelu(torch.zeros(4, 128, **bf), torch.zeros(200, 128, **bf))
    with pytest.raises(NotImplementedError, match="multiple of 256"):
        kernel.linear_gelu(torch.zeros(4, 96, **bf), torch.zeros(256, 96, **bf))
    with pytest.raises(ValueError, match="one dtype"):
        kernel.linear_gelu(torch.zeros(4, 128, **bf), torch.zeros(256, 128, dtype=torch.float16, device="cuda"))
    with pytest.raises(NotImplementedError, match="bf16 / fp16"):
        kernel.linear_gelu(torch.zeros(4, 128, device="cuda"), torch.zeros(256, 128, device="cuda"))
    with pytest.raises(ValueError, match="do not chain"):
        kernel.linear_gelu(torch.zeros(4, 128, **bf), torch.zeros(256, 256, **bf))
    # rows of 8-byte pitch are not 16-byte aligned
    odd = torch.zeros(4, 132, **bf)[:, :128]
    with pytest.raises(ValueError, match="16-byte aligned"):
        kernel.linear_gelu(odd, torch.zeros(256, 128, **bf))
    assert kernel.linear_gelu(torch.zeros(0, 128, **bf), torch.zeros(256, 128, **bf)).shape == (0, 256)
    assert not kernel.linear_gelu_usable(torch.zeros(4, 128, **bf), torch.zeros(200, 128, **bf))
    assert kernel.linear_gelu_usable(torch.zeros(4, 768, **bf), torch.zeros(3072, 768, **bf))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gelu_inplace_matches_oracle(dtype):
    """saf_gelu_inplace against the oracle's exact GELU (the linear_gelu
    restatement with an identity weight), over values that take both the
    polynomial and the tail formula, and torch's own bf16 / fp16 GELU."""
    import kernel
    g = torch.Generator().manual_seed(21)
    u = (torch.randn(3, 1000, 64, generator=g) * torch.logspace(-3, 1.5, 64)).to(dtype)
    y = kernel.gelu_(u.cuda().clone())
    ref = orc.linear_gelu(u.reshape(-1, 1).double().numpy(), np.eye(1)).reshape(u.shape)
    _check(y.reshape(-1, 64), ref.reshape(-1, 64), dtype, f"gelu_ {dtype}")
    # torch's own GELU rounds the same exact function once: the two agree to
    # two roundings plus the evaluations' absolute errors (the kernel's 5.3e-6,
    # fp32 erf's cancellation in the negative tail)
    y2 = torch.nn.functional.gelu(u.cuda())
    assert bool(((y.float() - y2.float()).abs() <= 2 * _RTOL[dtype] * y2.float().abs() + _ATOL).all())
    assert kernel.gelu_(torch.zeros(0, device="cuda", dtype=dtype)).numel() == 0
    with pytest.raises(ValueError, match="multiple of 8"):
        kernel.gelu_(torch.zeros(12, device="cuda", dtype=dtype))
