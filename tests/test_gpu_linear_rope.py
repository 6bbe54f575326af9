"""GPU parity of the fused QKV projection + rotary embedding (saf_linear_rope)
against the oracle's restatement of the reference's gathered projection and
rotation (nanogpt/model.py:920-944, :57-99), and at the full prefill shape
against the same product and rotation computed by torch in fp32.  The
kernel rotates the fp32 accumulator and rounds once, so each output is within
half an ulp of the output dtype (plus the fp32 accumulation-order error) of
the exact value for the given (16-bit) cos / sin."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc

pytestmark = pytest.mark.gpu

_RTOL = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}
_ATOL = 2e-5


def _cache(hd, T, dtype, extra=0):
    """The model's rotary cache (fp32 angles, then the activation dtype), with
    `extra` rows beyond T."""
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))
    emb = torch.outer(torch.arange(T + extra, dtype=torch.float32), inv)
    emb = torch.cat([emb, emb], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def _check(y, ref, dtype, what):
    y = y.double().cpu().numpy()
    err = np.abs(y - ref)
    bound = _RTOL[dtype] * np.abs(ref) + _ATOL
    worst = int(np.argmax(err - bound))
    assert (err <= bound).all(), (f"{what}: {int((err > bound).sum())} outputs off; worst at "
                                  f"{np.unravel_index(worst, err.shape)} got {y.flat[worst]:.6e} "
                                  f"want {ref.flat[worst]:.6e}")


@pytest.mark.parametrize("B,T,K,hd,n_live,n_v", [(1, 300, 256, 64, 3, 4), (2, 257, 128, 64, 9, 12),
                                                 (1, 64, 768, 64, 12, 12), (2, 100, 384, 128, 2, 4),
                                                 (1, 513, 256, 128, 3, 1)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_linear_rope_matches_oracle(B, T, K, hd, n_live, n_v, dtype):
    import kernel
    g = torch.Generator().manual_seed(B * 1000 + T + K + hd)
    n_rope = 2 * n_live * hd
    N = n_rope + n_v * hd
    N += -N % 256  # zero rows pad N to a multiple of 256, as the model's gathered weight
    x = torch.randn(B, T, K, generator=g).to(dtype)
    w = (0.05 * torch.randn(N, K, generator=g)).to(dtype)
    w[n_rope + n_v * hd:] = 0
    cos, sin = _cache(hd, T, dtype, extra=7)
    y = kernel.linear_rope(x.cuda(), w.cuda(), n_rope, hd, cos.cuda(), sin.cuda())
    torch.cuda.synchronize()
    assert y.shape == (B, T, N) and y.dtype == dtype
    ref = orc.linear_rope(x.reshape(B * T, K).double().numpy(), w.double().numpy(), n_rope, hd,
                          cos.double().numpy(), sin.double().numpy(), T)
    _check(y.reshape(B * T, N), ref, dtype, f"B={B} T={T} K={K} hd={hd} n_rope={n_rope} {dtype}")
    assert not y[..., n_rope + n_v * hd:].any(), "zero weight rows give zero columns"


def test_linear_rope_full_shape_against_torch_fp32():
    """The 124M model's QKV projection at T = 16384 (9 live heads, 12 V heads,
    2048 columns with the padding) against torch's fp32 product and rotation."""
    import kernel
    dtype = torch.bfloat16
    B, T, K, hd, n_live = 1, 16384, 768, 64, 9
    n_rope = 2 * n_live * hd
    N = 2048
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randn(B, T, K, device="cuda", generator=g).to(dtype)
    w = (0.02 * torch.randn(N, K, device="cuda", generator=g)).to(dtype)
    cos, sin = (c.cuda() for c in _cache(hd, T, dtype))
    y = kernel.linear_rope(x, w, n_rope, hd, cos, sin)
    u = (x.float().reshape(T, K) @ w.float().t())
    ref = u.clone()
    c, s = cos.float(), sin.float()
    for h0 in range(0, n_rope, hd):
        a, b = u[:, h0:h0 + hd // 2], u[:, h0 + hd // 2:h0 + hd]
        ref[:, h0:h0 + hd // 2] = a * c[:, :hd // 2] - b * s[:, :hd // 2]
        ref[:, h0 + hd // 2:h0 + hd] = b * c[:, hd // 2:] + a * s[:, hd // 2:]
    err = (y.reshape(T, N).float() - ref).abs()
    bound = _RTOL[dtype] * ref.abs() + 1e-4
    assert bool((err <= bound).all()), f"max excess {(err - bound).max().item():.3e}"


def test_linear_rope_no_rotation_is_the_plain_product():
    import kernel
    x = torch.randn(2, 128, 256, device="cuda").to(torch.bfloat16)
    w = (0.05 * torch.randn(512, 256, device="cuda")).to(torch.bfloat16)
    cos, sin = (c.cuda() for c in _cache(64, 128, torch.bfloat16))
    y = kernel.linear_rope(x, w, 0, 64, cos, sin)
    ref = orc.linear_rope(x.reshape(256, 256).double().cpu().numpy(), w.double().cpu().numpy(), 0, 64,
                          cos.double().cpu().numpy(), sin.double().cpu().numpy(), 128)
    _check(y.reshape(256, 512), ref, torch.bfloat16, "n_rope = 0")


def test_linear_rope_rejections():
    import kernel
    bf = dict(dtype=torch.bfloat16, device="cuda")
    x, w = torch.zeros(1, 64, 128, **bf), torch.zeros(256, 128, **bf)
    cos, sin = (c.cuda() for c in _cache(64, 64, torch.bfloat16))
    with pytest.raises(ValueError, match="multiple of 128"):
        kernel.linear_rope(x, w, 64, 64, cos, sin)
    with pytest.raises(NotImplementedError, match="head_dim 96"):
        kernel.linear_rope(x, w, 128, 96, cos, sin)
    with pytest.raises(ValueError, match="cos / sin must be"):
        kernel.linear_rope(x, w, 128, 64, cos[:32], sin[:32])
    with pytest.raises(ValueError, match="cos / sin must be"):
        kernel.linear_rope(x, w, 128, 64, cos.float(), sin.float())
    with pytest.raises(NotImplementedError, match="multiple of 256"):
        kernel.linear_rope(x, torch.zeros(200, 128, **bf), 128, 64, cos, sin)
    assert kernel.linear_rope_usable(x, w, 128, 64, cos)
    assert not kernel.linear_rope_usable(x, w, 128, 64, cos.float())
    assert not kernel.linear_rope_usable(x, w, 64, 64, cos)
