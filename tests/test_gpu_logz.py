"""GPU parity of the decomposed-pattern row normalisers (saf_decomposed_logz,
kernel.decomposed_logz on device tensors) against the oracle's float64
restatement of the reference's decomposed_logz (kernel/fused_attn.py:101-116):
z[h, i] = logsumexp_{j<=i}(alpha[h, j] + rho[h, i - j]).

Tolerance: fp32 accumulation of up to S exp terms per row, |z - z64| <=
atol + 1e-6 |z64| with atol 3e-5 up to S = 4096 and 2e-4 at S = 16384.
Rows whose logits are all -inf must be exactly -inf."""
import math

import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc

pytestmark = pytest.mark.gpu


def _logz(alpha, rho):
    import kernel
    z = kernel.decomposed_logz(alpha.cuda(), rho.cuda())
    torch.cuda.synchronize()
    return z.cpu()


def _close(got, want, atol):
    got = got.double().numpy()
    inf = np.isneginf(want)
    assert np.array_equal(np.isneginf(got), inf), "-inf rows differ"
    err = np.abs(got[~inf] - want[~inf])
    bound = atol + 1e-6 * np.abs(want[~inf])
    assert (err <= bound).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("H,S", [(1, 1), (2, 37), (3, 64), (2, 1000), (4, 1024), (2, 1088), (2, 4096)])
def test_logz_matches_oracle(H, S):
    g = torch.Generator().manual_seed(H * 1000 + S)
    alpha = torch.randn(H, S, generator=g) * 2
    rho = torch.randn(H, S, generator=g) * 2
    want = orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())
    _close(_logz(alpha, rho), want, 3e-5)


def test_logz_closed_forms_and_inf():
    """alpha = rho = 0 gives log(i + 1); a window rho (-inf from distance w)
    gives log(min(i + 1, w)); -inf alpha on the first keys makes the first
    rows exactly -inf; large logits stay finite."""
    S = 3000
    i = np.arange(S, dtype=np.float64)
    zero = torch.zeros(2, S)
    got = _logz(zero, zero)
    np.testing.assert_allclose(got[0].double().numpy(), np.log(i + 1), atol=3e-5, rtol=1e-6)
    w = 37
    rho = torch.zeros(1, S)
    rho[0, w:] = float("-inf")
    got = _logz(torch.zeros(1, S), rho)
    np.testing.assert_allclose(got[0].double().numpy(), np.log(np.minimum(i + 1, w)), atol=3e-5, rtol=1e-6)
    g = torch.Generator().manual_seed(11)
    alpha = torch.randn(3, S, generator=g) * 40
    alpha[:, :5] = float("-inf")
    rho = torch.randn(3, S, generator=g) * 40
    rho[1, 100:] = float("-inf")
    want = orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())
    assert np.isneginf(want[:, :5]).all()
    _close(_logz(alpha, rho), want, 3e-5)


def test_logz_strided_rows_and_dtype():
    """Row-strided fp32 views run in place; bf16 alpha / rho are widened to
    fp32 and z comes back in alpha's dtype."""
    g = torch.Generator().manual_seed(5)
    big = torch.randn(4, 2 * 513, generator=g)
    alpha, rho = big[:, :513], big[:, 513:]
    want = orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())
    _close(_logz(alpha, rho), want, 3e-5)
    ab, rb = alpha.bfloat16(), rho.bfloat16()
    z = _logz(ab, rb)
    assert z.dtype == torch.bfloat16
    want = orc.decomposed_logz(ab.double().numpy(), rb.double().numpy())
    np.testing.assert_allclose(z.double().numpy(), want, atol=0.05, rtol=1e-2)


def test_logz_full_size_sampled_rows():
    """C2 buffer size (12 heads, S = 16384): sampled rows against float64
    sums over their own keys, and z rises with i for alpha >= 0 patterns."""
    H, S = 12, 16384
    g = torch.Generator().manual_seed(7)
    alpha = torch.randn(H, S, generator=g)
    rho = -torch.rand(H, S, generator=g) * 0.01 * torch.arange(S)
    got = _logz(alpha, rho).double().numpy()
    a64, r64 = alpha.double().numpy(), rho.double().numpy()
    for h in range(H):
        for i in [0, 1, 63, 64, 1023, 1024, 5000, S - 65, S - 1]:
            x = a64[h, :i + 1] + r64[h, i::-1]
            m = x.max()
            want = m + math.log(np.exp(x - m).sum())
            assert abs(got[h, i] - want) <= 2e-4 + 1e-6 * abs(want), (h, i, got[h, i], want)
    mono = _logz(torch.zeros(2, S), torch.zeros(2, S)).double().numpy()
    assert (np.diff(mono, axis=1) > 0).all()


def test_logz_rejects_bad_arguments():
    import kernel
    from kernel import _ext
    a = torch.zeros(2, 64, device="cuda")
    z = torch.empty(2, 32, device="cuda")
    L = _ext.lib()
    rc = L.saf_decomposed_logz(_ext.tensor_desc(a), _ext.tensor_desc(a), _ext.tensor_desc(z), None)
    assert rc == _ext.SAF_EINVAL
    zi = torch.empty(2, 64, device="cuda", dtype=torch.float16)
    rc = L.saf_decomposed_logz(_ext.tensor_desc(a), _ext.tensor_desc(a), _ext.tensor_desc(zi), None)
    assert rc == _ext.SAF_EUNSUPPORTED
    assert kernel.decomposed_logz(a[:, :0], a[:, :0]).shape == (2, 0)
