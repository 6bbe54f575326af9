"""Parity of the indexed projections (kernel/indexed_linear.py) against a
float64 restatement of the reference's definitions
(/root/reference/kernel/indexed_linear.py:125-141):

    linear_rows(x, W, b, rows)          = x W[rows]^T + b[rows]
    linear_rows2(x, W1, W2, b1, b2, r)  = [x W1[r]^T + b1[r], x W2[r]^T + b2[r]]
    linear_permuted_cols(y, W, b, cols) = y W[:, cols]^T + b

Forward values and every gradient (input, weights, biases) are compared with
autograd through plain indexing of the same definition in float64; weight and
bias rows outside ``rows`` must get exactly zero gradient.  CPU tests run the
op on host tensors (it is a torch op: gathers plus library GEMMs); the GPU
test runs it in bf16 on the device.
"""
import pytest
import torch
import torch.nn.functional as F

import kernel


def _leaf(t):
    return t.clone().requires_grad_(True)


def _rand(*shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def _check_grads(got_leaves, ref_leaves, atol=1e-10):
    for g, r in zip(got_leaves, ref_leaves):
        if r is None:
            continue
        assert g.grad is not None
        torch.testing.assert_close(g.grad, r.grad, atol=atol, rtol=0)


@pytest.mark.parametrize("bias", [True, False])
def test_linear_rows_matches_definition(bias):
    x, W = _rand(3, 5, 16, seed=1), _rand(24, 16, seed=2)
    b = _rand(24, seed=3) if bias else None
    rows = torch.tensor([20, 3, 7, 8, 9, 0])
    xs, Ws = _leaf(x), _leaf(W)
    bs = _leaf(b) if bias else None
    y = kernel.linear_rows(xs, Ws, bs, rows)
    xr, Wr = _leaf(x), _leaf(W)
    br = _leaf(b) if bias else None
    yr = F.linear(xr, Wr[rows], None if br is None else br[rows])
    torch.testing.assert_close(y, yr, atol=1e-12, rtol=0)
    gy = _rand(*y.shape, seed=4)
    (y * gy).sum().backward()
    (yr * gy).sum().backward()
    _check_grads([xs, Ws, bs], [xr, Wr, br])
    unsel = torch.ones(24, dtype=torch.bool)
    unsel[rows] = False
    assert (Ws.grad[unsel] == 0).all()
    if bias:
        assert (bs.grad[unsel] == 0).all()


@pytest.mark.parametrize("bias", [True, False])
def test_linear_rows2_matches_definition(bias):
    x = _rand(2, 7, 12, seed=5)
    W1, W2 = _rand(12, 12, seed=6), _rand(12, 12, seed=7)
    b1, b2 = (_rand(12, seed=8), _rand(12, seed=9)) if bias else (None, None)
    rows = torch.tensor([4, 5, 6, 7, 0, 1])
    L = [_leaf(t) if t is not None else None for t in (x, W1, W2, b1, b2)]
    R = [_leaf(t) if t is not None else None for t in (x, W1, W2, b1, b2)]
    y = kernel.linear_rows2(*L, rows)
    yr = torch.cat([F.linear(R[0], R[1][rows], None if R[3] is None else R[3][rows]),
                    F.linear(R[0], R[2][rows], None if R[4] is None else R[4][rows])], dim=-1)
    assert y.shape == (2, 7, 12)
    torch.testing.assert_close(y, yr, atol=1e-12, rtol=0)
    gy = _rand(*y.shape, seed=10)
    (y * gy).sum().backward()
    (yr * gy).sum().backward()
    _check_grads(L, R)
    for w in (L[1], L[2]):
        assert (w.grad[[2, 3, 8, 9, 10, 11]] == 0).all()


@pytest.mark.parametrize("bias", [True, False])
def test_linear_permuted_cols_matches_definition(bias):
    y0, W = _rand(4, 3, 20, seed=11), _rand(9, 20, seed=12)
    b = _rand(9, seed=13) if bias else None
    cols = torch.randperm(20, generator=torch.Generator().manual_seed(14))
    ys, Ws = _leaf(y0), _leaf(W)
    bs = _leaf(b) if bias else None
    out = kernel.linear_permuted_cols(ys, Ws, bs, cols)
    yr, Wr = _leaf(y0), _leaf(W)
    br = _leaf(b) if bias else None
    ref = F.linear(yr, Wr[:, cols], br)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=0)
    g = _rand(*out.shape, seed=15)
    (out * g).sum().backward()
    (ref * g).sum().backward()
    _check_grads([ys, Ws, bs], [yr, Wr, br])


def test_head_order_fixup_round_trip():
    """The caller's use (nanogpt/model.py:1025, :1061): V projected in
    [live..., frozen...] head order by linear_rows and c_proj applied to the
    same column permutation equals the unpermuted projection pair."""
    C, hd = 12, 3
    x = _rand(2, 5, C, seed=16)
    Wv, Wc = _rand(C, C, seed=17), _rand(C, C, seed=18)
    frozen = torch.tensor([False, True, False, True])
    uf, fz = (~frozen).nonzero().flatten(), frozen.nonzero().flatten()
    cperm = torch.cat([(uf[:, None] * hd + torch.arange(hd)).flatten(),
                       (fz[:, None] * hd + torch.arange(hd)).flatten()])
    y = kernel.linear_permuted_cols(kernel.linear_rows(x, Wv, None, cperm), Wc, None, cperm)
    torch.testing.assert_close(y, F.linear(F.linear(x, Wv), Wc), atol=1e-12, rtol=0)


def test_planted_wrong_rows_are_detected():
    """The definition check is sensitive to the index: the same op with the
    rows reversed does not match."""
    x, W = _rand(2, 8, seed=19), _rand(6, 8, seed=20)
    rows = torch.tensor([1, 4, 5])
    y = kernel.linear_rows(x, W, None, rows.flip(0))
    assert (y - F.linear(x, W[rows])).abs().max() > 1e-3


def test_autocast_computes_in_autocast_dtype():
    x, W = torch.randn(4, 32), torch.randn(16, 32)
    rows = torch.tensor([0, 3, 9])
    with torch.autocast("cpu", dtype=torch.bfloat16):
        y = kernel.linear_rows(x, W, None, rows)
    assert y.dtype == torch.bfloat16
    ref = F.linear(x.bfloat16(), W.bfloat16()[rows]).float()
    torch.testing.assert_close(y.float(), ref, atol=1e-2, rtol=1e-2)


@pytest.mark.gpu
def test_gpu_bf16_rows2_and_cols():
    dev = "cuda"
    g = torch.Generator().manual_seed(21)
    x = torch.randn(2, 64, 256, generator=g)
    W1, W2, Wc = (torch.randn(256, 256, generator=g) * 0.05 for _ in range(3))
    rows = torch.arange(64, 192)
    cols = torch.randperm(256, generator=g)
    L = [t.to(dev, torch.bfloat16).requires_grad_(True) for t in (x, W1, W2, Wc)]
    y = kernel.linear_rows2(L[0], L[1], L[2], None, None, rows.to(dev))
    out = kernel.linear_permuted_cols(y.view(2, 64, 256), L[3], None, cols.to(dev))
    gy = torch.randn(out.shape, generator=g)
    (out.float() * gy.to(dev)).sum().backward()
    R = [t.double().requires_grad_(True) for t in (x, W1, W2, Wc)]
    yr = torch.cat([F.linear(R[0], R[1][rows]), F.linear(R[0], R[2][rows])], -1)
    outr = F.linear(yr, R[3][:, cols])
    (outr * gy.double()).sum().backward()
    cos = lambda a, b: F.cosine_similarity(a.double().flatten().cpu(), b.double().flatten().cpu(), dim=0)
    assert cos(out, outr) >= 0.9999
    for a, b in zip(L, R):
        assert cos(a.grad, b.grad) >= 0.999
    assert (L[1].grad[:64] == 0).all() and (L[1].grad[192:] == 0).all()
