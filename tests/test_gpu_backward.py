"""GPU parity of the fused_mixed_attn backward (saf_mixed_attn_bwd) against
the float64 oracle gradients (oracle.saf_oracle.eager_mixed_attention_grads,
itself pinned by finite differences in tests/test_oracle.py).

Mirrors the reference's backward checks (kernel/test_fused_attn.py:134-158,
:162-230): live / dense / decomposed mixes, nothing or everything frozen,
unaligned T with S > T, tiny T, hd 64 / 96 / 128 / 32, strided q/k views of
one projection (their gradients come back contiguous), bf16 decomposed
buffers, closed-form heads (run through their decomposed buffers); alpha and
rho receive no gradient.  Bound: the reference's bf16 tolerance on every
gradient, max-abs <= 2e-1 (kernel/test_fused_attn.py:191), and relative-L2
<= 2e-2 against the oracle from the same rounded inputs and upstream
gradient."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import closed_params, f64, make_decomp, make_pattern, qkv, routing, scale_of

pytestmark = pytest.mark.gpu
DEV = "cuda"
ATOL_B, RTOL_B = 2e-1, 2e-2


def _kernel():
    import kernel
    return kernel


def _cmp(got, ref, what):
    got = got.detach().float().cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all(), f"{what}: non-finite gradient"
    err = np.abs(got - ref)
    rel = float(np.linalg.norm(got - ref)) / (float(np.linalg.norm(ref)) or 1.0)
    assert err.max() <= ATOL_B and rel <= RTOL_B, f"{what}: max_abs={err.max():.3e} rel_l2={rel:.3e}"


def run_bwd(B, H, T, hd, S, dense, dec=(), closed=None, dtype=torch.bfloat16, strided=False,
            buf_dtype=torch.float32, dec_scale=0.8):
    K = _kernel()
    closed = closed or {}
    states = {h: 1 for h in dense}
    states.update({h: 2 for h in dec})
    states.update({h: 2 for h in closed})
    frozen, hidx, live = routing(H, states)
    patt = make_pattern(H, S, seed=H * S + T + 7)
    alpha, rho, z = make_decomp(H, S, seed=H + S + T + 7, scale=dec_scale)
    cf = None
    if closed:
        ca, cr, cz = closed_params(H, S, closed)
        for h in closed:
            alpha[h], rho[h], z[h] = ca[h], cr[h], cz[h]
        cf = K.classify_closed_form(alpha, rho, z)
    alpha, rho, z = (t.to(buf_dtype) for t in (alpha, rho, z))
    q, k, v = qkv(B, H, T, hd, seed=T * hd + B + 3, dtype=dtype)
    has_dec = bool(dec) or bool(closed)

    if strided:
        qk = torch.stack([q[:, live], k[:, live]], dim=2).transpose(1, 2).contiguous().transpose(1, 2)
        qk = qk.to(DEV).detach().requires_grad_(True)  # (B, U, 2, T, hd) non-dense views
        tq, tk = qk[:, :, 0], qk[:, :, 1]
    else:
        tq = q[:, live].contiguous().to(DEV).requires_grad_(True)
        tk = k[:, live].contiguous().to(DEV).requires_grad_(True)
    tv = v.to(DEV).requires_grad_(True)
    a_d = alpha.to(DEV).requires_grad_(True) if has_dec else None
    r_d = rho.to(DEV).requires_grad_(True) if has_dec else None
    z_d = z.to(DEV) if has_dec else None
    y = K.fused_mixed_attn(tq, tk, tv, patt.to(DEV), frozen.to(DEV), hidx.to(DEV), alpha=a_d, rho=r_d, z=z_d,
                           closed_form=cf)
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(T + hd)).to(DEV)
    (y.float() * w).sum().backward()
    torch.cuda.synchronize()
    dout = w.to(dtype)  # the gradient that reaches y (cast back to y's dtype)

    dq, dk, dv = orc.eager_mixed_attention_grads(
        f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), f64(dout), hidx.numpy(),
        patt=patt.numpy(), alpha=f64(alpha), rho=f64(rho), z=f64(z), sm_scale=scale_of(hd))
    what = f"B{B} H{H} T{T} hd{hd} dense={list(dense)} dec={list(dec)} closed={closed} {dtype}"
    _cmp(tv.grad, dv, "dv " + what)
    if live:
        gq = qk.grad[:, :, 0] if strided else tq.grad
        gk = qk.grad[:, :, 1] if strided else tk.grad
        _cmp(gq, dq, "dq " + what)
        _cmp(gk, dk, "dk " + what)
    if has_dec:
        assert a_d.grad is None and r_d.grad is None, "alpha/rho must receive no gradient"


CASES = [
    (2, 12, 1024, 64, 1024, [0, 1, 2]),
    (2, 12, 1024, 64, 1024, []),
    (2, 12, 1024, 64, 1024, list(range(12))),
    (2, 12, 700, 64, 1024, [0, 5, 11]),
    (2, 12, 37, 64, 1024, [0, 5]),
    (1, 16, 1000, 96, 1024, [0, 7, 8, 15]),
    (1, 8, 777, 128, 1024, [1, 6]),
    (2, 4, 333, 32, 512, [2]),
    (1, 4, 1, 64, 64, [1]),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}d{c[3]}nf{len(c[5])}")
def test_backward_dense_and_live(case):
    run_bwd(*case)


@pytest.mark.parametrize("case", CASES[:4], ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}d{c[3]}nf{len(c[5])}")
def test_backward_strided_qk(case):
    run_bwd(*case, strided=True)


def test_backward_fp16():
    run_bwd(2, 6, 513, 64, 640, [1, 4], dtype=torch.float16)


@pytest.mark.parametrize("case", [
    (2, 12, 1024, 64, 1024, [0, 1], [2, 3]),
    (2, 12, 700, 64, 1024, [3], [0, 7]),
    (2, 12, 37, 64, 1024, [5], [0, 2]),
    (1, 16, 1000, 96, 1024, [0, 8], [7, 15]),
], ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}d{c[3]}")
def test_backward_decomposed(case):
    B, H, T, hd, S, fz, dec = case
    run_bwd(B, H, T, hd, S, fz, dec)


def test_backward_decomposed_bf16_buffers_and_sharp_logits():
    run_bwd(2, 8, 700, 64, 1024, [3], [0, 7], buf_dtype=torch.bfloat16)
    run_bwd(2, 8, 700, 64, 1024, [3], [0, 7], dec_scale=40.0)


def test_backward_closed_forms():
    """Closed-form heads (scan in the forward) backpropagate through their
    decomposed buffers."""
    run_bwd(2, 8, 900, 64, 1024, [2], [], closed={0: ("mean", 0), 3: ("decay", 0.05), 6: ("window", 100)})


def test_backward_gqa_raises():
    K = _kernel()
    B, H, HKV, T, hd = 1, 4, 2, 64, 64
    frozen = torch.tensor([0, 1, 0, 0], dtype=torch.int32)
    hidx = torch.tensor([0, 0, 1, 2], dtype=torch.int32)
    kvidx = torch.tensor([0, 0, 1, 1], dtype=torch.int32)
    q = torch.randn(B, 3, T, hd, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    k = torch.randn(B, HKV, T, hd, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    v = torch.randn(B, HKV, T, hd, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    patt = make_pattern(1, T, seed=1).to(DEV)
    pidx = torch.zeros(H, dtype=torch.int32)
    y = K.fused_mixed_attn(q, k, v, patt, frozen.to(DEV), hidx.to(DEV), pidx.to(DEV), kvidx=kvidx.to(DEV))
    with pytest.raises(NotImplementedError):
        y.float().sum().backward()


@pytest.mark.parametrize("T,Tv,S,hd,nf", [(1, 1, 64, 64, 2), (37, 40, 64, 64, 3), (700, 700, 1024, 64, 3),
                                          (513, 600, 576, 128, 2), (1024, 1024, 1024, 96, 3)])
def test_frozen_pv_backward(T, Tv, S, hd, nf):
    """frozen_pv's backward dV = P^T dY (kernel/frozen_attn.py:91-128,
    kernel/test_frozen_attn.py:57-87) with compact frozen values, a
    non-identity fz_idx, S > T and V longer than T (rows at or past T get
    zero gradient) against the oracle's P^T dY in float64."""
    K = _kernel()
    B, Hp = 2, 6
    patt = make_pattern(Hp, S, seed=T + S + 1)
    fz = torch.tensor([5, 0, 3][:nf], dtype=torch.int32)
    g = torch.Generator().manual_seed(T * hd + 7)
    v = torch.randn(B, nf, Tv, hd, generator=g).bfloat16()
    dy = torch.randn(B, nf, T, hd, generator=g).bfloat16()
    vd = v.to(DEV).requires_grad_(True)
    y = K.frozen_pv(patt.to(DEV), vd, fz.to(DEV), T)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    ref = np.zeros((B, nf, Tv, hd))
    for f in range(nf):
        P = patt[int(fz[f]), :T, :T].double().numpy()
        for b in range(B):
            ref[b, f, :T] = P.T @ f64(dy[b, f])
    _cmp(vd.grad, ref, f"frozen_pv dV T={T} Tv={Tv} hd={hd}")
    assert (vd.grad[:, :, T:] == 0).all()
    # the forward of the same call is unchanged by the autograd wrapping
    y0 = K.frozen_pv(patt.to(DEV), v.to(DEV), fz.to(DEV), T)
    assert torch.equal(y.detach(), y0)
