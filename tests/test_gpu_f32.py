"""GPU parity of the float32 path (attn_f32.hip) against the float64 oracle,
at the reference's own fp32 contract (IEEE dots; kernel/test_fused_attn.py:
188-190): forward max-abs <= 2e-5, gradients max-abs <= 2e-4.

Mirrors the reference's fp32 grid (kernel/test_fused_attn.py:162-230): live /
dense / decomposed mixes, nothing or everything frozen, non-contiguous freeze
sets, unaligned T with S > T, tiny T, hd 96, strided q/k views of one fused
projection, compact pidx, bf16 decomposed buffers, extreme logits (scale 40);
plus hd 32 / 256, closed-form heads (run through their decomposed buffers),
the GQA map, the LSE, and frozen_pv forward / backward; alpha and rho receive
no gradient."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import closed_params, f64, make_decomp, make_pattern, routing, scale_of

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL_F, TOL_B = 2e-5, 2e-4


def _maxabs(got, ref, tol, what):
    got = got.detach().double().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite"
    err = float(np.abs(got - ref).max()) if got.size else 0.0
    assert err <= tol, f"{what}: max_abs={err:.3e} > {tol}"
    return err


def run_f32(B, H, T, hd, S, dense, dec=(), closed=None, strided=False, compact=False, buf_dtype=torch.float32,
            dec_scale=0.8, backward=True, check_lse=False):
    import kernel
    closed = closed or {}
    states = {h: 1 for h in dense}
    states.update({h: 2 for h in dec})
    states.update({h: 2 for h in closed})
    frozen, hidx, live = routing(H, states)
    patt = make_pattern(H, S, seed=H * S + T)
    alpha, rho, z = make_decomp(H, S, seed=H + S + T, scale=dec_scale)
    cf = None
    if closed:
        ca, cr, cz = closed_params(H, S, closed)
        for h in closed:
            alpha[h], rho[h], z[h] = ca[h], cr[h], cz[h]
        cf = kernel.classify_closed_form(alpha, rho, z)
    alpha, rho, z = (t.to(buf_dtype) for t in (alpha, rho, z))
    g = torch.Generator().manual_seed(T * hd + B)
    q, k, v = (torch.randn(B, H, T, hd, generator=g) for _ in range(3))
    pidx, kpatt = None, patt
    if compact:
        pidx = torch.zeros(H, dtype=torch.int32)
        for slot, h in enumerate(dense):
            pidx[h] = slot
        kpatt = patt[list(dense)].contiguous()
    has_dec = bool(dec) or bool(closed)
    if strided:
        qk = torch.stack([q[:, live], k[:, live]], dim=2).transpose(1, 2).contiguous().transpose(1, 2)
        qk = qk.to(DEV).requires_grad_(backward)
        tq, tk = qk[:, :, 0], qk[:, :, 1]
    else:
        tq = q[:, live].contiguous().to(DEV).requires_grad_(backward)
        tk = k[:, live].contiguous().to(DEV).requires_grad_(backward)
    tv = v.to(DEV).requires_grad_(backward)
    a_d = alpha.to(DEV).requires_grad_(backward) if has_dec else None
    r_d = rho.to(DEV).requires_grad_(backward) if has_dec else None
    lse = torch.empty(B, H, T, device=DEV) if check_lse else None
    y = kernel.fused_mixed_attn(tq, tk, tv, kpatt.to(DEV), frozen.to(DEV), hidx.to(DEV),
                                None if pidx is None else pidx.to(DEV), alpha=a_d, rho=r_d,
                                z=z.to(DEV) if has_dec else None, closed_form=cf, lse=lse)
    assert y.dtype == torch.float32
    what = f"f32 B{B} H{H} T{T} hd{hd} dense={list(dense)} dec={list(dec)} closed={closed}"
    kw = dict(patt=f64(kpatt), alpha=f64(alpha), rho=f64(rho), z=f64(z), sm_scale=scale_of(hd))
    ref = orc.eager_mixed_attention(f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), hidx.numpy(),
                                    None if pidx is None else pidx.numpy(), None, **kw)
    _maxabs(y, ref, TOL_F, "out " + what)
    if check_lse and live:
        for h in live:
            for b in range(B):
                s = (f64(q[b, h]) @ f64(k[b, h]).T) * scale_of(hd) * np.log2(np.e)
                s = np.where(np.tril(np.ones((T, T), dtype=bool)), s, -np.inf)
                m = s.max(-1)
                ref_lse = m + np.log2(np.exp2(s - m[:, None]).sum(-1))
                _maxabs(lse[b, h], ref_lse, 1e-4, f"lse b{b} h{h}")
    if not backward:
        return
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(T + hd))
    (y * w.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    dq, dk, dv = orc.eager_mixed_attention_grads(
        f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), f64(w), hidx.numpy(),
        None if pidx is None else pidx.numpy(), **kw)
    _maxabs(tv.grad, dv, TOL_B, "dv " + what)
    if live:
        gq = qk.grad[:, :, 0] if strided else tq.grad
        gk = qk.grad[:, :, 1] if strided else tk.grad
        _maxabs(gq, dq, TOL_B, "dq " + what)
        _maxabs(gk, dk, TOL_B, "dk " + what)
    if has_dec:
        assert a_d.grad is None and r_d.grad is None, "alpha/rho must receive no gradient"


CASES = [
    (2, 12, 1024, 64, 1024, [0, 1, 2]),
    (2, 12, 1024, 64, 1024, []),
    (2, 12, 1024, 64, 1024, list(range(12))),
    (2, 12, 1024, 64, 1024, [3, 7, 11]),
    (2, 12, 700, 64, 1024, [0, 5, 11]),
    (2, 12, 37, 64, 1024, [0, 5]),
    (1, 16, 2048, 96, 2048, [0, 7, 8, 15]),
    (4, 12, 2048, 64, 2048, [0, 1, 2]),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}d{c[3]}nf{len(c[5])}")
def test_f32_dense_and_live(case):
    run_f32(*case)


@pytest.mark.parametrize("case", CASES[:6], ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}nf{len(c[5])}")
def test_f32_strided_qk(case):
    run_f32(*case, strided=True)


@pytest.mark.parametrize("case", [
    (2, 12, 1024, 64, 1024, [0, 1], [2, 3]),
    (2, 12, 1024, 64, 1024, [], [0, 5, 11]),
    (2, 12, 1024, 64, 1024, [], list(range(12))),
    (2, 12, 700, 64, 1024, [3], [0, 7]),
    (2, 12, 37, 64, 1024, [5], [0, 2]),
    (1, 16, 2048, 96, 2048, [0, 8], [7, 15]),
], ids=lambda c: f"T{c[2]}d{c[3]}nf{len(c[5])}nd{len(c[6])}")
def test_f32_decomposed(case):
    B, H, T, hd, S, fz, dec = case
    run_f32(B, H, T, hd, S, fz, dec)


def test_f32_decomposed_bf16_buffers_extreme_logits_and_compact():
    run_f32(2, 12, 700, 64, 1024, [3], [0, 7], buf_dtype=torch.bfloat16)
    run_f32(2, 12, 700, 64, 1024, [3], [0, 7], dec_scale=40.0)
    run_f32(2, 12, 1000, 64, 1024, [], list(range(12)), dec_scale=40.0)
    run_f32(2, 12, 700, 64, 1024, [3, 9], [0, 7], strided=True, compact=True)


def test_f32_closed_forms_lse_and_head_dims():
    run_f32(2, 8, 900, 64, 1024, [2], [5], closed={0: ("mean", 0), 3: ("decay", 0.05), 6: ("window", 100)},
            check_lse=True)
    run_f32(2, 4, 333, 32, 512, [2], [1])
    run_f32(1, 6, 777, 128, 1024, [1, 4], [0])
    run_f32(1, 4, 600, 256, 640, [1], [2], check_lse=True)
    run_f32(1, 4, 1, 64, 64, [1], [2])


def test_f32_gqa_forward():
    import kernel
    B, H, HKV, T, hd, S = 2, 14, 2, 700, 64, 768
    kvidx = torch.from_numpy(orc.gqa_kvidx(H, HKV))
    frozen, hidx, live = routing(H, {0: 2, 3: 2, 8: 1, 13: 2})
    g = torch.Generator().manual_seed(7)
    q = torch.randn(B, len(live), T, hd, generator=g)
    k = torch.randn(B, HKV, T, hd, generator=g)
    v = torch.randn(B, HKV, T, hd, generator=g)
    patt = make_pattern(1, S, seed=3)
    pidx = torch.zeros(H, dtype=torch.int32)
    alpha, rho, z = closed_params(H, S, {0: ("mean", 0), 3: ("decay", 0.02)})
    a2, r2, z2 = make_decomp(H, S, seed=11)
    alpha[13], rho[13], z[13] = a2[13], r2[13], z2[13]
    cf = kernel.classify_closed_form(alpha, rho, z)
    y = kernel.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV), hidx.to(DEV),
                                pidx.to(DEV), alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV),
                                kvidx=kvidx.to(DEV), closed_form=cf)
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy(), hidx.numpy(), pidx.numpy(),
                                    kvidx.numpy(), patt=f64(patt), alpha=f64(alpha), rho=f64(rho), z=f64(z),
                                    sm_scale=scale_of(hd))
    _maxabs(y, ref, TOL_F, "f32 gqa")


@pytest.mark.parametrize("T,Tv,S,hd", [(37, 40, 64, 64), (700, 700, 1024, 128), (513, 513, 576, 256)])
def test_f32_frozen_pv_forward_backward(T, Tv, S, hd):
    import kernel
    nf, B = 3, 2
    patt = make_pattern(4, S, seed=T)
    fz = torch.tensor([3, 0, 2], dtype=torch.int32)
    v = torch.randn(B, nf, Tv, hd, generator=torch.Generator().manual_seed(T + hd))
    tv = v.to(DEV).requires_grad_(True)
    y = kernel.frozen_pv(patt.to(DEV), tv, fz.to(DEV), T)
    ref = orc.frozen_pv(f64(patt), f64(v), fz.numpy(), T)
    _maxabs(y, ref, TOL_F, f"frozen_pv f32 T{T} hd{hd}")
    w = torch.randn(y.shape, generator=torch.Generator().manual_seed(5))
    (y * w.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    dv_ref = np.zeros((B, nf, Tv, hd))
    for f in range(nf):
        pm = f64(patt[int(fz[f]), :T, :T])
        for b in range(B):
            dv_ref[b, f, :T] = pm.T @ f64(w[b, f])
    _maxabs(tv.grad, dv_ref, TOL_B, f"frozen_pv f32 dv T{T} hd{hd}")
