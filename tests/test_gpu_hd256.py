"""GPU parity of the hd-256 tier (Qwen3.5's head dim) against the float64
oracle: the two-slot live-head kernel (with and without the causal split and
the work queue, LSE included), dense and decomposed frozen heads, the
closed-form scan, GQA through kvidx at a Qwen3.5-like shape on sampled rows,
and frozen_pv.  Bound: max-abs <= 2e-2 and relative-L2 <= 1e-2, as the
rest of the operator grid (kernel/test_fused_attn.py:162-230 of the
reference, whose Triton kernels take any power-of-two head dim).  The
backward stops at hd 128 and says so."""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import compare, f64, make_pattern, qkv, routing, scale_of
from test_gpu_mixed_attn import run_case

pytestmark = pytest.mark.gpu
DEV = "cuda"
HD = 256


@pytest.mark.parametrize("case", [
    (2, 8, 1000, HD, 1024, [1, 6], [3]),
    (1, 4, 1, HD, 64, [1], []),
    (2, 4, 37, HD, 64, [], [0]),
    (1, 6, 2048, HD, 2048, [], []),
    (3, 4, 777, HD, 1024, list(range(4)), []),
    (2, 5, 513, HD, 576, [0], [2, 4]),
], ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}nd{len(c[5])}nc{len(c[6])}")
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_mixed_heads_hd256(case, dtype):
    B, H, T, hd, S, dense, dec = case
    run_case(B, H, T, hd, S, dense, dec, dtype=dtype)


def test_closed_forms_and_lse_hd256():
    run_case(2, 8, 900, HD, 1024, [2], dec=[5],
             closed={0: ("mean", 0), 3: ("decay", 0.03), 6: ("window", 200)}, check_lse=True)


@pytest.mark.parametrize("B,H,T", [(1, 2, 3000), (1, 1, 5000), (2, 3, 2100)])
def test_causal_split_hd256(B, H, T):
    """Few live heads at long T: split key segments merged by the combine
    kernel (values and LSE), work queue on."""
    import kernel
    q, k, v = qkv(B, H, T, HD, seed=T + H, dtype=torch.bfloat16)
    frozen = torch.zeros(H, dtype=torch.int32)
    lse = torch.empty(B, H, T, device=DEV, dtype=torch.float32)
    y = kernel.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), None, frozen.to(DEV), lse=lse)
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy())
    compare(y, ref, what=f"hd256 split B{B} H{H} T{T}")
    for b in range(B):
        for h in range(H):
            qh, kh = f64(q[b, h]), f64(k[b, h])
            s = (qh @ kh.T) * scale_of(HD) * np.log2(np.e)
            s = np.where(np.tril(np.ones((T, T), dtype=bool)), s, -np.inf)
            m = s.max(-1)
            ref_lse = m + np.log2(np.exp2(s - m[:, None]).sum(-1))
            assert np.abs(lse[b, h].cpu().numpy() - ref_lse).max() < 2e-2


def test_sharp_scores_hd256():
    """Scores that grow along the keys force the rare rebase from the raw
    scores kept in registers (no K tile is re-read in the two-slot kernel)."""
    import kernel
    B, H, T = 1, 2, 1500
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, H, T, HD, generator=g)
    k = torch.randn(B, H, T, HD, generator=g) * torch.linspace(0.2, 4.0, T)[None, None, :, None]
    v = torch.randn(B, H, T, HD, generator=g)
    q, k, v = (t.bfloat16() for t in (q, k, v))
    frozen = torch.zeros(H, dtype=torch.int32)
    y = kernel.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), None, frozen.to(DEV))
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy())
    compare(y, ref, what="hd256 growing scores")


def test_gqa_qwen35_shape_sampled_rows():
    """Qwen3.5-like attention layer: 16 query / 2 KV heads of hd 256,
    B=2, T=4096, four frozen heads (two dense mean patterns, a decay scan
    head, a learned decomposed head), compared on sampled rows."""
    import kernel
    B, H, HKV, T = 2, 16, 2, 4096
    kvidx = torch.as_tensor(orc.gqa_kvidx(H, HKV))
    frozen, hidx, live = routing(H, {1: 1, 6: 1, 9: 2, 14: 2})
    g = torch.Generator().manual_seed(256)
    q = torch.randn(B, len(live), T, HD, generator=g).bfloat16()
    k = torch.randn(B, HKV, T, HD, generator=g).bfloat16()
    v = torch.randn(B, HKV, T, HD, generator=g).bfloat16()
    mean = torch.from_numpy(orc.mean_pattern(T)).to(torch.bfloat16)
    patt = mean.unsqueeze(0)
    pidx = torch.zeros(H, dtype=torch.int32)
    alpha = torch.zeros(H, T)
    rho = torch.zeros(H, T)
    a9, r9 = orc.closed_form_params("decay", 0.01, T)
    alpha[9], rho[9] = torch.from_numpy(a9).float(), torch.from_numpy(r9).float()
    alpha[14] = torch.randn(T, generator=g) * 0.5
    rho[14] = torch.randn(T, generator=g) * 0.5
    z = torch.from_numpy(orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())).float()
    cf = kernel.classify_closed_form(alpha, rho, z)
    assert int(cf[0][9]) == kernel.CLOSED_DECAY and int(cf[0][14]) == 0
    y = kernel.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV), hidx.to(DEV),
                                pidx.to(DEV), alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV),
                                kvidx=kvidx.to(DEV), closed_form=cf)
    torch.cuda.synchronize()
    rows = orc.sample_rows(T, seed=256)
    prow = {h: f64(mean[torch.as_tensor(rows)]) for h in (1, 6)}
    ref = orc.eager_rows(f64(q), f64(k), f64(v), frozen.numpy(), rows, hidx.numpy(), pidx.numpy(),
                         kvidx=kvidx.numpy(), patt_rows=prow, alpha=f64(alpha), rho=f64(rho), z=f64(z))
    got = y[:, :, torch.as_tensor(rows, device=y.device)].float().cpu()
    compare(got, ref, what="hd256 GQA sampled rows")


@pytest.mark.parametrize("T,S,pdtype", [(1300, 1344, torch.bfloat16), (700, 700, torch.float32)])
def test_frozen_pv_hd256(T, S, pdtype):
    import kernel
    B, nf = 2, 3
    patt = make_pattern(4, S, seed=T).to(pdtype)
    fz = torch.tensor([3, 0, 2], dtype=torch.int32)
    v = torch.randn(B, nf, T, HD, generator=torch.Generator().manual_seed(T)).bfloat16()
    y = kernel.frozen_pv(patt.to(DEV), v.to(DEV), fz.to(DEV), T)
    torch.cuda.synchronize()
    ref = orc.frozen_pv(f64(patt), f64(v), fz.numpy(), T)
    compare(y, ref, what=f"frozen_pv hd256 T{T} {pdtype}")


def test_backward_refuses_hd256():
    import kernel
    B, H, T = 1, 2, 64
    q, k, v = (t.to(DEV).requires_grad_(True) for t in qkv(B, H, T, HD, seed=1, dtype=torch.bfloat16))
    frozen = torch.zeros(H, dtype=torch.int32, device=DEV)
    y = kernel.fused_mixed_attn(q, k, v, None, frozen)
    with pytest.raises(RuntimeError, match="head_dim 256"):
        y.float().sum().backward()
