"""GPU parity of fused_mixed_attn (libsafattn.so) against the CPU oracle.

Mirrors the reference's kernel test grid (kernel/test_fused_attn.py:162-230):
dense / decomposed / live mixes, nothing or everything frozen, non-contiguous
freeze sets, unaligned T with S > T, tiny T, hd in {32, 64, 96, 128}, strided
q/k views of one fused projection, bf16 decomposed buffers, extreme logits,
compact pidx; plus the GQA kvidx map (qwen/kernel/fused_attn.py:667-768), the
closed-form scan heads and the base-2 LSE.  Bound: max-abs <= 2e-2 and
relative-L2 <= 1e-2 against float64 oracle outputs computed from the same
(rounded) inputs.
"""
import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import (closed_params, compare, f64, make_decomp, make_pattern,
                       qkv, routing, scale_of)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _kernel():
    import kernel
    return kernel


def run_case(B, H, T, hd, S, dense, dec=(), dtype=torch.bfloat16, strided=False,
             no_patt=False, buf_dtype=torch.float32, dec_scale=0.8, compact_patt=False,
             closed=None, check_lse=False):
    K = _kernel()
    closed = closed or {}
    states = {h: 1 for h in dense}
    states.update({h: 2 for h in dec})
    states.update({h: 2 for h in closed})
    frozen, hidx, live = routing(H, states)
    patt = make_pattern(H, S, seed=H * S + T)
    alpha, rho, z = make_decomp(H, S, seed=H + S + T, scale=dec_scale)
    if closed:
        ca, cr, cz = closed_params(H, S, closed)
        for h in closed:
            alpha[h], rho[h], z[h] = ca[h], cr[h], cz[h]
    alpha, rho, z = (t.to(buf_dtype) for t in (alpha, rho, z))
    q, k, v = qkv(B, H, T, hd, seed=T * hd + B, dtype=dtype)

    pidx = None
    kern_patt = None if no_patt else patt
    if compact_patt:
        pidx = torch.zeros(H, dtype=torch.int32)
        for slot, h in enumerate(dense):
            pidx[h] = slot
        kern_patt = None if no_patt else patt[list(dense)].contiguous()

    qd = q[:, live].to(DEV)
    kd = k[:, live].to(DEV)
    if strided:
        # q/k as interleaved views of one (B, T, 2, U, hd) projection output
        qk = torch.stack([q[:, live], k[:, live]], dim=2).permute(0, 3, 2, 1, 4).contiguous().to(DEV)
        qd, kd = qk[:, :, 0].transpose(1, 2), qk[:, :, 1].transpose(1, 2)
    has_dec = bool(dec) or bool(closed)
    cf = None
    if closed:
        cf = K.classify_closed_form(alpha, rho, z)
        for h in closed:
            assert cf[0][h] != 0, f"head {h} not recognised as closed form"
    lse = torch.empty(B, H, T, device=DEV, dtype=torch.float32) if check_lse else None
    y = K.fused_mixed_attn(
        qd, kd, v.to(DEV), None if kern_patt is None else kern_patt.to(DEV),
        frozen.to(DEV), hidx.to(DEV), None if pidx is None else pidx.to(DEV),
        alpha=alpha.to(DEV) if has_dec else None, rho=rho.to(DEV) if has_dec else None,
        z=z.to(DEV) if has_dec else None, closed_form=cf, lse=lse)
    torch.cuda.synchronize()

    ref = orc.eager_mixed_attention(
        f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), hidx.numpy(),
        None if pidx is None else pidx.numpy(), None,
        patt=patt.numpy() if not compact_patt else patt[list(dense)].numpy(),
        alpha=f64(alpha), rho=f64(rho), z=f64(z), sm_scale=scale_of(hd))
    compare(y, ref, what=f"B{B} H{H} T{T} hd{hd} dense={list(dense)} dec={list(dec)} "
                         f"closed={closed} {dtype}")
    if check_lse and live:
        for h in live:
            for b in range(B):
                qh = f64(q[b, h]); kh = f64(k[b, h])
                s = (qh @ kh.T) * scale_of(hd) * orc.math.log2(orc.math.e)
                s = np.where(np.tril(np.ones((T, T), dtype=bool)), s, -np.inf)
                m = s.max(-1)
                ref_lse = m + np.log2(np.exp2(s - m[:, None]).sum(-1))
                got = lse[b, h].cpu().numpy()
                assert np.abs(got - ref_lse).max() < 2e-2, f"lse b{b} h{h}"
    return y


CASES = [
    (2, 12, 1024, 64, 1024, [0, 1, 2]),
    (2, 12, 1024, 64, 1024, []),
    (2, 12, 1024, 64, 1024, list(range(12))),
    (2, 12, 1024, 64, 1024, [3, 7, 11]),
    (2, 12, 700, 64, 1024, [0, 5, 11]),
    (2, 12, 37, 64, 1024, [0, 5]),
    (1, 16, 2048, 96, 2048, [0, 7, 8, 15]),
    (4, 12, 2048, 64, 2048, [0, 1, 2]),
    (1, 8, 1000, 128, 1024, [1, 6]),
    (2, 4, 333, 32, 512, [2]),
    (1, 4, 1, 64, 64, [1]),
    (3, 6, 777, 128, 1024, [1, 4]),
    (6, 4, 1500, 128, 1536, [0, 3]),
    (4, 5, 1200, 64, 1280, [2, 4]),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}d{c[3]}nf{len(c[5])}")
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_dense_and_live(case, dtype):
    run_case(*case, dtype=dtype)


@pytest.mark.parametrize("case", CASES[:6], ids=lambda c: f"B{c[0]}H{c[1]}T{c[2]}nf{len(c[5])}")
def test_strided_qk_views(case):
    run_case(*case, dtype=torch.bfloat16, strided=True)


DEC_CASES = [
    (2, 12, 1024, 64, 1024, [0, 1], [2, 3], False),
    (2, 12, 1024, 64, 1024, [], [0, 5, 11], True),
    (2, 12, 1024, 64, 1024, [], list(range(12)), True),
    (2, 12, 700, 64, 1024, [3], [0, 7], False),
    (2, 12, 37, 64, 1024, [5], [0, 2], False),
    (3, 12, 1, 64, 64, [], [0, 2], False),
    (2, 12, 65, 64, 128, [], [1, 4, 9], False),
    (1, 16, 2048, 96, 2048, [0, 8], [7, 15], False),
    (4, 12, 2048, 64, 2048, [1], [0, 2], False),
    (1, 8, 1000, 128, 1024, [2], [3, 5], False),
]


@pytest.mark.parametrize("case", DEC_CASES, ids=lambda c: f"T{c[2]}d{c[3]}nf{len(c[5])}nd{len(c[6])}")
def test_decomposed(case):
    B, H, T, hd, S, fz, dec, np_ = case
    run_case(B, H, T, hd, S, fz, dec, no_patt=np_)


@pytest.mark.parametrize("case", DEC_CASES[:3], ids=lambda c: f"nd{len(c[6])}")
def test_decomposed_bf16_buffers(case):
    B, H, T, hd, S, fz, dec, np_ = case
    run_case(B, H, T, hd, S, fz, dec, no_patt=np_, buf_dtype=torch.bfloat16)


@pytest.mark.parametrize("case", [
    (2, 12, 700, 64, 1024, [3], [0, 7], False),
    (2, 12, 37, 64, 1024, [], [0, 2, 5], True),
    (2, 12, 1000, 64, 1024, [], list(range(12)), True),
], ids=["T700", "T37", "T1000all"])
def test_decomposed_extreme_logits(case):
    B, H, T, hd, S, fz, dec, np_ = case
    run_case(B, H, T, hd, S, fz, dec, no_patt=np_, dec_scale=40.0)


def test_decomposed_fp16_bf16_and_rebuilt_forms():
    """The three decomposed forms in one call (bf16 inputs), each against the
    float64 oracle.  Head 0: a decay (alpha = 0, so the row factor is <= 1
    and every workgroup takes the fp16 form); head 1: moderate random
    alpha / rho (fp16 where the row factor allows, bf16 hi + lo elsewhere);
    head 2: an attention sink alpha[0] = +12 with a steep decay (row factors
    up to 2^17: the bf16 hi + lo form); head 3: an alpha spike of +150 at key
    1200 (workgroups past it rebuild cell by cell).  T = 2500 (so the fp16
    form needs row factors <= 2^2)."""
    import kernel
    B, H, T, hd, S = 2, 4, 2500, 64, 2560
    g = torch.Generator().manual_seed(91)
    d = torch.arange(S, dtype=torch.float32)
    alpha = torch.zeros(H, S)
    rho = torch.zeros(H, S)
    rho[0] = -0.03 * d
    alpha[1] = torch.randn(S, generator=g) * 0.7
    rho[1] = torch.randn(S, generator=g) * 0.7
    alpha[2, 0] = 12.0
    rho[2] = -0.5 * d
    alpha[3] = torch.randn(S, generator=g) * 0.5
    alpha[3, 1200] = 150.0
    rho[3] = -0.01 * d
    z = torch.from_numpy(orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())).float()
    frozen = torch.full((H,), 2, dtype=torch.int32)
    q, k, v = qkv(B, H, T, hd, seed=8, dtype=torch.bfloat16)
    y = kernel.fused_mixed_attn(q[:, :0].to(DEV), k[:, :0].to(DEV), v.to(DEV), None, frozen.to(DEV),
                                alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV))
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(None, None, f64(v), frozen.numpy(), alpha=f64(alpha), rho=f64(rho),
                                    z=f64(z))
    for h in range(H):
        compare(y[:, h:h + 1], ref[:, h:h + 1], what=f"decomposed forms head {h}")


def test_decomposed_fp16_activations_fp16_form_and_rebuild():
    """fp16 activations: the decomposed heads take the fp16 factored form
    where the row factor allows and rebuild P cell by cell elsewhere (the
    bf16 hi + lo form needs bf16 inputs), against the float64 oracle.  Head
    0: a decay (fp16 form everywhere); head 1: moderate random alpha / rho
    (both); head 2: an attention sink with a steep decay (rebuild); head 3:
    an alpha spike (rebuild past it).  Alone and beside live heads."""
    import kernel
    B, H, T, hd, S = 2, 6, 2500, 64, 2560
    g = torch.Generator().manual_seed(93)
    d = torch.arange(S, dtype=torch.float32)
    alpha = torch.zeros(H, S)
    rho = torch.zeros(H, S)
    rho[0] = -0.03 * d
    alpha[1] = torch.randn(S, generator=g) * 0.7
    rho[1] = torch.randn(S, generator=g) * 0.7
    alpha[2, 0] = 12.0
    rho[2] = -0.5 * d
    alpha[3] = torch.randn(S, generator=g) * 0.5
    alpha[3, 1200] = 150.0
    rho[3] = -0.01 * d
    z = torch.from_numpy(orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())).float()
    q, k, v = qkv(B, H, T, hd, seed=9, dtype=torch.float16)
    # decomposed only (heads 0-3), then heads 4 and 5 live beside them
    for n_live in (0, 2):
        Hc = 4 + n_live
        st = {h: 2 for h in range(4)}
        frozen, hidx, live = routing(Hc, st)
        y = kernel.fused_mixed_attn(q[:, live].to(DEV), k[:, live].to(DEV), v[:, :Hc].to(DEV), None,
                                    frozen.to(DEV), hidx.to(DEV), alpha=alpha[:Hc].to(DEV), rho=rho[:Hc].to(DEV),
                                    z=z[:Hc].to(DEV))
        torch.cuda.synchronize()
        ref = orc.eager_mixed_attention(f64(q[:, live]), f64(k[:, live]), f64(v[:, :Hc]), frozen.numpy(),
                                        hidx.numpy(), None, None, alpha=f64(alpha[:Hc]), rho=f64(rho[:Hc]),
                                        z=f64(z[:Hc]), sm_scale=scale_of(hd))
        for h in range(Hc):
            compare(y[:, h:h + 1], ref[:, h:h + 1], what=f"fp16 activations, {n_live} live, head {h}")


def test_decomposed_large_values_keep_the_bf16_form():
    """Values of magnitude ~1e5 scale to key-scaled values past the fp16
    range, so the workgroups of a decay head (row factor <= 1, otherwise an
    fp16 candidate) keep the bf16 form: finite outputs within bf16 rounding
    of the float64 oracle (relative bounds: the outputs are ~1e5)."""
    import kernel
    B, H, T, hd, S = 1, 2, 1200, 64, 1280
    d = torch.arange(S, dtype=torch.float32)
    alpha = torch.zeros(H, S)
    rho = torch.stack([-0.02 * d, -0.2 * d])
    z = torch.from_numpy(orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())).float()
    frozen = torch.full((H,), 2, dtype=torch.int32)
    _, _, v = qkv(B, H, T, hd, seed=12, dtype=torch.float32)
    v = (v * 1e5).bfloat16()
    y = kernel.fused_mixed_attn(v[:, :0].to(DEV), v[:, :0].to(DEV), v.to(DEV), None, frozen.to(DEV),
                                alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV))
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(None, None, f64(v), frozen.numpy(), alpha=f64(alpha), rho=f64(rho),
                                    z=f64(z))
    compare(y.float() / 1e5, ref / 1e5, what="decomposed, |v| ~ 1e5")


def test_decomposed_factored_and_rebuilt_workgroups():
    """The decomposed kernel picks, per workgroup, the factored form (key and
    row factors around a Toeplitz operand) when every row's z lies within
    kFactorRange of max(a) + max(r), else the cell-by-cell rebuild.  Head 0:
    moderate parameters (factored everywhere); head 1: an alpha spike of +150
    at key 1500 (workgroups past it rebuild, those before stay factored); head
    2: rho with -inf entries (a window) and a lane of -inf alpha; head 3: a
    slow ramp of alpha over 200 log units (factored only where the ramp's
    span allows).  Both forms against the float64 oracle, bf16 and fp16
    (fp16 always rebuilds)."""
    import kernel
    B, H, T, hd, S = 2, 4, 2500, 64, 2560
    g = torch.Generator().manual_seed(77)
    alpha = torch.randn(H, S, generator=g) * 0.7
    rho = torch.randn(H, S, generator=g) * 0.7
    alpha[1, 1500] = 150.0
    rho[2, 300:] = float("-inf")
    alpha[2, 40:48] = float("-inf")
    alpha[3] = torch.linspace(-100.0, 100.0, S)
    z = torch.from_numpy(orc.decomposed_logz(alpha.double().numpy(), rho.double().numpy())).float()
    frozen = torch.full((H,), 2, dtype=torch.int32)
    for dtype in (torch.bfloat16, torch.float16):
        q, k, v = qkv(B, H, T, hd, seed=5, dtype=dtype)
        y = kernel.fused_mixed_attn(q[:, :0].to(DEV), k[:, :0].to(DEV), v.to(DEV), None, frozen.to(DEV),
                                    alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV))
        torch.cuda.synchronize()
        ref = orc.eager_mixed_attention(None, None, f64(v), frozen.numpy(), alpha=f64(alpha), rho=f64(rho),
                                        z=f64(z))
        compare(y, ref, what=f"decomposed factored/rebuilt {dtype}")


def test_compact_pidx_with_decomposed():
    run_case(2, 12, 700, 64, 1024, [3, 9], [0, 7], strided=True, compact_patt=True)


CLOSED = [
    (2, 12, 1024, 64, 1024, {0: ("mean", 0), 5: ("decay", 0.01), 9: ("window", 64)}),
    (1, 12, 3000, 64, 3072, {1: ("decay", 0.001), 2: ("decay", 0.1), 3: ("window", 1000),
                             4: ("mean", 0), 11: ("window", 1)}),
    (2, 8, 777, 128, 1024, {0: ("mean", 0), 7: ("decay", 0.05), 3: ("window", 300)}),
    (1, 4, 600, 96, 640, {0: ("window", 700), 1: ("decay", 0.02)}),
    (1, 4, 1, 64, 64, {2: ("mean", 0)}),
    (2, 6, 513, 32, 576, {0: ("mean", 0), 1: ("window", 128)}),
]


@pytest.mark.parametrize("case", CLOSED, ids=lambda c: f"T{c[2]}d{c[3]}n{len(c[5])}")
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_closed_form_scan(case, dtype):
    B, H, T, hd, S, kinds = case
    run_case(B, H, T, hd, S, [], closed=kinds, dtype=dtype)


def test_closed_form_with_all_kinds_and_lse():
    run_case(2, 12, 1024, 64, 1024, [4], dec=[6],
             closed={0: ("mean", 0), 1: ("decay", 0.03), 2: ("window", 256)}, check_lse=True)


@pytest.mark.parametrize("B,H,T,hd,qt", [(1, 2, 4096, 64, 2), (1, 3, 3000, 128, 1), (2, 2, 2500, 64, 1),
                                         (1, 1, 8192, 32, 2)])
def test_causal_split_of_long_query_blocks(B, H, T, hd, qt):
    """Few heads at long T: the live-head kernel splits the heaviest query
    blocks into key segments and merges the fp32 partials (values and LSE)."""
    import kernel
    q, k, v = qkv(B, H, T, hd, seed=T + H, dtype=torch.bfloat16)
    frozen = torch.zeros(H, dtype=torch.int32)
    lse = torch.empty(B, H, T, device=DEV, dtype=torch.float32)
    y = kernel.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), None, frozen.to(DEV), lse=lse,
                                flash_qtiles=qt)
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy())
    compare(y, ref, what=f"split B{B} H{H} T{T} hd{hd} qt{qt}")
    for h in range(H):
        qh, kh = f64(q[0, h]), f64(k[0, h])
        s = (qh @ kh.T) * scale_of(hd) * np.log2(np.e)
        s = np.where(np.tril(np.ones((T, T), dtype=bool)), s, -np.inf)
        m = s.max(-1)
        ref_lse = m + np.log2(np.exp2(s - m[:, None]).sum(-1))
        assert np.abs(lse[0, h].cpu().numpy() - ref_lse).max() < 2e-2


@pytest.mark.parametrize("T,hd,pdtype", [(2000, 64, torch.bfloat16), (1537, 128, torch.float32),
                                         (2304, 128, torch.bfloat16), (1111, 32, torch.float16),
                                         (1300, 96, torch.bfloat16)])
def test_dense_causal_split(T, hd, pdtype):
    """Few dense heads at long T: the dense P.V kernel splits the heaviest
    query blocks into key segments whose fp32 partials the combine kernel
    sums; both the split (fused operator, workspace given) and the unsplit
    (frozen_pv, no workspace) paths match the oracle.  S = T + 40 covers both
    the 16-byte pattern rows and the element-wise path (fp32 rows of 1577)."""
    K = _kernel()
    B, H, S = 2, 3, T + 40
    frozen, hidx, live = routing(H, {0: 1, 2: 1})
    patt = make_pattern(2, S, seed=T)
    pidx = torch.tensor([0, 0, 1], dtype=torch.int32)
    q, k, v = qkv(B, H, T, hd, seed=T + hd, dtype=torch.bfloat16)
    q, k = q[:, live].contiguous(), k[:, live].contiguous()
    pd = patt.to(pdtype)
    y = K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), pd.to(DEV), frozen.to(DEV), hidx.to(DEV),
                           pidx.to(DEV))
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy(), hidx.numpy(), pidx.numpy(),
                                    patt=f64(pd))
    compare(y, ref, what=f"dense split T{T} hd{hd} {pdtype}")
    fz = torch.tensor([0, 1], dtype=torch.int32)
    yu = K.frozen_pv(pd.to(DEV), v[:, [0, 2]].contiguous().to(DEV), fz.to(DEV), T)
    torch.cuda.synchronize()
    compare(yu, ref[:, [0, 2]], what=f"dense unsplit T{T} hd{hd} {pdtype}")


@pytest.mark.parametrize("B,T,hd,dtype", [(1, 8, 64, torch.bfloat16), (2, 72, 32, torch.bfloat16),
                                          (3, 1000, 128, torch.bfloat16), (2, 1544, 64, torch.float16),
                                          (4, 520, 96, torch.bfloat16), (1, 2048, 128, torch.float16),
                                          (4, 777, 32, torch.bfloat16), (8, 600, 64, torch.float16)])
def test_dense_pattern_in_activation_dtype(B, T, hd, dtype):
    """Dense patterns stored in the activation dtype with 16-byte rows (the
    kernel's unconditional buffer-load path) and S = T, so the last rows'
    loads run past the end of the pattern buffer: both the fused operator
    (causal split with a workspace) and frozen_pv match the oracle; the last
    head's pattern is the last slab of the buffer."""
    K = _kernel()
    H = 3
    frozen, hidx, live = routing(H, {0: 1, 2: 1})
    patt = make_pattern(2, T, seed=T + hd).to(dtype)
    pidx = torch.tensor([1, 0, 0], dtype=torch.int32)
    q, k, v = qkv(B, H, T, hd, seed=T * 3 + hd, dtype=dtype)
    q, k = q[:, live].contiguous(), k[:, live].contiguous()
    y = K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV), hidx.to(DEV),
                           pidx.to(DEV))
    torch.cuda.synchronize()
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy(), hidx.numpy(), pidx.numpy(),
                                    patt=f64(patt))
    compare(y, ref, what=f"dense {dtype} patterns B{B} T{T} hd{hd}")
    fz = torch.tensor([1, 0], dtype=torch.int32)
    yu = K.frozen_pv(patt.to(DEV), v[:, [0, 2]].contiguous().to(DEV), fz.to(DEV), T)
    torch.cuda.synchronize()
    compare(yu, ref[:, [0, 2]], what=f"frozen_pv {dtype} patterns B{B} T{T} hd{hd}")


def test_gqa_kvidx():
    """Qwen-style map: 14 query heads over 2 KV heads, frozen query heads read
    the shared V of their group (qwen/kernel/fused_attn.py:254-259)."""
    K = _kernel()
    B, H, HKV, T, hd, S = 2, 14, 2, 700, 64, 768
    kvidx = torch.from_numpy(orc.gqa_kvidx(H, HKV))
    states = {0: 2, 3: 2, 8: 1, 13: 2}
    frozen, hidx, live = routing(H, states)
    g = torch.Generator().manual_seed(7)
    q = torch.randn(B, len(live), T, hd, generator=g).bfloat16()
    k = torch.randn(B, HKV, T, hd, generator=g).bfloat16()
    v = torch.randn(B, HKV, T, hd, generator=g).bfloat16()
    patt = make_pattern(1, S, seed=3)
    pidx = torch.zeros(H, dtype=torch.int32)
    alpha, rho, z = closed_params(H, S, {0: ("mean", 0), 3: ("decay", 0.02)})
    a2, r2, z2 = make_decomp(H, S, seed=11)
    alpha[13], rho[13], z[13] = a2[13], r2[13], z2[13]
    cf = K.classify_closed_form(alpha, rho, z)
    assert cf[0][0] == K.CLOSED_MEAN and cf[0][3] == K.CLOSED_DECAY and cf[0][13] == 0
    y = K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV),
                           hidx.to(DEV), pidx.to(DEV), alpha=alpha.to(DEV), rho=rho.to(DEV),
                           z=z.to(DEV), kvidx=kvidx.to(DEV), closed_form=cf)
    torch.cuda.synchronize()
    assert y.shape == (B, H, T, hd)
    ref = orc.eager_mixed_attention(f64(q), f64(k), f64(v), frozen.numpy(), hidx.numpy(),
                                    pidx.numpy(), kvidx.numpy(), patt=patt.numpy(),
                                    alpha=f64(alpha), rho=f64(rho), z=f64(z),
                                    sm_scale=scale_of(hd))
    compare(y, ref, what="gqa")


def test_frozen_heads_ignore_qk():
    """With the identity hidx (full Q/K), frozen heads' Q/K slots are never
    read: poisoning them with NaN leaves the output finite and unchanged."""
    K = _kernel()
    B, H, T, hd = 1, 6, 300, 64
    frozen, _, live = routing(H, {1: 1, 4: 1})
    hid = torch.arange(H, dtype=torch.int32)
    q, k, v = qkv(B, H, T, hd, seed=5, dtype=torch.bfloat16)
    patt = make_pattern(H, T, seed=9)
    y0 = K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV), hid.to(DEV))
    q2, k2 = q.clone(), k.clone()
    q2[:, [1, 4]] = float("nan")
    k2[:, [1, 4]] = float("nan")
    y1 = K.fused_mixed_attn(q2.to(DEV), k2.to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV), hid.to(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(y1).all()
    assert torch.equal(y0, y1)


def test_routing_bit_exact_vs_permutation():
    """Head-permutation equivariance: permuting heads (and their routing rows)
    permutes the output heads exactly."""
    K = _kernel()
    B, H, T, hd, S = 1, 8, 256, 64, 256
    frozen, hidx, live = routing(H, {0: 1, 3: 1, 6: 1})
    q, k, v = qkv(B, H, T, hd, seed=21, dtype=torch.bfloat16)
    patt = make_pattern(H, S, seed=4)
    y = K.fused_mixed_attn(q[:, live].to(DEV), k[:, live].to(DEV), v.to(DEV), patt.to(DEV),
                           frozen.to(DEV), hidx.to(DEV))
    perm = torch.tensor([5, 2, 7, 0, 1, 6, 4, 3])
    fz_p = frozen[perm]
    frozen_p, hidx_p, live_p = routing(H, {i: int(fz_p[i]) for i in range(H) if int(fz_p[i])})
    y_p = K.fused_mixed_attn(q[:, perm][:, live_p].to(DEV), k[:, perm][:, live_p].to(DEV),
                             v[:, perm].to(DEV), patt[perm].to(DEV), frozen_p.to(DEV), hidx_p.to(DEV))
    torch.cuda.synchronize()
    assert torch.equal(y[:, perm], y_p)


@pytest.mark.parametrize("T,S,hd,nf", [(1, 64, 64, 2), (37, 64, 64, 3), (700, 1024, 64, 3),
                                       (700, 1024, 96, 2), (513, 576, 128, 2)])
def test_frozen_pv_compact(T, S, hd, nf):
    """frozen_pv on compact frozen-head values (kernel/test_frozen_attn.py:57-87)."""
    K = _kernel()
    B, H = 2, 6
    patt = make_pattern(H, S, seed=T + S)
    fz = torch.tensor([5, 0, 3][:nf], dtype=torch.int32)
    g = torch.Generator().manual_seed(T * hd)
    v = torch.randn(B, nf, T, hd, generator=g).bfloat16()
    y = K.frozen_pv(patt.to(DEV), v.to(DEV), fz.to(DEV), T)
    torch.cuda.synchronize()
    compare(y, orc.frozen_pv(patt.numpy(), f64(v), fz.numpy(), T), what="frozen_pv")


def test_invalid_args_raise():
    K = _kernel()
    q, k, v = qkv(1, 4, 64, 80, seed=1, dtype=torch.bfloat16)
    frozen = torch.zeros(4, dtype=torch.int32, device=DEV)
    with pytest.raises(NotImplementedError):
        K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), None, frozen)
    q, k, v = qkv(1, 4, 64, 64, seed=1, dtype=torch.float64)
    with pytest.raises(NotImplementedError):
        K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), None, frozen)
    q, k, v = qkv(1, 4, 64, 64, seed=1, dtype=torch.bfloat16)
    with pytest.raises(AssertionError, match="dense-frozen heads require patt"):
        K.fused_mixed_attn(q.to(DEV), k.to(DEV), v.to(DEV), None,
                           torch.tensor([1, 0, 0, 0], dtype=torch.int32, device=DEV))


@pytest.mark.parametrize("with_scan", [False, True])
def test_decomposed_beside_live_heads_unsplit_vs_split(with_scan):
    """Decomposed heads next to live heads run one workgroup per query block
    on the side stream, beside the live-head kernel (the default); forced
    back to the key-segment split with partials and a combine on the current
    stream (decomp_unsplit=False) they give the same rows to fp32 rounding,
    both within the bound of the float64 oracle.  The live rows are
    bit-identical.  T = 3000 at B = 4 makes the split plan cut the long
    query blocks; with_scan adds a closed-form decay head, which shares the
    side stream with the decomposed heads."""
    K = _kernel()
    B, H, T, hd, S = 4, 6, 3000, 64, 3008
    dec = [1, 4]
    closed = {2: ("decay", 0.02)} if with_scan else {}
    states = {h: 2 for h in dec}
    states.update({h: 2 for h in closed})
    frozen, hidx, live = routing(H, states)
    alpha, rho, z = make_decomp(H, S, seed=77, scale=0.6)
    if closed:
        ca, cr, cz = closed_params(H, S, closed)
        for h in closed:
            alpha[h], rho[h], z[h] = ca[h], cr[h], cz[h]
    q, k, v = qkv(B, H, T, hd, seed=5, dtype=torch.bfloat16)
    cf = K.classify_closed_form(alpha, rho, z) if closed else None
    args = (q[:, live].to(DEV), k[:, live].to(DEV), v.to(DEV), None, frozen.to(DEV), hidx.to(DEV))
    kw = dict(alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV), closed_form=cf)
    y_side = K.fused_mixed_attn(*args, **kw)
    y_split = K.fused_mixed_attn(*args, decomp_unsplit=False, **kw)
    torch.cuda.synchronize()
    assert torch.equal(y_side[:, live], y_split[:, live])
    # one bf16 step of the value, or 2^-10 where a row's terms cancel to a
    # small sum (the fp32 orders differ by rounding of the terms' magnitude)
    d = (y_side[:, dec].float() - y_split[:, dec].float()).abs()
    step = (y_split[:, dec].float().abs() * 2.0 ** -7).clamp_min(2.0 ** -10)
    assert bool((d <= step).all()), f"unsplit and split differ by {d.max().item():.3e}"
    ref = orc.eager_mixed_attention(f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), hidx.numpy(),
                                    None, None, alpha=f64(alpha), rho=f64(rho), z=f64(z), sm_scale=scale_of(hd))
    compare(y_side, ref, what="decomposed beside live (unsplit)")
    compare(y_split, ref, what="decomposed after live (split)")


def test_timed_per_kind_path_matches_single_call():
    """With a KernelTimer installed, fused_mixed_attn runs each head kind
    through its own entry point (saf_flash_fwd, saf_frozen_dense_pv_fwd,
    saf_frozen_decomp_fwd, saf_frozen_scan_fwd; scan and decomposed heads on
    a second stream) and times each kernel; without one it makes the single
    saf_mixed_attn_fwd call, which forks the library's own side stream.  Both
    give the same rows (the scan's look-back order may move a last fp32 bit,
    so one bf16 step is allowed) and the timer records every kind."""
    K = _kernel()
    B, H, T, hd, S = 2, 8, 1500, 64, 1536
    dense, dec = [1, 6], [2, 5]
    closed = {3: ("decay", 0.05)}
    states = {h: 1 for h in dense}
    states.update({h: 2 for h in dec})
    states.update({h: 2 for h in closed})
    frozen, hidx, live = routing(H, states)
    patt = make_pattern(H, S, seed=5)
    alpha, rho, z = make_decomp(H, S, seed=6, scale=0.6)
    ca, cr, cz = closed_params(H, S, closed)
    for h in closed:
        alpha[h], rho[h], z[h] = ca[h], cr[h], cz[h]
    cf = K.classify_closed_form(alpha, rho, z)
    q, k, v = qkv(B, H, T, hd, seed=4, dtype=torch.bfloat16)
    args = (q[:, live].to(DEV), k[:, live].to(DEV), v.to(DEV), patt.to(DEV), frozen.to(DEV), hidx.to(DEV))
    kw = dict(alpha=alpha.to(DEV), rho=rho.to(DEV), z=z.to(DEV), closed_form=cf)
    y_one = K.fused_mixed_attn(*args, **kw)
    timer = K.KernelTimer()
    K.set_kernel_timer(timer)
    try:
        y_timed = K.fused_mixed_attn(*args, **kw)
    finally:
        K.set_kernel_timer(None)
    torch.cuda.synchronize()
    summary = timer.summary()
    assert {"flash", "dense", "decomp", "scan"} <= set(summary), summary
    d = (y_one.float() - y_timed.float()).abs()
    step = (y_one.float().abs() * 2.0 ** -7).clamp_min(2.0 ** -12)
    assert bool((d <= step).all()), f"timed and single-call paths differ by {d.max().item():.3e}"
    ref = orc.eager_mixed_attention(f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), hidx.numpy(),
                                    None, None, patt=patt.numpy(), alpha=f64(alpha), rho=f64(rho), z=f64(z),
                                    sm_scale=scale_of(hd))
    compare(y_one, ref, what="single call")
