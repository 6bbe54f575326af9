"""Pins the CPU oracle (oracle/saf_oracle.py) before it is trusted.

Each check is chosen so that a plausible slip in the oracle (dropped term,
wrong sign or index, transposed operand) fails one of them: library special
cases (torch SDPA), brute-force loops on tiny inputs, closed forms against
dense patterns, and invariants.
"""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc


def _rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_all_live_matches_torch_sdpa():
    B, H, T, hd = 2, 3, 97, 16
    q, k, v = (_rand((B, H, T, hd), s) for s in (1, 2, 3))
    y = orc.eager_mixed_attention(q, k, v, np.zeros(H, dtype=np.int32))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), is_causal=True).numpy()
    np.testing.assert_allclose(y, ref, atol=1e-12, rtol=1e-10)


def test_attention_brute_force_loops():
    T, hd = 6, 3
    q, k, v = (_rand((T, hd), s) for s in (4, 5, 6))
    scale = 0.7
    out = np.zeros((T, hd))
    for i in range(T):
        logits = [sum(q[i, d] * k[j, d] for d in range(hd)) * scale for j in range(i + 1)]
        m = max(logits)
        w = [math.exp(x - m) for x in logits]
        s = sum(w)
        for d in range(hd):
            out[i, d] = sum(w[j] / s * v[j, d] for j in range(i + 1))
    np.testing.assert_allclose(orc.causal_attention(q, k, v, scale), out, atol=1e-12)


def test_decomp_logits_and_logz_brute_force():
    H, S = 2, 7
    a, r = _rand((H, S), 7), _rand((H, S), 8)
    L = orc.decomp_logits(a, r)
    z = orc.decomposed_logz(a, r)
    for h in range(H):
        for i in range(S):
            for j in range(S):
                want = a[h, j] + r[h, i - j] if j <= i else -np.inf
                assert L[h, i, j] == want
            zz = math.log(sum(math.exp(a[h, j] + r[h, i - j]) for j in range(i + 1)))
            assert abs(z[h, i] - zz) < 1e-12


def test_decomp_pattern_rows_sum_to_one():
    H, S, T = 3, 64, 50
    a, r = _rand((H, S), 9) * 3, _rand((H, S), 10) * 3
    P = orc.decomp_pattern(a, r, orc.decomposed_logz(a, r), T)
    np.testing.assert_allclose(P.sum(-1), 1.0, atol=1e-12)
    assert (np.triu(P, 1) == 0).all()


def test_zero_logits_are_causal_mean():
    """alpha = rho = 0 is exactly the causal-uniform prior
    (nanogpt/bench_inference_triton.py:92-97)."""
    S, T = 32, 20
    z = np.zeros((1, S))
    P = orc.decomp_pattern(z, z, orc.decomposed_logz(z, z), T)[0]
    np.testing.assert_allclose(P, orc.mean_pattern(T), atol=1e-14)


@pytest.mark.parametrize("kind,prm", [("mean", 0), ("decay", 0.003), ("decay", 0.4),
                                      ("window", 1), ("window", 5), ("window", 100)])
def test_closed_forms_as_decomposed_heads(kind, prm):
    S, T = 96, 80
    a, r = orc.closed_form_params(kind, prm, S)
    z = orc.decomposed_logz(a[None], r[None])
    P = orc.decomp_pattern(a[None], r[None], z, T)[0]
    dense = {"mean": lambda: orc.mean_pattern(T), "decay": lambda: orc.decay_pattern(T, prm),
             "window": lambda: orc.window_pattern(T, prm)}[kind]()
    np.testing.assert_allclose(P, dense, atol=1e-13)


@pytest.mark.parametrize("kind,prm", [("mean", 0), ("decay", 0.02), ("window", 7)])
def test_closed_form_recurrences_match_patterns(kind, prm):
    T, hd = 200, 5
    v = _rand((2, T, hd), 11)
    if kind == "mean":
        y, P = orc.mean_apply(v), orc.mean_pattern(T)
    elif kind == "decay":
        y, P = orc.decay_apply(v, prm), orc.decay_pattern(T, prm)
    else:
        y, P = orc.window_apply(v, prm), orc.window_pattern(T, prm)
    np.testing.assert_allclose(y, P @ v, atol=1e-11)


def test_window_matches_reference_loop_definition():
    """local_window (nanogpt/model.py:347-353) restated as loops."""
    T, W = 40, 6
    ref = np.zeros((T, T))
    for i in range(T):
        start = max(0, i - W + 1)
        ref[i, start:i + 1] = 1.0 / (i - start + 1)
    np.testing.assert_allclose(orc.window_pattern(T, W), ref, atol=0)


def test_decay_matches_normalised_exponential_prior():
    """exp(-dist/scale) row-normalised (nanogpt/test_prior_flash.py:47-59)."""
    T, scale = 50, 7.0
    i = np.arange(T)
    dist = i[:, None] - i[None, :]
    p = np.where(dist >= 0, np.exp(-np.clip(dist, 0, None) / scale), 0.0)
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(orc.decay_pattern(T, 1.0 / scale), p, atol=1e-14)


def test_rho_band_addressing():
    """band[r, u] = rho[r - u + S - 64]: every aligned (i0, j) tile access of the
    reference kernel (kernel/fused_attn.py:157, :170) reads rho[i - j], and the
    cells with j > i are -inf."""
    H, S = 1, 192
    rho = _rand((H, S), 12)
    band = orc.make_rho_band(rho)
    for i0 in range(0, S, 64):
        for r in range(64):
            i = i0 + r
            for j in range(S):
                got = band[0, r, (S - 64) - i0 + j] if 0 <= (S - 64) - i0 + j < S else None
                if got is None:
                    continue
                if j <= i:
                    assert got == rho[0, i - j]
                else:
                    assert got == -np.inf


def test_t1_gives_v_for_every_head_kind():
    B, H, hd, S = 2, 4, 8, 16
    q, k, v = _rand((B, H, 1, hd), 13), _rand((B, H, 1, hd), 14), _rand((B, H, 1, hd), 15)
    frozen = np.array([0, 1, 2, 2])
    patt = np.tril(np.abs(_rand((H, S, S), 16)))
    patt /= patt.sum(-1, keepdims=True)
    a, r = _rand((H, S), 17), _rand((H, S), 18)
    y = orc.eager_mixed_attention(q, k, v, frozen, patt=patt, alpha=a, rho=r,
                                  z=orc.decomposed_logz(a, r))
    np.testing.assert_allclose(y, v, atol=1e-12)


def test_frozen_heads_ignore_qk_and_permutation_equivariance():
    B, H, T, hd = 1, 5, 30, 4
    q, k, v = (_rand((B, H, T, hd), s) for s in (19, 20, 21))
    frozen = np.array([0, 1, 0, 1, 0])
    patt = orc.decay_pattern(T, 0.1)[None].repeat(H, 0)
    y = orc.eager_mixed_attention(q, k, v, frozen, patt=patt)
    q2, k2 = q.copy(), k.copy()
    q2[:, [1, 3]] = np.nan
    k2[:, [1, 3]] = np.nan
    np.testing.assert_array_equal(orc.eager_mixed_attention(q2, k2, v, frozen, patt=patt), y)
    perm = np.array([3, 0, 4, 1, 2])
    yp = orc.eager_mixed_attention(q[:, perm], k[:, perm], v[:, perm], frozen[perm], patt=patt[perm])
    np.testing.assert_allclose(yp, y[:, perm], atol=0)


def test_gqa_map_equals_repeated_kv():
    B, H, HKV, T, hd = 1, 6, 2, 20, 4
    q = _rand((B, H, T, hd), 22)
    k, v = _rand((B, HKV, T, hd), 23), _rand((B, HKV, T, hd), 24)
    kvidx = orc.gqa_kvidx(H, HKV)
    assert list(kvidx) == [0, 0, 0, 1, 1, 1]
    frozen = np.array([0, 1, 0, 0, 1, 0])
    patt = orc.mean_pattern(T)[None].repeat(H, 0)
    y = orc.eager_mixed_attention(q, k, v, frozen, kvidx=kvidx, patt=patt)
    kr, vr = k[:, kvidx], v[:, kvidx]
    y2 = orc.eager_mixed_attention(q, kr, vr, frozen, patt=patt)
    np.testing.assert_allclose(y, y2, atol=0)


@pytest.mark.parametrize("H", [1, 3, 8])
def test_routing_tables_brute_force(H):
    hd = 3
    for bits in itertools.product([False, True], repeat=H):
        fz = np.array(bits)
        dec = np.array([b and (h % 2 == 0) for h, b in enumerate(bits)])
        t = orc.refresh_routing(fz, dec, hd)
        live = [h for h in range(H) if not fz[h]]
        frz = [h for h in range(H) if fz[h]]
        assert list(t["uf_idx"]) == live and list(t["fz_idx"]) == frz
        for slot, h in enumerate(live):
            assert t["hidx_i32"][h] == slot
        for h in range(H):
            want = 0 if not fz[h] else (2 if dec[h] else 1)
            assert t["mask_i32"][h] == want
        if frz:
            cols = [h * hd + d for h in live + frz for d in range(hd)]
            assert list(t["cperm_cols"]) == cols
        else:
            assert t["cperm_cols"] is None


def test_rope_is_a_rotation():
    T, dim = 9, 8
    cos, sin = orc.rope_cache(dim, T)
    x = _rand((T, dim), 25)
    y = orc.apply_rope(x, cos, sin)
    half = dim // 2
    inv = 1.0 / (10000.0 ** (np.arange(0, dim, 2) / dim))
    for t in range(T):
        zc = (x[t, :half] + 1j * x[t, half:]) * np.exp(1j * t * inv)
        np.testing.assert_allclose(y[t, :half], zc.real, atol=1e-12)
        np.testing.assert_allclose(y[t, half:], zc.imag, atol=1e-12)


def test_add_layernorm_matches_torch_layer_norm():
    # the library special case: torch's LayerNorm of x + delta (float64)
    g = torch.Generator().manual_seed(7)
    x, d = torch.randn(5, 96, generator=g, dtype=torch.float64), torch.randn(5, 96, generator=g, dtype=torch.float64)
    w, b = torch.randn(96, generator=g, dtype=torch.float64), torch.randn(96, generator=g, dtype=torch.float64)
    xn, y = orc.add_layernorm(x.numpy(), d.numpy(), w.numpy(), b.numpy())
    ref = torch.nn.functional.layer_norm(x + d, (96,), w, b, 1e-5)
    assert np.allclose(xn, (x + d).numpy())
    assert np.allclose(y, ref.numpy(), atol=1e-12)
    _, y0 = orc.add_layernorm(x.numpy(), None, w.numpy(), None)
    assert np.allclose(y0, torch.nn.functional.layer_norm(x, (96,), w, None, 1e-5).numpy(), atol=1e-12)
    # a mean-free, unit-variance output before the affine map
    _, y1 = orc.add_layernorm(x.numpy(), d.numpy(), np.ones(96), None)
    assert np.allclose(y1.mean(-1), 0, atol=1e-12) and np.allclose(y1.var(-1), 1 / (1 + 1e-5 / (x + d).numpy().var(-1)))


def test_add_rmsnorm_matches_transformers_qwen3_rmsnorm():
    # the library special case: transformers' own Qwen3RMSNorm module in float64
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    g = torch.Generator().manual_seed(17)
    x, d = torch.randn(5, 96, generator=g, dtype=torch.float64), torch.randn(5, 96, generator=g, dtype=torch.float64)
    norm = Qwen3RMSNorm(96, eps=1e-6).double()
    with torch.no_grad():
        norm.weight.copy_(torch.randn(96, generator=g, dtype=torch.float64))
        ref = norm(x + d)
    xn, y = orc.add_rmsnorm(x.numpy(), d.numpy(), norm.weight.detach().numpy(), 1e-6)
    assert np.allclose(xn, (x + d).numpy()) and np.allclose(y, ref.numpy(), atol=1e-12)
    # scale invariance with eps = 0, unit mean square with unit weight
    _, y1 = orc.add_rmsnorm(x.numpy(), None, np.ones(96), 0.0)
    _, y2 = orc.add_rmsnorm(3.5 * x.numpy(), None, np.ones(96), 0.0)
    assert np.allclose(y1, y2, atol=1e-12) and np.allclose((y1 ** 2).mean(-1), 1.0, atol=1e-12)


def test_linear_gelu_matches_torch_and_the_normal_cdf():
    # the library special case: torch's exact GELU of the float64 product
    g = torch.Generator().manual_seed(11)
    x, w = torch.randn(7, 48, generator=g, dtype=torch.float64), torch.randn(40, 48, generator=g, dtype=torch.float64)
    y = orc.linear_gelu(x.numpy(), w.numpy())
    ref = torch.nn.functional.gelu(x @ w.T, approximate="none")
    assert np.allclose(y, ref.numpy(), atol=1e-12, rtol=1e-12)
    # gelu(u) = u Phi(u): identity weight rows give the closed values
    # Phi(0) = 1/2, Phi(1) = 0.841344746068543, Phi(-2) = 0.022750131948179
    u = np.array([[0.0, 1.0, -2.0, 30.0]])
    y = orc.linear_gelu(u, np.eye(4))
    assert np.allclose(y, [[0.0, 0.841344746068543, -2 * 0.022750131948179, 30.0]], atol=1e-14)
    # gelu(u) - gelu(-u) = u (the odd part); a dropped 1/2 or sqrt 2 breaks it
    v = np.linspace(-6, 6, 97)[None, :]
    assert np.allclose(orc.linear_gelu(v, np.eye(97)) - orc.linear_gelu(-v, np.eye(97)), v, atol=1e-13)


def test_linear_swiglu_matches_torch_and_closed_values():
    g = torch.Generator().manual_seed(13)
    x = torch.randn(6, 32, generator=g, dtype=torch.float64)
    wg, wu = torch.randn(24, 32, generator=g, dtype=torch.float64), torch.randn(24, 32, generator=g, dtype=torch.float64)
    y = orc.linear_swiglu(x.numpy(), wg.numpy(), wu.numpy())
    ref = torch.nn.functional.silu(x @ wg.T) * (x @ wu.T)
    assert np.allclose(y, ref.numpy(), atol=1e-12, rtol=1e-12)
    # identity gate and up rows give silu(u) * u with silu(u) = u / (1 + e^-u):
    # silu(0) = 0, silu(1) = 0.7310585786300049, silu(-1) = -0.2689414213699951
    u = np.array([[0.0, 1.0, -1.0, 40.0, -40.0]])
    want = np.array([0.0, 0.7310585786300049, -0.2689414213699951, 40.0, -40.0 * math.exp(-40.0)]) * u
    assert np.allclose(orc.linear_swiglu(u, np.eye(5), np.eye(5)), want, rtol=1e-12, atol=1e-300)
    # up rows reading a constant-1 column give silu itself, whose odd part is
    # the identity: silu(v) - silu(-v) = v (a dropped sign in the logistic breaks it)
    n = 33
    v = np.linspace(-8, 8, n)
    xv = np.concatenate([v, [1.0]])[None, :]
    xm = np.concatenate([-v, [1.0]])[None, :]
    gate = np.eye(n, n + 1)
    up = np.zeros((n, n + 1))
    up[:, n] = 1.0
    assert np.allclose(orc.linear_swiglu(xv, gate, up) - orc.linear_swiglu(xm, gate, up), v[None, :], atol=1e-13)


def test_linear_rope_special_cases_and_invariants():
    rng = np.random.default_rng(31)
    T, B, K, hd, nh = 10, 2, 16, 8, 5
    x, w = rng.standard_normal((B * T, K)), rng.standard_normal((nh * hd, K))
    cos, sin = orc.rope_cache(hd, T)
    u = x @ w.T
    y = orc.linear_rope(x, w, 3 * hd, hd, cos, sin, T)
    # columns past n_rope are the plain product; position 0 of each sequence
    # is not rotated (cos 1, sin 0)
    np.testing.assert_allclose(y[:, 3 * hd:], u[:, 3 * hd:], atol=1e-13)
    np.testing.assert_allclose(y[[0, T]], u[[0, T]], atol=1e-13)
    np.testing.assert_allclose(orc.linear_rope(x, w, 0, hd, cos, sin, T), u, atol=1e-13)
    # each (d, d + hd/2) pair turns by the angle t * inv_freq[d]: the complex
    # product (u_d + i u_{d+hd/2}) e^{i t f_d}, which also keeps its modulus
    half = hd // 2
    inv = 1.0 / (10000.0 ** (np.arange(0, hd, 2) / hd))
    for r in (3, 7, T + 5):
        t = r % T
        for h0 in (0, hd, 2 * hd):
            z = (u[r, h0:h0 + half] + 1j * u[r, h0 + half:h0 + hd]) * np.exp(1j * t * inv)
            np.testing.assert_allclose(y[r, h0:h0 + half], z.real, atol=1e-12)
            np.testing.assert_allclose(y[r, h0 + half:h0 + hd], z.imag, atol=1e-12)


def test_planted_oracle_mistake_is_caught():
    """A transposed pattern (a plausible slip) breaks the causal-mean check."""
    T = 12
    wrong = orc.mean_pattern(T).T
    v = _rand((T, 3), 26)
    assert not np.allclose(wrong @ v, orc.mean_apply(v))
    assert np.allclose(orc.mean_pattern(T) @ v, orc.mean_apply(v))


def test_backward_oracle_matches_finite_differences():
    """eager_mixed_attention_grads (the closed-form backward of live, dense and
    decomposed heads) equals central differences of the pinned forward
    eager_mixed_attention on a tiny case."""
    rng = np.random.default_rng(3)
    B, H, T, HD = 1, 4, 6, 4
    frozen = np.array([0, 1, 2, 0], dtype=np.int32)
    hidx = np.array([1, 0, 0, 0], dtype=np.int32)   # live heads 0 -> slot 1, 3 -> slot 0
    q = rng.normal(size=(B, 2, T, HD))
    k = rng.normal(size=(B, 2, T, HD))
    v = rng.normal(size=(B, H, T, HD))
    p = np.tril(rng.random((H, T, T)))
    patt = p / p.sum(-1, keepdims=True)
    alpha = rng.normal(size=(H, T)) * 0.5
    rho = rng.normal(size=(H, T)) * 0.5
    z = orc.decomposed_logz(alpha, rho)
    do = rng.normal(size=(B, H, T, HD))
    kw = dict(patt=patt, alpha=alpha, rho=rho, z=z, sm_scale=0.7)

    def loss(qq, kk, vv):
        return float((orc.eager_mixed_attention(qq, kk, vv, frozen, hidx, **kw) * do).sum())

    dq, dk, dv = orc.eager_mixed_attention_grads(q, k, v, frozen, do, hidx, **kw)
    eps = 1e-6
    for which, (x, g) in enumerate(((q, dq), (k, dk), (v, dv))):
        num = np.zeros_like(x)
        for idx in np.ndindex(x.shape):
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            a = [q, k, v]
            a[which] = xp
            fp = loss(*a)
            a[which] = xm
            num[idx] = (fp - loss(*a)) / (2 * eps)
        assert np.abs(num - g).max() < 1e-6, f"gradient {which}"


# ---------------------------------------------------------------------------
# frozen_pv (kernel/frozen_attn.py:185-192; the reference's own check is
# torch.matmul(patt[fz, :T, :T], v), kernel/test_frozen_attn.py:27-28)
# ---------------------------------------------------------------------------

def _frozen_pv_loops(patt, v, fz_idx, T):
    B, nf, _, hd = v.shape
    out = np.zeros((B, nf, T, hd))
    for b in range(B):
        for f in range(nf):
            h = int(fz_idx[f])
            for i in range(T):
                for d in range(hd):
                    out[b, f, i, d] = sum(patt[h, i, j] * v[b, f, j, d] for j in range(T))
    return out


def test_frozen_pv_brute_force_non_identity_index():
    """Non-identity fz_idx, pattern buffer S > T, V longer than T: loops,
    and torch.matmul as the reference's own definition."""
    B, nh, S, T, hd = 2, 6, 9, 7, 3
    rng = np.random.default_rng(31)
    patt = np.tril(rng.random((nh, S, S)))
    patt /= patt.sum(-1, keepdims=True)
    fz = np.array([5, 0, 3])
    v = rng.standard_normal((B, 3, T + 2, hd))
    got = orc.frozen_pv(patt, v, fz, T)
    np.testing.assert_allclose(got, _frozen_pv_loops(patt, v, fz, T), atol=1e-12)
    tm = torch.matmul(torch.from_numpy(patt)[torch.from_numpy(fz), :T, :T].unsqueeze(0),
                      torch.from_numpy(v[:, :, :T]))
    np.testing.assert_allclose(got, tm.numpy(), atol=1e-12)


def test_frozen_pv_detects_a_wrong_index():
    """A planted mistake (the identity map in place of fz_idx, or the
    transposed pattern) must not pass the brute-force check."""
    B, nh, S, T, hd = 1, 6, 8, 8, 2
    rng = np.random.default_rng(32)
    patt = np.tril(rng.random((nh, S, S)))
    patt /= patt.sum(-1, keepdims=True)
    fz = np.array([5, 0, 3])
    v = rng.standard_normal((B, 3, T, hd))
    ref = _frozen_pv_loops(patt, v, fz, T)
    wrong_index = orc.frozen_pv(patt, v, np.arange(3), T)
    wrong_transpose = orc.frozen_pv(np.swapaxes(patt, 1, 2), v, fz, T)
    assert np.abs(wrong_index - ref).max() > 1e-3
    assert np.abs(wrong_transpose - ref).max() > 1e-3


# ---------------------------------------------------------------------------
# eager_rows: sampled rows of the full eager output (parity at config sizes)
# ---------------------------------------------------------------------------

def test_sample_rows_cover_tile_edges():
    rows = orc.sample_rows(1000, n_random=16, seed=3)
    assert rows[0] == 0 and rows[-1] == 999 and (np.diff(rows) > 0).all()
    for b in range(64, 1000, 64):
        assert b - 1 in rows and b in rows
    assert orc.sample_rows(1).tolist() == [0]


@pytest.mark.parametrize("gqa", [False, True])
def test_eager_rows_match_full_eager(gqa):
    """Every head kind (live, dense with compact pidx, decomposed, closed-form
    as decomposed) and the GQA map: the sampled rows equal the full eager
    output's rows."""
    B, H, T, hd, S = 2, 8, 150, 8, 160
    rng = np.random.default_rng(40)
    frozen = np.array([0, 1, 2, 0, 2, 1, 0, 2])
    live = np.nonzero(frozen == 0)[0]
    hidx = np.zeros(H, dtype=np.int32)
    hidx[live] = np.arange(live.size)
    pidx = np.zeros(H, dtype=np.int32)
    pidx[[1, 5]] = [1, 0]
    patt = np.tril(rng.random((2, S, S)))
    patt /= patt.sum(-1, keepdims=True)
    alpha = rng.standard_normal((H, S)) * 0.8
    rho = rng.standard_normal((H, S)) * 0.8
    alpha[7], rho[7] = orc.closed_form_params("window", 17, S)
    z = orc.decomposed_logz(alpha, rho)
    kvidx = None
    q = rng.standard_normal((B, live.size, T, hd))
    if gqa:
        kvidx = (np.arange(H) // 4).astype(np.int32)
        k = rng.standard_normal((B, 2, T, hd))
        v = rng.standard_normal((B, 2, T, hd))
    else:
        k = rng.standard_normal((B, live.size, T, hd))
        v = rng.standard_normal((B, H, T, hd))
    full = orc.eager_mixed_attention(q, k, v, frozen, hidx, pidx, kvidx, patt=patt, alpha=alpha,
                                     rho=rho, z=z)
    rows = orc.sample_rows(T, n_random=20, seed=1)
    prow = {h: patt[pidx[h]][rows] for h in range(H) if frozen[h] == 1}
    got = orc.eager_rows(q, k, v, frozen, rows, hidx, pidx, kvidx, patt_rows=prow, alpha=alpha,
                         rho=rho, z=z)
    np.testing.assert_allclose(got, full[:, :, rows], atol=1e-12)


# ---------------------------------------------------------------------------
# parameter gradients of decomposed patterns
# ---------------------------------------------------------------------------

def _dense_reference(v, alpha, rho):
    """supplement/trainable_patterns.py:7-13: softmax(alpha_j + rho_{i-j})
    (causal) applied to v, torch float64 (autograd is the library special case)."""
    T = v.shape[-2]
    i = torch.arange(T)
    dist = i[:, None] - i[None, :]
    logits = alpha[:, None, :T] + rho[:, dist.clamp_min(0)]
    p = logits.masked_fill(dist < 0, float("-inf")).softmax(-1)
    return p @ v


def test_pattern_grads_match_torch_autograd():
    rng = np.random.default_rng(50)
    B, H, T, hd, S = 2, 4, 23, 5, 30
    v = rng.standard_normal((B, H, T, hd))
    dout = rng.standard_normal((B, H, T, hd))
    alpha = rng.standard_normal((H, S)) * 0.7
    rho = rng.standard_normal((H, S)) * 0.7
    rho[2, 9:] = -np.inf                       # a window-like head
    frozen = np.array([2, 0, 2, 2])
    da, dr = orc.pattern_grads(v, dout, frozen, alpha, rho)
    a = torch.tensor(alpha, requires_grad=True)
    r = torch.tensor(rho, requires_grad=True)
    y = _dense_reference(torch.from_numpy(v), a, r)
    keep = torch.tensor([1.0, 0.0, 1.0, 1.0], dtype=torch.float64)[None, :, None, None]
    (y * torch.from_numpy(dout) * keep).sum().backward()
    np.testing.assert_allclose(da, a.grad.numpy(), atol=1e-10)
    rg = np.nan_to_num(r.grad.numpy())
    np.testing.assert_allclose(np.where(np.isfinite(rho), dr, 0.0), np.where(np.isfinite(rho), rg, 0.0), atol=1e-10)
    assert (da[1] == 0).all() and (dr[1] == 0).all()
    # delta from a given output: the exact output reproduces the default; a
    # perturbation e of one row i0 shifts sum_j dalpha_j by -sum_b dO_i0 . e
    # (P's rows sum to 1) and drho by the same amount over d <= i0
    y_np = y.detach().numpy()
    da_y, dr_y = orc.pattern_grads(v, dout, frozen, alpha, rho, out=y_np)
    np.testing.assert_allclose(da_y, da, atol=1e-10)
    np.testing.assert_allclose(dr_y, dr, atol=1e-10)
    i0, e = 11, rng.standard_normal((B, hd))
    y_p = y_np.copy()
    y_p[:, 0, i0] += e
    da_p, dr_p = orc.pattern_grads(v, dout, frozen, alpha, rho, out=y_p)
    shift = -float((dout[:, 0, i0] * e).sum())
    assert abs((da_p[0] - da[0]).sum() - shift) < 1e-9
    assert abs((dr_p[0] - dr[0]).sum() - shift) < 1e-9
    np.testing.assert_allclose(da_p[2:], da[2:], atol=1e-12)


def test_logz_grads_match_torch_autograd_and_fd():
    rng = np.random.default_rng(51)
    H, S = 3, 17
    alpha = rng.standard_normal((H, S))
    rho = rng.standard_normal((H, S))
    gz = rng.standard_normal((H, S))
    da, dr = orc.logz_grads(alpha, rho, gz)
    a = torch.tensor(alpha, requires_grad=True)
    r = torch.tensor(rho, requires_grad=True)
    i = torch.arange(S)
    dist = i[:, None] - i[None, :]
    lg = (a[:, None, :] + r[:, dist.clamp_min(0)]).masked_fill(dist < 0, float("-inf"))
    (lg.logsumexp(-1) * torch.from_numpy(gz)).sum().backward()
    np.testing.assert_allclose(da, a.grad.numpy(), atol=1e-10)
    np.testing.assert_allclose(dr, r.grad.numpy(), atol=1e-10)
    # finite difference on one alpha and one rho entry
    eps = 1e-6
    f = lambda al, rh: float((orc.decomposed_logz(al, rh) * gz).sum())
    a2 = alpha.copy(); a2[1, 4] += eps
    assert abs((f(a2, rho) - f(alpha, rho)) / eps - da[1, 4]) < 1e-4
    r2 = rho.copy(); r2[2, 3] += eps
    assert abs((f(alpha, r2) - f(alpha, rho)) / eps - dr[2, 3]) < 1e-4
