"""CPU oracle for SAF's mixed-head causal attention prefill (numpy, float64).

TEST INFRASTRUCTURE ONLY.  This module is the checker that the HIP path is
compared against; only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and never as the thing measured or shipped.

Each function restates the reference's algorithm from its source
(waylonli/Selective-Attention-Freezing, read-only at /root/reference):

  eager_mixed_attention   kernel/test_fused_attn.py:53-63 (ref) and
                          nanogpt/model.py:824-844 (_attend_dynamic), with the
                          GQA map of qwen/kernel/fused_attn.py:254-259
  eager_rows              the same output restricted to chosen query rows
                          (row i needs only q_i, K/V[:i+1] and P[i, :i+1]),
                          for parity at the configs' full sizes
  decomp_logits           kernel/fused_attn.py:83-98
  decomposed_logz         kernel/fused_attn.py:101-116
  make_rho_band           kernel/fused_attn.py:65-80
  decomp_pattern          nanogpt/model.py:796-803 (exp(L - z))
  frozen_pv               kernel/frozen_attn.py:185-192 / test_frozen_attn.py:27-28
  logz_grads              d z / d(alpha, rho) of decomposed_logz, the autograd of
                          decomp_log_normalizers_fft (nanogpt/dynamic_freeze.py:330-361)
  pattern_grads           dalpha / drho of decomposed heads' outputs
                          (supplement/trainable_pattern_kernels.py:20-56,
                          the softmax derivative of supplement/trainable_patterns.py:7-13)
  mean/decay/window       supplement/attention.py:10-25 (causal mean),
                          nanogpt/model.py:338-353 (uniform, local_window),
                          nanogpt/test_prior_flash.py:47-59 (exp(-dist/scale))
  refresh_routing         nanogpt/model.py:846-898 (_refresh_freeze_cache)
  rope                    nanogpt/model.py:57-99
  add_layernorm           nanogpt/model.py:45-54 (LayerNorm, eps 1e-5) with the
                          residual additions of Block.forward (:1214-1240)
  add_rmsnorm             transformers' Qwen3RMSNorm (the Qwen caller's decoder
                          norms) with the same optional residual update
  linear_gelu             nanogpt/model.py:1193-1207 (MLP: c_fc without bias,
                          then nn.GELU(), the exact erf form)
  linear_swiglu           transformers' Qwen3MLP (the C4 caller's MLP, SiLU):
                          act_fn(gate_proj(x)) * up_proj(x), before down_proj
  linear_rope             nanogpt/model.py:920-944 (the gathered QKV projection)
                          followed by :57-99 (the rotation of the live q / k)

How each is pinned (tests/test_oracle.py): torch SDPA as the library special
case of the all-live case (torch.nn.functional.layer_norm likewise for
add_layernorm, transformers' Qwen3RMSNorm in float64 for add_rmsnorm,
torch.nn.functional.gelu and the normal CDF's closed values
for linear_gelu, torch.nn.functional.silu and the logistic's closed values for
linear_swiglu); brute-force pure-Python loops on tiny inputs;
closed forms (prefix sums, IIR recurrences, box filters) against the dense
patterns; invariants (rows sum to 1, T = 1 gives y = v, frozen heads ignore
Q/K, head-permutation equivariance); routing tables brute-forced over every
mask for H <= 8; golden vectors written from the reference's own CPU code
(tests/golden/).
"""
import math

import numpy as np


def _f64(x):
    return np.asarray(x, dtype=np.float64)


# ---------------------------------------------------------------------------
# patterns
# ---------------------------------------------------------------------------

def decomp_logits(alpha, rho, rows=None):
    """L[h, i, j] = alpha[h, j] + rho[h, i - j] (j <= i), -inf above."""
    alpha, rho = _f64(alpha), _f64(rho)
    H, S = alpha.shape
    r0, r1 = (0, S) if rows is None else rows
    i = np.arange(r0, r1)[:, None]
    j = np.arange(S)[None, :]
    dist = i - j
    out = alpha[:, None, :] + rho[:, np.clip(dist, 0, None)]
    out = np.where(dist[None] < 0, -np.inf, out)
    return out


def logsumexp(x, axis=-1):
    m = np.max(x, axis=axis, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    with np.errstate(divide="ignore"):
        s = np.log(np.sum(np.exp(x - m_safe), axis=axis, keepdims=True)) + m_safe
    return np.squeeze(s, axis=axis)


def decomposed_logz(alpha, rho):
    """z[h, i] = logsumexp_{j <= i}(alpha[h, j] + rho[h, i - j])."""
    H, S = np.shape(alpha)
    z = np.empty((H, S))
    step = max(1, (1 << 22) // max(H * S, 1))
    for r0 in range(0, S, step):
        r1 = min(S, r0 + step)
        z[:, r0:r1] = logsumexp(decomp_logits(alpha, rho, rows=(r0, r1)), axis=-1)
    return z


def make_rho_band(rho, band_rows=64):
    """band[h, r, u] = rho[h, r - u + S - band_rows], -inf outside [0, S)."""
    rho = _f64(rho)
    H, S = rho.shape
    r = np.arange(band_rows)[:, None]
    u = np.arange(S)[None, :]
    src = r - u + (S - band_rows)
    valid = (src >= 0) & (src < S)
    band = rho[:, np.clip(src, 0, S - 1)]
    return np.where(valid[None], band, -np.inf)


def decomp_pattern(alpha, rho, z, T):
    """(H, T, T) pattern exp(alpha[j] + rho[i-j] - z[i]) with exact zeros above
    the diagonal (what the reference materialises for its eager oracle)."""
    alpha, rho, z = _f64(alpha), _f64(rho), _f64(z)
    lg = decomp_logits(alpha[:, :T], rho[:, :T])
    with np.errstate(invalid="ignore"):
        return np.exp(lg - z[:, :T, None])


def mean_pattern(T):
    i = np.arange(T)
    return np.where(i[None, :] <= i[:, None], 1.0 / (i[:, None] + 1.0), 0.0)


def decay_pattern(T, c):
    i = np.arange(T)
    dist = i[:, None] - i[None, :]
    w = np.where(dist >= 0, np.exp(-c * np.clip(dist, 0, None)), 0.0)
    return w / w.sum(-1, keepdims=True)


def window_pattern(T, w):
    i = np.arange(T)
    dist = i[:, None] - i[None, :]
    m = (dist >= 0) & (dist < w)
    return m / np.minimum(i + 1, w)[:, None]


def closed_form_params(kind, param, S):
    """(alpha, rho) vectors of length S encoding a closed-form pattern as a
    decomposed head: mean (rho = 0), decay (rho[d] = -c d), window (0 / -inf)."""
    d = np.arange(S, dtype=np.float64)
    alpha = np.zeros(S)
    if kind == "mean":
        rho = np.zeros(S)
    elif kind == "decay":
        rho = -float(param) * d
    elif kind == "window":
        rho = np.where(d < int(param), 0.0, -np.inf)
    else:
        raise ValueError(kind)
    return alpha, rho


# closed forms evaluated directly on V (independent of the dense patterns)

def mean_apply(v):
    """y_i = (1 / (i+1)) sum_{j<=i} v_j along axis -2."""
    v = _f64(v)
    T = v.shape[-2]
    return np.cumsum(v, axis=-2) / (np.arange(T) + 1.0)[:, None]


def decay_apply(v, c):
    """IIR s_i = e^{-c} s_{i-1} + v_i, y_i = s_i / sum_{d<=i} e^{-c d}."""
    v = _f64(v)
    T = v.shape[-2]
    r = math.exp(-c)
    s = np.zeros(v.shape[:-2] + (v.shape[-1],))
    out = np.empty_like(v)
    zsum = 0.0
    for i in range(T):
        s = r * s + v[..., i, :]
        zsum = r * zsum + 1.0
        out[..., i, :] = s / zsum
    return out


def window_apply(v, w):
    """Box filter: mean of v over rows max(0, i-w+1)..i."""
    v = _f64(v)
    T = v.shape[-2]
    c = np.concatenate([np.zeros(v.shape[:-2] + (1, v.shape[-1])), np.cumsum(v, axis=-2)], axis=-2)
    i = np.arange(T)
    lo = np.maximum(i - w + 1, 0)
    return (c[..., i + 1, :] - c[..., lo, :]) / (i - lo + 1.0)[:, None]


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def causal_attention(q, k, v, scale):
    """softmax(q k^T * scale) v with a causal mask, for one head (T, HD)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    T = q.shape[0]
    s = (q @ k.T) * scale
    s = np.where(np.tril(np.ones((T, T), dtype=bool)), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ v


def eager_mixed_attention(q, k, v, frozen, hidx=None, pidx=None, kvidx=None,
                          patt=None, alpha=None, rho=None, z=None, sm_scale=None,
                          heads=None):
    """Reference eager semantics of fused_mixed_attn for every head.

    q, k: (B, U, T, HD) compact live slots (or k raw (B, HKV, T, HD) with
    kvidx); v: (B, H or HKV, T, HD); frozen: (H,) states 0/1/2.  Returns
    (B, H, T, HD) float64.  `heads` restricts the computation to a subset
    (other heads are left as NaN)."""
    v = _f64(v)
    frozen = np.asarray(frozen)
    H = frozen.shape[0]
    B, _, T, HD = v.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HD)
    out = np.full((B, H, T, HD), np.nan)
    dec_cache = {}
    for h in (range(H) if heads is None else heads):
        vh = h if kvidx is None else int(kvidx[h])
        st = int(frozen[h])
        if st == 0:
            qs = h if hidx is None else int(hidx[h])
            ks = qs if kvidx is None else int(kvidx[h])
            for b in range(B):
                out[b, h] = causal_attention(q[b, qs], k[b, ks], v[b, vh], sm_scale)
            continue
        if st == 1:
            row = h if pidx is None else int(pidx[h])
            P = _f64(patt[row, :T, :T])
        else:
            if h not in dec_cache:
                dec_cache[h] = decomp_pattern(np.asarray(alpha)[h:h + 1], np.asarray(rho)[h:h + 1],
                                              np.asarray(z)[h:h + 1], T)[0]
            P = dec_cache[h]
        for b in range(B):
            out[b, h] = P @ v[b, vh]
    return out


def sample_rows(T, n_random=128, seed=0):
    """Query rows checked at a full-size shape: the first and last rows, both
    sides of every 64-row boundary (the tile edges of every kernel here), and
    `n_random` seeded random rows distinct from those; sorted, unique."""
    rng = np.random.default_rng(seed)
    b = np.arange(64, T, 64)
    fixed = np.unique(np.clip(np.concatenate([[0, 1, T - 2, T - 1], b - 1, b]), 0, T - 1))
    rest = np.setdiff1d(np.arange(T), fixed)
    extra = rng.choice(rest, size=min(n_random, rest.size), replace=False)
    return np.unique(np.concatenate([fixed, extra]))


def eager_rows(q, k, v, frozen, rows, hidx=None, pidx=None, kvidx=None, patt_rows=None,
               alpha=None, rho=None, z=None, sm_scale=None):
    """Rows `rows` of eager_mixed_attention's output, (B, H, len(rows), HD)
    float64, without materialising any (T, T) matrix.

    Live row i: softmax(scale q_i K[:i+1]^T) V[:i+1].  Dense row i:
    patt_rows[h][n, :i+1] V[:i+1], where patt_rows[h] holds the pattern rows
    `rows` of head h's pattern (an (R, >= T) array: the caller reads only
    those rows of a large pattern).  Decomposed row i:
    exp(alpha[j] + rho[i-j] - z[i]) for j <= i, times V[:i+1].  Arrays may be
    float32/bf16-rounded; everything is computed in float64."""
    frozen = np.asarray(frozen)
    rows = np.asarray(rows)
    H = frozen.shape[0]
    B, _, T, HD = np.shape(v)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HD)
    R = rows.size
    out = np.empty((B, H, R, HD))
    jj = np.arange(T)
    causal = jj[None, :] <= rows[:, None]          # (R, T)
    for h in range(H):
        vh = h if kvidx is None else int(kvidx[h])
        st = int(frozen[h])
        if st == 0:
            qs = h if hidx is None else int(hidx[h])
            ks = qs if kvidx is None else int(kvidx[h])
            for b in range(B):
                s = (_f64(q[b, qs][rows]) @ _f64(k[b, ks]).T) * sm_scale
                s = np.where(causal, s, -np.inf)
                s = np.exp(s - s.max(-1, keepdims=True))
                out[b, h] = (s / s.sum(-1, keepdims=True)) @ _f64(v[b, vh])
            continue
        if st == 1:
            P = _f64(patt_rows[h])[:, :T]
            P = np.where(causal, P, 0.0)
        else:
            a, r, zz = (_f64(np.asarray(t)[h]) for t in (alpha, rho, z))
            dist = rows[:, None] - jj[None, :]
            lg = a[None, :T] + r[np.clip(dist, 0, T - 1)] - zz[rows][:, None]
            with np.errstate(invalid="ignore"):
                P = np.where(causal, np.exp(lg), 0.0)
        for b in range(B):
            out[b, h] = P @ _f64(v[b, vh])
    return out


def eager_mixed_attention_grads(q, k, v, frozen, dout, hidx=None, pidx=None, patt=None, alpha=None,
                                rho=None, z=None, sm_scale=None):
    """Gradients of eager_mixed_attention with respect to q, k (compact live
    slots) and v, for the upstream gradient dout (B, H, T, HD): the backward
    of /root/reference/kernel/fused_attn.py:593-648 in closed form.  Live
    heads: P = softmax(scale q k^T) (causal), dV = P^T dO,
    dS = P (dO V^T - rowsum(dO * O)), dQ = scale dS K, dK = scale dS^T Q.
    Frozen heads: dV = P^T dO, and no q/k gradient.  float64."""
    q = None if q is None else _f64(q)
    k = None if k is None else _f64(k)
    v = _f64(v)
    dout = _f64(dout)
    frozen = np.asarray(frozen)
    H = frozen.shape[0]
    B, _, T, HD = v.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(HD)
    dq = None if q is None else np.zeros_like(q)
    dk = None if k is None else np.zeros_like(k)
    dv = np.zeros_like(v)
    mask = np.tril(np.ones((T, T), dtype=bool))
    for h in range(H):
        st = int(frozen[h])
        if st == 0:
            qs = h if hidx is None else int(hidx[h])
            for b in range(B):
                s = (q[b, qs] @ k[b, qs].T) * sm_scale
                s = np.where(mask, s, -np.inf)
                P = np.exp(s - s.max(-1, keepdims=True))
                P /= P.sum(-1, keepdims=True)
                o = P @ v[b, h]
                dv[b, h] += P.T @ dout[b, h]
                dP = dout[b, h] @ v[b, h].T
                delta = (dout[b, h] * o).sum(-1, keepdims=True)
                dS = P * (dP - delta)
                dq[b, qs] += sm_scale * dS @ k[b, qs]
                dk[b, qs] += sm_scale * dS.T @ q[b, qs]
            continue
        if st == 1:
            row = h if pidx is None else int(pidx[h])
            P = _f64(patt[row, :T, :T])
        else:
            P = decomp_pattern(np.asarray(alpha)[h:h + 1], np.asarray(rho)[h:h + 1], np.asarray(z)[h:h + 1], T)[0]
        for b in range(B):
            dv[b, h] += P.T @ dout[b, h]
    return dq, dk, dv


def logz_grads(alpha, rho, gz):
    """dalpha, drho of sum_i gz[h, i] z[h, i], z = decomposed_logz(alpha, rho):
    dalpha_j = sum_{i>=j} gz_i P_ij, drho_d = sum_{i-j=d} gz_i P_ij with P the
    row softmax of alpha_j + rho_{i-j} (float64)."""
    alpha, rho, gz = _f64(alpha), _f64(rho), _f64(gz)
    H, S = alpha.shape
    P = decomp_pattern(alpha, rho, decomposed_logz(alpha, rho), S)
    P = np.nan_to_num(P, nan=0.0)
    W = gz[:, :, None] * P                       # (H, i, j)
    da = W.sum(1)
    dr = np.zeros((H, S))
    for d in range(S):
        dr[:, d] = np.trace(W, offset=-d, axis1=1, axis2=2)
    return da, dr


def pattern_grads(v, dout, frozen, alpha, rho, heads=None, out=None):
    """dalpha, drho (H, S) of sum(dout * y) over the decomposed heads (state
    2) of eager_mixed_attention, summed over the batch: with P the row
    softmax of alpha_j + rho_{i-j}, y = P V, dP = dO V^T, delta_i = dO_i . y_i,
    dS = P (dP - delta) and dalpha_j = sum_i dS_ij, drho_d = sum_{i-j=d} dS_ij
    (float64, v / dout (B, H, T, HD)).  With `out` (B, H, T, HD) delta is
    taken from it instead of the exact y, as the reference's kernel takes it
    from the saved forward output (supplement/trainable_pattern_kernels.py:44)."""
    v, dout = _f64(v), _f64(dout)
    out = None if out is None else _f64(out)
    alpha, rho = _f64(alpha), _f64(rho)
    H, S = alpha.shape
    B, _, T, _ = v.shape
    da = np.zeros((H, S))
    dr = np.zeros((H, S))
    for h in (range(H) if heads is None else heads):
        if int(np.asarray(frozen)[h]) != 2:
            continue
        a, r = alpha[h:h + 1], rho[h:h + 1]
        P = decomp_pattern(a, r, decomposed_logz(a, r), T)[0]
        for b in range(B):
            y = P @ v[b, h]
            dP = dout[b, h] @ v[b, h].T
            delta = (dout[b, h] * (y if out is None else out[b, h])).sum(-1, keepdims=True)
            dS = P * (dP - delta)
            da[h, :T] += dS.sum(0)
            for d in range(T):
                dr[h, d] += np.trace(dS, offset=-d)
    return da, dr


def frozen_pv(patt, v, fz_idx, T):
    """y[b, f] = patt[fz_idx[f], :T, :T] @ v[b, f]."""
    v = _f64(v)
    B, nf = v.shape[:2]
    out = np.empty((B, nf, T, v.shape[-1]))
    for f in range(nf):
        P = _f64(patt[int(fz_idx[f]), :T, :T])
        for b in range(B):
            out[b, f] = P @ v[b, f, :T]
    return out


# ---------------------------------------------------------------------------
# routing tables (nanogpt/model.py:846-898)
# ---------------------------------------------------------------------------

def refresh_routing(frozen, decomp=None, head_dim=1):
    """Host restatement of _refresh_freeze_cache for one attention module."""
    frozen = np.asarray(frozen, dtype=bool)
    H = frozen.shape[0]
    fz_idx = np.nonzero(frozen)[0]
    uf_idx = np.nonzero(~frozen)[0]
    ar = np.arange(head_dim)
    uf_cols = (uf_idx[:, None] * head_dim + ar).reshape(-1) if uf_idx.size else None
    fz_cols = (fz_idx[:, None] * head_dim + ar).reshape(-1) if fz_idx.size else None
    if fz_cols is None:
        cperm = None
    else:
        cperm = fz_cols if uf_cols is None else np.concatenate([uf_cols, fz_cols])
    if decomp is None:
        mask = frozen.astype(np.int32)
    else:
        dec = np.asarray(decomp, dtype=bool) & frozen
        mask = frozen.astype(np.int32) + dec.astype(np.int32)
    hidx = np.zeros(H, dtype=np.int32)
    hidx[uf_idx] = np.arange(uf_idx.size, dtype=np.int32)
    return {"fz_idx": fz_idx, "uf_idx": uf_idx, "n_frozen": int(fz_idx.size),
            "uf_cols": uf_cols, "fz_cols": fz_cols, "cperm_cols": cperm,
            "mask_i32": mask, "hidx_i32": hidx,
            "hidx_id_i32": np.arange(H, dtype=np.int32),
            "fz_idx_i32": fz_idx.astype(np.int32)}


def gqa_kvidx(n_head, n_kv_head):
    """kvidx[h] = h // (H / HKV) (qwen/nanogpt/hybrid_prior_attention.py:526-528)."""
    groups = n_head // n_kv_head
    return (np.arange(n_head) // groups).astype(np.int32)


# ---------------------------------------------------------------------------
# RoPE (nanogpt/model.py:57-99)
# ---------------------------------------------------------------------------

def rope_cache(dim, T, base=10000.0):
    inv = 1.0 / (base ** (np.arange(0, dim, 2, dtype=np.float64) / dim))
    freqs = np.outer(np.arange(T, dtype=np.float64), inv)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb), np.sin(emb)


def apply_rope(x, cos, sin):
    x = _f64(x)
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos + rot * sin


def linear_gelu(x, weight):
    """MLP up-projection and activation of the GPT block (nanogpt/model.py:
    1193-1207, bias-free c_fc then nn.GELU()): u = x w^T, gelu(u) =
    u / 2 (1 + erf(u / sqrt 2)), in float64."""
    from scipy.special import erf
    u = _f64(x) @ _f64(weight).T
    return u * 0.5 * (1.0 + erf(u / math.sqrt(2.0)))


def linear_swiglu(x, w_gate, w_up):
    """The gated MLP's front half of transformers' Qwen3MLP with SiLU (the
    Qwen caller's MLP): silu(x Wg^T) * (x Wu^T), silu(u) = u sigma(u).
    float64."""
    from scipy.special import expit
    g = _f64(x) @ _f64(w_gate).T
    return g * expit(g) * (_f64(x) @ _f64(w_up).T)


def linear_rope(x, weight, n_rope, head_dim, cos, sin, seq_len):
    """The gathered QKV projection with its rotary embedding (nanogpt/model.py:
    920-944, :57-99): u = x w^T for rows r = b T + t; the first n_rope columns
    are heads of head_dim columns, each rotated at position t = r mod T by
    apply_rope with the given (>= T, head_dim) cos / sin rows; the remaining
    columns are u itself.  float64."""
    u = _f64(x) @ _f64(weight).T
    out = u.copy()
    t = np.arange(u.shape[0]) % seq_len
    c, s = _f64(cos)[t, :head_dim], _f64(sin)[t, :head_dim]
    for h0 in range(0, n_rope, head_dim):
        out[:, h0:h0 + head_dim] = apply_rope(u[:, h0:h0 + head_dim], c, s)
    return out


def add_rmsnorm(x, delta, weight, eps=1e-6, round_fn=None):
    """Residual update and Qwen3RMSNorm (transformers modeling_qwen3): x' = x
    + delta rounded by round_fn (the activation dtype's add), then
    y = w * round_fn(x' / sqrt(mean(x'^2) + eps)) over the last axis (the
    normalised value is cast back to the activation dtype before the weight
    multiplies it).  Returns (x', y) in float64, y before its own rounding."""
    xn = _f64(x) if delta is None else _f64(x) + _f64(delta)
    if round_fn is not None and delta is not None:
        xn = round_fn(xn)
    h = xn / np.sqrt((xn ** 2).mean(-1, keepdims=True) + eps)
    if round_fn is not None:
        h = round_fn(h)
    return xn, h * _f64(weight)


def add_layernorm(x, delta, weight, bias=None, eps=1e-5, round_fn=None):
    """Residual update and LayerNorm of the GPT block (nanogpt/model.py:45-54,
    :1214-1240): x' = x + delta, rounded by round_fn to the activation dtype
    (torch's bf16/fp16 add); y = (x' - mean) / sqrt(var + eps) * w + b over
    the last axis, var the biased variance.  Returns (x', y) in float64."""
    xn = _f64(x) if delta is None else _f64(x) + _f64(delta)
    if round_fn is not None and delta is not None:
        xn = round_fn(xn)
    mean = xn.mean(-1, keepdims=True)
    var = ((xn - mean) ** 2).mean(-1, keepdims=True)
    y = (xn - mean) / np.sqrt(var + eps) * _f64(weight)
    if bias is not None:
        y = y + _f64(bias)
    return xn, y
