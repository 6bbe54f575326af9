// float32 inputs: the reference's IEEE-dot contract (kernel/fused_attn.py:36-37,
// :128-140; tests at 2e-5 forward / 2e-4 backward, kernel/test_fused_attn.py:188-190).
//
// The MFMA kernels take bf16 / fp16 only; fp32 q/k/v run here, in fp32 FMAs
// on the vector ALUs throughout (no bf16 rounding of scores, P or
// products).  This is the precision path, not the fast one: one workgroup =
// 256 threads over a BQ x BK tile (64 x 64, or 32 x 32 at hd 256) staged in
// LDS; thread (tr, tc) = (tid / 16, tid % 16) owns rows tr * RPT + i and
// keys / columns tc + 16 c, so a row's 16 threads are 16 consecutive lanes
// and its reductions are four xor shuffles.
//
//   live heads     online softmax in base 2 (scale sm_scale log2 e), output
//                  divided by the row sum, LSE = m + log2(l) as the MFMA path
//   dense heads    P read from the (P, S, S) buffer (fp32 / bf16 / fp16)
//   decomposed     P = exp2((alpha_j + rho_{i-j} - z_i) log2 e) in fp32
//                  (closed-form heads run here through their decomposed
//                  buffers)
//   backward       delta = rowsum(out * dout); dQ per query block; dK / dV
//                  per key block (live heads); dV = P^T dO per key block
//                  (frozen heads)
#include "saf_kernels.h"

namespace saf {

namespace {

template <int HD> struct F32Tile {
  static constexpr int B = HD <= 128 ? 64 : 32;  // rows of a query or key tile
  static constexpr int RPT = B / 16;             // rows (or keys) per thread
  static constexpr int DPT = HD / 16;            // columns per thread
  static constexpr int LD = HD + 4;              // LDS row pitch (floats): float4 rows, banks spread
};

// rows r0 .. r0 + R - 1 of a (T, HD) fp32 matrix with row stride st -> dst
// (rows >= T are zero)
template <int R, int HD, int LD>
__device__ __forceinline__ void load_rows(float (*dst)[LD], const float* base, int64_t st, int r0, int T_len,
                                          int tid) {
  constexpr int V4 = HD / 4;
  for (int idx = tid; idx < R * V4; idx += 256) {
    const int r = idx / V4, c = idx % V4;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (r0 + r < T_len) v = *reinterpret_cast<const float4*>(base + (int64_t)(r0 + r) * st + 4 * c);
    *reinterpret_cast<float4*>(&dst[r][4 * c]) = v;
  }
}

// acc[i][c] = sum_d a[ra + i][d] * b[rb + 16 c][d]
template <int NI, int NC, int HD, int LD>
__device__ __forceinline__ void dots(float (&acc)[NI][NC], const float (*a)[LD], int ra, const float (*b)[LD],
                                     int rb) {
#pragma unroll
  for (int i = 0; i < NI; ++i)
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[i][c] = 0.f;
#pragma unroll 2
  for (int d = 0; d < HD; d += 4) {
    float4 av[NI], bv[NC];
#pragma unroll
    for (int i = 0; i < NI; ++i) av[i] = *reinterpret_cast<const float4*>(&a[ra + i][d]);
#pragma unroll
    for (int c = 0; c < NC; ++c) bv[c] = *reinterpret_cast<const float4*>(&b[rb + 16 * c][d]);
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        float s = acc[i][c];
        s = fmaf(av[i].x, bv[c].x, s);
        s = fmaf(av[i].y, bv[c].y, s);
        s = fmaf(av[i].z, bv[c].z, s);
        s = fmaf(av[i].w, bv[c].w, s);
        acc[i][c] = s;
      }
  }
}

__device__ __forceinline__ float group16_max(float x) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) x = fmaxf(x, __shfl_xor(x, off));
  return x;
}
__device__ __forceinline__ float group16_sum(float x) {
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) x += __shfl_xor(x, off);
  return x;
}

// frozen-head probability P[i, j] (0 outside j <= i < T)
struct FrozenP {
  int kind;  // 1 dense, 2 decomposed
  const void* patt;
  int patt_dtype;
  int64_t prow0, p_si, p_sj;  // element offset of the head's pattern, row / column strides
  const void* alpha;
  const void* rho;
  const void* z;
  int a_dtype, r_dtype, z_dtype;
  int64_t a0, a_ss, r0, r_ss, z0, z_ss;
  __device__ __forceinline__ float operator()(int i, int j, int T_len) const {
    if (j > i || i >= T_len) return 0.f;
    if (kind == 1) return load_as_f32(patt, prow0 + (int64_t)i * p_si + (int64_t)j * p_sj, patt_dtype);
    // alpha + rho - z with the rounding error of the sum carried (TwoSum):
    // where P matters z is close to alpha + rho, so (s - z) is exact and the
    // exponent keeps its low bits even for logits of scale 100+
    const float a = load_as_f32(alpha, a0 + (int64_t)j * a_ss, a_dtype);
    const float r = load_as_f32(rho, r0 + (int64_t)(i - j) * r_ss, r_dtype);
    const float s = a + r;
    const float zi = load_as_f32(z, z0 + (int64_t)i * z_ss, z_dtype);
    if (!__builtin_isfinite(s)) return expf(s - zi);  // -inf logits (masked keys, windows): exact zeros
    const float bp = s - a;
    const float e = (a - (s - bp)) + (r - bp);
    return expf((s - zi) + e);
  }
};

// ---- forward -------------------------------------------------------------

template <int HD>
__global__ __launch_bounds__(256) void f32_live_kernel(const FlashParams p) {
  using Tl = F32Tile<HD>;
  constexpr int BQ = Tl::B, BK = Tl::B, RPT = Tl::RPT, DPT = Tl::DPT, LD = Tl::LD;
  __shared__ __align__(16) float qs[BQ][LD];
  __shared__ __align__(16) float ks[BK][LD];
  __shared__ __align__(16) float vs[BK][LD];
  __shared__ float ps[BQ][BK + 1];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int nqb = (p.T + BQ - 1) / BQ;
  const int qb = nqb - 1 - (int)blockIdx.x;  // heaviest first
  const int slot = blockIdx.y, b = blockIdx.z;
  const int h = p.out_head[slot];
  const float* qbase = reinterpret_cast<const float*>(p.q) + b * p.q_sb + (int64_t)p.q_head[slot] * p.q_sh;
  const float* kbase = reinterpret_cast<const float*>(p.k) + b * p.k_sb + (int64_t)p.k_head[slot] * p.k_sh;
  const float* vbase = reinterpret_cast<const float*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh;
  float* obase = reinterpret_cast<float*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;
  const int T_len = p.T, q0 = qb * BQ;
  const int nkb = (min(q0 + BQ, T_len) + BK - 1) / BK;

  load_rows<BQ, HD, LD>(qs, qbase, p.q_st, q0, T_len, tid);
  float m[RPT], l[RPT], o[RPT][DPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int c = 0; c < DPT; ++c) o[i][c] = 0.f;
  }
  for (int jb = 0; jb < nkb; ++jb) {
    const int j0 = jb * BK;
    __syncthreads();  // the previous block's tiles are read
    load_rows<BK, HD, LD>(ks, kbase, p.k_st, j0, T_len, tid);
    load_rows<BK, HD, LD>(vs, vbase, p.v_st, j0, T_len, tid);
    __syncthreads();
    float s[RPT][RPT];
    dots<RPT, RPT, HD, LD>(s, qs, tr * RPT, ks, tc);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int row = q0 + tr * RPT + i;
      float mx = -INFINITY;
#pragma unroll
      for (int c = 0; c < RPT; ++c) {
        const int key = j0 + tc + 16 * c;
        s[i][c] = (key <= row && key < T_len) ? s[i][c] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, s[i][c]);
      }
      const float m_new = fmaxf(m[i], group16_max(mx));
      const float corr = m_new == -INFINITY ? 1.f : fast_exp2(m[i] - m_new);
      float sum = 0.f;
#pragma unroll
      for (int c = 0; c < RPT; ++c) {
        const float e = m_new == -INFINITY ? 0.f : fast_exp2(s[i][c] - m_new);
        ps[tr * RPT + i][tc + 16 * c] = e;
        sum += e;
      }
      l[i] = l[i] * corr + group16_sum(sum);
      m[i] = m_new;
#pragma unroll
      for (int c = 0; c < DPT; ++c) o[i][c] *= corr;
    }
    __syncthreads();
    for (int kk = 0; kk < BK; ++kk) {
      float vv[DPT];
#pragma unroll
      for (int c = 0; c < DPT; ++c) vv[c] = vs[kk][tc + 16 * c];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float pv = ps[tr * RPT + i][kk];
#pragma unroll
        for (int c = 0; c < DPT; ++c) o[i][c] = fmaf(pv, vv[c], o[i][c]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = q0 + tr * RPT + i;
    if (row >= T_len) continue;
    const float inv = l[i] > 0.f ? 1.f / l[i] : 1.f;
#pragma unroll
    for (int c = 0; c < DPT; ++c) obase[(int64_t)row * p.o_st + tc + 16 * c] = o[i][c] * inv;
    if (p.lse != nullptr && tc == 0)
      p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)row * p.l_st] = m[i] + __log2f(l[i] > 0.f ? l[i] : 1.f);
  }
}

template <int HD>
__global__ __launch_bounds__(256) void f32_frozen_kernel(const FrozenParams p, const int mode) {
  using Tl = F32Tile<HD>;
  constexpr int BQ = Tl::B, BK = Tl::B, RPT = Tl::RPT, DPT = Tl::DPT, LD = Tl::LD;
  __shared__ __align__(16) float vs[BK][LD];
  __shared__ float ps[BQ][BK + 1];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int nqb = (p.T + BQ - 1) / BQ;
  const int qb = nqb - 1 - (int)blockIdx.x;
  const int slot = blockIdx.y, b = blockIdx.z;
  const int h = p.out_head[slot], ph = p.pat_head[slot];
  const float* vbase = reinterpret_cast<const float*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh;
  float* obase = reinterpret_cast<float*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;
  const int T_len = p.T, q0 = qb * BQ;
  const int nkb = (min(q0 + BQ, T_len) + BK - 1) / BK;
  FrozenP P{};
  P.kind = mode == 0 ? 1 : 2;
  P.patt = p.patt; P.patt_dtype = p.patt_dtype;
  P.prow0 = (int64_t)ph * p.p_sh; P.p_si = p.p_si; P.p_sj = p.p_sj;
  P.alpha = p.alpha; P.rho = p.rho; P.z = p.z;
  P.a_dtype = p.a_dtype; P.r_dtype = p.r_dtype; P.z_dtype = p.z_dtype;
  P.a0 = (int64_t)ph * p.a_sh; P.a_ss = p.a_ss;
  P.r0 = (int64_t)ph * p.r_sh; P.r_ss = p.r_ss;
  P.z0 = (int64_t)ph * p.z_sh; P.z_ss = p.z_ss;

  float o[RPT][DPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
#pragma unroll
    for (int c = 0; c < DPT; ++c) o[i][c] = 0.f;
  for (int jb = 0; jb < nkb; ++jb) {
    const int j0 = jb * BK;
    __syncthreads();
    load_rows<BK, HD, LD>(vs, vbase, p.v_st, j0, T_len, tid);
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int c = 0; c < RPT; ++c)
        ps[tr * RPT + i][tc + 16 * c] = P(q0 + tr * RPT + i, j0 + tc + 16 * c, T_len);
    __syncthreads();
    for (int kk = 0; kk < BK; ++kk) {
      float vv[DPT];
#pragma unroll
      for (int c = 0; c < DPT; ++c) vv[c] = vs[kk][tc + 16 * c];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float pv = ps[tr * RPT + i][kk];
#pragma unroll
        for (int c = 0; c < DPT; ++c) o[i][c] = fmaf(pv, vv[c], o[i][c]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = q0 + tr * RPT + i;
    if (row >= T_len) continue;
#pragma unroll
    for (int c = 0; c < DPT; ++c) obase[(int64_t)row * p.o_st + tc + 16 * c] = o[i][c];
  }
}

// ---- backward ------------------------------------------------------------

__global__ __launch_bounds__(256) void f32_bwd_delta_kernel(const BwdParams p, const int HD) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = (int64_t)p.B * p.n_live * p.T;
  if (idx >= rows) return;
  const int row = (int)(idx % p.T);
  const int slot = (int)((idx / p.T) % p.n_live);
  const int b = (int)(idx / ((int64_t)p.T * p.n_live));
  const int h = p.out_head[slot];
  const float* o = reinterpret_cast<const float*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)row * p.o_st;
  const float* g = reinterpret_cast<const float*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh + (int64_t)row * p.do_st;
  float acc = 0.f;
  for (int d = 0; d < HD; ++d) acc = fmaf(o[d], g[d], acc);
  p.delta[idx] = acc;
}

template <int HD>
__global__ __launch_bounds__(256) void f32_bwd_dq_kernel(const BwdParams p) {
  using Tl = F32Tile<HD>;
  constexpr int BQ = Tl::B, BK = Tl::B, RPT = Tl::RPT, DPT = Tl::DPT, LD = Tl::LD;
  __shared__ __align__(16) float qs[BQ][LD];
  __shared__ __align__(16) float gs[BQ][LD];
  __shared__ __align__(16) float ks[BK][LD];
  __shared__ __align__(16) float vs[BK][LD];
  __shared__ float ds_[BQ][BK + 1];
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int nqb = (p.T + BQ - 1) / BQ;
  const int qb = nqb - 1 - (int)blockIdx.x;
  const int slot = blockIdx.y, b = blockIdx.z;
  const int h = p.out_head[slot], qs_h = p.q_head[slot];
  const float* qbase = reinterpret_cast<const float*>(p.q) + b * p.q_sb + (int64_t)qs_h * p.q_sh;
  const float* kbase = reinterpret_cast<const float*>(p.k) + b * p.k_sb + (int64_t)qs_h * p.k_sh;
  const float* vbase = reinterpret_cast<const float*>(p.v) + b * p.v_sb + (int64_t)h * p.v_sh;
  const float* gbase = reinterpret_cast<const float*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh;
  float* dqbase = reinterpret_cast<float*>(p.dq) + b * p.dq_sb + (int64_t)qs_h * p.dq_sh;
  const float* delta = p.delta + ((int64_t)b * p.n_live + slot) * p.T;
  const int T_len = p.T, q0 = qb * BQ;
  const int nkb = (min(q0 + BQ, T_len) + BK - 1) / BK;
  load_rows<BQ, HD, LD>(qs, qbase, p.q_st, q0, T_len, tid);
  load_rows<BQ, HD, LD>(gs, gbase, p.do_st, q0, T_len, tid);
  float lse[RPT], dl[RPT], acc[RPT][DPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = q0 + tr * RPT + i;
    lse[i] = row < T_len ? p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)row * p.l_st] : 0.f;
    dl[i] = row < T_len ? delta[row] : 0.f;
#pragma unroll
    for (int c = 0; c < DPT; ++c) acc[i][c] = 0.f;
  }
  for (int jb = 0; jb < nkb; ++jb) {
    const int j0 = jb * BK;
    __syncthreads();
    load_rows<BK, HD, LD>(ks, kbase, p.k_st, j0, T_len, tid);
    load_rows<BK, HD, LD>(vs, vbase, p.v_st, j0, T_len, tid);
    __syncthreads();
    float s[RPT][RPT], dp[RPT][RPT];
    dots<RPT, RPT, HD, LD>(s, qs, tr * RPT, ks, tc);
    dots<RPT, RPT, HD, LD>(dp, gs, tr * RPT, vs, tc);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int row = q0 + tr * RPT + i;
#pragma unroll
      for (int c = 0; c < RPT; ++c) {
        const int key = j0 + tc + 16 * c;
        const float pr = (key <= row && row < T_len && key < T_len) ? fast_exp2(s[i][c] * p.scale_log2 - lse[i]) : 0.f;
        ds_[tr * RPT + i][tc + 16 * c] = pr * (dp[i][c] - dl[i]);
      }
    }
    __syncthreads();
    for (int kk = 0; kk < BK; ++kk) {
      float kv[DPT];
#pragma unroll
      for (int c = 0; c < DPT; ++c) kv[c] = ks[kk][tc + 16 * c];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float d = ds_[tr * RPT + i][kk];
#pragma unroll
        for (int c = 0; c < DPT; ++c) acc[i][c] = fmaf(d, kv[c], acc[i][c]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int row = q0 + tr * RPT + i;
    if (row >= T_len) continue;
#pragma unroll
    for (int c = 0; c < DPT; ++c) dqbase[(int64_t)row * p.dq_st + tc + 16 * c] = acc[i][c] * p.sm_scale;
  }
}

// dK / dV of live heads (one workgroup per key block) and dV of frozen heads
// (FROZEN: P from the pattern, no dK)
template <int HD, bool FROZEN>
__global__ __launch_bounds__(256) void f32_bwd_kv_kernel(const BwdParams p) {
  using Tl = F32Tile<HD>;
  constexpr int BQ = Tl::B, BK = Tl::B, RPT = Tl::RPT, DPT = Tl::DPT, LD = Tl::LD;
  __shared__ __align__(16) float ks[FROZEN ? 1 : BK][LD];
  __shared__ __align__(16) float vs[FROZEN ? 1 : BK][LD];
  __shared__ __align__(16) float qs[FROZEN ? 1 : BQ][LD];
  __shared__ __align__(16) float gs[BQ][LD];
  __shared__ float pt[BK][BQ + 1];  // P^T, then dS^T, of the current query block
  const int tid = threadIdx.x, tr = tid >> 4, tc = tid & 15;
  const int nkb = (p.T + BK - 1) / BK;
  const int kb = nkb - 1 - (int)blockIdx.x;
  const int slot = blockIdx.y, b = blockIdx.z;
  const int T_len = p.T, k0 = kb * BK;
  const int nqb = (T_len + BQ - 1) / BQ;
  int h, qs_h = 0;
  FrozenP P{};
  if constexpr (FROZEN) {
    h = p.f_head[slot];
    const int ph = p.pat_head[slot];
    P.kind = p.f_kind[slot];
    P.patt = p.patt; P.patt_dtype = p.patt_dtype;
    P.prow0 = (int64_t)ph * p.p_sh; P.p_si = p.p_si; P.p_sj = p.p_sj;
    P.alpha = p.alpha; P.rho = p.rho; P.z = p.z;
    P.a_dtype = p.a_dtype; P.r_dtype = p.r_dtype; P.z_dtype = p.z_dtype;
    P.a0 = (int64_t)ph * p.a_sh; P.a_ss = p.a_ss;
    P.r0 = (int64_t)ph * p.r_sh; P.r_ss = p.r_ss;
    P.z0 = (int64_t)ph * p.z_sh; P.z_ss = p.z_ss;
  } else {
    h = p.out_head[slot];
    qs_h = p.q_head[slot];
  }
  const float* gbase = reinterpret_cast<const float*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh;
  const float* qbase = FROZEN ? nullptr : reinterpret_cast<const float*>(p.q) + b * p.q_sb + (int64_t)qs_h * p.q_sh;
  const float* delta = FROZEN ? nullptr : p.delta + ((int64_t)b * p.n_live + slot) * p.T;
  if constexpr (!FROZEN) {
    load_rows<BK, HD, LD>(ks, reinterpret_cast<const float*>(p.k) + b * p.k_sb + (int64_t)qs_h * p.k_sh, p.k_st, k0,
                          T_len, tid);
    load_rows<BK, HD, LD>(vs, reinterpret_cast<const float*>(p.v) + b * p.v_sb + (int64_t)h * p.v_sh, p.v_st, k0,
                          T_len, tid);
  }
  float dv[RPT][DPT], dk[RPT][DPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
#pragma unroll
    for (int c = 0; c < DPT; ++c) dv[i][c] = dk[i][c] = 0.f;
  for (int qb = k0 / BQ; qb < nqb; ++qb) {
    const int q0 = qb * BQ;
    __syncthreads();
    load_rows<BQ, HD, LD>(gs, gbase, p.do_st, q0, T_len, tid);
    if constexpr (!FROZEN) load_rows<BQ, HD, LD>(qs, qbase, p.q_st, q0, T_len, tid);
    __syncthreads();
    // thread (tr, tc): keys k0 + tr * RPT + i, queries q0 + tc + 16 c
    float s[RPT][RPT], dp[RPT][RPT];
    if constexpr (FROZEN) {
#pragma unroll
      for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int c = 0; c < RPT; ++c) s[i][c] = P(q0 + tc + 16 * c, k0 + tr * RPT + i, T_len);
    } else {
      dots<RPT, RPT, HD, LD>(s, ks, tr * RPT, qs, tc);
      dots<RPT, RPT, HD, LD>(dp, vs, tr * RPT, gs, tc);
#pragma unroll
      for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int c = 0; c < RPT; ++c) {
          const int key = k0 + tr * RPT + i, q = q0 + tc + 16 * c;
          const float lse = q < T_len ? p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)q * p.l_st] : 0.f;
          s[i][c] = (key <= q && q < T_len && key < T_len) ? fast_exp2(s[i][c] * p.scale_log2 - lse) : 0.f;
        }
    }
#pragma unroll
    for (int i = 0; i < RPT; ++i)
#pragma unroll
      for (int c = 0; c < RPT; ++c) pt[tr * RPT + i][tc + 16 * c] = s[i][c];
    __syncthreads();
    // dV[key] += sum_q P[q, key] dO[q]
    for (int qq = 0; qq < BQ; ++qq) {
      float gv[DPT];
#pragma unroll
      for (int c = 0; c < DPT; ++c) gv[c] = gs[qq][tc + 16 * c];
#pragma unroll
      for (int i = 0; i < RPT; ++i) {
        const float pv = pt[tr * RPT + i][qq];
#pragma unroll
        for (int c = 0; c < DPT; ++c) dv[i][c] = fmaf(pv, gv[c], dv[i][c]);
      }
    }
    if constexpr (!FROZEN) {
      __syncthreads();
#pragma unroll
      for (int i = 0; i < RPT; ++i)
#pragma unroll
        for (int c = 0; c < RPT; ++c) {
          const int q = q0 + tc + 16 * c;
          pt[tr * RPT + i][tc + 16 * c] = s[i][c] * (dp[i][c] - (q < T_len ? delta[q] : 0.f));
        }
      __syncthreads();
      // dK[key] += sum_q dS[q, key] Q[q]
      for (int qq = 0; qq < BQ; ++qq) {
        float qv[DPT];
#pragma unroll
        for (int c = 0; c < DPT; ++c) qv[c] = qs[qq][tc + 16 * c];
#pragma unroll
        for (int i = 0; i < RPT; ++i) {
          const float d = pt[tr * RPT + i][qq];
#pragma unroll
          for (int c = 0; c < DPT; ++c) dk[i][c] = fmaf(d, qv[c], dk[i][c]);
        }
      }
    }
  }
  float* dvbase = reinterpret_cast<float*>(p.dv) + b * p.dv_sb + (int64_t)h * p.dv_sh;
  float* dkbase = FROZEN ? nullptr : reinterpret_cast<float*>(p.dk) + b * p.dk_sb + (int64_t)qs_h * p.dk_sh;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int key = k0 + tr * RPT + i;
    if (key >= T_len) continue;
#pragma unroll
    for (int c = 0; c < DPT; ++c) {
      dvbase[(int64_t)key * p.dv_st + tc + 16 * c] = dv[i][c];
      if constexpr (!FROZEN) dkbase[(int64_t)key * p.dk_st + tc + 16 * c] = dk[i][c] * p.sm_scale;
    }
  }
}

template <int HD>
hipError_t f32_fwd_hd(const FlashParams* fp, const FrozenParams* zp, int mode, hipStream_t s) {
  constexpr int B = F32Tile<HD>::B;
  if (fp != nullptr) {
    const dim3 grid((unsigned)((fp->T + B - 1) / B), (unsigned)fp->n_slots, (unsigned)fp->B);
    hipLaunchKernelGGL((f32_live_kernel<HD>), grid, dim3(256), 0, s, *fp);
  } else {
    const dim3 grid((unsigned)((zp->T + B - 1) / B), (unsigned)zp->n_slots, (unsigned)zp->B);
    hipLaunchKernelGGL((f32_frozen_kernel<HD>), grid, dim3(256), 0, s, *zp, mode);
  }
  return hipGetLastError();
}

template <int HD>
hipError_t f32_bwd_hd(const BwdParams& p, int which, hipStream_t s) {
  constexpr int B = F32Tile<HD>::B;
  const unsigned nb = (unsigned)((p.T + B - 1) / B);
  switch (which) {
    case 0: {
      const int64_t rows = (int64_t)p.B * p.n_live * p.T;
      hipLaunchKernelGGL(f32_bwd_delta_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, p, HD);
      break;
    }
    case 1:
      hipLaunchKernelGGL((f32_bwd_dq_kernel<HD>), dim3(nb, (unsigned)p.n_live, (unsigned)p.B), dim3(256), 0, s, p);
      break;
    case 2:
      hipLaunchKernelGGL((f32_bwd_kv_kernel<HD, false>), dim3(nb, (unsigned)p.n_live, (unsigned)p.B), dim3(256), 0,
                         s, p);
      break;
    default:
      hipLaunchKernelGGL((f32_bwd_kv_kernel<HD, true>), dim3(nb, (unsigned)p.n_frozen, (unsigned)p.B), dim3(256), 0,
                         s, p);
      break;
  }
  return hipGetLastError();
}

template <typename F>
hipError_t by_hd(int hd, F&& f) {
  switch (hd) {
    case 32: return f(std::integral_constant<int, 32>());
    case 64: return f(std::integral_constant<int, 64>());
    case 96: return f(std::integral_constant<int, 96>());
    case 128: return f(std::integral_constant<int, 128>());
    case 256: return f(std::integral_constant<int, 256>());
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_f32_live(const FlashParams& p, int hd, hipStream_t s) {
  if (p.n_slots == 0 || p.T == 0 || p.B == 0) return hipSuccess;
  return by_hd(hd, [&](auto c) { return f32_fwd_hd<decltype(c)::value>(&p, nullptr, 0, s); });
}

hipError_t launch_f32_frozen(const FrozenParams& p, int hd, int mode, hipStream_t s) {
  if (p.n_slots == 0 || p.T == 0 || p.B == 0) return hipSuccess;
  return by_hd(hd, [&](auto c) { return f32_fwd_hd<decltype(c)::value>(nullptr, &p, mode, s); });
}

hipError_t launch_f32_bwd(const BwdParams& p, int hd, int which, hipStream_t s) {
  if (p.T == 0 || p.B == 0 || (which < 3 ? p.n_live == 0 : p.n_frozen == 0)) return hipSuccess;
  return by_hd(hd, [&](auto c) { return f32_bwd_hd<decltype(c)::value>(p, which, s); });
}

}  // namespace saf
