// Frozen heads applied as an MFMA P.V product on gfx950.
//
//   mode 0 (state 1, dense pattern): y_i = sum_{j<=i} P[pidx(h), i, j] v_j with
//     P read from the caller's (P, S, S) buffer in fp32 / bf16 / fp16 and
//     rounded to the input dtype before the product, as in the reference's
//     dense accumulator (/root/reference/kernel/fused_attn.py:125-143) and
//     the split-path kernel (/root/reference/kernel/frozen_attn.py:51-89).
//   mode 1 (state 2, decomposed pattern): P[i, j] = exp2((alpha[j] + rho[i-j]
//     - z[i]) * log2 e) rebuilt in registers from the fp32-widened (H, S)
//     buffers, as in /root/reference/kernel/fused_attn.py:145-180; cells with
//     j > i are exactly zero.
//
// The P.V half is the same as the live-head kernel: one workgroup = 4 waves
// x 32*QT query rows; V^T tiles double-buffered in LDS.  Dense: P tiles
// (BM rows x 64 keys) are staged through LDS as well, loaded with coalesced,
// prefetched 16-byte reads and rounded to the input dtype once; workgroups
// that share a P tile (the batch siblings) are placed on the same XCD so the
// second one reads it from that XCD's L2.  Decomposed: P^T is produced
// directly in the B-operand lane layout (lane (n, g) owns query n and keys
// 8g + 0..7 of each 16-key step).
#include "saf_kernels.h"

namespace saf {

template <typename T, int HD, int QT>
__global__ __launch_bounds__(256) void frozen_decomp_kernel(const FrozenParams p) {
  constexpr int MODE = 1;
  constexpr int NW = 4, NTHR = 256;
  constexpr int BM = NW * 32 * QT;
  constexpr int NDT = HD / 32;
  constexpr int RW = BM + 64;  // rho window staged per key block
  __shared__ __align__(16) uint4 v_lds[2][VLayout<HD>::BYTES / 16];
  __shared__ float a_lds[2][MODE == 1 ? 64 : 1];
  __shared__ float r_lds[2][MODE == 1 ? RW : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int n = lane & 31, g = lane >> 5;

  const int nbh = p.B * p.n_slots;
  const int qb = p.n_qblk - 1 - (int)(blockIdx.x / nbh);
  const int r = blockIdx.x % nbh;
  const int b = r / p.n_slots, slot = r % p.n_slots;
  const int h = p.out_head[slot];
  const int ph = p.pat_head[slot];

  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;

  const int T_len = p.T;
  const int q0 = qb * BM;
  const int q0w = q0 + wave * 32 * QT;
  const int kend_wg = min(q0 + BM, T_len);
  const int nkb = (kend_wg + 63) / 64;
  const int kend_w = min(q0w + 32 * QT, T_len);
  const int nkb_w = kend_w > 0 ? (kend_w + 63) / 64 : 0;

  // per-lane row normaliser (decomposed); rows >= T get +inf -> exact zeros
  float zq[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int i = q0w + 32 * qt + n;
    zq[qt] = INFINITY;
    if (MODE == 1 && i < T_len) zq[qt] = load_as_f32(p.z, (int64_t)ph * p.z_sh + (int64_t)i * p.z_ss, p.z_dtype);
  }

  f32x16_t o[QT][NDT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = zero16();

  // decomposed: alpha[j0 + t] for t < 64 and rho[d] for d = dmin + t, t < RW,
  // dmin = q0 - j0 - 63.  Out-of-range distances are -inf (exact zero cells).
  float a_reg = 0.f, r_reg[(RW + NTHR - 1) / NTHR];
  auto stage_params = [&](int j0) {
    if (MODE != 1) return;
    if (tid < 64) {
      const int j = j0 + tid;
      a_reg = j < T_len ? load_as_f32(p.alpha, (int64_t)ph * p.a_sh + (int64_t)j * p.a_ss, p.a_dtype) : 0.f;
    }
    const int dmin = q0 - j0 - 63;
#pragma unroll
    for (int u = 0; u < (RW + NTHR - 1) / NTHR; ++u) {
      const int t = tid + u * NTHR;
      const int d = dmin + t;
      r_reg[u] = (t < RW && d >= 0 && d < T_len)
                     ? load_as_f32(p.rho, (int64_t)ph * p.r_sh + (int64_t)d * p.r_ss, p.r_dtype)
                     : -INFINITY;
    }
  };
  auto store_params = [&](int buf) {
    if (MODE != 1) return;
    if (tid < 64) a_lds[buf][tid] = a_reg;
#pragma unroll
    for (int u = 0; u < (RW + NTHR - 1) / NTHR; ++u) {
      const int t = tid + u * NTHR;
      if (t < RW) r_lds[buf][t] = r_reg[u];
    }
  };

  VStager<T, HD, NTHR> vst;
  vst.load(vbase, p.v_st, 0, T_len, tid);
  stage_params(0);
  vst.store(reinterpret_cast<uint32_t*>(v_lds[0]), tid);
  store_params(0);
  __syncthreads();

  for (int j = 0; j < nkb; ++j) {
    const int buf = j & 1;
    const bool more = j + 1 < nkb;
    if (more) {
      vst.load(vbase, p.v_st, 64 * (j + 1), T_len, tid);
      stage_params(64 * (j + 1));
    }
    if (j < nkb_w) {
      const int j0 = 64 * j;
      uint4 pb[2][2][QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int i = q0w + 32 * qt + n;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int sh = 0; sh < 2; ++sh) {
            const int jb = j0 + 32 * ks + 16 * sh + 8 * g;
            float e[8];
            const int dbase = i - jb - (q0 - j0 - 63);  // index of d = i - jb in r_lds
#pragma unroll
            for (int u = 0; u < 8; ++u) {
              const float lg = a_lds[buf][jb - j0 + u] + r_lds[buf][dbase - u];
              e[u] = fast_exp2((lg - zq[qt]) * kLog2e);
            }
            pb[ks][sh][qt] = make_uint4(Elem<T>::pack2(e[0], e[1]), Elem<T>::pack2(e[2], e[3]),
                                        Elem<T>::pack2(e[4], e[5]), Elem<T>::pack2(e[6], e[7]));
          }
      }
      pv_block<T, HD, QT>(o, pb, v_lds[buf], lane);
    }
    if (more) {
      vst.store(reinterpret_cast<uint32_t*>(v_lds[buf ^ 1]), tid);
      store_params(buf ^ 1);
    }
    __syncthreads();
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int i = q0w + 32 * qt + n;
    if (i < T_len) store_out_tile<T, HD>(obase + (int64_t)i * p.o_st, o[qt], 1.f, g);
  }
}


// LDS tile of P (BM rows x 64 keys, activation dtype): row-major, 16-byte
// chunks XOR-swizzled by the row so the 32 B-operand lanes of an MFMA (32
// rows, same chunk) and the 8 writers of a row hit distinct banks.
template <int BM> struct PLayout {
  static constexpr int BYTES = BM * 128;
  __device__ static inline int chunk(int row, int c) { return row * 8 + (c ^ (row & 7)); }
};

// Pattern element types: 8 consecutive elements -> 8 floats.
template <typename PT> struct PatVec;
template <> struct PatVec<float> {
  __device__ static inline void load8(const float* src, float (&e)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w; e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
  }
  __device__ static inline float one(const float* src) { return *src; }
};
template <typename H> struct PatVec16 {
  __device__ static inline void load8(const H* src, float (&e)[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(src);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      e[2 * m] = Elem<H>::lo(w[m]);
      e[2 * m + 1] = Elem<H>::hi(w[m]);
    }
  }
  __device__ static inline float one(const H* src) { return (float)*src; }
};
template <> struct PatVec<__bf16> : PatVec16<__bf16> {};
template <> struct PatVec<_Float16> : PatVec16<_Float16> {};

// Stages P[q0 .. q0+BM)[j0 .. j0+64) rounded to T, zero above the diagonal
// and beyond T.  Eight consecutive threads read one row's 64 keys.
template <typename T, typename PT, int BM, int NTHR> struct PStager {
  static constexpr int PER_THR = BM * 8 / NTHR;
  uint4 r[PER_THR];

  __device__ inline void load(const FrozenParams& p, const PT* pbase, int q0, int j0, int T_len, int tid) {
#pragma unroll
    for (int u = 0; u < PER_THR; ++u) {
      const int idx = tid + u * NTHR;
      const int row = idx >> 3, c = idx & 7;
      const int i = q0 + row, jc = j0 + 8 * c;
      float e[8];
      if (i >= T_len || jc > i) {
#pragma unroll
        for (int m = 0; m < 8; ++m) e[m] = 0.f;
      } else {
        const PT* prow = pbase + (int64_t)i * p.p_si;
        if (p.patt_vec && jc + 8 <= p.p_cols) {
          PatVec<PT>::load8(prow + jc, e);
        } else {
#pragma unroll
          for (int m = 0; m < 8; ++m) e[m] = jc + m <= i ? PatVec<PT>::one(prow + (int64_t)(jc + m) * p.p_sj) : 0.f;
        }
        if (jc + 7 > i) {  // diagonal chunk: keys past the query are zero
#pragma unroll
          for (int m = 0; m < 8; ++m) e[m] = jc + m <= i ? e[m] : 0.f;
        }
      }
      r[u] = make_uint4(Elem<T>::pack2(e[0], e[1]), Elem<T>::pack2(e[2], e[3]), Elem<T>::pack2(e[4], e[5]),
                        Elem<T>::pack2(e[6], e[7]));
    }
  }

  __device__ inline void store(uint4* lds, int tid) const {
#pragma unroll
    for (int u = 0; u < PER_THR; ++u) {
      const int idx = tid + u * NTHR;
      lds[PLayout<BM>::chunk(idx >> 3, idx & 7)] = r[u];
    }
  }
};

// Two resident workgroups per CU double the pattern bytes in flight; the
// loop is bound by load latency, not by its short MFMA work.
template <typename T, typename PT, int HD, int QT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void frozen_dense_kernel(const FrozenParams p) {
  constexpr int NW = 4, NTHR = 256;
  constexpr int BM = NW * 32 * QT;
  constexpr int NDT = HD / 32;
  __shared__ __align__(16) uint4 v_lds[2][VLayout<HD>::BYTES / 16];
  __shared__ __align__(16) uint4 p_lds[2][PLayout<BM>::BYTES / 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;

  // XCD-aware order: workgroup i runs on XCD i % 8; the B batch siblings of a
  // (query block, head) group get ids 8 apart (same XCD, dispatched together)
  // and groups are numbered heaviest query block first.
  const int x = blockIdx.x & 7, t8 = blockIdx.x >> 3;
  const int b = t8 % p.B, grp = 8 * (t8 / p.B) + x;
  if (grp >= p.n_qblk * p.n_slots) return;
  const int qb = p.n_qblk - 1 - grp / p.n_slots;
  const int slot = grp % p.n_slots;
  const int h = p.out_head[slot];
  const PT* pbase = reinterpret_cast<const PT*>(p.patt) + (int64_t)p.pat_head[slot] * p.p_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;

  const int T_len = p.T;
  const int q0 = qb * BM;
  const int q0w = q0 + wave * 32 * QT;
  const int nkb = (min(q0 + BM, T_len) + 63) / 64;
  const int kend_w = min(q0w + 32 * QT, T_len);
  const int nkb_w = kend_w > 0 ? (kend_w + 63) / 64 : 0;

  f32x16_t o[QT][NDT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = zero16();

  VStager<T, HD, NTHR> vst;
  PStager<T, PT, BM, NTHR> pst;
  vst.load(vbase, p.v_st, 0, T_len, tid);
  pst.load(p, pbase, q0, 0, T_len, tid);
  vst.store(reinterpret_cast<uint32_t*>(v_lds[0]), tid);
  pst.store(p_lds[0], tid);
  __syncthreads();

  for (int j = 0; j < nkb; ++j) {
    const int buf = j & 1;
    const bool more = j + 1 < nkb;
    if (more) {
      vst.load(vbase, p.v_st, 64 * (j + 1), T_len, tid);
      pst.load(p, pbase, q0, 64 * (j + 1), T_len, tid);
    }
    if (j < nkb_w) {
      uint4 pb[2][2][QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int row = 32 * QT * wave + 32 * qt + n;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int sh = 0; sh < 2; ++sh) pb[ks][sh][qt] = p_lds[buf][PLayout<BM>::chunk(row, 4 * ks + 2 * sh + g)];
      }
      pv_block<T, HD, QT>(o, pb, v_lds[buf], lane);
    }
    if (more) {
      vst.store(reinterpret_cast<uint32_t*>(v_lds[buf ^ 1]), tid);
      pst.store(p_lds[buf ^ 1], tid);
    }
    __syncthreads();
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int i = q0w + 32 * qt + n;
    if (i < T_len) store_out_tile<T, HD>(obase + (int64_t)i * p.o_st, o[qt], 1.f, g);
  }
}

template <typename T, int HD, int QT>
static hipError_t launch_frozen_t(const FrozenParams& p, int mode, hipStream_t s) {
  if (mode == 0) {
    const int64_t groups = (int64_t)p.n_qblk * p.n_slots;
    const dim3 grid((unsigned)(8 * p.B * ((groups + 7) / 8)));
    if (p.patt_dtype == kF32)
      hipLaunchKernelGGL((frozen_dense_kernel<T, float, HD, QT>), grid, dim3(256), 0, s, p);
    else if (p.patt_dtype == kBF16)
      hipLaunchKernelGGL((frozen_dense_kernel<T, __bf16, HD, QT>), grid, dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL((frozen_dense_kernel<T, _Float16, HD, QT>), grid, dim3(256), 0, s, p);
  } else {
    const dim3 grid((unsigned)((int64_t)p.n_qblk * p.B * p.n_slots));
    hipLaunchKernelGGL((frozen_decomp_kernel<T, HD, QT>), grid, dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_frozen_hd(const FrozenParams& p, int hd, int mode, hipStream_t s) {
  switch (hd) {
    case 32: return launch_frozen_t<T, 32, 2>(p, mode, s);
    case 64: return launch_frozen_t<T, 64, 2>(p, mode, s);
    case 96: return launch_frozen_t<T, 96, 1>(p, mode, s);
    case 128: return launch_frozen_t<T, 128, 1>(p, mode, s);
    default: return hipErrorInvalidValue;
  }
}

int frozen_qt(int hd) { return hd <= 64 ? 2 : 1; }

hipError_t launch_frozen_pv(const FrozenParams& p, int dtype, int hd, int mode, hipStream_t s) {
  if (dtype == kBF16) return launch_frozen_hd<__bf16>(p, hd, mode, s);
  if (dtype == kF16) return launch_frozen_hd<_Float16>(p, hd, mode, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
