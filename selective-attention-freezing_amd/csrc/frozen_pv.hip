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
// x 32*QT query rows; V^T tiles double-buffered in LDS; P^T is produced
// directly in the B-operand lane layout (lane (n, g) owns query n and keys
// 8g + 0..7 of each 16-key step), so no LDS pass is needed for P.
#include "saf_kernels.h"

namespace saf {

// Eight pattern values P[row i][cols jb..jb+7] as fp32, zero where j > i.
__device__ inline void dense_p8(const FrozenParams& p, const char* prow, int i, int jb, float (&e)[8]) {
  if (jb > i) {
#pragma unroll
    for (int u = 0; u < 8; ++u) e[u] = 0.f;
    return;
  }
  if (p.patt_vec && jb + 7 <= i) {
    if (p.patt_dtype == kF32) {
      const float4 a = *reinterpret_cast<const float4*>(prow + (int64_t)jb * 4);
      const float4 b = *reinterpret_cast<const float4*>(prow + (int64_t)jb * 4 + 16);
      e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w;
      e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
    } else {
      const uint4 a = *reinterpret_cast<const uint4*>(prow + (int64_t)jb * 2);
      const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (p.patt_dtype == kBF16) {
          e[2 * m] = Elem<__bf16>::lo(w[m]);
          e[2 * m + 1] = Elem<__bf16>::hi(w[m]);
        } else {
          e[2 * m] = Elem<_Float16>::lo(w[m]);
          e[2 * m + 1] = Elem<_Float16>::hi(w[m]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int j = jb + u;
    e[u] = j <= i ? load_as_f32(prow, (int64_t)j * p.p_sj, p.patt_dtype) : 0.f;
  }
}

template <typename T, int HD, int QT, int MODE>
__global__ __launch_bounds__(256) void frozen_pv_kernel(const FrozenParams p) {
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

  const char* pbase = MODE == 0 ? reinterpret_cast<const char*>(p.patt) +
                                      (int64_t)ph * p.p_sh * (p.patt_dtype == kF32 ? 4 : 2)
                                : nullptr;
  const int esz = p.patt_dtype == kF32 ? 4 : 2;

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
        const char* prow = MODE == 0 ? pbase + (int64_t)min(i, T_len - 1) * p.p_si * esz : nullptr;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int sh = 0; sh < 2; ++sh) {
            const int jb = j0 + 32 * ks + 16 * sh + 8 * g;
            float e[8];
            if (MODE == 0) {
              if (i < T_len) {
                dense_p8(p, prow, i, jb, e);
              } else {
#pragma unroll
                for (int u = 0; u < 8; ++u) e[u] = 0.f;
              }
            } else {
              const int dbase = i - jb - (q0 - j0 - 63);  // index of d = i - jb in r_lds
#pragma unroll
              for (int u = 0; u < 8; ++u) {
                const float lg = a_lds[buf][jb - j0 + u] + r_lds[buf][dbase - u];
                e[u] = fast_exp2((lg - zq[qt]) * kLog2e);
              }
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

template <typename T, int HD, int QT>
static hipError_t launch_frozen_t(const FrozenParams& p, int mode, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.n_qblk * p.B * p.n_slots));
  if (mode == 0)
    hipLaunchKernelGGL((frozen_pv_kernel<T, HD, QT, 0>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((frozen_pv_kernel<T, HD, QT, 1>), grid, dim3(256), 0, s, p);
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
