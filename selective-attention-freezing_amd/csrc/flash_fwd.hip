// Live-head causal flash attention forward (state 0 heads) for gfx950.
//
// Semantics follow the reference's live-head accumulator
// (/root/reference/kernel/fused_attn.py:182-226, GQA variant
// /root/reference/qwen/kernel/fused_attn.py:183-231): base-2 online softmax
// with qk_scale = sm_scale * log2(e), fp32 running max / sum / accumulator,
// P rounded to the input dtype before the P.V product, output divided by the
// row sum, and LSE = m + log2(l) in base-2 units.  Two deliberate changes of
// bookkeeping, both exact up to rounding: the running max is only moved when
// a block exceeds it by more than kSlack (lazy rescale), and the row sum adds
// the rounded P values (v_dot2 on packed pairs), i.e. exactly the weights
// that multiply V.
//
// Work decomposition: one workgroup = 4 waves = (4 * 32 * QT) query rows of
// one (batch, live head); each wave owns 32*QT queries and walks 64-key
// blocks up to its own causal limit.  K and V^T tiles are double-buffered in
// LDS; the next tile's global loads are issued before the current tile's
// MFMAs.  Workgroups are ordered heaviest query block first.
#include <type_traits>

#include "saf_kernels.h"

namespace saf {

// Slack of the lazy rescale (base-2 units): P values stay below 2^8.
constexpr float kSlack = 8.f;

// Two waves per SIMD (one from each of two resident workgroups) lets one
// wave's softmax VALU work overlap the other's MFMAs; the register budget
// (256 per lane) fits every variant except hd >= 96 with two query tiles.
template <int HD, int QT>
constexpr int flash_waves_per_eu() { return (HD <= 64 || QT == 1) ? 2 : 1; }

template <typename T, int HD, int QT>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(flash_waves_per_eu<HD, QT>(), flash_waves_per_eu<HD, QT>())))
void flash_fwd_kernel(const FlashParams p) {
  constexpr int NW = 4, NTHR = 256;
  constexpr int BM = NW * 32 * QT;
  constexpr int NDT = HD / 32;   // 32-wide d tiles of O^T
  constexpr int NKT = HD / 16;   // 16-deep k steps of Q.K
  __shared__ __align__(16) uint4 k_lds[2][KLayout<HD>::BYTES / 16];
  __shared__ __align__(16) uint4 v_lds[2][VLayout<HD>::BYTES / 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int n = lane & 31, g = lane >> 5;

  // work item: query block (and key segment) of one (batch, live slot);
  // items are ordered heaviest first, (batch, live slot) fastest
  const int nbh = p.B * p.n_slots;
  const int r = blockIdx.x % nbh;
  const int b = r / p.n_slots, slot = r % p.n_slots;
  const int h = p.out_head[slot];
  int qb, seg = 0;
  if (p.n_items) {
    const int it = p.items[blockIdx.x / nbh];
    qb = it >> 8;
    seg = it & 255;
  } else {
    qb = p.n_qblk - 1 - (int)(blockIdx.x / nbh);
  }
  const T* qbase = reinterpret_cast<const T*>(p.q) + b * p.q_sb + (int64_t)p.q_head[slot] * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.k_sb + (int64_t)p.k_head[slot] * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;

  const int T_len = p.T;
  const int q0 = qb * BM;
  const int q0w = q0 + wave * 32 * QT;
  const int nkb_qb = (min(q0 + BM, T_len) + 63) / 64;  // key blocks of the query block
  const int kb0 = p.n_items ? seg * p.seg_len : 0;     // this item's key-block range
  const int nkb = p.n_items ? min(kb0 + p.seg_len, nkb_qb) : nkb_qb;
  const bool split = p.n_items && p.part_base[qb] >= 0;
  const int kend_w = min(q0w + 32 * QT, T_len);
  const int nkb_w = kend_w > 0 ? (kend_w + 63) / 64 : 0;

  // Q as the B operand: lane (n, g), step t -> Q[q][16t + 8g .. +7]
  uint4 qf[QT][NKT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = q0w + 32 * qt + n;
#pragma unroll
    for (int t = 0; t < NKT; ++t)
      qf[qt][t] = q < T_len ? *reinterpret_cast<const uint4*>(qbase + (int64_t)q * p.q_st + 16 * t + 8 * g)
                            : make_uint4(0, 0, 0, 0);
  }

  f32x16_t o[QT][NDT];
  float m_run[QT], l_run[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m_run[qt] = -INFINITY;
    l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = zero16();
  }
  const float c = p.scale_log2;

  KStager<T, HD, NTHR> kst;
  VStager<T, HD, NTHR> vst;
  kst.load(kbase, p.k_st, 64 * kb0, T_len, tid);
  vst.load(vbase, p.v_st, 64 * kb0, T_len, tid);
  kst.store(k_lds[0], tid);
  vst.store(reinterpret_cast<uint32_t*>(v_lds[0]), tid);
  __syncthreads();

  auto block = [&](const int j, auto masked) {
    const int buf = (j - kb0) & 1;
    const bool more = j + 1 < nkb;
    if (more) {
      kst.load(kbase, p.k_st, 64 * (j + 1), T_len, tid);
      vst.load(vbase, p.v_st, 64 * (j + 1), T_len, tid);
    }
    if (j < nkb_w) {
      const uint4* kt = k_lds[buf];
      const uint4* vt = v_lds[buf];
      // two 32-key sub-blocks: S^T, softmax and P.V per sub-block keeps the
      // live S / P registers at 16 + 8 per query tile
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int j0 = 64 * j + 32 * ks;
        f32x16_t sacc[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) sacc[qt] = zero16();
        const int key = 32 * ks + kperm(n);
        // all A operands of the sub-block are read from LDS up front, so only
        // the first MFMA waits for LDS latency
        uint4 ka[NKT];
#pragma unroll
        for (int t = 0; t < NKT; ++t) ka[t] = kt[KLayout<HD>::chunk(key, 2 * t + g)];
        // MFMA phases run at raised wave priority so that, of the two waves
        // sharing a SIMD, the one with matrix work ready issues it first and
        // the other fills the VALU with its softmax
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int t = 0; t < NKT; ++t)
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) sacc[qt] = Elem<T>::mfma(ka[t], qf[qt][t], sacc[qt]);
        __builtin_amdgcn_s_setprio(0);
        // V^T operands of this sub-block arrive while the softmax runs
        uint4 va[2][NDT];
#pragma unroll
        for (int sh = 0; sh < 2; ++sh)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) va[sh][dt] = vt[VLayout<HD>::chunk(32 * dt + n, 4 * ks + 2 * sh + g)];
        if (decltype(masked)::value && j0 + 31 > q0w) {  // keys past a query of this wave
#pragma unroll
          for (int qt = 0; qt < QT; ++qt) {
            const int q = q0w + 32 * qt + n;
#pragma unroll
            for (int i = 0; i < 16; ++i)
              if (j0 + acc_key(i, g) > q) sacc[qt][i] = -INFINITY;
          }
        }
        uint4 pb[2][QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          float mx = sacc[qt][0];
#pragma unroll
          for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sacc[qt][i]);
          mx = half_swap_max(mx);
          // Lazy rescaling: a query's reference max only moves when the block
          // max exceeds it by more than kSlack (base-2 units), so P stays
          // <= 2^kSlack and most blocks skip the O rescale.  Exact: O and l
          // always share the same reference max.
          const float mb = mx * c;
          const bool up = mb > m_run[qt] + kSlack;
          if (__builtin_amdgcn_ballot_w64(up)) {
            const float m_new = up ? mb : m_run[qt];
            const float alpha = up ? fast_exp2(m_run[qt] - m_new) : 1.f;
            m_run[qt] = m_new;
            l_run[qt] *= alpha;
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
              for (int i = 0; i < 16; ++i) o[qt][dt][i] *= alpha;
          }
          const float mneg = -m_run[qt];
          float psum = l_run[qt];
#pragma unroll
          for (int sh = 0; sh < 2; ++sh) {
            uint32_t w[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float e0 = fast_exp2(fmaf(sacc[qt][8 * sh + 2 * u], c, mneg));
              const float e1 = fast_exp2(fmaf(sacc[qt][8 * sh + 2 * u + 1], c, mneg));
              w[u] = Elem<T>::pack2(e0, e1);
              psum = Elem<T>::sum2(w[u], psum);
            }
            pb[sh][qt] = make_uint4(w[0], w[1], w[2], w[3]);
          }
          l_run[qt] = psum;
        }
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int sh = 0; sh < 2; ++sh)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) o[qt][dt] = Elem<T>::mfma(va[sh][dt], pb[sh][qt], o[qt][dt]);
        __builtin_amdgcn_s_setprio(0);
      }
    }
    if (more) {
      kst.store(k_lds[buf ^ 1], tid);
      vst.store(reinterpret_cast<uint32_t*>(v_lds[buf ^ 1]), tid);
    }
    __syncthreads();
  };
  // blocks wholly below the workgroup's first query need no causal mask; the
  // masked variant runs only for the last BM/64 blocks of a query block
  const int jd = min(nkb, max(kb0, q0 / 64));
  for (int j = kb0; j < jd; ++j) block(j, std::false_type());
  for (int j = jd; j < nkb; ++j) block(j, std::true_type());

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = q0w + 32 * qt + n;
    const float l_tot = half_swap_sum(l_run[qt]);
    if (split) {
      // unnormalised partial of this key segment, merged by flash_combine_kernel
      const int64_t pidx = (int64_t)r * p.n_part_per_head + p.part_base[qb] + seg;
      const int rl = q - q0;
      float* po = p.part_o + (pidx * BM + rl) * HD;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(po + 32 * dt + 8 * r4 + 4 * g) =
              make_float4(o[qt][dt][4 * r4], o[qt][dt][4 * r4 + 1], o[qt][dt][4 * r4 + 2], o[qt][dt][4 * r4 + 3]);
      if (g == 0) {
        p.part_ml[(pidx * 2) * BM + rl] = m_run[qt];
        p.part_ml[(pidx * 2 + 1) * BM + rl] = l_tot;
      }
      continue;
    }
    const float l_safe = l_tot == 0.f ? 1.f : l_tot;
    if (q < T_len) {
      store_out_tile<T, HD>(obase + (int64_t)q * p.o_st, o[qt], 1.f / l_safe, g);
      if (p.lse != nullptr && g == 0) {
        const float m_store = m_run[qt] == -INFINITY ? 0.f : m_run[qt];
        p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)q * p.l_st] = m_store + __log2f(l_safe);
      }
    }
  }
}

// Merge the key-segment partials of split query blocks (one workgroup per
// (batch, slot, split query block); HD/4 threads x 4 columns per row): the
// flash partials by their (m, l) rescaling, dense P.V partials (part_ml null)
// by a plain sum.
template <typename T, int HD>
__global__ __launch_bounds__(256) void flash_combine_kernel(const CombineParams p) {
  const int tid = threadIdx.x;
  const int nbh = p.B * p.n_slots;
  const int bh = blockIdx.x % nbh;
  const int qb = p.split_qb[blockIdx.x / nbh];
  const int b = bh / p.n_slots, slot = bh % p.n_slots;
  const int h = p.out_head[slot];
  const int BM = p.BM;
  const int q0 = qb * BM;
  const int nkb_qb = (min(q0 + BM, p.T) + 63) / 64;
  const int nseg = (nkb_qb + p.seg_len - 1) / p.seg_len;
  const int64_t pbase = (int64_t)bh * p.n_part_per_head + p.part_base[qb];
  constexpr int CPR = HD / 4;          // float4 columns per row
  constexpr int RPP = 256 / CPR;       // rows per pass
  const int c4 = tid % CPR;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;
  if (tid >= RPP * CPR) return;
  for (int rl = tid / CPR; rl < BM; rl += RPP) {
    const int q = q0 + rl;
    if (q >= p.T) break;
    if (p.part_ml == nullptr) {  // dense P.V partials: a plain sum
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int s = 0; s < nseg; ++s) {
        const float4 v = *reinterpret_cast<const float4*>(p.part_o + ((pbase + s) * BM + rl) * HD + 4 * c4);
        acc.x += v.x;
        acc.y += v.y;
        acc.z += v.z;
        acc.w += v.w;
      }
      uint2 wv;
      wv.x = Elem<T>::pack2(acc.x, acc.y);
      wv.y = Elem<T>::pack2(acc.z, acc.w);
      *reinterpret_cast<uint2*>(obase + (int64_t)q * p.o_st + 4 * c4) = wv;
      continue;
    }
    float mmax = -INFINITY;
    for (int s = 0; s < nseg; ++s) mmax = fmaxf(mmax, p.part_ml[((pbase + s) * 2) * BM + rl]);
    const float mref = mmax == -INFINITY ? 0.f : mmax;
    float l = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int s = 0; s < nseg; ++s) {
      const float w = fast_exp2(p.part_ml[((pbase + s) * 2) * BM + rl] - mref);
      l = fmaf(w, p.part_ml[((pbase + s) * 2 + 1) * BM + rl], l);
      const float4 v = *reinterpret_cast<const float4*>(p.part_o + ((pbase + s) * BM + rl) * HD + 4 * c4);
      acc.x = fmaf(w, v.x, acc.x);
      acc.y = fmaf(w, v.y, acc.y);
      acc.z = fmaf(w, v.z, acc.z);
      acc.w = fmaf(w, v.w, acc.w);
    }
    const float inv = 1.f / (l == 0.f ? 1.f : l);
    uint2 wv;
    wv.x = Elem<T>::pack2(acc.x * inv, acc.y * inv);
    wv.y = Elem<T>::pack2(acc.z * inv, acc.w * inv);
    *reinterpret_cast<uint2*>(obase + (int64_t)q * p.o_st + 4 * c4) = wv;
    if (p.lse != nullptr && c4 == 0)
      p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)q * p.l_st] = mref + __log2f(l == 0.f ? 1.f : l);
  }
}

template <typename T, int HD, int QT>
static hipError_t launch_flash_t(const FlashParams& p, hipStream_t s) {
  const int64_t items = p.n_items ? p.n_items : p.n_qblk;
  const dim3 grid((unsigned)(items * p.B * p.n_slots));
  hipLaunchKernelGGL((flash_fwd_kernel<T, HD, QT>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_flash_hd(const FlashParams& p, int hd, int qt, hipStream_t s) {
  switch (hd * 4 + qt) {
    case 32 * 4 + 1: return launch_flash_t<T, 32, 1>(p, s);
    case 32 * 4 + 2: return launch_flash_t<T, 32, 2>(p, s);
    case 64 * 4 + 1: return launch_flash_t<T, 64, 1>(p, s);
    case 64 * 4 + 2: return launch_flash_t<T, 64, 2>(p, s);
    case 96 * 4 + 1: return launch_flash_t<T, 96, 1>(p, s);
    case 96 * 4 + 2: return launch_flash_t<T, 96, 2>(p, s);
    case 128 * 4 + 1: return launch_flash_t<T, 128, 1>(p, s);
    case 128 * 4 + 2: return launch_flash_t<T, 128, 2>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_flash(const FlashParams& p, int dtype, int hd, int qt, hipStream_t s) {
  if (dtype == kBF16) return launch_flash_hd<__bf16>(p, hd, qt, s);
  if (dtype == kF16) return launch_flash_hd<_Float16>(p, hd, qt, s);
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t launch_combine_t(const CombineParams& p, int hd, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.n_split * p.B * p.n_slots));
  switch (hd) {
    case 32: hipLaunchKernelGGL((flash_combine_kernel<T, 32>), grid, dim3(256), 0, s, p); break;
    case 64: hipLaunchKernelGGL((flash_combine_kernel<T, 64>), grid, dim3(256), 0, s, p); break;
    case 96: hipLaunchKernelGGL((flash_combine_kernel<T, 96>), grid, dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL((flash_combine_kernel<T, 128>), grid, dim3(256), 0, s, p); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_flash_combine(const CombineParams& p, int dtype, int hd, hipStream_t s) {
  if (dtype == kBF16) return launch_combine_t<__bf16>(p, hd, s);
  if (dtype == kF16) return launch_combine_t<_Float16>(p, hd, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
