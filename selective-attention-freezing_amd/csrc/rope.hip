// Rotary position embedding of the live-head Q and K, in place (gfx950).
//
// Llama half rotation (/root/reference/nanogpt/model.py:57-99, applied to the
// compact live-head q/k on the fused path at :1007-1008):
//   x[d] <- x[d] cos[t][d] - x[d + hd/2] sin[t][d]      d <  hd/2
//   x[d] <- x[d] cos[t][d] + x[d - hd/2] sin[t][d]      d >= hd/2
// computed in fp32 from the caller's cos/sin cache (fp32 or bf16) and rounded
// once to the activation dtype.  One pass over the projection output replaces
// the reference's chain of elementwise ops (mul, neg, cat, mul, add per
// tensor).  A thread owns one chunk pair: 8 columns of the first half and the
// matching 8 columns of the second half of one row, loaded as 16-byte words.
// The same kernel optionally applies the Qwen3 per-head q/k RMSNorm first.
#include "saf_kernels.h"

namespace saf {

// Eight consecutive elements of a cos/sin cache row or a norm weight, as fp32.
template <typename H>
__device__ inline void load8_16(const void* src, float (&e)[8]) {
  const uint4 w = *reinterpret_cast<const uint4*>(src);
  const uint32_t w4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    e[2 * m] = Elem<H>::lo(w4[m]);
    e[2 * m + 1] = Elem<H>::hi(w4[m]);
  }
}

__device__ inline void load8(const void* base, int dtype, int64_t off, float (&e)[8]) {
  if (dtype == kF32) {
    const float* f = reinterpret_cast<const float*>(base) + off;
    const float4 a = *reinterpret_cast<const float4*>(f), b = *reinterpret_cast<const float4*>(f + 4);
    e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w; e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
  } else if (dtype == kBF16) {
    load8_16<__bf16>(reinterpret_cast<const uint16_t*>(base) + off, e);
  } else {
    load8_16<_Float16>(reinterpret_cast<const uint16_t*>(base) + off, e);
  }
}

template <typename T>
__device__ inline float round_to(float x) { return (float)static_cast<T>(x); }

// Lanes per row: the row's chunk pairs rounded up to a power of two, so the
// lanes of one row are an aligned group inside a wavefront (hd = 96 leaves
// two of its eight lanes idle).
inline int rope_lanes(int hd) {
  int l = 1;
  while (l < hd / 16) l <<= 1;
  return l;
}

// With NORM, each row is first RMS-normalised over the head dimension as
// Qwen3RMSNorm does (transformers modeling_qwen3, used as q_norm / k_norm at
// /root/reference/qwen/nanogpt/hybrid_prior_attention.py:543-572):
//   x <- w * round(x * rsqrt(mean(x^2) + eps)),  rounded to the activation dtype
// (fp32 statistics; the two roundings of the reference module are kept), then
// rotated.  The row's sum of squares is reduced across its lane group.
//
// Grid: blockIdx.y = one (batch, head) of q (the first B Uq) or of k, so the
// head's base address is wave-uniform scalar arithmetic; blockIdx.x covers
// the head's rows, LANES threads per row (a shift, no integer division).
template <typename T, bool NORM, int LANES>
__global__ __launch_bounds__(256) void rope_kernel(const RopeParams p) {
  const int np = p.hd / 16;  // chunk pairs per row
  const int head = blockIdx.y;
  const bool is_k = head >= p.B * p.Uq;
  const int hh = is_k ? head - p.B * p.Uq : head;
  const int U = is_k ? p.Uk : p.Uq;
  const int b = hh / U, u = hh - b * U;
  const int gid = (int)blockIdx.x * 256 + (int)threadIdx.x;
  const int t = gid / LANES;
  const int c = gid & (LANES - 1);
  const bool active = t < p.T && c < np;
  T* x = reinterpret_cast<T*>(is_k ? p.k : p.q) +
         (is_k ? b * p.k_sb + (int64_t)u * p.k_sh + (int64_t)(active ? t : 0) * p.k_st
               : b * p.q_sb + (int64_t)u * p.q_sh + (int64_t)(active ? t : 0) * p.q_st);
  const int d0 = 8 * c, half = p.hd / 2;
  uint4* lo_p = reinterpret_cast<uint4*>(x + d0);
  uint4* hi_p = reinterpret_cast<uint4*>(x + d0 + half);
  float a[8], bv[8];
  {
    uint4 lo = make_uint4(0, 0, 0, 0), hi = lo;
    if (active) {
      lo = *lo_p;
      hi = *hi_p;
    }
    const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w}, hw[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      a[2 * m] = Elem<T>::lo(lw[m]); a[2 * m + 1] = Elem<T>::hi(lw[m]);
      bv[2 * m] = Elem<T>::lo(hw[m]); bv[2 * m + 1] = Elem<T>::hi(hw[m]);
    }
  }
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int m = 0; m < 8; ++m) ss = fmaf(a[m], a[m], fmaf(bv[m], bv[m], ss));
#pragma unroll
    for (int m = 1; m < LANES; m <<= 1) ss += __shfl_xor(ss, m, LANES);
    const float r = rsqrtf(ss / (float)p.hd + p.eps);
    if (active) {
      float wl[8], wh[8];
      const void* w = is_k ? p.k_w : p.q_w;
      load8(w, p.w_dtype, d0, wl);
      load8(w, p.w_dtype, d0 + half, wh);
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        a[m] = round_to<T>(wl[m] * round_to<T>(a[m] * r));
        bv[m] = round_to<T>(wh[m] * round_to<T>(bv[m] * r));
      }
    }
  }
  if (!active) return;
  float cs[8], sn[8];
  load8(p.cos, p.cs_dtype, (int64_t)t * p.cs_st + d0, cs);
  load8(p.sin, p.cs_dtype, (int64_t)t * p.sn_st + d0, sn);
  // the cache repeats its frequencies in both halves (cos[t][d] = cos[t][d + hd/2])
  uint32_t ol[4], oh[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float a0 = a[2 * m], a1 = a[2 * m + 1], b0 = bv[2 * m], b1 = bv[2 * m + 1];
    const float c0 = cs[2 * m], c1 = cs[2 * m + 1], s0 = sn[2 * m], s1 = sn[2 * m + 1];
    ol[m] = Elem<T>::pack2(fmaf(a0, c0, -b0 * s0), fmaf(a1, c1, -b1 * s1));
    oh[m] = Elem<T>::pack2(fmaf(b0, c0, a0 * s0), fmaf(b1, c1, a1 * s1));
  }
  *lo_p = make_uint4(ol[0], ol[1], ol[2], ol[3]);
  *hi_p = make_uint4(oh[0], oh[1], oh[2], oh[3]);
}

template <typename T, int LANES>
static void launch_rope_l(const RopeParams& p, hipStream_t s) {
  const dim3 grid((unsigned)(((int64_t)p.T * LANES + 255) / 256), (unsigned)(p.B * (p.Uq + p.Uk)));
  if (p.q_w != nullptr)
    hipLaunchKernelGGL((rope_kernel<T, true, LANES>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((rope_kernel<T, false, LANES>), grid, dim3(256), 0, s, p);
}

template <typename T>
static hipError_t launch_rope_t(const RopeParams& p, hipStream_t s) {
  switch (rope_lanes(p.hd)) {
    case 2: launch_rope_l<T, 2>(p, s); break;
    case 4: launch_rope_l<T, 4>(p, s); break;
    case 8: launch_rope_l<T, 8>(p, s); break;
    case 16: launch_rope_l<T, 16>(p, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope(const RopeParams& p, int dtype, hipStream_t s) {
  if ((int64_t)p.B * (p.Uq + p.Uk) * p.T == 0) return hipSuccess;
  if (dtype == kBF16) return launch_rope_t<__bf16>(p, s);
  if (dtype == kF16) return launch_rope_t<_Float16>(p, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
