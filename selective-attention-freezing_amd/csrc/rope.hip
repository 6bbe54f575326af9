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
#include "saf_kernels.h"

namespace saf {

template <typename T>
__global__ __launch_bounds__(256) void rope_kernel(const RopeParams p) {
  const int np = p.hd / 16;  // chunk pairs per row
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t rows_q = (int64_t)p.B * p.Uq * p.T;
  const int64_t rows = rows_q + (int64_t)p.B * p.Uk * p.T;
  const int64_t row = gid / np;
  if (row >= rows) return;
  const int c = (int)(gid % np);
  const bool is_k = row >= rows_q;
  const int64_t rr = is_k ? row - rows_q : row;
  const int U = is_k ? p.Uk : p.Uq;
  const int t = (int)(rr % p.T);
  const int64_t bu = rr / p.T;
  const int u = (int)(bu % U), b = (int)(bu / U);
  T* x = reinterpret_cast<T*>(is_k ? p.k : p.q) +
         (is_k ? b * p.k_sb + (int64_t)u * p.k_sh + (int64_t)t * p.k_st
               : b * p.q_sb + (int64_t)u * p.q_sh + (int64_t)t * p.q_st);
  const int d0 = 8 * c, half = p.hd / 2;
  uint4* lo_p = reinterpret_cast<uint4*>(x + d0);
  uint4* hi_p = reinterpret_cast<uint4*>(x + d0 + half);
  const uint4 lo = *lo_p, hi = *hi_p;
  float cs[8], sn[8];
  if (p.cs_dtype == kF32) {
    const float* cp = reinterpret_cast<const float*>(p.cos) + (int64_t)t * p.cs_st + d0;
    const float* sp = reinterpret_cast<const float*>(p.sin) + (int64_t)t * p.sn_st + d0;
    const float4 c0 = *reinterpret_cast<const float4*>(cp), c1 = *reinterpret_cast<const float4*>(cp + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(sp), s1 = *reinterpret_cast<const float4*>(sp + 4);
    cs[0] = c0.x; cs[1] = c0.y; cs[2] = c0.z; cs[3] = c0.w; cs[4] = c1.x; cs[5] = c1.y; cs[6] = c1.z; cs[7] = c1.w;
    sn[0] = s0.x; sn[1] = s0.y; sn[2] = s0.z; sn[3] = s0.w; sn[4] = s1.x; sn[5] = s1.y; sn[6] = s1.z; sn[7] = s1.w;
  } else {
    const uint4 cw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.cos) + (int64_t)t * p.cs_st + d0);
    const uint4 sw = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p.sin) + (int64_t)t * p.sn_st + d0);
    const uint32_t cw4[4] = {cw.x, cw.y, cw.z, cw.w}, sw4[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (p.cs_dtype == kBF16) {
        cs[2 * m] = Elem<__bf16>::lo(cw4[m]); cs[2 * m + 1] = Elem<__bf16>::hi(cw4[m]);
        sn[2 * m] = Elem<__bf16>::lo(sw4[m]); sn[2 * m + 1] = Elem<__bf16>::hi(sw4[m]);
      } else {
        cs[2 * m] = Elem<_Float16>::lo(cw4[m]); cs[2 * m + 1] = Elem<_Float16>::hi(cw4[m]);
        sn[2 * m] = Elem<_Float16>::lo(sw4[m]); sn[2 * m + 1] = Elem<_Float16>::hi(sw4[m]);
      }
    }
  }
  // the cache repeats its frequencies in both halves (cos[t][d] = cos[t][d + hd/2])
  const uint32_t lw[4] = {lo.x, lo.y, lo.z, lo.w}, hw[4] = {hi.x, hi.y, hi.z, hi.w};
  uint32_t ol[4], oh[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const float a0 = Elem<T>::lo(lw[m]), a1 = Elem<T>::hi(lw[m]);
    const float b0 = Elem<T>::lo(hw[m]), b1 = Elem<T>::hi(hw[m]);
    const float c0 = cs[2 * m], c1 = cs[2 * m + 1], s0 = sn[2 * m], s1 = sn[2 * m + 1];
    ol[m] = Elem<T>::pack2(fmaf(a0, c0, -b0 * s0), fmaf(a1, c1, -b1 * s1));
    oh[m] = Elem<T>::pack2(fmaf(b0, c0, a0 * s0), fmaf(b1, c1, a1 * s1));
  }
  *lo_p = make_uint4(ol[0], ol[1], ol[2], ol[3]);
  *hi_p = make_uint4(oh[0], oh[1], oh[2], oh[3]);
}

hipError_t launch_rope(const RopeParams& p, int dtype, hipStream_t s) {
  const int64_t rows = (int64_t)p.B * (p.Uq + p.Uk) * p.T;
  const int64_t threads = rows * (p.hd / 16);
  if (threads == 0) return hipSuccess;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (dtype == kBF16)
    hipLaunchKernelGGL(rope_kernel<__bf16>, grid, dim3(256), 0, s, p);
  else if (dtype == kF16)
    hipLaunchKernelGGL(rope_kernel<_Float16>, grid, dim3(256), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace saf
