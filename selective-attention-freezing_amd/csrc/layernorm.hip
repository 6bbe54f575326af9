// Residual add + LayerNorm of the GPT block on gfx950 (the caller side of
// the attention path: /root/reference/nanogpt/model.py:45-54 LayerNorm with
// eps 1e-5 and optional bias, applied as in Block.forward :1214-1240,
// x = x + attn(ln_1(x)); x = x + mlp(ln_2(x))).
//
// One wave per row: x += delta (one rounding to the activation dtype, as
// torch's bf16/fp16 add), then y = (x - mean) * rsqrt(var + eps) * w + b
// from the rounded x in fp32 (two passes over registers: mean, then the
// centred sum of squares), one rounding of y.  The same kernels run the
// RMSNorm of the Qwen caller's decoder blocks (transformers' Qwen3RMSNorm:
// fp32 mean of squares, x * rsqrt(. + eps) rounded to the activation dtype,
// then times the weight and rounded again) when p.rms is set.  Each lane holds NCH chunks of
// VEC consecutive channels, chunk k at channel VEC * (64 k + lane), so every
// load and store of the wave is one coalesced run; chunks past C are idle.
#include "saf_kernels.h"

namespace saf {

template <typename T, int VEC> struct Vec;
template <typename T> struct Vec<T, 4> {
  using raw = uint2;
  __device__ static inline void unpack(raw r, float (&f)[4]) {
    f[0] = Elem<T>::lo(r.x); f[1] = Elem<T>::hi(r.x); f[2] = Elem<T>::lo(r.y); f[3] = Elem<T>::hi(r.y);
  }
  __device__ static inline raw pack(const float (&f)[4]) {
    raw r;
    r.x = Elem<T>::pack2(f[0], f[1]);
    r.y = Elem<T>::pack2(f[2], f[3]);
    return r;
  }
};
template <typename T> struct Vec<T, 8> {
  using raw = uint4;
  __device__ static inline void unpack(raw r, float (&f)[8]) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      f[2 * m] = Elem<T>::lo(w[m]);
      f[2 * m + 1] = Elem<T>::hi(w[m]);
    }
  }
  __device__ static inline raw pack(const float (&f)[8]) {
    raw r;
    r.x = Elem<T>::pack2(f[0], f[1]);
    r.y = Elem<T>::pack2(f[2], f[3]);
    r.z = Elem<T>::pack2(f[4], f[5]);
    r.w = Elem<T>::pack2(f[6], f[7]);
    return r;
  }
};
template <typename T> struct Vec<T, 2> {
  using raw = uint32_t;
  __device__ static inline void unpack(raw r, float (&f)[2]) { f[0] = Elem<T>::lo(r); f[1] = Elem<T>::hi(r); }
  __device__ static inline raw pack(const float (&f)[2]) { return Elem<T>::pack2(f[0], f[1]); }
};

template <typename T>
__device__ inline float round_to_elem(float x) { return (float)static_cast<T>(x); }

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Eight channels of a weight / bias vector as fp32, from fp32, bf16 or fp16.
__device__ inline void load8_f32(const void* p, int c, int dtype, float (&f)[8]) {
  if (dtype == kF32) {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + c);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(p) + c + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w; f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    return;
  }
  const uint4 r = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(p) + c);
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (dtype == kBF16) {
      f[2 * m] = Elem<__bf16>::lo(w[m]);
      f[2 * m + 1] = Elem<__bf16>::hi(w[m]);
    } else {
      f[2 * m] = Elem<_Float16>::lo(w[m]);
      f[2 * m + 1] = Elem<_Float16>::hi(w[m]);
    }
  }
}

template <typename T, int VEC, int NCH>
__global__ __launch_bounds__(256) void add_layernorm_kernel(const AddLnParams p) {
  using V = Vec<T, VEC>;
  using raw = typename V::raw;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows) return;
  const int C = (int)p.C;
  T* xr = reinterpret_cast<T*>(p.x) + row * p.x_rs;
  const T* dr = p.delta ? reinterpret_cast<const T*>(p.delta) + row * p.d_rs : nullptr;
  T* yr = reinterpret_cast<T*>(p.y) + row * p.y_rs;
  float v[NCH][VEC];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = VEC * (64 * k + lane);
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[k][e] = 0.f;
    if (c < C) {  // C is a multiple of VEC: a chunk is wholly in or out
      V::unpack(*reinterpret_cast<const raw*>(xr + c), v[k]);
      if (dr) {
        float d[VEC];
        V::unpack(*reinterpret_cast<const raw*>(dr + c), d);
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[k][e] += d[e];
        const raw r = V::pack(v[k]);
        *reinterpret_cast<raw*>(xr + c) = r;
        V::unpack(r, v[k]);  // the statistics see the rounded residual, as torch's LayerNorm of it does
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int e = 0; e < VEC; ++e) s += v[k][e];
  const float inv_c = 1.f / (float)C;
  const float mean = p.rms ? 0.f : wave_sum(s) * inv_c;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k)
    if (VEC * (64 * k + lane) < C)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float t = v[k][e] - mean;
        q = fmaf(t, t, q);
      }
  const float rstd = rsqrtf(wave_sum(q) * inv_c + p.eps);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = VEC * (64 * k + lane);
    if (c >= C) continue;
    float o[VEC], w[VEC], b[VEC];
    if constexpr (VEC == 8) {  // 16-byte aligned weight / bias (the host checks)
      load8_f32(p.w, c, p.wb_dtype, w);
      if (p.b) load8_f32(p.b, c, p.wb_dtype, b);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        w[e] = load_as_f32(p.w, c + e, p.wb_dtype);
        if (p.b) b[e] = load_as_f32(p.b, c + e, p.wb_dtype);
      }
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float be = p.b ? b[e] : 0.f;
      o[e] = p.rms ? round_to_elem<T>(v[k][e] * rstd) * w[e] : fmaf((v[k][e] - mean) * rstd, w[e], be);
    }
    *reinterpret_cast<raw*>(yr + c) = V::pack(o);
  }
}

// C a multiple of 256 with 16-byte aligned rows: half a wave per row, so each
// wave carries two rows and every lane moves 16-byte pieces (twice the bytes
// per load of the one-wave-per-row kernel): lane l of the half holds NCH
// chunks of 8 channels at 8 (32 k + l), and each chunk load of the half is
// one coalesced 512-byte run.  The row's sums stay inside its half (xor
// shuffles over offsets 16..1).  Same arithmetic as add_layernorm_kernel.
__device__ inline float half_sum(float v) {
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

template <typename T, int NCH>
__global__ __launch_bounds__(256) void add_layernorm_hw_kernel(const AddLnParams p) {
  using V = Vec<T, 4>;
  const int lane = threadIdx.x & 63, hl = lane & 31;
  const int64_t row = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
  if (row >= p.rows) return;  // the other half of the wave only shuffles within itself
  const int C = (int)p.C;
  T* xr = reinterpret_cast<T*>(p.x) + row * p.x_rs;
  const T* dr = p.delta ? reinterpret_cast<const T*>(p.delta) + row * p.d_rs : nullptr;
  T* yr = reinterpret_cast<T*>(p.y) + row * p.y_rs;
  uint4 raw[NCH], draw[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k) raw[k] = *reinterpret_cast<const uint4*>(xr + 8 * (32 * k + hl));
  if (dr) {
#pragma unroll
    for (int k = 0; k < NCH; ++k) draw[k] = *reinterpret_cast<const uint4*>(dr + 8 * (32 * k + hl));
  }
  float v[NCH][8];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    float* vk = v[k];
    V::unpack(make_uint2(raw[k].x, raw[k].y), *reinterpret_cast<float(*)[4]>(vk));
    V::unpack(make_uint2(raw[k].z, raw[k].w), *reinterpret_cast<float(*)[4]>(vk + 4));
    if (dr) {
      float d[8];
      V::unpack(make_uint2(draw[k].x, draw[k].y), *reinterpret_cast<float(*)[4]>(d));
      V::unpack(make_uint2(draw[k].z, draw[k].w), *reinterpret_cast<float(*)[4]>(d + 4));
#pragma unroll
      for (int e = 0; e < 8; ++e) vk[e] += d[e];
      const uint2 r0 = V::pack(*reinterpret_cast<float(*)[4]>(vk));
      const uint2 r1 = V::pack(*reinterpret_cast<float(*)[4]>(vk + 4));
      *reinterpret_cast<uint4*>(xr + 8 * (32 * k + hl)) = make_uint4(r0.x, r0.y, r1.x, r1.y);
      V::unpack(r0, *reinterpret_cast<float(*)[4]>(vk));  // statistics of the rounded residual
      V::unpack(r1, *reinterpret_cast<float(*)[4]>(vk + 4));
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += v[k][e];
  const float inv_c = 1.f / (float)C;
  const float mean = p.rms ? 0.f : half_sum(s) * inv_c;
  float q = 0.f;
#pragma unroll
  for (int k = 0; k < NCH; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = v[k][e] - mean;
      q = fmaf(t, t, q);
    }
  const float rstd = rsqrtf(half_sum(q) * inv_c + p.eps);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int c = 8 * (32 * k + hl);
    float w[8], b[8];
    load8_f32(p.w, c, p.wb_dtype, w);
    if (p.b) {
      load8_f32(p.b, c, p.wb_dtype, b);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) b[e] = 0.f;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      o[e] = p.rms ? round_to_elem<T>(v[k][e] * rstd) * w[e] : fmaf((v[k][e] - mean) * rstd, w[e], b[e]);
    const uint2 r0 = V::pack(*reinterpret_cast<float(*)[4]>(o));
    const uint2 r1 = V::pack(*reinterpret_cast<float(*)[4]>(o + 4));
    *reinterpret_cast<uint4*>(yr + c) = make_uint4(r0.x, r0.y, r1.x, r1.y);
  }
}

template <typename T, int NCH>
static hipError_t launch_ln_hw(const AddLnParams& p, hipStream_t s) {
  hipLaunchKernelGGL((add_layernorm_hw_kernel<T, NCH>), dim3((unsigned)((p.rows + 7) / 8)), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T, int VEC, int NCH>
static hipError_t launch_ln_t(const AddLnParams& p, hipStream_t s) {
  hipLaunchKernelGGL((add_layernorm_kernel<T, VEC, NCH>), dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, s, p);
  return hipGetLastError();
}

// Channel layouts: multiples of 256 use 8-byte chunks (VEC 4); other
// multiples of 8 with 16-byte aligned rows 16-byte chunks (VEC 8: C = 896 of
// the Qwen caller is 1.75 chunks per lane); other even C up to 2048 4-byte
// chunks (VEC 2); the tail lanes idle.
template <typename T>
static hipError_t launch_ln_dt(const AddLnParams& p, hipStream_t s) {
  if (p.vec16) {
    switch (p.C / 256) {
      case 1: return launch_ln_hw<T, 1>(p, s);
      case 2: return launch_ln_hw<T, 2>(p, s);
      case 3: return launch_ln_hw<T, 3>(p, s);
      case 4: return launch_ln_hw<T, 4>(p, s);
      case 5: return launch_ln_hw<T, 5>(p, s);
      case 6: return launch_ln_hw<T, 6>(p, s);
      case 7: return launch_ln_hw<T, 7>(p, s);
      case 8: return launch_ln_hw<T, 8>(p, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.C % 256 == 0) {
    switch (p.C / 256) {
      case 1: return launch_ln_t<T, 4, 1>(p, s);
      case 2: return launch_ln_t<T, 4, 2>(p, s);
      case 3: return launch_ln_t<T, 4, 3>(p, s);
      case 4: return launch_ln_t<T, 4, 4>(p, s);
      case 5: return launch_ln_t<T, 4, 5>(p, s);
      case 6: return launch_ln_t<T, 4, 6>(p, s);
      case 7: return launch_ln_t<T, 4, 7>(p, s);
      case 8: return launch_ln_t<T, 4, 8>(p, s);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.vec16_rows && p.C % 8 == 0) {
    switch ((p.C + 511) / 512) {
      case 1: return launch_ln_t<T, 8, 1>(p, s);
      case 2: return launch_ln_t<T, 8, 2>(p, s);
      case 3: return launch_ln_t<T, 8, 3>(p, s);
      case 4: return launch_ln_t<T, 8, 4>(p, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch ((p.C + 127) / 128) {
    case 1: return launch_ln_t<T, 2, 1>(p, s);
    case 2: return launch_ln_t<T, 2, 2>(p, s);
    case 3: return launch_ln_t<T, 2, 3>(p, s);
    case 4: return launch_ln_t<T, 2, 4>(p, s);
    case 5: return launch_ln_t<T, 2, 5>(p, s);
    case 6: return launch_ln_t<T, 2, 6>(p, s);
    case 7: return launch_ln_t<T, 2, 7>(p, s);
    case 8: return launch_ln_t<T, 2, 8>(p, s);
    case 9: return launch_ln_t<T, 2, 9>(p, s);
    case 10: return launch_ln_t<T, 2, 10>(p, s);
    case 11: return launch_ln_t<T, 2, 11>(p, s);
    case 12: return launch_ln_t<T, 2, 12>(p, s);
    case 13: return launch_ln_t<T, 2, 13>(p, s);
    case 14: return launch_ln_t<T, 2, 14>(p, s);
    case 15: return launch_ln_t<T, 2, 15>(p, s);
    case 16: return launch_ln_t<T, 2, 16>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_add_layernorm(const AddLnParams& p, int dtype, hipStream_t s) {
  if (dtype == kBF16) return launch_ln_dt<__bf16>(p, s);
  if (dtype == kF16) return launch_ln_dt<_Float16>(p, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
