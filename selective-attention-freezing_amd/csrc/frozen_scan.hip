// Closed-form frozen heads as a bandwidth-bound scan along T (gfx950).
//
// A decomposed frozen head (/root/reference/kernel/fused_attn.py:12-19,
// :145-180) whose logits are alpha[j] = 0 and
//   mean    rho[d] = 0                      -> P[i, j] = 1 / (i + 1)
//   decay   rho[d] = -c d  (c > 0)          -> P[i, j] = e^{-c(i-j)} / Z_i
//   window  rho[d] = 0 (d < w), -inf (d>=w) -> P[i, j] = 1 / min(i + 1, w)
// (the reference's own causal-mean prior is supplement/attention.py:10-25 and
// nanogpt/bench_inference_triton.py:92-97; the window prior is
// nanogpt/model.py:347-353) is applied to V as the linear recurrence
//   s_i = r s_{i-1} + u_i,   y_i = s_i / Z_i
// with r = 1 (mean, window) or e^{-c} (decay), u_i = v_i for mean / decay and
// u_i = v_i - v_{i-w} for the window, and Z_i = i + 1, (1 - r^{i+1})/(1 - r)
// or min(i + 1, w).  Reads V once and writes Y once, in fp32 arithmetic.
//
// Parallelisation: each (batch, head) sequence is cut into chunks of CH rows;
// a workgroup takes a ticket from an atomic counter (chunk-major order, so a
// chunk's predecessors always hold smaller tickets and are already running),
// scans its chunk in registers (threads = column groups x row lanes, R rows
// per thread), publishes its chunk aggregate, and obtains the carry from its
// predecessors by decoupled look-back over tagged 64-bit words.  Every wait is
// bounded by spin_limit.
#include "saf_kernels.h"

namespace saf {

__device__ inline uint64_t pack_word(uint32_t tag, float v) {
  return ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v);
}
__device__ inline float word_value(uint64_t w) { return __uint_as_float((uint32_t)(w & 0xffffffffu)); }

template <typename T, int HD, int R>
__global__ __launch_bounds__(256) void scan_kernel(const ScanParams p) {
  constexpr int NCG = HD / 8;                 // 16-byte column groups
  constexpr int NRL = HD <= 64 ? 32 : 16;     // row lanes
  constexpr int NTHR = NCG * NRL;
  constexpr int CH = NRL * R;
  constexpr int LOG_NRL = NRL == 32 ? 5 : 4;
  __shared__ float sh_x[NRL][HD];
  __shared__ float sh_carry[HD];
  __shared__ uint32_t sh_ticket;

  const int tid = threadIdx.x;
  const int cg = tid % NCG, rl = tid / NCG;
  if (tid == 0) sh_ticket = atomicAdd(p.counter, 1u);
  __syncthreads();
  const int ticket = (int)sh_ticket;
  const int nseq = p.B * p.n_slots;
  const int chunk = ticket / nseq, seq = ticket % nseq;
  const int b = seq / p.n_slots, slot = seq % p.n_slots;
  const int kind = p.kind[slot];
  const float prm = p.param[slot];
  const float rate = kind == kScanDecay ? prm : 0.f;
  const float rr = kind == kScanDecay ? expf(-rate) : 1.f;
  const int win = kind == kScanWindow ? (int)prm : 0;
  auto rpow = [&](float k) { return kind == kScanDecay ? expf(-rate * k) : 1.f; };

  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh + 8 * cg;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)p.out_head[slot] * p.o_sh + 8 * cg;
  const int T_len = p.T;
  const int row0 = chunk * CH + rl * R;

  uint4 raw[R], lag[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int row = row0 + i;
    raw[i] = row < T_len ? *reinterpret_cast<const uint4*>(vbase + (int64_t)row * p.v_st) : make_uint4(0, 0, 0, 0);
    lag[i] = make_uint4(0, 0, 0, 0);
    if (kind == kScanWindow && row < T_len && row - win >= 0)
      lag[i] = *reinterpret_cast<const uint4*>(vbase + (int64_t)(row - win) * p.v_st);
  }
  auto unpack = [&](int i, float (&u)[8]) {
    const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
    const uint32_t x[4] = {lag[i].x, lag[i].y, lag[i].z, lag[i].w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      u[2 * m] = Elem<T>::lo(w[m]) - Elem<T>::lo(x[m]);
      u[2 * m + 1] = Elem<T>::hi(w[m]) - Elem<T>::hi(x[m]);
    }
  };

  // thread aggregate: contribution of its R rows to s at its last row
  float agg[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) agg[c] = 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float u[8];
    unpack(i, u);
#pragma unroll
    for (int c = 0; c < 8; ++c) agg[c] = fmaf(agg[c], rr, u[c]);
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) sh_x[rl][8 * cg + c] = agg[c];
  __syncthreads();

  // inclusive scan over row lanes: X_rl = sum_{k <= rl} r^{R (rl - k)} agg_k
#pragma unroll
  for (int st = 0; st < LOG_NRL; ++st) {
    const int off = 1 << st;
    const float f = rpow((float)(R * off));
    float t[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) t[c] = rl >= off ? sh_x[rl - off][8 * cg + c] * f : 0.f;
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 8; ++c) sh_x[rl][8 * cg + c] += t[c];
    __syncthreads();
  }

  // Decoupled look-back (wave 0; lane owns columns lane, lane + 64).  Each
  // published value is one 64-bit word: tag in the high half (1 = chunk
  // aggregate, 2 = inclusive prefix, 0 = not yet written), fp32 value in the
  // low half, so a single relaxed device-scope atomic store publishes it and
  // no fence (L2 write-back / invalidate) is needed on either side.  Columns
  // are independent, so lanes may look back to different depths.
  if (tid < 64) {
    const int lane = tid;
    constexpr int NC = (HD + 63) / 64;
    const int64_t idx = (int64_t)seq * p.n_chunks + chunk;
    const float r_ch = rpow((float)CH);
#pragma unroll
    for (int u = 0; u < NC; ++u) {
      const int col = lane + 64 * u;
      if (col >= HD) continue;
      const float a_wg = sh_x[NRL - 1][col];
      float carry = 0.f;
      if (chunk > 0) {
        __hip_atomic_store(p.agg + idx * HD + col, pack_word(1u, a_wg), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        float factor = 1.f;
        int k = chunk - 1;
        int spins = 0;
        while (k >= 0) {
          const int64_t kc = ((int64_t)seq * p.n_chunks + k) * HD + col;
          const uint64_t wi = __hip_atomic_load(p.incl + kc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (wi >> 32) {
            carry = fmaf(factor, word_value(wi), carry);
            break;
          }
          const uint64_t wa = __hip_atomic_load(p.agg + kc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (wa >> 32) {
            carry = fmaf(factor, word_value(wa), carry);
            factor *= r_ch;
            --k;
            continue;
          }
          if (++spins > p.spin_limit) {  // give up: carry incomplete, kernel still drains
            atomicOr(p.error, 1u);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      }
      __hip_atomic_store(p.incl + idx * HD + col, pack_word(2u, fmaf(carry, r_ch, a_wg)), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      sh_carry[col] = carry;
    }
  }
  __syncthreads();

  // carry into this thread's first row, then the sequential rows
  float s[8];
  {
    const float f = rpow((float)(R * rl));
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float prev = rl > 0 ? sh_x[rl - 1][8 * cg + c] : 0.f;
      s[c] = fmaf(sh_carry[8 * cg + c], f, prev);
    }
  }
  const float em1 = kind == kScanDecay ? expm1f(-rate) : 0.f;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int row = row0 + i;
    float u[8];
    unpack(i, u);
#pragma unroll
    for (int c = 0; c < 8; ++c) s[c] = fmaf(s[c], rr, u[c]);
    if (row < T_len) {
      float inv;
      if (kind == kScanDecay)
        inv = em1 / expm1f(-rate * (float)(row + 1));
      else if (kind == kScanWindow)
        inv = 1.f / (float)min(row + 1, win);
      else
        inv = 1.f / (float)(row + 1);
      uint4 w;
      w.x = Elem<T>::pack2(s[0] * inv, s[1] * inv);
      w.y = Elem<T>::pack2(s[2] * inv, s[3] * inv);
      w.z = Elem<T>::pack2(s[4] * inv, s[5] * inv);
      w.w = Elem<T>::pack2(s[6] * inv, s[7] * inv);
      *reinterpret_cast<uint4*>(obase + (int64_t)row * p.o_st) = w;
    }
  }
}

__global__ void zero_u32_kernel(uint32_t* ptr, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) ptr[i] = 0u;
}

hipError_t launch_zero_u32(uint32_t* ptr, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_u32_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ptr, n);
  return hipGetLastError();
}

template <typename T, int HD>
static hipError_t launch_scan_t(const ScanParams& p, hipStream_t s) {
  constexpr int NTHR = (HD / 8) * (HD <= 64 ? 32 : 16);
  const dim3 grid((unsigned)((int64_t)p.n_chunks * p.B * p.n_slots));
  hipLaunchKernelGGL((scan_kernel<T, HD, 16>), grid, dim3(NTHR), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_scan_hd(const ScanParams& p, int hd, hipStream_t s) {
  switch (hd) {
    case 32: return launch_scan_t<T, 32>(p, s);
    case 64: return launch_scan_t<T, 64>(p, s);
    case 96: return launch_scan_t<T, 96>(p, s);
    case 128: return launch_scan_t<T, 128>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_scan(const ScanParams& p, int dtype, int hd, hipStream_t s) {
  if (dtype == kBF16) return launch_scan_hd<__bf16>(p, hd, s);
  if (dtype == kF16) return launch_scan_hd<_Float16>(p, hd, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
