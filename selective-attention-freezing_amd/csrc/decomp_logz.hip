// Row normalisers of decomposed patterns on gfx950:
//   z[h, i] = logsumexp_{j <= i} (alpha[h, j] + rho[h, i - j]),  i < S
// (/root/reference/kernel/fused_attn.py:101-116 decomposed_logz, which the
// reference computes in chunks of materialised (H, rows, S) logits; the model
// calls it at freeze time, nanogpt/model.py freeze_heads_decomposed, and
// fused_mixed_attn calls it per call when alpha comes without z, :690-694).
//
// One work-group of 4 waves per (64-row block, head), heaviest row blocks
// first.  Lane l of every wave owns row i = i0 + l; the keys j < min(i0+64, S)
// are staged in LDS chunks of kLzChunk columns: alpha[j0 .. j0+C) and the rho
// window rho[i0 - j0 - C + 1 .. i0 - j0 + 63] (-inf at negative distances, so
// the causal mask is free, and past S), both pre-scaled by log2(e) so that the
// running maximum and every exp2 argument are plain fp32 differences (a
// rescale then costs no rounding of a large product: rounding m*log2e and
// mn*log2e separately would add ~ulp(|z|) of error per new row maximum).
// Wave w takes the w-th quarter of each chunk's columns; per 16 columns a lane forms the 16 logits, folds them into
// its running (max, sum) with one rescale, and the four waves' partial
// (max, sum) pairs are merged through LDS at the end.  alpha reads are
// wave-uniform (LDS broadcast), rho reads are consecutive across lanes.
// Work: S(S+1)/2 logits per head, one exp2 each plus one per 16 (the rescale);
// the kernel is bound by exp / VALU issue, HBM traffic is 3 * S * 4 bytes.
#include "saf_kernels.h"

namespace saf {

constexpr int kLzRows = 64;
constexpr int kLzWaves = 4;
constexpr int kLzChunk = 1024;
constexpr int kLzGroup = 16;
static_assert(kLzChunk % (kLzWaves * kLzGroup) == 0, "chunk must split into whole groups per wave");

__global__ __launch_bounds__(64 * kLzWaves) void decomp_logz_kernel(const LogzParams p) {
  __shared__ float as[kLzChunk];
  __shared__ float rs[kLzChunk + kLzRows];
  __shared__ float part_m[kLzWaves][kLzRows];
  __shared__ float part_s[kLzWaves][kLzRows];

  constexpr float kLog2e = 1.4426950408889634f;
  constexpr float kLn2 = 0.6931471805599453f;
  const float ninf = -__builtin_inff();
  const int S = p.S;
  const int nblk = (S + kLzRows - 1) / kLzRows;
  const int i0 = (nblk - 1 - (int)blockIdx.x) * kLzRows;
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float* alpha = p.alpha + (int64_t)h * p.a_hs;
  const float* rho = p.rho + (int64_t)h * p.r_hs;
  const int jend = min(i0 + kLzRows, S);  // keys any row of the block can see

  float m = ninf, s = 0.f;
  for (int j0 = 0; j0 < jend; j0 += kLzChunk) {
    const int dlo = i0 - j0 - kLzChunk + 1;
    __syncthreads();  // previous chunk fully consumed
    for (int t = tid; t < kLzChunk; t += 64 * kLzWaves) {
      const int j = j0 + t;
      as[t] = j < jend ? alpha[j] * kLog2e : ninf;
    }
    for (int t = tid; t < kLzChunk + kLzRows - 1; t += 64 * kLzWaves) {
      const int d = dlo + t;
      rs[t] = (d >= 0 && d < S) ? rho[d] * kLog2e : ninf;
    }
    __syncthreads();
    const int tw0 = w * (kLzChunk / kLzWaves);
    const int tw1 = min(tw0 + kLzChunk / kLzWaves, jend - j0);
    // rho index of column t for this lane: (i0 + lane) - (j0 + t) - dlo
    const int rbase = lane + kLzChunk - 1;
    for (int t = tw0; t < tw1; t += kLzGroup) {
      float x[kLzGroup];
      float gm = ninf;
#pragma unroll
      for (int k = 0; k < kLzGroup; ++k) {
        x[k] = as[t + k] + rs[rbase - t - k];
        gm = fmaxf(gm, x[k]);
      }
      const float mn = fmaxf(m, gm);
      if (mn == ninf) continue;  // every logit so far is -inf: nothing to add
      float acc = s * __builtin_amdgcn_exp2f(m - mn);
#pragma unroll
      for (int k = 0; k < kLzGroup; ++k) acc += __builtin_amdgcn_exp2f(x[k] - mn);
      s = acc;
      m = mn;
    }
  }
  part_m[w][lane] = m;
  part_s[w][lane] = s;
  __syncthreads();
  if (w == 0) {
    float M = part_m[0][lane];
#pragma unroll
    for (int q = 1; q < kLzWaves; ++q) M = fmaxf(M, part_m[q][lane]);
    float zi = ninf;
    if (M != ninf) {
      float tot = 0.f;
#pragma unroll
      for (int q = 0; q < kLzWaves; ++q) tot += part_s[q][lane] * __builtin_amdgcn_exp2f(part_m[q][lane] - M);
      zi = (M + log2f(tot)) * kLn2;
    }
    const int i = i0 + lane;
    if (i < S) p.z[(int64_t)h * p.z_hs + i] = zi;
  }
}

hipError_t launch_decomp_logz(const LogzParams& p, hipStream_t s) {
  const int nblk = (p.S + kLzRows - 1) / kLzRows;
  hipLaunchKernelGGL(decomp_logz_kernel, dim3(nblk, p.H), dim3(64 * kLzWaves), 0, s, p);
  return hipGetLastError();
}


// ---- backward of the row normalisers ------------------------------------------
//   dalpha[h, j] = sum_{i >= j} gz[h, i] exp(alpha[h, j] + rho[h, i - j] - z[h, i])
//   drho[h, d]   = sum_{i >= d} gz[h, i] exp(alpha[h, i - d] + rho[h, d] - z[h, i])
// (the derivative of z = logsumexp_{j<=i}(alpha_j + rho_{i-j}); every term is
// gz_i times a probability <= 1, so no shift is needed).  Both are one sweep
// over the rows i >= o of an output index o: o's own logit part ("fixed":
// alpha_j for dalpha, rho_d for drho) plus a window of the other vector at
// i - o.  One work-group of 4 waves per (64-output block, head, which),
// lane l owns output o = o0 + l; rows are staged in LDS chunks (gz_i and
// -z_i log2 e, 0 / +inf-free for rows past S) with the window of the other
// vector (-inf outside [0, S)), each wave sums a quarter of the chunk's rows,
// and the four partial sums are added through LDS.  Rows whose z is -inf
// (every logit -inf) contribute nothing.
__global__ __launch_bounds__(64 * kLzWaves) void decomp_logz_bwd_kernel(const LogzBwdParams p) {
  __shared__ float gs[kLzChunk], es[kLzChunk];
  __shared__ float ws[kLzChunk + kLzRows];
  __shared__ float part[kLzWaves][kLzRows];

  constexpr float kLog2e = 1.4426950408889634f;
  const float ninf = -__builtin_inff();
  const int S = p.S;
  const int nblk = (S + kLzRows - 1) / kLzRows;
  const int o0 = (int)blockIdx.x * kLzRows;   // lightest blocks (late outputs) last
  const int h = blockIdx.y;
  const bool dr = blockIdx.z == 1;             // 0: dalpha, 1: drho
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const float* alpha = p.alpha + (int64_t)h * p.a_hs;
  const float* rho = p.rho + (int64_t)h * p.r_hs;
  const float* own = dr ? rho : alpha;       // logit part indexed by the output
  const float* other = dr ? alpha : rho;     // logit part indexed by i - o
  const int o = o0 + lane;
  const float fixed = o < S ? own[o] * kLog2e : ninf;
  (void)nblk;

  float acc = 0.f;
  for (int c0 = o0; c0 < S; c0 += kLzChunk) {
    const int tlo = c0 - o0 - (kLzRows - 1);   // smallest i - o of the chunk
    __syncthreads();
    for (int t = tid; t < kLzChunk; t += 64 * kLzWaves) {
      const int i = c0 + t;
      float g = 0.f, e = ninf;
      if (i < S) {
        const float zi = p.z[(int64_t)h * p.z_hs + i];
        if (zi != ninf) {
          g = p.gz[(int64_t)h * p.g_hs + i];
          e = -zi * kLog2e;
        }
      }
      gs[t] = g;
      es[t] = e;
    }
    for (int t = tid; t < kLzChunk + kLzRows - 1; t += 64 * kLzWaves) {
      const int d = tlo + t;
      ws[t] = (d >= 0 && d < S) ? other[d] * kLog2e : ninf;
    }
    __syncthreads();
    const int tw0 = w * (kLzChunk / kLzWaves);
    const int tw1 = min(tw0 + kLzChunk / kLzWaves, S - c0);
    // window index of row c0 + t for this lane: (c0 + t) - o - tlo
    const int wbase = kLzRows - 1 - lane;
    for (int t = tw0; t < tw1; ++t) {
      const float x = fixed + ws[wbase + t] + es[t];
      acc = fmaf(gs[t], __builtin_amdgcn_exp2f(x), acc);
    }
  }
  part[w][lane] = acc;
  __syncthreads();
  if (w == 0 && o < S) {
    float tot = 0.f;
#pragma unroll
    for (int q = 0; q < kLzWaves; ++q) tot += part[q][lane];
    float* out = dr ? p.drho + (int64_t)h * p.dr_hs : p.dalpha + (int64_t)h * p.da_hs;
    out[o] = tot;
  }
}

hipError_t launch_decomp_logz_bwd(const LogzBwdParams& p, hipStream_t s) {
  const int nblk = (p.S + kLzRows - 1) / kLzRows;
  hipLaunchKernelGGL(decomp_logz_bwd_kernel, dim3(nblk, p.H, 2), dim3(64 * kLzWaves), 0, s, p);
  return hipGetLastError();
}

}  // namespace saf
