// Projection GEMMs with fused epilogues, on gfx950: C = epi(A W^T) for A
// (M x K) activations, W (N x K) an nn.Linear weight without bias and C
// (M x N), all bf16 / fp16 and row-major (N a multiple of 256, K of 128, any
// M); fp32 accumulation, the epilogue in fp32 on the accumulator, one
// rounding of C.  Two epilogues (the caller side of the attention path):
//
// * the exact GELU of the MLP's up-projection (/root/reference/nanogpt/
//   model.py:1193-1207, c_fc followed by nn.GELU()):
//     C[m][n] = gelu(u) = u Phi(u) = u (1 + erf(u / sqrt 2)) / 2,  u = (A W^T)[m][n]
//   Phi comes from an odd polynomial fitted to it on |u| <= 3.5 and, beyond,
//   from Abramowitz and Stegun's rational approximation of erfc (7.1.26,
//   Handbook of Mathematical Functions, 1964, absolute error at most 1.5e-7);
//   either way the GELU is within 5.3e-6 of the exact value, far below the
//   output's half-ulp for values of that size.  Fusing it removes the pass that
//   reads and writes C again.
// * the rotary embedding of the indexed QKV projection (the gathered
//   [Wq[live]; Wk[live]; Wv] weight of nanogpt/model.py:920-944 and the Llama
//   half rotation of :57-99 applied to the live q / k at :1003-1008): the
//   first n_rope columns are heads of hd columns, each rotated at position
//   t = m mod T,
//     C[m][d] = u[d] cos[t][d] - u[d + hd/2] sin[t][d]            d <  hd/2
//     C[m][d] = u[d] cos[t][d] + u[d - hd/2] sin[t][d]            d >= hd/2
//   and the columns after them (V, zero padding) are stored as they are.
//   Fusing it removes the pass over q and k.
// * the SwiGLU of a Qwen3 MLP (transformers' Qwen3MLP, the C4 caller's
//   down_proj(act_fn(gate_proj(x)) * up_proj(x)) with act_fn = SiLU): W holds
//   the gate and up rows interleaved in blocks of 64 (gate rows 64 b.., then
//   the up rows 64 b..), and C (M x N/2) = silu(x Wg^T) * (x Wu^T), silu(u) =
//   u / (1 + e^-u); the two products never reach memory.
//
// Tiling: 256 x 256 tiles of C, one persistent workgroup of 8 waves per CU
// walking its tiles in turn; wave w computes the 64 (rows of A) x 128 (rows
// of W) block (64 (w / 2), 128 (w % 2)).  The product runs transposed
// (C^T = W A^T on v_mfma_f32_32x32x16): W rows are the MFMA's A operand, A
// rows its B operand, both read with ds_read_b128 (8 consecutive k of a row)
// from LDS tiles of 256 rows x 32 k, so each lane's accumulator holds 4 runs
// of 4 consecutive columns of one row of C (a rotation pair d, d + hd/2 sits
// in one lane), paired across the wave's halves into 16-byte pieces for the
// stores.  The k tiles arrive by buffer_load ... lds DMA into four LDS stages,
// three k steps ahead, as one stream over the workgroup's tiles: the last
// steps of a tile load the first k tiles of the next, which land while the
// epilogue runs.  The 16-byte chunks of a tile row are XOR-swizzled by the
// row so that the reads of a 16-lane group hit distinct banks.
#include "saf_kernels.h"

namespace saf {

namespace {

constexpr int kGBM = 256, kGBN = 256, kGBK = 32, kGStages = 4, kGWaves = 8;
constexpr int kGRowBytes = kGBK * 2;          // one k-tile row (64 bytes)
constexpr int kGTileBytes = kGBM * kGRowBytes;  // one operand's k tile (16 KB)
constexpr int kGChunks = kGBK / 8;            // 16-byte chunks per row
constexpr int kGDma = kGBM * kGChunks / (64 * kGWaves);  // DMA loads per thread, operand and step
static_assert(kGBM == kGBN, "both operand tiles have kGBM rows");
static_assert(kGDma * 64 * kGWaves == kGBM * kGChunks, "DMA chunks split evenly over the threads");

// logical chunk c of row r sits at chunk c ^ swz(r): rows r .. r + 15 of one
// chunk land on 16 distinct 4-bank groups (row pitch 64 bytes); the swizzle
// depends on r % 16 only
__device__ __forceinline__ int gswz(int r) { return (r >> 2) & 3; }

// byte offset in a k tile of row r, logical chunk c
__device__ __forceinline__ int gtile_off(int r, int c) { return r * kGRowBytes + 16 * (c ^ gswz(r)); }

// gelu(u) = u Phi(u) with Phi(u) = 1 - erfc(u / sqrt 2) / 2 for u >= 0 and
// erfc(|u| / sqrt 2) / 2 below, erfc(z) = t (a1 + t (a2 + ... + t a5)) e^{-z^2},
// t = 1 / (1 + p z) (A&S 7.1.26; the 1/2 folded into the a_i): any u
__device__ __forceinline__ float gelu_tail(float u) {
  constexpr float kSqrtHalf = 0.70710678118654752440f;
  const float z = fabsf(u) * kSqrtHalf;
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, z, 1.f));
  float pol = fmaf(t, 0.5f * 1.061405429f, 0.5f * -1.453152027f);
  pol = fmaf(t, pol, 0.5f * 1.421413741f);
  pol = fmaf(t, pol, 0.5f * -0.284496736f);
  pol = fmaf(t, pol, 0.5f * 0.254829592f);
  const float h = pol * t * __builtin_amdgcn_exp2f(z * (z * -kLog2e));
  return u * (u >= 0.f ? 1.f - h : h);
}

// gelu(u) for |u| <= kGeluPolyMax: Phi(u) - 1/2 as an odd polynomial of
// degree 17, its coefficients fitted (reweighted least squares on Chebyshev
// nodes) to erf(u / sqrt 2) / 2 on that range (the leading one is
// 1 / sqrt(2 pi)); evaluated in fp32 the GELU is within 5.3e-6 of the exact
// value there.  Ten VALU slots against gelu_tail's ~23 (two of them
// quarter-rate transcendentals).
constexpr float kGeluPolyMax = 3.5f;
__device__ __forceinline__ float gelu_poly(float u) {
  const float u2 = u * u;
  float p = 1.635428320545529e-10f;
  p = fmaf(p, u2, -1.1564693203069965e-08f);
  p = fmaf(p, u2, 3.7499219729397737e-07f);
  p = fmaf(p, u2, -7.5377106441010255e-06f);
  p = fmaf(p, u2, 0.00010740307334344834f);
  p = fmaf(p, u2, -0.0011667633662000299f);
  p = fmaf(p, u2, 0.009944464080035686f);
  p = fmaf(p, u2, -0.06647146493196487f);
  p = fmaf(p, u2, 0.3989386558532715f);
  return u * fmaf(p, u, 0.5f);
}

// gelu of n accumulator values in place: the polynomial for all, and, only
// when some lane of the wave holds one beyond its range, the tail formula
// for those (a wave-uniform branch, rarely taken for MLP activations)
template <int n>
__device__ __forceinline__ void gelu_group(float (&x)[n]) {
  float v[n], big = 0.f;
#pragma unroll
  for (int i = 0; i < n; ++i) {
    v[i] = gelu_poly(x[i]);
    big = fmaxf(big, fabsf(x[i]));
  }
  if (__builtin_amdgcn_ballot_w64(!(big <= kGeluPolyMax)) != 0) {
#pragma unroll
    for (int i = 0; i < n; ++i)
      if (!(fabsf(x[i]) <= kGeluPolyMax)) v[i] = gelu_tail(x[i]);
  }
#pragma unroll
  for (int i = 0; i < n; ++i) x[i] = v[i];
}

enum : int { kEpiGelu = 0, kEpiRope = 1, kEpiSwiglu = 2 };

// EPI: kEpiGelu, or kEpiRope with head dimension HD (64 or 128)
template <typename T, int EPI, int HD>
__global__ __launch_bounds__(64 * kGWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void proj_gemm_kernel(const ProjGemmParams p) {
  // one array per operand and stage, so that the compiler's wait insertion
  // sees that a read of one stage does not depend on the DMAs into the others
  __shared__ __align__(16) char sw0[kGTileBytes], sw1[kGTileBytes], sw2[kGTileBytes], sw3[kGTileBytes];
  __shared__ __align__(16) char sa0[kGTileBytes], sa1[kGTileBytes], sa2[kGTileBytes], sa3[kGTileBytes];
  auto wst = [&](auto stage) -> char* {
    constexpr int S = decltype(stage)::value;
    return S == 0 ? sw0 : (S == 1 ? sw1 : (S == 2 ? sw2 : sw3));
  };
  auto ast = [&](auto stage) -> char* {
    constexpr int S = decltype(stage)::value;
    return S == 0 ? sa0 : (S == 1 ? sa1 : (S == 2 ? sa2 : sa3));
  };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n32 = lane & 31, g = lane >> 5;
  const int wm = wave >> 1, wn = wave & 1;

  // tile order: workgroup b runs on XCD b % 8; each XCD owns a contiguous
  // run of per_xcd tiles (columns fastest), which its gridDim / 8 workgroups
  // take in strides, so the tiles in flight on an XCD stay contiguous and the
  // A rows of a tile row stay in that XCD's L2
  const int tiles_n = p.N / kGBN, tiles = ((p.M + kGBM - 1) / kGBM) * tiles_n;
  const int per_xcd = (tiles + 7) / 8;
  const int xcd = (int)(blockIdx.x % 8), local = (int)(blockIdx.x / 8), n_local = (int)(gridDim.x / 8);
  auto tile_of = [&](int i) {
    const int v = local + i * n_local, t = xcd * per_xcd + v;
    return v < per_xcd && t < tiles ? t : -1;
  };
  int cur = tile_of(0);
  if (cur < 0) return;
  int nxt = tile_of(1);

  // DMA: load q of a thread writes chunk X = (8 q + wave) * 64 + lane of a
  // tile, i.e. row X / 4, stored chunk X % 4 = logical chunk (X % 4) ^ swz(row);
  // source offsets from the tile's first row at k = 0
  uint32_t aoff[kGDma], woff[kGDma];
#pragma unroll
  for (int q = 0; q < kGDma; ++q) {
    const int X = (kGWaves * q + wave) * 64 + lane;
    const int r = X / kGChunks, c = (X % kGChunks) ^ gswz(r);
    aoff[q] = (uint32_t)(r * p.a_rs * 2 + 16 * c);
    woff[q] = (uint32_t)(r * p.w_rs * 2 + 16 * c);
  }
  const int nk = p.K / kGBK;  // a multiple of kGStages
  // descriptors over a tile's rows of A (rows past M read as zero) and W; a
  // missing tile gets empty ones, whose loads write zeros
  auto a_rsrc = [&](int t) {
    const int m0 = t < 0 ? 0 : (t / tiles_n) * kGBM;
    const T* base = reinterpret_cast<const T*>(p.a) + (int64_t)m0 * p.a_rs;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, t < 0 ? 0 : min(kGBM, p.M - m0) * p.a_rs * 2,
                                             kBufferWord3);
  };
  auto w_rsrc = [&](int t) {
    const int n0 = t < 0 ? 0 : (t % tiles_n) * kGBN;
    const T* base = reinterpret_cast<const T*>(p.w) + (int64_t)n0 * p.w_rs;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, t < 0 ? 0 : kGBN * p.w_rs * 2, kBufferWord3);
  };
  __amdgpu_buffer_rsrc_t ars = a_rsrc(cur), wrs = w_rsrc(cur), arn = a_rsrc(nxt), wrn = w_rsrc(nxt);

  // the DMA of k step j of the stream position: j < nk reads the current
  // tile at k step j, j >= nk the next tile at k step j - nk
  auto load_step = [&](int j, auto stage) {
    char* const tw = wst(stage);
    char* const ta = ast(stage);
    const bool here = j < nk;
    const int so = kGRowBytes * (here ? j : j - nk);
#pragma unroll
    for (int q = 0; q < kGDma; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(here ? ars : arn, SAF_LDS_PTR(ta + (kGWaves * q + wave) * 1024), 16,
                                               aoff[q], so, 0, 0);
#pragma unroll
    for (int q = 0; q < kGDma; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(here ? wrs : wrn, SAF_LDS_PTR(tw + (kGWaves * q + wave) * 1024), 16,
                                               woff[q], so, 0, 0);
  };

  // read offsets of this lane: W rows 128 wn + 32 nt + n32, A rows
  // 64 wm + 32 mt + n32, logical chunk 2 s + g for k substep s; the 32-row
  // subtiles nt / mt sit 2 KB apart
  int wrd[2], ard[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    wrd[s] = gtile_off(128 * wn + n32, 2 * s + g);
    ard[s] = gtile_off(64 * wm + n32, 2 * s + g);
  }
  constexpr int kSub = 32 * kGRowBytes;

  f32x16_t acc[4][2];
  auto read_sub = [&](auto stage, auto sub, uint4 (&wa)[4], uint4 (&ab)[2]) {
    constexpr int s = decltype(sub)::value;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) wa[nt] = *reinterpret_cast<const uint4*>(wst(stage) + wrd[s] + nt * kSub);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) ab[mt] = *reinterpret_cast<const uint4*>(ast(stage) + ard[s] + mt * kSub);
  };
  auto mma = [&](const uint4 (&wa)[4], const uint4 (&ab)[2]) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) acc[nt][mt] = Elem<T>::mfma(wa[nt], ab[mt], acc[nt][mt]);
  };

  using G0 = std::integral_constant<int, 0>;
  using G1 = std::integral_constant<int, 1>;
  using G2 = std::integral_constant<int, 2>;
  using G3 = std::integral_constant<int, 3>;
  using Sub0 = std::integral_constant<int, 0>;
  using Sub1 = std::integral_constant<int, 1>;
  load_step(0, G0());
  load_step(1, G1());
  load_step(2, G2());
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(4 * kGDma));  // step 0 landed, steps 1, 2 in flight
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  uint4 wa0[4], ab0[2], wa1[4], ab1[2];
  read_sub(G0(), Sub0(), wa0, ab0);

  // k step j in stage j % 4 (nk is a multiple of 4, so every tile starts at
  // stage 0), its substep 0 operands already in registers: the DMA of stream
  // step j + 3 goes to stage (j + 3) % 4, last read in step j - 1 (every
  // wave's reads of it completed before the previous barrier); substep 1's
  // reads run under substep 0's products; the barrier follows the wait for
  // step j + 1's DMA (steps j + 2, j + 3 stay in flight) and for this wave's
  // reads of stage j, and step j + 1's substep 0 reads (the next tile's
  // first k tile after a tile's last step) run under substep 1's products.
  // The scheduling barriers keep each group of reads ahead of the products
  // it overlaps.
  auto step = [&](int j, auto stage) {
    constexpr int S = decltype(stage)::value;
    using Ahead = std::integral_constant<int, (S + 3) % kGStages>;
    using Next = std::integral_constant<int, (S + 1) % kGStages>;
    load_step(j + 3, Ahead());
    read_sub(stage, Sub1(), wa1, ab1);
    __builtin_amdgcn_sched_barrier(0);
    mma(wa0, ab0);
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(4 * kGDma));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_sub(Next(), Sub0(), wa0, ab0);
    __builtin_amdgcn_sched_barrier(0);
    mma(wa1, ab1);
    __builtin_amdgcn_sched_barrier(0);
  };

  for (int i = 1;; ++i) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) acc[nt][mt] = zero16();
    for (int j = 0; j < nk; j += kGStages) {
      step(j, G0());
      step(j + 1, G1());
      step(j + 2, G2());
      step(j + 3, G3());
    }

    // epilogue of tile cur (the next tile's first k tiles are in flight):
    // lane (n32, g), tile (nt, mt), register 4 q + e holds C[row][col],
    // row = m0 + 64 wm + 32 mt + n32, col = n0 + 128 wn + 32 nt + 8 q + 4 g + e.
    // v_permlane32_swap(vdst, vsrc) exchanges vdst of lanes 32..63 with vsrc
    // of lanes 0..31: with vdst = piece q = 2 r and vsrc = piece 2 r + 1, lane
    // (n32, 0) ends with columns 16 r + 0..7 and lane (n32, 1) with
    // 16 r + 8..15 of the row, one 16-byte store each
    const int m0 = (cur / tiles_n) * kGBM, n0 = (cur % tiles_n) * kGBN;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int row = m0 + 64 * wm + 32 * mt + n32;
      if constexpr (EPI == kEpiRope) {
        // the wave's 128 columns are two heads (hd 64: pairs nt 0 / 1 and
        // 2 / 3, the same d for both) or one (hd 128: pairs nt 0 / 2 and 1 / 3),
        // all rotated or none (n_rope is a multiple of 128)
        if (n0 + 128 * wn < p.n_rope) {
          const int t = (row < p.M ? row : 0) % p.T;
          const uint16_t* cs = reinterpret_cast<const uint16_t*>(p.cos) + (int64_t)t * p.cs_st + 4 * g;
          const uint16_t* sn = reinterpret_cast<const uint16_t*>(p.sin) + (int64_t)t * p.sn_st + 4 * g;
          constexpr int kHalf = HD / 2, kPairs = HD == 64 ? 1 : 2;
#pragma unroll
          for (int pi = 0; pi < kPairs; ++pi) {
            // cos / sin at d1 = 32 pi + 8 q + 4 g + e and d1 + hd/2, in the
            // activation dtype, four per 8-byte load
            uint2 c1[4], s1[4], c2[4], s2[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int d1 = 32 * pi + 8 * q;
              c1[q] = *reinterpret_cast<const uint2*>(cs + d1);
              s1[q] = *reinterpret_cast<const uint2*>(sn + d1);
              c2[q] = *reinterpret_cast<const uint2*>(cs + d1 + kHalf);
              s2[q] = *reinterpret_cast<const uint2*>(sn + d1 + kHalf);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const uint32_t wc1 = e < 2 ? c1[q].x : c1[q].y, ws1 = e < 2 ? s1[q].x : s1[q].y;
                const uint32_t wc2 = e < 2 ? c2[q].x : c2[q].y, ws2 = e < 2 ? s2[q].x : s2[q].y;
                const float fc1 = e % 2 ? Elem<T>::hi(wc1) : Elem<T>::lo(wc1);
                const float fs1 = e % 2 ? Elem<T>::hi(ws1) : Elem<T>::lo(ws1);
                const float fc2 = e % 2 ? Elem<T>::hi(wc2) : Elem<T>::lo(wc2);
                const float fs2 = e % 2 ? Elem<T>::hi(ws2) : Elem<T>::lo(ws2);
#pragma unroll
                for (int hh = 0; hh < 2 / kPairs; ++hh) {
                  const int lo = HD == 64 ? 2 * hh : pi, hi = HD == 64 ? 2 * hh + 1 : pi + 2;
                  const float x1 = acc[lo][mt][4 * q + e], x2 = acc[hi][mt][4 * q + e];
                  acc[lo][mt][4 * q + e] = x1 * fc1 - x2 * fs1;
                  acc[hi][mt][4 * q + e] = x2 * fc2 + x1 * fs2;
                }
              }
            __builtin_amdgcn_sched_barrier(0);  // one pair's cos / sin live at a time
          }
        }
      }
      // SwiGLU: the wave's 128 columns are 64 gate features (nt 0, 1) and the
      // same 64 up features (nt 2, 3); it writes their 64 products at output
      // column n0 / 2 + 64 wn + d, d = 32 nt + 8 q + 4 g + e
      constexpr int kOutTiles = EPI == kEpiSwiglu ? 2 : 4;
      T* crow = reinterpret_cast<T*>(p.c) + (int64_t)row * p.c_rs +
                (EPI == kEpiSwiglu ? n0 / 2 + 64 * wn : n0 + 128 * wn) + 8 * g;
#pragma unroll
      for (int nt = 0; nt < kOutTiles; ++nt)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const f32x16_t& a = acc[nt][mt];
          float y[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) y[i] = a[8 * r + i];
          if constexpr (EPI == kEpiGelu) gelu_group(y);
          if constexpr (EPI == kEpiSwiglu) {
            // silu(x) = x / (1 + e^-x), in fp32, times the up projection
            const f32x16_t& up = acc[nt + 2][mt];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const float x = y[i];
              y[i] = x * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -kLog2e)) * up[8 * r + i];
            }
          }
          uint32_t pc[2][2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            pc[h][0] = Elem<T>::pack2(y[4 * h], y[4 * h + 1]);
            pc[h][1] = Elem<T>::pack2(y[4 * h + 2], y[4 * h + 3]);
          }
          const auto s0 = __builtin_amdgcn_permlane32_swap(pc[0][0], pc[1][0], false, false);
          const auto s1 = __builtin_amdgcn_permlane32_swap(pc[0][1], pc[1][1], false, false);
          if (row < p.M) *reinterpret_cast<uint4*>(crow + 32 * nt + 16 * r) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
        }
    }
    if (nxt < 0) break;
    cur = nxt;
    nxt = tile_of(i + 1);
    ars = arn;
    wrs = wrn;
    arn = a_rsrc(nxt);
    wrn = w_rsrc(nxt);
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // the trailing (empty) DMAs land before exit
}

}  // namespace

namespace {

// In-place exact GELU over n elements (n % 8 == 0, 16-byte aligned), for a
// GEMM output that the fused kernel does not produce (the 1B-class model's
// MLP at K = 2048): eight elements per thread and grid-stride step, the
// polynomial for every group of eight whose wave holds no value beyond its
// range, else the tail formula, as the fused epilogue.
template <typename T>
__global__ __launch_bounds__(256) void gelu_inplace_kernel(T* x, int64_t n8) {
  uint4* v = reinterpret_cast<uint4*>(x);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const uint4 r = v[i];
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    float y[8];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      y[2 * m] = Elem<T>::lo(w[m]);
      y[2 * m + 1] = Elem<T>::hi(w[m]);
    }
    gelu_group(y);
    v[i] = make_uint4(Elem<T>::pack2(y[0], y[1]), Elem<T>::pack2(y[2], y[3]), Elem<T>::pack2(y[4], y[5]),
                      Elem<T>::pack2(y[6], y[7]));
  }
}

}  // namespace

hipError_t launch_gelu_inplace(void* x, int64_t n, int dtype, int n_cu, hipStream_t s) {
  const int64_t n8 = n / 8;
  const unsigned grid = (unsigned)std::min<int64_t>((n8 + 255) / 256, (int64_t)n_cu * 16);
  if (n8 == 0) return hipSuccess;
  if (dtype == kBF16)
    hipLaunchKernelGGL(gelu_inplace_kernel<__bf16>, dim3(grid), dim3(256), 0, s, reinterpret_cast<__bf16*>(x), n8);
  else if (dtype == kF16)
    hipLaunchKernelGGL(gelu_inplace_kernel<_Float16>, dim3(grid), dim3(256), 0, s, reinterpret_cast<_Float16*>(x), n8);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

bool proj_gemm_shape_ok(int64_t M, int64_t N, int64_t K) {
  return M > 0 && N > 0 && K > 0 && N % kGBN == 0 && K % (kGBK * kGStages) == 0;
}

namespace {

// one workgroup per CU (a multiple of the 8 XCDs), fewer for small problems
dim3 proj_grid(const ProjGemmParams& p) {
  const int tiles = ((p.M + kGBM - 1) / kGBM) * (p.N / kGBN);
  const int per_xcd = (tiles + 7) / 8;
  const int n_local = max(1, min(p.n_cu / 8, per_xcd));
  return dim3((unsigned)(8 * n_local));
}

template <int EPI, int HD>
hipError_t launch_proj(const ProjGemmParams& p, int dtype, hipStream_t s) {
  if (dtype == kBF16)
    hipLaunchKernelGGL((proj_gemm_kernel<__bf16, EPI, HD>), proj_grid(p), dim3(64 * kGWaves), 0, s, p);
  else if (dtype == kF16)
    hipLaunchKernelGGL((proj_gemm_kernel<_Float16, EPI, HD>), proj_grid(p), dim3(64 * kGWaves), 0, s, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_gelu(const ProjGemmParams& p, int dtype, hipStream_t s) {
  return launch_proj<kEpiGelu, 0>(p, dtype, s);
}

hipError_t launch_gemm_swiglu(const ProjGemmParams& p, int dtype, hipStream_t s) {
  return launch_proj<kEpiSwiglu, 0>(p, dtype, s);
}

hipError_t launch_gemm_rope(const ProjGemmParams& p, int dtype, hipStream_t s) {
  if (p.hd == 64) return launch_proj<kEpiRope, 64>(p, dtype, s);
  if (p.hd == 128) return launch_proj<kEpiRope, 128>(p, dtype, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
