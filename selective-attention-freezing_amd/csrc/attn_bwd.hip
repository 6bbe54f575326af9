// Backward of the mixed-head attention operator on gfx950.
//
// Semantics follow the reference's backward (/root/reference/kernel/
// fused_attn.py:291-591): delta = rowsum(out * dout) per live row
// (_bwd_preprocess :291-310); live heads get dQ, dK, dV of causal softmax
// attention recomputed from the forward's base-2 LSE (_dkdv_flash, _bwd_dq
// :360-540); frozen heads get only dV = P^T dO with the dense pattern
// (_dv_dense :314-331) or the decomposed pattern rebuilt from alpha, rho, z
// (_dv_decomp :333-358), and no dQ / dK.  P and dS are rounded to the input
// dtype before the products that consume them, as the reference's bf16 dots.
//
// All products use v_mfma_f32_32x32x16 on 64-row tiles staged in LDS by
// buffer_load ... lds DMA in the VRow layout (row-major, 32-byte segments
// XOR-swizzled by row), which serves both operand orientations:
//   tile_row_op: 8 consecutive columns of one row (ds_read_b128), and
//   tile_col_op: 8 consecutive rows of one column (two ds_read_b64_tr_b16).
// Each wave owns 32 rows of the output (queries for dQ, keys for dK / dV);
// a lane owns one of them, so the per-row softmax statistics are per lane
// (dQ) or, with the row-permuted (kperm) products, per register (dK / dV).
#include <type_traits>

#include "saf_kernels.h"

namespace saf {

namespace {

constexpr int kBwdWaves = 4;

// 16-byte operand of a VRow tile: elements 8c .. 8c+7 of row r.
template <int HD>
__device__ __forceinline__ uint4 tile_row_op(const char* tile, int r, int c) {
  return *reinterpret_cast<const uint4*>(tile + r * VRow<HD>::PITCH + 16 * (c ^ VRow<HD>::swz(r)));
}

// Transposed operand of a VRow tile: lane (n, g) receives rows
// 16 ks + 8 g + 0..7 of column 32 dt + n.  The lane's read offsets are
// computed once (ColOffsets): computed next to each read, their XOR-swizzled
// column was unbounded to the compiler, which then let a read reach the
// neighbouring LDS slots and waited for the DMA in flight into them.
template <int HD> struct ColOffsets {
  int lo[HD / 32], hi[HD / 32];
  __device__ __forceinline__ void init(int lane) {
#pragma unroll
    for (int dt = 0; dt < HD / 32; ++dt) {
      lo[dt] = vt_read_offset<HD>(lane, dt, 0);
      hi[dt] = vt_read_offset<HD>(lane, dt, 1);
    }
  }
};

template <int HD>
__device__ __forceinline__ uint4 tile_col_op(const char* tile, int ks, int dt, const ColOffsets<HD>& cof) {
  const char* base = tile + 16 * ks * VRow<HD>::PITCH;
  const uint2 lo = ds_read_tr16(base + cof.lo[dt]);
  const uint2 hi = ds_read_tr16(base + cof.hi[dt]);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// DMA source offsets of this thread's chunks of a 64-row VRow tile.
template <typename T, int HD>
struct TileOffsets {
  static constexpr int VN = VRow<HD>::CHP / kBwdWaves;
  uint32_t off[VN];
  __device__ __forceinline__ void init(int wave, int lane, int64_t st) {
#pragma unroll
    for (int pp = 0; pp < VN; ++pp) off[pp] = vrow_dma_offset<T, HD>((kBwdWaves * pp + wave) * 64 + lane, st);
  }
  // rows r0 .. r0+63 of a (T_len, st) tensor at base; rows >= T_len read zero
  __device__ __forceinline__ void load(const T* base, int64_t st, int r0, int T_len, char* tile, int wave) const {
    const __amdgpu_buffer_rsrc_t r = rows_rsrc(base, st, r0, T_len);
#pragma unroll
    for (int pp = 0; pp < VN; ++pp)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, SAF_LDS_PTR(tile + (kBwdWaves * pp + wave) * 1024), 16, off[pp], 0,
                                               0, 0);
  }
};

__device__ __forceinline__ uint4 load16(const void* p) { return *reinterpret_cast<const uint4*>(p); }

// The eight 16-bit elements of w (bf16 or fp16) with their signs flipped.
__device__ __forceinline__ uint4 neg_halves(uint4 w) {
  return make_uint4(w.x ^ 0x80008000u, w.y ^ 0x80008000u, w.z ^ 0x80008000u, w.w ^ 0x80008000u);
}

}  // namespace

// delta[b, slot, i] = sum_d out[b, h, i, d] * dout[b, h, i, d] over the live
// rows, fp32.  A row is read by delta_lanes(HD) lanes, 16 bytes each, so one
// load instruction covers whole rows (one lane per row touched 64 rows per
// instruction), and the lanes' sums meet by shuffles.
constexpr int delta_lanes(int hd) { return hd <= 32 ? 4 : (hd <= 64 ? 8 : (hd <= 128 ? 16 : 32)); }

template <typename T, int HD>
__global__ __launch_bounds__(256) void bwd_delta_kernel(const BwdParams p) {
  constexpr int NC = HD / 8, LANES = delta_lanes(HD);
  const int c = (int)(threadIdx.x & (LANES - 1));
  const int64_t row = (int64_t)blockIdx.x * (256 / LANES) + threadIdx.x / LANES;
  const int64_t n_rows = (int64_t)p.B * p.n_live * p.T;
  float acc = 0.f;
  if (row < n_rows && c < NC) {
    const int i = (int)(row % p.T);
    const int bs = (int)(row / p.T);
    const int b = bs / p.n_live, slot = bs % p.n_live;
    const int h = p.out_head[slot];
    const T* o = reinterpret_cast<const T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh + (int64_t)i * p.o_st;
    const T* d = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh + (int64_t)i * p.do_st;
    const uint4 a = load16(o + 8 * c), e = load16(d + 8 * c);
    const uint32_t wa[4] = {a.x, a.y, a.z, a.w}, we[4] = {e.x, e.y, e.z, e.w};
#pragma unroll
    for (int m = 0; m < 4; ++m)
      acc += Elem<T>::lo(wa[m]) * Elem<T>::lo(we[m]) + Elem<T>::hi(wa[m]) * Elem<T>::hi(we[m]);
  }
  // the lanes of a row are an aligned group of the wave (all in or all out of range)
#pragma unroll
  for (int m = LANES / 2; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, LANES);
  if (row < n_rows && c == 0) p.delta[row] = acc;
}

// dQ of the live heads.  Workgroup = 4 waves x 32 queries of one (batch,
// live slot); key blocks of 64 up to the diagonal.  Per 32-key sub-block a
// wave forms S^T = K Q^T and dP^T = V dO^T (keys in the kperm row order, so
// register i of lane-half g is key acc_key(i, g)), P^T = 2^(S^T c - lse),
// dS^T = P^T (dP^T - delta), and accumulates dQ^T += K^T dS^T (K^T from
// transposing tile reads).  K and V tiles arrive by DMA into static slots with
// counted waits and a bare barrier per block, as in the dK/dV kernel below:
// up to hd 64 two blocks ahead in three slots; above, one block ahead in two
// (three 32 KB slot pairs would leave one workgroup per CU: hd 128 dQ 610 ->
// 840 us).
template <typename T, int HD>
__global__ __launch_bounds__(256) void bwd_dq_kernel(const BwdParams p) {
  constexpr int BM = kBwdWaves * 32, NKT = HD / 16, NDT = HD / 32, VB = VRow<HD>::BYTES;
  constexpr int NS = HD <= 64 ? 3 : 2, AHEAD = NS - 1;
  constexpr int kOps = 2 * TileOffsets<T, HD>::VN;  // loads per wave per block
  __shared__ __align__(16) char k0[VB], k1[VB], k2[NS == 3 ? VB : 16], v0[VB], v1[VB], v2[NS == 3 ? VB : 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int T_len = p.T;
  const int nbh = p.B * p.n_live;
  const int n_qb = (T_len + BM - 1) / BM;
  const int r = blockIdx.x % nbh;
  const int qb = n_qb - 1 - (int)(blockIdx.x / nbh);  // heaviest first
  const int b = r / p.n_live, slot = r % p.n_live;
  const int h = p.out_head[slot], qs = p.q_head[slot];
  const T* qbase = reinterpret_cast<const T*>(p.q) + b * p.q_sb + (int64_t)qs * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.k_sb + (int64_t)qs * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)h * p.v_sh;
  const T* dobase = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh;
  T* dqbase = reinterpret_cast<T*>(p.dq) + b * p.dq_sb + (int64_t)qs * p.dq_sh;

  const int q0w = qb * BM + wave * 32;
  const int q = q0w + n;
  const bool qv = q < T_len;
  uint4 qf[NKT], dof[NKT];
#pragma unroll
  for (int t = 0; t < NKT; ++t) {
    qf[t] = qv ? load16(qbase + (int64_t)q * p.q_st + 16 * t + 8 * g) : make_uint4(0, 0, 0, 0);
    dof[t] = qv ? load16(dobase + (int64_t)q * p.do_st + 16 * t + 8 * g) : make_uint4(0, 0, 0, 0);
  }
  const float lse2 = qv ? p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)q * p.l_st] : 0.f;
  const float dl = qv ? p.delta[((int64_t)b * p.n_live + slot) * T_len + q] : 0.f;
  const float c = p.scale_log2;
  f32x16_t dqa[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dqa[dt] = zero16();

  TileOffsets<T, HD> ko, vo;
  ColOffsets<HD> cof;
  cof.init(lane);
  ko.init(wave, lane, p.k_st);
  vo.init(wave, lane, p.v_st);
  const int nkb = (min(qb * BM + BM, T_len) + 63) / 64;

  auto load_block = [&](int j, auto slotc) {
    constexpr int S = decltype(slotc)::value;
    const int lim = j < nkb ? T_len : 0;  // past the last block: an empty descriptor
    ko.load(kbase, p.k_st, 64 * j, lim, S == 0 ? k0 : (S == 1 ? k1 : k2), wave);
    vo.load(vbase, p.v_st, 64 * j, lim, S == 0 ? v0 : (S == 1 ? v1 : v2), wave);
  };
  auto meet = [&]() {  // the next block has landed (with three slots the one after stays in flight)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm((AHEAD - 1) * kOps));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  auto block = [&](const int j, auto phase) {
    constexpr int R = decltype(phase)::value;
    const char* const kt = R == 0 ? k0 : (R == 1 ? k1 : k2);
    const char* const vt = R == 0 ? v0 : (R == 1 ? v1 : v2);
    load_block(j + AHEAD, std::integral_constant<int, (R + AHEAD) % NS>());
    if (64 * j <= q0w + 31) {  // else every key of the block is past this wave's queries
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int row = 32 * ks + kperm(n);
        f32x16_t s = zero16(), dp = zero16();
#pragma unroll
        for (int t = 0; t < NKT; ++t) s = Elem<T>::mfma(tile_row_op<HD>(kt, row, 2 * t + g), qf[t], s);
#pragma unroll
        for (int t = 0; t < NKT; ++t) dp = Elem<T>::mfma(tile_row_op<HD>(vt, row, 2 * t + g), dof[t], dp);
        uint32_t w[8];
        // dS = P (dP - delta); a sub-block with every key at or below every
        // query of the wave (and every query < T) skips the per-element mask
        // through a uniform branch; masked scores go through exp2(-inf) = 0
        auto ds_pack = [&](auto masked) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float ds2[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
              const int i = 2 * e + u;
              float x = s[i] * c - lse2;
              if constexpr (decltype(masked)::value) {
                const int key = 64 * j + 32 * ks + acc_key(i, g);
                x = (qv && key <= q) ? x : -__builtin_inff();
              }
              ds2[u] = fast_exp2(x) * (dp[i] - dl);
            }
            w[e] = Elem<T>::pack2(ds2[0], ds2[1]);
          }
        };
        if (64 * j + 32 * ks + 31 <= q0w && q0w + 31 < T_len)
          ds_pack(std::false_type());
        else
          ds_pack(std::true_type());
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const uint4 bop = make_uint4(w[4 * s2], w[4 * s2 + 1], w[4 * s2 + 2], w[4 * s2 + 3]);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt)
            dqa[dt] = Elem<T>::mfma(tile_col_op<HD>(kt, 2 * ks + s2, dt, cof), bop, dqa[dt]);
        }
      }
    }
    meet();  // block j+1 has landed and slot R is read
  };

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  load_block(0, S0());
  if constexpr (NS == 3) load_block(1, S1());
  meet();
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2 % NS>;
  for (int j = 0;;) {
    if (j >= nkb) break;
    block(j++, P0());
    if (j >= nkb) break;
    block(j++, P1());
    if constexpr (NS == 3) {
      if (j >= nkb) break;
      block(j++, P2());
    }
  }
  // the last (empty) DMAs land before the workgroup's LDS is released
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  if (qv) store_out_tile<T, HD>(dqbase + (int64_t)q * p.dq_st, dqa, p.sm_scale, g);
}

// Waves per SIMD of the dK/dV kernel: its accumulators, K / V rows and three
// pipeline slots fit three waves only up to hd 32 (at hd 64 three waves spilled
// 59 registers and ran 1.8x slower than two).
constexpr int dkdv_waves_per_eu(int hd) { return hd <= 32 ? 3 : (hd <= 64 ? 2 : 1); }

template <typename T, int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(dkdv_waves_per_eu(HD), dkdv_waves_per_eu(HD))))
void bwd_dkdv_kernel(const BwdParams p) {
  constexpr int BN = kBwdWaves * 32, NKT = HD / 16, NDT = HD / 32, VB = VRow<HD>::BYTES;
  constexpr int kOps = 2 * TileOffsets<T, HD>::VN + 1;  // loads per wave per block
  constexpr bool kBatch = dkdv_waves_per_eu(HD) == 1;
  __shared__ __align__(16) char q0[VB], q1[VB], q2[VB], o0[VB], o1[VB], o2[VB];
  __shared__ __align__(16) float ls0[4][64], ls1[4][64], ls2[4][64];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int T_len = p.T;
  const int nbh = p.B * p.n_live;
  const int r = blockIdx.x % nbh;
  const int kb = (int)(blockIdx.x / nbh);  // heaviest (most queries) first
  const int b = r / p.n_live, slot = r % p.n_live;
  const int h = p.out_head[slot], qs = p.q_head[slot];
  const T* qbase = reinterpret_cast<const T*>(p.q) + b * p.q_sb + (int64_t)qs * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.k_sb + (int64_t)qs * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)h * p.v_sh;
  const T* dobase = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh;
  const float* lsebase = p.lse + b * p.l_sb + (int64_t)h * p.l_sh;
  const float* dlbase = p.delta + ((int64_t)b * p.n_live + slot) * T_len;
  T* dkbase = reinterpret_cast<T*>(p.dk) + b * p.dk_sb + (int64_t)qs * p.dk_sh;
  T* dvbase = reinterpret_cast<T*>(p.dv) + b * p.dv_sb + (int64_t)h * p.dv_sh;

  const int k0w = kb * BN + wave * 32;
  const int kk = k0w + n;
  const bool kv = kk < T_len;
  uint4 kf[NKT], vf[NKT];
#pragma unroll
  for (int t = 0; t < NKT; ++t) {
    kf[t] = kv ? load16(kbase + (int64_t)kk * p.k_st + 16 * t + 8 * g) : make_uint4(0, 0, 0, 0);
    // -V: the dP chain starts from delta, so it ends at delta - dP
    vf[t] = kv ? neg_halves(load16(vbase + (int64_t)kk * p.v_st + 16 * t + 8 * g)) : make_uint4(0, 0, 0, 0);
  }
  const float c = p.scale_log2;
  f32x16_t dka[NDT], dva[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dka[dt] = zero16();
    dva[dt] = zero16();
  }

  TileOffsets<T, HD> qo, oo;
  ColOffsets<HD> cof;
  cof.init(lane);
  qo.init(wave, lane, p.q_st);
  oo.init(wave, lane, p.do_st);
  const int ib0 = (kb * BN) / 64, nqb = (T_len + 63) / 64;
  const bool lse_wave = wave < 2;
  const uint32_t ls_off =
      lane < 32 ? (uint32_t)((int64_t)(32 * (wave & 1) + lane) * (lse_wave ? p.l_st : 1) * 4) : 0x80000000u;

  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  auto load_block = [&](int i, auto slotc) {
    constexpr int S = decltype(slotc)::value;
    char* const qt = S == 0 ? q0 : (S == 1 ? q1 : q2);
    char* const ot = S == 0 ? o0 : (S == 1 ? o1 : o2);
    float(*const lt)[64] = S == 0 ? ls0 : (S == 1 ? ls1 : ls2);
    const int lim = i < nqb ? T_len : 0;  // past the last block: an empty descriptor
    qo.load(qbase, p.q_st, 64 * i, lim, qt, wave);
    oo.load(dobase, p.do_st, 64 * i, lim, ot, wave);
    const __amdgpu_buffer_rsrc_t lr =
        lse_wave ? rows_rsrc(lsebase, p.l_st, 64 * i, lim) : rows_rsrc(dlbase, (int64_t)1, 64 * i, lim);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(lr, SAF_LDS_PTR(&lt[wave][0]), 4, ls_off, 0, 0, 0);
  };
  auto meet = [&]() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(kOps));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  auto block = [&](const int i, auto phase) {
    constexpr int R = decltype(phase)::value;
    const char* const qt = R == 0 ? q0 : (R == 1 ? q1 : q2);
    const char* const ot = R == 0 ? o0 : (R == 1 ? o1 : o2);
    float(*const ls)[64] = R == 0 ? ls0 : (R == 1 ? ls1 : ls2);
    load_block(i + 2, std::integral_constant<int, (R + 2) % 3>());
#pragma unroll
    for (int qs2 = 0; qs2 < 2; ++qs2) {
      const int qbase_row = 64 * i + 32 * qs2;
      if (qbase_row + 31 < k0w) continue;  // every query of the sub-block precedes this wave's keys
      const int row = 32 * qs2 + kperm(n);
      // dp starts from the delta of each element's query and ends at delta - dP
      f32x16_t s = zero16(), dp;
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) dp[i2] = ls[2 + qs2][acc_key(i2, g)];
      uint4 co[2][NDT], cq[2][NDT];  // column operands of the dV / dK products (kBatch)
      if constexpr (kBatch) {
        // one wave per SIMD: no other wave covers the LDS latency, so the
        // row operands are read in one batch before the S / dP MFMAs and the
        // column operands before the softmax VALU work (the scheduler keeps
        // each read next to its MFMA otherwise)
        uint4 qa[NKT], oa[NKT];
#pragma unroll
        for (int t = 0; t < NKT; ++t) {
          qa[t] = tile_row_op<HD>(qt, row, 2 * t + g);
          oa[t] = tile_row_op<HD>(ot, row, 2 * t + g);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int t = 0; t < NKT; ++t) {
          s = Elem<T>::mfma(qa[t], kf[t], s);
          dp = Elem<T>::mfma(oa[t], vf[t], dp);
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            co[s2][dt] = tile_col_op<HD>(ot, 2 * qs2 + s2, dt, cof);
            cq[s2][dt] = tile_col_op<HD>(qt, 2 * qs2 + s2, dt, cof);
          }
        __builtin_amdgcn_sched_barrier(0);
      } else {
#pragma unroll
        for (int t = 0; t < NKT; ++t) s = Elem<T>::mfma(tile_row_op<HD>(qt, row, 2 * t + g), kf[t], s);
#pragma unroll
        for (int t = 0; t < NKT; ++t) dp = Elem<T>::mfma(tile_row_op<HD>(ot, row, 2 * t + g), vf[t], dp);
      }
      uint32_t pw[8], dw[8];
      // a sub-block with every query at or past every key of the wave (all
      // valid) skips the per-element mask through a uniform branch; query
      // acc_key(i2, g) of sub-block qs2 has its lse in row qs2 of the slot's
      // statistics and its delta in row 2 + qs2
      auto p_ds_pack = [&](auto masked) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float pr2[2], ds2[2];
#pragma unroll
          for (int u = 0; u < 2; ++u) {
            const int i2 = 2 * e + u;
            const int ql = acc_key(i2, g);  // query within the sub-block
            float x = s[i2] * c - ls[qs2][ql];
            if constexpr (decltype(masked)::value) {
              const int qq = qbase_row + ql;
              x = (kv && qq >= kk && qq < T_len) ? x : -__builtin_inff();
            }
            const float pr = fast_exp2(x);
            pr2[u] = pr;
            ds2[u] = pr * -dp[i2];
          }
          pw[e] = Elem<T>::pack2(pr2[0], pr2[1]);
          dw[e] = Elem<T>::pack2(ds2[0], ds2[1]);
        }
      };
      if (qbase_row >= k0w + 31 && k0w + 31 < T_len && qbase_row + 31 < T_len)
        p_ds_pack(std::false_type());
      else
        p_ds_pack(std::true_type());
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const uint4 bp = make_uint4(pw[4 * s2], pw[4 * s2 + 1], pw[4 * s2 + 2], pw[4 * s2 + 3]);
        const uint4 bd = make_uint4(dw[4 * s2], dw[4 * s2 + 1], dw[4 * s2 + 2], dw[4 * s2 + 3]);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          dva[dt] = Elem<T>::mfma(kBatch ? co[s2][dt] : tile_col_op<HD>(ot, 2 * qs2 + s2, dt, cof), bp, dva[dt]);
          dka[dt] = Elem<T>::mfma(kBatch ? cq[s2][dt] : tile_col_op<HD>(qt, 2 * qs2 + s2, dt, cof), bd, dka[dt]);
        }
      }
    }
    meet();  // block i+1 has landed (block i+2 stays in flight) and slot R is read
  };

  if (ib0 < nqb) {
    load_block(ib0, S0());
    load_block(ib0 + 1, S1());
    meet();
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    for (int i = ib0;;) {
      if (i >= nqb) break;
      block(i++, P0());
      if (i >= nqb) break;
      block(i++, P1());
      if (i >= nqb) break;
      block(i++, P2());
    }
    // the last (empty) DMAs land before the workgroup's LDS is released
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  if (kv) {
    store_out_tile<T, HD>(dkbase + (int64_t)kk * p.dk_st, dka, p.sm_scale, g);
    store_out_tile<T, HD>(dvbase + (int64_t)kk * p.dv_st, dva, 1.f, g);
  }
}

// dV of the frozen heads: dV[j] = sum_{i >= j} P[i, j] dO[i].  Workgroup =
// 4 waves x 32 keys of one (batch, frozen slot); query blocks of 64 from the
// diagonal.  The B operand of dV^T += dO^T P is a column of P for 8
// consecutive queries: gathered from the dense pattern (rounded to the
// activation dtype) or rebuilt as P[i, j] = 2^((alpha_j + rho_{i-j} - z_i)
// log2 e) for decomposed heads (closed-form heads included); cells with
// i < j or i >= T are zero.
//
// dO tiles arrive by DMA two blocks ahead in three static LDS slots (an
// empty descriptor past the last block, so every block issues the same
// loads); a decomposed block's z and rho window is loaded into registers one
// block ahead, before that DMA, and written into the next block's slot.  The
// block ends with a counted wait (the DMA two ahead stays in flight) and a
// bare barrier: one barrier per block instead of two draining ones.
template <typename T, int HD, int KIND>
__global__ __launch_bounds__(256) void bwd_frozen_dv_kernel(const BwdParams p) {
  constexpr int BN = kBwdWaves * 32, NDT = HD / 32, VB = VRow<HD>::BYTES;
  constexpr int VN = TileOffsets<T, HD>::VN;  // DMA loads per wave per dO tile
  __shared__ __align__(16) char o0[VB], o1[VB], o2[VB];
  // decomposed heads: z_q log2 e of the block's 64 queries and rho_d log2 e
  // for every distance d = q - key the block meets (64 + 128 - 1 values)
  __shared__ float zs3[3][64], rs3[3][64 + BN];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int T_len = p.T;
  const int nbf = p.B * p.n_frozen;
  const int r = blockIdx.x % nbf;
  const int kb = (int)(blockIdx.x / nbf);
  const int b = r / p.n_frozen, fs = r % p.n_frozen;
  if (p.f_kind[fs] != KIND) return;
  const int h = p.f_head[fs], ph = p.pat_head[fs];
  const T* dobase = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh;
  T* dvbase = reinterpret_cast<T*>(p.dv) + b * p.dv_sb + (int64_t)h * p.dv_sh;
  const int k0w = kb * BN + wave * 32;
  const int kk = k0w + n;
  const bool kv = kk < T_len;
  float alpha_k = 0.f;
  if (KIND == 2 && kv) alpha_k = load_as_f32(p.alpha, (int64_t)ph * p.a_sh + (int64_t)kk * p.a_ss, p.a_dtype) * kLog2e;
  f32x16_t dva[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dva[dt] = zero16();

  TileOffsets<T, HD> oo;
  oo.init(wave, lane, p.do_st);
  ColOffsets<HD> cof;
  cof.init(lane);
  const int ib0 = (kb * BN) / 64, nqb = (T_len + 63) / 64;
  auto z_of = [&](int qq) {
    return qq < T_len ? load_as_f32(p.z, (int64_t)ph * p.z_sh + (int64_t)qq * p.z_ss, p.z_dtype) * kLog2e : 0.f;
  };
  auto rho_of = [&](int dd) {
    return (dd >= 0 && dd < T_len)
               ? load_as_f32(p.rho, (int64_t)ph * p.r_sh + (int64_t)dd * p.r_ss, p.r_dtype) * kLog2e
               : 0.f;
  };
  // the next block's values as raw bits: converted where they are written,
  // so the wait for them falls there too
  // Every thread loads (from a clamped index) so that every wave issues the
  // same loads and the counted waits hold; values out of range are dropped.
  auto z_bits = [&](int qq) {
    const uint32_t w = load_bits(p.z, (int64_t)ph * p.z_sh + (int64_t)min(max(qq, 0), T_len - 1) * p.z_ss, p.z_dtype);
    return qq < T_len ? w : 0u;
  };
  auto rho_bits = [&](int dd) {
    const uint32_t w = load_bits(p.rho, (int64_t)ph * p.r_sh + (int64_t)min(max(dd, 0), T_len - 1) * p.r_ss, p.r_dtype);
    return (dd >= 0 && dd < T_len) ? w : 0u;
  };
  auto dmin_of = [&](int i) { return 64 * i - kb * BN - (BN - 1); };  // smallest q - key of block i
  auto load_do = [&](int i, auto slotc) {
    constexpr int S = decltype(slotc)::value;
    oo.load(dobase, p.do_st, 64 * i, i < nqb ? T_len : 0, S == 0 ? o0 : (S == 1 ? o1 : o2), wave);
  };
  auto meet = [&]() {  // the next block's dO tile has landed (the one after stays in flight)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(VN));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  auto block = [&](const int i, auto phase) {
    constexpr int R = decltype(phase)::value;
    const char* const ot = R == 0 ? o0 : (R == 1 ? o1 : o2);
    const float* const zs = zs3[R];
    const float* const rs = rs3[R];
    const int dmin = dmin_of(i);
    // the next block's z / rho, then the dO tile two blocks ahead: waiting
    // for the register loads leaves that DMA in flight
    uint32_t nz = 0u, nr = 0u;
    if (KIND == 2) {
      nz = z_bits(64 * (i + 1) + min(tid, 63));
      nr = rho_bits(dmin + 64 + min(tid, 64 + BN - 2));
    }
    asm volatile("" ::: "memory");
    load_do(i + 2, std::integral_constant<int, (R + 2) % 3>());
    asm volatile("" ::: "memory");
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int q0 = 64 * i + 16 * ks;
      if (q0 + 15 < k0w) continue;  // every query of the step precedes this wave's keys
      // B operand: P[q0 + 8g + e, kk] for e = 0..7, in the activation dtype;
      // a step with every query at or past every key of the wave (all
      // valid) skips the per-element mask through a uniform branch
      float e8[8];
      auto p_col = [&](auto masked) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int qq = q0 + 8 * g + e;
          const bool ok = !decltype(masked)::value || (kv && qq >= kk && qq < T_len);
          float v = 0.f;
          if (KIND == 1) {
            if (ok)
              v = load_as_f32(p.patt, (int64_t)ph * p.p_sh + (int64_t)qq * p.p_si + (int64_t)kk * p.p_sj,
                              p.patt_dtype);
          } else {
            // every (query, key) pair of the block indexes inside the staged
            // rho window and z row, so the reads need no guard; masked pairs
            // take exp2(-inf) = 0
            const float x = alpha_k + rs[qq - kk - dmin] - zs[qq - 64 * i];
            v = fast_exp2(ok ? x : -__builtin_inff());
          }
          e8[e] = v;
        }
      };
      if (q0 >= k0w + 31 && k0w + 31 < T_len && q0 + 15 < T_len)
        p_col(std::false_type());
      else
        p_col(std::true_type());
      const uint4 bop = make_uint4(Elem<T>::pack2(e8[0], e8[1]), Elem<T>::pack2(e8[2], e8[3]),
                                   Elem<T>::pack2(e8[4], e8[5]), Elem<T>::pack2(e8[6], e8[7]));
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) dva[dt] = Elem<T>::mfma(tile_col_op<HD>(ot, ks, dt, cof), bop, dva[dt]);
    }
    if (KIND == 2) {  // the next block's slot was last read two blocks ago
      constexpr int RN = (R + 1) % 3;
      if (tid < 64) zs3[RN][tid] = bits_to_f32(nz, p.z_dtype) * kLog2e;
      if (tid < 64 + BN - 1) rs3[RN][tid] = bits_to_f32(nr, p.r_dtype) * kLog2e;
    }
    meet();
  };

  if (ib0 < nqb) {
    if (KIND == 2) {
      if (tid < 64) zs3[0][tid] = z_of(64 * ib0 + tid);
      if (tid < 64 + BN - 1) rs3[0][tid] = rho_of(dmin_of(ib0) + tid);
    }
    asm volatile("" ::: "memory");
    load_do(ib0, std::integral_constant<int, 0>());
    load_do(ib0 + 1, std::integral_constant<int, 1>());
    meet();
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    for (int i = ib0;;) {
      if (i >= nqb) break;
      block(i++, P0());
      if (i >= nqb) break;
      block(i++, P1());
      if (i >= nqb) break;
      block(i++, P2());
    }
    // the last (empty) DMAs land before the workgroup's LDS is released
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
  if (kv) store_out_tile<T, HD>(dvbase + (int64_t)kk * p.dv_st, dva, 1.f, g);
}

// Parameter gradients of decomposed frozen heads (trainable alpha / rho,
// supplement/trainable_pattern_kernels.py:20-56 of the reference): with
// P[i, j] = exp(alpha_j + rho_{i-j} - z_i) the softmax of alpha + rho over
// j <= i, dP = dO V^T and delta_i = dO_i . O_i,
//   dS[i, j] = P[i, j] (dP[i, j] - delta_i),
//   dalpha[h, j] += sum_i dS[i, j],   drho[h, d] += sum_{i - j = d} dS[i, j]
// (z's own dependence on alpha and rho is inside the softmax derivative).
// Workgroup = 4 waves x 32 keys of one (batch, decomposed slot); query blocks
// of 64 from the diagonal to T (dO tiles double-buffered in LDS by DMA, the
// block's z, delta and rho window staged in LDS).  Per 32-query sub-block a
// wave forms dP = dO V^T with the queries in the kperm row order (the lane is
// the key, register i of lane-half g is query acc_key(i, g)), rebuilds P and
// forms dS; dalpha accumulates per lane over every block and goes out with one
// atomic add per key; drho goes through a ring of 256 LDS accumulators indexed
// by distance (ds_add_f32): the distances a block can reach form a window of
// 64 + 128 - 1 that slides by 64 per block, so after each block the 64
// distances no later block reaches are added to drho (global atomics) and
// their slots cleared.
template <typename T, int HD>
__global__ __launch_bounds__(256) void bwd_decomp_param_kernel(const BwdParams p) {
  constexpr int BN = kBwdWaves * 32, NKT = HD / 16, VB = VRow<HD>::BYTES;
  constexpr int RING = 256;
  static_assert(RING >= 64 + BN - 1 + 64, "the distance ring must hold a block's window and the lag");
  __shared__ __align__(16) char o0[VB], o1[VB];
  __shared__ float zd0[128], zd1[128];        // z log2 e (0..63) and delta (64..127) of the block's queries
  __shared__ float rs0[64 + BN], rs1[64 + BN];  // rho log2 e for the block's distances
  __shared__ float ring[RING];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;
  const int T_len = p.T;
  const int nbh = p.B * p.n_live;               // slots here are the decomposed heads
  const int r = blockIdx.x % nbh;
  const int kb = (int)(blockIdx.x / nbh);       // heaviest (most queries) first
  const int b = r / p.n_live, slot = r % p.n_live;
  const int h = p.out_head[slot], ph = p.pat_head[slot];
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)h * p.v_sh;
  const T* dobase = reinterpret_cast<const T*>(p.dout) + b * p.do_sb + (int64_t)h * p.do_sh;
  const float* dlbase = p.delta + ((int64_t)b * p.n_live + slot) * T_len;

  const int kblo = kb * BN;
  const int k0w = kblo + wave * 32;
  const int kk = k0w + n;
  const bool kv = kk < T_len;
  uint4 vf[NKT];
#pragma unroll
  for (int t = 0; t < NKT; ++t)
    vf[t] = kv ? load16(vbase + (int64_t)kk * p.v_st + 16 * t + 8 * g) : make_uint4(0, 0, 0, 0);
  const float alpha_k =
      kv ? load_as_f32(p.alpha, (int64_t)ph * p.a_sh + (int64_t)kk * p.a_ss, p.a_dtype) * kLog2e : 0.f;
  auto z_of = [&](int qq) {
    return qq < T_len ? load_as_f32(p.z, (int64_t)ph * p.z_sh + (int64_t)qq * p.z_ss, p.z_dtype) * kLog2e : 0.f;
  };
  auto rho_of = [&](int dd) {
    return (dd >= 0 && dd < T_len)
               ? load_as_f32(p.rho, (int64_t)ph * p.r_sh + (int64_t)dd * p.r_ss, p.r_dtype) * kLog2e
               : 0.f;
  };
  ring[tid] = 0.f;  // 256 threads, 256 slots

  TileOffsets<T, HD> oo;
  oo.init(wave, lane, p.do_st);
  const int ib0 = kblo / 64, nqb = (T_len + 63) / 64;
  // distances of query block i: [64 i - kblo - (BN - 1), 64 i + 63 - kblo]
  auto dlo_of = [&](int i) { return 64 * i - kblo - (BN - 1); };
  if (ib0 < nqb) {
    oo.load(dobase, p.do_st, 64 * ib0, T_len, o0, wave);
    if (tid < 64) {
      zd0[tid] = z_of(64 * ib0 + tid);
      zd0[64 + tid] = 64 * ib0 + tid < T_len ? dlbase[64 * ib0 + tid] : 0.f;
    }
    if (tid < 64 + BN - 1) rs0[tid] = rho_of(dlo_of(ib0) + tid);
  }
  float dacc = 0.f;
  int flushed = 0;  // distances below this are in drho
  for (int i = ib0; i < nqb; ++i) {
    const char* ot = ((i - ib0) & 1) ? o1 : o0;
    const float* zd = ((i - ib0) & 1) ? zd1 : zd0;
    const float* rs = ((i - ib0) & 1) ? rs1 : rs0;
    const int dmin = dlo_of(i);
    __syncthreads();  // this block's tile and statistics are in LDS (and the ring is cleared)
    float nz = 0.f, ndl = 0.f, nr = 0.f;
    if (i + 1 < nqb) {
      oo.load(dobase, p.do_st, 64 * (i + 1), T_len, ((i - ib0) & 1) ? o0 : o1, wave);
      const int qq = 64 * (i + 1) + tid;
      if (tid < 64) {
        nz = z_of(qq);
        ndl = qq < T_len ? dlbase[qq] : 0.f;
      }
      if (tid < 64 + BN - 1) nr = rho_of(dmin + 64 + tid);
    }
#pragma unroll
    for (int qs2 = 0; qs2 < 2; ++qs2) {
      if (64 * i + 32 * qs2 + 31 < k0w) continue;  // every query of the sub-block precedes this wave's keys
      const int row = 32 * qs2 + kperm(n);
      f32x16_t dp = zero16();
#pragma unroll
      for (int t = 0; t < NKT; ++t) dp = Elem<T>::mfma(tile_row_op<HD>(ot, row, 2 * t + g), vf[t], dp);
#pragma unroll
      for (int i2 = 0; i2 < 16; ++i2) {
        const int ql = 32 * qs2 + acc_key(i2, g);
        const int qq = 64 * i + ql;
        const bool ok = kv && qq >= kk && qq < T_len;
        const float pr = fast_exp2(ok ? alpha_k + rs[qq - kk - dmin] - zd[ql] : -__builtin_inff());
        const float ds = pr * (dp[i2] - zd[64 + ql]);
        dacc += ds;
        if (ok) atomicAdd(&ring[(qq - kk) & (RING - 1)], ds);
      }
    }
    if (tid < 64) {  // the idle slot's readers finished before the previous barrier
      float* zn = ((i - ib0) & 1) ? zd0 : zd1;
      zn[tid] = nz;
      zn[64 + tid] = ndl;
    }
    if (tid < 64 + BN - 1) (((i - ib0) & 1) ? rs0 : rs1)[tid] = nr;
    __syncthreads();  // every wave's ring updates of this block are in; the slot may be refilled
    // distances below the next block's lowest are final
    const int done = i + 1 < nqb ? min(max(dlo_of(i + 1), 0), T_len) : T_len;
    for (int d = flushed + tid; d < done; d += 256) {
      const float x = ring[d & (RING - 1)];
      if (x != 0.f) atomicAdd(p.drho + (int64_t)ph * p.dr_hs + d, x);
      ring[d & (RING - 1)] = 0.f;
    }
    flushed = max(flushed, done);
  }
  dacc = half_swap_sum(dacc);
  if (kv && g == 0 && dacc != 0.f) atomicAdd(p.dalpha + (int64_t)ph * p.da_hs + kk, dacc);
}

// Explicit instantiations: the host pass emits a kernel's launch stub only
// for an explicitly instantiated template here (implicit instantiation from
// the launcher left the dK/dV and frozen-dV stubs undefined).
#define SAF_BWD_INST(T, HD)                                                              \
  template __global__ void bwd_delta_kernel<T, HD>(const BwdParams);                    \
  template __global__ void bwd_dq_kernel<T, HD>(const BwdParams);                       \
  template __global__ void bwd_dkdv_kernel<T, HD>(const BwdParams);                     \
  template __global__ void bwd_frozen_dv_kernel<T, HD, 1>(const BwdParams);             \
  template __global__ void bwd_frozen_dv_kernel<T, HD, 2>(const BwdParams);             \
  template __global__ void bwd_decomp_param_kernel<T, HD>(const BwdParams);
#define SAF_BWD_INST_T(T) SAF_BWD_INST(T, 32) SAF_BWD_INST(T, 64) SAF_BWD_INST(T, 96) SAF_BWD_INST(T, 128)
SAF_BWD_INST_T(__bf16)
SAF_BWD_INST_T(_Float16)
#undef SAF_BWD_INST_T
#undef SAF_BWD_INST

// ---- launchers ---------------------------------------------------------------

template <typename T, int HD>
static hipError_t bwd_launch_hd(const BwdParams& p, int which, hipStream_t s) {
  const int64_t T_len = p.T;
  const int64_t nk = (T_len + 127) / 128;
  switch (which) {
    case 0: {
      const int64_t rows = (int64_t)p.B * p.n_live * T_len;
      const int64_t per_wg = 256 / delta_lanes(HD);
      hipLaunchKernelGGL((bwd_delta_kernel<T, HD>), dim3((unsigned)((rows + per_wg - 1) / per_wg)), dim3(256), 0, s, p);
      break;
    }
    case 1:
      hipLaunchKernelGGL((bwd_dq_kernel<T, HD>), dim3((unsigned)(nk * p.B * p.n_live)), dim3(256), 0, s, p);
      break;
    case 2:
      hipLaunchKernelGGL((bwd_dkdv_kernel<T, HD>), dim3((unsigned)(nk * p.B * p.n_live)), dim3(256), 0, s, p);
      break;
    case 3: {
      const dim3 grid((unsigned)(nk * p.B * p.n_frozen));
      hipLaunchKernelGGL((bwd_frozen_dv_kernel<T, HD, 1>), grid, dim3(256), 0, s, p);
      hipLaunchKernelGGL((bwd_frozen_dv_kernel<T, HD, 2>), grid, dim3(256), 0, s, p);
      break;
    }
    default:
      hipLaunchKernelGGL((bwd_decomp_param_kernel<T, HD>), dim3((unsigned)(nk * p.B * p.n_live)), dim3(256), 0, s,
                         p);
      break;
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t bwd_launch(const BwdParams& p, int hd, int which, hipStream_t s) {
  switch (hd) {
    case 32: return bwd_launch_hd<T, 32>(p, which, s);
    case 64: return bwd_launch_hd<T, 64>(p, which, s);
    case 96: return bwd_launch_hd<T, 96>(p, which, s);
    case 128: return bwd_launch_hd<T, 128>(p, which, s);
    default: return hipErrorInvalidValue;
  }
}

static hipError_t bwd_dispatch(const BwdParams& p, int dtype, int hd, int which, hipStream_t s) {
  if (dtype == kF32) return which <= 3 ? launch_f32_bwd(p, hd, which, s) : hipErrorInvalidValue;
  if (dtype == kBF16) return bwd_launch<__bf16>(p, hd, which, s);
  if (dtype == kF16) return bwd_launch<_Float16>(p, hd, which, s);
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_delta(const BwdParams& p, int dtype, int hd, hipStream_t s) { return bwd_dispatch(p, dtype, hd, 0, s); }
hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int hd, hipStream_t s) { return bwd_dispatch(p, dtype, hd, 1, s); }
hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int hd, hipStream_t s) { return bwd_dispatch(p, dtype, hd, 2, s); }
hipError_t launch_bwd_frozen_dv(const BwdParams& p, int dtype, int hd, hipStream_t s) {
  return bwd_dispatch(p, dtype, hd, 3, s);
}
hipError_t launch_bwd_decomp_param(const BwdParams& p, int dtype, int hd, hipStream_t s) {
  return bwd_dispatch(p, dtype, hd, 4, s);
}

}  // namespace saf
