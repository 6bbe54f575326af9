// Kernel parameter blocks and host-side launchers of the SAF attention
// library.  Everything here is internal to libsafattn.so; the public C-ABI
// lives in include/saf_attn.h.
#pragma once
#include "saf_device.h"

namespace saf {

// Largest number of heads one launch can route (per-head tables are passed
// by value in the kernel arguments).
constexpr int kMaxHeads = 128;

// dtype codes shared with the C-ABI (saf_attn.h)
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2, kI32 = 3 };

// Causal load balancing of the live-head kernel: the per-head work list
// holds (query block, key segment) items, heaviest first; query blocks whose
// key range spans several segments write fp32 partials that a combine kernel
// merges.  Limits keep the parameter block under the 4 KiB kernel-argument
// budget.
constexpr int kMaxItems = 384;
constexpr int kMaxQblk = 256;

// Live heads (state 0).
struct FlashParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;  // may be null
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int64_t l_sb, l_sh, l_st;
  int B, T, n_slots, n_qblk;
  float scale_log2;  // sm_scale * log2(e)
  int16_t out_head[kMaxHeads];
  int16_t q_head[kMaxHeads];
  int16_t k_head[kMaxHeads];
  int16_t v_head[kMaxHeads];
  // work list (n_items == 0: one item per query block, heaviest first)
  int n_items;
  int seg_len;          // key blocks (of 64 keys) per segment
  int n_part_per_head;  // partial slots per (batch, live head)
  float* part_o;        // [bh][part][BM][HD] unnormalised O (fp32)
  float* part_ml;       // [bh][part][2][BM]: running max (base 2), row sum
  int32_t items[kMaxItems];      // (qb << 8) | segment
  int16_t part_base[kMaxQblk];   // first partial slot of a split query block, -1 if not split
  // work queue (null: one workgroup per unit): a word zeroed before the
  // launch, from which the resident workgroups claim their next unit
  unsigned* queue;
  int max_grid;  // with a queue: the resident workgroups (grid = min(units, max_grid))
};

// Merge of split query blocks: out = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s.
struct CombineParams {
  void* out;
  float* lse;
  int64_t o_sb, o_sh, o_st;
  int64_t l_sb, l_sh, l_st;
  int B, T, n_slots, BM, seg_len, n_part_per_head, n_split;
  const float* part_o;
  const float* part_ml;  // null: the partials are plain sums (dense P.V)
  int16_t out_head[kMaxHeads];
  int16_t split_qb[kMaxQblk];    // split query blocks
  int16_t part_base[kMaxQblk];   // indexed by query block
};

// Frozen heads whose pattern is applied as an MFMA P.V product: dense
// patterns (state 1) and decomposed patterns rebuilt in registers (state 2).
struct FrozenParams {
  const void* v;
  void* out;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  // dense pattern buffer (P, S, S) and its dtype code
  const void* patt;
  int patt_dtype;
  int patt_vec;  // rows contiguous and aligned for 16/32-byte loads
  int p_cols;    // S: row length of the pattern buffer
  int64_t p_sh, p_si, p_sj;
  int64_t patt_elems;  // elements from patt to the end of its last row
  // decomposed buffers (H, S) indexed by the natural head
  const void* alpha;
  const void* rho;
  const void* z;
  int a_dtype, r_dtype, z_dtype;
  int64_t a_sh, a_ss, r_sh, r_ss, z_sh, z_ss;
  int B, T, n_slots, n_qblk;
  // decomposed heads, factored form (null: cell-by-cell rebuild only):
  // a_off[slot][k] = max alpha log2 e over 64-key block k of the slot's head
  // (n_slots x ceil(T / 64)), followed by the same layout of maxima of
  // rho log2 e over 64-distance blocks and of minima of z log2 e over 64-row
  // blocks, vp = the key-scaled values 2^(alpha_j log2 e - a_off[slot][j / 64]) v_j,
  // (B, n_slots, T, HD) in the input dtype, r2[slot][d] = rho_d log2 e and
  // z2[slot][i] = z_i log2 e (n_slots x T each) (workspace, all written by
  // launch_decomp_prescale)
  float* a_off;
  void* vp;
  float* r2;
  float* z2;
  // the same key-scaled values in fp16 (vp16, null: no fp16 factored form)
  // and their largest magnitude per (batch, slot, 64-key block) (vmax,
  // B x n_slots x ceil(T / 64)): the fp16 form needs every |V'| it reads
  // below the fp16 range limit
  void* vp16;
  float* vmax;
  int16_t out_head[kMaxHeads];
  int16_t v_head[kMaxHeads];
  int16_t pat_head[kMaxHeads];  // dense: pattern row; decomposed: buffer row
  // dense P.V causal balance (as FlashParams): work items (qb << 8) | seg,
  // fp32 partials of split query blocks summed by the combine kernel;
  // n_items == 0: one item per query block, heaviest first
  int n_items, seg_len, n_part_per_head;
  float* part_o;
  int32_t items[kMaxItems];
  int16_t part_base[kMaxQblk];
};
static_assert(sizeof(FrozenParams) <= 4096, "FrozenParams must fit the kernel argument segment");
static_assert(offsetof(FrozenParams, out_head) % 4 == 0 && offsetof(FrozenParams, v_head) % 4 == 0 &&
                  offsetof(FrozenParams, pat_head) % 4 == 0,
              "the head tables are read as aligned 32-bit words (arg_i16)");

// Closed-form frozen heads (state 2 heads recognised as causal mean,
// exponential decay or sliding window): a single-pass chunked scan along T
// with decoupled look-back between chunks (workgroup g = chunk g / n_seq of
// sequence g % n_seq).
enum : int { kScanMean = 1, kScanDecay = 2, kScanWindow = 3 };

struct ScanParams {
  const void* v;
  void* out;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int B, T, n_slots, n_chunks;
  uint32_t* error;  // set to 1 if a look-back wait hit the spin limit
  // [n_seq][n_chunks][HD] status words (tag << 32 | fp32 bits), zeroed before
  // launch: tag 1 = chunk aggregate, 2 = inclusive prefix
  uint64_t* status;
  int spin_limit;
  int16_t out_head[kMaxHeads];
  int16_t v_head[kMaxHeads];
  int8_t kind[kMaxHeads];
  float param[kMaxHeads];  // decay rate (> 0) or window length
};

// In-place rotary embedding of the live-head q and k.
struct RopeParams {
  void* q;
  void* k;
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  const void* cos;
  const void* sin;
  int64_t cs_st, sn_st;  // row strides of the (T', hd) caches
  int cs_dtype;
  int B, Uq, Uk, T, hd;
  // optional per-head RMSNorm of q and k before the rotation (null: none)
  const void* q_w;
  const void* k_w;
  int w_dtype;
  float eps;
};

// Residual add + LayerNorm of (rows, C) activations: x += delta (when
// present), y = LayerNorm(x) * w + b.
struct AddLnParams {
  void* x;
  const void* delta;  // may be null: plain LayerNorm of x
  void* y;
  const void* w;
  const void* b;      // may be null
  int64_t rows, C;
  int64_t x_rs, d_rs, y_rs;  // row strides in elements
  float eps;
  int wb_dtype;
  // C % 256 == 0, every row and the weight / bias 16-byte aligned: the
  // half-wave-per-row kernel with 16-byte pieces
  int vec16;
  // every row and the weight / bias 16-byte aligned (any C): 16-byte chunks
  // when C % 8 == 0
  int vec16_rows;
  // RMSNorm instead (Qwen3RMSNorm): y = w * round(x * rsqrt(mean(x^2) + eps)),
  // no centring, no bias, the normalised x rounded to the activation dtype
  // before the weight multiplies it and the product rounded again
  int rms;
};

// Projection GEMMs with a fused epilogue: c = epi(a w^T) for (M, K)
// activations a, (N, K) weight w and (M, N) output c, row-major with unit
// column stride; N a multiple of 256, K of 128 (any M).  The epilogue is the
// exact GELU (MLP up-projection) or the rotary embedding of the first n_rope
// columns (the live heads' q and k of the QKV projection, head dim hd,
// position t = row mod T, cos / sin caches (>= T, hd) in the activation
// dtype with row strides cs_st / sn_st in elements).
struct ProjGemmParams {
  const void* a;
  const void* w;
  void* c;
  int M, N, K;
  int a_rs, w_rs, c_rs;  // row strides in elements
  int n_cu;              // compute units of the device (persistent workgroups)
  int n_rope, hd, T;
  const void* cos;
  const void* sin;
  int64_t cs_st, sn_st;
};

// Rows of one scan chunk for a head dimension (must match ScanShape in the
// kernel): 8 rows per thread, 32 KB of V per chunk for hd 64 / 128.
inline int scan_chunk_rows(int hd) { return hd == 32 ? 512 : (hd == 64 ? 256 : 128); }

// Launchers: return hipSuccess or the launch error.  dtype is kBF16 / kF16.
hipError_t launch_flash(const FlashParams& p, int dtype, int hd, int qt, hipStream_t s);
hipError_t launch_flash_combine(const CombineParams& p, int dtype, int hd, hipStream_t s);
hipError_t launch_frozen_pv(const FrozenParams& p, int dtype, int hd, int mode, hipStream_t s);
// Factored decomposed heads: a_off and the key-scaled values vp in one launch
// (bf16, hd <= 128).
hipError_t launch_decomp_prescale(const FrozenParams& p, int dtype, int hd, hipStream_t s);
hipError_t launch_scan(const ScanParams& p, int dtype, int hd, hipStream_t s);
hipError_t launch_zero_u32(uint32_t* ptr, int64_t n, hipStream_t s);
hipError_t launch_rope(const RopeParams& p, int dtype, hipStream_t s);
hipError_t launch_add_layernorm(const AddLnParams& p, int dtype, hipStream_t s);
bool proj_gemm_shape_ok(int64_t M, int64_t N, int64_t K);
// exact GELU in place over n elements (n % 8 == 0, 16-byte aligned)
hipError_t launch_gelu_inplace(void* x, int64_t n, int dtype, int n_cu, hipStream_t s);
hipError_t launch_gemm_gelu(const ProjGemmParams& p, int dtype, hipStream_t s);
hipError_t launch_gemm_rope(const ProjGemmParams& p, int dtype, hipStream_t s);
// SwiGLU: w holds 64-row blocks of gate and up rows in turn; c is (M, N / 2)
hipError_t launch_gemm_swiglu(const ProjGemmParams& p, int dtype, hipStream_t s);

// Row normalisers of decomposed patterns, z[h, i] = logsumexp_{j<=i}(alpha[h, j]
// + rho[h, i - j]) for i < S; (H, S) fp32 rows with unit column stride.
struct LogzParams {
  const float* alpha;
  const float* rho;
  float* z;
  int64_t a_hs, r_hs, z_hs;  // head (row) strides, elements
  int H, S;
};

hipError_t launch_decomp_logz(const LogzParams& p, hipStream_t s);

// Backward of the row normalisers: dalpha, drho (H, S) fp32 from gz = dL/dz.
struct LogzBwdParams {
  const float* alpha;
  const float* rho;
  const float* z;
  const float* gz;
  float* dalpha;
  float* drho;
  int64_t a_hs, r_hs, z_hs, g_hs, da_hs, dr_hs;
  int H, S;
};

hipError_t launch_decomp_logz_bwd(const LogzBwdParams& p, hipStream_t s);

// Backward of the mixed-head operator (gradients of out = attention(q, k, v)
// with respect to q, k, v; patterns and decomposed buffers are constants).
// Live slots index the compact q/k (q_head) and the natural head (out_head);
// frozen slots list the dense / decomposed heads.
struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* out;
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  const float* lse;  // (B, H, T) base-2 log-sum-exp of the forward
  float* delta;      // (B, n_live, T) workspace: rowsum(out * dout) per live row
  int64_t q_sb, q_sh, q_st;
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t o_sb, o_sh, o_st;
  int64_t do_sb, do_sh, do_st;
  int64_t dq_sb, dq_sh, dq_st;
  int64_t dk_sb, dk_sh, dk_st;
  int64_t dv_sb, dv_sh, dv_st;
  int64_t l_sb, l_sh, l_st;
  int B, T, n_live, n_frozen;
  float scale_log2;  // sm_scale * log2(e)
  float sm_scale;
  int16_t out_head[kMaxHeads];   // live slot -> natural head
  int16_t q_head[kMaxHeads];     // live slot -> compact q/k slot
  // frozen slots
  int16_t f_head[kMaxHeads];     // frozen slot -> natural head
  int16_t pat_head[kMaxHeads];   // dense: pattern row; decomposed: buffer row
  int8_t f_kind[kMaxHeads];      // 1 dense, 2 decomposed
  const void* patt;
  int patt_dtype, patt_vec;
  int64_t p_sh, p_si, p_sj, patt_elems;
  const void* alpha;
  const void* rho;
  const void* z;
  int a_dtype, r_dtype, z_dtype;
  int64_t a_sh, a_ss, r_sh, r_ss, z_sh, z_ss;
  // parameter gradients of decomposed heads (fp32 (H, S), accumulated)
  float* dalpha;
  float* drho;
  int64_t da_hs, dr_hs;
};
static_assert(sizeof(BwdParams) <= 4096, "BwdParams must fit the kernel argument segment");

// Backward: delta = rowsum(out * dout) of the live rows; dQ; dK and dV of the
// live heads; dV of the frozen heads.
hipError_t launch_bwd_delta(const BwdParams& p, int dtype, int hd, hipStream_t s);
hipError_t launch_bwd_dq(const BwdParams& p, int dtype, int hd, hipStream_t s);
hipError_t launch_bwd_dkdv(const BwdParams& p, int dtype, int hd, hipStream_t s);
hipError_t launch_bwd_frozen_dv(const BwdParams& p, int dtype, int hd, hipStream_t s);
// dalpha / drho of the decomposed heads: slots 0..n_live-1 are the decomposed
// heads (out_head = head, pat_head = buffer row), delta of those rows in p.delta.
hipError_t launch_bwd_decomp_param(const BwdParams& p, int dtype, int hd, hipStream_t s);

// float32 inputs (attn_f32.hip): the same parameter blocks, no causal split
// (n_items 0), no work queue; which: 0 delta, 1 dQ, 2 dK / dV, 3 frozen dV.
hipError_t launch_f32_live(const FlashParams& p, int hd, hipStream_t s);
hipError_t launch_f32_frozen(const FrozenParams& p, int hd, int mode, hipStream_t s);
hipError_t launch_f32_bwd(const BwdParams& p, int hd, int which, hipStream_t s);

// Queries per frozen-head workgroup (4 waves) for a query-tile count.
inline int block_rows(int qt) { return 4 * 32 * qt; }

// Dense P.V shape: a workgroup of kDenseWaves waves (two per SIMD, one
// query tile of 32 rows each) serves a group of NB batch elements that share
// every pattern operand, as many as 128 accumulator registers per wave
// allow: 4 at hd <= 64 (batch a multiple of 4), 2 at hd <= 128 (even batch),
// else 1; one workgroup per CU (its three V slots fill most of the LDS at
// hd 128).
constexpr int kDenseWaves = 8;
constexpr int dense_batch_group(int B, int hd) {
  return B % 4 == 0 && hd <= 64 ? 4 : (B % 2 == 0 && hd <= 128 ? 2 : 1);
}
constexpr int dense_qtiles(int, int) { return 1; }
constexpr int dense_block_rows(int, int) { return kDenseWaves * 32; }
constexpr int kDenseResident = 1;

// Waves of a live-head workgroup: 8 for hd 96 / 128 (two per SIMD sharing
// one set of LDS tiles), else 4 (hd 256: one wave per SIMD, whose 512
// registers hold the 32 x 256 O^T accumulators and the Q operands).
constexpr int flash_waves(int hd) { return hd > 64 && hd <= 128 ? 8 : 4; }
// Queries per live-head workgroup.
inline int flash_block_rows(int hd, int qt) { return flash_waves(hd) * 32 * qt; }

}  // namespace saf
