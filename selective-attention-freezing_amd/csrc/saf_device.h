// Device-side building blocks shared by the SAF mixed-head attention kernels
// (gfx950 / CDNA4 only).
//
// Every attention kernel in this library uses the same "transposed" MFMA
// formulation on v_mfma_f32_32x32x16_{bf16,f16}:
//
//   S^T[key][query] = K[key][:] . Q^T[:][query]      (A = K tile from LDS,
//                                                      B = Q held in VGPRs)
//   O^T[d][query]  += V^T[d][key] . P^T[key][query]   (A = V^T tile from LDS,
//                                                      B = P^T in VGPRs)
//
// With a 32x32 accumulator, lane l owns column (l % 32) = one query, and its
// 16 accumulator registers hold 16 rows.  So every per-query quantity of the
// online softmax (running max, running sum, rescale factor) lives in a single
// lane (plus its partner lane l ^ 32), and no cross-lane row reduction is
// needed apart from one swap between the two wave halves.
//
// Lane layout of v_mfma_f32_32x32x16 (A: 32xK16, B: K16x32, C: 32x32):
//   A: lane l holds row (l % 32), k = 8*(l/32) + 0..7       (8 x 16-bit)
//   B: lane l holds col (l % 32), k = 8*(l/32) + 0..7       (8 x 16-bit)
//   C: lane l, reg i holds col (l % 32), row 8*(i/4) + 4*(l/32) + (i%4)
// A k-permutation applied identically to A and B leaves the product
// unchanged, and a row permutation of A permutes the rows of C.  The kernels
// use the latter: A-lane row m of the S^T product is loaded with key
// kperm(m), chosen so that C register i of lane-half g holds key
// 16*(i/8) + 8*g + (i%8).  Registers 8s..8s+7 of a lane are then exactly the
// B operand (keys 16s + 8g + 0..7) of the P.V product, with no shuffles.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace saf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;  // 1 / ln(2)

// Word 3 of a raw gfx9 buffer resource: 32-bit data format, no swizzle.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of buffer stores: non-temporal (streaming) store.
constexpr int kBufferNT = 2;

// ---- element types: bf16 and fp16 storage, fp32 arithmetic -----------------

template <typename T> struct Elem;

template <> struct Elem<__bf16> {
  static constexpr bool is_bf16 = true;
  __device__ static inline f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // two fp32 values -> one dword of two round-to-nearest-even bf16
  __device__ static inline uint32_t pack2(float lo, float hi) {
    bf16x2_t v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline float lo(uint32_t w) { return __uint_as_float(w << 16); }
  __device__ static inline float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  // acc + lo(w) + hi(w) with one v_dot2 (row sums of packed P)
  __device__ static inline float sum2(uint32_t w, float acc) {
    const bf16x2_t one = {(__bf16)1.f, (__bf16)1.f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one, acc, false);
  }
  // acc + the sum of this lane's four values in w (two dwords), on the
  // matrix pipe: in a 4x4x4 MFMA block, lane 4b + j supplies column j of B
  // and receives column j of D, so with an all-ones A every register of the
  // lane's result holds acc + its own four values
  __device__ static inline f32x4_t sum4(uint2 w, f32x4_t acc) {
    const i16x4_t ones = {0x3f80, 0x3f80, 0x3f80, 0x3f80};
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(ones, __builtin_bit_cast(i16x4_t, w), acc, 0, 0, 0);
  }
};

template <> struct Elem<_Float16> {
  static constexpr bool is_bf16 = false;
  __device__ static inline f32x16_t mfma(uint4 a, uint4 b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(
        __builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
  }
  __device__ static inline uint32_t pack2(float lo, float hi) {
    f16x2_t v;
    v[0] = (_Float16)lo;
    v[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
  __device__ static inline float lo(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
  }
  __device__ static inline float hi(uint32_t w) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
  }
  __device__ static inline float sum2(uint32_t w, float acc) {
    const f16x2_t one = {(_Float16)1.f, (_Float16)1.f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), one, acc, false);
  }
  __device__ static inline f32x4_t sum4(uint2 w, f32x4_t acc) {
    const f16x4_t ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
    return __builtin_amdgcn_mfma_f32_4x4x4f16(ones, __builtin_bit_cast(f16x4_t, w), acc, 0, 0, 0);
  }
};

// Pattern / parameter buffers may be stored in fp32, bf16 or fp16; the
// kernels always widen them to fp32 first.
__device__ inline float load_as_f32(const void* p, int64_t idx, int dtype) {
  if (dtype == 0) return reinterpret_cast<const float*>(p)[idx];
  uint16_t bits = reinterpret_cast<const uint16_t*>(p)[idx];
  if (dtype == 2) return __uint_as_float(((uint32_t)bits) << 16);
  return (float)__builtin_bit_cast(_Float16, bits);
}

// load_as_f32 in two halves, so that a caller can place the wait for the
// load at the value's use: the element's raw bits (fp32, or a 16-bit element
// zero-extended), then their value as fp32.
__device__ inline uint32_t load_bits(const void* p, int64_t idx, int dtype) {
  return dtype == 0 ? reinterpret_cast<const uint32_t*>(p)[idx] : (uint32_t)reinterpret_cast<const uint16_t*>(p)[idx];
}
__device__ inline float bits_to_f32(uint32_t bits, int dtype) {
  if (dtype == 0) return __uint_as_float(bits);
  if (dtype == 2) return __uint_as_float(bits << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

__device__ inline f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine a per-lane value with the partner lane l ^ 32 (v_permlane32_swap
// hands each lane both its own and its partner's value, in some order).
__device__ inline float half_swap_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float half_swap_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Maximum of x over the 64 lanes of a wave (every lane active), as a
// wave-uniform value.  GFX9 DPP moves (a few cycles each, no LDS round trip
// as __shfl_xor's ds_bpermute has): lane pairs and quads (quad_perm), then
// 8- and 16-lane rows (row_half_mirror, row_mirror), then lane 15 of rows 0
// and 2 into rows 1 and 3 (row_bcast:15) and lane 31 into rows 2 and 3
// (row_bcast:31), after which lane 63 holds the maximum of all 64.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, ROWMASK, 0xf, false));
}
__device__ inline float wave_max(float x) {
  x = fmaxf(x, dpp_move<0xb1, 0xf>(x));   // quad_perm [1, 0, 3, 2]
  x = fmaxf(x, dpp_move<0x4e, 0xf>(x));   // quad_perm [2, 3, 0, 1]
  x = fmaxf(x, dpp_move<0x141, 0xf>(x));  // row_half_mirror
  x = fmaxf(x, dpp_move<0x140, 0xf>(x));  // row_mirror
  x = fmaxf(x, dpp_move<0x142, 0xa>(x));  // row_bcast:15, rows 1 and 3
  x = fmaxf(x, dpp_move<0x143, 0xc>(x));  // row_bcast:31, rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}
__device__ inline float wave_min(float x) { return -wave_max(-x); }

// Entry i (wave-uniform) of an int16 table in the kernel arguments, read as
// its aligned 32-bit word: the compiler then reads it with a scalar load
// (waited with the other argument reads) instead of a 16-bit vector load
// that the next use has to wait for.  The table must start 4-byte aligned.
__device__ inline int arg_i16(const int16_t* t, int i) {
  const int32_t w = reinterpret_cast<const int32_t*>(t)[i >> 1];
  return (int)(int16_t)(uint32_t)(w >> (16 * (i & 1)));
}

// Row permutation of the S^T product (see header comment).  A-lane row
// m = 8a + 4g + r  loads key 16*(a/2) + 8g + 4*(a%2) + r.
__device__ inline int kperm(int m) {
  const int a = m >> 3, g = (m >> 2) & 1, r = m & 3;
  return 16 * (a >> 1) + 8 * g + 4 * (a & 1) + r;
}

// Key held by accumulator register i of lane-half g (0..31 within a 32-key
// S^T subtile), given the kperm row order above.
__device__ inline int acc_key(int i, int g) { return 16 * (i >> 3) + 8 * g + (i & 7); }

// ---- LDS layouts -------------------------------------------------------------
// K tile: 64 keys x HD, row pitch KCHP 16-byte chunks (KCHP = next pow2 of
// HD/8).  Chunk c of key row `key` is stored at slot c ^ swz(key), swz an
// XOR-linear function of the key's low four bits, chosen (by exhaustive
// search over such functions) so that the ds_read_b128 of one K operand
// (lane (n, g): key kperm(n), chunk 2t + g) is free of bank conflicts both
// in 8-lane groups over 32 banks and in 16-lane groups over 64 banks.
template <int HD> struct KLayout {
  static constexpr int KCH = HD / 8;
  static constexpr int KCHP = KCH <= 4 ? 4 : (KCH <= 8 ? 8 : (KCH <= 16 ? 16 : 32));
  static constexpr int BYTES = 64 * KCHP * 16;
  // XOR masks contributed by key bits 0..3
  static constexpr int M0 = KCHP == 4 ? 0 : 1, M1 = KCHP == 4 ? 1 : 2, M2 = KCHP == 4 ? 1 : (KCHP == 8 ? 1 : 4),
                       M3 = KCHP == 4 ? 2 : (KCHP == 8 ? 4 : 12);
  __device__ static inline int swz(int key) {
    return ((key & 1) ? M0 : 0) ^ ((key & 2) ? M1 : 0) ^ ((key & 4) ? M2 : 0) ^ ((key & 8) ? M3 : 0);
  }
  __device__ static inline int chunk(int key, int c) { return key * KCHP + (c ^ swz(key)); }
};

// V^T tile: HD rows (d) x 64 keys = 8 chunks of 8 keys per row, swizzled so
// that both the transposing 4-byte writes and the 16-byte A-operand reads are
// spread over all banks.
template <int HD> struct VLayout {
  static constexpr int BYTES = HD * 128;
  __device__ static inline int chunk(int d, int kc) {
    return d * 8 + (kc ^ ((d ^ (d >> 3)) & 7));
  }
};

#define SAF_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt
// 6:4, lgkmcnt 11:8): vmcnt <= n alone, and vmcnt <= n with lgkmcnt 0.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }

// V tile: 64 key rows of HD values, row pitch VSEG 32-byte segments.  The
// logical 16-byte chunk c of row r is stored at chunk c ^ swz(r), swz an
// XOR-linear function of the row's low four bits chosen (by exhaustive
// search over such functions) so that both reads of a tile are free of
// bank conflicts, in 8-lane groups over 32 banks and in 16-lane groups over
// 64 banks (32 lanes for the 8-byte reads): ds_read_b64_tr_b16 (the V^T
// operand: rows 8g + 0..3 (+4), two chunks of one column block) and
// ds_read_b128 (a row operand: rows kperm(0..31), one chunk).  hd 256 tiles
// (no row operands: the backward stops at hd 128) take M2 = 0, so a lane's
// second transposing read is its first plus 4 rows and needs no register.
template <int HD> struct VRow {
  static constexpr int VSEG = HD / 16 <= 4 ? 4 : (HD / 16 <= 8 ? 8 : 16);
  static constexpr int PITCH = VSEG * 32;
  static constexpr int CHP = 2 * VSEG;  // 16-byte chunks per row
  static constexpr int BYTES = 64 * PITCH;
  // XOR masks contributed by row bits 0..3
  static constexpr int M0 = CHP == 8 ? 2 : 4, M1 = CHP == 8 ? 4 : 10, M2 = CHP == 32 ? 0 : 1,
                       M3 = CHP == 32 ? 0 : 3;
  __device__ static inline int swz(int r) {
    return ((r & 1) ? M0 : 0) ^ ((r & 2) ? M1 : 0) ^ ((r & 4) ? M2 : 0) ^ ((r & 8) ? M3 : 0);
  }
};

typedef short short4_t __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: a transposing LDS read (16-bit elements).
__device__ __forceinline__ uint2 ds_read_tr16(const char* p) {
  const short4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(p));
  return __builtin_bit_cast(uint2, r);
}

// Lane offset (within a V tile in the VRow layout) of the ds_read_tr16 pair
// that builds the V^T A operand of rows d = 32 dt + (lane % 32) for keys
// 8 (lane / 32) + 0..7 of a 16-key step: the operand is
// (tr16(base + off(0)), tr16(base + off(1))) with base at the step's first
// key row (a multiple of 16, which leaves the swizzle unchanged); `hi` = 1
// reads keys 4..7 of the lane's eight.
template <int HD>
__device__ inline int vt_read_offset(int lane, int dt, int hi) {
  const int i = lane & 15, gh = (lane >> 4) & 1, g = lane >> 5;
  const int vkey = 8 * g + (i >> 2) + 4 * hi;
  const int c = 4 * dt + 2 * gh + ((i >> 1) & 1);
  return vkey * VRow<HD>::PITCH + 16 * (c ^ VRow<HD>::swz(vkey)) + 8 * (i & 1);
}

// Source offset of DMA chunk X of a 64-key V tile in the VRow layout:
// buffer_load ... lds writes chunk X (16 bytes) at tile + 16 X; the chunk
// holds logical 16-byte column c of key row X / CHP.  Padding chunks (hd 32,
// 96) re-read column 0.
template <typename T, int HD>
__device__ inline uint32_t vrow_dma_offset(int X, int64_t v_st) {
  constexpr int KCH = HD / 8;
  const int key = X / VRow<HD>::CHP, pc = X % VRow<HD>::CHP;
  const int c = pc ^ VRow<HD>::swz(key);
  return (uint32_t)(key * v_st * (int64_t)sizeof(T)) + 16u * (c < KCH ? c : 0);
}

// Buffer descriptor over `bytes` bytes from base (clamped to [0, 2^31)):
// loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void* base, int64_t bytes) {
  const int num = (int)(bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, num, kBufferWord3);
}

// Buffer descriptor over rows j0.. of a (rows, st) tensor ending after row
// T_len - 1: loads past the end return zero.
template <typename T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const T* base, int64_t st, int j0, int T_len) {
  const int64_t bytes = (int64_t)(T_len - j0) * st * (int64_t)sizeof(T);
  const int num = (int)(bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes));
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base + (int64_t)j0 * st), 0, num, kBufferWord3);
}

// rows_rsrc for a sequence of row blocks walked in order, without a 64-bit
// multiply or compare per block: the address of the current first row and
// the rows left before T_len, advanced by a fixed row count.  The record
// count is the rows left (at least 0, at most lim_rows) times the row pitch,
// which is below 2^31 whenever the host's limit on row pitches (kMaxRowBytes)
// holds; it then equals rows_rsrc's count for every row a 64-row tile reads.
constexpr int kMaxRowBytes = 1 << 24;
struct RowCursor {
  const char* ptr;
  int rows_left, row_bytes, lim_rows;

  template <typename T>
  __device__ __forceinline__ void init(const T* base, int64_t st, int j0, int T_len) {
    row_bytes = (int)(st * (int64_t)sizeof(T));
    lim_rows = 0x7fffffff / (row_bytes > 0 ? row_bytes : 1);
    ptr = reinterpret_cast<const char*>(base + (int64_t)j0 * st);
    rows_left = T_len - j0;
  }
  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc() const {
    const int r = min(max(rows_left, 0), lim_rows);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(ptr), 0, r * row_bytes, kBufferWord3);
  }
  __device__ __forceinline__ void advance(int rows) {
    ptr += (int64_t)rows * row_bytes;
    rows_left -= rows;
  }
};

// Stage a 64-key V tile (rows j0..j0+63 of one head) into registers:
// item idx covers keys 2kp, 2kp+1 and columns 8c..8c+7.  Rows >= T are zero.
template <typename T, int HD, int NTHR> struct VStager {
  static constexpr int KCH = HD / 8;
  static constexpr int ITEMS = 32 * KCH;
  static constexpr int PER_THR = (ITEMS + NTHR - 1) / NTHR;
  uint4 r0[PER_THR], r1[PER_THR];

  __device__ inline void load(const T* vbase, int64_t v_st, int j0, int T_len, int tid) {
#pragma unroll
    for (int p = 0; p < PER_THR; ++p) {
      const int idx = tid + p * NTHR;
      r0[p] = make_uint4(0, 0, 0, 0);
      r1[p] = make_uint4(0, 0, 0, 0);
      if (ITEMS % NTHR == 0 || idx < ITEMS) {
        const int kp = idx / KCH, c = idx % KCH;
        const int row = j0 + 2 * kp;
        if (row < T_len)
          r0[p] = *reinterpret_cast<const uint4*>(vbase + (int64_t)row * v_st + 8 * c);
        if (row + 1 < T_len)
          r1[p] = *reinterpret_cast<const uint4*>(vbase + (int64_t)(row + 1) * v_st + 8 * c);
      }
    }
  }

  // Transposed store: dword (key 2kp, key 2kp+1) of column d = 8c + e.
  __device__ inline void store(uint32_t* vt, int tid) const {
#pragma unroll
    for (int p = 0; p < PER_THR; ++p) {
      const int idx = tid + p * NTHR;
      if (ITEMS % NTHR == 0 || idx < ITEMS) {
        const int kp = idx / KCH, c = idx % KCH;
        const int kc = kp >> 2, sub = kp & 3;
        const uint32_t a[4] = {r0[p].x, r0[p].y, r0[p].z, r0[p].w};
        const uint32_t b[4] = {r1[p].x, r1[p].y, r1[p].z, r1[p].w};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const uint32_t even = (a[m] & 0xffffu) | (b[m] << 16);
          const uint32_t odd = (a[m] >> 16) | (b[m] & 0xffff0000u);
          const int d0 = 8 * c + 2 * m;
          vt[VLayout<HD>::chunk(d0, kc) * 4 + sub] = even;
          vt[VLayout<HD>::chunk(d0 + 1, kc) * 4 + sub] = odd;
        }
      }
    }
  }
};

// Stage a 64-key K tile (rows j0..j0+63) into registers / swizzled LDS.
template <typename T, int HD, int NTHR> struct KStager {
  static constexpr int KCH = HD / 8;
  static constexpr int ITEMS = 64 * KCH;
  static constexpr int PER_THR = (ITEMS + NTHR - 1) / NTHR;
  uint4 r[PER_THR];

  __device__ inline void load(const T* kbase, int64_t k_st, int j0, int T_len, int tid) {
#pragma unroll
    for (int p = 0; p < PER_THR; ++p) {
      const int idx = tid + p * NTHR;
      r[p] = make_uint4(0, 0, 0, 0);
      if (ITEMS % NTHR == 0 || idx < ITEMS) {
        const int key = idx / KCH, c = idx % KCH;
        if (j0 + key < T_len)
          r[p] = *reinterpret_cast<const uint4*>(kbase + (int64_t)(j0 + key) * k_st + 8 * c);
      }
    }
  }

  __device__ inline void store(uint4* ks, int tid) const {
#pragma unroll
    for (int p = 0; p < PER_THR; ++p) {
      const int idx = tid + p * NTHR;
      if (ITEMS % NTHR == 0 || idx < ITEMS) {
        const int key = idx / KCH, c = idx % KCH;
        ks[KLayout<HD>::chunk(key, c)] = r[p];
      }
    }
  }
};

// O^T accumulation for one 64-key block: o[qt][dt] += V^T(dt) . P^T(qt).
// pb[ks][s][qt] is the B operand for keys 32ks + 16s + (8g + 0..7).
template <typename T, int HD, int QT>
__device__ inline void pv_block(f32x16_t (&o)[QT][HD / 32], const uint4 (&pb)[2][2][QT],
                                const uint4* vt, int lane) {
  const int m = lane & 31, g = lane >> 5;
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int dt = 0; dt < HD / 32; ++dt) {
        const uint4 a = vt[VLayout<HD>::chunk(32 * dt + m, 4 * ks + 2 * s + g)];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][dt] = Elem<T>::mfma(a, pb[ks][s][qt], o[qt][dt]);
      }
}

// Store O^T (already normalised) for one 32-query tile: lane (n, g) writes
// query `q`, columns 32dt + 8r + 4g + 0..3 as 8-byte packets.
template <typename T, int HD>
__device__ inline void store_out_tile(T* orow, const f32x16_t (&o)[HD / 32], float scale, int g) {
#pragma unroll
  for (int dt = 0; dt < HD / 32; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      uint2 w;
      w.x = Elem<T>::pack2(o[dt][4 * r + 0] * scale, o[dt][4 * r + 1] * scale);
      w.y = Elem<T>::pack2(o[dt][4 * r + 2] * scale, o[dt][4 * r + 3] * scale);
      *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * r + 4 * g) = w;
    }
}

}  // namespace saf
