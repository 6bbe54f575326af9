// Live-head causal flash attention forward (state 0 heads) for gfx950.
//
// Semantics follow the reference's live-head accumulator
// (/root/reference/kernel/fused_attn.py:182-226, GQA variant
// /root/reference/qwen/kernel/fused_attn.py:183-231): base-2 online softmax
// with qk_scale = sm_scale * log2(e), fp32 running reference / sum /
// accumulator, P rounded to the input dtype before the P.V product, output
// divided by the row sum, and LSE = m + log2(l) in base-2 units.  Two
// deliberate changes of bookkeeping, both exact up to rounding:
//   - the reference value m of a query is not the running maximum.  P is
//     computed against the current m, and only when some lane's sum of its 16
//     P values of a 32-key sub-block exceeds kRedoSum (so some P > 2^16, or
//     m is still the initial kMinit) is the sub-block recomputed against
//     max(m, block max), rescaling O and l.  That happens for the first
//     sub-block of every query and whenever the scores grow by more than 16
//     (base 2) over the reference; the common sub-block needs no max at all.
//   - the row sum adds the rounded P values (v_dot2 on packed pairs), i.e.
//     exactly the weights that multiply V.
//
// Work decomposition: one workgroup = 4 waves = (4 * 32 * QT) query rows of
// one (batch, live head); each wave owns 32*QT queries.  Keys are walked in
// 64-key blocks of two 32-key sub-blocks.  K and V tiles arrive by
// global_load_lds DMA (no staging registers) into three static LDS slots
// each: block j reads K_j, K_{j+1}, V_{j-1}, V_j while K_{j+2} and V_{j+1}
// load.  K is stored XOR-swizzled for the ds_read_b128 A operand of
// S^T = K.Q^T; V stays row-major (32-byte segments XOR-swizzled by key) and
// its V^T A operands come from ds_read_b64_tr_b16 transposing reads.
//
// Software pipeline: iteration u issues the MFMAs of S_{u+1} and of
// P_{u-1}.V together with the softmax VALU work of S_u, all in one basic
// block, so the matrix pipe always has independent work while the exps run.
// Workgroups are ordered heaviest query block first.
#include <type_traits>

#include "saf_kernels.h"

namespace saf {

// Initial reference value: finite, so masked scores (-inf) give exp2 = 0
// rather than NaN, and any real score overflows the first sum and forces
// the recompute against the true maximum.
constexpr float kMinit = -1.0e30f;
// A lane whose 16 P values of a sub-block sum above this recomputes them
// against the true maximum: every P used in a product is <= 2^16.
constexpr float kRedoSum = 65536.f;


// One 64-key K and V tile copy by DMA: thread (wave w, lane L), load p
// writes LDS chunk X = (4p + w) * 64 + L of the tile (buffer_load ... lds
// puts consecutive lanes' 16 bytes at consecutive addresses from a
// wave-uniform base).  The per-thread source (row in the tile, column) of
// each chunk is the inverse of the tile's swizzle; padding chunks (hd 96)
// re-read column 0.  Each tile gets a buffer descriptor starting at its
// first row and ending after row T-1, so rows past the end read as zero
// (those keys are masked, and zero V rows meet P = 0).  Buffer loads count
// only vmcnt, which leaves the compiler's LDS-read waits exact.

template <typename T, int HD> struct TileDma {
  static constexpr int NW = flash_waves(HD);
  static constexpr int KCH = HD / 8;
  static constexpr int KCHP = KLayout<HD>::KCHP;
  static constexpr int KN = KCHP / NW;
  static constexpr int VN = VRow<HD>::CHP / NW;
  static_assert(KCHP % NW == 0 && VRow<HD>::CHP % NW == 0, "tile chunks must split evenly over the waves");
  uint32_t koff[KN], voff[VN];  // byte offset of this thread's chunks from the tile's first row

  __device__ __forceinline__ void init(int wave, int lane, int64_t k_st, int64_t v_st) {
#pragma unroll
    for (int p = 0; p < KN; ++p) {
      const int X = (NW * p + wave) * 64 + lane;
      const int key = X / KCHP, slot = X % KCHP;
      const int c = slot ^ KLayout<HD>::swz(key);
      koff[p] = (uint32_t)(key * k_st * (int64_t)sizeof(T)) + 16u * (c < KCH ? c : 0);
    }
#pragma unroll
    for (int p = 0; p < VN; ++p) voff[p] = vrow_dma_offset<T, HD>((NW * p + wave) * 64 + lane, v_st);
  }

  __device__ __forceinline__ void load_k(const T* base, int64_t st, int j0, int T_len, char* tile, int wave) const {
    load_k_rs(rows_rsrc(base, st, j0, T_len), tile, wave);
  }
  __device__ __forceinline__ void load_v(const T* base, int64_t st, int j0, int T_len, char* tile, int wave) const {
    load_v_rs(rows_rsrc(base, st, j0, T_len), tile, wave);
  }
  // the same from a descriptor of the tile's rows (a RowCursor's)
  __device__ __forceinline__ void load_k_rs(const __amdgpu_buffer_rsrc_t r, char* tile, int wave) const {
#pragma unroll
    for (int p = 0; p < KN; ++p)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, SAF_LDS_PTR(tile + (NW * p + wave) * 1024), 16, koff[p], 0, 0, 0);
  }
  __device__ __forceinline__ void load_v_rs(const __amdgpu_buffer_rsrc_t r, char* tile, int wave) const {
#pragma unroll
    for (int p = 0; p < VN; ++p)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r, SAF_LDS_PTR(tile + (NW * p + wave) * 1024), 16, voff[p], 0, 0, 0);
  }
};


template <typename T, int HD, int QT>
struct FlashState {
  static constexpr int NDT = HD / 32, NKT = HD / 16;
  static constexpr int KCHP = KLayout<HD>::KCHP;
  uint4 qf[QT][NKT];          // Q^T as B operand: lane (n, g), step t -> Q[q][16t + 8g + 0..7]
  f32x16_t o[QT][NDT];        // O^T accumulators
  float m_run[QT], l_run[QT];
  int koff[NKT];              // byte offset of this lane's K A operand of step t in a sub-block
  int voff[NDT], voffh[NDT];  // byte offsets of this lane's V^T tr-read pair for d tile dt
  float c;                    // sm_scale * log2(e)
  int n, g, q0w;

  __device__ __forceinline__ void init_offsets(int lane) {
    n = lane & 31;
    g = lane >> 5;
    const int key = kperm(n);
#pragma unroll
    for (int t = 0; t < NKT; ++t) koff[t] = 16 * KLayout<HD>::chunk(key, 2 * t + g);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      voff[dt] = vt_read_offset<HD>(lane, dt, 0);
      voffh[dt] = vt_read_offset<HD>(lane, dt, 1);
    }
  }

  // K A operands of sub-block ks (0/1) of a K tile
  __device__ __forceinline__ void load_ka(uint4 (&ka)[NKT], const char* ktile, int ks) const {
#pragma unroll
    for (int t = 0; t < NKT; ++t)
      ka[t] = *reinterpret_cast<const uint4*>(ktile + ks * 32 * KCHP * 16 + koff[t]);
  }

  // S^T of one 32-key sub-block from its K A operands: s[qt] = K_sub . Q^T
  __device__ __forceinline__ void scores_from(f32x16_t (&s)[QT], const uint4 (&ka)[NKT]) const {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) s[qt] = zero16();
#pragma unroll
    for (int t = 0; t < NKT; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) s[qt] = Elem<T>::mfma(ka[t], qf[qt][t], s[qt]);
  }

  // S^T of sub-block ks (0/1) of the K tile
  __device__ __forceinline__ void scores(f32x16_t (&s)[QT], const char* ktile, int ks) const {
    uint4 ka[NKT];
    load_ka(ka, ktile, ks);
    scores_from(s, ka);
  }

  // O^T += V_sub^T . P^T for sub-block ks of the V tile; P^T (packed) sits in
  // registers 0..7 of the S tile it was computed from: words 4 s2 + 0..3 are
  // the B operand of the 16-key step s2
  __device__ __forceinline__ void pv(const f32x16_t (&pt)[QT], const char* vtile, int ks) {
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const char* base = vtile + (32 * ks + 16 * s2) * VRow<HD>::PITCH;
        const uint2 lo = ds_read_tr16(base + voff[dt]);
        const uint2 hi = ds_read_tr16(base + (VRow<HD>::M2 ? voffh[dt] : voff[dt] + 4 * VRow<HD>::PITCH));
        const uint4 a = make_uint4(lo.x, lo.y, hi.x, hi.y);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const uint4 b = make_uint4(__float_as_uint(pt[qt][4 * s2]), __float_as_uint(pt[qt][4 * s2 + 1]),
                                     __float_as_uint(pt[qt][4 * s2 + 2]), __float_as_uint(pt[qt][4 * s2 + 3]));
          o[qt][dt] = Elem<T>::mfma(a, b, o[qt][dt]);
        }
      }
  }

  // keys past a query of this wave -> -inf (sub-block starting at key j0):
  // register i of lane-half g holds key j0 + 8g + (16 (i / 8) + i % 8), so
  // each element compares a constant against one per-lane limit
  __device__ __forceinline__ void mask(f32x16_t (&s)[QT], int j0) const {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int lim = q0w + 32 * qt + n - j0 - 8 * g;
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (16 * (i >> 3) + (i & 7) > lim) s[qt][i] = -INFINITY;
    }
  }

  // P = 2^(s c - m) rounded to T, packed in place into registers 0..7 of s
  // (word 4 sh + u = keys 16 sh + 8g + 2u, 2u + 1); bs = the lane's sum of
  // its rounded P values, added on the matrix pipe (four 4x4x4 MFMAs with an
  // all-ones operand), which has issue slots to spare where the VALU has none
  __device__ __forceinline__ void exp_pack(f32x16_t (&s)[QT], float (&bs)[QT]) const {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float mneg = -m_run[qt];
      uint32_t wd[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const float e0 = fast_exp2(fmaf(s[qt][2 * w], c, mneg));
        const float e1 = fast_exp2(fmaf(s[qt][2 * w + 1], c, mneg));
        wd[w] = Elem<T>::pack2(e0, e1);
        s[qt][w] = __uint_as_float(wd[w]);
      }
      f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int w = 0; w < 8; w += 2) acc = Elem<T>::sum4(make_uint2(wd[w], wd[w + 1]), acc);
      bs[qt] = acc[0];
    }
  }

  // Rare path: S_u is recomputed from its K tile, the reference moves to
  // max(m, block max) for every query of the wave, O and l are rescaled and
  // P recomputed.  After it every P of the sub-block is <= 1.  The causal
  // mask is applied whether or not the block holds the diagonal: below it,
  // every key of the sub-block precedes every query of the workgroup, so the
  // mask changes nothing there (and no flag has to reach this path).
  __device__ __forceinline__ void redo(f32x16_t (&s)[QT], float (&bs)[QT], const char* ktile, int ks, int j0) {
    scores(s, ktile, ks);
    mask(s, j0);
    rebase(s, bs);
  }

  // Before any accumulation: the reference maximum from the item's first
  // sub-block of raw (masked) scores, so its softmax stays on the common path
  // (from kMinit every item's first step took the recompute).  O and l are
  // still zero; a row with no finite score keeps kMinit.
  __device__ __forceinline__ void seed_max(const f32x16_t (&s)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = s[qt][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[qt][i]);
      mx = half_swap_max(mx);
      m_run[qt] = fmaxf(m_run[qt], mx * c);
    }
  }

  // The recompute from raw (masked) scores s: move the reference to
  // max(m, block max), rescale O and l, and recompute P.
  __device__ __forceinline__ void rebase(f32x16_t (&s)[QT], float (&bs)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float mx = s[qt][0];
#pragma unroll
      for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[qt][i]);
      mx = half_swap_max(mx);
      const float m_new = fmaxf(m_run[qt], mx * c);
      const float alpha = fast_exp2(m_run[qt] - m_new);
      m_run[qt] = m_new;
      l_run[qt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) o[qt][dt][i] *= alpha;
    }
    exp_pack(s, bs);
  }

  // K A operands of the next step's S product are read a whole step ahead
  // (kpre) up to hd 64; above, the 32 more VGPRs would spill, and each step
  // reads its own
  static constexpr bool kPrefetchK = HD <= 64;
  // hd 256: two LDS slots per operand (four 32 KB tiles); see flash_unit
  static constexpr bool kTwoSlot = HD > 128;

  // One pipeline step u.  On entry `nxt` holds P_{u-1} (packed), `cur`
  // holds S_u and, with kPrefetchK, `kpre` the K A operands of S_{u+1}.
  // O += P_{u-1} V (tile vP, sub-block ksP) is issued first, then S_{u+1}
  // (tile kS, sub-block ksS) overwrites `nxt` (from `kpre`, whose next
  // contents, the operands of S_{u+2} in tile kN / sub-block ksN, are read
  // right after), and the softmax of S_u packs P_u into `cur` (tile kR /
  // sub-block ksR for the rare recompute).
  __device__ __forceinline__ void step(f32x16_t (&cur)[QT], f32x16_t (&nxt)[QT], uint4 (&kpre)[NKT], int u,
                                       int masked, const char* kS, int ksS, const char* kN, int ksN,
                                       const char* kR, int ksR, const char* vP, int ksP) {
    // the mask touches only S_u, complete before the step: applying it first
    // keeps the MFMAs and the softmax below in one basic block.  The empty
    // volatile asm keeps the (uniform) branch a real scalar branch, so the
    // mask's selects stay out of the step's schedule: 140 VGPRs instead of
    // 152 at hd 64, 198 instead of 228 at hd 128.
    if (masked) {
      asm volatile("" ::: "memory");
      mask(cur, 32 * u);
    }
    pv(nxt, vP, ksP);
    if constexpr (kPrefetchK) {
      scores_from(nxt, kpre);
      load_ka(kpre, kN, ksN);
    } else {
      scores(nxt, kS, ksS);
    }
    float bs[QT];
    exp_pack(cur, bs);
    bool bad = false;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) bad |= bs[qt] > kRedoSum;
    if (__builtin_amdgcn_ballot_w64(bad)) redo(cur, bs, kR, ksR, 32 * u);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l_run[qt] += bs[qt];
  }

  // The step of the two-slot schedule: as step() without the K prefetch,
  // and the rare recompute starts from a register copy of the masked raw
  // scores, so no K tile has to outlive the step that reads it.
  __device__ __forceinline__ void step_raw(f32x16_t (&cur)[QT], f32x16_t (&nxt)[QT], int u, int masked,
                                           const char* kS, int ksS, const char* vP, int ksP) {
    if (masked) {
      asm volatile("" ::: "memory");
      mask(cur, 32 * u);
    }
    pv(nxt, vP, ksP);
    scores(nxt, kS, ksS);
    f32x16_t raw[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) raw[qt] = cur[qt];
    float bs[QT];
    exp_pack(cur, bs);
    bool bad = false;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) bad |= bs[qt] > kRedoSum;
    if (__builtin_amdgcn_ballot_w64(bad)) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) cur[qt] = raw[qt];
      rebase(cur, bs);
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l_run[qt] += bs[qt];
  }
};

// hd <= 64: three waves per SIMD (three resident 4-wave workgroups of 128
// queries, within 170 registers) or two of 256 queries (within 256
// registers).  hd 96 / 128: one workgroup's three K and V slots fill most of
// the CU's LDS, so the workgroup has 8 waves (two per SIMD) sharing them.
// hd 256: 4 waves, one per SIMD (512 registers each), over two slots per
// operand.  The host's flash_resident() and flash_block_rows() mirror this.
template <int HD, int QT>
constexpr int flash_waves_per_eu() { return HD <= 64 ? (QT == 1 ? 3 : 2) : (HD <= 128 && QT == 1 ? 2 : 1); }

// One work unit of the live-head kernel: unit = item * (B * n_slots) + r,
// item = a query block (and key segment), r = (batch, live slot).
template <typename T, int HD, int QT, typename Params>
__device__ __forceinline__ void flash_unit(Params& p, const int unit, char* k0, char* k1, char* k2, char* v0,
                                           char* v1, char* v2) {
  using St = FlashState<T, HD, QT>;
  constexpr int NW = flash_waves(HD);
  constexpr int BM = NW * 32 * QT;
  constexpr int NDT = St::NDT, NKT = St::NKT;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)

  // work item: query block (and key segment) of one (batch, live slot);
  // items are ordered heaviest first, (batch, live slot) fastest
  const int nbh = p.B * p.n_slots;
  const int r = unit % nbh;
  const int b = r / p.n_slots, slot = r % p.n_slots;
  const int h = p.out_head[slot];
  int qb, seg = 0;
  if (p.n_items) {
    const int it = p.items[unit / nbh];
    qb = it >> 8;
    seg = it & 255;
  } else {
    qb = p.n_qblk - 1 - unit / nbh;
  }
  const T* qbase = reinterpret_cast<const T*>(p.q) + b * p.q_sb + (int64_t)p.q_head[slot] * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + b * p.k_sb + (int64_t)p.k_head[slot] * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)p.v_head[slot] * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;

  const int T_len = p.T;
  const int q0 = qb * BM;
  const int nkb_qb = (min(q0 + BM, T_len) + 63) / 64;  // key blocks of the query block
  const int kb0 = p.n_items ? seg * p.seg_len : 0;     // this item's key-block range
  const int nkb = p.n_items ? min(kb0 + p.seg_len, nkb_qb) : nkb_qb;
  const bool split = p.n_items && p.part_base[qb] >= 0;
  // blocks wholly below the workgroup's first query need no causal mask
  const int jd = min(nkb, max(kb0, q0 / 64));

  St st;
  st.init_offsets(lane);
  st.q0w = q0 + wave * 32 * QT;
  st.c = p.scale_log2;
  TileDma<T, HD> dma;
  dma.init(wave, lane, p.k_st, p.v_st);

  // prologue DMA: K_kb0, K_kb0+1, V_kb0 into slot 0 / 1 / 0; the V slot of
  // "V_{kb0-1}" (slot 2, or slot 1 of the two-slot schedule), multiplied by
  // P = 0 in the first step, gets finite data too, since 0 * NaN from stale
  // LDS would poison O
  dma.load_k(kbase, p.k_st, 64 * kb0, T_len, k0, wave);
  if (kb0 + 1 < nkb) dma.load_k(kbase, p.k_st, 64 * (kb0 + 1), T_len, k1, wave);
  dma.load_v(vbase, p.v_st, 64 * kb0, T_len, v0, wave);
  dma.load_v(vbase, p.v_st, 64 * kb0, T_len, St::kTwoSlot ? v1 : v2, wave);

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = st.q0w + 32 * qt + st.n;
#pragma unroll
    for (int t = 0; t < NKT; ++t)
      st.qf[qt][t] = q < T_len ? *reinterpret_cast<const uint4*>(qbase + (int64_t)q * p.q_st + 16 * t + 8 * st.g)
                               : make_uint4(0, 0, 0, 0);
    st.m_run[qt] = kMinit;
    st.l_run[qt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) st.o[qt][dt] = zero16();
  }
  __syncthreads();

  // descriptors of the next K block to load (K_{kb0+2}) and the next V
  // block (V_{kb0+1}), advanced by 64 rows per block
  RowCursor kcur, vcur;
  kcur.init(kbase, p.k_st, 64 * (kb0 + 2), T_len);
  vcur.init(vbase, p.v_st, 64 * (kb0 + 1), T_len);

  // pipeline registers: sA / sB alternate between S_u and P_{u-1} / S_{u+1};
  // P_{-1} = 0 makes the first P.V a no-op
  f32x16_t sA[QT], sB[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) sB[qt] = zero16();
  st.scores(sA, k0, 0);
  if (kb0 >= jd) st.mask(sA, 64 * kb0);  // as the first step will
  st.seed_max(sA);
  if constexpr (St::kTwoSlot) {
    // hd 256: four 32 KB tiles fit the LDS, not six.  Block j (phase R =
    // (j - kb0) & 1): K_j in k_R, K_{j+1} in k_{1-R}, V_j in v_R, V_{j-1} in
    // v_{1-R}.  After the first step K_j and V_{j-1} are dead (the rare
    // recompute keeps raw scores in registers), so one barrier mid-block
    // frees their slots for K_{j+2} and V_{j+1}, each with two steps to
    // land before the next block's barrier waits for them.
    auto block2 = [&](const int j, auto phase) {
      constexpr int R = decltype(phase)::value;
      char* const kJ = R ? k1 : k0;
      char* const kJ1 = R ? k0 : k1;
      char* const vJ = R ? v1 : v0;
      char* const vJm = R ? v0 : v1;
      const int masked = j >= jd;
      // u = 2j: S_{2j+1} (K_j sub 1), P_{2j-1} V_{j-1} sub 1, softmax S_{2j}
      st.step_raw(sA, sB, 2 * j, masked, kJ, 1, vJm, 1);
      __syncthreads();  // K_j and V_{j-1} read by every wave; K_{j+1} and V_j landed (vmcnt 0)
      if (j + 2 < nkb) dma.load_k_rs(kcur.rsrc(), kJ, wave);
      if (j + 1 < nkb) dma.load_v_rs(vcur.rsrc(), vJm, wave);
      kcur.advance(64);
      vcur.advance(64);
      // u = 2j+1: S_{2j+2} (K_{j+1} sub 0; past the last block a stale slot
      // whose scores are never used), P_{2j} V_j sub 0, softmax S_{2j+1}
      st.step_raw(sB, sA, 2 * j + 1, masked, kJ1, 0, vJ, 0);
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    int j = kb0, ph;
    for (;;) {
      if (j >= nkb) { ph = 0; break; }
      block2(j++, P0());
      if (j >= nkb) { ph = 1; break; }
      block2(j++, P1());
    }
    // P_{2 nkb - 1} . V_{nkb-1} sub 1 (V_{nkb-1} is in v0 when the last block had phase 0)
    st.pv(sB, ph == 1 ? v0 : v1, 1);
  } else {
    uint4 kpre[NKT];  // K operands of the next S product, read one step ahead
    if constexpr (St::kPrefetchK) st.load_ka(kpre, k0, 1);

    // block j in phase R (slots: K_j = R, K_{j+1} = R+1, K_{j+2} = R+2 (loading),
    // V_{j-1} = R+2, V_j = R, V_{j+1} = R+1 (loading), all mod 3); blocks at
    // or past jd hold the diagonal and run the masked steps
    auto block = [&](const int j, auto phase) {
      constexpr int R = decltype(phase)::value;
      char* const ks[3] = {k0, k1, k2};
      char* const vs[3] = {v0, v1, v2};
      char* const kJ = ks[R];
      char* const kJ1 = ks[(R + 1) % 3];
      char* const kJ2 = ks[(R + 2) % 3];
      char* const vJm = vs[(R + 2) % 3];
      char* const vJ = vs[R];
      char* const vJ1 = vs[(R + 1) % 3];
      if (j + 2 < nkb) dma.load_k_rs(kcur.rsrc(), kJ2, wave);
      if (j + 1 < nkb) dma.load_v_rs(vcur.rsrc(), vJ1, wave);
      kcur.advance(64);
      vcur.advance(64);
      const int masked = j >= jd;
      // u = 2j: S_{2j+1} (K_j sub 1), operands of S_{2j+2} (K_{j+1} sub 0),
      // P_{2j-1} V_{j-1} sub 1, softmax S_{2j}
      st.step(sA, sB, kpre, 2 * j, masked, kJ, 1, kJ1, 0, kJ, 0, vJm, 1);
      // u = 2j+1: S_{2j+2} (K_{j+1} sub 0), operands of S_{2j+3} (K_{j+1}
      // sub 1), P_{2j} V_j sub 0, softmax S_{2j+1}.  Past the last block these
      // read a stale slot whose products are never used.
      st.step(sB, sA, kpre, 2 * j + 1, masked, kJ1, 0, kJ1, 1, kJ, 1, vJ, 0);
      __syncthreads();  // waits for this block's DMA (vmcnt 0) before any wave moves on
    };
    using P0 = std::integral_constant<int, 0>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    // blocks run as a chain of phases 0 -> 1 -> 2 -> 0, so every DMA target and
    // every read names a static LDS slot
    int j = kb0, ph;
    for (;;) {
      if (j >= nkb) { ph = 0; break; }
      block(j++, P0());
      if (j >= nkb) { ph = 1; break; }
      block(j++, P1());
      if (j >= nkb) { ph = 2; break; }
      block(j++, P2());
    }
    // P_{2 nkb - 1} . V_{nkb-1} sub 1 (V_{nkb-1} sits in the slot of phase ph - 1)
    st.pv(sB, ph == 1 ? v0 : (ph == 2 ? v1 : v2), 1);
  }

#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int q = st.q0w + 32 * qt + st.n;
    const float l_tot = half_swap_sum(st.l_run[qt]);
    if (split) {
      // unnormalised partial of this key segment, merged by flash_combine_kernel
      const int64_t pidx = (int64_t)r * p.n_part_per_head + p.part_base[qb] + seg;
      const int rl = q - q0;
      float* po = p.part_o + (pidx * BM + rl) * HD;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(po + 32 * dt + 8 * r4 + 4 * st.g) =
              make_float4(st.o[qt][dt][4 * r4], st.o[qt][dt][4 * r4 + 1], st.o[qt][dt][4 * r4 + 2],
                          st.o[qt][dt][4 * r4 + 3]);
      if (st.g == 0) {
        p.part_ml[(pidx * 2) * BM + rl] = st.m_run[qt];
        p.part_ml[(pidx * 2 + 1) * BM + rl] = l_tot;
      }
      continue;
    }
    const float l_safe = l_tot == 0.f ? 1.f : l_tot;
    if (q < T_len) {
      store_out_tile<T, HD>(obase + (int64_t)q * p.o_st, st.o[qt], 1.f / l_safe, st.g);
      if (p.lse != nullptr && st.g == 0)
        p.lse[b * p.l_sb + (int64_t)h * p.l_sh + (int64_t)q * p.l_st] = st.m_run[qt] + __log2f(l_safe);
    }
  }
}

// hd <= 64: three waves per SIMD (three resident 4-wave workgroups of 128
// queries) or two of 256 queries; larger heads: one 8-wave workgroup per CU.
// PERSIST (with a queue word p.queue, zeroed before the launch): the grid
// holds only the resident workgroups, and each takes its next unit from the
// queue when it finishes one (units in heaviest-first order), so a CU or XCD
// that runs faster takes more units instead of each XCD working through a
// fixed 1/8 of the grid.  Otherwise one workgroup per unit.
template <typename T, int HD, int QT, bool PERSIST>
__global__ __launch_bounds__(64 * flash_waves(HD))
__attribute__((amdgpu_waves_per_eu(flash_waves_per_eu<HD, QT>(), flash_waves_per_eu<HD, QT>())))
void flash_fwd_kernel(const FlashParams p) {
  constexpr int KB = KLayout<HD>::BYTES, VB = VRow<HD>::BYTES;
  // hd 256 uses two slots per operand (k2 / v2 are never touched there and
  // take one byte)
  constexpr int KB3 = HD > 128 ? 1 : KB, VB3 = HD > 128 ? 1 : VB;
  __shared__ __align__(16) char k0[KB], k1[KB], k2[KB3];
  __shared__ __align__(16) char v0[VB], v1[VB], v2[VB3];
  if constexpr (!PERSIST) {
    // XCD-aware head order.  Workgroup i runs on XCD i % 8, and unit
    // item * nbh + r takes (batch, live slot) r of an item.  Within each
    // aligned group of 8 slots, slot r is swapped for the slot of the same
    // group whose index is i mod 8: slot s < 8 * (nbh / 8) then always runs
    // on XCD s % 8, so each XCD's L2 holds the K / V of its own heads (the
    // nbh % 8 remaining slots spread over the XCDs).  A permutation of the
    // slots within each item; the identity when nbh is a multiple of 8.
    int unit = blockIdx.x;
    const int nbh = p.B * p.n_slots, r = unit % nbh;
    if (r < (nbh & ~7)) unit += ((r & ~7) | (unit & 7)) - r;
    flash_unit<T, HD, QT>(p, unit, k0, k1, k2, v0, v1, v2);
  } else {
    __shared__ int next_unit;
    const int n_units = (p.n_items ? p.n_items : p.n_qblk) * p.B * p.n_slots;
    int unit = blockIdx.x;
    for (;;) {
      // claim the next unit now, so the atomic's latency hides behind this one
      if (threadIdx.x == 0) next_unit = (int)atomicAdd(p.queue, 1u) + (int)gridDim.x;
      // the parameter block is read through a kernarg-segment pointer that
      // the compiler cannot follow across iterations: its fields are loaded
      // (scalar loads) per unit instead of being kept live in SGPRs across
      // units, which spilled
      const __attribute__((address_space(4))) FlashParams* pk =
          (const __attribute__((address_space(4))) FlashParams*)__builtin_amdgcn_kernarg_segment_ptr();
      asm volatile("" : "+s"(pk));
      flash_unit<T, HD, QT>(*pk, unit, k0, k1, k2, v0, v1, v2);
      __syncthreads();
      unit = __builtin_amdgcn_readfirstlane(next_unit);
      __syncthreads();  // every wave has read next_unit before it is claimed again
      if (unit >= n_units) break;
    }
  }
}

// Merge the key-segment partials of split query blocks (one workgroup per
// (batch, slot, split query block) and 64-row chunk; HD/4 threads x 4
// columns per row): the
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
  // blockIdx.y picks a 64-row chunk of the query block: four times the
  // workgroups of one per query block, for the latency of the partial reads
  const int r_end = min(BM, 64 * ((int)blockIdx.y + 1));
  for (int rl = 64 * (int)blockIdx.y + tid / CPR; rl < r_end; rl += RPP) {
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

// Explicit instantiations: every (dtype, head_dim, query tiles) the
// launcher dispatches to gets its host stub emitted.
#define SAF_FLASH_INST(T, HD, QT) \
  template __global__ void flash_fwd_kernel<T, HD, QT, false>(const FlashParams); \
  template __global__ void flash_fwd_kernel<T, HD, QT, true>(const FlashParams);
#define SAF_FLASH_INST_HD(T) \
  SAF_FLASH_INST(T, 32, 1) SAF_FLASH_INST(T, 32, 2) SAF_FLASH_INST(T, 64, 1) SAF_FLASH_INST(T, 64, 2) \
  SAF_FLASH_INST(T, 96, 1) SAF_FLASH_INST(T, 128, 1) SAF_FLASH_INST(T, 256, 1)
SAF_FLASH_INST_HD(__bf16)
SAF_FLASH_INST_HD(_Float16)
#undef SAF_FLASH_INST_HD
#undef SAF_FLASH_INST

template <typename T, int HD, int QT>
static hipError_t launch_flash_t(const FlashParams& p, hipStream_t s) {
  const int64_t units = (int64_t)(p.n_items ? p.n_items : p.n_qblk) * p.B * p.n_slots;
  if (p.queue != nullptr) {
    const int64_t g = p.max_grid > 0 && units > p.max_grid ? p.max_grid : units;
    hipLaunchKernelGGL((flash_fwd_kernel<T, HD, QT, true>), dim3((unsigned)g), dim3(64 * flash_waves(HD)), 0, s, p);
  } else {
    hipLaunchKernelGGL((flash_fwd_kernel<T, HD, QT, false>), dim3((unsigned)units), dim3(64 * flash_waves(HD)), 0, s,
                       p);
  }
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
    case 128 * 4 + 1: return launch_flash_t<T, 128, 1>(p, s);
    case 256 * 4 + 1: return launch_flash_t<T, 256, 1>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_flash(const FlashParams& p, int dtype, int hd, int qt, hipStream_t s) {
  if (dtype == kF32) return launch_f32_live(p, hd, s);
  if (dtype == kBF16) return launch_flash_hd<__bf16>(p, hd, qt, s);
  if (dtype == kF16) return launch_flash_hd<_Float16>(p, hd, qt, s);
  return hipErrorInvalidValue;
}

template <typename T>
static hipError_t launch_combine_t(const CombineParams& p, int hd, hipStream_t s) {
  const dim3 grid((unsigned)((int64_t)p.n_split * p.B * p.n_slots), (unsigned)((p.BM + 63) / 64));
  switch (hd) {
    case 32: hipLaunchKernelGGL((flash_combine_kernel<T, 32>), grid, dim3(256), 0, s, p); break;
    case 64: hipLaunchKernelGGL((flash_combine_kernel<T, 64>), grid, dim3(256), 0, s, p); break;
    case 96: hipLaunchKernelGGL((flash_combine_kernel<T, 96>), grid, dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL((flash_combine_kernel<T, 128>), grid, dim3(256), 0, s, p); break;
    case 256: hipLaunchKernelGGL((flash_combine_kernel<T, 256>), grid, dim3(256), 0, s, p); break;
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
