// Frozen heads applied as an MFMA P.V product on gfx950.
//
//   mode 0 (state 1, dense pattern): y_i = sum_{j<=i} P[pidx(h), i, j] v_j with
//     P read from the caller's (P, S, S) buffer in fp32 / bf16 / fp16 and
//     rounded to the input dtype before the product, as in the reference's
//     dense accumulator (/root/reference/kernel/fused_attn.py:125-143) and
//     the split-path kernel (/root/reference/kernel/frozen_attn.py:51-89).
//   mode 1 (state 2, decomposed pattern): P[i, j] = exp2((alpha[j] + rho[i-j]
//     - z[i]) * log2 e) rebuilt in registers from the fp32-widened (H, S)
//     buffers, as in /root/reference/kernel/fused_attn.py:145-180; cells with
//     j > i are exactly zero.
//
// The P.V half is the live-head kernel's: O^T += V^T P^T on MFMA, V^T
// operands from VRow tiles in LDS (transposing reads), P^T in the B-operand
// lane layout (lane (n, g) owns query n and keys 8g + 0..7 of each 16-key
// step).  Dense (frozen_dense_kernel): 8 waves x 32 rows, each lane reading
// its P^T operands straight from the pattern rows (16 bytes per operand,
// rounded to the input dtype once unless already in it) for the 2 or 4 batch
// elements that share them, causally balanced work items.  Decomposed
// (frozen_decomp_kernel): 4 waves x 32 QT rows, P^T from a Toeplitz window in
// LDS (factored form) or rebuilt in registers.
#include <type_traits>

#include "saf_kernels.h"

namespace saf {

// Resident decomposed workgroups per CU (decomp_resident() on the host):
// three up to hd 64; two above, where the factored form's three V' slots and
// two distance windows take 62.5 KB of LDS (three workgroups need <= 53 KB)
// and hd 256's 128 accumulator registers per wave need the 256-register
// budget of two waves per SIMD.
constexpr int decomp_waves_per_eu(int hd) { return hd > 64 ? 2 : 3; }

// Decomposed frozen heads, P = exp(alpha_j + rho_{i-j} - z_i), in one of
// two forms chosen per workgroup.
//
// Factored form (bf16, hd <= 128, with the workspace's key-scaled values):
// in log2 units (a = alpha log2 e, r, z likewise), with A_k the maximum of a
// over 64-key block k, A the maximum of A_k over the blocks the workgroup
// reads and R the maximum of r over the distances it reaches,
//   P_ij = 2^(A + R - z_i) . E_ij . 2^(a_j - A_k),  E_ij = 2^(r_{i-j} - R + A_k - A)
// for key j in block k.  So Y = 2^(A + R - z_i) (E V'), V'_j = 2^(a_j - A_k) v_j:
//   - V' is written once per (batch, head) by decomp_prescale_kernel and
//     arrives here by buffer_load ... lds DMA into the live-head kernel's VRow
//     tiles, two blocks ahead in three static slots; its V'^T operands come
//     from ds_read_b64_tr_b16 pairs;
//   - E costs one exp per distance per 64-key block, not one per cell: the
//     block's distance window (with its block shift A_k - A) goes to LDS in 8
//     copies shifted by 0..7 elements (two slots, staged one block ahead),
//     so each lane's E^T operand (8 consecutive distances, reversed) is one
//     aligned ds_read_b128 whose copy and offset are per-lane constants;
//     E is held as a bf16 pair hi + lo and costs two MFMAs per operand, so
//     the form rounds only V' (once, like the rebuild form's P);
//   - the row factor multiplies the fp32 accumulators at the end.
// Every factor is <= 1 before the row factor, and the form is used only when
// every row's z is within kFactorRange of A + R, so every cell that matters
// (P > 2^-24) has both bf16 factors far above the normal range limit and the
// products stay normal in fp32; otherwise (and without the workspace) the
// workgroup rebuilds P cell by cell.  That bf16 hi + lo form needs bf16
// activations; fp16 activations have the fp16 form below or the rebuild.
//
// Rebuild form: P^T rebuilt in registers, one 16-key operand at a time and
// consumed by its MFMAs right away (building a whole 64-key block of
// operands first pushed the accumulators into AGPR copies at one wave per
// SIMD).  alpha, rho and z are staged pre-multiplied by log2(e), so a cell
// costs one add, one subtract and one exp2.
constexpr float kFactorRange = 80.f;
// fp16 factored form: E and V' as fp16 (unit roundoff 2^-11 each, so a cell
// carries less rounding than the reference's bf16 P) and one MFMA per
// operand instead of the hi + lo pair.  fp16's range is short: a factor
// below 2^-24 flushes to zero and a subnormal one keeps an absolute error of
// at most 2^-25.  Those errors reach y multiplied by the row factor
// F = 2^(A + R - z_i) and at most |v|, so over T keys they stay below
// T F 2^-24 max|v|; the form is used only where F <= 2^(kF16Budget - log2 T),
// i.e. that sum is at most 2^-10 max|v|, and where every |V'| the workgroup
// reads is at most kF16Max (no overflow).  Everything else takes the bf16
// hi + lo form (bf16 activations) or the rebuild.  The form serves fp16
// activations as well: their V' is fp16 already in range.
constexpr int kF16Budget = 14;
constexpr float kF16Max = 65504.f;

// (The body is a device function: the kernel template's host stub is then
// emitted for every launch site.)
template <typename T, int HD, int QT>
__device__ __forceinline__ void decomp_body(const FrozenParams& p) {
  constexpr int NW = 4, NTHR = 256;
  constexpr int BM = NW * 32 * QT;
  constexpr int NDT = HD / 32;
  constexpr int RW = BM + 64;  // rho / distance window per key block
  // the factored window's 8 shifted copies (bf16 elements): copy c starts at
  // element c RWL + (c ? 8 : 0), which (searched over copy pitches and
  // shifts) keeps every 16-lane group of one E^T read on distinct banks
  constexpr int RWL = RW + 16;
  constexpr int ERN = (RW + NTHR - 1) / NTHR;
  static_assert(RW % 2 == 0 && RW / 2 <= NTHR, "one thread per pair of factored-window elements");
  // bf16 activations: the fp16 form, else the bf16 hi + lo form, else the
  // rebuild; fp16 activations: the fp16 form, else the rebuild
  constexpr bool kBf16 = std::is_same<T, __bf16>::value;
  constexpr bool kFactorable = (kBf16 || std::is_same<T, _Float16>::value) && HD <= 128;
  // LDS: the factored form's three V' tiles (vs0..vs2) and two distance
  // windows of hi and lo copies (eb0, eb1), or the rebuild form's two V^T
  // tiles (vs0, vs1) and alpha / rho windows (eb0).  Separate objects, so the
  // compiler sees that reading one slot cannot alias the DMA into another
  // and puts no vmcnt wait before the block's LDS reads.
  constexpr int VB = VRow<HD>::BYTES, PITCH = VRow<HD>::PITCH;
  constexpr int VN = VRow<HD>::CHP / NW;  // V' DMA chunks per thread per tile
  constexpr int kEBytes = 2 * 8 * RWL * 2;  // one E slot: hi and lo, 8 shifted copies each
  constexpr int kVtBytes = VLayout<HD>::BYTES;
  constexpr int kPrmBytes = 2 * 64 * 4 + 2 * RW * 4;  // rebuild: alpha and rho windows, two buffers
  constexpr int kVSlot = kFactorable && VB > kVtBytes ? VB : kVtBytes;
  constexpr int kE0 = kFactorable && kEBytes > kPrmBytes ? kEBytes : kPrmBytes;
  __shared__ __align__(16) char vs0[kVSlot], vs1[kVSlot];
  __shared__ __align__(16) char vs2[kFactorable ? VB : 16];
  __shared__ __align__(16) char eb0[kE0];
  __shared__ __align__(16) char eb1[kFactorable ? kEBytes : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int n = lane & 31, g = lane >> 5;

  // work item (query block, key segment) of one (batch, head), heaviest
  // first, (batch, head) fastest; without items one per query block.  The
  // item word is read unconditionally (index clamped), so the compiler can
  // issue it together with the head-table reads below
  const int nbh = p.B * p.n_slots;
  const int r = blockIdx.x % nbh;
  const int iu = (int)(blockIdx.x / nbh);
  const int w_item = p.items[min(iu, kMaxItems - 1)];
  const int qb = p.n_items ? w_item >> 8 : p.n_qblk - 1 - iu;
  const int seg = p.n_items ? w_item & 255 : 0;
  const int b = r / p.n_slots, slot = r % p.n_slots;
  const int h = arg_i16(p.out_head, slot);
  const int ph = arg_i16(p.pat_head, slot);

  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)arg_i16(p.v_head, slot) * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;

  const int T_len = p.T;
  const int q0 = qb * BM;
  const int q0w = q0 + wave * 32 * QT;
  const int kend_wg = min(q0 + BM, T_len);
  const int nkb_qb = (kend_wg + 63) / 64;
  // an unsplit query block's item is segment 0 and spans at most seg_len
  // blocks, so the range needs no part_base lookup (that is read for the
  // epilogue only)
  const int kb0 = p.n_items ? seg * p.seg_len : 0;
  const int nkb = p.n_items ? min(nkb_qb, kb0 + p.seg_len) : nkb_qb;
  const int kend_w = min(q0w + 32 * QT, T_len);
  const int nkb_w = min(nkb, kend_w > 0 ? (kend_w + 63) / 64 : 0);  // blocks this wave's rows reach

  auto alpha_at = [&](int j) { return load_as_f32(p.alpha, (int64_t)ph * p.a_sh + (int64_t)j * p.a_ss, p.a_dtype); };
  auto rho_at = [&](int d) { return load_as_f32(p.rho, (int64_t)ph * p.r_sh + (int64_t)d * p.r_ss, p.r_dtype); };

  // per-lane row normalisers in log2 units; rows >= T get +inf -> exact zeros
  float zq[QT];
  f32x16_t o[QT][NDT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) o[qt][dt] = zero16();
  float rowscale[QT];

  // Factored form: A = max A_k over this segment's key blocks, R = max r
  // over the 64-distance blocks below kend_wg (a superset of what any key
  // segment of this block reaches) and the smallest z of the block's rows
  // decide it for the whole workgroup.  Every input comes from the pre-pass,
  // so the prologue issues all its loads before the first wait: the fp16 V'
  // of the first two blocks (the usual form; the others reload them), the
  // first window's rho values, the rows' normalisers and the per-block
  // maxima and minima.  Each wave reduces the same values itself (DPP, no LDS
  // and no barrier), so the four waves reach the same decision.
  bool factored = false, form16 = false, spec = false;
  float aoff = 0.f, roff = 0.f;
  const int nblk = (T_len + 63) / 64;
  const float* const ablk = p.a_off + (int64_t)slot * nblk;
  uint32_t voff[VN];
#pragma unroll
  for (int pp = 0; pp < VN; ++pp) voff[pp] = vrow_dma_offset<T, HD>((NW * pp + wave) * 64 + lane, HD);
  // V'_j from the copy at vpb into V slot `slot`; a block past this segment
  // gets an empty descriptor (no memory read, the slot is filled with
  // zeros), so every block issues the same loads and the vmcnt counts of the
  // block loop are static
  auto load_v = [&](const auto* vpb, int j, auto slot) {
    constexpr int V = decltype(slot)::value;
    char* const tile = V == 0 ? vs0 : (V == 1 ? vs1 : vs2);
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(vpb, (int64_t)HD, 64 * j, j < nkb ? T_len : 0);
#pragma unroll
    for (int pp = 0; pp < VN; ++pp)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, SAF_LDS_PTR(tile + (NW * pp + wave) * 1024), 16, voff[pp], 0, 0, 0);
  };
  // The fp32 rho log2 e values (r2) of block jb's distance window (elements
  // 2t, 2t + 1 and 2t + 2 of thread t: distances d0, d0 - 1, d0 - 2 with
  // d0 = q0 - 64 jb + BM - 2t) and the block's alpha maximum, into register
  // set `set` (two sets: the block loop loads them two blocks ahead).  One
  // explicit 12-byte buffer load and one 4-byte load per block, so the
  // block loop's vmcnt count is exact: the descriptor starts two elements
  // before the slot's row, so byte offset 4 d0 covers d0 - 2 .. d0; below
  // zero the offset wraps and reads zeros, past the row it reads the
  // workspace that follows (within BM + 64 elements), and every such
  // distance (d < 0 or d >= T) is masked where the window is written.
  float er[2][3], ab[2] = {0.f, 0.f};
  const float* const r2 = p.r2 + (int64_t)slot * T_len;
  const __amdgpu_buffer_rsrc_t r2rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(r2 - 2), 0, (T_len + BM + 66) * 4, kBufferWord3);
  const __amdgpu_buffer_rsrc_t abrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ablk), 0, nblk * 4,
                                                                        kBufferWord3);
  auto load_er = [&](auto set, int jb) {
    constexpr int S = decltype(set)::value;
    const int d0 = q0 - 64 * jb + BM - 2 * tid;
    const auto w3 = __builtin_amdgcn_raw_buffer_load_b96(r2rs, d0 * 4, 0, 0);
    er[S][0] = __uint_as_float(w3[2]);
    er[S][1] = __uint_as_float(w3[1]);
    er[S][2] = __uint_as_float(w3[0]);
    ab[S] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(abrs, min(jb, nblk - 1) * 4, 0, 0));
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  const int64_t vrow0 = ((int64_t)b * p.n_slots + slot) * T_len * HD;
  const _Float16* const vp16base = reinterpret_cast<const _Float16*>(p.vp16) + vrow0;
  const T* const vpbase = reinterpret_cast<const T*>(p.vp) + vrow0;
  if constexpr (kFactorable) {
    if (p.vp != nullptr) {
      load_v(vp16base, kb0, S0());
      load_v(vp16base, kb0 + 1, S1());
      spec = true;
      load_er(S0(), kb0);
      const float* const z2 = p.z2 + (int64_t)slot * T_len;
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int i = q0w + 32 * qt + n;
        zq[qt] = i < T_len ? z2[i] : INFINITY;
      }
      const float* const rblk = p.a_off + (int64_t)(p.n_slots + slot) * nblk;
      const float* const zblk = p.a_off + (int64_t)(2 * p.n_slots + slot) * nblk;
      const float* const vblk = p.vmax + ((int64_t)b * p.n_slots + slot) * nblk;
      // each lane's first element of every range is read before any wait
      // (more than 64 blocks per range only at T above 4096 rows per
      // query block's reach)
      const int ka = kb0 + lane, kz = q0 / 64 + lane;
      float am = ka < nkb ? ablk[ka] : -INFINITY;
      float vm = ka < nkb ? vblk[ka] : 0.f;
      float rm = lane < nkb_qb ? rblk[lane] : -INFINITY;
      float zm = kz < nkb_qb ? zblk[kz] : INFINITY;
      for (int k = ka + 64; k < nkb; k += 64) {
        am = fmaxf(am, ablk[k]);
        vm = fmaxf(vm, vblk[k]);
      }
      for (int k = lane + 64; k < nkb_qb; k += 64) rm = fmaxf(rm, rblk[k]);
      for (int k = kz + 64; k < nkb_qb; k += 64) zm = fminf(zm, zblk[k]);
      am = wave_max(am);
      rm = wave_max(rm);
      zm = wave_min(zm);
      vm = wave_max(vm);
      factored = __builtin_isfinite(am) && __builtin_isfinite(rm) && __builtin_isfinite(zm) &&
                 zm >= am + rm - kFactorRange;
      // fp16 form: every V' this workgroup reads in fp16 range, and the row
      // factor at most 2^(14 - ceil(log2 T)) (see kF16Budget)
      const int lgT = T_len > 1 ? 32 - __clz(T_len - 1) : 0;
      form16 = factored && vm <= kF16Max && zm >= am + rm - (float)(kF16Budget - lgT);
      if constexpr (!kBf16) factored = form16;
      aoff = am;
      roff = rm;
      load_er(S1(), kb0 + 1);
    }
  }
  if (!spec) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int i = q0w + 32 * qt + n;
      zq[qt] = i < T_len ? load_as_f32(p.z, (int64_t)ph * p.z_sh + (int64_t)i * p.z_ss, p.z_dtype) * kLog2e
                         : INFINITY;
    }
  }

  if constexpr (kFactorable) {
    // F16: the fp16 form (E and V' in fp16, one MFMA per operand); else the
    // bf16 form with E as a hi + lo pair.  vpb is the V' copy of the form,
    // whose blocks kb0 and kb0 + 1 are already on their way to V slots 0 and
    // 1, as are the rho values of block kb0's window.
    auto run_factored = [&](auto f16tag, const auto* vpb) {
      constexpr bool F16 = decltype(f16tag)::value;
      using TE = typename std::conditional<F16, _Float16, T>::type;
      int vro[NDT], vroh[NDT];
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        vro[dt] = vt_read_offset<HD>(lane, dt, 0);
        vroh[dt] = vt_read_offset<HD>(lane, dt, 1);
      }
      // distance window of block j0: m in [0, RW) holds E(d), d = q0 - j0 + BM - m
      // (the window reversed), as a bf16 pair hi + lo (E - hi rounded), so E
      // costs no rounding beyond V''s; copy c holds window element c + k at k.
      // The fp32 rho log2 e values (r2) are loaded (branch-free, clamped index)
      // one block ahead, their exps written after the block's MFMAs into the
      // other slot.
      // Thread t < RW / 2 owns window elements 2t and 2t + 1 and also computes
      // 2t + 2, so that every copy is written in aligned 32-bit words: an even
      // copy c stores (2t, 2t + 1) at its position 2t - c, an odd one
      // (2t + 1, 2t + 2) at 2t + 1 - c (16-bit stores put two lanes on one
      // bank word).
      auto e_slot = [&](auto slot) {
        return reinterpret_cast<uint16_t(*)[8 * RWL]>(decltype(slot)::value ? eb1 : eb0);
      };
      auto ecopy = [](int c) { return c * RWL + (c ? 8 : 0); };
      // window of block jb into E slot `slot` from register set `set`
      auto store_er = [&](auto slot, auto set, int jb) {
        constexpr int S = decltype(set)::value;
        uint16_t(*const ew)[8 * RWL] = e_slot(slot);
        if (tid < RW / 2) {
          uint32_t hv[3], lv[3];  // hi and lo bits of window elements 2t, 2t + 1, 2t + 2
#pragma unroll
          for (int u = 0; u < 3; ++u) {
            const int m = 2 * tid + u;
            const int d = q0 - 64 * jb + BM - m;
            // A_k - A - R; -inf for a block whose keys all have alpha -inf
            const float x = m < RW && d >= 0 && d < T_len ? fast_exp2(er[S][u] + (ab[S] - aoff - roff)) : 0.f;
            if constexpr (F16) {
              hv[u] = Elem<_Float16>::pack2(x, 0.f) & 0xffffu;
              lv[u] = 0u;
            } else {
              hv[u] = Elem<T>::pack2(x, 0.f) & 0xffffu;
              lv[u] = Elem<T>::pack2(x - Elem<T>::lo(hv[u]), 0.f) & 0xffffu;
            }
          }
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const int e0 = c & 1;             // the word's first element: 2t + e0
            const int pos = 2 * tid + e0 - c;  // even: its position in copy c
            if (pos >= 0) {
              *reinterpret_cast<uint32_t*>(&ew[0][ecopy(c) + pos]) = hv[e0] | (hv[e0 + 1] << 16);
              if constexpr (!F16) *reinterpret_cast<uint32_t*>(&ew[1][ecopy(c) + pos]) = lv[e0] | (lv[e0 + 1] << 16);
            }
          }
        }
      };
      // lane (n, g), query tile qt reads keys jb + 0..7 (jb = j0 + 16 st + 8g)
      // of row i: window elements s .. s+7, s = BM - (i - q0) + 16 st + 8g, from
      // copy (s & 7) = (-(i - q0)) & 7 at element s - (s & 7): eo = the element
      // offset of the lane's first read in the slot
      int eo[QT];
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        const int il = q0w + 32 * qt + n - q0;
        const int ec = (-il) & 7;
        eo[qt] = ecopy(ec) + BM - il - ec + 8 * g;
      }

      // prologue: E of block kb0 in E slot 0 from register set 0 (V' of kb0
      // and kb0+1 land in V slots 0, 1; set 1 holds block kb0 + 1's inputs)
      store_er(S0(), S0(), kb0);
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(VN));
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      // block j in phase P: V'_j in V slot P % 3, E_j in E slot P % 2 (both
      // compile-time, so every LDS access names one array and none waits on
      // another slot's DMA).  E_{j+1} goes to the other E slot (from register
      // set (P + 1) % 2, loaded in block j - 1) and V'_{j+2} to V slot
      // (P + 2) % 3, both last read in block j-1; block j + 2's window inputs
      // go to register set P % 2 after that DMA.  The closing barrier waits
      // for everything issued before this block (vmcnt VN + 2: V'_{j+1} and
      // block j + 1's inputs; V'_{j+2} and block j + 2's inputs stay in
      // flight, a __syncthreads would drain them) and for this block's LDS
      // writes (lgkmcnt 0).
      auto block = [&](const int j, auto phase) {
        constexpr int PH = decltype(phase)::value;
        constexpr int R = PH % 3;
        using ESlot = std::integral_constant<int, PH % 2>;
        using ENext = std::integral_constant<int, 1 - PH % 2>;
        using VAhead = std::integral_constant<int, (R + 2) % 3>;
        using SetNow = std::integral_constant<int, (PH + 1) % 2>;
        using SetAhead = std::integral_constant<int, PH % 2>;
        const char* const vt = R == 0 ? vs0 : (R == 1 ? vs1 : vs2);
        uint16_t(*const ew)[8 * RWL] = e_slot(ESlot());
        load_v(vpb, j + 2, VAhead());
        load_er(SetAhead(), j + 2);
        if (j < nkb_w) {
          // Toeplitz reuse: query tile 1 sits 32 rows below tile 0, so its
          // operand of key step (1, sh) is tile 0's of step (0, sh)
          uint4 keep_b[2], keep_l[2];
#pragma unroll
          for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int sh = 0; sh < 2; ++sh) {
              uint4 pb[QT], pl[QT] = {};
#pragma unroll
              for (int qt = 0; qt < QT; ++qt) {
                if (QT == 2 && qt == 1 && ks == 1) {
                  pb[qt] = keep_b[sh];
                  pl[qt] = keep_l[sh];
                } else {
                  pb[qt] = *reinterpret_cast<const uint4*>(&ew[0][eo[qt] + 32 * ks + 16 * sh]);
                  if constexpr (!F16) pl[qt] = *reinterpret_cast<const uint4*>(&ew[1][eo[qt] + 32 * ks + 16 * sh]);
                }
              }
              if (ks == 0) {
                keep_b[sh] = pb[0];
                keep_l[sh] = pl[0];
              }
              uint4 a[NDT];
#pragma unroll
              for (int dt = 0; dt < NDT; ++dt) {
                const char* base = vt + (32 * ks + 16 * sh) * PITCH;
                const uint2 lo = ds_read_tr16(base + vro[dt]);
                const uint2 hi = ds_read_tr16(base + (VRow<HD>::M2 ? vroh[dt] : vro[dt] + 4 * PITCH));
                a[dt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
              }
              // the hi products of every accumulator, then the lo ones: no
              // MFMA waits on the one before it
#pragma unroll
              for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) o[qt][dt] = Elem<TE>::mfma(a[dt], pb[qt], o[qt][dt]);
              if constexpr (!F16) {
#pragma unroll
                for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
                  for (int qt = 0; qt < QT; ++qt) o[qt][dt] = Elem<TE>::mfma(a[dt], pl[qt], o[qt][dt]);
              }
            }
        }
        if (j + 1 < nkb) store_er(ENext(), SetNow(), j + 1);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(VN + 2));
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      };
      using Q0 = std::integral_constant<int, 0>;
      using Q1 = std::integral_constant<int, 1>;
      using Q2 = std::integral_constant<int, 2>;
      using Q3 = std::integral_constant<int, 3>;
      using Q4 = std::integral_constant<int, 4>;
      using Q5 = std::integral_constant<int, 5>;
      for (int j = kb0;;) {
        if (j >= nkb) break;
        block(j++, Q0());
        if (j >= nkb) break;
        block(j++, Q1());
        if (j >= nkb) break;
        block(j++, Q2());
        if (j >= nkb) break;
        block(j++, Q3());
        if (j >= nkb) break;
        block(j++, Q4());
        if (j >= nkb) break;
        block(j++, Q5());
      }
      // the last (empty) DMAs land before the workgroup's LDS is released
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) rowscale[qt] = fast_exp2(aoff + roff - zq[qt]);
    };
    if (factored) {
      if constexpr (kBf16) {
        if (form16) {
          run_factored(std::true_type(), vp16base);
        } else {
          // the bf16 copy replaces the fp16 one in V slots 0 and 1: each
          // thread's DMA chunks are its own, so its own earlier loads landing
          // first is all the order needed
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
          load_v(vpbase, kb0, S0());
          load_v(vpbase, kb0 + 1, S1());
          run_factored(std::false_type(), vpbase);
        }
      } else {
        run_factored(std::true_type(), vp16base);
      }
    }
  }
  if (!factored) {
    if (spec) {
      // the rebuild writes V slots 0 and 1 from every thread: the fp16 V'
      // loaded there for the factored form lands first
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
      __syncthreads();
    }
    // alpha[j0 + t] for t < 64 and rho[d] for d = dmin + t, t < RW,
    // dmin = q0 - j0 - 63.  Out-of-range distances are -inf (exact zero cells).
    auto v_lds = [&](int buf) { return reinterpret_cast<uint4*>(buf ? vs1 : vs0); };
    float(*const a_lds)[64] = reinterpret_cast<float(*)[64]>(eb0);
    float(*const r_lds)[RW] = reinterpret_cast<float(*)[RW]>(eb0 + 2 * 64 * 4);
    float a_reg = 0.f, r_reg[ERN];
    auto stage_params = [&](int j0) {
      if (tid < 64) {
        const int j = j0 + tid;
        a_reg = j < T_len ? alpha_at(j) * kLog2e : 0.f;
      }
      const int dmin = q0 - j0 - 63;
#pragma unroll
      for (int u = 0; u < ERN; ++u) {
        const int t = tid + u * NTHR;
        const int d = dmin + t;
        r_reg[u] = (t < RW && d >= 0 && d < T_len) ? rho_at(d) * kLog2e : -INFINITY;
      }
    };
    auto store_params = [&](int buf) {
      if (tid < 64) a_lds[buf][tid] = a_reg;
#pragma unroll
      for (int u = 0; u < ERN; ++u) {
        const int t = tid + u * NTHR;
        if (t < RW) r_lds[buf][t] = r_reg[u];
      }
    };

    VStager<T, HD, NTHR> vst;
    vst.load(vbase, p.v_st, 64 * kb0, T_len, tid);
    stage_params(64 * kb0);
    vst.store(reinterpret_cast<uint32_t*>(v_lds(0)), tid);
    store_params(0);
    __syncthreads();

    for (int j = kb0; j < nkb; ++j) {
      const int buf = (j - kb0) & 1;
      const bool more = j + 1 < nkb;
      if (more) {
        vst.load(vbase, p.v_st, 64 * (j + 1), T_len, tid);
        stage_params(64 * (j + 1));
      }
      if (j < nkb_w) {
        const int j0 = 64 * j;
        const uint4* vt = v_lds(buf);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int sh = 0; sh < 2; ++sh) {
            const int jb = j0 + 32 * ks + 16 * sh + 8 * g;
            uint4 pb[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
              const int i = q0w + 32 * qt + n;
              const int dbase = i - jb - (q0 - j0 - 63);  // index of d = i - jb in r_lds
              float e[8];
#pragma unroll
              for (int u = 0; u < 8; ++u)
                e[u] = fast_exp2(a_lds[buf][jb - j0 + u] + r_lds[buf][dbase - u] - zq[qt]);
              pb[qt] = make_uint4(Elem<T>::pack2(e[0], e[1]), Elem<T>::pack2(e[2], e[3]),
                                  Elem<T>::pack2(e[4], e[5]), Elem<T>::pack2(e[6], e[7]));
            }
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
              const uint4 a = vt[VLayout<HD>::chunk(32 * dt + n, 4 * ks + 2 * sh + g)];
#pragma unroll
              for (int qt = 0; qt < QT; ++qt) o[qt][dt] = Elem<T>::mfma(a, pb[qt], o[qt][dt]);
            }
          }
      }
      if (more) {
        vst.store(reinterpret_cast<uint32_t*>(v_lds(buf ^ 1)), tid);
        store_params(buf ^ 1);
      }
      __syncthreads();
    }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) rowscale[qt] = 1.f;
  }

  const bool split = p.n_items != 0 && p.part_base[qb] >= 0;
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int i = q0w + 32 * qt + n;
    if (i >= T_len) continue;
    const float sc = rowscale[qt];
    if (split) {  // plain-sum partial of this key segment, added up by the combine kernel
      const int64_t pidx = (int64_t)r * p.n_part_per_head + p.part_base[qb] + seg;
      float* po = p.part_o + (pidx * BM + (i - q0)) * HD;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4)
          *reinterpret_cast<float4*>(po + 32 * dt + 8 * r4 + 4 * g) =
              make_float4(o[qt][dt][4 * r4] * sc, o[qt][dt][4 * r4 + 1] * sc, o[qt][dt][4 * r4 + 2] * sc,
                          o[qt][dt][4 * r4 + 3] * sc);
    } else {
      store_out_tile<T, HD>(obase + (int64_t)i * p.o_st, o[qt], sc, g);
    }
  }
}

template <typename T, int HD, int QT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(decomp_waves_per_eu(HD), decomp_waves_per_eu(HD))))
void frozen_decomp_kernel(const FrozenParams p) {
  decomp_body<T, HD, QT>(p);
}

// vp[b, slot, j] = 2^(alpha_j log2 e - A_k) v[b, v_head, j] in T (and in
// fp16 in vp16, with the block's largest |value| in vmax[(b, slot), k]), with
// A_k = max alpha log2 e over the 64-key block k = j / 64 of the slot's head
// (a_off[slot * nblk + k], nblk = ceil(T / 64)).  Batch 0's workgroup also
// writes r2[slot, d] = rho_d log2 e for the block's 64 distances (the main
// kernel then reads rho as plain fp32) and their maximum
// a_off[(n_slots + slot) * nblk + k] (so a workgroup's R is a maximum over
// at most nblk values), and z2[slot, i] = z_i log2 e for the block's 64 rows
// with their minimum a_off[(2 n_slots + slot) * nblk + k] (the main kernel's
// row normalisers and the smallest z of its rows).  One workgroup per (key
// block, slot, batch); every wave reduces the block's alpha itself, so
// nothing orders workgroups.  vp
// holds T rows per (batch, slot); the main kernel's buffer-resource bound
// reads rows past T as zero.
template <typename T, int HD>
__global__ __launch_bounds__(256) void decomp_prescale_kernel(const FrozenParams p) {
  constexpr int CH = HD / 8;          // 16-byte chunks per row
  constexpr int PER = 64 * CH / 256;  // chunks per thread
  static_assert(64 * CH % 256 == 0, "a key block's chunks split evenly over the threads");
  const int kb = blockIdx.x, slot = blockIdx.y, b = blockIdx.z, j0 = 64 * kb;
  const int tid = threadIdx.x, lane = tid & 63;
  const int ph = p.pat_head[slot];
  const T* vbase = reinterpret_cast<const T*>(p.v) + b * p.v_sb + (int64_t)arg_i16(p.v_head, slot) * p.v_sh;
  uint4 w[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int idx = tid + 256 * u, row = j0 + idx / CH, c = idx % CH;
    w[u] = row < p.T ? *reinterpret_cast<const uint4*>(vbase + (int64_t)row * p.v_st + 8 * c) : make_uint4(0, 0, 0, 0);
  }
  const float al =
      j0 + lane < p.T ? load_as_f32(p.alpha, (int64_t)ph * p.a_sh + (int64_t)(j0 + lane) * p.a_ss, p.a_dtype) * kLog2e
                      : -INFINITY;
  const float am = wave_max(al);
  if (b == 0) {
    const int nblk = (p.T + 63) / 64;
    if (tid == 0) p.a_off[(int64_t)slot * nblk + kb] = am;
    if (tid >= 64 && tid < 128) {  // wave 1: the block's distances
      const float rv = j0 + lane < p.T
                           ? load_as_f32(p.rho, (int64_t)ph * p.r_sh + (int64_t)(j0 + lane) * p.r_ss, p.r_dtype) * kLog2e
                           : -INFINITY;
      if (j0 + lane < p.T) p.r2[(int64_t)slot * p.T + j0 + lane] = rv;
      const float rmx = wave_max(rv);
      if (lane == 0) p.a_off[(int64_t)(p.n_slots + slot) * nblk + kb] = rmx;
    }
    if (tid >= 128 && tid < 192) {  // wave 2: the block's rows
      const float zv = j0 + lane < p.T
                           ? load_as_f32(p.z, (int64_t)ph * p.z_sh + (int64_t)(j0 + lane) * p.z_ss, p.z_dtype) * kLog2e
                           : INFINITY;
      if (j0 + lane < p.T) p.z2[(int64_t)slot * p.T + j0 + lane] = zv;
      const float zmn = wave_min(zv);
      if (lane == 0) p.a_off[(int64_t)(2 * p.n_slots + slot) * nblk + kb] = zmn;
    }
  }
  const int64_t row0 = ((int64_t)b * p.n_slots + slot) * p.T;
  T* vp = reinterpret_cast<T*>(p.vp) + row0 * HD;
  _Float16* vp16 = reinterpret_cast<_Float16*>(p.vp16) + row0 * HD;
  float vmx = 0.f;  // largest |V'| of this block (NaN inputs are left to the bf16 copy)
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int idx = tid + 256 * u, rl = idx / CH, c = idx % CH;
    const float ar = __shfl(al, rl);
    const float f = ar == -INFINITY ? 0.f : fast_exp2(ar - am);  // am is finite when ar is
    if (j0 + rl < p.T) {
      const uint32_t in[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
      uint32_t out[4], out16[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const float x0 = Elem<T>::lo(in[m]) * f, x1 = Elem<T>::hi(in[m]) * f;
        out[m] = Elem<T>::pack2(x0, x1);
        out16[m] = Elem<_Float16>::pack2(x0, x1);
        vmx = fmaxf(vmx, fmaxf(fabsf(x0), fabsf(x1)));
      }
      if constexpr (std::is_same<T, __bf16>::value)  // the bf16 forms' copy (fp16 inputs have only the fp16 form)
        *reinterpret_cast<uint4*>(vp + (int64_t)(j0 + rl) * HD + 8 * c) = make_uint4(out[0], out[1], out[2], out[3]);
      *reinterpret_cast<uint4*>(vp16 + (int64_t)(j0 + rl) * HD + 8 * c) =
          make_uint4(out16[0], out16[1], out16[2], out16[3]);
    }
  }
  __shared__ float red[4];
  vmx = wave_max(vmx);
  if (lane == 0) red[tid >> 6] = vmx;
  __syncthreads();
  if (tid == 0)
    p.vmax[((int64_t)b * p.n_slots + slot) * ((p.T + 63) / 64) + kb] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}


// Pattern element types: 8 consecutive elements -> 8 floats.
template <typename PT> struct PatVec;
template <> struct PatVec<float> {
  __device__ static inline void load8(const float* src, float (&e)[8]) {
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    e[0] = a.x; e[1] = a.y; e[2] = a.z; e[3] = a.w; e[4] = b.x; e[5] = b.y; e[6] = b.z; e[7] = b.w;
  }
  __device__ static inline float one(const float* src) { return *src; }
};
template <typename H> struct PatVec16 {
  __device__ static inline void load8(const H* src, float (&e)[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(src);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      e[2 * m] = Elem<H>::lo(w[m]);
      e[2 * m + 1] = Elem<H>::hi(w[m]);
    }
  }
  __device__ static inline float one(const H* src) { return (float)*src; }
};
template <> struct PatVec<__bf16> : PatVec16<__bf16> {};
template <> struct PatVec<_Float16> : PatVec16<_Float16> {};

// Keep the first n (0..8) 16-bit elements of a packed chunk, zero the rest.
__device__ inline uint4 keep_leading(uint4 w, int n) {
  uint32_t d[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int m = 0; m < 4; ++m) d[m] = 2 * m + 1 < n ? d[m] : (2 * m < n ? d[m] & 0xffffu : 0u);
  return make_uint4(d[0], d[1], d[2], d[3]);
}

// One B-operand chunk of P^T: keys kstart .. kstart+7 of one query row in
// the activation dtype, the first `nvalid` kept (keys past the query and rows
// past T are zero; nvalid <= 0 loads nothing).  Same-dtype patterns are used
// as loaded; others are widened and rounded once.  A chunk that would cross
// the row end, or a pattern not laid out for 16-byte loads, is read element
// by element (only the kept elements).
template <typename T, typename PT>
__device__ inline uint4 p_chunk(const FrozenParams& p, const PT* prow, int kstart, int nvalid) {
  if (nvalid <= 0) return make_uint4(0, 0, 0, 0);
  const bool vec = p.patt_vec && kstart + 8 <= p.p_cols;
  if constexpr (std::is_same<PT, T>::value) {
    if (vec) {
      const uint4 w = *reinterpret_cast<const uint4*>(prow + kstart);
      return nvalid < 8 ? keep_leading(w, nvalid) : w;
    }
  }
  float e[8];
  if (vec) {
    PatVec<PT>::load8(prow + kstart, e);
  } else {
#pragma unroll
    for (int m = 0; m < 8; ++m) e[m] = m < nvalid ? PatVec<PT>::one(prow + (int64_t)(kstart + m) * p.p_sj) : 0.f;
  }
#pragma unroll
  for (int m = 0; m < 8; ++m) e[m] = m < nvalid ? e[m] : 0.f;
  return make_uint4(Elem<T>::pack2(e[0], e[1]), Elem<T>::pack2(e[2], e[3]), Elem<T>::pack2(e[4], e[5]),
                    Elem<T>::pack2(e[6], e[7]));
}

// Per-wave state of the dense P.V kernel (below): the lane's pattern rows,
// the V DMA and V^T read offsets, and the O^T accumulators of NB sequences.
template <typename T, typename PT, int HD, int QT, int NB, int NW, bool FAST>
struct DenseState {
  static constexpr int NDT = HD / 32;
  static constexpr int VB = VRow<HD>::BYTES;
  static constexpr int PITCH = VRow<HD>::PITCH;
  static constexpr int VN = VRow<HD>::CHP / NW;  // DMA chunks per thread per V tile
  static_assert(VRow<HD>::CHP % NW == 0, "V tile chunks must split evenly over the waves");
  // end-of-block wait: this wave's V_{j+1} DMA has landed.  Fast path: the
  // loads issued after it (P_{j+1}, V_{j+2}, P_{j+2}) may stay in flight.
  static constexpr int kWaitV = waitcnt_vm(FAST ? 8 * QT + NB * VN : 0);
  const T* vbase[NB];
  int64_t v_st;
  int T_len, wave, g, q0w;
  int row[QT];
  const PT* prow[QT];    // general path: the lane's pattern rows
  uint32_t poff[QT];     // fast path: byte offset of key 8g of the row in the descriptor
  __amdgpu_buffer_rsrc_t prs;
  uint32_t voff[VN];
  int vro[NDT], vroh[NDT];  // V^T tr-read pair offsets of d tile dt
  f32x16_t o[NB][QT][NDT];

  // DMA of the 64-key V tiles of block j of the NB sequences into `tile`:
  // load pp of a wave writes chunk (NW pp + wave) * 64 + lane of each tile
  __device__ __forceinline__ void load_v(int j, char* tile) const {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const __amdgpu_buffer_rsrc_t r = rows_rsrc(vbase[nb], v_st, 64 * j, T_len);
#pragma unroll
      for (int pp = 0; pp < VN; ++pp)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, SAF_LDS_PTR(tile + nb * VB + (NW * pp + wave) * 1024), 16,
                                                 voff[pp], 0, 0, 0);
    }
  }

  // P^T operand of key step (ks, sh) of block j for query tile qt.  Fast
  // path: one raw buffer load; keys past the row and rows past T are
  // cleared at use (mask_p).  General path: masked and widened here.
  __device__ __forceinline__ uint4 p_op(const FrozenParams& p, int j, int ks, int sh, int qt) const {
    if constexpr (FAST) {
      // per-lane part in the VGPR offset (row, 8g, step), the block in the
      // scalar offset: no per-block address arithmetic in vector registers
      return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                           prs, poff[qt] + (uint32_t)(64 * ks + 32 * sh), 128 * j, 0));
    } else {
      const int kstart = 64 * j + 32 * ks + 16 * sh + 8 * g;
      const int nvalid = row[qt] < T_len ? min(row[qt] - kstart + 1, 8) : 0;
      return p_chunk<T, PT>(p, prow[qt], kstart, nvalid);
    }
  }
  __device__ __forceinline__ void load_p(const FrozenParams& p, uint4 (&pb)[2][2][QT], int j) const {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int sh = 0; sh < 2; ++sh)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) pb[ks][sh][qt] = p_op(p, j, ks, sh, qt);
  }
  __device__ __forceinline__ void mask_p(uint4 (&pb)[2][2][QT], int j) const {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int sh = 0; sh < 2; ++sh)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
          const int kstart = 64 * j + 32 * ks + 16 * sh + 8 * g;
          const int nvalid = row[qt] < T_len ? min(row[qt] - kstart + 1, 8) : 0;
          pb[ks][sh][qt] = keep_leading(pb[ks][sh][qt], nvalid);
        }
  }

  // V^T operands of every d tile for 16-key step k (keys 16k..16k+15 of the
  // block) of sequence nb
  __device__ __forceinline__ void read_vt(const char* cur, int k, int nb, uint4 (&a)[NDT]) const {
    const char* base = cur + nb * VB + 16 * k * PITCH;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      const uint2 lo = ds_read_tr16(base + vro[dt]);
      const uint2 hi = ds_read_tr16(base + (VRow<HD>::M2 ? vroh[dt] : vro[dt] + 4 * PITCH));
      a[dt] = make_uint4(lo.x, lo.y, hi.x, hi.y);
    }
  }

  // O^T += V^T P^T for one 64-key block (V tiles at `cur`), in 4 NB steps
  // (16 keys, one sequence): the V^T operands of step t + 1 are read while
  // the MFMAs of step t run, in two register sets, so each group of NDT QT
  // MFMAs waits for reads issued one group earlier (read next to its MFMA,
  // every MFMA waited for a full LDS round trip)
  __device__ __forceinline__ void mma_block(const char* cur, const uint4 (&pb)[2][2][QT]) {
    constexpr int NS = 4 * NB;
    uint4 a[2][NDT];
    read_vt(cur, 0, 0, a[0]);
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      if (t + 1 < NS) read_vt(cur, (t + 1) / NB, (t + 1) % NB, a[(t + 1) & 1]);
      // keep the order: the scheduler otherwise sinks each read next to its
      // MFMA again to save registers
      __builtin_amdgcn_sched_barrier(0);
      const int k = t / NB, nb = t % NB;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          o[nb][qt][dt] = Elem<T>::mfma(a[t & 1][dt], pb[k >> 1][k & 1][qt], o[nb][qt][dt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Block j of the key range [kb0, kb1) (this wave's rows reach blocks
  // < kb1_w): V_j in `cur` and P_j in `pc` (loaded two blocks earlier);
  // V_{j+2} -> `fut`, P_{j+2} -> `pf`.  In the fast path the loads are issued
  // unconditionally (past the end they read zeros or data that is never
  // used), so the compiler's own waits before the MFMAs count exactly the
  // loads issued after P_j.
  __device__ __forceinline__ void block(const FrozenParams& p, int j, int kb1, int kb1_w, const char* cur,
                                        char* fut, uint4 (&pc)[2][2][QT], uint4 (&pf)[2][2][QT]) {
    if (FAST || j + 2 < kb1) load_v(j + 2, fut);
    asm volatile("" ::: "memory");
    if (FAST || j + 2 < kb1_w) load_p(p, pf, j + 2);
    asm volatile("" ::: "memory");
    if (j < kb1_w) {
      if (FAST && (64 * j + 63 > q0w || q0w + 32 * QT > T_len)) {
        // a diagonal block or the last rows: clear keys past each row and rows past T
        asm volatile("" ::: "memory");
        mask_p(pc, j);
      }
      mma_block(cur, pc);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitV);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  }
};

// Dense P.V.  Each lane loads its own B operands straight from the pattern
// rows (lane (n, g): query n of a 32-row tile, keys 8g + 0..7 of each 16-key
// step = one 16-byte read), so P needs no LDS staging.  A workgroup of NW = 8
// waves (256 query rows, two waves per SIMD) serves NB batch elements of one
// head: every P^T operand feeds the MFMAs of all NB of them, so the pattern
// (the dominant traffic) is read from HBM once per NB sequences, and each V
// tile is shared by 256 rows.  The V tiles of the NB sequences arrive by
// buffer_load ... lds DMA into three static LDS slots (the VRow layout of the
// live-head kernel); their V^T operands come from transposing
// ds_read_b64_tr_b16 reads.
//
// The kernel is latency-bound unless enough bytes are in flight, so V and P
// run two blocks ahead: block j issues the DMA of V_{j+2} and the P^T loads
// of block j+2 (a third register set), then the MFMAs of block j.  When the
// pattern is in the activation dtype with 16-byte rows (FAST) every P load is
// one unconditional buffer load, so a wave knows how many loads were issued
// after its V_{j+1} DMA: it waits for exactly those to remain (vmcnt) and
// meets the others at a bare s_barrier; a __syncthreads would drain the
// pattern loads at every block.  Other pattern dtypes wait for vmcnt 0.
// Work items cover a key segment of a query block; split blocks write fp32
// partials that the combine kernel sums.
template <typename T, typename PT, int HD, int QT, int NB, bool FAST>
__global__ __launch_bounds__(64 * kDenseWaves) __attribute__((amdgpu_waves_per_eu(2, 2)))
void frozen_dense_kernel(const FrozenParams p) {
  constexpr int NW = kDenseWaves;
  using St = DenseState<T, PT, HD, QT, NB, NW, FAST>;
  constexpr int BM = NW * 32 * QT;
  constexpr int NDT = St::NDT;
  static_assert(NB * QT * NDT <= 8, "accumulators must fit two waves per SIMD");
  static_assert(!FAST || std::is_same<T, PT>::value, "the fast path loads the pattern in the activation dtype");
  __shared__ __align__(16) char vs0[NB * St::VB], vs1[NB * St::VB], vs2[NB * St::VB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31, g = lane >> 5;

  // XCD-aware order: workgroup i runs on XCD i % 8; the batch-group siblings
  // of a (work item, head) group get ids 8 apart (same XCD, dispatched
  // together, so later ones read the P tiles from that XCD's L2); items
  // heaviest first.
  const int nbg = p.B / NB;
  const int x = blockIdx.x & 7, t8 = blockIdx.x >> 3;
  const int bg = t8 % nbg, grp = 8 * (t8 / nbg) + x;
  const int n_work = p.n_items ? p.n_items : p.n_qblk;
  if (grp >= n_work * p.n_slots) return;
  const int it = grp / p.n_slots, slot = grp % p.n_slots;
  // item word (index clamped, no branch) and head tables (scalar word
  // reads) issued together, ahead of any wait
  const int w_item = p.items[min(it, kMaxItems - 1)];
  const int qb = __builtin_amdgcn_readfirstlane(p.n_items ? w_item >> 8 : p.n_qblk - 1 - it);
  const int seg = __builtin_amdgcn_readfirstlane(p.n_items ? w_item & 255 : 0);
  const int h = arg_i16(p.out_head, slot);
  const int64_t pat_off = (int64_t)arg_i16(p.pat_head, slot) * p.p_sh;
  const PT* pbase = reinterpret_cast<const PT*>(p.patt) + pat_off;

  const int T_len = p.T;
  const int q0 = qb * BM;
  const int nkb = (min(q0 + BM, T_len) + 63) / 64;
  // an unsplit query block's item is segment 0 and spans at most seg_len
  // blocks: the range needs no part_base lookup (read for the epilogue)
  const int kb0 = p.n_items ? seg * p.seg_len : 0;
  const int kb1 = p.n_items ? min(nkb, kb0 + p.seg_len) : nkb;

  St st;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
    st.vbase[nb] = reinterpret_cast<const T*>(p.v) + (int64_t)(bg * NB + nb) * p.v_sb + (int64_t)arg_i16(p.v_head, slot) * p.v_sh;
  st.v_st = p.v_st;
  st.T_len = T_len;
  st.wave = wave;
  st.g = g;
  st.q0w = q0 + wave * 32 * QT;
  const int kend_w = min(st.q0w + 32 * QT, T_len);
  const int kb1_w = min(kb1, kend_w > 0 ? (kend_w + 63) / 64 : 0);  // blocks this wave's rows reach
#pragma unroll
  for (int pp = 0; pp < St::VN; ++pp) st.voff[pp] = vrow_dma_offset<T, HD>((NW * pp + wave) * 64 + lane, p.v_st);
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    st.vro[dt] = vt_read_offset<HD>(lane, dt, 0);
    st.vroh[dt] = vt_read_offset<HD>(lane, dt, 1);
  }
  // pattern rows of this lane (rows past T read row T-1 and are masked); the
  // descriptor runs from the workgroup's first pattern row to the end of the
  // buffer
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    st.row[qt] = st.q0w + 32 * qt + n;
    const int rc = min(st.row[qt], T_len - 1);
    st.prow[qt] = pbase + (int64_t)rc * p.p_si;
    st.poff[qt] = (uint32_t)((int64_t)(rc - q0) * p.p_si * (int64_t)sizeof(PT)) + 16u * g;
  }
  const int64_t pfirst = pat_off + (int64_t)q0 * p.p_si;
  st.prs = span_rsrc(reinterpret_cast<const PT*>(p.patt) + pfirst, (p.patt_elems - pfirst) * (int64_t)sizeof(PT));
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) st.o[nb][qt][dt] = zero16();

  // prologue: blocks kb0 and kb0+1 in flight, then V_kb0 landed everywhere
  uint4 pA[2][2][QT], pB[2][2][QT], pC[2][2][QT];
  st.load_v(kb0, vs0);
  asm volatile("" ::: "memory");
  if (FAST || kb0 < kb1_w) st.load_p(p, pA, kb0);
  asm volatile("" ::: "memory");
  if (FAST || kb0 + 1 < kb1) st.load_v(kb0 + 1, vs1);
  asm volatile("" ::: "memory");
  if (FAST || kb0 + 1 < kb1_w) st.load_p(p, pB, kb0 + 1);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(St::kWaitV);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  // three blocks per iteration, so every DMA target and read names a static
  // slot and register set.  The iteration is straight-line (blocks past kb1
  // issue their loads and barrier but no MFMAs): the compiler then counts
  // the loads in flight across the back edge exactly.
  for (int j = kb0; j < kb1; j += 3) {
    st.block(p, j, kb1, kb1_w, vs0, vs2, pA, pC);
    st.block(p, j + 1, kb1, kb1_w, vs1, vs0, pB, pA);
    st.block(p, j + 2, kb1, kb1_w, vs2, vs1, pC, pB);
  }

  const bool split = p.n_items != 0 && p.part_base[qb] >= 0;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int b = bg * NB + nb;
    T* obase = reinterpret_cast<T*>(p.out) + b * p.o_sb + (int64_t)h * p.o_sh;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int i = st.row[qt];
      if (i >= T_len) continue;
      if (split) {
        const int64_t pidx = ((int64_t)b * p.n_slots + slot) * p.n_part_per_head + p.part_base[qb] + seg;
        float* po = p.part_o + (pidx * BM + (i - q0)) * HD;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            *reinterpret_cast<float4*>(po + 32 * dt + 8 * r4 + 4 * g) =
                make_float4(st.o[nb][qt][dt][4 * r4], st.o[nb][qt][dt][4 * r4 + 1], st.o[nb][qt][dt][4 * r4 + 2],
                            st.o[nb][qt][dt][4 * r4 + 3]);
      } else {
        store_out_tile<T, HD>(obase + (int64_t)i * p.o_st, st.o[nb][qt], 1.f, g);
      }
    }
  }
}

template <typename T, typename PT, int HD, int NB>
static void launch_dense_t(const FrozenParams& p, hipStream_t s) {
  constexpr int QT = dense_qtiles(HD, NB);
  const int64_t groups = (int64_t)(p.n_items ? p.n_items : p.n_qblk) * p.n_slots;
  const dim3 grid((unsigned)(8 * (p.B / NB) * ((groups + 7) / 8)));
  if constexpr (std::is_same<T, PT>::value) {
    if (p.patt_vec) {
      hipLaunchKernelGGL((frozen_dense_kernel<T, PT, HD, QT, NB, true>), grid, dim3(64 * kDenseWaves), 0, s, p);
      return;
    }
  }
  hipLaunchKernelGGL((frozen_dense_kernel<T, PT, HD, QT, NB, false>), grid, dim3(64 * kDenseWaves), 0, s, p);
}

template <typename T, typename PT, int HD>
static void launch_dense_nb(const FrozenParams& p, hipStream_t s) {
  if constexpr (HD <= 64) {
    if (dense_batch_group(p.B, HD) == 4) {
      launch_dense_t<T, PT, HD, 4>(p, s);
      return;
    }
  }
  if constexpr (HD <= 128) {
    if (dense_batch_group(p.B, HD) == 2) {
      launch_dense_t<T, PT, HD, 2>(p, s);
      return;
    }
  }
  launch_dense_t<T, PT, HD, 1>(p, s);
}

template <typename T, int HD, int QT>
static hipError_t launch_frozen_t(const FrozenParams& p, int mode, hipStream_t s) {
  if (mode == 0) {
    if (p.patt_dtype == kF32)
      launch_dense_nb<T, float, HD>(p, s);
    else if (p.patt_dtype == kBF16)
      launch_dense_nb<T, __bf16, HD>(p, s);
    else
      launch_dense_nb<T, _Float16, HD>(p, s);
  } else {
    const dim3 grid((unsigned)((int64_t)(p.n_items ? p.n_items : p.n_qblk) * p.B * p.n_slots));
    hipLaunchKernelGGL((frozen_decomp_kernel<T, HD, QT>), grid, dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_frozen_hd(const FrozenParams& p, int hd, int mode, hipStream_t s) {
  switch (hd) {
    case 32: return launch_frozen_t<T, 32, 2>(p, mode, s);
    case 64: return launch_frozen_t<T, 64, 2>(p, mode, s);
    case 96: return launch_frozen_t<T, 96, 1>(p, mode, s);
    case 128: return launch_frozen_t<T, 128, 1>(p, mode, s);
    case 256: return launch_frozen_t<T, 256, 1>(p, mode, s);
    default: return hipErrorInvalidValue;
  }
}


template <typename T, int HD>
static hipError_t launch_prescale_hd(const FrozenParams& p, hipStream_t s) {
  const dim3 grid((unsigned)((p.T + 63) / 64), (unsigned)p.n_slots, (unsigned)p.B);
  hipLaunchKernelGGL((decomp_prescale_kernel<T, HD>), grid, dim3(256), 0, s, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_prescale_t(const FrozenParams& p, int hd, hipStream_t s) {
  switch (hd) {
    case 32: return launch_prescale_hd<T, 32>(p, s);
    case 64: return launch_prescale_hd<T, 64>(p, s);
    case 96: return launch_prescale_hd<T, 96>(p, s);
    case 128: return launch_prescale_hd<T, 128>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decomp_prescale(const FrozenParams& p, int dtype, int hd, hipStream_t s) {
  if (dtype == kBF16) return launch_prescale_t<__bf16>(p, hd, s);
  if (dtype == kF16) return launch_prescale_t<_Float16>(p, hd, s);
  return hipErrorInvalidValue;
}

hipError_t launch_frozen_pv(const FrozenParams& p, int dtype, int hd, int mode, hipStream_t s) {
  if (dtype == kF32) return launch_f32_frozen(p, hd, mode, s);
  if (dtype == kBF16) return launch_frozen_hd<__bf16>(p, hd, mode, s);
  if (dtype == kF16) return launch_frozen_hd<_Float16>(p, hd, mode, s);
  return hipErrorInvalidValue;
}

}  // namespace saf
