// Host side of libsafattn.so: argument validation, head routing and kernel
// launches behind the C-ABI declared in include/saf_attn.h.
//
// Routing follows the reference's per-head state machine
// (/root/reference/nanogpt/model.py:846-898, kernel/fused_attn.py:650-734,
// qwen/kernel/fused_attn.py:667-768): state 0 heads read Q/K slot hidx[h]
// (and K/V head kvidx[h] under a GQA map), state 1 heads read pattern row
// pidx[h] (identity when absent), state 2 heads read row h of alpha/rho/z.
// Each head kind becomes its own kernel launch over a compact head list, and
// every kernel writes its heads' rows of the natural-order output directly.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>
#include <vector>

#include "saf_attn.h"
#include "saf_kernels.h"

using namespace saf;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

bool present(const saf_tensor_t& t) { return t.data != nullptr; }

int elem_size(int dtype) { return dtype == SAF_F32 || dtype == SAF_I32 ? 4 : 2; }

const char* dtype_name(int d) {
  switch (d) {
    case SAF_F32: return "float32";
    case SAF_F16: return "float16";
    case SAF_BF16: return "bfloat16";
    case SAF_I32: return "int32";
    default: return "unknown";
  }
}

// Row-aligned 4-D activation: stride[3] == 1, base and row strides aligned to
// `align` bytes.
int check_act(const saf_tensor_t& t, const char* name, int align) {
  if (t.ndim != 4) return fail(SAF_EINVAL, "%s must be 4-D (got %d-D)", name, t.ndim);
  if (t.stride[3] != 1 && t.size[3] != 1)
    return fail(SAF_EALIGN, "%s must have a contiguous last dimension (stride %lld)", name,
                (long long)t.stride[3]);
  const int es = elem_size(t.dtype);
  if (reinterpret_cast<uintptr_t>(t.data) % align != 0)
    return fail(SAF_EALIGN, "%s data pointer is not %d-byte aligned", name, align);
  for (int i = 0; i < 3; ++i)
    if (t.size[i] > 1 && (t.stride[i] * es) % align != 0)
      return fail(SAF_EALIGN, "%s stride %d (%lld elements) is not a multiple of %d bytes", name, i,
                  (long long)t.stride[i], align);
  // the kernels walk rows through 32-bit buffer descriptors (RowCursor)
  if (t.size[2] > 1 && (t.stride[2] < 0 || t.stride[2] * es >= kMaxRowBytes))
    return fail(SAF_EUNSUPPORTED, "%s row stride (%lld elements) must be below %d bytes", name,
                (long long)t.stride[2], kMaxRowBytes);
  return SAF_OK;
}

// Head dims of the forward kernels; the backward kernels and the fused
// RoPE / q-k norm prologue stop at 128.
bool supported_hd(int64_t hd) { return hd == 32 || hd == 64 || hd == 96 || hd == 128 || hd == 256; }
bool supported_bwd_hd(int64_t hd) { return hd == 32 || hd == 64 || hd == 96 || hd == 128; }

int n_scan_chunks(int T, int hd) { return (T + scan_chunk_rows(hd) - 1) / scan_chunk_rows(hd); }

// Workspace: [reserved u32, error u32, pad to 256] [status u64 x n] with
// n = n_seq * n_chunks * hd; the whole block is cleared before a scan.
struct WsLayout {
  int64_t status_off, total;
};

WsLayout ws_layout(int64_t B, int64_t T, int hd, int64_t n_scan) {
  WsLayout w{0, 0};
  if (n_scan <= 0 || T <= 0 || B <= 0) return w;
  const int64_t n = B * n_scan * n_scan_chunks((int)T, hd) * hd;
  w.status_off = 256;
  w.total = w.status_off + 8 * n;
  return w;
}

// Bytes of the workspace used by the closed-form scan (placed first).
struct Plan;
int64_t scan_ws_bytes(const Plan& pl);

enum Which : unsigned { kDoFlash = 1, kDoDense = 2, kDoDecomp = 4, kDoScan = 8, kDoAll = 15 };

struct Plan {
  int B = 0, T = 0, H = 0, HD = 0, HV = 0, dtype = 0;
  std::vector<int> live, dense, decomp, scan;
};

int plan_and_validate(const saf_mixed_attn_args* a, unsigned which, Plan& pl, bool need_workspace = true) {
  if (a == nullptr) return fail(SAF_EINVAL, "args is NULL");
  const saf_tensor_t& v = a->v;
  if (!present(v)) return fail(SAF_EINVAL, "v is required");
  if (v.ndim != 4) return fail(SAF_EINVAL, "q, k, v must be 4-D");
  if (v.dtype != SAF_BF16 && v.dtype != SAF_F16 && v.dtype != SAF_F32)
    return fail(SAF_EUNSUPPORTED, "unsupported v dtype %s", dtype_name(v.dtype));
  pl.B = (int)v.size[0];
  pl.HV = (int)v.size[1];
  pl.T = (int)v.size[2];
  pl.HD = (int)v.size[3];
  pl.dtype = v.dtype;
  pl.H = a->n_heads;
  if (!supported_hd(pl.HD))
    return fail(SAF_EUNSUPPORTED, "head_dim %d is not supported (32, 64, 96, 128, 256)", pl.HD);
  if (pl.H <= 0 || pl.H > SAF_MAX_HEADS)
    return fail(SAF_EUNSUPPORTED, "n_heads %d outside 1..%d", pl.H, SAF_MAX_HEADS);
  if (a->frozen == nullptr) return fail(SAF_EINVAL, "frozen (host head-state table) is required");
  if (a->kvidx == nullptr && pl.HV != pl.H)
    return fail(SAF_EINVAL, "v must hold one head per output head (or pass kvidx)");
  if (int rc = check_act(v, "v", 16)) return rc;

  const saf_tensor_t& o = a->out;
  if (!present(o)) return fail(SAF_EINVAL, "out is required");
  if (o.ndim != 4 || o.size[0] != pl.B || o.size[1] != pl.H || o.size[2] != pl.T || o.size[3] != pl.HD)
    return fail(SAF_EINVAL, "out must have shape (B, H, T, HD) = (%d, %d, %d, %d)", pl.B, pl.H, pl.T, pl.HD);
  if (o.dtype != v.dtype) return fail(SAF_EINVAL, "out dtype must match v");
  if (int rc = check_act(o, "out", 8)) return rc;

  for (int h = 0; h < pl.H; ++h) {
    const int st = a->frozen[h];
    if (st < 0 || st > 2) return fail(SAF_EINVAL, "frozen[%d] = %d is not a head state (0, 1, 2)", h, st);
    if (a->kvidx && (a->kvidx[h] < 0 || a->kvidx[h] >= pl.HV))
      return fail(SAF_EINVAL, "kvidx must index the HKV heads of k/v (kvidx[%d] = %d)", h, a->kvidx[h]);
    if (st == 0) {
      pl.live.push_back(h);
    } else if (st == 1) {
      pl.dense.push_back(h);
    } else {
      const int ck = a->closed_kind ? a->closed_kind[h] : SAF_CLOSED_NONE;
      if (ck < SAF_CLOSED_NONE || ck > SAF_CLOSED_WINDOW)
        return fail(SAF_EINVAL, "closed_kind[%d] = %d is not a closed form", h, ck);
      if (ck != SAF_CLOSED_NONE) {
        if (a->closed_param == nullptr) return fail(SAF_EINVAL, "closed_param is required with closed_kind");
        const float prm = a->closed_param[h];
        if (ck == SAF_CLOSED_DECAY && !(prm > 0.f && std::isfinite(prm)))
          return fail(SAF_EINVAL, "decay rate of head %d must be finite and > 0 (got %g)", h, prm);
        if (ck == SAF_CLOSED_WINDOW && !(prm >= 1.f && prm < 2.1e9f && prm == std::floor(prm)))
          return fail(SAF_EINVAL, "window length of head %d must be an integer >= 1 (got %g)", h, prm);
        // float32 inputs have no scan kernel: closed forms run through their
        // decomposed buffers with the other state-2 heads
        if (v.dtype == SAF_F32)
          pl.decomp.push_back(h);
        else
          pl.scan.push_back(h);
      } else {
        pl.decomp.push_back(h);
      }
    }
  }

  if ((which & kDoFlash) && !pl.live.empty()) {
    const saf_tensor_t& q = a->q;
    const saf_tensor_t& k = a->k;
    if (!present(q) || !present(k)) return fail(SAF_EINVAL, "live heads require q and k");
    if (q.ndim != 4 || k.ndim != 4) return fail(SAF_EINVAL, "q, k, v must be 4-D");
    if (q.dtype != v.dtype || k.dtype != v.dtype) return fail(SAF_EINVAL, "q, k and v must share a dtype");
    if (q.size[0] != pl.B || q.size[2] != pl.T || q.size[3] != pl.HD)
      return fail(SAF_EINVAL, "q/k batch, sequence, and head dimensions must match v");
    if (a->kvidx) {
      for (int i = 0; i < 4; ++i)
        if (k.size[i] != v.size[i]) return fail(SAF_EINVAL, "with kvidx, k and v are the raw (B, HKV, T, HD) heads");
    } else {
      for (int i = 0; i < 4; ++i)
        if (k.size[i] != q.size[i]) return fail(SAF_EINVAL, "q and k must have the same compact shape");
    }
    if (int rc = check_act(q, "q", 16)) return rc;
    if (int rc = check_act(k, "k", 16)) return rc;
    const int U = (int)q.size[1];
    for (int h : pl.live) {
      const int slot = a->hidx ? a->hidx[h] : h;
      if (slot < 0 || slot >= U)
        return fail(SAF_EINVAL, "hidx[%d] = %d does not index the %d compact q/k heads", h, slot, U);
    }
  }
  if ((which & kDoDense) && !pl.dense.empty()) {
    const saf_tensor_t& p = a->patt;
    if (!present(p)) return fail(SAF_EINVAL, "dense-frozen heads require patt");
    if (p.ndim != 3 || p.size[1] < pl.T || p.size[2] < pl.T)
      return fail(SAF_EINVAL, "patt must have shape (P, S, S) with S >= T");
    if (p.dtype != SAF_F32 && p.dtype != SAF_BF16 && p.dtype != SAF_F16)
      return fail(SAF_EUNSUPPORTED, "unsupported patt dtype %s", dtype_name(p.dtype));
    for (int h : pl.dense) {
      const int row = a->pidx ? a->pidx[h] : h;
      if (row < 0 || row >= p.size[0])
        return fail(a->pidx ? SAF_EINVAL : SAF_EINVAL,
                    a->pidx ? "pidx for dense-frozen heads must index patt (pidx[%d] = %d)"
                            : "identity pattern mapping requires at least H pattern rows (head %d)",
                    h, row);
    }
  }
  if ((which & kDoDecomp) && !pl.decomp.empty()) {
    const saf_tensor_t* bufs[3] = {&a->alpha, &a->rho, &a->z};
    const char* names[3] = {"alpha", "rho", "z"};
    for (int i = 0; i < 3; ++i) {
      const saf_tensor_t& t = *bufs[i];
      if (!present(t)) return fail(SAF_EINVAL, "decomposed-frozen heads require alpha/rho/z");
      if (t.ndim != 2 || t.size[0] != pl.H || t.size[1] < pl.T)
        return fail(SAF_EINVAL, "decomposed buffers must have shape (H, S) with S >= T (%s)", names[i]);
      if (t.dtype != SAF_F32 && t.dtype != SAF_BF16 && t.dtype != SAF_F16)
        return fail(SAF_EUNSUPPORTED, "unsupported %s dtype %s", names[i], dtype_name(t.dtype));
    }
  }
  if ((which & kDoScan) && !pl.scan.empty()) {
    // the scan addresses one chunk of rows with 32-bit buffer offsets
    const int64_t lim = (int64_t)1 << 31, es = 2, ch = scan_chunk_rows(pl.HD);
    if (v.stride[2] * es * ch >= lim || o.stride[2] * es * ch >= lim)
      return fail(SAF_EUNSUPPORTED, "closed-form heads: row stride of v or out too large (%lld x %lld rows >= 2 GiB)",
                  (long long)std::max(v.stride[2], o.stride[2]) * es, (long long)ch);
  }
  if (need_workspace && (which & kDoScan) && !pl.scan.empty()) {
    const WsLayout w = ws_layout(pl.B, pl.T, pl.HD, (int64_t)pl.scan.size());
    if (a->workspace == nullptr || a->workspace_bytes < w.total)
      return fail(SAF_EWORKSPACE, "closed-form heads need a %lld-byte workspace (got %lld)", (long long)w.total,
                  (long long)a->workspace_bytes);
    if (reinterpret_cast<uintptr_t>(a->workspace) % 256 != 0)
      return fail(SAF_EALIGN, "workspace must be 256-byte aligned");
  }
  return SAF_OK;
}

// ---- causal load balancing of the live-head kernel ------------------------
// Compute units of the current device, cached per device per thread.
int cu_count() {
  thread_local int cached_dev = -1, cached_cus = 0;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev != cached_dev) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    cached_dev = dev;
    cached_cus = cus;
  }
  return cached_cus;
}

// Resident live-head workgroups per CU (flash_waves_per_eu in the kernel:
// three 128-query workgroups at hd <= 64, two of 256 queries; one 8-wave
// workgroup at hd 96 / 128, where its LDS slots fill most of the CU; one
// 4-wave workgroup of 128 queries at hd 256, one wave per SIMD).
int flash_resident(int HD, int qt) { return HD <= 64 ? (qt == 1 ? 3 : 2) : 1; }

struct FlashPlan {
  int n_items = 0, seg_len = 0, n_part_per_head = 0, n_split = 0;
  std::vector<int32_t> items;
  std::vector<int16_t> part_base, split_qb;
  int64_t part_bytes = 0;  // workspace for the partials
};

// Splits the key range of the heaviest query blocks into segments of about
// the average per-slot work, so the causal tail (the last query block walks
// every key) does not outlast the rest of the grid.  B counts the work units
// per slot; each writes part_mult sequences' partials.
FlashPlan plan_flash(int B, int n_slots, int T, int HD, int BM, int per_cu, int part_mult = 1) {
  FlashPlan fp;
  const int BMb = BM / 64;
  const int nqb = (T + BM - 1) / BM;
  if (nqb <= 1 || nqb > kMaxQblk) return fp;
  std::vector<int> nkb(nqb);
  int64_t per_head = 0;
  for (int qb = 0; qb < nqb; ++qb) {
    nkb[qb] = (std::min((qb + 1) * BM, T) + 63) / 64;
    per_head += nkb[qb];
  }
  const int64_t nbh = (int64_t)B * n_slots;
  const int64_t slots = (int64_t)cu_count() * per_cu;
  int64_t L = (nbh * per_head + slots - 1) / slots;
  L = std::max<int64_t>(L, 4 * BMb);
  L = (L + BMb - 1) / BMb * BMb;
  for (;; L *= 2) {
    if (L >= nkb[nqb - 1]) return fp;  // nothing to split
    int64_t n = 0;
    for (int qb = 0; qb < nqb; ++qb) n += (nkb[qb] + L - 1) / L;
    if (n <= kMaxItems && L < 65536) break;
  }
  struct It { int len, qb, seg; };
  std::vector<It> its;
  fp.part_base.assign(kMaxQblk, (int16_t)-1);
  int parts = 0;
  for (int qb = 0; qb < nqb; ++qb) {
    const int nseg = (int)((nkb[qb] + L - 1) / L);
    if (nseg > 1) {
      fp.part_base[qb] = (int16_t)parts;
      fp.split_qb.push_back((int16_t)qb);
      parts += nseg;
    }
    for (int sg = 0; sg < nseg; ++sg) its.push_back({(int)std::min<int64_t>(L, nkb[qb] - sg * L), qb, sg});
  }
  std::stable_sort(its.begin(), its.end(), [](const It& a, const It& b) {
    return a.len != b.len ? a.len > b.len : a.qb > b.qb;
  });
  for (const It& it : its) fp.items.push_back((it.qb << 8) | it.seg);
  fp.n_items = (int)fp.items.size();
  fp.seg_len = (int)L;
  fp.n_part_per_head = parts;
  fp.n_split = (int)fp.split_qb.size();
  fp.part_bytes = nbh * part_mult * parts * (int64_t)BM * (HD + 2) * 4;
  return fp;
}

// Workspace bytes of the live-head kernel's work queue (one word used).
constexpr int64_t kQueueBytes = 256;

int flash_qtiles_for(const saf_mixed_attn_args* a, int HD) {
  int qt = a->flash_qtiles;
  // one query tile per wave by default; two (256-query workgroups) only up
  // to hd 64, where they fit two waves per SIMD
  if (qt == 0 || (qt == 2 && HD > 64)) qt = 1;
  return qt;
}

int64_t scan_ws_bytes(const Plan& pl) {
  const int64_t t = ws_layout(pl.B, pl.T, pl.HD, (int64_t)pl.scan.size()).total;
  return (t + 255) / 256 * 256;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(SAF_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return SAF_OK;
}

// Pending events of saf_time_next_kernel (per host thread, consumed by the
// next main kernel).
thread_local hipEvent_t g_time_begin = nullptr, g_time_end = nullptr;

// Runs launch() between the pending timing events, if any, on stream s.
template <class F>
hipError_t timed(F&& launch, hipStream_t s) {
  hipEvent_t b = g_time_begin, e = g_time_end;
  if (b == nullptr) return launch();
  g_time_begin = g_time_end = nullptr;
  hipError_t rc = hipEventRecord(b, s);
  if (rc == hipSuccess) rc = launch();
  if (rc == hipSuccess) rc = hipEventRecord(e, s);
  return rc;
}

int run_flash(const saf_mixed_attn_args* a, const Plan& pl, hipStream_t s) {
  if (pl.live.empty() || pl.T == 0 || pl.B == 0) return SAF_OK;
  FlashParams p{};
  p.q = a->q.data;
  p.k = a->k.data;
  p.v = a->v.data;
  p.out = a->out.data;
  p.lse = present(a->lse) ? reinterpret_cast<float*>(a->lse.data) : nullptr;
  p.q_sb = a->q.stride[0]; p.q_sh = a->q.stride[1]; p.q_st = a->q.stride[2];
  p.k_sb = a->k.stride[0]; p.k_sh = a->k.stride[1]; p.k_st = a->k.stride[2];
  p.v_sb = a->v.stride[0]; p.v_sh = a->v.stride[1]; p.v_st = a->v.stride[2];
  p.o_sb = a->out.stride[0]; p.o_sh = a->out.stride[1]; p.o_st = a->out.stride[2];
  if (p.lse) {
    const saf_tensor_t& l = a->lse;
    if (l.ndim != 3 || l.size[0] != pl.B || l.size[1] != pl.H || l.size[2] != pl.T || l.dtype != SAF_F32)
      return fail(SAF_EINVAL, "lse must be (B, H, T) float32");
    p.l_sb = l.stride[0]; p.l_sh = l.stride[1]; p.l_st = l.stride[2];
  }
  const int qt = flash_qtiles_for(a, pl.HD);
  if (qt != 1 && qt != 2) return fail(SAF_EINVAL, "flash_qtiles must be 0, 1 or 2");
  p.B = pl.B;
  p.T = pl.T;
  p.n_slots = (int)pl.live.size();
  const int BM = flash_block_rows(pl.HD, qt);
  p.n_qblk = (pl.T + BM - 1) / BM;
  p.scale_log2 = a->sm_scale * kLog2e;
  // split the causal tail when the caller's workspace holds the partials;
  // the workspace's first 256 bytes after the scan region hold the queue word
  FlashPlan fp = plan_flash(pl.B, p.n_slots, pl.T, pl.HD, BM, flash_resident(pl.HD, qt));
  const int64_t queue_off = scan_ws_bytes(pl), part_off = queue_off + kQueueBytes;
  const bool have_ws = a->workspace != nullptr && reinterpret_cast<uintptr_t>(a->workspace) % 16 == 0;
  // the work queue pays off for the one-workgroup-per-CU kernel above hd 64
  // (C3 flash 458 -> 426 us); at hd <= 64 the three resident workgroups per
  // CU keep the CUs fed and the queue measured 4% slower
  const bool f32 = pl.dtype == SAF_F32;  // the float32 kernel neither splits nor queues
  if (!f32 && pl.HD > 64 && have_ws && a->workspace_bytes >= part_off) {
    p.queue = reinterpret_cast<unsigned*>(reinterpret_cast<char*>(a->workspace) + queue_off);
    p.max_grid = cu_count() * flash_resident(pl.HD, qt);
  }
  if (!f32 && fp.n_items && have_ws && a->workspace_bytes >= part_off + fp.part_bytes) {
    char* ws = reinterpret_cast<char*>(a->workspace) + part_off;
    const int64_t nbh = (int64_t)pl.B * p.n_slots;
    p.n_items = fp.n_items;
    p.seg_len = fp.seg_len;
    p.n_part_per_head = fp.n_part_per_head;
    p.part_o = reinterpret_cast<float*>(ws);
    p.part_ml = reinterpret_cast<float*>(ws + nbh * fp.n_part_per_head * (int64_t)BM * pl.HD * 4);
    std::copy(fp.items.begin(), fp.items.end(), p.items);
    std::copy(fp.part_base.begin(), fp.part_base.end(), p.part_base);
  } else {
    fp = FlashPlan();
  }
  for (int i = 0; i < p.n_slots; ++i) {
    const int h = pl.live[i];
    const int slot = a->hidx ? a->hidx[h] : h;
    p.out_head[i] = (int16_t)h;
    p.q_head[i] = (int16_t)slot;
    p.k_head[i] = (int16_t)(a->kvidx ? a->kvidx[h] : slot);
    p.v_head[i] = (int16_t)(a->kvidx ? a->kvidx[h] : h);
  }
  if (p.queue != nullptr)
    if (int rc = launched(launch_zero_u32(p.queue, 1, s), "flash queue clear")) return rc;
  if (int rc = launched(timed([&] { return launch_flash(p, pl.dtype, pl.HD, qt, s); }, s), "flash")) return rc;
  if (fp.n_split == 0) return SAF_OK;
  CombineParams c{};
  c.out = p.out;
  c.lse = p.lse;
  c.o_sb = p.o_sb; c.o_sh = p.o_sh; c.o_st = p.o_st;
  c.l_sb = p.l_sb; c.l_sh = p.l_sh; c.l_st = p.l_st;
  c.B = p.B; c.T = p.T; c.n_slots = p.n_slots; c.BM = BM;
  c.seg_len = fp.seg_len; c.n_part_per_head = fp.n_part_per_head; c.n_split = fp.n_split;
  c.part_o = p.part_o;
  c.part_ml = p.part_ml;
  std::copy(p.out_head, p.out_head + kMaxHeads, c.out_head);
  std::copy(fp.split_qb.begin(), fp.split_qb.end(), c.split_qb);
  std::copy(fp.part_base.begin(), fp.part_base.end(), c.part_base);
  return launched(launch_flash_combine(c, pl.dtype, pl.HD, s), "flash combine");
}

void fill_frozen_common(FrozenParams& p, const saf_tensor_t& v, const saf_tensor_t& o, int B, int T) {
  p.v = v.data;
  p.out = o.data;
  p.v_sb = v.stride[0]; p.v_sh = v.stride[1]; p.v_st = v.stride[2];
  p.o_sb = o.stride[0]; p.o_sh = o.stride[1]; p.o_st = o.stride[2];
  p.B = B;
  p.T = T;
}

int frozen_qtiles(int hd) { return hd <= 64 ? 2 : 1; }
// Resident rebuild workgroups per CU (decomp_waves_per_eu in the kernel).
int decomp_resident(int hd) { return hd > 64 ? 2 : 3; }

// Dense P.V work plan: query blocks of the kernel's shape, balanced over the
// batch groups that share a pattern (dense_batch_group).
FlashPlan plan_dense(int B, int n_slots, int T, int HD) {
  const int nb = dense_batch_group(B, HD);
  return plan_flash(B / nb, n_slots, T, HD, dense_block_rows(B, HD), kDenseResident, nb);
}

// Dense P.V over the heads listed; with a workspace large enough for the
// plan's partials, long query blocks are split into key segments (the flash
// planner's causal balance) and summed by the combine kernel.
int run_dense(const saf_tensor_t& patt, const saf_tensor_t& v, const saf_tensor_t& o, int B, int T, int HD,
              int dtype, const std::vector<int>& out_head, const std::vector<int>& v_head,
              const std::vector<int>& pat_head, void* ws, int64_t ws_bytes, hipStream_t s) {
  if (out_head.empty() || T == 0 || B == 0) return SAF_OK;
  FrozenParams p{};
  fill_frozen_common(p, v, o, B, T);
  p.patt = patt.data;
  p.patt_dtype = patt.dtype;
  p.p_sh = patt.stride[0]; p.p_si = patt.stride[1]; p.p_sj = patt.stride[2];
  p.p_cols = (int)patt.size[2];
  p.patt_elems = 1 + (patt.size[0] - 1) * patt.stride[0] + (patt.size[1] - 1) * patt.stride[1] +
                 (patt.size[2] - 1) * patt.stride[2];
  const int es = elem_size(patt.dtype);
  p.patt_vec = patt.stride[2] == 1 && reinterpret_cast<uintptr_t>(patt.data) % 16 == 0 &&
               (patt.stride[1] * es) % 16 == 0 && (patt.stride[0] * es) % 16 == 0;
  p.n_slots = (int)out_head.size();
  const int BM = dense_block_rows(B, HD);
  p.n_qblk = (T + BM - 1) / BM;
  for (int i = 0; i < p.n_slots; ++i) {
    p.out_head[i] = (int16_t)out_head[i];
    p.v_head[i] = (int16_t)v_head[i];
    p.pat_head[i] = (int16_t)pat_head[i];
  }
  FlashPlan fp = plan_dense(B, p.n_slots, T, HD);
  if (dtype != SAF_F32 && fp.n_items && ws != nullptr && ws_bytes >= fp.part_bytes &&
      reinterpret_cast<uintptr_t>(ws) % 16 == 0) {
    p.n_items = fp.n_items;
    p.seg_len = fp.seg_len;
    p.n_part_per_head = fp.n_part_per_head;
    p.part_o = reinterpret_cast<float*>(ws);
    std::copy(fp.items.begin(), fp.items.end(), p.items);
    std::copy(fp.part_base.begin(), fp.part_base.end(), p.part_base);
  } else {
    fp = FlashPlan();
  }
  if (int rc = launched(timed([&] { return launch_frozen_pv(p, dtype, HD, 0, s); }, s), "dense P.V")) return rc;
  if (fp.n_split == 0) return SAF_OK;
  CombineParams c{};
  c.out = p.out;
  c.o_sb = p.o_sb; c.o_sh = p.o_sh; c.o_st = p.o_st;
  c.B = p.B; c.T = p.T; c.n_slots = p.n_slots; c.BM = BM;
  c.seg_len = fp.seg_len; c.n_part_per_head = fp.n_part_per_head; c.n_split = fp.n_split;
  c.part_o = p.part_o;
  c.part_ml = nullptr;
  std::copy(p.out_head, p.out_head + kMaxHeads, c.out_head);
  std::copy(fp.split_qb.begin(), fp.split_qb.end(), c.split_qb);
  std::copy(fp.part_base.begin(), fp.part_base.end(), c.part_base);
  return launched(launch_flash_combine(c, dtype, HD, s), "dense P.V combine");
}

// Workspace regions after the scan's: the fp32 partials of split query
// blocks (flash, dense and decomposed kernels run one after the other and
// share them), then the factored decomposed form's per-64-block maxima of
// alpha and of rho and minima of z log2 e a_off (3 x n_dec x ceil(T / 64)
// floats), rho log2 e r2 and z log2 e z2 (n_dec x T floats each), key-scaled
// values vp (B, n_dec, T, HD) in bf16 (bf16 activations only) and in fp16,
// and their per-block largest magnitudes vmax (B x n_dec x ceil(T / 64)
// floats) (bf16 and fp16, hd <= 128 only).
int64_t round256(int64_t n) { return (n + 255) / 256 * 256; }

int64_t part_region_bytes(const saf_mixed_attn_args* args, const Plan& pl) {
  int64_t part = 0;
  if (!pl.live.empty()) {
    const int qt = flash_qtiles_for(args, pl.HD);
    const FlashPlan fp = plan_flash(pl.B, (int)pl.live.size(), pl.T, pl.HD, flash_block_rows(pl.HD, qt),
                                    flash_resident(pl.HD, qt));
    part = kQueueBytes + fp.part_bytes;
  }
  if (!pl.dense.empty())
    part = std::max(part, plan_dense(pl.B, (int)pl.dense.size(), pl.T, pl.HD).part_bytes);
  if (!pl.decomp.empty())
    part = std::max(part, plan_flash(pl.B, (int)pl.decomp.size(), pl.T, pl.HD, block_rows(frozen_qtiles(pl.HD)),
                                     decomp_resident(pl.HD)).part_bytes);
  return round256(part);
}

// Per-64-block maxima of alpha and of rho and minima of z (3 x n_dec x
// ceil(T / 64) floats), rho log2 e and z log2 e in fp32 (n_dec x T each),
// then the key-scaled values.
int64_t decomp_aoff_bytes(const Plan& pl) {
  return round256(3 * (int64_t)pl.decomp.size() * ((pl.T + 63) / 64) * 4);
}
int64_t decomp_r2_bytes(const Plan& pl) { return round256((int64_t)pl.decomp.size() * pl.T * 4); }

// key-scaled values in bf16, then in fp16, then their per-block maxima
int64_t decomp_v1_bytes(const Plan& pl) { return round256((int64_t)pl.B * pl.decomp.size() * pl.T * pl.HD * 2); }
int64_t decomp_vmax_bytes(const Plan& pl) {
  return round256((int64_t)pl.B * pl.decomp.size() * ((pl.T + 63) / 64) * 4);
}

int64_t decomp_vp_bytes(const Plan& pl) {
  if ((pl.dtype != SAF_BF16 && pl.dtype != SAF_F16) || pl.HD > 128 || pl.decomp.empty()) return 0;
  return decomp_aoff_bytes(pl) + 2 * decomp_r2_bytes(pl) + 2 * decomp_v1_bytes(pl) + decomp_vmax_bytes(pl);
}

// Decomposed P.V, causally balanced like run_dense when the workspace holds
// the plan's partials (same region as the flash and dense partials: the
// kernels run one after the other on the stream) unless `unsplit` asks for
// one workgroup per query block (the call then shares no workspace region
// with the live-head and dense kernels and may run beside them).
int run_decomp(const saf_mixed_attn_args* a, const Plan& pl, hipStream_t s, bool unsplit) {
  if (pl.decomp.empty() || pl.T == 0 || pl.B == 0) return SAF_OK;
  FrozenParams p{};
  fill_frozen_common(p, a->v, a->out, pl.B, pl.T);
  p.alpha = a->alpha.data; p.a_dtype = a->alpha.dtype; p.a_sh = a->alpha.stride[0]; p.a_ss = a->alpha.stride[1];
  p.rho = a->rho.data; p.r_dtype = a->rho.dtype; p.r_sh = a->rho.stride[0]; p.r_ss = a->rho.stride[1];
  p.z = a->z.data; p.z_dtype = a->z.dtype; p.z_sh = a->z.stride[0]; p.z_ss = a->z.stride[1];
  p.n_slots = (int)pl.decomp.size();
  p.n_qblk = (pl.T + block_rows(frozen_qtiles(pl.HD)) - 1) / block_rows(frozen_qtiles(pl.HD));
  for (int i = 0; i < p.n_slots; ++i) {
    const int h = pl.decomp[i];
    p.out_head[i] = (int16_t)h;
    p.v_head[i] = (int16_t)(a->kvidx ? a->kvidx[h] : h);
    p.pat_head[i] = (int16_t)h;
  }
  const int BM = block_rows(frozen_qtiles(pl.HD));
  FlashPlan fp = plan_flash(pl.B, p.n_slots, pl.T, pl.HD, BM, decomp_resident(pl.HD));
  const int64_t part_off = scan_ws_bytes(pl);
  if (pl.dtype != SAF_F32 && fp.n_items && !unsplit && a->workspace != nullptr &&
      a->workspace_bytes >= part_off + fp.part_bytes && reinterpret_cast<uintptr_t>(a->workspace) % 16 == 0) {
    p.n_items = fp.n_items;
    p.seg_len = fp.seg_len;
    p.n_part_per_head = fp.n_part_per_head;
    p.part_o = reinterpret_cast<float*>(reinterpret_cast<char*>(a->workspace) + part_off);
    std::copy(fp.items.begin(), fp.items.end(), p.items);
    std::copy(fp.part_base.begin(), fp.part_base.end(), p.part_base);
  } else {
    fp = FlashPlan();
  }
  // the factored form needs the key-scaled values in the workspace
  const int64_t vp_off = part_off + part_region_bytes(a, pl), vp_bytes = decomp_vp_bytes(pl);
  const bool factored = vp_bytes > 0 && a->workspace != nullptr && a->workspace_bytes >= vp_off + vp_bytes &&
                        reinterpret_cast<uintptr_t>(a->workspace) % 256 == 0;
  if (factored) {
    char* w = reinterpret_cast<char*>(a->workspace) + vp_off;
    p.a_off = reinterpret_cast<float*>(w);
    p.r2 = reinterpret_cast<float*>(w + decomp_aoff_bytes(pl));
    p.z2 = reinterpret_cast<float*>(w + decomp_aoff_bytes(pl) + decomp_r2_bytes(pl));
    p.vp = w + decomp_aoff_bytes(pl) + 2 * decomp_r2_bytes(pl);
    p.vp16 = reinterpret_cast<char*>(p.vp) + decomp_v1_bytes(pl);
    p.vmax = reinterpret_cast<float*>(reinterpret_cast<char*>(p.vp16) + decomp_v1_bytes(pl));
  }
  if (int rc = launched(timed([&] {
                          if (factored) {
                            const hipError_t e = launch_decomp_prescale(p, pl.dtype, pl.HD, s);
                            if (e != hipSuccess) return e;
                          }
                          return launch_frozen_pv(p, pl.dtype, pl.HD, 1, s);
                        }, s),
                        "decomposed P.V"))
    return rc;
  if (fp.n_split == 0) return SAF_OK;
  CombineParams c{};
  c.out = p.out;
  c.o_sb = p.o_sb; c.o_sh = p.o_sh; c.o_st = p.o_st;
  c.B = p.B; c.T = p.T; c.n_slots = p.n_slots; c.BM = BM;
  c.seg_len = fp.seg_len; c.n_part_per_head = fp.n_part_per_head; c.n_split = fp.n_split;
  c.part_o = p.part_o;
  c.part_ml = nullptr;
  std::copy(p.out_head, p.out_head + kMaxHeads, c.out_head);
  std::copy(fp.split_qb.begin(), fp.split_qb.end(), c.split_qb);
  std::copy(fp.part_base.begin(), fp.part_base.end(), c.part_base);
  return launched(launch_flash_combine(c, pl.dtype, pl.HD, s), "decomposed P.V combine");
}

int run_scan(const saf_mixed_attn_args* a, const Plan& pl, hipStream_t s) {
  if (pl.scan.empty() || pl.T == 0 || pl.B == 0) return SAF_OK;
  const WsLayout w = ws_layout(pl.B, pl.T, pl.HD, (int64_t)pl.scan.size());
  char* ws = reinterpret_cast<char*>(a->workspace);
  ScanParams p{};
  p.v = a->v.data;
  p.out = a->out.data;
  p.v_sb = a->v.stride[0]; p.v_sh = a->v.stride[1]; p.v_st = a->v.stride[2];
  p.o_sb = a->out.stride[0]; p.o_sh = a->out.stride[1]; p.o_st = a->out.stride[2];
  p.B = pl.B;
  p.T = pl.T;
  p.n_slots = (int)pl.scan.size();
  p.n_chunks = n_scan_chunks(pl.T, pl.HD);
  p.error = reinterpret_cast<uint32_t*>(ws + 4);
  p.status = reinterpret_cast<uint64_t*>(ws + w.status_off);
  // 0 = the default bound; a negative value is the give-up drill (tests)
  p.spin_limit = a->scan_spin_limit != 0 ? a->scan_spin_limit : (1 << 20);
  for (int i = 0; i < p.n_slots; ++i) {
    const int h = pl.scan[i];
    p.out_head[i] = (int16_t)h;
    p.v_head[i] = (int16_t)(a->kvidx ? a->kvidx[h] : h);
    p.kind[i] = (int8_t)a->closed_kind[h];
    p.param[i] = a->closed_param[h];
  }
  if (int rc = launched(launch_zero_u32(reinterpret_cast<uint32_t*>(ws), w.total / 4, s), "workspace clear")) return rc;
  return launched(timed([&] { return launch_scan(p, pl.dtype, pl.HD, s); }, s), "closed-form scan");
}

int run_dense_mixed(const saf_mixed_attn_args* a, const Plan& pl, hipStream_t s) {
  std::vector<int> vh, ph;
  for (int h : pl.dense) {
    vh.push_back(a->kvidx ? a->kvidx[h] : h);
    ph.push_back(a->pidx ? a->pidx[h] : h);
  }
  // the partials share the flash kernel's region: same stream, flash's
  // combine has consumed it before the dense kernel starts
  const int64_t part_off = scan_ws_bytes(pl);
  void* ws = nullptr;
  int64_t ws_bytes = 0;
  if (a->workspace != nullptr && a->workspace_bytes > part_off) {
    ws = reinterpret_cast<char*>(a->workspace) + part_off;
    ws_bytes = a->workspace_bytes - part_off;
  }
  return run_dense(a->patt, a->v, a->out, pl.B, pl.T, pl.HD, pl.dtype, pl.dense, vh, ph, ws, ws_bytes, s);
}

// A second stream per device (default priority, non-blocking) with a fork
// and a join event, for kernels of one call that run beside each other: the
// caller's stream records `fork` and the side stream waits for it; after the
// side kernels the side stream records `join` and the caller's stream waits
// for it before the call returns.  g_side_mu is held from the fork to the
// join, so calls from several host threads do not interleave their records.
struct SideStream {
  hipStream_t s = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};
constexpr int kMaxSideDevices = 64;
std::mutex g_side_mu;
SideStream g_side[kMaxSideDevices];

// With g_side_mu held: the current device's side stream (created on first
// use) made to wait for the work enqueued so far on `s`.  *out stays null
// (and the caller runs everything on `s`) where a fork could mix graph
// captures: when `s` is being captured and the side stream does not exist
// yet (creating streams and events is left out of captures), and when the
// side stream is still part of a capture (a stream that joined one stays in
// it until it ends) other than the one `s` is in.
int side_fork_locked(hipStream_t s, SideStream** out) {
  *out = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SAF_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxSideDevices)
    return fail(SAF_EUNSUPPORTED, "device %d beyond %d devices", dev, kMaxSideDevices);
  SideStream& ss = g_side[dev];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  e = hipStreamGetCaptureInfo(s, &cs, &cid);
  if (e != hipSuccess) return fail(SAF_ELAUNCH, "hipStreamGetCaptureInfo failed: %s", hipGetErrorString(e));
  if (ss.s != nullptr) {
    hipStreamCaptureStatus side_cs = hipStreamCaptureStatusNone;
    unsigned long long side_cid = 0;
    e = hipStreamGetCaptureInfo(ss.s, &side_cs, &side_cid);
    if (e != hipSuccess) return fail(SAF_ELAUNCH, "hipStreamGetCaptureInfo failed: %s", hipGetErrorString(e));
    if (side_cs != hipStreamCaptureStatusNone && (cs != hipStreamCaptureStatusActive || side_cid != cid))
      return SAF_OK;
  } else {
    if (cs != hipStreamCaptureStatusNone) return SAF_OK;
    SideStream n;
    e = hipStreamCreateWithFlags(&n.s, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&n.fork, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&n.join, hipEventDisableTiming);
    if (e != hipSuccess) return fail(SAF_ELAUNCH, "side stream set-up failed: %s", hipGetErrorString(e));
    ss = n;
  }
  e = hipEventRecord(ss.fork, s);
  if (e == hipSuccess) e = hipStreamWaitEvent(ss.s, ss.fork, 0);
  if (e != hipSuccess) return fail(SAF_ELAUNCH, "side stream fork failed: %s", hipGetErrorString(e));
  *out = &ss;
  return SAF_OK;
}

// With g_side_mu held: `s` waits for everything enqueued on the side stream.
int side_join_locked(SideStream* ss, hipStream_t s) {
  hipError_t e = hipEventRecord(ss->join, ss->s);
  if (e == hipSuccess) e = hipStreamWaitEvent(s, ss->join, 0);
  if (e != hipSuccess) return fail(SAF_ELAUNCH, "side stream join failed: %s", hipGetErrorString(e));
  return SAF_OK;
}

// The head kinds of `which`.  With may_fork (saf_mixed_attn_fwd), the
// HBM-bound closed-form scan and, when live heads share the call, the
// decomposed heads (one workgroup per query block, unless decomp_unsplit < 0)
// run on the side stream beside the live-head and dense kernels: disjoint
// output rows and workspace regions, joined before returning.  Otherwise
// everything runs in order on `stream`.
int run(const saf_mixed_attn_args* a, unsigned which, void* stream, bool may_fork = false) {
  Plan pl;
  if (int rc = plan_and_validate(a, which, pl)) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool has_dec = (which & kDoDecomp) && !pl.decomp.empty();
  const bool has_live = (which & kDoFlash) && !pl.live.empty();
  const bool dec_side = may_fork && has_dec && has_live && a->decomp_unsplit >= 0;
  const bool scan_side = may_fork && (which & kDoScan) && !pl.scan.empty() &&
                         (has_live || has_dec || ((which & kDoDense) && !pl.dense.empty()));
  const bool dec_unsplit = a->decomp_unsplit > 0;
  if (!dec_side && !scan_side) {
    if (which & kDoFlash)
      if (int rc = run_flash(a, pl, s)) return rc;
    if (which & kDoScan)
      if (int rc = run_scan(a, pl, s)) return rc;
    if (which & kDoDense)
      if (int rc = run_dense_mixed(a, pl, s)) return rc;
    if (which & kDoDecomp)
      if (int rc = run_decomp(a, pl, s, dec_unsplit)) return rc;
    return SAF_OK;
  }
  std::lock_guard<std::mutex> lock(g_side_mu);
  SideStream* ss = nullptr;
  if (int rc = side_fork_locked(s, &ss)) return rc;
  // without a side stream (first use inside a graph capture) the same
  // kernels run in order on `s`
  hipStream_t t = ss != nullptr ? ss->s : s;
  int rc = SAF_OK;
  if (dec_side) rc = run_decomp(a, pl, t, true);
  if (rc == SAF_OK && scan_side) rc = run_scan(a, pl, t);
  if (rc == SAF_OK && (which & kDoFlash)) rc = run_flash(a, pl, s);
  if (rc == SAF_OK && (which & kDoScan) && !scan_side) rc = run_scan(a, pl, s);
  if (rc == SAF_OK && (which & kDoDense)) rc = run_dense_mixed(a, pl, s);
  if (rc == SAF_OK && (which & kDoDecomp) && !dec_side) rc = run_decomp(a, pl, s, dec_unsplit);
  if (ss == nullptr) return rc;
  // joined on every path, so the side stream's work is ordered before
  // whatever the caller enqueues next
  const int jrc = side_join_locked(ss, s);
  return rc == SAF_OK ? jrc : rc;
}

// Shared checks of the projection GEMMs: x (M, K), weight (N, K) and out
// (M, N / out_div) of one 16-bit dtype; fills the GEMM part of p.
int proj_common(const char* what, const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out,
                ProjGemmParams& p, int out_div = 1) {
  if (x == nullptr || weight == nullptr || out == nullptr || !present(*x) || !present(*weight) || !present(*out))
    return fail(SAF_EINVAL, "x, weight and out are required");
  if (x->ndim != 2 || weight->ndim != 2 || out->ndim != 2)
    return fail(SAF_EINVAL, "x (M, K), weight (N, K) and out (M, N) must be 2-D");
  if (x->dtype != SAF_BF16 && x->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "%s supports bf16 / fp16 (got %s)", what, dtype_name(x->dtype));
  if (weight->dtype != x->dtype || out->dtype != x->dtype)
    return fail(SAF_EINVAL, "x, weight and out must share one dtype");
  const int64_t M = x->size[0], K = x->size[1], N = weight->size[0];
  if (weight->size[1] != K || out->size[0] != M || out->size[1] * out_div != N)
    return fail(SAF_EINVAL, "shapes do not chain: x (%lld, %lld), weight (%lld, %lld), out (%lld, %lld)",
                (long long)M, (long long)K, (long long)weight->size[0], (long long)weight->size[1],
                (long long)out->size[0], (long long)out->size[1]);
  if (x->stride[1] != 1 || weight->stride[1] != 1 || out->stride[1] != 1)
    return fail(SAF_EALIGN, "x, weight and out need a unit column stride");
  if (M > 0 && (!proj_gemm_shape_ok(M, N, K) || M > 0x7fffffff))
    return fail(SAF_EUNSUPPORTED, "%s: N = %lld must be a multiple of 256 and K = %lld of 128", what, (long long)N,
                (long long)K);
  // 16-byte pieces of x and weight rows, 16-byte pieces of out rows; the
  // buffer descriptors span 256 rows of x and weight
  auto rows_ok = [](const saf_tensor_t& t, int align) {
    return reinterpret_cast<uintptr_t>(t.data) % align == 0 && (t.stride[0] * 2) % align == 0 &&
           t.stride[0] >= t.size[1] && t.stride[0] < (1 << 22);
  };
  if (M > 0 && (!rows_ok(*x, 16) || !rows_ok(*weight, 16) || !rows_ok(*out, 16)))
    return fail(SAF_EALIGN, "x, weight and out rows must be 16-byte aligned (row strides below 2^22 elements)");
  p.a = x->data;
  p.w = weight->data;
  p.c = out->data;
  p.M = (int)M;
  p.N = (int)N;
  p.K = (int)K;
  p.a_rs = (int)x->stride[0];
  p.w_rs = (int)weight->stride[0];
  p.c_rs = (int)out->stride[0];
  p.n_cu = cu_count();
  return SAF_OK;
}

int add_norm(const char* what, bool rms, const saf_tensor_t* x, const saf_tensor_t* delta, const saf_tensor_t* weight,
             const saf_tensor_t* bias, float eps, const saf_tensor_t* out, void* stream) {
  if (x == nullptr || weight == nullptr || out == nullptr || !present(*x) || !present(*weight) || !present(*out))
    return fail(SAF_EINVAL, "x, weight and out are required");
  const bool has_d = delta != nullptr && present(*delta);
  const bool has_b = bias != nullptr && present(*bias);
  if (x->ndim != 2 || out->ndim != 2 || (has_d && delta->ndim != 2))
    return fail(SAF_EINVAL, "x, delta and out must be 2-D (rows, C)");
  if (x->dtype != SAF_BF16 && x->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "%s supports bf16 / fp16 activations (got %s)", what, dtype_name(x->dtype));
  const int64_t rows = x->size[0], C = x->size[1];
  if (out->dtype != x->dtype || out->size[0] != rows || out->size[1] != C)
    return fail(SAF_EINVAL, "out must match x in shape and dtype");
  if (has_d && (delta->dtype != x->dtype || delta->size[0] != rows || delta->size[1] != C))
    return fail(SAF_EINVAL, "delta must match x in shape and dtype");
  if (x->stride[1] != 1 || out->stride[1] != 1 || (has_d && delta->stride[1] != 1))
    return fail(SAF_EALIGN, "x, delta and out need a unit channel stride");
  if (C < 2 || C > 2048 || C % 2 != 0)
    return fail(SAF_EUNSUPPORTED, "%s: C = %lld is not supported (even, at most 2048)", what, (long long)C);
  const int vec_bytes = (C % 256 == 0 ? 4 : 2) * 2;
  auto aligned = [&](const saf_tensor_t& t) {
    return reinterpret_cast<uintptr_t>(t.data) % vec_bytes == 0 && (t.size[0] <= 1 || (t.stride[0] * 2) % vec_bytes == 0);
  };
  if (!aligned(*x) || !aligned(*out) || (has_d && !aligned(*delta)))
    return fail(SAF_EALIGN, "x, delta and out rows must be %d-byte aligned", vec_bytes);
  if (weight->ndim != 1 || weight->size[0] != C || weight->stride[0] != 1 ||
      (has_b && (bias->ndim != 1 || bias->size[0] != C || bias->stride[0] != 1 || bias->dtype != weight->dtype)))
    return fail(SAF_EINVAL, "weight and bias must be contiguous (C,) of one dtype");
  if (weight->dtype != SAF_F32 && weight->dtype != SAF_BF16 && weight->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "weight dtype %s is not supported", dtype_name(weight->dtype));
  if (rows == 0) return SAF_OK;
  AddLnParams p{};
  p.x = x->data;
  p.delta = has_d ? delta->data : nullptr;
  p.y = out->data;
  p.w = weight->data;
  p.b = has_b ? bias->data : nullptr;
  p.rows = rows;
  p.C = C;
  p.x_rs = x->stride[0];
  p.d_rs = has_d ? delta->stride[0] : 0;
  p.y_rs = out->stride[0];
  p.eps = eps;
  p.wb_dtype = weight->dtype;
  auto al16 = [&](const saf_tensor_t& t) {
    return reinterpret_cast<uintptr_t>(t.data) % 16 == 0 && (t.size[0] <= 1 || (t.stride[0] * 2) % 16 == 0);
  };
  p.vec16_rows = al16(*x) && al16(*out) && (!has_d || al16(*delta)) &&
                 reinterpret_cast<uintptr_t>(weight->data) % 16 == 0 &&
                 (!has_b || reinterpret_cast<uintptr_t>(bias->data) % 16 == 0);
  p.vec16 = C % 256 == 0 && p.vec16_rows;
  p.rms = rms ? 1 : 0;
  return launched(launch_add_layernorm(p, x->dtype, reinterpret_cast<hipStream_t>(stream)), what);
}

}  // namespace

extern "C" {

int saf_mixed_attn_fwd(const saf_mixed_attn_args* args, void* stream) { return run(args, kDoAll, stream, true); }
int saf_flash_fwd(const saf_mixed_attn_args* args, void* stream) { return run(args, kDoFlash, stream); }
int saf_frozen_dense_pv_fwd(const saf_mixed_attn_args* args, void* stream) { return run(args, kDoDense, stream); }
int saf_frozen_decomp_fwd(const saf_mixed_attn_args* args, void* stream) { return run(args, kDoDecomp, stream); }
int saf_frozen_scan_fwd(const saf_mixed_attn_args* args, void* stream) { return run(args, kDoScan, stream); }

int saf_frozen_pv_fwd(const saf_tensor_t* patt, const saf_tensor_t* v, const int32_t* fz_idx, int32_t nf,
                      int32_t T, const saf_tensor_t* out, void* stream) {
  if (patt == nullptr || v == nullptr || out == nullptr) return fail(SAF_EINVAL, "patt, v and out are required");
  if (!present(*v) || !present(*out)) return fail(SAF_EINVAL, "v and out must be device tensors");
  if (v->ndim != 4 || out->ndim != 4) return fail(SAF_EINVAL, "v and out must be 4-D (B, nf, T, hd)");
  if (v->dtype != SAF_BF16 && v->dtype != SAF_F16 && v->dtype != SAF_F32)
    return fail(SAF_EUNSUPPORTED, "unsupported v dtype %s", dtype_name(v->dtype));
  const int B = (int)v->size[0], HD = (int)v->size[3];
  if (nf != v->size[1]) return fail(SAF_EINVAL, "fz_idx must have one entry per compact head (%d != %lld)", nf,
                                    (long long)v->size[1]);
  if (nf > SAF_MAX_HEADS) return fail(SAF_EUNSUPPORTED, "more than %d frozen heads", SAF_MAX_HEADS);
  if (T < 0 || T > v->size[2]) return fail(SAF_EINVAL, "T must be within v's sequence length");
  if (!supported_hd(HD)) return fail(SAF_EUNSUPPORTED, "head_dim %d is not supported (32, 64, 96, 128, 256)", HD);
  if (out->size[0] != B || out->size[1] != nf || out->size[2] != T || out->size[3] != HD || out->dtype != v->dtype)
    return fail(SAF_EINVAL, "out must be (B, nf, T, hd) in v's dtype");
  if (int rc = check_act(*v, "v", 16)) return rc;
  if (int rc = check_act(*out, "out", 8)) return rc;
  if (nf == 0 || T == 0 || B == 0) return SAF_OK;
  if (!present(*patt) || patt->ndim != 3 || patt->size[1] < T || patt->size[2] < T)
    return fail(SAF_EINVAL, "patt must have shape (P, S, S) with S >= T");
  if (patt->dtype != SAF_F32 && patt->dtype != SAF_BF16 && patt->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "unsupported patt dtype %s", dtype_name(patt->dtype));
  if (fz_idx == nullptr) return fail(SAF_EINVAL, "fz_idx (host) is required");
  std::vector<int> oh, vh, ph;
  for (int f = 0; f < nf; ++f) {
    if (fz_idx[f] < 0 || fz_idx[f] >= patt->size[0])
      return fail(SAF_EINVAL, "fz_idx[%d] = %d does not index patt", f, fz_idx[f]);
    oh.push_back(f);
    vh.push_back(f);
    ph.push_back(fz_idx[f]);
  }
  return run_dense(*patt, *v, *out, B, T, HD, v->dtype, oh, vh, ph, nullptr, 0,
                   reinterpret_cast<hipStream_t>(stream));
}

int saf_frozen_pv_bwd(const saf_tensor_t* patt, const saf_tensor_t* dy, const int32_t* fz_idx, int32_t nf,
                      int32_t T, const saf_tensor_t* dv, void* stream) {
  if (patt == nullptr || dy == nullptr || dv == nullptr) return fail(SAF_EINVAL, "patt, dy and dv are required");
  if (!present(*dy) || !present(*dv)) return fail(SAF_EINVAL, "dy and dv must be device tensors");
  if (dy->ndim != 4 || dv->ndim != 4) return fail(SAF_EINVAL, "dy and dv must be 4-D (B, nf, T, hd)");
  if (dy->dtype != SAF_BF16 && dy->dtype != SAF_F16 && dy->dtype != SAF_F32)
    return fail(SAF_EUNSUPPORTED, "frozen_pv backward: unsupported gradient dtype %s", dtype_name(dy->dtype));
  const int B = (int)dv->size[0], HD = (int)dv->size[3];
  if (nf != dv->size[1]) return fail(SAF_EINVAL, "fz_idx must have one entry per compact head (%d != %lld)", nf,
                                    (long long)dv->size[1]);
  if (nf > SAF_MAX_HEADS) return fail(SAF_EUNSUPPORTED, "more than %d frozen heads", SAF_MAX_HEADS);
  if (T < 0 || T > dv->size[2]) return fail(SAF_EINVAL, "T must be within dv's sequence length");
  if (!supported_bwd_hd(HD) && !(HD == 256 && dy->dtype == SAF_F32))
    return fail(SAF_EUNSUPPORTED, "frozen_pv backward: head_dim %d is not supported (32, 64, 96, 128)", HD);
  if (dy->size[0] != B || dy->size[1] != nf || dy->size[2] != T || dy->size[3] != HD || dy->dtype != dv->dtype)
    return fail(SAF_EINVAL, "dy must be (B, nf, T, hd) in dv's dtype");
  if (int rc = check_act(*dy, "dy", 16)) return rc;
  if (int rc = check_act(*dv, "dv", 8)) return rc;
  if (nf == 0 || T == 0 || B == 0) return SAF_OK;
  if (!present(*patt) || patt->ndim != 3 || patt->size[1] < T || patt->size[2] < T)
    return fail(SAF_EINVAL, "patt must have shape (P, S, S) with S >= T");
  if (patt->dtype != SAF_F32 && patt->dtype != SAF_BF16 && patt->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "unsupported patt dtype %s", dtype_name(patt->dtype));
  if (fz_idx == nullptr) return fail(SAF_EINVAL, "fz_idx (host) is required");
  BwdParams p{};
  p.dout = dy->data;
  p.dv = dv->data;
  p.do_sb = dy->stride[0]; p.do_sh = dy->stride[1]; p.do_st = dy->stride[2];
  p.dv_sb = dv->stride[0]; p.dv_sh = dv->stride[1]; p.dv_st = dv->stride[2];
  p.B = B;
  p.T = T;
  p.n_frozen = nf;
  for (int f = 0; f < nf; ++f) {
    if (fz_idx[f] < 0 || fz_idx[f] >= patt->size[0])
      return fail(SAF_EINVAL, "fz_idx[%d] = %d does not index patt", f, fz_idx[f]);
    p.f_head[f] = (int16_t)f;  // compact head of dy and dv
    p.pat_head[f] = (int16_t)fz_idx[f];
    p.f_kind[f] = 1;
  }
  p.patt = patt->data;
  p.patt_dtype = patt->dtype;
  p.p_sh = patt->stride[0]; p.p_si = patt->stride[1]; p.p_sj = patt->stride[2];
  return launched(launch_bwd_frozen_dv(p, dy->dtype, HD, reinterpret_cast<hipStream_t>(stream)),
                  "frozen_pv backward");
}

static int rope_common(const saf_tensor_t* q, const saf_tensor_t* k, const saf_tensor_t* qw,
                       const saf_tensor_t* kw, float eps, const saf_tensor_t* cos, const saf_tensor_t* sin,
                       void* stream) {
  if (q == nullptr || k == nullptr || cos == nullptr || sin == nullptr)
    return fail(SAF_EINVAL, "q, k, cos and sin are required");
  if (!present(*q) || !present(*k) || !present(*cos) || !present(*sin))
    return fail(SAF_EINVAL, "q, k, cos and sin must be device tensors");
  if (q->ndim != 4 || k->ndim != 4) return fail(SAF_EINVAL, "q and k must be 4-D (B, U, T, HD)");
  if (q->dtype != k->dtype) return fail(SAF_EINVAL, "q and k must share a dtype");
  if (q->dtype != SAF_BF16 && q->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "rope: unsupported q/k dtype %s (bf16 or fp16)", dtype_name(q->dtype));
  const int64_t B = q->size[0], T = q->size[2], hd = q->size[3];
  if (k->size[0] != B || k->size[2] != T || k->size[3] != hd)
    return fail(SAF_EINVAL, "q and k batch, sequence and head dimensions must match");
  if (!supported_bwd_hd(hd))
    return fail(SAF_EUNSUPPORTED, "rope: head_dim %lld is not supported (32, 64, 96, 128)", (long long)hd);
  const saf_tensor_t* cs[2] = {cos, sin};
  for (int i = 0; i < 2; ++i) {
    const saf_tensor_t& t = *cs[i];
    if (t.ndim != 2 || t.size[0] < T || t.size[1] != hd)
      return fail(SAF_EINVAL, "cos/sin must be (T', HD) caches with T' >= T");
    if (t.dtype != SAF_F32 && t.dtype != SAF_BF16 && t.dtype != SAF_F16)
      return fail(SAF_EUNSUPPORTED, "rope: unsupported cache dtype %s", dtype_name(t.dtype));
    if (t.stride[1] != 1 || (t.stride[0] * elem_size(t.dtype)) % 16 || reinterpret_cast<uintptr_t>(t.data) % 16)
      return fail(SAF_EALIGN, "cos/sin rows must be contiguous and 16-byte aligned");
  }
  if (cos->dtype != sin->dtype) return fail(SAF_EINVAL, "cos and sin must share a dtype");
  const bool norm = qw != nullptr || kw != nullptr;
  if (norm) {
    if (qw == nullptr || kw == nullptr || !present(*qw) || !present(*kw))
      return fail(SAF_EINVAL, "q_weight and k_weight are both required for the RMSNorm");
    const saf_tensor_t* ws[2] = {qw, kw};
    for (int i = 0; i < 2; ++i) {
      const saf_tensor_t& w = *ws[i];
      if (w.ndim != 1 || w.size[0] != hd) return fail(SAF_EINVAL, "norm weights must be (HD,) vectors");
      if (w.dtype != SAF_F32 && w.dtype != SAF_BF16 && w.dtype != SAF_F16)
        return fail(SAF_EUNSUPPORTED, "rmsnorm: unsupported weight dtype %s", dtype_name(w.dtype));
      if (w.stride[0] != 1 || reinterpret_cast<uintptr_t>(w.data) % 16)
        return fail(SAF_EALIGN, "norm weights must be contiguous and 16-byte aligned");
    }
    if (qw->dtype != kw->dtype) return fail(SAF_EINVAL, "q_weight and k_weight must share a dtype");
    if (!(eps >= 0.f)) return fail(SAF_EINVAL, "eps must be a non-negative number");
  }
  if (int rc = check_act(*q, "q", 16)) return rc;
  if (int rc = check_act(*k, "k", 16)) return rc;
  // one grid row per (batch, head) of q and k; T x 16 threads per grid row
  if (B * (q->size[1] + k->size[1]) > 65535 || T > (int64_t(1) << 26))
    return fail(SAF_EUNSUPPORTED, "rope: B x (Uq + Uk) must be at most 65535 and T at most 2^26");
  RopeParams p{};
  p.q = q->data; p.k = k->data;
  p.q_sb = q->stride[0]; p.q_sh = q->stride[1]; p.q_st = q->stride[2];
  p.k_sb = k->stride[0]; p.k_sh = k->stride[1]; p.k_st = k->stride[2];
  p.cos = cos->data; p.sin = sin->data;
  p.cs_st = cos->stride[0]; p.sn_st = sin->stride[0];
  p.cs_dtype = cos->dtype;
  p.B = (int)B; p.Uq = (int)q->size[1]; p.Uk = (int)k->size[1]; p.T = (int)T; p.hd = (int)hd;
  if (norm) {
    p.q_w = qw->data; p.k_w = kw->data;
    p.w_dtype = qw->dtype;
    p.eps = eps;
  }
  return launched(launch_rope(p, q->dtype, reinterpret_cast<hipStream_t>(stream)), "rope");
}

int saf_rope_qk_inplace(const saf_tensor_t* q, const saf_tensor_t* k, const saf_tensor_t* cos,
                        const saf_tensor_t* sin, void* stream) {
  return rope_common(q, k, nullptr, nullptr, 0.f, cos, sin, stream);
}

int saf_qk_rmsnorm_rope_inplace(const saf_tensor_t* q, const saf_tensor_t* k, const saf_tensor_t* q_weight,
                                const saf_tensor_t* k_weight, float eps, const saf_tensor_t* cos,
                                const saf_tensor_t* sin, void* stream) {
  if (q_weight == nullptr || k_weight == nullptr)
    return fail(SAF_EINVAL, "q_weight and k_weight are required");
  return rope_common(q, k, q_weight, k_weight, eps, cos, sin, stream);
}

int saf_add_layernorm(const saf_tensor_t* x, const saf_tensor_t* delta, const saf_tensor_t* weight,
                      const saf_tensor_t* bias, float eps, const saf_tensor_t* out, void* stream) {
  return add_norm("add_layernorm", false, x, delta, weight, bias, eps, out, stream);
}

int saf_add_rmsnorm(const saf_tensor_t* x, const saf_tensor_t* delta, const saf_tensor_t* weight, float eps,
                    const saf_tensor_t* out, void* stream) {
  return add_norm("add_rmsnorm", true, x, delta, weight, nullptr, eps, out, stream);
}

int saf_linear_gelu(const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out, void* stream) {
  ProjGemmParams p{};
  if (int rc = proj_common("linear_gelu", x, weight, out, p)) return rc;
  if (p.M == 0) return SAF_OK;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return launched(timed([&] { return launch_gemm_gelu(p, x->dtype, s); }, s), "linear_gelu");
}

int saf_gelu_inplace(const saf_tensor_t* x, void* stream) {
  if (x == nullptr || !present(*x)) return fail(SAF_EINVAL, "x is required");
  if (x->dtype != SAF_BF16 && x->dtype != SAF_F16)
    return fail(SAF_EUNSUPPORTED, "gelu_inplace supports bf16 / fp16 (got %s)", dtype_name(x->dtype));
  int64_t n = 1, expect = 1;
  for (int d = x->ndim - 1; d >= 0; --d) {
    if (x->size[d] != 1 && x->stride[d] != expect) return fail(SAF_EALIGN, "gelu_inplace needs a contiguous x");
    expect *= x->size[d];
    n *= x->size[d];
  }
  if (n == 0) return SAF_OK;
  if (n % 8 != 0 || reinterpret_cast<uintptr_t>(x->data) % 16 != 0)
    return fail(SAF_EALIGN, "gelu_inplace needs a 16-byte aligned x of a multiple of 8 elements");
  return launched(launch_gelu_inplace(x->data, n, x->dtype, cu_count(), reinterpret_cast<hipStream_t>(stream)),
                  "gelu_inplace");
}

int saf_linear_swiglu(const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out, void* stream) {
  ProjGemmParams p{};
  if (int rc = proj_common("linear_swiglu", x, weight, out, p, 2)) return rc;
  if (p.M == 0) return SAF_OK;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return launched(timed([&] { return launch_gemm_swiglu(p, x->dtype, s); }, s), "linear_swiglu");
}

int saf_linear_rope(const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out, int32_t n_rope,
                    int32_t head_dim, int32_t seq_len, const saf_tensor_t* cos, const saf_tensor_t* sin,
                    void* stream) {
  ProjGemmParams p{};
  if (int rc = proj_common("linear_rope", x, weight, out, p)) return rc;
  if (head_dim != 64 && head_dim != 128)
    return fail(SAF_EUNSUPPORTED, "linear_rope: head_dim %d is not supported (64 or 128)", (int)head_dim);
  if (n_rope < 0 || n_rope > p.N || n_rope % 128 != 0)
    return fail(SAF_EINVAL, "linear_rope: n_rope = %d must be a multiple of 128 in [0, N = %d]", (int)n_rope, p.N);
  if (seq_len < 1 || p.M % seq_len != 0)
    return fail(SAF_EINVAL, "linear_rope: the %d rows are not whole sequences of %d", p.M, (int)seq_len);
  if (n_rope > 0) {
    if (cos == nullptr || sin == nullptr || !present(*cos) || !present(*sin))
      return fail(SAF_EINVAL, "linear_rope: cos and sin are required");
    for (const saf_tensor_t* c : {cos, sin}) {
      if (c->ndim != 2 || c->dtype != x->dtype || c->size[0] < seq_len || c->size[1] < head_dim || c->stride[1] != 1)
        return fail(SAF_EINVAL, "linear_rope: cos / sin must be (>= %d, >= %d) in x's dtype with unit column stride",
                    (int)seq_len, (int)head_dim);
      if (reinterpret_cast<uintptr_t>(c->data) % 8 != 0 || (c->stride[0] * 2) % 8 != 0)
        return fail(SAF_EALIGN, "linear_rope: cos / sin rows must be 8-byte aligned");
    }
    p.cos = cos->data;
    p.sin = sin->data;
    p.cs_st = cos->stride[0];
    p.sn_st = sin->stride[0];
  }
  p.n_rope = n_rope;
  p.hd = head_dim;
  p.T = seq_len;
  if (p.M == 0) return SAF_OK;
  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  return launched(timed([&] { return launch_gemm_rope(p, x->dtype, s); }, s), "linear_rope");
}

int saf_decomposed_logz(const saf_tensor_t* alpha, const saf_tensor_t* rho, const saf_tensor_t* z, void* stream) {
  if (alpha == nullptr || rho == nullptr || z == nullptr || !present(*alpha) || !present(*rho) || !present(*z))
    return fail(SAF_EINVAL, "alpha, rho and z are required");
  const saf_tensor_t* ts[3] = {alpha, rho, z};
  const char* names[3] = {"alpha", "rho", "z"};
  for (int i = 0; i < 3; ++i) {
    const saf_tensor_t& t = *ts[i];
    if (t.ndim != 2 || t.size[0] != alpha->size[0] || t.size[1] != alpha->size[1])
      return fail(SAF_EINVAL, "%s must be 2-D (H, S) like alpha", names[i]);
    if (t.dtype != SAF_F32) return fail(SAF_EUNSUPPORTED, "%s must be fp32 (got %s)", names[i], dtype_name(t.dtype));
    if (t.size[1] > 1 && t.stride[1] != 1) return fail(SAF_EALIGN, "%s needs a unit column stride", names[i]);
  }
  const int64_t H = alpha->size[0], S = alpha->size[1];
  if (H > 65535 || S > (int64_t(1) << 30))
    return fail(SAF_EUNSUPPORTED, "decomposed_logz: H = %lld, S = %lld out of range", (long long)H, (long long)S);
  if (H == 0 || S == 0) return SAF_OK;
  LogzParams p{};
  p.alpha = static_cast<const float*>(alpha->data);
  p.rho = static_cast<const float*>(rho->data);
  p.z = static_cast<float*>(z->data);
  p.a_hs = alpha->stride[0];
  p.r_hs = rho->stride[0];
  p.z_hs = z->stride[0];
  p.H = (int)H;
  p.S = (int)S;
  return launched(launch_decomp_logz(p, reinterpret_cast<hipStream_t>(stream)), "decomposed_logz");
}

int saf_decomposed_logz_bwd(const saf_tensor_t* alpha, const saf_tensor_t* rho, const saf_tensor_t* z,
                            const saf_tensor_t* gz, const saf_tensor_t* dalpha, const saf_tensor_t* drho,
                            void* stream) {
  const saf_tensor_t* ts[6] = {alpha, rho, z, gz, dalpha, drho};
  const char* names[6] = {"alpha", "rho", "z", "gz", "dalpha", "drho"};
  for (int i = 0; i < 6; ++i) {
    if (ts[i] == nullptr || !present(*ts[i])) return fail(SAF_EINVAL, "%s is required", names[i]);
    const saf_tensor_t& t = *ts[i];
    if (t.ndim != 2 || t.size[0] != alpha->size[0] || t.size[1] != alpha->size[1])
      return fail(SAF_EINVAL, "%s must be 2-D (H, S) like alpha", names[i]);
    if (t.dtype != SAF_F32) return fail(SAF_EUNSUPPORTED, "%s must be fp32 (got %s)", names[i], dtype_name(t.dtype));
    if (t.size[1] > 1 && t.stride[1] != 1) return fail(SAF_EALIGN, "%s needs a unit column stride", names[i]);
  }
  const int64_t H = alpha->size[0], S = alpha->size[1];
  if (H > 65535 || S > (int64_t(1) << 30))
    return fail(SAF_EUNSUPPORTED, "decomposed_logz backward: H = %lld, S = %lld out of range", (long long)H,
                (long long)S);
  if (H == 0 || S == 0) return SAF_OK;
  LogzBwdParams p{};
  p.alpha = static_cast<const float*>(alpha->data);
  p.rho = static_cast<const float*>(rho->data);
  p.z = static_cast<const float*>(z->data);
  p.gz = static_cast<const float*>(gz->data);
  p.dalpha = static_cast<float*>(dalpha->data);
  p.drho = static_cast<float*>(drho->data);
  p.a_hs = alpha->stride[0]; p.r_hs = rho->stride[0]; p.z_hs = z->stride[0]; p.g_hs = gz->stride[0];
  p.da_hs = dalpha->stride[0]; p.dr_hs = drho->stride[0];
  p.H = (int)H;
  p.S = (int)S;
  return launched(launch_decomp_logz_bwd(p, reinterpret_cast<hipStream_t>(stream)), "decomposed_logz backward");
}

// ---- backward -------------------------------------------------------------

static int64_t bwd_delta_bytes(const Plan& pl) {
  return ((int64_t)pl.B * (int64_t)pl.live.size() * pl.T * 4 + 255) / 256 * 256;
}

int64_t saf_mixed_attn_bwd_workspace_bytes(const saf_mixed_attn_args* args) {
  Plan pl;
  if (plan_and_validate(args, kDoFlash, pl, false)) return -1;
  return bwd_delta_bytes(pl);
}

int saf_mixed_attn_bwd(const saf_mixed_attn_args* a, const saf_tensor_t* dout, const saf_tensor_t* dq,
                       const saf_tensor_t* dk, const saf_tensor_t* dv, void* stream) {
  Plan pl;
  if (int rc = plan_and_validate(a, kDoFlash | kDoDense | kDoDecomp, pl, false)) return rc;
  if (a->kvidx != nullptr)
    return fail(SAF_EUNSUPPORTED, "backward with kvidx (GQA) is not implemented (forward / prefill only)");
  if (!supported_bwd_hd(pl.HD) && pl.dtype != SAF_F32)  // the float32 kernels take hd 256 too
    return fail(SAF_EUNSUPPORTED, "backward: head_dim %d is not supported (32, 64, 96, 128)", pl.HD);
  if (dout == nullptr || dv == nullptr) return fail(SAF_EINVAL, "dout and dv are required");
  auto same4 = [](const saf_tensor_t& t, const saf_tensor_t& ref) {
    for (int i = 0; i < 4; ++i)
      if (t.size[i] != ref.size[i]) return false;
    return t.ndim == 4 && t.dtype == ref.dtype;
  };
  if (!present(*dout) || !same4(*dout, a->out)) return fail(SAF_EINVAL, "dout must match out's shape and dtype");
  if (!present(*dv) || !same4(*dv, a->v)) return fail(SAF_EINVAL, "dv must match v's shape and dtype");
  if (int rc = check_act(*dout, "dout", 16)) return rc;
  if (int rc = check_act(*dv, "dv", 8)) return rc;
  // closed-form heads run as decomposed heads here: their alpha/rho/z are needed
  std::vector<int> fz_dec = pl.decomp;
  fz_dec.insert(fz_dec.end(), pl.scan.begin(), pl.scan.end());
  if (!pl.scan.empty()) {
    const saf_tensor_t* bufs[3] = {&a->alpha, &a->rho, &a->z};
    for (int i = 0; i < 3; ++i) {
      const saf_tensor_t& t = *bufs[i];
      if (!present(t) || t.ndim != 2 || t.size[0] != pl.H || t.size[1] < pl.T)
        return fail(SAF_EINVAL, "the backward of closed-form heads needs their (H, S) alpha/rho/z buffers");
      if (t.dtype != SAF_F32 && t.dtype != SAF_BF16 && t.dtype != SAF_F16)
        return fail(SAF_EUNSUPPORTED, "unsupported decomposed buffer dtype %s", dtype_name(t.dtype));
    }
  }
  const int nf = (int)(pl.dense.size() + fz_dec.size());
  if (pl.T == 0 || pl.B == 0) return SAF_OK;

  BwdParams p{};
  p.v = a->v.data;
  p.out = a->out.data;
  p.dout = dout->data;
  p.dv = dv->data;
  p.v_sb = a->v.stride[0]; p.v_sh = a->v.stride[1]; p.v_st = a->v.stride[2];
  p.o_sb = a->out.stride[0]; p.o_sh = a->out.stride[1]; p.o_st = a->out.stride[2];
  p.do_sb = dout->stride[0]; p.do_sh = dout->stride[1]; p.do_st = dout->stride[2];
  p.dv_sb = dv->stride[0]; p.dv_sh = dv->stride[1]; p.dv_st = dv->stride[2];
  p.B = pl.B;
  p.T = pl.T;
  p.scale_log2 = a->sm_scale * kLog2e;
  p.sm_scale = a->sm_scale;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  if (!pl.live.empty()) {
    if (dq == nullptr || dk == nullptr || !present(*dq) || !present(*dk) || !same4(*dq, a->q) || !same4(*dk, a->k))
      return fail(SAF_EINVAL, "live heads require dq and dk shaped like q and k");
    if (int rc = check_act(*dq, "dq", 8)) return rc;
    if (int rc = check_act(*dk, "dk", 8)) return rc;
    if (int rc = check_act(a->out, "out", 16)) return rc;
    const saf_tensor_t& l = a->lse;
    if (!present(l) || l.ndim != 3 || l.size[0] != pl.B || l.size[1] != pl.H || l.size[2] != pl.T || l.dtype != SAF_F32)
      return fail(SAF_EINVAL, "live heads require the forward's lse, (B, H, T) float32");
    const int64_t need = bwd_delta_bytes(pl);
    if (a->workspace == nullptr || a->workspace_bytes < need || reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
      return fail(SAF_EWORKSPACE, "the backward needs a 16-byte aligned %lld-byte workspace (got %lld)",
                  (long long)need, (long long)a->workspace_bytes);
    p.q = a->q.data;
    p.k = a->k.data;
    p.dq = dq->data;
    p.dk = dk->data;
    p.lse = reinterpret_cast<const float*>(l.data);
    p.delta = reinterpret_cast<float*>(a->workspace);
    p.q_sb = a->q.stride[0]; p.q_sh = a->q.stride[1]; p.q_st = a->q.stride[2];
    p.k_sb = a->k.stride[0]; p.k_sh = a->k.stride[1]; p.k_st = a->k.stride[2];
    p.dq_sb = dq->stride[0]; p.dq_sh = dq->stride[1]; p.dq_st = dq->stride[2];
    p.dk_sb = dk->stride[0]; p.dk_sh = dk->stride[1]; p.dk_st = dk->stride[2];
    p.l_sb = l.stride[0]; p.l_sh = l.stride[1]; p.l_st = l.stride[2];
    p.n_live = (int)pl.live.size();
    for (int i = 0; i < p.n_live; ++i) {
      const int h = pl.live[i];
      p.out_head[i] = (int16_t)h;
      p.q_head[i] = (int16_t)(a->hidx ? a->hidx[h] : h);
    }
  }
  if (nf > 0) {
    p.n_frozen = nf;
    int i = 0;
    for (int h : pl.dense) {
      p.f_head[i] = (int16_t)h;
      p.pat_head[i] = (int16_t)(a->pidx ? a->pidx[h] : h);
      p.f_kind[i++] = 1;
    }
    for (int h : fz_dec) {
      p.f_head[i] = (int16_t)h;
      p.pat_head[i] = (int16_t)h;
      p.f_kind[i++] = 2;
    }
    if (!pl.dense.empty()) {
      const saf_tensor_t& pt = a->patt;
      p.patt = pt.data;
      p.patt_dtype = pt.dtype;
      p.p_sh = pt.stride[0]; p.p_si = pt.stride[1]; p.p_sj = pt.stride[2];
    }
    if (!fz_dec.empty()) {
      p.alpha = a->alpha.data; p.rho = a->rho.data; p.z = a->z.data;
      p.a_dtype = a->alpha.dtype; p.r_dtype = a->rho.dtype; p.z_dtype = a->z.dtype;
      p.a_sh = a->alpha.stride[0]; p.a_ss = a->alpha.stride[1];
      p.r_sh = a->rho.stride[0]; p.r_ss = a->rho.stride[1];
      p.z_sh = a->z.stride[0]; p.z_ss = a->z.stride[1];
    }
  }
  // the frozen heads' dV (its own rows of dv, no workspace) on the side
  // stream beside the live heads' kernels, whose tails leave slots idle
  const bool fork = !pl.live.empty() && nf > 0;
  std::unique_lock<std::mutex> lock(g_side_mu, std::defer_lock);
  SideStream* ss = nullptr;
  if (fork) {
    lock.lock();
    if (int rc = side_fork_locked(s, &ss)) return rc;
  }
  int rc = SAF_OK;
  if (nf > 0) rc = launched(launch_bwd_frozen_dv(p, pl.dtype, pl.HD, ss != nullptr ? ss->s : s), "backward frozen dv");
  if (rc == SAF_OK && !pl.live.empty()) {
    rc = launched(launch_bwd_delta(p, pl.dtype, pl.HD, s), "backward delta");
    if (rc == SAF_OK) rc = launched(launch_bwd_dq(p, pl.dtype, pl.HD, s), "backward dq");
    if (rc == SAF_OK) rc = launched(launch_bwd_dkdv(p, pl.dtype, pl.HD, s), "backward dk/dv");
  }
  if (ss != nullptr) {
    // joined on every path, so the side stream never outlives the call's
    // ordering on the caller's stream
    const int jrc = side_join_locked(ss, s);
    if (rc == SAF_OK) rc = jrc;
  }
  return rc;
}

static std::vector<int> decomp_heads_all(const Plan& pl) {
  std::vector<int> v = pl.decomp;
  v.insert(v.end(), pl.scan.begin(), pl.scan.end());
  std::sort(v.begin(), v.end());
  return v;
}

int64_t saf_decomp_param_bwd_workspace_bytes(const saf_mixed_attn_args* args) {
  Plan pl;
  if (plan_and_validate(args, 0, pl, false)) return -1;
  const int64_t n = (int64_t)pl.B * (int64_t)decomp_heads_all(pl).size() * pl.T;
  return (n * 4 + 255) / 256 * 256;
}

int saf_decomp_param_bwd(const saf_mixed_attn_args* a, const saf_tensor_t* dout, const saf_tensor_t* dalpha,
                         const saf_tensor_t* drho, void* stream) {
  Plan pl;
  if (int rc = plan_and_validate(a, 0, pl, false)) return rc;
  if (a->kvidx != nullptr)
    return fail(SAF_EUNSUPPORTED, "pattern gradients with kvidx (GQA) are not implemented (forward / prefill only)");
  if (pl.dtype == SAF_F32)
    return fail(SAF_EUNSUPPORTED, "pattern gradients take bf16 / fp16 attention inputs (float32 is not implemented)");
  if (!supported_bwd_hd(pl.HD))
    return fail(SAF_EUNSUPPORTED, "pattern gradients: head_dim %d is not supported (32, 64, 96, 128)", pl.HD);
  if (dout == nullptr || dalpha == nullptr || drho == nullptr)
    return fail(SAF_EINVAL, "dout, dalpha and drho are required");
  const std::vector<int> heads = decomp_heads_all(pl);
  if (heads.empty() || pl.T == 0 || pl.B == 0) return SAF_OK;
  const saf_tensor_t* bufs[3] = {&a->alpha, &a->rho, &a->z};
  const char* names[3] = {"alpha", "rho", "z"};
  for (int i = 0; i < 3; ++i) {
    const saf_tensor_t& t = *bufs[i];
    if (!present(t) || t.ndim != 2 || t.size[0] != pl.H || t.size[1] < pl.T)
      return fail(SAF_EINVAL, "pattern gradients need the (H, S) decomposed buffers (%s)", names[i]);
    if (t.dtype != SAF_F32 && t.dtype != SAF_BF16 && t.dtype != SAF_F16)
      return fail(SAF_EUNSUPPORTED, "unsupported %s dtype %s", names[i], dtype_name(t.dtype));
  }
  const saf_tensor_t* gr[2] = {dalpha, drho};
  for (int i = 0; i < 2; ++i) {
    const saf_tensor_t& t = *gr[i];
    if (!present(t) || t.ndim != 2 || t.size[0] != pl.H || t.size[1] < pl.T || t.dtype != SAF_F32)
      return fail(SAF_EINVAL, "dalpha and drho must be (H, S) float32 with S >= T");
    if (t.size[1] > 1 && t.stride[1] != 1) return fail(SAF_EALIGN, "dalpha and drho need a unit column stride");
  }
  if (!present(*dout) || dout->ndim != 4 || dout->dtype != a->out.dtype)
    return fail(SAF_EINVAL, "dout must match out's shape and dtype");
  for (int i = 0; i < 4; ++i)
    if (dout->size[i] != a->out.size[i]) return fail(SAF_EINVAL, "dout must match out's shape and dtype");
  if (int rc = check_act(*dout, "dout", 16)) return rc;
  if (int rc = check_act(a->out, "out", 16)) return rc;
  if ((int)heads.size() > kMaxHeads) return fail(SAF_EUNSUPPORTED, "too many decomposed heads");
  const int64_t need = saf_decomp_param_bwd_workspace_bytes(a);
  if (a->workspace == nullptr || a->workspace_bytes < need || reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
    return fail(SAF_EWORKSPACE, "pattern gradients need a 16-byte aligned %lld-byte workspace (got %lld)",
                (long long)need, (long long)a->workspace_bytes);
  BwdParams p{};
  p.v = a->v.data;
  p.out = a->out.data;
  p.dout = dout->data;
  p.v_sb = a->v.stride[0]; p.v_sh = a->v.stride[1]; p.v_st = a->v.stride[2];
  p.o_sb = a->out.stride[0]; p.o_sh = a->out.stride[1]; p.o_st = a->out.stride[2];
  p.do_sb = dout->stride[0]; p.do_sh = dout->stride[1]; p.do_st = dout->stride[2];
  p.B = pl.B;
  p.T = pl.T;
  p.n_live = (int)heads.size();   // the decomposed heads take the live slots here
  for (int i = 0; i < p.n_live; ++i) {
    p.out_head[i] = (int16_t)heads[i];
    p.pat_head[i] = (int16_t)heads[i];
  }
  p.delta = reinterpret_cast<float*>(a->workspace);
  p.alpha = a->alpha.data; p.rho = a->rho.data; p.z = a->z.data;
  p.a_dtype = a->alpha.dtype; p.r_dtype = a->rho.dtype; p.z_dtype = a->z.dtype;
  p.a_sh = a->alpha.stride[0]; p.a_ss = a->alpha.stride[1];
  p.r_sh = a->rho.stride[0]; p.r_ss = a->rho.stride[1];
  p.z_sh = a->z.stride[0]; p.z_ss = a->z.stride[1];
  p.dalpha = static_cast<float*>(dalpha->data);
  p.drho = static_cast<float*>(drho->data);
  p.da_hs = dalpha->stride[0];
  p.dr_hs = drho->stride[0];
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (int rc = launched(launch_bwd_delta(p, pl.dtype, pl.HD, st), "pattern-gradient delta")) return rc;
  return launched(launch_bwd_decomp_param(p, pl.dtype, pl.HD, st), "pattern gradients");
}

int64_t saf_mixed_attn_workspace_bytes(const saf_mixed_attn_args* args) {
  Plan pl;
  if (plan_and_validate(args, kDoFlash | kDoScan, pl, false)) return -1;
  if (pl.dtype == SAF_F32) return 0;  // no scan, no split
  return scan_ws_bytes(pl) + part_region_bytes(args, pl) + decomp_vp_bytes(pl);
}

}  // extern "C"

// ---- allocation-free forward ------------------------------------------------
// The workspace of saf_mixed_attn_fwd_noalloc: one fixed array per GPU that
// the library runs on, held until the process ends.  In host code `scratch`
// names a host-side stand-in, never a device address: its device address is
// read once per device (with that device current) by hipGetSymbolAddress and
// only that address is used.
namespace {

constexpr int64_t kScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device (looked up on the first
// call per device).
int scratch_address(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SAF_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SAF_EUNSUPPORTED, "device %d beyond %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(SAF_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SAF_OK;
}

}  // namespace

extern "C" {

int saf_mixed_attn_fwd_noalloc(const saf_mixed_attn_args* args, void* stream) {
  Plan pl;
  if (int rc = plan_and_validate(args, kDoAll, pl, false)) return rc;
  // the scan's look-back words must fit; the partials of the causally
  // balanced kernels are used when they fit too (else those kernels run
  // unsplit, with the same results)
  const int64_t need = scan_ws_bytes(pl);
  if (need > kScratchBytes)
    return fail(SAF_EWORKSPACE,
                "saf_mixed_attn_fwd_noalloc: the closed-form heads need %lld bytes of scratch, above the "
                "%lld-byte maximum (use saf_mixed_attn_fwd with a caller workspace)",
                (long long)need, (long long)kScratchBytes);
  const int64_t want = saf_mixed_attn_workspace_bytes(args);
  if (want < 0) return fail(SAF_EINVAL, "invalid arguments");
  saf_mixed_attn_args a = *args;
  if (int rc = scratch_address(&a.workspace)) return rc;
  a.workspace_bytes = std::min(want, kScratchBytes);
  return run(&a, kDoAll, stream);
}

int64_t saf_workspace_bytes(int32_t B, int32_t T, int32_t head_dim, int32_t n_scan_heads) {
  if (!supported_hd(head_dim)) return 0;
  return ws_layout(B, T, head_dim, n_scan_heads).total;
}

int saf_workspace_error(const void* workspace, void* stream, int32_t* error_out) {
  if (workspace == nullptr || error_out == nullptr) return fail(SAF_EINVAL, "workspace and error_out are required");
  uint32_t e = 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t rc = hipMemcpyAsync(&e, reinterpret_cast<const char*>(workspace) + 4, 4, hipMemcpyDeviceToHost, s);
  if (rc == hipSuccess) rc = hipStreamSynchronize(s);
  if (rc != hipSuccess) return fail(SAF_ELAUNCH, "reading the workspace failed: %s", hipGetErrorString(rc));
  *error_out = (int32_t)e;
  return SAF_OK;
}

int saf_time_next_kernel(void* begin_event, void* end_event) {
  if ((begin_event == nullptr) != (end_event == nullptr))
    return fail(SAF_EINVAL, "saf_time_next_kernel takes two events or none");
  g_time_begin = reinterpret_cast<hipEvent_t>(begin_event);
  g_time_end = reinterpret_cast<hipEvent_t>(end_event);
  return SAF_OK;
}

const char* saf_last_error(void) { return g_last_error.c_str(); }

const char* saf_version(void) { return "saf-mi355x 0.1.0 (gfx950)"; }

}  // extern "C"
