/*
 * saf_attn.h — C-ABI of libsafattn.so, the MI355X (gfx950) implementation of
 * Selective Attention Freezing's mixed-head causal attention prefill.
 *
 * The entry points replace the GPU launches behind the reference's operator
 * surface (reference files under waylonli/Selective-Attention-Freezing):
 *
 *   saf_mixed_attn_fwd       kernel/fused_attn.py:572-591 (_fwd + _fwd_kernel,
 *                            all head states in one call) and the GQA twin
 *                            qwen/kernel/fused_attn.py:581-603 (kvidx map)
 *   saf_flash_fwd            kernel/fused_attn.py:182-226 (_acc_flash, state 0)
 *   saf_frozen_dense_pv_fwd  kernel/fused_attn.py:125-143 (_acc_dense, state 1)
 *   saf_frozen_decomp_fwd    kernel/fused_attn.py:145-180 (_acc_decomp, state 2)
 *   saf_frozen_scan_fwd      state-2 heads whose pattern is the causal mean,
 *                            an exponential decay or a sliding window
 *                            (kernel/fused_attn.py:12-19 defines the pattern;
 *                            the reference evaluates it with _acc_decomp)
 *   saf_frozen_pv_fwd        kernel/frozen_attn.py:133-148 (_launch_fwd of
 *                            frozen_pv, compact frozen-head V)
 *
 * Conventions
 *   - Every tensor is described by saf_tensor_t: a device pointer, a dtype
 *     code, and 4-D sizes/strides counted in elements.  The innermost stride
 *     must be 1; q/k/v rows must start on 16-byte boundaries and out rows on
 *     8-byte boundaries (status SAF_EALIGN otherwise: make the tensor
 *     contiguous and call again).
 *   - The caller allocates every buffer, including out, the optional lse and
 *     the workspace.  The library allocates no device memory; its one device
 *     array (the scratch of saf_mixed_attn_fwd_noalloc) exists from the
 *     library's load on each GPU it runs on.
 *   - Head-routing tables (frozen, hidx, pidx, kvidx, closed_kind,
 *     closed_param) are HOST arrays of n_heads entries, read during the call.
 *   - Kernels are enqueued on `stream` (a hipStream_t) without any host
 *     synchronisation.  saf_mixed_attn_fwd and saf_mixed_attn_bwd also use a
 *     second stream of the library per device (created at first use, default
 *     priority), forked from `stream` and joined back into it by events within
 *     the call, under a mutex, so each call stays ordered on `stream`.  Calls
 *     are re-entrant; the other mutable global state is the thread-local error
 *     string (and the noalloc scratch array, shared by the calls of that one
 *     entry point).
 *   - Head dims: the forward entry points take HD in {32, 64, 96, 128, 256}
 *     (the reference's Triton kernels take any power of two; 256 is
 *     Qwen3.5's); the bf16 / fp16 backward entry points and the fused RoPE /
 *     q-k norm prologue take HD <= 128 and return SAF_EUNSUPPORTED above.
 *   - Activation dtypes: bf16 and fp16 run the MFMA kernels; float32 q/k/v
 *     (the reference's IEEE-dot contract, kernel/fused_attn.py:36-37) run
 *     fp32 vector-ALU kernels in saf_mixed_attn_fwd / _bwd, the per-kind
 *     entry points and saf_frozen_pv_fwd / _bwd, every HD above, with no
 *     workspace (closed-form heads go through their alpha / rho / z in the
 *     decomposed pass, so saf_frozen_scan_fwd has nothing to do for them).
 *     saf_decomp_param_bwd takes bf16 / fp16 only.
 *   - Return value: SAF_OK (0) or a negative status; saf_last_error() then
 *     holds a message for the calling thread.
 */
#ifndef SAF_ATTN_H
#define SAF_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  SAF_OK = 0,
  SAF_EINVAL = -1,        /* inconsistent shapes, indices or arguments */
  SAF_EUNSUPPORTED = -2,  /* dtype / head_dim / head count not implemented */
  SAF_EALIGN = -3,        /* pointer or stride alignment not met */
  SAF_ELAUNCH = -4,       /* a kernel launch failed */
  SAF_EWORKSPACE = -5     /* workspace missing or too small */
};

enum { SAF_F32 = 0, SAF_F16 = 1, SAF_BF16 = 2, SAF_I32 = 3 };

/* Head states (kernel/fused_attn.py:12-19, nanogpt/model.py:869-874). */
enum { SAF_LIVE = 0, SAF_FROZEN_DENSE = 1, SAF_FROZEN_DECOMP = 2 };

/* Closed forms of a decomposed pattern softmax(alpha[j] + rho[i-j]) with
 * alpha = 0: mean (rho = 0), decay (rho[d] = -c*d, param c > 0) and window
 * (rho[d] = 0 for d < w and -inf beyond, param w >= 1). */
enum { SAF_CLOSED_NONE = 0, SAF_CLOSED_MEAN = 1, SAF_CLOSED_DECAY = 2, SAF_CLOSED_WINDOW = 3 };

#define SAF_MAX_HEADS 128

typedef struct saf_tensor {
  void* data;         /* device pointer (NULL = absent) */
  int32_t dtype;      /* SAF_F32 / SAF_F16 / SAF_BF16 / SAF_I32 */
  int32_t ndim;       /* number of used sizes/strides (<= 4) */
  int64_t size[4];
  int64_t stride[4];  /* in elements */
} saf_tensor_t;

typedef struct saf_mixed_attn_args {
  /* q, k: (B, U, T, HD) compact live-head slots (U = live heads), or with
   * kvidx: k is (B, HKV, T, HD) raw key heads.  May be absent (data NULL)
   * when no head is live. */
  saf_tensor_t q, k;
  /* v: (B, H, T, HD), or (B, HKV, T, HD) with kvidx. */
  saf_tensor_t v;
  /* out: (B, H, T, HD), any strides with stride[3] == 1. */
  saf_tensor_t out;
  /* lse: optional (B, H, T) fp32, base-2 log-sum-exp of live heads. */
  saf_tensor_t lse;
  /* patt: (P, S, S) dense patterns, S >= T (required iff a head is state 1). */
  saf_tensor_t patt;
  /* alpha, rho, z: (H, S) decomposed buffers (required iff a head is
   * state 2 without a closed form), fp32 / bf16 / fp16. */
  saf_tensor_t alpha, rho, z;
  int32_t n_heads;              /* H (output heads) */
  const int32_t* frozen;        /* [H] head state, host */
  const int32_t* hidx;          /* [H] live head -> q/k slot, host; NULL = identity */
  const int32_t* pidx;          /* [H] dense head -> patt row, host; NULL = identity */
  const int32_t* kvidx;         /* [H] head -> k/v head (GQA), host; NULL = none */
  const int32_t* closed_kind;   /* [H] SAF_CLOSED_*, host; NULL = none */
  const float* closed_param;    /* [H] decay rate or window length, host */
  float sm_scale;               /* softmax scale (1/sqrt(HD) by default) */
  void* workspace;              /* device scratch, saf_workspace_bytes() bytes */
  int64_t workspace_bytes;
  int32_t flash_qtiles;         /* 0 = auto (1); 1 or 2 query tiles per wave (2 only up to hd 64) */
  int32_t scan_spin_limit;      /* 0 = default bound of each look-back wait; < 0 = give-up
                                   drill: every scan chunk after the first gives up at once
                                   (tests of the error path) */
  int32_t decomp_unsplit;       /* schedule of the decomposed heads (same results to fp32
                                   rounding):
                                   0 = automatic: saf_mixed_attn_fwd runs them with one
                                   workgroup per query block on the library's side stream
                                   beside the live-head kernel when live heads share the call
                                   (its workgroups fill the slots the causal imbalance leaves
                                   idle); otherwise, and in saf_frozen_decomp_fwd, their long
                                   query blocks are split into key segments (fp32 partials in
                                   the workspace region the live-head and dense kernels also
                                   use, then a combine);
                                   1 = one workgroup per query block, no partials, so a
                                   saf_frozen_decomp_fwd call may run on a caller's second
                                   stream beside saf_flash_fwd;
                                   -1 = always split, after the live-head kernel */
} saf_mixed_attn_args;

/* All head kinds: live flash, dense P.V, decomposed P.V, closed-form scan.
 * The closed-form scan and (see decomp_unsplit) the decomposed heads run on a
 * second stream of the library (one per device, default priority), forked
 * from and joined back into `stream` by events within the call, so the call
 * is ordered on `stream` like a single kernel. */
int saf_mixed_attn_fwd(const saf_mixed_attn_args* args, void* stream);

/* saf_mixed_attn_fwd without a caller workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation).  No counterpart in the reference (its
 * Triton launch needs no workspace).  args->workspace and workspace_bytes are
 * ignored: the call uses a fixed 64 MiB device array of the library instead
 * (one per GPU, held until the process ends) and calls no allocator.
 *   - Calls whose closed-form heads need more than 64 MiB of look-back words
 *     return SAF_EWORKSPACE before launching anything; the partials of the
 *     causally balanced kernels are used only when they fit as well (else
 *     those kernels run unsplit, with the same results).
 *   - Every call on a GPU shares that GPU's array: calls that overlap on one
 *     GPU (concurrent streams or threads) race and must be serialised by the
 *     caller.  What must start at zero is cleared by a fill kernel on
 *     `stream` at each call.
 *   - A scan look-back that gives up cannot be read back through
 *     saf_workspace_error here; its rows are NaN, as in saf_mixed_attn_fwd. */
int saf_mixed_attn_fwd_noalloc(const saf_mixed_attn_args* args, void* stream);

/* Subsets of saf_mixed_attn_fwd: each computes only its heads' rows of out. */
int saf_flash_fwd(const saf_mixed_attn_args* args, void* stream);
int saf_frozen_dense_pv_fwd(const saf_mixed_attn_args* args, void* stream);
int saf_frozen_decomp_fwd(const saf_mixed_attn_args* args, void* stream);
int saf_frozen_scan_fwd(const saf_mixed_attn_args* args, void* stream);

/* Backward of saf_mixed_attn_fwd (replaces _bwd and _FusedMixedAttn.backward,
 * kernel/fused_attn.py:593-648, with _bwd_preprocess / _bwd_dkdv / _bwd_dq
 * :291-591).  args is the forward's argument block, with args->lse the
 * forward's (B, H, T) base-2 LSE (required when a head is live) and a
 * workspace of saf_mixed_attn_bwd_workspace_bytes() bytes.  Writes dq, dk
 * (shaped like the compact q, k; only the slots of live heads) and dv (shaped
 * like v, every head): live heads get the gradients of causal softmax
 * attention, frozen heads only dV = P^T dO (closed-form heads through their
 * decomposed buffers, which must be passed); patterns and decomposed buffers
 * get no gradient.  kvidx (GQA) is refused as in the reference
 * (qwen/kernel/fused_attn.py:605-609). */
int saf_mixed_attn_bwd(const saf_mixed_attn_args* args, const saf_tensor_t* dout, const saf_tensor_t* dq,
                       const saf_tensor_t* dk, const saf_tensor_t* dv, void* stream);
int64_t saf_mixed_attn_bwd_workspace_bytes(const saf_mixed_attn_args* args);

/* Gradients of the decomposed heads' pattern parameters (trainable alpha /
 * rho; replaces _parameter_backward and PatternGradient.backward,
 * supplement/trainable_pattern_kernels.py:20-80, and the dispatch of
 * supplement/trainable_patterns.py:61-93).  args is the forward's argument
 * block (z the normalisers of the current alpha / rho), with a workspace of
 * saf_decomp_param_bwd_workspace_bytes() bytes; for every state-2 head
 * (closed-form ones through their buffers), summed over the batch:
 *   dS[i, j] = P[i, j] (dP[i, j] - delta_i), dP = dO V^T, delta_i = dO_i . out_i,
 *   dalpha[h, j] += sum_i dS[i, j],  drho[h, d] += sum_{i-j=d} dS[i, j]
 * into (H, S) float32 dalpha / drho that the caller zeroes (accumulated with
 * atomic adds: the summation order, and so the last bits, vary between
 * runs).  kvidx (GQA) is refused. */
int saf_decomp_param_bwd(const saf_mixed_attn_args* args, const saf_tensor_t* dout, const saf_tensor_t* dalpha,
                         const saf_tensor_t* drho, void* stream);
int64_t saf_decomp_param_bwd_workspace_bytes(const saf_mixed_attn_args* args);

/* frozen_pv: out[b, f] = patt[fz_idx[f], :T, :T] @ v[b, f] for compact
 * frozen-head values v (B, nf, T, HD); fz_idx is a host array of nf entries. */
int saf_frozen_pv_fwd(const saf_tensor_t* patt, const saf_tensor_t* v, const int32_t* fz_idx,
                      int32_t nf, int32_t T, const saf_tensor_t* out, void* stream);

/* Backward of frozen_pv (replaces _pv_bwd_kernel and _FrozenPV.backward,
 * kernel/frozen_attn.py:91-128, :150-182): dv[b, f, j] = sum over i >= j,
 * i < T of patt[fz_idx[f], i, j] dy[b, f, i] for j < T, with the pattern
 * rounded to dy's dtype and fp32 accumulation.  dy is (B, nf, T, HD), dv is
 * (B, nf, T', HD) with T' >= T: rows j >= T are not written (the caller
 * zeroes them).  The pattern must be lower-triangular, as for the forward. */
int saf_frozen_pv_bwd(const saf_tensor_t* patt, const saf_tensor_t* dy, const int32_t* fz_idx,
                      int32_t nf, int32_t T, const saf_tensor_t* dv, void* stream);

/* Rotary embedding of the live-head q (B, Uq, T, HD) and k (B, Uk, T, HD), in
 * place (the two may be interleaved views of one projection output): Llama
 * half rotation with the (T', HD) cos/sin caches (fp32, bf16 or fp16),
 * positions 0..T-1, fp32 arithmetic, one rounding to the activation dtype.
 * Replaces apply_rotary_pos_emb (nanogpt/model.py:63-68) on the fused
 * path (:1007-1008). */
int saf_rope_qk_inplace(const saf_tensor_t* q, const saf_tensor_t* k, const saf_tensor_t* cos,
                        const saf_tensor_t* sin, void* stream);

/* Qwen3 attention prologue on the live-head q (B, Uq, T, HD) and the raw key
 * heads k (B, HKV, T, HD), in place: per-head RMSNorm over HD with the
 * (HD,) weights (fp32 statistics, x <- w * round(x * rsqrt(mean(x^2) + eps))
 * rounded to the activation dtype, as Qwen3RMSNorm), then the rotation of
 * saf_rope_qk_inplace.  Replaces q_norm / k_norm + apply_rotary_pos_emb of the
 * Qwen3 fused branch (qwen/nanogpt/hybrid_prior_attention.py:543-572). */
int saf_qk_rmsnorm_rope_inplace(const saf_tensor_t* q, const saf_tensor_t* k, const saf_tensor_t* q_weight,
                                const saf_tensor_t* k_weight, float eps, const saf_tensor_t* cos,
                                const saf_tensor_t* sin, void* stream);

/* Residual add + LayerNorm of the GPT block, in place on the residual x
 * (rows, C): x += delta when delta is present (one rounding to x's dtype),
 * then out = (x - mean) * rsqrt(var + eps) * weight + bias over C, computed
 * in fp32 from the rounded x (bias may be absent).  x, delta and out are 2-D
 * bf16 / fp16 with unit channel stride; weight and bias (C,) in fp32, bf16
 * or fp16.  C is even and at most 2048.  Replaces LayerNorm.forward (nanogpt/model.py:45-54) and the
 * residual additions of Block.forward (:1214-1240) on the prefill path. */
int saf_add_layernorm(const saf_tensor_t* x, const saf_tensor_t* delta, const saf_tensor_t* weight,
                      const saf_tensor_t* bias, float eps, const saf_tensor_t* out, void* stream);

/* Residual add + RMSNorm of a Qwen3 decoder block, with the operand rules of
 * saf_add_layernorm (no bias): x += delta when delta is present, then
 * out = weight * round(x * rsqrt(mean(x^2) + eps)) over C, the mean of
 * squares in fp32 from the rounded x, the normalised x rounded to x's dtype
 * before the weight multiplies it and the product rounded again.  Replaces
 * transformers' Qwen3RMSNorm.forward on the decoder blocks of the Qwen caller
 * (input_layernorm, post_attention_layernorm, the final norm). */
int saf_add_rmsnorm(const saf_tensor_t* x, const saf_tensor_t* delta, const saf_tensor_t* weight, float eps,
                    const saf_tensor_t* out, void* stream);

/* MLP up-projection and activation of the GPT block in one kernel:
 * out = gelu(x weight^T) with gelu(u) = u / 2 (1 + erf(u / sqrt 2)) (the exact
 * GELU, nn.GELU's default), for x (M, K), weight (N, K) (an nn.Linear weight
 * without bias) and out (M, N), all bf16 or all fp16 with unit column stride;
 * fp32 accumulation, the GELU in fp32 on the accumulator, one rounding of out.
 * N is a multiple of 256 and K of 128 (any M); x and weight rows 16-byte
 * aligned, out rows 16-byte aligned.  No workspace.  Replaces c_fc followed by
 * gelu in MLP.forward (nanogpt/model.py:1202-1204) on the prefill path. */
int saf_linear_gelu(const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out, void* stream);

/* Exact GELU (nn.GELU()) of a contiguous bf16 / fp16 tensor x in place:
 * x <- x Phi(x), in fp32 (the polynomial / A&S evaluation of
 * saf_linear_gelu, within 5.3e-6 of exact), one rounding; the element count a
 * multiple of 8 and x 16-byte aligned.  For the MLP whose up-projection runs
 * as a library GEMM (K above the fused kernel's range): replaces the GELU of
 * MLP.forward (nanogpt/model.py:1204). */
int saf_gelu_inplace(const saf_tensor_t* x, void* stream);

/* SwiGLU half of a gated MLP in one kernel: out = silu(x Wg^T) * (x Wu^T),
 * silu(u) = u / (1 + e^-u), for x (M, K) and weight (N, K) holding the gate
 * and up rows interleaved in blocks of 64 (gate rows 64b..64b+63, then up
 * rows 64b..64b+63, for b = 0, 1, ...), out (M, N / 2); fp32 accumulation and
 * activation, one rounding of out.  Same dtype, N / K and alignment rules as
 * saf_linear_gelu (so the MLP width N / 2 is a multiple of 128).  No
 * workspace.  Replaces act_fn(gate_proj(x)) * up_proj(x) of transformers'
 * Qwen3MLP (the C4 caller's MLP, SiLU activation) on the prefill path. */
int saf_linear_swiglu(const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out, void* stream);

/* Indexed QKV projection with the rotary embedding in one kernel:
 * out = x weight^T for x (M, K) = (B T, K) and weight (N, K) the gathered
 * [Wq[live]; Wk[live]; Wv] rows (zero rows may pad N), with the first n_rope
 * columns (the live heads' q and k, heads of head_dim columns) rotated at
 * position t = row mod seq_len by the Llama half rotation
 *   out[d] = u[d] cos[t][d] - u[d + hd/2] sin[t][d]   (d < hd/2),
 *   out[d] = u[d] cos[t][d] + u[d - hd/2] sin[t][d]   (d >= hd/2),
 * computed in fp32 on the accumulator and rounded once; the other columns are
 * the plain product.  bf16 / fp16 throughout (cos / sin (>= seq_len, >= hd)
 * in x's dtype, unit column stride, 8-byte aligned rows); N a multiple of 256,
 * K of 128, n_rope a multiple of 128, head_dim 64 or 128, M a multiple of
 * seq_len; x, weight and out rows 16-byte aligned.  No workspace.  Replaces
 * the projection of the gathered weight (nanogpt/model.py:920-944,
 * :1003-1004) and apply_rotary_pos_emb on the live q / k (:57-99,
 * :1007-1008) on the prefill path. */
int saf_linear_rope(const saf_tensor_t* x, const saf_tensor_t* weight, const saf_tensor_t* out, int32_t n_rope,
                    int32_t head_dim, int32_t seq_len, const saf_tensor_t* cos, const saf_tensor_t* sin,
                    void* stream);

/* Row normalisers of decomposed patterns: z[h, i] = logsumexp over j <= i of
 * alpha[h, j] + rho[h, i - j], for (H, S) fp32 alpha, rho and z with unit
 * column stride (any row stride).  Rows whose logits are all -inf get -inf.
 * One pass, no workspace.  Replaces decomposed_logz
 * (kernel/fused_attn.py:101-116), which the reference computes in row chunks
 * of materialised (H, rows, S) logits at freeze time (nanogpt/model.py) and
 * per call when alpha comes without z (kernel/fused_attn.py:690-694). */
int saf_decomposed_logz(const saf_tensor_t* alpha, const saf_tensor_t* rho, const saf_tensor_t* z, void* stream);

/* Backward of saf_decomposed_logz for an upstream gradient gz = dL/dz:
 *   dalpha[h, j] = sum_{i >= j} gz[h, i] exp(alpha[h, j] + rho[h, i - j] - z[h, i])
 *   drho[h, d]   = sum_{i >= d} gz[h, i] exp(alpha[h, i - d] + rho[h, d] - z[h, i])
 * with z the forward's normalisers; all six (H, S) fp32 with unit column
 * stride; dalpha and drho are written (not accumulated).  Rows whose z is
 * -inf contribute nothing.  Replaces the autograd of the reference's
 * differentiable normalisers decomp_log_normalizers_fft
 * (nanogpt/dynamic_freeze.py:330-361), which the pattern fits backpropagate
 * through (:362-390); the sums here are exact O(S^2) sweeps, not an FFT. */
int saf_decomposed_logz_bwd(const saf_tensor_t* alpha, const saf_tensor_t* rho, const saf_tensor_t* z,
                            const saf_tensor_t* gz, const saf_tensor_t* dalpha, const saf_tensor_t* drho,
                            void* stream);

/* Workspace needed by saf_frozen_scan_fwd for n_scan_heads closed-form heads
 * (0 bytes when there are none). */
int64_t saf_workspace_bytes(int32_t B, int32_t T, int32_t head_dim, int32_t n_scan_heads);

/* Workspace that lets one saf_mixed_attn_fwd (or per-kind) call with these
 * arguments (workspace fields ignored) use every optimisation: the closed-form
 * scan's look-back words, then one region of fp32 partials shared by the
 * live-head, dense P.V and decomposed kernels' causal load balancing (long
 * query blocks split into key segments and merged by a combine kernel; the
 * kernels run one after the other on the stream), then the inputs of the
 * decomposed heads' factored form (bf16 / fp16, hd <= 128: key-scaled values,
 * rho and z in log2 units and their per-64-block maxima and minima, written
 * by a pre-pass).  A smaller
 * workspace still works if it covers the scan: those kernels then run
 * unsplit, and decomposed heads rebuild P cell by cell (equal to rounding).
 * Partials need a 16-byte aligned workspace, the factored form a 256-byte
 * aligned one.  Returns -1 on invalid arguments.  No counterpart in the
 * reference (its Triton launch needs no workspace). */
int64_t saf_mixed_attn_workspace_bytes(const saf_mixed_attn_args* args);

/* Reads the scan's look-back error word of a workspace (synchronises
 * `stream` first): 1 if a look-back wait gave up, else 0.  A wait that gives
 * up leaves NaN in its chunk's rows and in every later chunk of that
 * (batch, head) sequence, never a silently incomplete sum. */
int saf_workspace_error(const void* workspace, void* stream, int32_t* error_out);

/* Kernel timing: the next main kernel this host thread launches through an
 * attention entry point (the flash, dense P.V, decomposed P.V or scan kernel;
 * not the workspace clear or the merge of split query blocks) is bracketed by
 * hipEventRecord(begin_event) and hipEventRecord(end_event) on its stream, so
 * hipEventElapsedTime gives that kernel's own duration.  One-shot; two NULLs
 * cancel.  No counterpart in the reference (profiling hook for the roofline
 * measurement). */
int saf_time_next_kernel(void* begin_event, void* end_event);

const char* saf_last_error(void);
const char* saf_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SAF_ATTN_H */
