"""Mixed-head causal attention: live and frozen heads behind one call.

Drop-in for the reference operator ``fused_mixed_attn``
(/root/reference/kernel/fused_attn.py:650-734, with the GQA ``kvidx`` map of
/root/reference/qwen/kernel/fused_attn.py:667-768).  Head states:

    0  live               y = softmax(Q K^T * sm_scale) V, causal
    1  frozen, dense      y_i = sum_{j<=i} patt[pidx(h), i, j] v_j
    2  frozen, decomposed y_i = sum_{j<=i} exp(alpha[j] + rho[i-j] - z[i]) v_j

The work runs in libsafattn.so on the current HIP stream: a live-head flash
kernel on bf16/fp16 MFMA, a dense P.V MFMA kernel, a decomposed P.V kernel
(factored Toeplitz form or P rebuilt per cell), and, for decomposed heads
whose pattern is the causal mean, an exponential decay or a sliding window
(``closed_form=``), a single-pass scan that reads V once.  The scan and the
decomposed heads run on a second stream beside the live-head kernel, joined
before the call returns.  Output is in natural head order.

Pattern helpers (``make_rho_band``, ``decomp_logits``, ``decomposed_logz``)
follow the reference's definitions (/root/reference/kernel/fused_attn.py:50-116).
``decomposed_logz`` of device tensors runs one HIP kernel
(``saf_decomposed_logz``); the other two are single torch ops.
"""
import math

import numpy as np
import torch

from . import _ext

RCP_LN2 = 1.4426950408889634   # 1 / ln 2

# Rows of the reference's pre-expanded rho band (its BLOCK_M).  The HIP
# decomposed kernel reads rho directly, so the band is accepted for API
# compatibility and validated for shape, but never read.
BAND_ROWS = 64

# Closed-form codes (include/saf_attn.h SAF_CLOSED_*)
CLOSED_NONE, CLOSED_MEAN, CLOSED_DECAY, CLOSED_WINDOW = 0, 1, 2, 3


def fused_attn_usable(q):
    """True for tensors on a HIP device (torch's "cuda" device on ROCm).

    Deliberately independent of whether libsafattn.so was built: on a GPU the
    operator must run the HIP path or fail loudly, never fall back."""
    return bool(q.is_cuda)


def make_rho_band(rho):
    """(H, S) rho -> (H, BAND_ROWS, S) band with band[h, r, u] =
    rho[h, r - u + S - BAND_ROWS], -inf where that index leaves [0, S)
    (/root/reference/kernel/fused_attn.py:65-80)."""
    H, S = rho.shape
    assert S % BAND_ROWS == 0, \
        f"decomposed prior buffer length {S} must be a multiple of {BAND_ROWS}"
    src = (torch.arange(BAND_ROWS, device=rho.device)[:, None]
           - torch.arange(S, device=rho.device)[None, :] + (S - BAND_ROWS))
    valid = (src >= 0) & (src < S)
    band = rho[:, src.clamp(0, S - 1)]
    return band.masked_fill(~valid, float("-inf")).contiguous()


def decomp_logits(alpha, rho, rows=None):
    """L[h, i, j] = alpha[h, j] + rho[h, i - j] for j <= i, -inf above the
    diagonal; rows=(r0, r1) selects a row range
    (/root/reference/kernel/fused_attn.py:83-98)."""
    H, S = alpha.shape
    r0, r1 = (0, S) if rows is None else rows
    i = torch.arange(r0, r1, device=alpha.device)[:, None]
    j = torch.arange(S, device=alpha.device)[None, :]
    dist = i - j
    logits = alpha[:, None, :] + rho[:, dist.clamp(min=0)]
    return logits.masked_fill(dist < 0, float("-inf"))


@torch.no_grad()
def decomposed_logz(alpha, rho, chunk=None):
    """z[h, i] = logsumexp_{j <= i}(alpha[h, j] + rho[h, i - j])
    (/root/reference/kernel/fused_attn.py:101-116).

    Device tensors: one pass of libsafattn.so ``saf_decomposed_logz`` on the
    current stream (fp32 arithmetic, no (H, rows, S) logits materialised;
    ``chunk`` is ignored).  Host tensors (freeze-time set-up on the CPU, as
    the reference's helper allows): the reference's row-chunked definition,
    the (H, chunk, S) workspace near 2^27 elements.  Returns alpha's dtype."""
    H, S = alpha.shape
    if alpha.is_cuda:
        z = torch.empty(H, S, device=alpha.device, dtype=torch.float32)
        if H * S == 0:
            return z.to(alpha.dtype)
        a32 = alpha.float()
        r32 = rho.to(device=alpha.device, dtype=torch.float32)
        if S > 1:
            a32 = a32 if a32.stride(1) == 1 else a32.contiguous()
            r32 = r32 if r32.stride(1) == 1 else r32.contiguous()
        rc = _ext.lib().saf_decomposed_logz(_ext.tensor_desc(a32), _ext.tensor_desc(r32), _ext.tensor_desc(z),
                                            _ext.current_stream_ptr(alpha.device))
        _ext.check(rc)
        return z if alpha.dtype == torch.float32 else z.to(alpha.dtype)
    if chunk is None:
        chunk = max(1, (1 << 27) // max(H * S, 1))
    z = torch.empty_like(alpha)
    for r0 in range(0, S, chunk):
        r1 = min(r0 + chunk, S)
        z[:, r0:r1] = decomp_logits(alpha, rho, rows=(r0, r1)).logsumexp(-1)
    return z


class _NormalisersFn(torch.autograd.Function):
    """z = logsumexp_{j<=i}(alpha_j + rho_{i-j}) on HIP, with its exact
    backward (saf_decomposed_logz_bwd)."""

    @staticmethod
    def forward(ctx, alpha, rho):
        a32 = alpha.detach().float().contiguous()
        r32 = rho.detach().float().contiguous()
        z = decomposed_logz(a32, r32)
        ctx.save_for_backward(a32, r32, z)
        ctx.dtypes = (alpha.dtype, rho.dtype)
        return z.to(alpha.dtype)

    @staticmethod
    def backward(ctx, gz):
        a32, r32, z = ctx.saved_tensors
        da = torch.empty_like(a32)
        dr = torch.empty_like(r32)
        g = gz.float().contiguous()
        if a32.numel():
            _ext.check(_ext.lib().saf_decomposed_logz_bwd(
                _ext.tensor_desc(a32), _ext.tensor_desc(r32), _ext.tensor_desc(z), _ext.tensor_desc(g),
                _ext.tensor_desc(da), _ext.tensor_desc(dr), _ext.current_stream_ptr(a32.device)))
        return da.to(ctx.dtypes[0]), dr.to(ctx.dtypes[1])


def decomp_log_normalizers(alpha, rho):
    """Row log-normalisers z[h, i] = logsumexp_{j <= i}(alpha[h, j] +
    rho[h, i - j]) of (N, T) logit vectors, differentiable in alpha and rho.

    The quantity of the reference's decomp_log_normalizers_fft
    (/root/reference/nanogpt/dynamic_freeze.py:330-361), which the pattern
    fits backpropagate through.  Device tensors: the exact O(T^2) sums of
    saf_decomposed_logz and saf_decomposed_logz_bwd (fp32, no FFT round-off,
    no range shifts needed); host tensors: the row-chunked torch definition
    under torch autograd."""
    if alpha.shape != rho.shape or alpha.ndim != 2:
        raise ValueError("alpha and rho must have matching (N, T) shapes")
    if alpha.is_cuda:
        return _NormalisersFn.apply(alpha, rho)
    H, S = alpha.shape
    rows = []
    chunk = max(1, (1 << 24) // max(H * S, 1))
    for r0 in range(0, S, chunk):
        rows.append(decomp_logits(alpha, rho, rows=(r0, min(S, r0 + chunk))).logsumexp(-1))
    return torch.cat(rows, dim=-1)


# reference name (nanogpt/dynamic_freeze.py:330): same contract, exact sums
decomp_log_normalizers_fft = decomp_log_normalizers


# ---------------------------------------------------------------------------
# Closed-form recognition of decomposed patterns
# ---------------------------------------------------------------------------

@torch.no_grad()
def classify_closed_form(alpha, rho, z=None, heads=None, rtol=1e-5):
    """Recognise decomposed heads whose pattern softmax(alpha[j] + rho[i-j]) is
    the causal mean, an exponential decay or a sliding window.

    Returns (kind int32[H], param float32[H]) as numpy arrays: kind is
    CLOSED_MEAN (alpha = rho = 0), CLOSED_DECAY (alpha = 0, rho[d] = -c d with
    c > 0; param = c) or CLOSED_WINDOW (alpha = 0, rho[d] = 0 for d < w and
    -inf beyond; param = w), else CLOSED_NONE.  If z is given it must be the
    pattern's own normaliser (checked against the closed form), otherwise the
    head is left to the decomposed P.V kernel, which uses z as given.  Runs once
    per freeze change (one host sync)."""
    H, S = alpha.shape
    a = alpha.detach().float().cpu()
    r = rho.detach().float().cpu()
    zz = None if z is None else z.detach().float().cpu()
    kind = np.zeros(H, dtype=np.int32)
    param = np.zeros(H, dtype=np.float32)
    d = torch.arange(S, dtype=torch.float64)
    rows = heads if heads is not None else range(H)
    for h in rows:
        if not bool((a[h] == 0).all()):
            continue
        rh = r[h].double()
        finite = torch.isfinite(rh)
        k = CLOSED_NONE
        if bool((rh == 0).all()):
            k, p = CLOSED_MEAN, 0.0
            logz = torch.log(d + 1.0)
        elif bool(finite[0]) and rh[0] == 0 and not bool(finite.all()) and \
                bool((rh[finite] == 0).all()):
            w = int(finite.long().sum())
            if bool(finite[:w].all()) and bool((rh[w:] == float("-inf")).all()):
                k, p = CLOSED_WINDOW, float(w)
                logz = torch.log(torch.clamp(d + 1.0, max=float(w)))
        elif bool(finite.all()) and rh[0] == 0 and S > 1 and rh[1] < 0:
            c = -float(r[h, 1])
            if bool(((rh + c * d).abs() <= rtol * (1.0 + c * d)).all()):
                k, p = CLOSED_DECAY, c
                # log sum_{t<=i} e^{-c t} = log(-expm1(-c (i+1))) - log(-expm1(-c))
                logz = torch.log(-torch.expm1(-c * (d + 1.0))) - math.log(-math.expm1(-c))
        if k == CLOSED_NONE:
            continue
        if zz is not None:
            zerr = (zz[h].double() - logz).abs()
            if not bool((zerr <= 1e-4 * (1.0 + logz.abs())).all()):
                continue
        kind[h] = k
        param[h] = p
    return kind, param


# ---------------------------------------------------------------------------
# Host copies of the device routing tables
# ---------------------------------------------------------------------------

def _host_table(t, np_dtype=np.int32):
    """Host copy of a small per-head table, cached on the tensor itself and
    refreshed when its version counter moves (one sync per change, the same
    moment the reference syncs: nanogpt/model.py:853, :875)."""
    if t is None:
        return None
    if not isinstance(t, torch.Tensor):
        return np.asarray(t, dtype=np_dtype)
    cached = getattr(t, "_saf_host", None)
    if cached is not None and cached[0] == t._version and cached[1] == t.data_ptr():
        return cached[2]
    arr = t.detach().cpu().numpy().astype(np_dtype, copy=False).reshape(-1)
    arr = np.ascontiguousarray(arr)
    try:
        t._saf_host = (t._version, t.data_ptr(), arr)
    except (AttributeError, RuntimeError):
        pass
    return arr


def _row_aligned(t, align):
    if t is None:
        return True
    if t.stride(-1) != 1 and t.size(-1) != 1:
        return False
    es = t.element_size()
    if t.data_ptr() % align:
        return False
    return all(s <= 1 or (st * es) % align == 0
               for s, st in zip(t.shape[:-1], t.stride()[:-1]))


def _aligned_view(t, align=16):
    return t if _row_aligned(t, align) else t.contiguous()


class KernelTimer:
    """Times the main kernel of each per-kind launch of fused_mixed_attn with
    HIP events that the library records on the launch stream right around
    that kernel (saf_time_next_kernel: the flash, dense P.V, decomposed P.V or
    scan kernel alone, without the workspace clear or the merge of split
    query blocks), and records the algorithmic work of that launch:
    flash: 4*hd*T(T+1)/2 flops per (batch, live head); scan: V read once and
    Y written once, 2*T*hd*elem bytes per (batch, closed-form head)."""

    KINDS = ("flash", "scan", "dense", "decomp")

    def __init__(self):
        self.records = {k: [] for k in self.KINDS}

    def summary(self):
        """{kind: (launches, total_ms, total_work)} after synchronisation."""
        out = {}
        for k, recs in self.records.items():
            if recs:
                ms = sum(a.elapsed_time(b) for a, b, _ in recs)
                out[k] = (len(recs), ms, sum(w for _, _, w in recs))
        return out


_TIMER = None
_SIDE_STREAMS = {}


def _side_stream(device):
    """A second stream per device (default priority) for the closed-form scan
    and the decomposed heads when each kernel of a call is timed
    (KernelTimer); untimed calls use the library's own side stream."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _SIDE_STREAMS:
        _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return _SIDE_STREAMS[idx]


def set_kernel_timer(timer):
    """Install (or remove with None) a KernelTimer for subsequent calls."""
    global _TIMER
    _TIMER = timer


class _MixedAttnFn(torch.autograd.Function):
    """Autograd node of fused_mixed_attn (kernel/fused_attn.py:621-647 of the
    reference): the forward runs the HIP forward and keeps what the backward
    needs (the output through save_for_backward, so no reference cycle holds
    it; the base-2 LSE of the live heads, the routing tables and the fixed
    pattern buffers in the backward closure); the backward runs
    saf_mixed_attn_bwd.  Frozen heads have no q/k slot, so they get no Q/K
    gradient; patterns and the decomposed buffers are constants here (no
    gradient: trainable alpha / rho go through supplement.PatternGradient,
    as in the reference's supplement/trainable_patterns.py:61-93)."""

    @staticmethod
    def forward(ctx, q, k, v, run, bwd):
        out = run()
        ctx.bwd = bwd
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx, dout):
        (out,) = ctx.saved_tensors
        dq, dk, dv = ctx.bwd(dout, out)
        ctx.bwd = None   # release the forward's buffers now
        return dq, dk, dv, None, None


def fused_mixed_attn(q, k, v, patt, frozen, hidx=None, pidx=None,
                     sm_scale=None, alpha=None, rho=None, z=None,
                     rho_band=None, validate=True, kvidx=None,
                     closed_form=None, lse=None, flash_qtiles=0, scan_spin_limit=0,
                     decomp_unsplit=None):
    """Causal attention over all heads, frozen heads using a fixed prior.

    Arguments follow /root/reference/kernel/fused_attn.py:650-680 (and
    ``kvidx`` from the GQA twin):
      v        (B, H, T, HD), or the raw (B, HKV, T, HD) heads with kvidx
      q, k     (B, U, T, HD) compact live-head slots (hidx[h] = slot of h);
               with kvidx, k is the raw (B, HKV, T, HD) key heads
      patt     (P, S, S) dense patterns, S >= T (pidx[h] selects a row)
      frozen   (H,) int32 head states 0 / 1 / 2
      alpha, rho, z  (H, S) decomposed buffers; z defaults to
               decomposed_logz(alpha, rho) computed per call
      rho_band accepted for compatibility (shape-checked, not read)
    Extensions of this build:
      closed_form  (kind int32[H], param float32[H]) from
               classify_closed_form(): state-2 heads with a non-zero kind run
               the closed-form scan instead of the decomposed P.V kernel
      lse      optional (B, H, T) fp32 output for the live heads' base-2 LSE
      flash_qtiles 0 (auto: 1) / 1 / 2 query tiles per wave of the flash kernel
               (2 applies up to hd 64; larger heads use 1)
      scan_spin_limit  0 = default bound of the scan's look-back waits; < 0
               is the give-up drill that tests the error path (every scan
               chunk after the first gives up: NaN rows, and with validate
               a RuntimeError)
      decomp_unsplit  None (auto) = True when live heads share the call;
               True: decomposed heads run one workgroup per query block,
               beside the live-head kernel on a side stream when there is
               one; False: key-segment split with partials and a combine,
               after the live-head kernel on the current stream
    Returns (B, H, T, HD) in natural head order, strided like v (like the
    reference's empty_like(v)).
    """
    H = frozen.numel()
    if sm_scale is None:
        sm_scale = 1.0 / (v.size(-1) ** 0.5)
    kv_identity = kvidx is None
    if alpha is not None and z is None:
        z = decomposed_logz(alpha.float(), rho.float()).to(alpha.dtype)
    if v.dtype == torch.float32:
        # the float32 kernels have no scan: closed forms run through their
        # decomposed buffers like the other state-2 heads
        closed_form = None
    if validate:
        _validate(q, k, v, patt, frozen, hidx, pidx, alpha, rho, z, rho_band, kvidx)
    if not v.is_cuda:
        raise RuntimeError(
            "fused_mixed_attn runs on HIP devices only (got a CPU tensor); "
            "this build has no CPU kernel path")

    frozen_h = _host_table(frozen)
    hidx_h = None if hidx is None else _host_table(hidx)
    pidx_h = None if pidx is None else _host_table(pidx)
    kvidx_h = None if kvidx is None else _host_table(kvidx)
    ck = cp = None
    if closed_form is not None:
        ck = _host_table(closed_form[0], np.int32)
        cp = _host_table(closed_form[1], np.float32)

    B, HV, T, HD = v.shape
    n_live = int((frozen_h == 0).sum())
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q, k, v))
    if needs_grad and n_live and lse is None:
        # the backward recomputes P from the forward's base-2 LSE
        lse = torch.empty((B, H, T), device=v.device, dtype=torch.float32)
    q_d = k_d = None
    if n_live:
        q_d = _aligned_view(q, 16)
        k_d = _aligned_view(k, 16)
    v_d = _aligned_view(v, 16)
    if v_d.stride(2) > v_d.stride(1):
        # v is a T-major view (the model's (B, T, H, hd) projection output):
        # keep that layout so the caller's transpose(1, 2).reshape is free,
        # as the reference's empty_like(v) does for a dense v (with kvidx the
        # output still has all H query heads)
        out = torch.empty((B, T, H, HD), device=v.device, dtype=v.dtype).transpose(1, 2)
    elif kv_identity:
        out = torch.empty_like(v_d)
        if not _row_aligned(out, 8):
            out = torch.empty((B, H, T, HD), device=v.device, dtype=v.dtype)
    else:
        out = torch.empty((B, H, T, HD), device=v.device, dtype=v.dtype)

    n_scan = 0
    if ck is not None:
        n_scan = int(((frozen_h == 2) & (ck != 0)).sum())
    L = _ext.lib()

    need_dec = alpha is not None and bool(
        ((frozen_h == 2) & ((ck == 0) if ck is not None else True)).any())
    # the backward runs closed-form heads through their decomposed buffers
    need_dec = need_dec or (needs_grad and alpha is not None and bool((frozen_h == 2).any()))

    args = _ext.SafMixedAttnArgs()
    args.q = _ext.tensor_desc(q_d)
    args.k = _ext.tensor_desc(k_d)
    args.v = _ext.tensor_desc(v_d)
    args.out = _ext.tensor_desc(out)
    args.lse = _ext.tensor_desc(lse)
    args.patt = _ext.tensor_desc(patt)
    if need_dec:
        args.alpha = _ext.tensor_desc(alpha)
        args.rho = _ext.tensor_desc(rho)
        args.z = _ext.tensor_desc(z)
    args.n_heads = H
    keep = [_ext.host_i32(frozen_h), _ext.host_i32(hidx_h), _ext.host_i32(pidx_h),
            _ext.host_i32(kvidx_h), _ext.host_i32(ck), _ext.host_f32(cp)]
    args.frozen, args.hidx, args.pidx, args.kvidx, args.closed_kind = keep[:5]
    args.closed_param = keep[5]
    args.sm_scale = float(sm_scale)
    args.flash_qtiles = int(flash_qtiles)
    args.scan_spin_limit = int(scan_spin_limit)
    # scan look-back words + partials of the causally balanced live-head kernel
    ws_bytes = int(L.saf_mixed_attn_workspace_bytes(args))
    if ws_bytes < 0:
        _ext.check(L.saf_mixed_attn_fwd(args, None))  # raises with the validation message
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=v.device) if ws_bytes else None
    args.workspace = None if ws is None else ws.data_ptr()
    args.workspace_bytes = ws_bytes

    n_dense = int((frozen_h == 1).sum())
    n_dec = int((frozen_h == 2).sum()) - n_scan

    work = {"flash": (L.saf_flash_fwd, n_live * B * 4 * HD * T * (T + 1) // 2),
            "scan": (L.saf_frozen_scan_fwd, n_scan * B * 2 * T * HD * v.element_size()),
            "dense": (L.saf_frozen_dense_pv_fwd, n_dense * B * 2 * HD * T * (T + 1) // 2),
            "decomp": (L.saf_frozen_decomp_fwd, n_dec * B * 2 * HD * T * (T + 1) // 2)}

    def run():
        timer = _TIMER
        cur = torch.cuda.current_stream(v.device)

        def launch(kind, strm):  # one timed per-kind call
            fn, w = work[kind]
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(strm)  # creates the HIP events; the library re-records them
            e1.record(strm)
            _ext.check(L.saf_time_next_kernel(e0.cuda_event, e1.cuda_event))
            rc = fn(args, strm.cuda_stream)
            L.saf_time_next_kernel(None, None)  # never left pending for a later call
            _ext.check(rc)
            timer.records[kind].append((e0, e1, w))

        if timer is None:
            # one call: the library runs the closed-form scan and the
            # decomposed heads on its side stream beside the live-head kernel
            args.decomp_unsplit = {None: 0, True: 1, False: -1}[decomp_unsplit]
            _ext.check(L.saf_mixed_attn_fwd(args, cur.cuda_stream))
        else:
            # the same schedule through the per-kind entry points, each kernel
            # timed on its own stream: decomposed heads beside live ones run
            # one workgroup per query block (decomp_unsplit = 1), so the
            # live-head kernel's workgroups fill the slots their causal
            # imbalance leaves idle and no key-segment partials are needed
            unsplit = bool(n_live) if decomp_unsplit is None else bool(decomp_unsplit)
            args.decomp_unsplit = 1 if unsplit else -1
            dec_side = bool(n_dec and n_live and unsplit)
            if (n_scan and (n_live or n_dense or n_dec)) or dec_side:
                # disjoint output rows and workspace regions; joined before
                # returning
                side = _side_stream(v.device)
                side.wait_stream(cur)
                if dec_side:
                    launch("decomp", side)
                if n_scan:
                    launch("scan", side)
                for kind in ("flash", "dense", "decomp"):
                    if work[kind][1] and not (kind == "decomp" and dec_side):
                        launch(kind, cur)
                cur.wait_stream(side)
            else:
                for kind in KernelTimer.KINDS:
                    if work[kind][1]:
                        launch(kind, cur)
        if n_scan and validate:
            # a look-back wait that gave up leaves NaN rows (never a silently
            # incomplete sum); with validate the call also raises
            err = _ext.ctypes.c_int32(0)
            _ext.check(L.saf_workspace_error(args.workspace, cur.cuda_stream, _ext.ctypes.byref(err)))
            if err.value:
                raise RuntimeError(
                    "closed-form scan: a look-back wait gave up (scan_spin_limit reached); "
                    "the affected rows of the output are NaN")
        return out

    # every tensor the argument block points to stays alive until the backward
    # (out itself is saved by the autograd node and passed back in)
    held = (q_d, k_d, v_d, lse, patt, alpha if need_dec else None,
            rho if need_dec else None, z if need_dec else None)

    def bwd(dout, out_saved):
        """dq, dk (compact, contiguous; zero for slots no live head uses) and
        dv (contiguous) through saf_mixed_attn_bwd."""
        if kvidx is not None:
            raise NotImplementedError(
                "fused_mixed_attn backward with kvidx (GQA) is not implemented "
                "(as in qwen/kernel/fused_attn.py:605-609 of the reference)")
        if bool((frozen_h == 2).any()) and alpha is None:
            raise ValueError("the backward of decomposed heads needs alpha/rho/z")
        do = dout.contiguous()
        dq = torch.zeros(q_d.shape, device=v.device, dtype=v.dtype) if n_live else None
        dk = torch.zeros(k_d.shape, device=v.device, dtype=v.dtype) if n_live else None
        dv = torch.empty(v_d.shape, device=v.device, dtype=v.dtype)
        bws = int(L.saf_mixed_attn_bwd_workspace_bytes(args))
        if bws < 0:
            bws = 0
        bw = torch.empty(max(bws, 1), dtype=torch.uint8, device=v.device)
        bargs = _ext.SafMixedAttnArgs.from_buffer_copy(args)
        bargs.workspace = bw.data_ptr()
        bargs.workspace_bytes = bws
        cur = torch.cuda.current_stream(v.device)
        _ext.check(L.saf_mixed_attn_bwd(bargs, _ext.tensor_desc(do), _ext.tensor_desc(dq),
                                        _ext.tensor_desc(dk), _ext.tensor_desc(dv), cur.cuda_stream))
        _ = (keep, held, out_saved)  # what the argument block points to
        gq = dq.to(q.dtype) if dq is not None and q is not None else None
        gk = dk.to(k.dtype) if dk is not None and k is not None else None
        return gq, gk, dv

    if needs_grad:
        return _MixedAttnFn.apply(q, k, v, run, bwd)
    return run()


def _validate(q, k, v, patt, frozen, hidx, pidx, alpha, rho, z, rho_band, kvidx):
    """The reference's argument checks (kernel/fused_attn.py:695-732 and
    qwen/kernel/fused_attn.py:720-731), same messages."""
    assert q.ndim == k.ndim == v.ndim == 4, "q, k, v must be 4-D"
    B, HV, T, HD = v.shape
    H = frozen.numel()
    if kvidx is None:
        assert HV == H, "v must hold one head per output head (or pass kvidx)"
        assert q.shape == k.shape, "q and k must have the same compact shape"
    else:
        assert k.shape == v.shape, "with kvidx, k and v are the raw (B, HKV, T, HD) heads"
        assert kvidx.shape == (H,) and kvidx.dtype == torch.int32 \
            and kvidx.device == v.device, "kvidx must be (H,) int32 on v.device"
        assert int(kvidx.max()) < HV and int(kvidx.min()) >= 0, \
            "kvidx must index the HKV heads of k/v"
    assert q.shape[0] == B and q.shape[2:] == (T, HD), \
        "q/k batch, sequence, and head dimensions must match v"
    hidx_t = hidx if hidx is not None else frozen
    pidx_t = pidx if pidx is not None else frozen
    assert frozen.shape == hidx_t.shape == pidx_t.shape == (H,), \
        "frozen, hidx, and pidx must have one entry per output head"
    assert frozen.dtype == hidx_t.dtype == pidx_t.dtype == torch.int32, \
        "frozen, hidx, and pidx must be int32"
    assert frozen.device == hidx_t.device == pidx_t.device == v.device, \
        "head-state and index tensors must be on v.device"
    assert q.device == k.device == v.device, "q, k, v must share a device"
    if patt is not None:
        assert patt.ndim == 3 and patt.shape[1] >= T and patt.shape[2] >= T, \
            "patt must have shape (P, S, S) with S >= T"
        assert patt.device == v.device, "patt must be on v.device"
        if pidx is None:
            assert patt.shape[0] >= H, \
                "identity pattern mapping requires at least H pattern rows"
        elif bool((frozen == 1).any()):
            dense_pidx = pidx[frozen == 1]
            assert int(dense_pidx.min()) >= 0 and \
                int(dense_pidx.max()) < patt.shape[0], \
                "pidx for dense-frozen heads must index patt"
    else:
        assert not bool((frozen == 1).any()), "dense-frozen heads require patt"
    if alpha is not None:
        assert rho is not None and alpha.shape == rho.shape == z.shape, \
            "alpha, rho, and z must have matching (H, S) shapes"
        assert alpha.shape[0] == H and alpha.shape[1] >= T, \
            "decomposed buffers must have shape (H, S) with S >= T"
        assert alpha.device == rho.device == z.device == v.device, \
            "decomposed buffers must be on v.device"
        if rho_band is not None:
            assert rho_band.shape == (H, BAND_ROWS, alpha.size(1)), \
                "rho_band must be make_rho_band(rho) with matching block size"
    else:
        assert not bool((frozen == 2).any()), \
            "decomposed-frozen heads require alpha/rho/z"
