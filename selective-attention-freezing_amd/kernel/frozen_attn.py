"""Split-path frozen-head operator ``frozen_pv``: y = P[fz_idx[f], :T, :T] @ V.

Drop-in for /root/reference/kernel/frozen_attn.py:185-192.  V and the output
are COMPACT (B, nf, T, hd) tensors holding only the frozen heads; the pattern
buffer keeps its (n_head, S, S) layout and is indexed through ``fz_idx``.  The
product runs in libsafattn.so's dense P.V kernel (causal j-block skipping,
pattern rounded to V's dtype before the bf16/fp16 MFMA).  The backward,
dV = P^T dY (/root/reference/kernel/frozen_attn.py:91-128, :174-182), runs the
frozen-head dV kernel of the attention backward (saf_frozen_pv_bwd); rows of
V at or past T get zero gradient.
"""
import torch

from . import _ext
from .fused_attn import _aligned_view, _host_table, _row_aligned

HAVE_TRITON = False   # this build has no Triton; kept for import compatibility


def frozen_pv_usable(v):
    """True for tensors on a HIP device (no silent fallback once on the GPU)."""
    return bool(v.is_cuda)


class _FrozenPVFn(torch.autograd.Function):
    """v is the only differentiable input; patterns get no gradient."""

    @staticmethod
    def forward(ctx, v, run, bwd):
        ctx.bwd = bwd
        return run()

    @staticmethod
    def backward(ctx, dy):
        dv = ctx.bwd(dy)
        ctx.bwd = None
        return dv, None, None


def frozen_pv(patt, v, fz_idx, T):
    """y[b, f] = patt[fz_idx[f], :T, :T] @ v[b, f]  ->  (B, nf, T, hd)."""
    if not v.is_cuda:
        raise RuntimeError("frozen_pv runs on HIP devices only (got a CPU tensor)")
    B, nf, Tv, hd = v.shape
    fz = _host_table(fz_idx)
    v_d = _aligned_view(v, 16)
    out = torch.empty((B, nf, T, hd), device=v.device, dtype=v.dtype)
    L = _ext.lib()
    pd = _ext.tensor_desc(patt)
    vd = _ext.tensor_desc(v_d)
    od = _ext.tensor_desc(out)
    fz_c = _ext.host_i32(fz)

    def run():
        stream = _ext.current_stream_ptr(v.device)
        _ext.check(L.saf_frozen_pv_fwd(pd, vd, fz_c, nf, int(T), od, stream))
        return out

    def bwd(dy):
        """dv (v's shape, contiguous) = P^T dy over the first T rows."""
        dy_d = dy.to(v.dtype)
        if not _row_aligned(dy_d, 16):
            dy_d = dy_d.contiguous()
        make = torch.empty if Tv == T else torch.zeros
        dv = make((B, nf, Tv, hd), device=v.device, dtype=v.dtype)
        stream = _ext.current_stream_ptr(v.device)
        _ext.check(L.saf_frozen_pv_bwd(_ext.tensor_desc(patt), _ext.tensor_desc(dy_d), fz_c, nf, int(T),
                                       _ext.tensor_desc(dv), stream))
        return dv

    if torch.is_grad_enabled() and v.requires_grad:
        return _FrozenPVFn.apply(v, run, bwd)
    return run()
