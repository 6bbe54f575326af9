"""The allocation-free forward (saf_mixed_attn_fwd_noalloc) against the
workspace forward (saf_mixed_attn_fwd), both called through the C-ABI.

Two calls in a row on the library's one scratch array, the second with a
smaller input, each compared with the workspace entry point's output on the
same arguments (max-abs <= 2e-2, relative-L2 <= 1e-2: the same kernels run,
and only the closed-form scan's look-back order can move a last bit) and with
the float64 oracle.  Every head kind is present (live at hd 128, which uses
the work-queue word and the split partials, dense, decomposed, closed-form
scan).  A call whose scan needs more than the scratch's maximum is refused
before anything is launched.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import saf_oracle as orc
from saf_cases import closed_params, compare, f64, make_decomp, make_pattern, qkv, routing, scale_of

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ext():
    from kernel import _ext
    return _ext


def _args(E, q, k, v, out, patt, frozen, hidx, alpha, rho, z, ck, cp, hd):
    a = E.SafMixedAttnArgs()
    a.q, a.k, a.v, a.out = E.tensor_desc(q), E.tensor_desc(k), E.tensor_desc(v), E.tensor_desc(out)
    a.patt = E.tensor_desc(patt)
    a.alpha, a.rho, a.z = E.tensor_desc(alpha), E.tensor_desc(rho), E.tensor_desc(z)
    a.n_heads = frozen.numel()
    keep = [E.host_i32(frozen.tolist()), E.host_i32(hidx.tolist()), E.host_i32(ck), E.host_f32(cp)]
    a.frozen, a.hidx, a.closed_kind, a.closed_param = keep
    a.sm_scale = scale_of(hd)
    return a, keep


def _case(B, H, T, hd, S, seed):
    """One mixed call: head 0 dense, 1 decomposed, 2 closed-form decay,
    3 closed-form window (when H > 4), the rest live."""
    import kernel
    E = _ext()
    L = E.lib()
    states = {0: 1, 1: 2, 2: 2}
    closed = {2: ("decay", 0.02)}
    if H > 4:
        states[3] = 2
        closed[3] = ("window", 100)
    frozen, hidx, live = routing(H, states)
    q, k, v = qkv(B, H, T, hd, seed=seed, dtype=torch.bfloat16)
    patt = make_pattern(H, S, seed=seed)
    alpha, rho, z = make_decomp(H, S, seed=seed)
    ca, cr, cz = closed_params(H, S, closed)
    for h in closed:
        alpha[h], rho[h], z[h] = ca[h], cr[h], cz[h]
    ck, cp = kernel.classify_closed_form(alpha, rho, z)
    assert all(ck[h] != 0 for h in closed) and ck[1] == 0
    qd, kd, vd = q[:, live].to(DEV), k[:, live].to(DEV), v.to(DEV)
    pd, ad, rd, zd = patt.to(DEV), alpha.to(DEV), rho.to(DEV), z.to(DEV)
    stream = torch.cuda.current_stream().cuda_stream

    out_ref = torch.empty(B, H, T, hd, device=DEV, dtype=torch.bfloat16)
    a, keep = _args(E, qd, kd, vd, out_ref, pd, frozen, hidx, ad, rd, zd, ck, cp, hd)
    nbytes = int(L.saf_mixed_attn_workspace_bytes(ctypes.byref(a)))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    E.check(L.saf_mixed_attn_fwd(ctypes.byref(a), stream))

    out_na = torch.empty_like(out_ref)
    b, keep2 = _args(E, qd, kd, vd, out_na, pd, frozen, hidx, ad, rd, zd, ck, cp, hd)
    E.check(L.saf_mixed_attn_fwd_noalloc(ctypes.byref(b), stream))
    torch.cuda.synchronize()
    _ = (keep, keep2)

    compare(out_na, f64(out_ref), what=f"noalloc vs workspace B{B} H{H} T{T} hd{hd}")
    ref = orc.eager_mixed_attention(f64(q[:, live]), f64(k[:, live]), f64(v), frozen.numpy(), hidx.numpy(),
                                    patt=patt.numpy(), alpha=f64(alpha), rho=f64(rho), z=f64(z),
                                    sm_scale=scale_of(hd))
    compare(out_na, ref, what=f"noalloc vs oracle B{B} H{H} T{T} hd{hd}")


def test_noalloc_matches_workspace_entry_two_calls():
    _case(2, 6, 1000, 128, 1024, seed=5)   # queue word, split partials, scan, dense, decomposed
    _case(1, 4, 300, 128, 512, seed=6)     # smaller: the scratch keeps the first call's contents


def test_noalloc_matches_workspace_entry_hd64():
    _case(2, 6, 2048, 64, 2048, seed=7)
    _case(1, 5, 129, 64, 192, seed=8)


def test_noalloc_refuses_oversized_scan():
    """B * n_scan * T large enough that the scan's look-back words exceed the
    scratch (2 x 128 closed-form heads at hd 256, T = 16384: 64 MiB of words
    plus the 256-byte header): refused with SAF_EWORKSPACE before any launch.
    v and out are real tensors of that shape (2.1 GB each), so even a
    regressed size check would run in bounds of them."""
    E = _ext()
    L = E.lib()
    B, H, T, hd = 2, 128, 16384, 256
    need = 256 + 8 * B * H * (T // 128) * hd
    assert need > (64 << 20)
    v = torch.zeros(B, H, T, hd, dtype=torch.bfloat16, device=DEV)
    out = torch.empty_like(v)
    a = E.SafMixedAttnArgs()
    a.v = E.tensor_desc(v)
    a.out = E.tensor_desc(out)
    a.n_heads = H
    keep = [E.host_i32([2] * H), E.host_i32([1] * H), E.host_f32([0.0] * H)]
    a.frozen, a.closed_kind, a.closed_param = keep
    a.sm_scale = 0.0625
    assert L.saf_mixed_attn_workspace_bytes(ctypes.byref(a)) >= need
    rc = L.saf_mixed_attn_fwd_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream)
    assert rc == E.SAF_EWORKSPACE
    assert b"maximum" in L.saf_last_error()
    torch.cuda.synchronize()
