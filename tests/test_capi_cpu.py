"""C-ABI checks that need no GPU: libsafattn.so loads, exports every entry
point declared in include/saf_attn.h, and rejects invalid arguments with a
status and message before any device work is enqueued."""
import ctypes
import os
import re

import pytest
import torch

from kernel import _ext

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "saf_attn.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(saf_[a-z_0-9]+)\s*\(", text)))


def test_library_loads_and_exports_header_symbols():
    L = _ext.lib()
    declared = _declared()
    assert declared, "no declarations found"
    for name in declared:
        assert hasattr(L, name), f"{name} declared in saf_attn.h but not exported"
    assert set(declared) == set(_ext.EXPORTS)
    assert L.saf_version().startswith(b"saf-mi355x")


def test_workspace_bytes():
    L = _ext.lib()
    assert L.saf_workspace_bytes(8, 16384, 64, 0) == 0
    # 256-byte header (error word) + one 8-byte status word per (sequence,
    # 256-row chunk, column) at hd 64
    n = L.saf_workspace_bytes(8, 16384, 64, 12)
    nseq, nch = 8 * 12, 16384 // 256
    assert n == 256 + 8 * nseq * nch * 64
    assert L.saf_workspace_bytes(1, 1000, 128, 1) == 256 + 8 * 8 * 128   # 128-row chunks at hd 128
    assert L.saf_workspace_bytes(1, 1000, 80, 3) == 0   # unsupported head dim


def _args(H=4, T=64, hd=64, dtype=_ext.SAF_BF16, frozen=None, ptr=0x100000):
    a = _ext.SafMixedAttnArgs()

    def t4(shape):
        d = _ext.SafTensor()
        d.data, d.dtype, d.ndim = ptr, dtype, 4
        st = [shape[1] * shape[2] * shape[3], shape[2] * shape[3], shape[3], 1]
        for i in range(4):
            d.size[i], d.stride[i] = shape[i], st[i]
        return d

    a.q = t4((1, H, T, hd))
    a.k = t4((1, H, T, hd))
    a.v = t4((1, H, T, hd))
    a.out = t4((1, H, T, hd))
    a.n_heads = H
    fz = frozen if frozen is not None else [0] * H
    a._keep = (ctypes.c_int32 * H)(*fz)
    a.frozen = a._keep
    a.sm_scale = 0.125
    return a


@pytest.mark.parametrize("mutate,code,msg", [
    (lambda a: setattr(a, "n_heads", 0), _ext.SAF_EUNSUPPORTED, "n_heads"),
    (lambda a: setattr(a.v, "dtype", _ext.SAF_I32), _ext.SAF_EUNSUPPORTED, "int32"),
    (lambda a: setattr(a.v, "dtype", _ext.SAF_F32), _ext.SAF_EINVAL, "dtype must match"),
    (lambda a: a.v.size.__setitem__(3, 80), _ext.SAF_EUNSUPPORTED, "head_dim"),
    (lambda a: a.out.size.__setitem__(2, 63), _ext.SAF_EINVAL, "out must have shape"),
    (lambda a: a.v.stride.__setitem__(3, 2), _ext.SAF_EALIGN, "contiguous last"),
    (lambda a: setattr(a.v, "data", 0x100002), _ext.SAF_EALIGN, "aligned"),
    (lambda a: a._keep.__setitem__(0, 5), _ext.SAF_EINVAL, "head state"),
    (lambda a: a._keep.__setitem__(0, 1), _ext.SAF_EINVAL, "require patt"),
    (lambda a: setattr(a, "frozen", None), _ext.SAF_EINVAL, "frozen"),
])
def test_invalid_arguments_rejected_without_launch(mutate, code, msg):
    L = _ext.lib()
    a = _args()
    mutate(a)
    rc = L.saf_mixed_attn_fwd(ctypes.byref(a), None)
    assert rc == code
    assert msg in L.saf_last_error().decode()


def test_closed_form_needs_workspace():
    L = _ext.lib()
    a = _args(frozen=[0, 2, 0, 0])
    kinds = (ctypes.c_int32 * 4)(0, 1, 0, 0)
    prm = (ctypes.c_float * 4)(0, 0, 0, 0)
    a.closed_kind, a.closed_param = kinds, prm
    rc = L.saf_mixed_attn_fwd(ctypes.byref(a), None)
    assert rc == _ext.SAF_EWORKSPACE
    kinds[1] = 2
    prm[1] = -1.0
    assert L.saf_mixed_attn_fwd(ctypes.byref(a), None) == _ext.SAF_EINVAL
    assert "decay rate" in L.saf_last_error().decode()


def test_cpu_tensors_fail_loudly():
    import kernel
    q = torch.zeros(1, 1, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        kernel.fused_mixed_attn(q, q, q, None, torch.zeros(1, dtype=torch.int32))
    with pytest.raises(RuntimeError, match="HIP devices only"):
        kernel.frozen_pv(torch.zeros(1, 4, 4), q, torch.zeros(1, dtype=torch.int32), 4)


def test_host_table_cached_per_tensor_and_version():
    """The routing tables are planned on the host: the copy is made once per
    tensor and refreshed only when the tensor changes in place, so callers
    that keep their tables (as the reference's models keep buffers) pay no
    device-to-host copy per call."""
    from kernel import fused_attn as F
    t = torch.tensor([0, 2, 1, 0], dtype=torch.int32)
    a = F._host_table(t)
    assert a.tolist() == [0, 2, 1, 0]
    assert F._host_table(t) is a                      # cached on the tensor
    t[1] = 1                                          # in-place change: version moves
    b = F._host_table(t)
    assert b.tolist() == [0, 1, 1, 0]
    assert F._host_table(t.clone()) is not b          # another tensor: its own copy
    assert F._host_table(None) is None
    assert F._host_table([1, 2]).tolist() == [1, 2]
