"""Row normalisers and parameter gradients of decomposed patterns on HIP.

Restates /root/reference/supplement/trainable_pattern_kernels.py over
libsafattn.so:
  normalisers      (:8-17, :59-63)  z[h, i] = logsumexp_{j <= i, j < length}
                   (alpha[h, j] + rho[h, i - j]) for rows i < length, zero
                   beyond; saf_decomposed_logz over the first `length` columns.
  PatternGradient  (:66-85)  an identity on the attention output whose
                   backward adds dalpha / drho of every decomposed head (state
                   2): with P = exp(alpha_j + rho_{i-j} - z_i), dP = dO V^T and
                   delta_i = dO_i . O_i, dS = P (dP - delta); dalpha_j sums dS
                   over rows, drho_d over the diagonal i - j = d, summed over
                   the batch.  saf_decomp_param_bwd does it in one MFMA pass
                   per (batch, head, key block): dS never reaches HBM, diagonal
                   sums go through an LDS ring before their global atomics.
The gradient that reaches the output passes through unchanged (V and Q/K get
theirs from the attention operator's own backward)."""
import numpy as np
import torch

import kernel._ext as _ext
from kernel.fused_attn import _host_table, decomposed_logz


@torch.no_grad()
def normalisers(alpha, rho, length):
    """(H, S) float32 log-normalisers of rows < length (zero beyond)."""
    if not alpha.is_cuda:
        raise RuntimeError("normalisers run on HIP devices only (got a CPU tensor)")
    length = int(length)
    H, S = alpha.shape
    if not 0 <= length <= S:
        raise ValueError(f"length {length} outside 0..{S}")
    z = torch.zeros(H, S, device=alpha.device, dtype=torch.float32)
    if length:
        z[:, :length] = decomposed_logz(alpha[:, :length].float().contiguous(),
                                        rho[:, :length].float().contiguous())
    return z


def pattern_gradients(out, value, alpha, rho, z, states, grad):
    """dalpha, drho (float32, alpha's / rho's shape) of sum(grad * out) over
    the decomposed heads of `states` (H,) with out = P V.  value / out / grad:
    (B, H, T, HD) bf16 or fp16 (any strides with a unit feature stride);
    alpha, rho, z: (H, S) with S >= T."""
    if not value.is_cuda:
        raise RuntimeError("pattern_gradients runs on HIP devices only (got a CPU tensor)")
    st = _host_table(states) if torch.is_tensor(states) else np.asarray(states, dtype=np.int32)
    da = torch.zeros(alpha.shape, device=value.device, dtype=torch.float32)
    dr = torch.zeros(rho.shape, device=value.device, dtype=torch.float32)
    if not (st == 2).any():
        return da, dr
    L = _ext.lib()
    a, r, zz = (t.detach() for t in (alpha, rho, z))
    a, r, zz = (t if t.stride(-1) == 1 else t.contiguous() for t in (a, r, zz))
    go = grad if grad.stride(-1) == 1 else grad.contiguous()
    args = _ext.SafMixedAttnArgs()
    args.v = _ext.tensor_desc(value)
    args.out = _ext.tensor_desc(out)
    args.alpha = _ext.tensor_desc(a)
    args.rho = _ext.tensor_desc(r)
    args.z = _ext.tensor_desc(zz)
    args.n_heads = int(st.size)
    frozen = _ext.host_i32(st)
    args.frozen = frozen
    need = int(L.saf_decomp_param_bwd_workspace_bytes(args))
    if need < 0:
        _ext.check(L.saf_decomp_param_bwd(args, _ext.tensor_desc(go), _ext.tensor_desc(da),
                                          _ext.tensor_desc(dr), None))  # raises with the message
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=value.device)
    args.workspace = ws.data_ptr()
    args.workspace_bytes = need
    _ext.check(L.saf_decomp_param_bwd(args, _ext.tensor_desc(go), _ext.tensor_desc(da),
                                      _ext.tensor_desc(dr), _ext.current_stream_ptr(value.device)))
    return da, dr


class PatternGradient(torch.autograd.Function):
    """out -> out, with dalpha / drho of the decomposed heads in the backward."""

    @staticmethod
    def forward(ctx, out, value, alpha, rho, z, states):
        ctx.save_for_backward(out, value, alpha, rho, z)
        # host copy of the head states: cached per table version, so no
        # device-to-host copy drains the stream per call
        ctx.states = _host_table(states) if torch.is_tensor(states) else np.asarray(states, dtype=np.int32)
        return out

    @staticmethod
    def backward(ctx, grad):
        out, value, alpha, rho, z = ctx.saved_tensors
        da, dr = pattern_gradients(out, value, alpha, rho, z, ctx.states, grad)
        return grad, None, da.to(alpha.dtype), dr.to(rho.dtype), None, None
