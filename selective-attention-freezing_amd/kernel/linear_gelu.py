"""MLP up-projection and GELU of the GPT block, fused into one HIP GEMM.

The reference's MLP runs ``c_proj(gelu(c_fc(x)))`` with ``nn.GELU()`` (the
exact, erf-based GELU) (/root/reference/nanogpt/model.py:1193-1207): the
up-projection writes its (rows, 4 C) output, and the activation reads and
writes it again.  ``linear_gelu`` (libsafattn.so ``saf_linear_gelu``) applies
the GELU to the GEMM's fp32 accumulator in the kernel's epilogue and writes
the activation once, rounded once.  Forward only, no bias.
"""
import torch

from . import _ext

# Shapes the kernel takes: N (output features) a multiple of 256, K (input
# features) a multiple of 128.
_N_MULT, _K_MULT = 256, 128


def linear_gelu_usable(x, weight):
    """True when linear_gelu runs x (..., K) against weight (N, K)."""
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
            and weight.dim() == 2 and x.size(-1) == weight.size(1)
            and weight.size(0) % _N_MULT == 0 and weight.size(1) % _K_MULT == 0)


def linear_gelu(x, weight):
    """gelu(x @ weight.T) for x (..., K) and weight (N, K); returns (..., N)."""
    if not x.is_cuda:
        raise RuntimeError("linear_gelu runs on HIP devices only (got a CPU tensor)")
    K = x.size(-1)
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = weight.detach()
    if w.stride(-1) != 1:
        w = w.contiguous()
    out = torch.empty(x2.size(0), w.size(0), device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out.view(*x.shape[:-1], w.size(0))
    L = _ext.lib()
    rc = L.saf_linear_gelu(_ext.tensor_desc(x2), _ext.tensor_desc(w), _ext.tensor_desc(out),
                           _ext.current_stream_ptr(x.device))
    _ext.check(rc)
    return out.view(*x.shape[:-1], w.size(0))
