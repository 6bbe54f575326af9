"""Projection GEMMs of the GPT block with their elementwise follow-ups fused
into one HIP kernel each (libsafattn.so, forward only, no bias).

* ``linear_gelu`` (``saf_linear_gelu``): the MLP's ``gelu(c_fc(x))``
  (/root/reference/nanogpt/model.py:1193-1207, ``nn.GELU()``: the exact,
  erf-based GELU).  The reference's up-projection writes its (rows, 4 C)
  output and the activation reads and writes it again; here the GELU runs on
  the GEMM's fp32 accumulator and the activation is written once, rounded once.
* ``gelu_`` (``saf_gelu_inplace``): the same GELU evaluation in place on a
  GEMM output, for MLPs whose up-projection stays a library GEMM.
* ``linear_swiglu`` (``saf_linear_swiglu``): ``act_fn(gate_proj(x)) *
  up_proj(x)`` of transformers' Qwen3MLP (SiLU), the MLP of the Qwen caller,
  from one GEMM over the gate and up rows interleaved in blocks of 64
  (``swiglu_weight``); the two (rows, I) products never reach memory.
* ``linear_rope`` (``saf_linear_rope``): the indexed QKV projection of the
  gathered ``[Wq[live]; Wk[live]; Wv]`` weight (nanogpt/model.py:920-944) with
  the rotary embedding of the live q and k (:57-99, :1007-1008) applied to the
  accumulator, instead of a GEMM followed by a pass over q and k.
"""
import torch

from . import _ext

# Shapes the kernels take: N (output features) a multiple of 256, K (input
# features) a multiple of 128.
_N_MULT, _K_MULT = 256, 128


def _gemm_usable(x, weight):
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and weight.dtype == x.dtype
            and weight.dim() == 2 and x.size(-1) == weight.size(1)
            and weight.size(0) % _N_MULT == 0 and weight.size(1) % _K_MULT == 0)


def _rows(x, weight):
    K = x.size(-1)
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w = weight.detach()
    if w.stride(-1) != 1:
        w = w.contiguous()
    return x2, w


def linear_gelu_usable(x, weight):
    """True when linear_gelu runs x (..., K) against weight (N, K)."""
    return _gemm_usable(x, weight)


def gelu_usable(x):
    """True when gelu_ runs on x in place."""
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float16) and x.is_contiguous()
            and x.numel() % 8 == 0 and x.data_ptr() % 16 == 0)


def gelu_(x):
    """Exact GELU of x in place (``saf_gelu_inplace``, the fused kernel's
    evaluation); returns x."""
    if not x.is_cuda:
        raise RuntimeError("gelu_ runs on HIP devices only (got a CPU tensor)")
    if x.numel() == 0:
        return x
    L = _ext.lib()
    _ext.check(L.saf_gelu_inplace(_ext.tensor_desc(x.view(-1)), _ext.current_stream_ptr(x.device)))
    return x


def linear_gelu(x, weight):
    """gelu(x @ weight.T) for x (..., K) and weight (N, K); returns (..., N)."""
    if not x.is_cuda:
        raise RuntimeError("linear_gelu runs on HIP devices only (got a CPU tensor)")
    x2, w = _rows(x, weight)
    out = torch.empty(x2.size(0), w.size(0), device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out.view(*x.shape[:-1], w.size(0))
    L = _ext.lib()
    rc = L.saf_linear_gelu(_ext.tensor_desc(x2), _ext.tensor_desc(w), _ext.tensor_desc(out),
                           _ext.current_stream_ptr(x.device))
    _ext.check(rc)
    return out.view(*x.shape[:-1], w.size(0))


SWIGLU_BLOCK = 64  # rows per gate / up block of the interleaved weight


def swiglu_weight(w_gate, w_up):
    """(2 I, K) weight of linear_swiglu from the gate and up projections'
    (I, K) weights: 64-row blocks of gate rows and up rows in turn."""
    I, K = w_gate.shape
    if w_up.shape != (I, K) or I % SWIGLU_BLOCK:
        raise ValueError("gate and up weights must share a shape (I, K) with I a multiple of 64")
    nb = I // SWIGLU_BLOCK
    return torch.stack([w_gate.reshape(nb, SWIGLU_BLOCK, K), w_up.reshape(nb, SWIGLU_BLOCK, K)], 1).reshape(2 * I, K)


def linear_swiglu_usable(x, weight):
    """True when linear_swiglu runs x (..., K) against the interleaved (2 I, K) weight."""
    return _gemm_usable(x, weight)


def linear_swiglu(x, weight):
    """silu(x @ Wg.T) * (x @ Wu.T) for x (..., K) and the interleaved weight
    of swiglu_weight(Wg, Wu); returns (..., I)."""
    if not x.is_cuda:
        raise RuntimeError("linear_swiglu runs on HIP devices only (got a CPU tensor)")
    x2, w = _rows(x, weight)
    out = torch.empty(x2.size(0), w.size(0) // 2, device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out.view(*x.shape[:-1], w.size(0) // 2)
    L = _ext.lib()
    rc = L.saf_linear_swiglu(_ext.tensor_desc(x2), _ext.tensor_desc(w), _ext.tensor_desc(out),
                             _ext.current_stream_ptr(x.device))
    _ext.check(rc)
    return out.view(*x.shape[:-1], w.size(0) // 2)


def linear_rope_usable(x, weight, n_rope, head_dim, cos):
    """True when linear_rope runs x (B, T, K) against weight (N, K) with the
    first n_rope output columns rotated (heads of head_dim) by the cos cache."""
    return (_gemm_usable(x, weight) and x.dim() == 3 and head_dim in (64, 128)
            and n_rope % 128 == 0 and 0 <= n_rope <= weight.size(0)
            and cos.dtype == x.dtype and cos.size(-1) >= head_dim)


def linear_rope(x, weight, n_rope, head_dim, cos, sin):
    """x (B, T, K) @ weight.T with the first n_rope columns rotated at each
    row's position t by the Llama half rotation (cos / sin: (T', head_dim)
    caches, any leading singleton dims); returns (B, T, N)."""
    if not x.is_cuda:
        raise RuntimeError("linear_rope runs on HIP devices only (got a CPU tensor)")
    if x.dim() != 3:
        raise ValueError("linear_rope takes x as (B, T, K)")
    T = x.size(1)
    x2, w = _rows(x, weight)
    out = torch.empty(x2.size(0), w.size(0), device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out.view(x.size(0), T, w.size(0))
    cos2 = cos.reshape(-1, cos.size(-1))
    sin2 = sin.reshape(-1, sin.size(-1))
    L = _ext.lib()
    rc = L.saf_linear_rope(_ext.tensor_desc(x2), _ext.tensor_desc(w), _ext.tensor_desc(out), int(n_rope),
                           int(head_dim), int(T), _ext.tensor_desc(cos2), _ext.tensor_desc(sin2),
                           _ext.current_stream_ptr(x.device))
    _ext.check(rc)
    return out.view(x.size(0), T, w.size(0))
