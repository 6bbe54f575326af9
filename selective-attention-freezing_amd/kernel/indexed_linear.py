"""Projections over row-sliced / column-permuted weights.

Drop-in for /root/reference/kernel/indexed_linear.py:125-141: the indexed QKV
projection of the cheap frozen-head path emits Q/K columns only for live
heads.  Indices are unique (head slices or a full permutation), so the weight
gradient is scattered with ``index_copy_`` rather than autograd's atomic
``index_add``; unselected rows get exactly zero gradient.  These are plain
library GEMMs (hipBLASLt through torch) over gathered weights.
"""
import torch
import torch.nn.functional as F


def _cast_for_autocast(x, *ws):
    dev = x.device.type
    if torch.is_autocast_enabled(dev):
        dt = torch.get_autocast_dtype(dev)
        return (x.to(dt),) + tuple(None if w is None else w.to(dt) for w in ws)
    return (x,) + ws


def _flat(t):
    return t.reshape(-1, t.size(-1))


class _RowsLinear(torch.autograd.Function):
    """F.linear(x, weight[rows], bias[rows])."""

    @staticmethod
    def forward(ctx, x, weight, bias, rows):
        ctx.save_for_backward(x, weight, rows)
        ctx.has_bias = bias is not None
        b = None if bias is None else bias.index_select(0, rows)
        return F.linear(x, weight.index_select(0, rows), b)

    @staticmethod
    def backward(ctx, g):
        x, weight, rows = ctx.saved_tensors
        g2, x2 = _flat(g), _flat(x)
        dx = dw = db = None
        if ctx.needs_input_grad[0]:
            dx = (g2 @ weight.index_select(0, rows)).view(x.shape)
        if ctx.needs_input_grad[1]:
            dw = torch.zeros_like(weight).index_copy_(0, rows, g2.t() @ x2)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = torch.zeros(weight.size(0), device=g.device, dtype=g.dtype)
            db.index_copy_(0, rows, g2.sum(0))
        return dx, dw, db, None


class _PermutedColsLinear(torch.autograd.Function):
    """F.linear(y, weight[:, cols], bias) for a full column permutation."""

    @staticmethod
    def forward(ctx, y, weight, bias, cols):
        ctx.save_for_backward(y, weight, cols)
        ctx.has_bias = bias is not None
        return F.linear(y, weight.index_select(1, cols), bias)

    @staticmethod
    def backward(ctx, g):
        y, weight, cols = ctx.saved_tensors
        g2, y2 = _flat(g), _flat(y)
        dy = dw = db = None
        if ctx.needs_input_grad[0]:
            dy = (g2 @ weight.index_select(1, cols)).view(y.shape)
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(weight).index_copy_(1, cols, g2.t() @ y2)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            db = g2.sum(0)
        return dy, dw, db, None


class _TwoRowsLinear(torch.autograd.Function):
    """One GEMM producing [x @ w1[rows]^T, x @ w2[rows]^T] on the last dim."""

    @staticmethod
    def forward(ctx, x, w1, w2, b1, b2, rows):
        ctx.save_for_backward(x, w1, w2, rows)
        ctx.has_bias = b1 is not None
        w = torch.cat([w1.index_select(0, rows), w2.index_select(0, rows)])
        b = None if b1 is None else torch.cat([b1.index_select(0, rows),
                                               b2.index_select(0, rows)])
        return F.linear(x, w, b)

    @staticmethod
    def backward(ctx, g):
        x, w1, w2, rows = ctx.saved_tensors
        g2, x2 = _flat(g), _flat(x)
        R = g.size(-1) // 2
        dx = dw1 = dw2 = db1 = db2 = None
        if ctx.needs_input_grad[0]:
            w = torch.cat([w1.index_select(0, rows), w2.index_select(0, rows)])
            dx = (g2 @ w).view(x.shape)
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dw = g2.t() @ x2
            dw1 = torch.zeros_like(w1).index_copy_(0, rows, dw[:R])
            dw2 = torch.zeros_like(w2).index_copy_(0, rows, dw[R:])
        if ctx.has_bias and (ctx.needs_input_grad[3] or ctx.needs_input_grad[4]):
            db = g2.sum(0)
            db1 = torch.zeros(w1.size(0), device=g.device, dtype=g.dtype).index_copy_(0, rows, db[:R])
            db2 = torch.zeros(w2.size(0), device=g.device, dtype=g.dtype).index_copy_(0, rows, db[R:])
        return dx, dw1, dw2, db1, db2, None


def linear_rows(x, weight, bias, rows):
    """Linear over the unique rows ``rows`` of ``weight``."""
    x, weight, bias = _cast_for_autocast(x, weight, bias)
    return _RowsLinear.apply(x, weight, bias, rows)


def linear_rows2(x, w1, w2, b1, b2, rows):
    """Fused two-weight row-sliced linear -> (..., 2R)."""
    x, w1, w2, b1, b2 = _cast_for_autocast(x, w1, w2, b1, b2)
    return _TwoRowsLinear.apply(x, w1, w2, b1, b2, rows)


def linear_permuted_cols(y, weight, bias, cols):
    """Linear over a column-permuted ``weight`` (head-order fix-up)."""
    y, weight, bias = _cast_for_autocast(y, weight, bias)
    return _PermutedColsLinear.apply(y, weight, bias, cols)
