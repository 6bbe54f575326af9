"""Indexed projections: Q/K columns only for live heads, head-order fix-ups.

Entry points of /root/reference/kernel/indexed_linear.py:125-141 (same names,
arguments and results):

    linear_rows(x, weight, bias, rows)          x @ weight[rows]^T + bias[rows]
    linear_rows2(x, w1, w2, b1, b2, rows)       [x @ w1[rows]^T, x @ w2[rows]^T]
                                                (+ the biases) in one GEMM
    linear_permuted_cols(y, weight, bias, cols) y @ weight[:, cols]^T + bias

All three are one operator here, ``_GatheredLinear``: n weights gathered by
one shared index along one axis (0 = output rows, 1 = input columns), stacked
along the output features and applied as a single library GEMM (hipBLASLt
through torch).  The gathered weight is built once in the forward and kept
for the backward, which is then two GEMMs over all n weights at once
(dX = dY . W_g and dW_g = dY^T . X) plus one gather per weight that maps dW_g
back onto the full weight: through the inverse permutation for columns, and
for rows through an inverse row map whose unselected rows point at an
appended zero row, so unselected rows get exactly zero gradient without a
zero fill followed by a scatter.  Indices must be unique (head slices, or a
full permutation for columns), as in every caller of the reference.
"""
import torch
import torch.nn.functional as F


def _compute_args(x, tensors):
    """Under autocast, the activation and every weight/bias in the autocast
    dtype (what the reference's projections compute in); else unchanged."""
    dev = x.device.type
    if not torch.is_autocast_enabled(dev):
        return x, tensors
    dt = torch.get_autocast_dtype(dev)
    return x.to(dt), [None if t is None else t.to(dt) for t in tensors]


def _row_map(index, n_rows):
    """inv[r] = position of row r in `index`, or len(index) (the zero row)."""
    inv = torch.full((n_rows,), index.numel(), dtype=torch.long, device=index.device)
    inv[index] = torch.arange(index.numel(), device=index.device)
    return inv


class _GatheredLinear(torch.autograd.Function):
    """Y = X . cat_i(G(W_i))^T + cat_i(G(b_i)), G = gather by `index` along
    `axis` (biases are gathered only for axis 0; for axis 1 there is one
    weight and its bias is used as is)."""

    @staticmethod
    def forward(ctx, x, index, axis, n, *params):
        ws, bs = params[:n], params[n:]
        if axis == 0:
            wg = torch.cat([w.index_select(0, index) for w in ws]) if n > 1 else ws[0].index_select(0, index)
            bg = None
            if bs[0] is not None:
                bg = torch.cat([b.index_select(0, index) for b in bs]) if n > 1 else bs[0].index_select(0, index)
            inv = _row_map(index, ws[0].size(0))
        else:
            wg = ws[0].index_select(1, index)
            bg = bs[0]
            inv = torch.argsort(index)
        ctx.axis, ctx.n = axis, n
        ctx.shapes = [w.shape for w in ws]
        ctx.has_bias = bs[0] is not None
        ctx.save_for_backward(x, wg, inv)
        return F.linear(x, wg, bg)

    @staticmethod
    def backward(ctx, gy):
        x, wg, inv = ctx.saved_tensors
        axis, n = ctx.axis, ctx.n
        g2 = gy.reshape(-1, gy.size(-1))
        need_x = ctx.needs_input_grad[0]
        need_w = any(ctx.needs_input_grad[4:4 + n])
        need_b = ctx.has_bias and any(ctx.needs_input_grad[4 + n:])
        dx = (g2 @ wg).view(x.shape) if need_x else None
        dws = [None] * n
        dbs = [None] * n
        if need_w:
            dwg = g2.t() @ x.reshape(-1, x.size(-1))
            if axis == 0:
                R = dwg.size(0) // n
                zero = dwg.new_zeros(1, dwg.size(1))
                dws = [torch.cat([dwg[i * R:(i + 1) * R], zero]).index_select(0, inv) for i in range(n)]
            else:
                dws = [dwg.index_select(1, inv)]
        if need_b:
            dbg = g2.sum(0)
            if axis == 0:
                R = dbg.numel() // n
                zero = dbg.new_zeros(1)
                dbs = [torch.cat([dbg[i * R:(i + 1) * R], zero]).index_select(0, inv) for i in range(n)]
            else:
                dbs = [dbg]
        return (dx, None, None, None, *dws, *dbs)


def linear_rows(x, weight, bias, rows):
    """F.linear(x, weight[rows], bias[rows]) for unique ``rows``; weight and
    bias rows outside ``rows`` get zero gradient."""
    x, (weight, bias) = _compute_args(x, [weight, bias])
    return _GatheredLinear.apply(x, rows, 0, 1, weight, bias)


def linear_rows2(x, w1, w2, b1, b2, rows):
    """(..., 2R) = [x @ w1[rows]^T + b1[rows], x @ w2[rows]^T + b2[rows]] as
    one GEMM (the live heads' Q and K projections)."""
    x, (w1, w2, b1, b2) = _compute_args(x, [w1, w2, b1, b2])
    return _GatheredLinear.apply(x, rows, 0, 2, w1, w2, b1, b2)


def linear_permuted_cols(y, weight, bias, cols):
    """F.linear(y, weight[:, cols], bias) for a full column permutation
    ``cols`` (c_proj applied to heads in [live..., frozen...] order)."""
    y, (weight, bias) = _compute_args(y, [weight, bias])
    return _GatheredLinear.apply(y, cols, 1, 1, weight, bias)
