"""Parameter gathers with deterministic backward.

The macro operators and the banked core read per-sample / per-recipe slices of
parameters (rte/macro.py:208-212, rte/layers.py:725-778).  Autograd of advanced
indexing scatters those gradients with a sort-based index_put; here the gradient
of a gather is a one-hot matrix product in fp32 instead: one GEMM, run-to-run
deterministic, no atomics."""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _acc_dtype(g: torch.Tensor) -> torch.dtype:
    return torch.float64 if g.dtype == torch.float64 else torch.float32


class _GatherRows(torch.autograd.Function):
    @staticmethod
    def forward(ctx, table: torch.Tensor, idx: torch.Tensor):
        flat = table.reshape(table.shape[0], -1)
        ctx.save_for_backward(idx)
        ctx.shape = table.shape
        return flat.index_select(0, idx).view(idx.shape[0], *table.shape[1:])

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        (idx,) = ctx.saved_tensors
        rows = ctx.shape[0]
        dt = _acc_dtype(g)
        onehot = F.one_hot(idx, rows).to(dt)  # [n, rows]
        grad = onehot.t() @ g.reshape(idx.shape[0], -1).to(dt)
        return grad.view(ctx.shape), None


def gather_rows(table: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """table[idx] along dim 0 (idx: 1-D long)."""
    return _GatherRows.apply(table, idx.long())


def gather_rk(table: torch.Tensor, recipe_ids: torch.Tensor, stride_ids: torch.Tensor) -> torch.Tensor:
    """table[recipe_ids, stride_ids] for a [r, k, ...] parameter."""
    r, k = table.shape[0], table.shape[1]
    flat = table.reshape(r * k, *table.shape[2:])
    return gather_rows(flat, recipe_ids.long() * k + stride_ids.long())


class _GatherCols(torch.autograd.Function):
    @staticmethod
    def forward(ctx, mat: torch.Tensor, cols: torch.Tensor):
        ctx.save_for_backward(cols)
        ctx.n = mat.shape[-1]
        return mat.index_select(-1, cols)

    @staticmethod
    def backward(ctx, g: torch.Tensor):
        (cols,) = ctx.saved_tensors
        dt = _acc_dtype(g)
        onehot = F.one_hot(cols, ctx.n).to(dt)  # [c, n]
        return g.to(dt) @ onehot, None


def gather_cols(mat: torch.Tensor, cols: torch.Tensor) -> torch.Tensor:
    """mat[..., cols] for a 2-D matrix."""
    return _GatherCols.apply(mat, cols.long())
