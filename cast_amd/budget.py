"""Per-row key-block budgets (host side, as in the reference).

The reference keeps its budget logic in host PyTorch; so does this module.
It covers the parts that set the selector's per-row ``k``:

* ``budget_blocks`` / ``mean_degree``: the fixed per-row budget of the
  compact path (P/matrix_curvature_phase_frame_weave.py:5727-5731);
* ``apportion``: largest-remainder integer apportionment of a global edge
  budget by non-negative weights, fp32 arithmetic and ties to the lower index
  (P/qk_uncertainty_tangent_attention.py:847-865);
* ``apportion_section_matrix``: the same per row of a weight matrix
  (P/qk_uncertainty_tangent_attention.py:1239-1264);
* ``motion_row_degrees``: the trajectory-adaptive budget, weights
  1 + motion / mean(motion) (P/qk_uncertainty_tangent_attention.py:867-870,
  944-963);
* ``saturate``: clamp rows to the number of key blocks and hand the overflow
  back to rows with capacity (P/matrix_curvature_phase_frame_weave.py:5807-5817).
"""
from __future__ import annotations

import torch


def budget_blocks(fraction: float, n_blocks: int) -> int:
    """k = int(round(fraction * n_blocks)), Python round-half-even."""
    return int(round(fraction * n_blocks))


def mean_degree(local: torch.Tensor, density: float, n_blocks: int) -> int:
    """Per-row degree of the compact path: at least the widest local row,
    at least round(density * blocks), at most all blocks."""
    widest = int(local.sum(dim=-1).max())
    return min(max(widest, budget_blocks(density, n_blocks)), n_blocks)


def _largest_remainder(raw: torch.Tensor, floor: torch.Tensor, remainder: torch.Tensor):
    # hand one extra unit to the `remainder` largest fractional parts of each
    # row; a stable descending sort keeps ties on the lower index
    frac = raw - floor
    order = torch.sort(frac, dim=-1, descending=True, stable=True).indices
    rank = torch.empty_like(order)
    rank.scatter_(-1, order, torch.arange(order.shape[-1], device=order.device)
                  .expand_as(order).contiguous())
    return floor + (rank < remainder[..., None]).to(floor.dtype)


def apportion(weights: torch.Tensor, total: int) -> torch.Tensor:
    """Integer split of ``total`` proportional to ``weights`` (int64 vector)."""
    w = torch.as_tensor(weights)
    if w.ndim != 1 or w.numel() == 0:
        raise ValueError("apportion: weights must be a non-empty vector")
    if total <= 0:
        raise ValueError("apportion: total must be positive")
    w = w.float().clamp_min(0.0)
    if not bool(w.sum() > 0):
        w = torch.ones_like(w)
    raw = float(total) * w / w.sum()
    floor = torch.floor(raw).to(torch.long)
    res = _largest_remainder(raw, floor, torch.tensor(total) - floor.sum())
    if int(res.sum()) != total:
        raise RuntimeError("apportion: integer split lost the total")
    return res


def apportion_section_matrix(weights: torch.Tensor, total_per_section: int) -> torch.Tensor:
    """Row-wise :func:`apportion` of a ``[sections, n]`` weight matrix."""
    w = torch.as_tensor(weights).float().clamp_min(0.0)
    w = torch.where(w.sum(dim=-1, keepdim=True) > 0, w, torch.ones_like(w))
    raw = float(total_per_section) * w / w.sum(dim=-1, keepdim=True)
    floor = torch.floor(raw).to(torch.long)
    return _largest_remainder(raw, floor, total_per_section - floor.sum(dim=-1))


def motion_row_degrees(ray_motion: torch.Tensor, degree: int,
                       local: torch.Tensor) -> torch.Tensor:
    """Trajectory-adaptive row budgets: ``n_blocks * degree`` edges split by
    1 + motion / (mean(motion) + eps); every row must still hold its local
    stencil and no row may exceed the number of blocks."""
    motion = torch.as_tensor(ray_motion).float()
    n = motion.numel()
    eps = torch.finfo(motion.dtype).eps
    weights = 1.0 + motion / (motion.mean() + eps)
    rows = apportion(weights, n * int(degree))
    if int(rows.min()) < int(local.sum(dim=-1).max()):
        raise RuntimeError("row budget is too small to protect the local stencil")
    if int(rows.max()) > n:
        raise RuntimeError("row budget assigns more keys than exist")
    return rows


def saturate(degrees: torch.Tensor, n_blocks: int, target_total: int) -> torch.Tensor:
    """Clamp every row to ``n_blocks`` and give the lost edges, one each, to
    the lowest-index rows with capacity until ``target_total`` is reached or
    no capacity remains."""
    d = torch.as_tensor(degrees).to(torch.long).clamp(max=n_blocks)
    missing = int(target_total) - int(d.sum())
    while missing > 0:
        cand = torch.nonzero(d < n_blocks).flatten()
        if cand.numel() == 0:
            break
        take = min(missing, int(cand.numel()))
        d[cand[:take]] += 1
        missing -= take
    return d
