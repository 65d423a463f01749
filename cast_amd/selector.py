"""The native layers' ``select()`` boundary on the HIP kernels.

:func:`taba_select` keeps the method surface, argument meaning, output format
and errors of ``MatrixTrajectoryAdaptiveBudgetAttentionCompiler.select``
(P/qk_uncertainty_tangent_attention.py:988-1082), the select at the bottom of
the chain that CAST's attention compiler
(``MatrixClosedLoopCWCAAttentionCompiler``,
P/control_response_cwca_attention.py:2083-2099) ends in:

* Q/K ``[B, H, T*h*w, D]`` are tiled into (tt, th, tw) blocks of the latent
  grid, mean-pooled and L2-normalised (``rcsa_pack_tokens`` +
  ``rcsa_pool_query`` / ``rcsa_pool_key``; a zero-padded mean and the
  valid-token mean have the same direction);
* cosine block scores (``rcsa_block_scores``);
* the row budgets are read at call time from the compiler's
  ``_runtime_degrees(q_blocks)`` (P/qk_uncertainty_tangent_attention.py:982,
  :1040), which ``set_layer_index`` re-installs for every layer
  (P/control_response_cwca_attention.py:1389-1529);
* the Manhattan <= 1 local stencil is kept first, then the other blocks by
  score, ties to the lower index (``rcsa_select_topk`` in rank order); the
  local blocks are ordered among themselves by fl(score + 1e6), which is
  what the reference's ``score + 1e6 * local`` ranks by;
* every row lists ``max(row_degrees)`` blocks and ``counts`` holds each row's
  own budget; the consumer reads the prefix;
* the duplicate / missing-local certificate, then the report.

The wrappers above it in the reference's method resolution order (section
and worldline report fields, P/qk_uncertainty_tangent_attention.py:1201-1209,
1722-1734; the pending budget record, P/control_response_cwca_attention.py:
2030-2034) run unchanged when a compiler subclass places its ``select`` just
above the TABA class (see :func:`taba_select`).

:class:`BlockSelector` is the same selection for callers without a compiler
object: it holds the budgets itself, or takes them per call.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Sequence

import torch

from . import budget, layout, ops


@dataclass(frozen=True)
class SelectionReport:
    """Field names and meaning of QKUncertaintyTangentSelectionReport
    (P/qk_uncertainty_tangent_attention.py:26-63)."""
    batch_heads: int
    query_rows: int
    edges_per_row: int
    row_duplicate_violations: int
    selected_orientation_violations: int
    max_orientation_violations_per_row: int
    mean_selected_ray_cosine: float
    mean_selected_qk_cosine: float
    qk_read_for_selection: bool
    selector_count: int
    protected_local_edges: int
    missing_local_edges: int
    mean_geometry_gate: float
    max_geometry_gate: float
    mean_rank_margin_gate: float = 0.0
    max_rank_margin_gate: float = 0.0
    action_geometry_trust: float = 1.0
    budget_min: int = 0
    budget_max: int = 0
    budget_total: int = 0
    mean_ray_motion: float = 0.0
    max_ray_motion: float = 0.0
    trajectory_complexity_kind: str = "motion_magnitude"
    persistence_quota_min: int = 0
    persistence_quota_max: int = 0
    mean_first_order_motion: float = 0.0
    section_budget_min: int = 0
    section_budget_max: int = 0
    mean_query_uncertainty: float = 0.0
    max_query_uncertainty: float = 0.0
    remote_quota_min: int = 0
    remote_quota_max: int = 0
    remote_quota_violations: int = 0
    memory_budget_total: int = 0
    current_worldline_budget_min: int = 0
    current_worldline_budget_max: int = 0


class BlockSelector:
    """Fixed-budget block selector over the latent grid's (tt, th, tw) tiles."""

    trajectory_complexity_kind = "motion_magnitude"

    def __init__(self, block_shape: Sequence[int], degree: int, num_blocks: int):
        self._block_shape = tuple(int(x) for x in block_shape)
        self._degree = int(degree)
        self._num_blocks = int(num_blocks)
        self._row_degrees: Optional[torch.Tensor] = None
        self._ray_motion: Optional[torch.Tensor] = None
        self._first_order_motion: Optional[torch.Tensor] = None

    def compile_budgets(self, *, token_h: int, token_w: int,
                        row_degrees: Optional[torch.Tensor] = None,
                        ray_motion: Optional[torch.Tensor] = None,
                        first_order_motion: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Fix the per-row budgets: ``row_degrees`` as given, or the
        trajectory-adaptive split of ``num_blocks * degree`` edges by
        ``ray_motion`` (a fixed budget when neither is given)."""
        _, th, tw = self._block_shape
        nh, nw = math.ceil(token_h / th), math.ceil(token_w / tw)
        local = layout.local_stencil(self._num_blocks, nh, nw)
        if row_degrees is not None:
            rows = torch.as_tensor(row_degrees).to(torch.long).reshape(-1).cpu()
            if rows.numel() != self._num_blocks:
                raise RuntimeError("row budgets do not match the attention blocks")
            if int(rows.min()) < int(local.sum(dim=-1).max()):
                raise RuntimeError("row budget is too small to protect the local stencil")
            if int(rows.max()) > self._num_blocks:
                raise RuntimeError("row budget assigns more keys than exist")
        elif ray_motion is not None:
            rows = budget.motion_row_degrees(torch.as_tensor(ray_motion).cpu(), self._degree,
                                             local)
        else:
            rows = torch.full((self._num_blocks,), self._degree, dtype=torch.long)
        motion = (torch.zeros(self._num_blocks) if ray_motion is None
                  else torch.as_tensor(ray_motion).float().cpu())
        self._row_degrees = rows
        self._ray_motion = motion
        self._first_order_motion = (motion if first_order_motion is None
                                    else torch.as_tensor(first_order_motion).float().cpu())
        return rows

    def select(self, q: torch.Tensor, k: torch.Tensor, *, geometry_indices: torch.Tensor,
               geometry_counts: torch.Tensor, latent_hw: tuple[int, int],
               block_shape: tuple[int, int, int], row_degrees=None):
        """Returns ``(selected int32 [B, H, N, maxK], counts int32 [B, H, N], report)``.

        ``row_degrees`` (length N, or a callable ``q_blocks -> degrees``) replaces
        the compiled budgets for this call only."""
        del geometry_indices
        if self._row_degrees is None or self._ray_motion is None:
            raise RuntimeError("row budgets were not compiled")
        if row_degrees is None:
            row_degrees = self._row_degrees
        rows_fn = row_degrees if callable(row_degrees) else (lambda _qb: row_degrees)
        return select_blocks(q, k, geometry_counts=geometry_counts, latent_hw=latent_hw,
                             block_shape=block_shape, compiled_shape=self._block_shape,
                             num_blocks=self._num_blocks, degree=self._degree,
                             runtime_degrees=rows_fn, ray_motion=self._ray_motion,
                             first_order_motion=self._first_order_motion,
                             kind=self.trajectory_complexity_kind)


def taba_select(compiler, q: torch.Tensor, k: torch.Tensor, *,
                geometry_indices: torch.Tensor, geometry_counts: torch.Tensor,
                latent_hw: tuple[int, int], block_shape: tuple[int, int, int],
                report_cls=None):
    """``select`` of a trajectory-adaptive-budget compiler on the HIP kernels.

    ``compiler`` is the reference's compiler object (or anything with its
    attributes): ``_block_shape``, ``_num_blocks``, ``_degree``,
    ``_row_degrees``, ``_ray_motion``, ``_first_order_motion``,
    ``trajectory_complexity_kind`` and ``_runtime_degrees(q_blocks)``.  Every
    attribute is read at call time, so budgets installed by
    ``set_layer_index`` between two calls take effect.  ``q_blocks`` is the
    packed query ``[B, H, N, tt*th*tw, D]``: the tile members of
    ``_tile_visual_tensor`` (P/reciprocal_joint_attention.py:64-103) in token
    order with the zero padding last, the same multiset per tile.
    ``report_cls`` (default :class:`SelectionReport`) is built with the field
    names of ``QKUncertaintyTangentSelectionReport``.

    A compiler subclass binds it one level above the TABA class, so that every
    ``select`` wrapper of the subclasses still runs::

        class HipTABA(MatrixTrajectoryAdaptiveBudgetAttentionCompiler):
            def select(self, q, k, **kw):
                return taba_select(self, q, k, **kw)

        class Compiler(MatrixClosedLoopCWCAAttentionCompiler, HipTABA):
            pass   # MRO: ..., ResidualTABA, HipTABA, TABA, ...
    """
    del geometry_indices
    if getattr(compiler, "_row_degrees", None) is None or \
            getattr(compiler, "_ray_motion", None) is None:
        raise RuntimeError("TABA budgets were not compiled")
    ray = compiler._ray_motion
    first = getattr(compiler, "_first_order_motion", None)
    return select_blocks(q, k, geometry_counts=geometry_counts, latent_hw=latent_hw,
                         block_shape=block_shape,
                         compiled_shape=tuple(int(x) for x in compiler._block_shape),
                         num_blocks=int(compiler._num_blocks), degree=int(compiler._degree),
                         runtime_degrees=compiler._runtime_degrees, ray_motion=ray,
                         first_order_motion=ray if first is None else first,
                         kind=getattr(compiler, "trajectory_complexity_kind",
                                      "motion_magnitude"),
                         report_cls=report_cls)


def select_blocks(q: torch.Tensor, k: torch.Tensor, *, geometry_counts: torch.Tensor,
                  latent_hw, block_shape, compiled_shape, num_blocks: int, degree: int,
                  runtime_degrees, ray_motion, first_order_motion, kind: str,
                  report_cls=None):
    """The selection itself (P/qk_uncertainty_tangent_attention.py:998-1082)."""
    if q.shape != k.shape or q.ndim != 4:
        raise ValueError("TABA requires equal B,H,L,D Q/K")
    if tuple(int(v) for v in block_shape) != tuple(compiled_shape):
        raise RuntimeError("TABA runtime block shape differs from compilation")
    ref_counts = geometry_counts[0, 0].detach().to("cpu", torch.long)
    if ref_counts.numel() != num_blocks or not torch.all(ref_counts == degree):
        raise RuntimeError("TABA baseline layout does not have fixed K")
    height, width = (int(v) for v in latent_hw)
    B, H, L, D = q.shape
    if L % (height * width):
        raise ValueError("visual token length does not match the latent grid")
    temporal = L // (height * width)
    shape = tuple(compiled_shape)
    lay = layout.compact_layout(range(temporal), 0, height, width, shape, q.device)
    if lay.n_blocks != num_blocks:
        raise RuntimeError("latent grid does not give the compiled number of blocks")
    bs, nb = lay.block_size, lay.n_blocks
    # packed [B, H, nb*bs, D] tiles (q viewed as [B, L, H, D], no copy of q itself)
    qp = ops.pack_tokens(q.transpose(1, 2), lay.slot_token)
    kp = ops.pack_tokens(k.transpose(1, 2), lay.slot_token)
    qhat, _, _ = ops.pool_query(qp, lay.slot_valid, bs)
    khat, _, _, _ = ops.pool_key(kp, lay.slot_valid, bs)
    score = ops.block_scores(qhat, khat)                      # [B*H, nb, nb]
    local = layout.local_stencil(nb, *lay.grid, device=q.device)
    ranking = torch.where(local, (score + 1e6) - 1e6, score)  # order of fl(s + 1e6)
    rows = torch.as_tensor(runtime_degrees(qp.view(B, H, nb, bs, D)))
    rows = rows.detach().to("cpu", torch.long).reshape(-1)
    if rows.numel() != nb:
        raise RuntimeError("row budgets do not match the attention blocks")
    if int(rows.min()) < 0 or int(rows.max()) > nb:
        raise RuntimeError("TABA assigned more keys than exist")
    max_degree = int(rows.max())
    selected, _ = ops.select_topk(ranking, max_degree, forced=local, max_k=max_degree,
                                  order="rank")
    selected = selected.view(B, H, nb, max_degree)
    counts = rows.to(device=q.device, dtype=torch.int32)[None, None].expand(B, H, -1)
    counts = counts.contiguous()
    # certificate: no repeated neighbour in a row's prefix, every local block kept
    live = torch.arange(max_degree, device=q.device)[None, None, None, :] < counts[..., None]
    dup = ((selected[..., 1:] == selected[..., :-1]) & live[..., 1:]).sum()
    chosen = (torch.gather(local[None, None].expand(B, H, -1, -1), -1, selected.long())
              & live).sum()
    host = torch.stack([dup.double(), chosen.double(), score.double().mean()]).cpu()
    duplicates = int(host[0])
    expected_local = int(layout.local_stencil(nb, *lay.grid).sum()) * B * H
    missing_local = expected_local - int(host[1])
    if duplicates or missing_local:
        raise RuntimeError("TABA selection certificate failed")
    ray = torch.as_tensor(ray_motion).float()
    first = torch.as_tensor(first_order_motion).float()
    report = (report_cls or SelectionReport)(
        batch_heads=B * H, query_rows=nb, edges_per_row=int(degree),
        row_duplicate_violations=duplicates, selected_orientation_violations=0,
        max_orientation_violations_per_row=0, mean_selected_ray_cosine=0.0,
        mean_selected_qk_cosine=float(host[2]), qk_read_for_selection=True,
        selector_count=1, protected_local_edges=expected_local,
        missing_local_edges=missing_local, mean_geometry_gate=0.0, max_geometry_gate=0.0,
        budget_min=int(rows.min()), budget_max=max_degree, budget_total=int(rows.sum()),
        mean_ray_motion=float(ray.mean()), max_ray_motion=float(ray.max()),
        trajectory_complexity_kind=kind, mean_first_order_motion=float(first.mean()))
    return selected, counts, report
