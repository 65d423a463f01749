"""FC-PASM swap router with its per-row work on the device.

Mirrors ``FCPASMSwapRoutingConfig`` and ``FCPASMLocalCoordinateSwapRouter``
(P/fc_pasm_swap_routing.py:23-61, 109-1115): same configuration fields and
checks, same ``refine`` keyword arguments, return value (the refined route and
a record) and fallback records, ``summary`` and ``reset``.  The router never
changes a row's degree: it starts from the pooled-Q/K top-k and applies at most
``num_swap_rounds`` single exchanges of one kept key block for one candidate,
each the best over all current rows under the anchor + reconstruction
omission objective.

Per row, the softmax, the pooled attention output, the 2k candidates, their
omission proxies and the row errors (``rcsa_route_proxy``) and the best
exchange (``rcsa_route_best_swap``) run on the device; the objective's
quadratic terms (small [S, S] operator products over the current cells), the
choice of the strongest row and the checks at the end are torch on the same
device, as in the reference.  The FC transport operator of an anchor pair
comes from ``operator(transport, pair, spatial_shape, exponent)`` (a [S, S]
matrix, output x input; by default ``cast_amd.transport.fc_transport_operator``,
built from the transport's published phases); for every pair the transport
does not hold, or with ``operator=None``, the operator is the identity (the
reference's g = 0 propagation).  The historical-only ablation is not built.
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass
from typing import Any, Callable, Optional

import numpy as np
import torch

from . import ops
from .transport import fc_transport_operator


@dataclass(frozen=True)
class FCPASMSwapRoutingConfig:
    """The router's configuration (P/fc_pasm_swap_routing.py:23-61)."""
    candidate_multiplier: int = 2
    num_swap_rounds: int = 1
    swap_eps: float = 1e-6
    lambda_anchor: float = 1.0
    lambda_reconstruction: float = 1.0
    sketch_groups: int = 16
    require_fc_transport: bool = False
    min_transport_affinity: float = 0.0
    min_pair_transport_affinity: float = 0.0
    max_swaps_per_call: int = 0
    active_layers: tuple = ()
    historical_only: bool = False
    same_bank_only: bool = False

    def __post_init__(self) -> None:
        if self.candidate_multiplier < 1:
            raise ValueError("candidate multiplier must be positive")
        if self.num_swap_rounds not in {0, 1, 2}:
            raise ValueError("FC-PASM routing supports zero to two swap rounds")
        if not math.isfinite(self.swap_eps) or self.swap_eps < 0.0:
            raise ValueError("swap epsilon must be finite and non-negative")
        if self.lambda_anchor < 0.0 or self.lambda_reconstruction < 0.0:
            raise ValueError("routing objective weights must be non-negative")
        if self.lambda_anchor + self.lambda_reconstruction <= 0.0:
            raise ValueError("routing objective must contain a positive term")
        if self.sketch_groups < 2 or self.sketch_groups % 2:
            raise ValueError("routing sketch groups must be a positive even number")
        if not 0.0 <= self.min_transport_affinity <= 1.0:
            raise ValueError("minimum FC transport affinity must be in [0, 1]")
        if not 0.0 <= self.min_pair_transport_affinity <= 1.0:
            raise ValueError("minimum pair FC transport affinity must be in [0, 1]")
        if self.max_swaps_per_call < 0:
            raise ValueError("maximum swaps per call must be non-negative")
        if any(layer < 0 for layer in self.active_layers):
            raise ValueError("routing active layers must be non-negative")
        if self.historical_only and self.same_bank_only:
            raise ValueError("historical-only routing already fixes the KV bank")


def _affinity(entry: Any) -> float:
    if not isinstance(entry, dict):
        return 0.0
    a = entry.get("mean_affinity", 0.0)
    return float(a.detach().float().item()) if isinstance(a, torch.Tensor) else float(a)


class FCPASMSwapRouter:
    """Fixed-budget refinement of compact pooled-Q/K routes (the reference's
    ``FCPASMLocalCoordinateSwapRouter``), its per-row work on the device."""

    def __init__(self, config: FCPASMSwapRoutingConfig,
                 operator: Optional[Callable[..., Optional[torch.Tensor]]] = fc_transport_operator
                 ) -> None:
        self.config = config
        self.operator = operator
        self._records: list[dict[str, Any]] = []
        self._plans: dict = {}

    # ---- the objective over the current cells (torch on the device) ----
    def _matrix(self, transport, pair, shape, exponent, device):
        """The pair's operator at ``exponent``, or None for the identity."""
        if self.operator is not None and isinstance(transport, dict):
            entry = transport.get("pairs", {}).get(pair)
            if isinstance(entry, dict):
                m = self.operator(transport, pair, shape, exponent)
                if m is not None:
                    return m.to(device=device, dtype=torch.float32)
        return None

    @staticmethod
    def _cells(frames, group, cells):
        return {int(f): min(int(f) // int(group), cells - 1) for f in frames}

    def _grid(self, transport, spatial):
        if transport is None:
            return (1, spatial)
        return (int(transport.get("attention_spatial_h", 1)),
                int(transport.get("attention_spatial_w", spatial)))

    def _pairs(self, frames, boundary):
        return [(int(l), int(r)) for l, r in zip(frames, frames[1:])
                if (l < boundary) == (r < boundary) and r - l > 1]

    def _plan(self, cells, spatial, frames, group, boundary, transport, device):
        """The objective's structure over the current cells
        (P/fc_pasm_swap_routing.py:414-614), built once per refine on the host:

        * anchor counts and every pair propagated with the identity (g = 0) fold
          into per-cell quadratic coefficients and weights of the cells' squared
          error norms and cross products (the value), and per-pair cross weights
          (the linear term), fp32 like the reference's scalar products;
        * a pair with a transport operator keeps its skipped frames' operators
          stacked, ((1 - a) T^a, a T^-(1-a)) [frames, S, S], for batched products.

        Plans of identity-only objectives are cached per geometry."""
        cfg = self.config
        key = (cells, spatial, tuple(frames), group, boundary, str(device),
               cfg.lambda_anchor, cfg.lambda_reconstruction)
        if transport is None and key in self._plans:
            return self._plans[key]
        f32 = np.float32
        cell = self._cells(frames, group, cells)
        count = [0.0] * cells
        for f in frames:
            count[cell[int(f)]] += 1.0
        la, lr = cfg.lambda_anchor, cfg.lambda_reconstruction
        coef = [f32(c) * f32(la) for c in count]
        weight = np.zeros((cells, cells), dtype=np.float64)
        for c in range(cells):
            weight[c, c] += la * count[c]
        cross, stacks = [], []
        used = False
        shape = self._grid(transport, spatial)
        for left, right in self._pairs(frames, boundary):
            lc, rc = cell[left], cell[right]
            alphas = [float(t - left) / float(right - left) for t in range(left + 1, right)]
            mats = [(self._matrix(transport, (left, right), shape, a, device),
                     self._matrix(transport, (left, right), shape, -(1.0 - a), device))
                    for a in alphas]
            if all(lm is None and rm is None for lm, rm in mats):
                x = f32(0.0)
                for a in alphas:
                    wl, wr, lam = f32(1.0 - a), f32(a), f32(lr)
                    if lc == rc:
                        c = wl + wr
                        coef[lc] += lam * (c * c)
                    else:
                        coef[lc] += lam * (wl * wl)
                        coef[rc] += lam * (wr * wr)
                        x += lam * (wl * wr)
                    weight[lc, lc] += lr * (1.0 - a) ** 2
                    weight[rc, rc] += lr * a * a
                    weight[lc, rc] += lr * a * (1.0 - a)
                    weight[rc, lc] += lr * a * (1.0 - a)
                if lc != rc:
                    cross.append((lc, rc, float(x)))
                continue
            used = True
            eye = torch.eye(spatial, device=device, dtype=torch.float32)
            lo = torch.stack([(1.0 - a) * (eye if lm is None else lm)
                              for a, (lm, _) in zip(alphas, mats)])
            ro = torch.stack([a * (eye if rm is None else rm) for a, (_, rm) in zip(alphas, mats)])
            stacks.append((lc, rc, lo, ro))

        def dev32(a):
            return torch.from_numpy(np.asarray(a, dtype=np.float32)).pin_memory().to(
                device, non_blocking=True)
        diag = [weight[c, c] for c in range(cells)]
        cross_w = [(c, d, weight[c, d] + weight[d, c]) for c in range(cells)
                   for d in range(c + 1, cells) if weight[c, d] + weight[d, c] != 0.0]
        plan = {"coef": dev32(coef).repeat_interleave(spatial), "diag": dev32(diag),
                "cross_value": cross_w, "cross": cross, "stacks": stacks, "used": used}
        if transport is None:
            self._plans[key] = plan
        return plan

    def _terms(self, error, cells, spatial, plan):
        """Quadratic coefficient (per row) and linear term (per row and group)
        of the objective at ``error`` (P/fc_pasm_swap_routing.py:414-547)."""
        lam = self.config.lambda_reconstruction
        BH, rows, G = error.shape
        view = error.reshape(BH, cells, spatial, G)
        lin = torch.zeros_like(view)
        for lc, rc, x in plan["cross"]:
            lin[:, lc].add_(view[:, rc], alpha=x)
            lin[:, rc].add_(view[:, lc], alpha=x)
        coef = plan["coef"]
        if plan["stacks"]:
            coef = coef.clone().reshape(cells, spatial)
        for lc, rc, lo, ro in plan["stacks"]:
            el, er = view[:, lc], view[:, rc]
            if lc == rc:
                comb = lo + ro
                hess = lam * torch.einsum("tka,tkb->ab", comb, comb)
                dg = torch.diagonal(hess)
                coef[lc] += dg
                lin[:, lc] += torch.einsum("st,btg->bsg", hess, el) - dg[None, :, None] * el
            else:
                hl = lam * torch.einsum("tka,tkb->ab", lo, lo)
                hr = lam * torch.einsum("tka,tkb->ab", ro, ro)
                hx = lam * torch.einsum("tka,tkb->ab", lo, ro)
                dl, dr = torch.diagonal(hl), torch.diagonal(hr)
                coef[lc] += dl
                coef[rc] += dr
                lin[:, lc] += (torch.einsum("st,btg->bsg", hl, el) - dl[None, :, None] * el
                               + torch.einsum("st,btg->bsg", hx, er))
                lin[:, rc] += (torch.einsum("st,btg->bsg", hr, er) - dr[None, :, None] * er
                               + torch.einsum("st,btg->bsg", hx.T, el))
        return coef.reshape(rows), lin.reshape(BH, rows, G)

    def _value(self, error, cells, spatial, plan):
        """The objective (P/fc_pasm_swap_routing.py:550-614): the anchor and
        identity-propagated terms as weighted squared norms and cross products
        of the cells' errors, the transported frames through their stacked
        operators."""
        BH, rows, G = error.shape
        view = error.reshape(BH, cells, spatial, G)
        value = (plan["diag"] * view.square().sum(dim=(0, 2, 3))).sum()
        for c, d, wcd in plan["cross_value"]:
            value = value + wcd * (view[:, c] * view[:, d]).sum()
        lam = self.config.lambda_reconstruction
        for lc, rc, lo, ro in plan["stacks"]:
            prop = (torch.einsum("tuv,bvg->tbug", lo, view[:, lc])
                    + torch.einsum("tuv,bvg->tbug", ro, view[:, rc]))
            value = value + lam * prop.square().sum()
        return value

    def _fallback(self, layer_index, reason, **extra):
        rec = {"layer_index": int(layer_index), "status": "independent_topk_fallback",
               "fallback_reason": reason, "swap_count": 0, "fixed_budget": True}
        rec.update(extra)
        self._records.append(rec)
        return rec

    def refine(self, *, score: torch.Tensor, pooled_value: torch.Tensor, selected: torch.Tensor,
               counts: torch.Tensor, local: torch.Tensor, memory_blocks: int,
               spatial_shape: tuple, exact_current_frames: tuple, temporal_group_size: int,
               current_boundary: int, transport: Optional[dict], layer_index: int):
        """Refine ``selected`` [B, H, N, K] (first ``counts`` entries of each row
        kept) without changing any row's degree; returns (selected, record)."""
        cfg = self.config
        if score.ndim != 4 or pooled_value.ndim != 4:
            raise ValueError("routing requires BHQK score and BHKD pooled values")
        if score.shape[:2] != pooled_value.shape[:2] or score.shape[-1] != pooled_value.shape[-2]:
            raise ValueError("routing score/value layouts differ")
        if selected.shape[:3] != score.shape[:3] or counts.shape != score.shape[:3]:
            raise ValueError("routing selection/count layouts differ")
        if local.shape != score.shape[-2:]:
            raise ValueError("routing local stencil has invalid shape")
        score = score.detach()
        pooled_value = pooled_value.detach()
        baseline = selected.clone()
        if cfg.active_layers and layer_index not in cfg.active_layers:
            return baseline, self._fallback(layer_index, "layer_not_enabled")
        B, H, N = score.shape[:3]
        M = int(memory_blocks)
        rows = score.shape[-2] - M
        spatial = int(spatial_shape[0] * spatial_shape[1])
        if rows <= 0 or rows % spatial:
            return baseline, self._fallback(layer_index, "no_rectangular_current_rows",
                                            fc_cache_used=False)
        cells = rows // spatial
        frames = tuple(int(f) for f in exact_current_frames)
        if tuple(sorted(set(frames))) != frames:
            raise ValueError("routing Exact Current frames must be unique and chronological")
        pairs = self._pairs(frames, current_boundary)
        if cfg.num_swap_rounds == 0 or len(frames) < 2 or not pairs:
            reason = ("zero_swap_rounds" if cfg.num_swap_rounds == 0 else
                      "fewer_than_two_exact_anchors" if len(frames) < 2 else "no_skipped_frames")
            return baseline, self._fallback(layer_index, reason, fc_cache_used=False)
        tpairs = transport.get("pairs", {}) if isinstance(transport, dict) else {}
        matching = [tpairs[p] for p in pairs if isinstance(tpairs.get(p), dict)
                    and isinstance(tpairs[p].get("theta"), torch.Tensor)]
        affinity = max((_affinity(e) for e in matching), default=0.0)
        strong = bool(matching) and affinity >= cfg.min_transport_affinity
        if cfg.require_fc_transport and not strong:
            return baseline, self._fallback(
                layer_index, "weak_previous_layer_fc_transport" if matching
                else "missing_previous_layer_fc_transport",
                matching_transport_affinity=affinity, fc_cache_used=False, g0_fallback=True)
        if cfg.historical_only:
            raise NotImplementedError("the historical-only routing ablation is not built")
        gate = None
        gate_cells = 0
        if cfg.min_pair_transport_affinity > 0.0:
            cg = torch.zeros(cells, dtype=torch.bool)
            for left, right in pairs:
                if _affinity(tpairs.get((left, right))) < cfg.min_pair_transport_affinity:
                    continue
                for t in range(left + 1, right):
                    c = min(t // int(temporal_group_size), cells - 1)
                    gate_cells += int(not bool(cg[c]))
                    cg[c] = True
            if not bool(cg.any()):
                return baseline, self._fallback(
                    layer_index, "no_strong_transport_pair_cells",
                    matching_transport_affinity=affinity,
                    min_pair_transport_affinity=cfg.min_pair_transport_affinity,
                    pair_gate_cells=0, fc_cache_used=bool(matching))
            gate = cg.repeat_interleave(spatial).pin_memory().to(score.device, non_blocking=True)

        dev = score.device
        K = selected.shape[-1]
        cnt = counts.clamp(0, K).to(torch.int32)
        sel = selected.to(torch.int32).contiguous()
        if sel.data_ptr() == selected.data_ptr():
            sel = sel.clone()  # the caller's route stays as it was
        # Candidates for the widest possible row (the list width bounds every
        # count): each row still uses only its first min(mult * count, N), so the
        # result is that of the reference's min(N, mult * max count) candidates
        # without reading the counts back.
        L = min(N, cfg.candidate_multiplier * K)
        cand, proxy, error = ops.route_proxy(
            score, pooled_value, local, sel, cnt, memory_blocks=M, n_cand=L,
            cand_mult=cfg.candidate_multiplier, sketch_groups=cfg.sketch_groups)
        plan = self._plan(cells, spatial, frames, int(temporal_group_size),
                          int(current_boundary), transport, dev)
        obj_before = self._value(error, cells, spatial, plan)
        cache_used = bool(matching) or plan["used"]
        rounds = cfg.num_swap_rounds
        # swap count, stop flag and the applied swaps, written by the device
        state = torch.zeros(2 + 6 * rounds, device=dev, dtype=torch.int32)
        for _ in range(rounds):
            coef, lin = self._terms(error, cells, spatial, plan)
            best, flat = ops.route_best_swap(proxy, cand, local, sel, cnt, coef, lin, error,
                                             memory_blocks=M, cand_mult=cfg.candidate_multiplier,
                                             same_bank=cfg.same_bank_only, row_gate=gate)
            ops.route_apply_swap(best, flat, cand, proxy, sel, error, state, memory_blocks=M,
                                 max_swaps=cfg.max_swaps_per_call, eps=cfg.swap_eps)
        # the checks at the end (P/fc_pasm_swap_routing.py:983-1033) as device
        # sums, read back once with the objective and the applied swaps
        checks = ops.route_check(baseline, sel, cnt, local, memory_blocks=M)
        obj_after = self._value(error, cells, spatial, plan)
        host = torch.cat([checks.double(), torch.stack([obj_before, obj_after]).double(),
                          state.double()]).cpu()  # the one read-back of a refine
        vals = [int(x) for x in host[:10].tolist()]
        before_f, after_f = float(host[10]), float(host[11])
        st = [int(x) for x in host[12:].tolist()]
        swaps = st[0]
        if vals[7] == 0:  # no row keeps a block
            return baseline, self._fallback(layer_index, "no_swappable_kv_selected")
        if cfg.same_bank_only and vals[0]:
            raise RuntimeError("same-bank FC-PASM routing changed Memory KV counts")
        if vals[1]:
            raise RuntimeError("FC-PASM routing emitted duplicate keys")
        if vals[2] != vals[9]:
            raise RuntimeError("FC-PASM routing removed a protected local edge")
        if after_f > before_f + 1e-5 * max(abs(before_f), 1.0):
            raise RuntimeError("FC-PASM swap increased its refinement objective")
        hb, ha = vals[4], vals[5]
        kmin, kmax, ksum, max_swappable = K - vals[6], vals[7], vals[8], vals[7]
        cur_unchanged = vals[3] == 0
        chosen = []
        for i in range(swaps):
            r = st[2 + 6 * i: 8 + 6 * i]
            b, h = divmod(r[0], H)
            imp = struct.unpack("<f", struct.pack("<i", r[5]))[0]
            chosen.append({"b": b, "h": h, "row": r[1], "slot": r[2], "removed": r[3],
                           "added": r[4], "improvement": imp})
        record = {
            "layer_index": int(layer_index), "status": "refined",
            "candidate_multiplier": cfg.candidate_multiplier,
            "candidate_max": min(N, cfg.candidate_multiplier * max_swappable),
            "swap_rounds": cfg.num_swap_rounds, "max_swaps_per_call": cfg.max_swaps_per_call,
            "swap_count": swaps, "objective_before": before_f,
            "objective_after": after_f,
            "objective_improvement": before_f - after_f,
            "average_swap_improvement": (sum(c["improvement"] for c in chosen) / swaps
                                         if swaps else 0.0),
            "anchor_term_weight": cfg.lambda_anchor,
            "reconstruction_term_weight": cfg.lambda_reconstruction,
            "reconstruction_terms": sum(max(0, r - l - 1) for l, r in zip(frames, frames[1:])
                                        if (l < current_boundary) == (r < current_boundary)),
            "fc_cache_used": cache_used, "matching_transport_affinity": affinity,
            "min_pair_transport_affinity": cfg.min_pair_transport_affinity,
            "pair_gate_cells": gate_cells, "g0_fallback": not cache_used, "fixed_budget": True,
            "historical_only": cfg.historical_only, "same_bank_only": cfg.same_bank_only,
            "historical_budget_before": hb, "historical_budget_after": ha,
            "current_kv_support_unchanged": bool(cur_unchanged),
            "minimum_k": kmin, "maximum_k": kmax, "budget_before": ksum, "budget_after": ksum,
            "unique_indices": True, "local_support_preserved": True, "swaps": chosen,
        }
        self._records.append(record)
        return sel.to(selected.dtype), record

    def summary(self) -> dict[str, Any]:
        """The configuration and every call's record, tensors as floats."""
        records = []
        for raw in self._records:
            row = {}
            for key, value in raw.items():
                if isinstance(value, torch.Tensor):
                    cpu = value.detach().float().cpu()
                    row[key] = (float(cpu.item()) if cpu.numel() == 1
                                else [float(x) for x in cpu.flatten().tolist()])
                else:
                    row[key] = value
            records.append(row)
        cfg = self.config
        return {"routing_mode": "fc_pasm_swap",
                "config": {f: (list(getattr(cfg, f)) if f == "active_layers" else getattr(cfg, f))
                           for f in cfg.__dataclass_fields__},
                "records": records}

    def reset(self) -> None:
        self._records.clear()
