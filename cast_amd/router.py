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
from dataclasses import dataclass
from typing import Any, Callable, Optional

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
    def _f32(x: float) -> torch.Tensor:
        return torch.tensor(x, dtype=torch.float32)

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

    def _terms(self, error, cells, spatial, frames, group, boundary, transport):
        """Quadratic coefficient (per row) and linear term (per row and group)
        of the objective at ``error`` (P/fc_pasm_swap_routing.py:414-547)."""
        cfg = self.config
        BH, rows, G = error.shape
        view = error.reshape(BH, cells, spatial, G)
        cell = self._cells(frames, group, cells)
        count = [0.0] * cells
        for f in frames:
            count[cell[int(f)]] += 1.0
        coef = (torch.tensor(count, dtype=torch.float32, device=error.device)[:, None]
                .expand(-1, spatial).clone() * cfg.lambda_anchor)
        lin = torch.zeros_like(view)
        used = False
        shape = self._grid(transport, spatial)
        for left, right in self._pairs(frames, boundary):
            lc, rc = cell[left], cell[right]
            el, er = view[:, lc], view[:, rc]
            for target in range(left + 1, right):
                a = float(target - left) / float(right - left)
                lm = self._matrix(transport, (left, right), shape, a, error.device)
                rm = self._matrix(transport, (left, right), shape, -(1.0 - a), error.device)
                lam = cfg.lambda_reconstruction
                if lm is None and rm is None:
                    # identity operators (g = 0): the same products in fp32 scalars
                    wl, wr, la = self._f32(1.0 - a), self._f32(a), self._f32(lam)
                    if lc == rc:
                        c = wl + wr
                        coef[lc] += float(la * (c * c))
                    else:
                        coef[lc] += float(la * (wl * wl))
                        coef[rc] += float(la * (wr * wr))
                        x = float(la * (wl * wr))
                        lin[:, lc] += x * er
                        lin[:, rc] += x * el
                    continue
                used = True
                eye = torch.eye(spatial, device=error.device, dtype=torch.float32)
                lm = eye if lm is None else lm
                rm = eye if rm is None else rm
                lo, ro = (1.0 - a) * lm, a * rm
                if lc == rc:
                    comb = lo + ro
                    hess = lam * (comb.T @ comb)
                    dg = torch.diagonal(hess)
                    coef[lc] += dg
                    lin[:, lc] += torch.einsum("st,btg->bsg", hess, el) - dg[None, :, None] * el
                else:
                    hl, hr, hx = lam * (lo.T @ lo), lam * (ro.T @ ro), lam * (lo.T @ ro)
                    dl, dr = torch.diagonal(hl), torch.diagonal(hr)
                    coef[lc] += dl
                    coef[rc] += dr
                    lin[:, lc] += (torch.einsum("st,btg->bsg", hl, el) - dl[None, :, None] * el
                                   + torch.einsum("st,btg->bsg", hx, er))
                    lin[:, rc] += (torch.einsum("st,btg->bsg", hr, er) - dr[None, :, None] * er
                                   + torch.einsum("st,btg->bsg", hx.T, el))
        return coef.reshape(rows), lin.reshape(BH, rows, G), used

    def _value(self, error, cells, spatial, frames, group, boundary, transport):
        """The objective (P/fc_pasm_swap_routing.py:550-614)."""
        cfg = self.config
        BH, rows, G = error.shape
        view = error.reshape(BH, cells, spatial, G)
        cell = self._cells(frames, group, cells)
        count = [0.0] * cells
        for f in frames:
            count[cell[int(f)]] += 1.0
        cw = torch.tensor(count, dtype=torch.float32, device=error.device)
        value = cfg.lambda_anchor * (view.square() * cw[None, :, None, None]).sum()
        shape = self._grid(transport, spatial)
        for left, right in self._pairs(frames, boundary):
            el, er = view[:, cell[left]], view[:, cell[right]]
            for target in range(left + 1, right):
                a = float(target - left) / float(right - left)
                lm = self._matrix(transport, (left, right), shape, a, error.device)
                rm = self._matrix(transport, (left, right), shape, -(1.0 - a), error.device)
                pl = el if lm is None else torch.einsum("st,btg->bsg", lm, el)
                pr = er if rm is None else torch.einsum("st,btg->bsg", rm, er)
                prop = (1.0 - a) * pl + a * pr
                value = value + cfg.lambda_reconstruction * prop.square().sum()
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
            gate = cg.repeat_interleave(spatial).to(score.device)

        dev = score.device
        K = selected.shape[-1]
        cnt = counts.clamp(0, K).to(torch.int32)
        sel = selected.to(torch.int32).contiguous()
        valid = torch.arange(K, device=dev)[None, None, None] < cnt[..., None]
        hist_before = ((sel < M) & valid).sum(-1)
        max_swappable = int(cnt.max().item())
        if max_swappable == 0:
            return baseline, self._fallback(layer_index, "no_swappable_kv_selected")
        L = min(N, cfg.candidate_multiplier * max_swappable)
        cand, proxy, error = ops.route_proxy(
            score, pooled_value, local, sel, cnt, memory_blocks=M, n_cand=L,
            cand_mult=cfg.candidate_multiplier, sketch_groups=cfg.sketch_groups)
        geo = (cells, spatial, frames, int(temporal_group_size), int(current_boundary), transport)
        obj_before = self._value(error, *geo)
        cache_used = bool(matching)
        swaps, improvements = 0, []
        for _ in range(cfg.num_swap_rounds):
            coef, lin, used = self._terms(error, *geo)
            cache_used = cache_used or used
            best, flat = ops.route_best_swap(proxy, cand, local, sel, cnt, coef, lin, error,
                                             memory_blocks=M, cand_mult=cfg.candidate_multiplier,
                                             same_bank=cfg.same_bank_only, row_gate=gate)
            strongest = int(torch.argmin(best.reshape(-1)).item())
            value = float(best.reshape(-1)[strongest].item())
            if cfg.max_swaps_per_call and swaps >= cfg.max_swaps_per_call:
                break
            if not value < -cfg.swap_eps:
                break
            bh, rr = divmod(strongest, rows)
            fl = int(flat[bh, rr].item())
            slot, pos = divmod(fl, L)
            b, h = divmod(bh, H)
            row = M + rr
            removed = sel[b, h, row, slot]
            hit = (cand[bh, rr] == removed).nonzero()
            rem = proxy[bh, rr, int(hit[0, 0])] if hit.numel() else torch.zeros_like(proxy[bh, rr, 0])
            sel[b, h, row, slot] = cand[bh, rr, pos]
            error = error.clone()
            error[bh, rr] += rem - proxy[bh, rr, pos]
            swaps += 1
            improvements.append(-value)

        valid_final = valid
        hist_after = ((sel < M) & valid_final).sum(-1)
        if cfg.same_bank_only and not torch.equal(hist_before, hist_after):
            raise RuntimeError("same-bank FC-PASM routing changed Memory KV counts")
        s64 = sel.long()
        # duplicates among a row's kept entries: equal neighbours once sorted
        # (padding slots become distinct values past every block)
        pad = N + torch.arange(K, device=dev)
        srt = torch.where(valid_final, s64, pad).sort(dim=-1).values
        if bool((srt[..., 1:] == srt[..., :-1]).any()):
            raise RuntimeError("FC-PASM routing emitted duplicate keys")
        loc = local.to(device=dev, dtype=torch.bool)
        final_local = torch.gather(loc[None, None].expand(B, H, -1, -1), -1,
                                   s64.clamp_min(0)) & valid_final
        if int(final_local.sum().item()) != int(loc.sum().item()) * B * H:
            raise RuntimeError("FC-PASM routing removed a protected local edge")
        obj_after = self._value(error, *geo)
        if bool(obj_after > obj_before + 1e-5 * obj_before.abs().clamp_min(1.0)):
            raise RuntimeError("FC-PASM swap increased its refinement objective")
        record = {
            "layer_index": int(layer_index), "status": "refined",
            "candidate_multiplier": cfg.candidate_multiplier, "candidate_max": L,
            "swap_rounds": cfg.num_swap_rounds, "max_swaps_per_call": cfg.max_swaps_per_call,
            "swap_count": swaps, "objective_before": obj_before.detach(),
            "objective_after": obj_after.detach(),
            "objective_improvement": (obj_before - obj_after).detach(),
            "average_swap_improvement": (sum(improvements) / swaps if swaps else 0.0),
            "anchor_term_weight": cfg.lambda_anchor,
            "reconstruction_term_weight": cfg.lambda_reconstruction,
            "reconstruction_terms": sum(max(0, r - l - 1) for l, r in zip(frames, frames[1:])
                                        if (l < current_boundary) == (r < current_boundary)),
            "fc_cache_used": cache_used, "matching_transport_affinity": affinity,
            "min_pair_transport_affinity": cfg.min_pair_transport_affinity,
            "pair_gate_cells": gate_cells, "g0_fallback": not cache_used, "fixed_budget": True,
            "historical_only": cfg.historical_only, "same_bank_only": cfg.same_bank_only,
            "historical_budget_before": int(hist_before.sum().item()),
            "historical_budget_after": int(hist_after.sum().item()),
            "minimum_k": int(counts.min().item()), "maximum_k": int(counts.max().item()),
            "budget_before": int(counts.sum().item()), "budget_after": int(counts.sum().item()),
            "unique_indices": True, "local_support_preserved": True,
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
