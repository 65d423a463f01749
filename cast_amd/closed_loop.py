"""The closed-loop compiler's compact budget on the device.

``DeviceClosedLoopBudget`` is a mixin for ``MatrixClosedLoopCWCAAttentionCompiler``
(P/control_response_cwca_attention.py:2083-2099).  It overrides the two methods
the compact woven layer calls per layer
(P/matrix_curvature_phase_frame_weave.py:5754-5767, 5820-5828):

* ``compact_closed_loop_degrees`` (:1188-1363) returns the same
  ``([Tc, S] degrees, metadata)`` pair, the degrees computed by
  ``rcsa_closed_loop_degrees`` on the device.  The checks the reference makes on
  host values (mode, layer chronology, curvature, spatial worldlines, the
  active frames against the memory origin and the frame capacity, the previous
  layer's response) raise the reference's errors at the call.  The allocator's
  own breaches (a frame past the curvature tiles, a worldline with no capacity
  left) become bits of a device status word instead of host reads; they are
  raised with the reference's messages by ``check_compact_status`` (called by
  ``summary``).
* ``record_compact_budget`` (:1365-1387) keeps the reference's record.  The
  degree statistics (``k_min``, ``k_max``, ``k_mean``) and the curvature and
  response statistics of the metadata stay device scalars until ``summary``
  materialises them, as the reference's own records of the native path do
  (``global_edge_budget`` at :1522-1526).

So a compact layer reads nothing back to the host.  The metadata's keys and
values, the records and ``summary()`` are the reference's once materialised.
"""
from __future__ import annotations

from typing import Any

import torch

from . import ops

_STATUS_ERRORS = ((1, "compact Current frame lies outside CWCA tiles"),
                  (4, "compact Closed-Loop Current set contains Memory frames"),
                  (2, "compact Closed-Loop CWCA exhausted key capacity"))


class _DeviceStats:
    """min / max / mean / std (population) of a device tensor, computed when
    read (``_stats`` of P/control_response_cwca_attention.py:1532-1541)."""

    def __init__(self, value: torch.Tensor):
        self.value = value

    def resolve(self) -> dict:
        v = self.value.float()
        return {"min": float(v.min()), "max": float(v.max()), "mean": float(v.mean()),
                "std": float(v.std(unbiased=False))}


def _time_cells(values: torch.Tensor, local, compact_group: int, source_group: int,
                offset: int) -> torch.Tensor:
    """``_compact_time_cells`` (P/control_response_cwca_attention.py:1123-1163) on the
    values' device with the frames on the host: frame f >= offset reads tile
    (f - offset) // source_group, earlier frames read 0, and each run of
    compact_group frames is averaged.  No host read-back."""
    rows = []
    for lo in range(0, len(local), compact_group):
        group = local[lo:lo + compact_group]
        tiles = [(f - offset) // source_group for f in group if f >= offset]
        if tiles:
            idx = torch.tensor(tiles, dtype=torch.long).pin_memory().to(values.device,
                                                                       non_blocking=True)
            rows.append(values.index_select(0, idx).sum(0) / float(len(group)))
        else:
            rows.append(torch.zeros(values.shape[1], device=values.device, dtype=values.dtype))
    return torch.stack(rows)


class DeviceClosedLoopBudget:
    """Mixin: put it before ``MatrixClosedLoopCWCAAttentionCompiler`` in the bases."""

    def compact_closed_loop_degrees(self, *, layer_index: int, active_current,
                                    current_frame_origin: int, temporal_group_size: int,
                                    spatial_blocks: int, mean_degree: int, base_degree: int,
                                    total_blocks: int, memory_blocks: int
                                    ) -> tuple[torch.Tensor, dict[str, Any]]:
        layer_index = int(layer_index)
        if self.mode != "closed_loop":
            raise RuntimeError("compact feedback is defined for Closed-Loop CWCA")
        if self._compact_layer_index != layer_index or self._layer_index != layer_index:
            raise RuntimeError("compact Closed-Loop layer was not entered")
        curvature = self._curvature_matrix
        if curvature is None:
            raise RuntimeError("compact Closed-Loop CWCA has no curvature prior")
        if int(curvature.shape[1]) != int(spatial_blocks):
            raise RuntimeError("compact Closed-Loop spatial worldlines differ from CWCA")
        origin = int(current_frame_origin)
        frames = [int(f) for f in torch.as_tensor(active_current).reshape(-1).tolist()]
        if not frames:
            raise RuntimeError("compact Closed-Loop has no active Current frames")
        if any(f < origin for f in frames):
            raise RuntimeError("compact Closed-Loop Current set contains Memory frames")
        local = [f - origin for f in frames]
        offset = int(self._current_temporal_offset)
        source_group = int(self._block_shape[0])
        capacity = offset + int(curvature.shape[0]) * source_group
        if any(f >= capacity for f in local):
            raise RuntimeError("compact Current frame lies outside CWCA frame capacity")
        group = int(temporal_group_size)
        cells = -(-len(local) // group)
        spatial = int(spatial_blocks)
        if cells * spatial != int(total_blocks) - int(memory_blocks):
            raise RuntimeError("compact Closed-Loop degree layout differs from packed rows")
        dev = curvature.device if curvature.is_cuda else torch.device("cuda")
        curv = curvature.to(device=dev, dtype=torch.float32)
        eps = torch.finfo(torch.float32).eps
        normalized = curv / curv.mean(dim=0, keepdim=True).clamp_min(eps)
        compact_curvature = _time_cells(normalized, local, group, source_group, offset)
        response = None
        response_weight = 0.0
        feedback = self.feedback_form
        fixed = bool(self.fixed_query_budget)
        response_stats: Any = {"min": None, "max": None, "mean": None, "std": None}
        if fixed:
            source, previous = "compact_light_interaction_fixed_query_budget", None
        elif layer_index == 0:
            source, previous = "compact_cwca_curvature_bootstrap", None
        elif self.response_weight == 0.0:
            source, previous = "compact_curvature_only_response_weight_0", None
        else:
            resp = self._responses.get(layer_index - 1)
            if resp is None:
                raise RuntimeError(f"compact layer {layer_index} has no response from layer "
                                   f"{layer_index - 1}")
            response = resp.to(device=dev, dtype=torch.float32)
            response_weight = float(self.response_weight)
            source = (f"compact_{feedback}_curvature_control_response_"
                      f"lambda_{self.response_weight:g}")
            previous = layer_index - 1
            response_stats = _DeviceStats(
                _time_cells(response, local, group, source_group, offset))
        degrees, status = ops.closed_loop_degrees(
            curv, local, current_temporal_offset=offset, source_group=source_group,
            compact_group=group, mean_degree=int(mean_degree), base_degree=int(base_degree),
            total_blocks=int(total_blocks), memory_blocks=int(memory_blocks),
            response=response, response_weight=response_weight, feedback_form=feedback,
            fixed_query_budget=fixed, check_status=False)
        pending = getattr(self, "_rcsa_pending_status", None)
        if pending is None:
            pending = self._rcsa_pending_status = []
        pending.append(status)
        current = degrees[int(memory_blocks):].view(cells, spatial).long()
        worldline = cells * int(mean_degree)
        current_edges = cells * spatial * int(mean_degree)
        metadata = {
            "call": self._call_index,
            "layer": layer_index,
            "source": source,
            "previous_layer": previous,
            "active_current_global_frames": frames,
            "active_current_local_frames": local,
            "current_frame_origin": origin,
            "native_current_temporal_offset": offset,
            "compact_time_cells": cells,
            "spatial_worldlines": spatial,
            "response": response_stats,
            "curvature": _DeviceStats(compact_curvature),
            "current_worldline_budget": worldline,
            "current_edge_budget": current_edges,
            "global_edge_budget": int(memory_blocks) * int(mean_degree) + current_edges,
            "reference_edge_budget": int(total_blocks) * int(mean_degree),
        }
        if fixed:
            metadata["uniform_query_budget"] = True
        return current, metadata

    def record_compact_budget(self, metadata: dict[str, Any], degrees: torch.Tensor, *,
                              local_support_preserved: bool, native_qk_topk: bool) -> None:
        record = dict(metadata)
        d = degrees.detach()
        record.update({
            "k_min": d.min(), "k_max": d.max(), "k_mean": d.float().mean(),
            "budget_exact": metadata["global_edge_budget"] == metadata["reference_edge_budget"],
            "local_support_preserved": bool(local_support_preserved),
            "native_qk_topk": bool(native_qk_topk),
        })
        if not record["budget_exact"]:
            raise RuntimeError("compact Closed-Loop global edge certificate failed")
        self._compact_budget_records.append(record)

    def check_compact_status(self) -> None:
        """Read the device status words of the compact layers since the last
        check (one read) and raise the reference's error for a breach; resolve
        the records' device statistics."""
        pending = getattr(self, "_rcsa_pending_status", None) or []
        if pending:
            codes = torch.cat([s.reshape(-1) for s in pending]).cpu().tolist()
            pending.clear()
            for code in codes:
                for bit, msg in _STATUS_ERRORS:
                    if code & bit:
                        raise RuntimeError(msg)
        for record in self._compact_budget_records:
            for key in ("response", "curvature"):
                if isinstance(record.get(key), _DeviceStats):
                    record[key] = record[key].resolve()

    def summary(self) -> dict[str, Any]:
        self.check_compact_status()
        return super().summary()
