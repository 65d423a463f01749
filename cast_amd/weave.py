"""The compact woven layer's attention on the HIP path: a drop-in for
``MatrixCurvaturePhaseFrameWeave._compact_cwca_attention``
(P/matrix_curvature_phase_frame_weave.py:5643-6124).

``compact_cwca_attention(weave, module, q, k, v, layout)`` has the method's
arguments (``weave`` is its ``self``) and result (``module.o`` of the
token-major attention output), reads the same weave attributes at call time
(``geometry_provider``, ``sparse_density``, ``fc_pasm_swap_router``,
``world_spectral_corrector``, ``routing_skip_inactive_layers``,
``current_segment_boundary``, ``routing_pair_alias_max_distance``,
``routing_mode``, ``_current_curvature``) and sets ``_last_compact_attention``.
One call composes:

* the pooling pass over the layout's slot map (``rcsa_pool_query_key``; with
  the pooled V ``v_content`` in the same launch when the router will refine,
  ``rcsa_pool_query_key_value``), the cosine block scores
  (``rcsa_block_scores``);
* the layer's degrees: memory rows ``mean_degree``, current rows from the
  closed-loop provider's ``compact_closed_loop_degrees`` (with
  :class:`cast_amd.closed_loop.DeviceClosedLoopBudget` on the device) or, for
  other providers, from the current curvature as the reference does it;
* the top-k of every row at its own degree with the local stencil forced
  (``rcsa_select_topk``, per-row k, descending score);
* the FC-PASM router's three cases (V21 bypass, inactive layer, refine with
  the previous layer's transport and its endpoint aliasing);
* the block-sparse attention over the slot maps with the output written to the
  token rows (``rcsa_sparse_attn_bf16``; int8 Q/K with ``weave.rcsa_int8_qk``).

With the closed-loop provider of the device, a layer the router does not
refine reads nothing back to the host: ``minimum_degree`` / ``maximum_degree``
of ``_last_compact_attention`` stay device scalars (``int()`` reads them), and
the provider's records keep theirs until its ``summary()``.
"""
from __future__ import annotations

import math
from bisect import bisect_left
from typing import Any, Optional

import torch

from . import layout as rlayout
from . import ops


def _cache(layout, device: torch.device) -> dict:
    """Slot map, block grid and local stencil of a compact layout, kept on
    the layout object (the reference caches the layout itself per chunk)."""
    key = str(device)
    store = getattr(layout, "_rcsa_cache", None)
    if store is None:
        store = {}
        try:
            layout._rcsa_cache = store
        except AttributeError:  # a frozen layout: no cache
            pass
    if key in store:
        return store[key]
    packed = layout.compact_block_indices
    blocks, bs = int(packed.shape[0]), int(packed.shape[1])
    tt, th, tw = (int(x) for x in layout.compact_block_shape)
    nh = math.ceil(layout.spatial_height / th)
    nw = math.ceil(layout.spatial_width / tw)
    spatial = nh * nw
    cells = blocks // spatial
    # widest row of the Manhattan <= 1 stencil on the full (cell, h, w) grid
    widest = 1 + sum(min(2, n - 1) for n in (cells, nh, nw))
    slot = packed.reshape(-1).to(device=device, dtype=torch.int32).contiguous()
    entry = {"slot": slot, "blocks": blocks, "block_size": bs, "shape": (tt, th, tw),
             "nh": nh, "nw": nw, "spatial": spatial, "local_degree": widest,
             "local": rlayout.local_stencil(blocks, nh, nw, device)}
    store[key] = entry
    return entry


def _closed_loop_provider(weave):
    p = weave.geometry_provider
    if getattr(p, "mode", None) == "closed_loop" and hasattr(p, "compact_closed_loop_degrees"):
        return p
    return None


def _curvature_degrees(weave, degrees, layout, blocks, memory_blocks, spatial, tt,
                       mean_degree, base, active_current_local, current_frames):
    """The current rows' degrees without a closed-loop provider: base + the
    largest-remainder split of the residual by 1 + log1p of the normalised
    per-cell curvature (P/matrix_curvature_phase_frame_weave.py:5769-5806), on
    the host as in the reference (this path is not CAST's configuration)."""
    current_blocks = blocks - memory_blocks
    residual = current_blocks * (mean_degree - base)
    curvature = weave._current_curvature(layout.total_temporal - layout.memory_temporal)
    if curvature is None or current_frames <= 0:
        return
    frame_weight = curvature.to(degrees.device)[active_current_local.to(degrees.device)]
    time_cells = current_blocks // spatial
    cell_weight = []
    for cell in range(time_cells):
        low, high = cell * tt, min(current_frames, (cell + 1) * tt)
        cell_weight.append(frame_weight[low:high].mean() if low < high else frame_weight.mean())
    weight = torch.stack(cell_weight)[:, None].expand(-1, spatial)
    weight = 1.0 + torch.log1p(weight / weight.mean().clamp_min(1e-8))
    raw = residual * weight.reshape(-1) / weight.sum().clamp_min(1e-8)
    bonus = torch.floor(raw).long()
    left = residual - int(bonus.sum().item())
    if left > 0:
        order = torch.argsort(raw - bonus, descending=True, stable=True)
        bonus[order[:left]] += 1
    degrees[memory_blocks:] = base + bonus


def _saturate(degrees, blocks, mean_degree):
    """Clamp rows to the block count and hand the overflow back
    (P/matrix_curvature_phase_frame_weave.py:5807-5817), on the host."""
    degrees.clamp_(max=blocks)
    missing = blocks * mean_degree - int(degrees.sum().item())
    while missing > 0:
        candidates = torch.nonzero(blocks - degrees > 0).flatten()
        if not int(candidates.numel()):
            break
        take = min(missing, int(candidates.numel()))
        degrees[candidates[:take]] += 1
        missing -= take


def _transport_with_aliases(weave, transport, layout, active_current_values):
    """The previous layer's transport with missing endpoint pairs aliased to the
    nearest published pair of the same current segment
    (P/matrix_curvature_phase_frame_weave.py:5969-6031)."""
    aliases: list = []
    if not isinstance(transport, dict):
        return transport, aliases
    previous_pairs = transport.get("pairs", {})
    if not (isinstance(previous_pairs, dict) and previous_pairs):
        return transport, aliases
    boundary = int(weave.current_segment_boundary or 4)
    local = tuple(int(v) - int(layout.memory_temporal) for v in active_current_values)
    current_pairs = [(l, r) for l, r in zip(local, local[1:])
                     if r - l > 1 and (l < boundary) == (r < boundary)]
    missing = [p for p in current_pairs if p not in previous_pairs]
    if not missing:
        return transport, aliases
    candidates = [p for p in previous_pairs
                  if isinstance(p, tuple) and len(p) == 2 and int(p[1]) > int(p[0])
                  and (int(p[0]) < boundary) == (int(p[1]) < boundary)]
    if not candidates:
        return transport, aliases
    transport = dict(transport)
    transport["pairs"] = dict(previous_pairs)
    for pair in missing:
        source = min(candidates, key=lambda c: (
            abs(int(c[0]) - int(pair[0])) + abs(int(c[1]) - int(pair[1])),
            abs((int(c[0]) + int(c[1])) - (int(pair[0]) + int(pair[1]))),
            int(c[0]), int(c[1])))
        limit = weave.routing_pair_alias_max_distance
        if limit >= 0 and max(abs(int(source[0]) - int(pair[0])),
                              abs(int(source[1]) - int(pair[1]))) > limit:
            continue
        transport["pairs"][pair] = previous_pairs[source]
        aliases.append({"requested": pair, "source": source})
    return transport, aliases


def _available_layers(weave):
    cache = getattr(weave.world_spectral_corrector, "_fc_routing_transport", {})
    step = int(getattr(weave.world_spectral_corrector, "_step", -1))
    return step, sorted(int(k[1]) for k in cache
                        if isinstance(k, tuple) and len(k) == 2 and int(k[0]) == step)


def _attention(q, k, v, idx4, cnt3, slot, token_to_packed, mask, bs, int8: bool, kq=None):
    """Block-sparse attention of the packed blocks named by the slot map, the
    output in the token rows [B, L, H, D] (bf16).  The copy rings read the
    token-major sources through the slot map for D 128 and 128-token blocks;
    other shapes are packed first."""
    B, L, H, D = q.shape
    ring = D == 128 and bs == 128
    vb = v if v.dtype == torch.bfloat16 else v.to(torch.bfloat16)
    if int8:
        q_i8, q_scale, k_i8, k_scale = kq
        return ops.sparse_attn_int8(q_i8, q_scale, k_i8, k_scale,
                                    vb if ring else ops.pack_tokens(vb, slot), idx4, cnt3, None,
                                    block_m=bs, block_n=bs, block_mask=mask, out_token=slot,
                                    out_len=L, v_token=slot if ring else None)
    qb, kb = (x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16) for x in (q, k))
    if ring:
        return ops.sparse_attn_bf16(qb, kb, vb, idx4, cnt3, None, block_m=bs, block_n=bs,
                                    block_mask=mask, q_token=slot, kv_token=slot)
    packed = [ops.pack_tokens(x, slot) for x in (qb, kb, vb)]
    out = ops.sparse_attn_bf16(*packed, idx4, cnt3, None, block_m=bs, block_n=bs,
                               block_mask=mask)
    return ops.unpack_tokens(out, token_to_packed.to(device=q.device, dtype=torch.long))


def compact_cwca_attention(weave, module: Any, q: torch.Tensor, k: torch.Tensor,
                           v: torch.Tensor, layout) -> torch.Tensor:
    """``_compact_cwca_attention`` (P/matrix_curvature_phase_frame_weave.py:5643-6124)
    on the HIP kernels.  q, k, v: token-major ``[B, L, H, D]`` (bf16 or fp32) of the
    compact frames; ``layout``: the weave's ``_FrameLayout`` with its compact block
    map.  Returns ``module.o`` of the attention output."""
    provider = _closed_loop_provider(weave)
    layer_index = int(getattr(module, "block_idx", -1))
    if provider is not None:
        if layer_index < 0:
            raise RuntimeError("compact Closed-Loop CWCA lacks a layer index")
        provider.begin_compact_layer(layer_index)
    if (layout.compact_block_indices is None or layout.compact_block_valid is None
            or layout.compact_token_to_packed is None):
        raise RuntimeError("compact CWCA layout was not constructed")
    if layout.compact_block_shape is None:
        raise RuntimeError("compact CWCA block shape is missing")
    dev = q.device
    c = _cache(layout, dev)
    bs, blocks, spatial = c["block_size"], c["blocks"], c["spatial"]
    if bs != int(layout.packed_block_size):
        raise RuntimeError("compact CWCA block size differs from the packed layout")
    tt = c["shape"][0]
    B, L, H, D = q.shape
    slot, local = c["slot"], c["local"]
    compact_frames = len(layout.active_frame_values)
    memory_frames = bisect_left(layout.active_frame_values, int(layout.memory_temporal))
    expected_cells = math.ceil(memory_frames / tt) + math.ceil((compact_frames - memory_frames) / tt)
    if blocks != expected_cells * spatial:
        raise RuntimeError("compact CWCA block-grid cardinality mismatch")

    # ---- degrees (P/matrix_curvature_phase_frame_weave.py:5727-5817) ----
    local_degree = c["local_degree"]
    mean_degree = min(max(local_degree, int(round(weave.sparse_density * blocks))), blocks)
    memory_cells = math.ceil(memory_frames / tt)
    memory_blocks = min(blocks, memory_cells * spatial)
    current_blocks = blocks - memory_blocks
    active_current_values = tuple(int(x) for x in layout.active_frame_values
                                  if int(x) >= int(layout.memory_temporal))
    degrees = torch.full((blocks,), mean_degree, device=dev, dtype=torch.long)
    width = mean_degree  # a bound of every row's degree, known on the host
    metadata = None
    host_degrees = provider is None
    if current_blocks > 0 and mean_degree > local_degree:
        base = max(local_degree, math.ceil(4 * mean_degree / 5))
        current_frames = compact_frames - memory_frames
        cells = current_blocks // spatial
        if provider is not None:
            active_current = torch.tensor(active_current_values, dtype=torch.long)
            current, metadata = provider.compact_closed_loop_degrees(
                layer_index=layer_index, active_current=active_current,
                current_frame_origin=layout.memory_temporal, temporal_group_size=tt,
                spatial_blocks=spatial, mean_degree=mean_degree, base_degree=base,
                total_blocks=blocks, memory_blocks=memory_blocks)
            if int(current.numel()) != current_blocks:
                raise RuntimeError("compact Closed-Loop degree layout differs from packed rows")
            degrees[memory_blocks:] = current.reshape(-1).to(device=dev, dtype=torch.long)
            # every row keeps base, and a worldline's cells share cells * mean edges
            width = max(mean_degree, min(blocks, base + cells * (mean_degree - base)))
        else:
            active_local = torch.tensor(active_current_values, dtype=torch.long) - \
                int(layout.memory_temporal)
            _curvature_degrees(weave, degrees, layout, blocks, memory_blocks, spatial, tt,
                               mean_degree, base, active_local, current_frames)
    if host_degrees:
        _saturate(degrees, blocks, mean_degree)
        width = int(degrees.max().item())
    # With a closed-loop provider the saturation of :5807-5817 changes nothing:
    # its rows never exceed the block count (memory rows hold mean_degree, the
    # current ones are capped at total_blocks by _redistribute_compact_capacity)
    # and they sum to blocks * mean_degree (each worldline keeps cells * mean).
    if provider is not None:
        if metadata is None:
            raise RuntimeError("compact Closed-Loop CWCA did not allocate a feedback budget")
        provider.record_compact_budget(metadata, degrees, local_support_preserved=True,
                                       native_qk_topk=True)
    width = min(max(width, 1), blocks)

    # ---- router case (P/matrix_curvature_phase_frame_weave.py:5833-6085) ----
    router = weave.fc_pasm_swap_router
    corrector = weave.world_spectral_corrector
    route = None
    if router is not None:
        if corrector is not None and bool(getattr(corrector, "fc_v21_bypass", False)):
            route = "bypass"
        elif corrector is None:
            raise RuntimeError("FC-PASM routing has no spectral corrector")
        else:
            active_layers = tuple(int(x) for x in router.config.active_layers)
            if (weave.routing_skip_inactive_layers and active_layers
                    and layer_index not in active_layers):
                route = "inactive"
            else:
                route = "refine"
    transport = aliases = None
    if route == "refine":
        transport = corrector.fc_pasm_routing_transport(layer_index=layer_index)
        transport, aliases = _transport_with_aliases(weave, transport, layout,
                                                     active_current_values)
    # the pooled V only when refine can use it (a transport to consult, or
    # a router that propagates without one)
    need_v = route == "refine" and (isinstance(transport, dict)
                                    or not router.config.require_fc_transport)

    # ---- pooling, scores (P/matrix_curvature_phase_frame_weave.py:5677-5701) ----
    int8 = bool(getattr(weave, "rcsa_int8_qk", False))
    kq = None
    vmean = None
    if need_v:
        pooled = ops.pool_query_key_value(q, None, k, None, v, bs, q_slot_token=slot,
                                          k_slot_token=slot, quantize=int8)
        qhat, q_i8, q_scale, khat, ksum, kmin, kmax, mask, vmean = pooled
    else:
        qhat, q_i8, q_scale, khat, ksum, kmin, kmax, mask = ops.pool_query_key(
            q, None, k, None, bs, q_slot_token=slot, k_slot_token=slot, quantize=int8)
    score = ops.block_scores(qhat, khat)                          # [B*H, N, N]
    if int8:
        k_i8, k_scale, _ = ops.quantize_key(k, None, bs, ksum, kmin, kmax, slot_token=slot)
        kq = (q_i8, q_scale, k_i8, k_scale)

    # ---- top-k at each row's degree, local blocks first (:5829-5832) ----
    row_k = degrees.to(torch.int32)
    indices, _ = ops.select_topk(score, row_k, forced=local, max_k=width, order="rank")
    selected = indices.view(B, H, blocks, width)
    counts = row_k[None, None].expand(B, H, -1).contiguous()

    routing_record: Optional[dict] = None
    if route == "bypass":
        routing_record = {"layer_index": layer_index, "status": "independent_topk_fallback",
                          "fallback_reason": "fc_v21_bypass", "swap_count": 0,
                          "fc_cache_used": False, "g0_fallback": True, "fixed_budget": True,
                          "fc_v21_bypass": True}
        router._records.append(routing_record)
    elif route == "inactive":
        step, available = _available_layers(weave)
        routing_record = {"layer_index": layer_index, "status": "independent_topk_fallback",
                          "fallback_reason": "layer_not_enabled", "swap_count": 0,
                          "transport_query_step": step,
                          "transport_query_source_layer": layer_index - 1,
                          "transport_available_layers": available,
                          "transport_pair_aliases": [], "fc_cache_used": False,
                          "fixed_budget": True, "routing_skip_inactive_layers": True}
        router._records.append(routing_record)
    elif route == "refine":
        step, available = _available_layers(weave)
        if transport is not None:
            transport = dict(transport)
            transport["attention_spatial_h"] = c["nh"]
            transport["attention_spatial_w"] = c["nw"]
        exact = tuple(int(x) - int(layout.memory_temporal) for x in active_current_values)
        if vmean is None:
            vmean = torch.zeros(B * H, blocks, D, device=dev, dtype=torch.float32)
        # the router receives score + 1e6 local - 1e6 local (fp32), as the
        # reference passes it back after its top-k bonus (:6037, :5829)
        bonus = local.to(score.dtype) * 1e6
        router_score = ((score.view(B, H, blocks, blocks) + bonus) - bonus)
        selected, routing_record = router.refine(
            score=router_score, pooled_value=vmean.view(B, H, blocks, D), selected=selected,
            counts=counts, local=local, memory_blocks=memory_blocks, spatial_shape=(c["nh"],
                                                                                    c["nw"]),
            exact_current_frames=exact, temporal_group_size=tt,
            current_boundary=weave.current_segment_boundary or 4, transport=transport,
            layer_index=layer_index)
        routing_record = dict(routing_record)
        routing_record.update({"transport_query_step": step,
                               "transport_query_source_layer": layer_index - 1,
                               "transport_available_layers": available})
        records = getattr(router, "_records", None)
        if isinstance(records, list) and records:
            records[-1].update({"transport_query_step": step,
                                "transport_query_source_layer": layer_index - 1,
                                "transport_available_layers": available,
                                "transport_pair_aliases": aliases or []})

    # ---- attention and unpack (:6086-6095) ----
    out = _attention(q, k, v, selected.to(torch.int32).contiguous(), counts, slot,
                     layout.compact_token_to_packed, mask, bs, int8, kq)
    if provider is not None:  # the closed loop conserves blocks * mean_degree edges
        edges, mean_f = blocks * mean_degree, float(mean_degree)
    else:
        edges, mean_f = int(degrees.sum().item()), float(degrees.float().mean().item())
    weave._last_compact_attention = {
        "compact_blocks": blocks,
        "requested_density": weave.sparse_density,
        "mean_degree": mean_f,
        "minimum_degree": degrees.min(),
        "maximum_degree": degrees.max(),
        "edge_budget": edges,
        "effective_density": edges / float(blocks * blocks),
        "empty_blocks": 0,
        "budget_source": metadata["source"] if metadata is not None else "compact_curvature",
        "closed_loop_previous_layer": metadata["previous_layer"] if metadata is not None
        else None,
        "closed_loop_feedback_consumed": metadata is not None
        and metadata["previous_layer"] is not None,
        "native_qk_topk": True,
        "local_support_preserved": True,
        "routing_mode": weave.routing_mode,
        "routing": routing_record,
    }
    return module.o(out.flatten(2).to(q.dtype))
