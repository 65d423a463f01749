"""The composed compact woven layer (cast_amd.weave.compact_cwca_attention, the
drop-in for _compact_cwca_attention, P/matrix_curvature_phase_frame_weave.py:
5643-6124) with the device closed-loop provider
(cast_amd.closed_loop.DeviceClosedLoopBudget, P/control_response_cwca_attention.py:
1188-1387) and the device router, against the oracle's composition
(orc.compact_cwca_layer: gathers, pooling, closed_loop_degrees, select_topk,
fc_pasm_refine, sparse_attention, scatter) on the Matrix latent grid (22 x 40
tokens per frame, (4, 4, 8) tiles with 64-token bottom tiles, 6 x 5 spatial
worldlines).

Stand-ins replace the reference's objects (its modules do not travel to the GPU
box): a compiler holding the attributes compact_closed_loop_degrees reads, a
weave holding the attributes _compact_cwca_attention reads, a spectral
corrector publishing one transport, and a module with block_idx and o.
"""
import math
from dataclasses import dataclass
from types import SimpleNamespace
from typing import Optional

import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu

HW, SHAPE, MEM_T, D, H = (22, 40), (4, 4, 8), 8, 128, 2
FRAMES = tuple(range(8)) + (8, 10, 11, 13, 14, 15)   # 8 memory + 6 current frames
T_SRC, OFFSET = 3, 1


@dataclass
class FrameLayout:
    """The fields of the weave's _FrameLayout (P/matrix_curvature_phase_frame_weave.py:50-68)
    that the compact attention reads."""
    total_temporal: int
    spatial_height: int
    spatial_width: int
    memory_temporal: int
    active_frames: torch.Tensor
    active_frame_values: tuple
    packed_block_size: int
    compact_block_indices: torch.Tensor
    compact_block_valid: torch.Tensor
    compact_token_to_packed: torch.Tensor
    compact_block_shape: tuple


class StandInCompiler:
    """The attributes and methods of MatrixControlResponseCWCAAttentionCompiler
    (P/control_response_cwca_attention.py:35-176, 1365-1387, 1532-1556,
    1911-1988) that the compact path uses."""

    def __init__(self, curvature, response_weight, feedback_form, fixed=False):
        self.mode = "closed_loop"
        self._curvature_matrix = curvature
        self._current_temporal_offset = OFFSET
        self._block_shape = (4, 1, 1)
        self.fixed_query_budget = fixed
        self.response_weight = response_weight
        self.feedback_form = feedback_form
        self._responses = {}
        self._call_index = 0
        self._layer_index = 0
        self._compact_layer_index = None
        self._compact_budget_records = []

    def begin_compact_layer(self, layer_index):
        if self._compact_layer_index is not None:
            raise RuntimeError("nested compact control-response layer")
        self._compact_layer_index = int(layer_index)
        self._layer_index = int(layer_index)

    def end_compact_layer(self, layer_index):
        self._compact_layer_index = None

    @classmethod
    def _materialize(cls, value):
        if isinstance(value, torch.Tensor) and value.numel() == 1:
            s = value.item()
            return bool(s) if value.dtype == torch.bool else (
                int(s) if not value.dtype.is_floating_point else float(s))
        if isinstance(value, dict):
            return {k: cls._materialize(v) for k, v in value.items()}
        if isinstance(value, list):
            return [cls._materialize(v) for v in value]
        return value

    def summary(self):
        return self._materialize({"compact_budget_records": self._compact_budget_records})


def _provider(curvature, response_weight=0.5, feedback_form="additive", fixed=False):
    from cast_amd.closed_loop import DeviceClosedLoopBudget

    class Provider(DeviceClosedLoopBudget, StandInCompiler):
        pass
    return Provider(curvature, response_weight, feedback_form, fixed)


def _layout(dev):
    from cast_amd.layout import compact_layout
    lay = compact_layout(FRAMES, MEM_T, *HW, SHAPE, dev)
    return FrameLayout(16, HW[0], HW[1], MEM_T, torch.tensor(FRAMES, device=dev), FRAMES,
                       lay.block_size, lay.block_indices, lay.block_valid,
                       lay.token_to_packed, SHAPE)


def _transport(seed):
    g = torch.Generator().manual_seed(seed)
    theta = (torch.rand(18, 6, 3, generator=g) * 2 - 1) * math.pi
    gain = torch.rand(18, 6, 3, generator=g)
    return {"output_shape": HW, "transport_shape": (6, 5), "window_shape": (11, 10),
            "stride": (8, 8), "padding": (4, 5), "tile_grid": (3, 6),
            "pairs": {(0, 2): {"theta": theta, "affinity": gain,
                               "mean_affinity": torch.tensor(0.9)}}}


def _oracle_operator(tr, shape=(6, 5)):
    S = shape[0] * shape[1]
    eye = torch.eye(S).reshape(S, 1, *shape)

    def op(pair, exponent):
        if pair not in tr["pairs"]:
            return None
        return (torch.eye(S) + orc.transport_maps(tr, pair, eye, exponent).reshape(S, S)).T
    return op


def _inputs(seed):
    g = torch.Generator().manual_seed(seed)
    L = len(FRAMES) * HW[0] * HW[1]
    q, k, v = (torch.randn(1, L, H, D, generator=g) / math.sqrt(D) for _ in range(3))
    # per-frame mean shifts, so that block scores have structure
    shift = torch.randn(len(FRAMES), 1, H, D, generator=g) * 0.3 / math.sqrt(D)
    k = (k.reshape(1, len(FRAMES), -1, H, D) + shift).reshape(1, L, H, D)
    curvature = torch.rand(T_SRC, 30, generator=g) + 0.05
    response = torch.rand(T_SRC, 30, generator=g) * 2
    return q.bfloat16(), k.bfloat16(), v.bfloat16(), curvature, response


def _weave(provider, router=None, transport=None, layer=1, int8=False):
    corrector = SimpleNamespace(
        fc_v21_bypass=False, _step=0, _fc_routing_transport={(0, layer - 1): transport},
        fc_pasm_routing_transport=lambda layer_index: transport)
    return SimpleNamespace(geometry_provider=provider, sparse_density=0.25,
                           fc_pasm_swap_router=router, world_spectral_corrector=corrector,
                           routing_skip_inactive_layers=True, current_segment_boundary=4,
                           routing_pair_alias_max_distance=-1, routing_mode="fc_pasm_swap",
                           _current_curvature=None, _last_compact_attention=None,
                           rcsa_int8_qk=int8)


def _oracle(q, k, v, lay, curvature, response, layer, weight=0.5, form="additive",
            router=None):
    return orc.compact_cwca_layer(
        q.float(), k.float(), v.float(), lay.compact_block_indices.cpu(), block_shape=SHAPE,
        spatial_hw=HW, active_frame_values=FRAMES, memory_temporal=MEM_T,
        sparse_density=0.25, layer_index=layer, router=router,
        closed_loop=dict(curvature=curvature, current_temporal_offset=OFFSET, source_group=4,
                         response=response if layer > 0 else None, response_weight=weight,
                         feedback_form=form))


def _check_out(got, want):
    st = orc.equivalence_stats(want.flatten(2), got.float().cpu())
    assert st["cosine"] >= 0.999 and st["max_abs"] <= 3e-2, st


def _check_sets(selected, counts, want):
    sel, cnt = selected.cpu().long(), counts.cpu().long()
    assert torch.equal(cnt, want["counts"].long())
    B, Hh, N, _ = sel.shape
    for h in range(Hh):
        for r in range(N):
            c = int(cnt[0, h, r])
            assert set(sel[0, h, r, :c].tolist()) == set(want["selected"][0, h, r, :c].tolist()), \
                (h, r)


def _run(weave, q, k, v, lay, layer, capture: Optional[dict] = None):
    from cast_amd import weave as W
    module = SimpleNamespace(block_idx=layer, o=lambda x: x)
    if capture is not None:  # keep the selection the attention consumes
        from cast_amd import ops
        orig = ops.sparse_attn_bf16 if not weave.rcsa_int8_qk else ops.sparse_attn_int8

        def spy(*a, **kw):
            capture["selected"], capture["counts"] = a[3 if not weave.rcsa_int8_qk else 5], \
                a[4 if not weave.rcsa_int8_qk else 6]
            return orig(*a, **kw)
        name = "sparse_attn_bf16" if not weave.rcsa_int8_qk else "sparse_attn_int8"
        setattr(ops, name, spy)
        try:
            out = W.compact_cwca_attention(weave, module, q, k, v, lay)
        finally:
            setattr(ops, name, orig)
    else:
        out = W.compact_cwca_attention(weave, module, q, k, v, lay)
    weave.geometry_provider.end_compact_layer(layer)
    return out


def test_woven_layer_matches_oracle_without_router(dev):
    q, k, v, curvature, response = _inputs(0)
    lay = _layout(dev)
    prov = _provider(curvature.to(dev))
    prov._responses[0] = response.to(dev)
    weave = _weave(prov)
    print("woven layer 1, no router", flush=True)
    cap = {}
    out = _run(weave, q.to(dev), k.to(dev), v.to(dev), lay, 1, cap)
    torch.cuda.synchronize()
    want = _oracle(q, k, v, lay, curvature, response, 1)
    _check_sets(cap["selected"], cap["counts"], want)
    _check_out(out, want["out"])
    rec = weave._last_compact_attention
    assert rec["edge_budget"] == int(want["degrees"].sum())
    assert int(rec["minimum_degree"]) == int(want["degrees"].min())
    assert int(rec["maximum_degree"]) == int(want["degrees"].max())
    assert rec["budget_source"] == "compact_additive_curvature_control_response_lambda_0.5"
    assert rec["closed_loop_feedback_consumed"] and rec["routing"] is None
    s = prov.summary()["compact_budget_records"]
    assert len(s) == 1 and s[0]["budget_exact"] and s[0]["k_max"] == int(want["degrees"].max())
    assert s[0]["k_min"] == int(want["degrees"].min())
    assert isinstance(s[0]["curvature"]["mean"], float)


def test_woven_layer_reads_nothing_back(dev):
    """A layer the router does not refine runs with torch's synchronisation
    check set to error: no host read-back anywhere in the call."""
    from cast_amd.router import FCPASMSwapRouter, FCPASMSwapRoutingConfig
    q, k, v, curvature, response = _inputs(1)
    lay = _layout(dev)
    prov = _provider(curvature.to(dev))
    prov._responses[4] = response.to(dev)
    router = FCPASMSwapRouter(FCPASMSwapRoutingConfig(
        candidate_multiplier=2, num_swap_rounds=1, swap_eps=0.10, require_fc_transport=True,
        min_transport_affinity=0.5, max_swaps_per_call=1, active_layers=(22, 26),
        same_bank_only=True))
    weave = _weave(prov, router=router, layer=5)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    _run(weave, qd, kd, vd, lay, 5)  # first call: caches, library loads
    prov._responses[4] = response.to(dev)
    torch.cuda.synchronize()
    print("woven layer 5 under the sync check", flush=True)
    torch.cuda.set_sync_debug_mode("error")
    try:
        _run(weave, qd, kd, vd, lay, 5)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    assert weave._last_compact_attention["routing"]["fallback_reason"] == "layer_not_enabled"
    prov.check_compact_status()


@pytest.mark.parametrize("same_bank", [True, False])
def test_woven_router_layer_matches_oracle(dev, same_bank):
    from cast_amd.router import FCPASMSwapRouter, FCPASMSwapRoutingConfig
    q, k, v, curvature, response = _inputs(2)
    lay = _layout(dev)
    tr = _transport(7)
    cfg = FCPASMSwapRoutingConfig(candidate_multiplier=2, num_swap_rounds=2, swap_eps=1e-6,
                                  require_fc_transport=True, min_transport_affinity=0.5,
                                  same_bank_only=same_bank, active_layers=(22, 26))
    prov = _provider(curvature.to(dev), feedback_form="centered_inverse", response_weight=0.7)
    prov._responses[21] = response.to(dev)
    dev_tr = {**tr, "pairs": {p: {kk: (vv.to(dev) if vv.ndim else vv) for kk, vv in e.items()}
                              for p, e in tr["pairs"].items()}}
    weave = _weave(prov, router=FCPASMSwapRouter(cfg), transport=dev_tr, layer=22)
    print(f"woven router layer 22, same_bank {same_bank}", flush=True)
    cap = {}
    out = _run(weave, q.to(dev), k.to(dev), v.to(dev), lay, 22, cap)
    torch.cuda.synchronize()
    host_tr = dict(tr, attention_spatial_h=6, attention_spatial_w=5)
    want = _oracle(q, k, v, lay, curvature, response, 22, weight=0.7, form="centered_inverse",
                   router=dict(config=cfg, transport=host_tr, operator=_oracle_operator(tr)))
    rec = weave._last_compact_attention["routing"]
    assert rec["status"] == "refined" and want["record"]["status"] == "refined"
    assert rec["swap_count"] == want["record"]["swap_count"] >= 1
    assert abs(rec["objective_after"] - want["record"]["objective_after"]) <= \
        1e-4 * abs(want["record"]["objective_after"])
    _check_sets(cap["selected"], cap["counts"], want)
    _check_out(out, want["out"])
    assert rec["transport_query_source_layer"] == 21 and rec["transport_available_layers"] == [21]


def test_woven_layers_in_sequence_int8(dev):
    """Layer 0 (bootstrap), then layers 1 and 2 fed the previous layer's
    response, on the int8-QK path: degrees, selection and output per layer."""
    q, k, v, curvature, response = _inputs(3)
    lay = _layout(dev)
    prov = _provider(curvature.to(dev), feedback_form="centered_multiplicative",
                     response_weight=0.6)
    weave = _weave(prov, int8=True)
    qd, kd, vd = q.to(dev), k.to(dev), v.to(dev)
    for layer in range(3):
        prov._responses[layer - 1] = (response * (layer + 1)).to(dev)
        print(f"woven int8 layer {layer}", flush=True)
        cap = {}
        out = _run(weave, qd, kd, vd, lay, layer, cap)
        torch.cuda.synchronize()
        want = _oracle(q, k, v, lay, curvature, response * (layer + 1), layer, weight=0.6,
                       form="centered_multiplicative")
        _check_sets(cap["selected"], cap["counts"], want)
        _check_out(out, want["out"])
    recs = prov.summary()["compact_budget_records"]
    assert [r["source"] for r in recs] == [
        "compact_cwca_curvature_bootstrap"] + \
        ["compact_centered_multiplicative_curvature_control_response_lambda_0.6"] * 2
    assert [r["previous_layer"] for r in recs] == [None, 0, 1]
