"""Loading of the reference-produced router and closed-loop fixtures
(tests/golden/ref_router.npz, ref_closed_loop.npz; written by
tests/golden/make_ref_golden.py) into the oracle's and the product's argument
forms.  Shared by the CPU and GPU fixture tests."""
import functools

import numpy as np
import torch

from tests._golden import GOLDEN


@functools.lru_cache(maxsize=None)
def router_fixture(which: str = "router") -> dict:
    with np.load(GOLDEN / f"ref_{which}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def _t(a):
    return torch.from_numpy(np.array(a))


def _transport(fx: dict, prefix: str):
    """(transport dict with the reference's keys, attention block grid)."""
    geo = [int(v) for v in fx[f"{prefix}geometry"]]
    out, trs, win, stride, pad, grid, block = (tuple(geo[i:i + 2]) for i in range(0, 14, 2))
    pairs = {}
    for i, (left, right) in enumerate(fx[f"{prefix}pairs"].tolist()):
        pairs[(int(left), int(right))] = {
            "theta": _t(fx[f"{prefix}theta{i}"]), "affinity": _t(fx[f"{prefix}affinity{i}"]),
            "mean_affinity": torch.tensor(float(fx[f"{prefix}mean_affinity{i}"]))}
    tr = {"output_shape": out, "transport_shape": trs, "window_shape": win, "stride": stride,
          "padding": pad, "tile_grid": grid, "pairs": pairs,
          "attention_spatial_h": block[0], "attention_spatial_w": block[1]}
    return tr, block


def transport_case(ci: int):
    fx = router_fixture()
    pre = f"transport{ci}_"
    tr, block = _transport(fx, pre)
    exps = [float(a) for a in fx[pre + "exponents"]]
    outs = [_t(fx[f"{pre}maps_out{j}"]) for j in range(len(exps))]
    mats = [_t(fx[f"{pre}matrix{j}"]) for j in range(len(exps))]
    return tr, block, _t(fx[pre + "maps"]), exps, outs, mats


def oracle_operator(transport, block):
    """operator(pair, exponent) for the oracle's objective and refine: the
    oracle's window-loop transport of the unit maps, [output, input]; None
    (the identity) for a pair the transport does not hold."""
    from oracle import rcsa_oracle as orc
    if transport is None:
        return None
    S = block[0] * block[1]
    eye = torch.eye(S).reshape(S, 1, *block)

    def op(pair, exponent):
        if pair not in transport["pairs"]:
            return None
        d = orc.transport_maps(transport, pair, eye, exponent).reshape(S, S)
        return (torch.eye(S) + d).T
    return op


def objective_case(tag: str):
    fx = router_fixture()
    tr, block = _transport(fx, "objective_")
    cells, group, boundary = (int(v) for v in fx["objective_params"])
    la, lr = (float(v) for v in fx["objective_lambdas"])
    kw = dict(temporal_cells=cells, spatial=block[0] * block[1],
              exact_frames=tuple(int(f) for f in fx["objective_frames"]),
              temporal_group_size=group, current_boundary=boundary, lambda_anchor=la,
              lambda_reconstruction=lr)
    op = oracle_operator(tr, block) if tag == "fc" else None
    return (_t(fx["objective_error"]), kw, op, float(fx[f"objective_{tag}_value"]),
            _t(fx[f"objective_{tag}_a"]), _t(fx[f"objective_{tag}_b"]))


def refine_count() -> int:
    return int(router_fixture()["refine_cases"].shape[0])


def refine_case(ci: int) -> dict:
    from cast_amd.router import FCPASMSwapRoutingConfig
    from oracle import rcsa_oracle as orc
    fx = router_fixture()
    same_bank, rounds = (int(v) for v in fx["refine_cases"][ci])
    mem, cells, bh, bw, group, boundary, layer = (int(v) for v in fx["refine_params"])
    pre = f"refine{ci}_"
    tr, block = _transport(fx, pre)
    N = mem + cells * bh * bw
    cfg = FCPASMSwapRoutingConfig(candidate_multiplier=2, num_swap_rounds=rounds, swap_eps=1e-6,
                                  sketch_groups=16, require_fc_transport=True,
                                  min_transport_affinity=0.5, same_bank_only=bool(same_bank))
    return {
        "score": _t(fx[pre + "score"]), "pooled_value": _t(fx[pre + "pooled_value"]),
        "selected": _t(fx[pre + "selected"]), "counts": _t(fx[pre + "counts"]),
        "local": orc.local_stencil(N, bh, bw), "transport": tr, "block": block, "config": cfg,
        "out": _t(fx[pre + "out"]), "swap_count": int(fx[pre + "swap_count"]),
        "objective": [float(v) for v in fx[pre + "objective"]],
        "historical_budget": [int(v) for v in fx[pre + "historical_budget"]],
        "kw": dict(memory_blocks=mem, spatial_shape=block,
                   exact_current_frames=tuple(int(f) for f in fx["refine_frames"]),
                   temporal_group_size=group, current_boundary=boundary, layer_index=layer),
    }


def closed_loop_count() -> int:
    return int(router_fixture("closed_loop")["cl_count"])


def closed_loop_case(ci: int) -> dict:
    fx = router_fixture("closed_loop")
    pre = f"cl{ci}_"
    layer, fixed, offset, src_group, cg, mean, base, total, memory = \
        (int(v) for v in fx[pre + "params"])
    curvature = _t(fx[pre + "curvature"])
    frames = [int(f) for f in fx[pre + "frames"]]
    eps = torch.finfo(torch.float32).eps
    params = dict(layer=layer, fixed=bool(fixed), offset=offset, source_group=src_group,
                  compact_group=cg, mean=mean, base=base, total=total, memory=memory)
    oracle_kw = dict(current_temporal_offset=offset, source_group=src_group, compact_group=cg,
                     mean_degree=mean, base_degree=base, total_blocks=total,
                     memory_blocks=memory, response=_t(fx[pre + "response"]),
                     response_weight=float(fx[pre + "weight"]),
                     feedback_form=str(fx[pre + "form"]), fixed_query_budget=bool(fixed),
                     layer_index=layer)
    return {"curvature": curvature, "frames": frames, "params": params,
            "oracle_kw": oracle_kw, "degrees": _t(fx[pre + "degrees"]),
            "source": str(fx[pre + "source"]),
            "budgets": [int(v) for v in fx[pre + "budgets"]],
            "curvature_stats": [float(v) for v in fx[pre + "curvature_stats"]],
            "normalized": curvature / curvature.mean(dim=0, keepdim=True).clamp_min(eps),
            "time_cells": _t(fx[pre + "time_cells"])}
