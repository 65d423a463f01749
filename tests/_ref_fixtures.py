"""Loading of the reference-produced router, closed-loop, select and
apportionment fixtures (tests/golden/ref_router.npz, ref_closed_loop.npz,
ref_select.npz, ref_apportion.npz; written by
tests/golden/make_ref_golden.py) into the oracle's and the product's argument
forms.  Shared by the CPU and GPU fixture tests (and by the script, for the
select cases' seeded inputs)."""
import functools
import math
import random

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


# ---- the native layers' select() (P/qk_uncertainty_tangent_attention.py:988-1082) ----
# (seed, batch, heads, head_dim, frames, latent height, latent width, tile, degree)
SELECT_CASES = [
    dict(seed=400, B=1, H=2, D=64, T=8, height=6, width=10, block_shape=(4, 4, 4), degree=7),
    dict(seed=401, B=1, H=2, D=128, T=8, height=22, width=40, block_shape=(4, 4, 8),
         degree=15),
    dict(seed=402, B=2, H=1, D=64, T=10, height=8, width=16, block_shape=(4, 4, 8), degree=6),
]


def select_grid(case: dict):
    tt, th, tw = case["block_shape"]
    cells = math.ceil(case["T"] / tt)
    nh, nw = math.ceil(case["height"] / th), math.ceil(case["width"] / tw)
    return cells, nh, nw


def select_inputs(case: dict):
    """fp32 q, k [B, H, T*height*width, D]: N(0, 1)/sqrt(D) plus a per-frame
    N(0, 0.3) mean shift; and their fingerprint (sum, |sum| of each)."""
    g = torch.Generator().manual_seed(case["seed"])
    B, H, D, T = case["B"], case["H"], case["D"], case["T"]
    L = T * case["height"] * case["width"]
    out = []
    for _ in range(2):
        x = torch.randn(B, H, T, L // T, D, generator=g) / math.sqrt(D)
        x = x + torch.randn(B, H, T, 1, D, generator=g) * 0.3
        out.append(x.reshape(B, H, L, D).contiguous())
    q, k = out
    fp = [float(q.double().sum()), float(q.double().abs().sum()),
          float(k.double().sum()), float(k.double().abs().sum())]
    return q, k, fp


def select_budgets(case: dict):
    """(blocks, degree, per-row budgets): the fixed degree moved between rows,
    every row keeping at least its local stencil and at most every block."""
    cells, nh, nw = select_grid(case)
    nb = cells * nh * nw
    local_max = 1 + sum(min(2, n - 1) for n in (cells, nh, nw))
    degree = case["degree"]
    rows = [degree] * nb
    rng = random.Random(case["seed"])
    for _ in range(nb):
        a, b, t = rng.randrange(nb), rng.randrange(nb), rng.randint(1, 2)
        if a != b and rows[a] - t >= local_max and rows[b] + t <= nb:
            rows[a] -= t
            rows[b] += t
    return nb, degree, rows


def select_case(ci: int) -> dict:
    fx = router_fixture("select")
    pre = f"select{ci}_"
    case = SELECT_CASES[ci]
    q, k, fp = select_inputs(case)
    if not np.allclose(np.array(fp), fx[pre + "fingerprint"], rtol=1e-12, atol=1e-9):
        raise RuntimeError(f"select case {ci}: seeded inputs drifted from the fixture")
    return {"case": case, "q": q, "k": k, "rows": fx[pre + "rows"].tolist(),
            "selected": _t(fx[pre + "selected"]), "counts": _t(fx[pre + "counts"]),
            "report": fx[pre + "report"].tolist()}


# ---- largest-remainder apportionments (P/qk_uncertainty_tangent_attention.py:847-870,
# 1239-1264) ----

def apportion_cases() -> list:
    """Every stored split: (name, weights [n] or [sections, n] float32, total,
    reference result int64 of the same shape)."""
    fx = router_fixture("apportion")
    out = []
    for key in sorted(k for k in fx if k.endswith("_w") and not k.startswith("motion")):
        pre = key[:-2]
        out.append((pre, _t(fx[key]), int(fx[pre + "_total"]), _t(fx[pre + "_out"])))
    return out


def motion_cases() -> list:
    """(ray motion [n], degree, reference weights, reference row budgets)."""
    fx = router_fixture("apportion")
    return [(_t(fx[f"motion{i}_m"]), int(fx[f"motion{i}_degree"]), _t(fx[f"motion{i}_w"]),
             _t(fx[f"motion{i}_out"])) for i in range(2)]


def fp32_near_tie(weights: torch.Tensor, total: int, tol: float = 1e-5) -> bool:
    """Whether two fractional parts of total * w / sum(w) (clamped weights, in
    float64) lie within ``tol``: the rows where the fp32 rounding of the
    quotient, not the exact quotient, decides the order."""
    w = weights.double().clamp_min(0.0)
    if not bool(w.sum() > 0):
        w = torch.ones_like(w)
    raw = w * total / w.sum()
    fr = sorted((raw - raw.floor()).tolist(), reverse=True)
    return any(abs(a - b) < tol for a, b in zip(fr, fr[1:]))
