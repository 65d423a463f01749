"""Write reference-produced fixtures for the router transport / objective /
refine, the closed-loop allocator, the native select and the largest-remainder
apportionments: ``tests/golden/ref_router.npz``, ``ref_closed_loop.npz``,
``ref_select.npz`` and ``ref_apportion.npz``.

Run in the build container only (the reference never travels to a GPU box):

    python tests/golden/make_ref_golden.py [/path/to/CAST]

It imports three torch-only modules of the CAST reference and records, on small
seeded CPU inputs, what these functions return:

* ``FCPASMLocalCoordinateSwapRouter._apply_transport_maps`` and
  ``._transport_matrix`` (P/fc_pasm_swap_routing.py:116-412): a pooled
  transport grid (11 x 10 windows averaged to 6 x 5) and an unpooled one
  (8 x 8 windows), exponents of both signs;
* ``._objective_value`` and ``._objective_terms`` (:414-614), with no
  transport (g = 0) and with a published transport;
* ``.refine`` (:616-1077), four calls with a published transport: same-bank
  on and off, one and two rounds;
* ``MatrixControlResponseCWCAAttentionCompiler._compact_time_cells``,
  ``._redistribute_compact_capacity`` and ``.compact_closed_loop_degrees``
  (P/control_response_cwca_attention.py:1123-1363): the additive, centred
  multiplicative and centred inverse feedback forms with a nonzero response,
  the layer-0 bootstrap, response weight 0, the fixed query budget, prefix
  frames before the profiled offset, a partial last cell and a peaked
  curvature that saturates rows.  The method runs on an instance whose
  attributes are set directly (the fields it reads), not through compile().

* ``MatrixTrajectoryAdaptiveBudgetAttentionCompiler.select``
  (P/qk_uncertainty_tangent_attention.py:988-1082): the native layers'
  selection (visual tiling, pooled cosine scores, the +1e6 local stencil,
  the stable descending argsort cut at each row's budget) on three seeded
  cases with non-uniform row budgets (``tests/golden/ref_select.npz``).  The
  inputs are regenerated from their seeds (``select_inputs``, also used by
  the tests) and fingerprinted.

Fixtures hold inputs and outputs only (numpy arrays, no pickles); the tests
feed the inputs to the oracle and the product and compare with the outputs.
P/ = src/interaction_accel/methods/proposed/.

* ``MatrixTrajectoryAdaptiveBudgetAttentionCompiler._apportion`` and
  ``._motion_weights`` (P/qk_uncertainty_tangent_attention.py:847-870) and
  ``MatrixCurvatureTemperedUncertaintyAttentionCompiler._apportion_section_matrix``
  (:1239-1264): the fp32 largest-remainder splits on random, zero, equal,
  negative, decimal (near-tie) and peaked weights
  (``tests/golden/ref_apportion.npz``, inputs stored beside the outputs).

    python tests/golden/make_ref_golden.py [/path/to/CAST] [router|closed_loop|select|apportion ...]
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
GROUPS = ("router", "closed_loop", "select", "apportion")
_ARGS = [a for a in sys.argv[1:] if a not in GROUPS]
ONLY = [a for a in sys.argv[1:] if a in GROUPS]
REF = _ARGS[0] if _ARGS else "/root/reference"
sys.path.insert(0, os.path.join(REF, "src"))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from interaction_accel.methods.proposed import fc_pasm_swap_routing as R  # noqa: E402
from interaction_accel.methods.proposed import control_response_cwca_attention as C  # noqa: E402
from interaction_accel.methods.proposed import qk_uncertainty_tangent_attention as Q  # noqa: E402
from tests._ref_fixtures import SELECT_CASES, select_budgets, select_inputs  # noqa: E402

Router = R.FCPASMLocalCoordinateSwapRouter

# transport geometries: (output, transport, window, stride, padding, tile grid, block grid)
GEOMETRIES = {
    "pooled": ((22, 40), (6, 5), (11, 10), (8, 8), (4, 5), (3, 6), (6, 5)),
    "unpooled": ((16, 20), (8, 8), (8, 8), (4, 4), (2, 2), (4, 5), (4, 5)),
}


def transport_dict(name, seed, pairs, mean_affinity=0.9):
    out, tr, win, stride, pad, grid, _ = GEOMETRIES[name]
    g = torch.Generator().manual_seed(seed)
    tiles = grid[0] * grid[1]
    spec = (tr[0], tr[1] // 2 + 1)
    entries = {}
    for p in pairs:
        entries[p] = {"theta": (torch.rand(tiles, *spec, generator=g) * 2 - 1) * math.pi,
                      "affinity": torch.rand(tiles, *spec, generator=g),
                      "mean_affinity": torch.tensor(mean_affinity)}
    return {"output_shape": out, "transport_shape": tr, "window_shape": win, "stride": stride,
            "padding": pad, "tile_grid": grid, "pairs": entries}


def put_transport(fx, prefix, name, tr):
    out, trs, win, stride, pad, grid, block = GEOMETRIES[name]
    fx[f"{prefix}geometry"] = np.array([*out, *trs, *win, *stride, *pad, *grid, *block],
                                       dtype=np.int64)
    pairs = sorted(tr["pairs"])
    fx[f"{prefix}pairs"] = np.array(pairs, dtype=np.int64).reshape(-1, 2)
    for i, p in enumerate(pairs):
        e = tr["pairs"][p]
        fx[f"{prefix}theta{i}"] = e["theta"].numpy()
        fx[f"{prefix}affinity{i}"] = e["affinity"].numpy()
        fx[f"{prefix}mean_affinity{i}"] = np.float32(float(e["mean_affinity"]))


def transport_cases(fx):
    for ci, (name, exps) in enumerate((("pooled", (0.25, -0.6, 1.0)),
                                       ("unpooled", (0.4, -0.35, -1.0)))):
        block = GEOMETRIES[name][6]
        tr = transport_dict(name, 100 + ci, [(0, 6)])
        put_transport(fx, f"transport{ci}_", name, tr)
        g = torch.Generator().manual_seed(200 + ci)
        maps = torch.randn(3, 2, *block, generator=g)
        fx[f"transport{ci}_maps"] = maps.numpy()
        fx[f"transport{ci}_exponents"] = np.array(exps, dtype=np.float32)
        for j, a in enumerate(exps):
            moved, used = Router._apply_transport_maps(tr, (0, 6), maps, spatial_shape=block,
                                                       exponent=a)
            assert used
            fx[f"transport{ci}_maps_out{j}"] = moved.numpy()
            mat, used = Router._transport_matrix(tr, (0, 6), spatial_shape=block,
                                                 device=torch.device("cpu"), exponent=a)
            assert used
            fx[f"transport{ci}_matrix{j}"] = mat.numpy()


OBJ_KW = dict(temporal_cells=3, exact_frames=(0, 3, 7, 9), temporal_group_size=4,
              current_boundary=8, lambda_anchor=1.0, lambda_reconstruction=0.7)


def objective_cases(fx):
    name = "pooled"
    block = GEOMETRIES[name][6]
    S = block[0] * block[1]
    tr = transport_dict(name, 300, [(0, 3), (3, 7)])
    tr = dict(tr, attention_spatial_h=block[0], attention_spatial_w=block[1])
    put_transport(fx, "objective_", name, tr)
    g = torch.Generator().manual_seed(301)
    err = torch.randn(1, 2, OBJ_KW["temporal_cells"] * S, 4, generator=g) * 0.1
    fx["objective_error"] = err.numpy()
    fx["objective_frames"] = np.array(OBJ_KW["exact_frames"], dtype=np.int64)
    fx["objective_params"] = np.array([OBJ_KW["temporal_cells"], OBJ_KW["temporal_group_size"],
                                       OBJ_KW["current_boundary"]], dtype=np.int64)
    fx["objective_lambdas"] = np.array([OBJ_KW["lambda_anchor"],
                                        OBJ_KW["lambda_reconstruction"]], dtype=np.float32)
    for tag, t in (("g0", None), ("fc", tr)):
        v = Router._objective_value(err, spatial=S, transport=t, **OBJ_KW)
        a, b, _, used, terms = Router._objective_terms(err, spatial=S, transport=t, **OBJ_KW)
        assert used == (t is not None) and terms == 5
        fx[f"objective_{tag}_value"] = np.float32(float(v))
        fx[f"objective_{tag}_a"] = a.numpy()
        fx[f"objective_{tag}_b"] = b.numpy()


# refine: a compact layer of 63 memory blocks and 4 current cells of 6 x 5
MEM, CELLS, D, HEADS, K = 63, 4, 64, 2, 24


def local_stencil(n, nh, nw):
    ids = torch.arange(n)
    spatial = nh * nw
    bt, rem = ids // spatial, ids % spatial
    bh, bw = rem // nw, rem % nw
    return ((bt[:, None] - bt[None, :]).abs() + (bh[:, None] - bh[None, :]).abs()
            + (bw[:, None] - bw[None, :]).abs()) <= 1


def refine_cases(fx):
    block = GEOMETRIES["pooled"][6]
    S = block[0] * block[1]
    N = MEM + CELLS * S
    local = local_stencil(N, *block)
    cases = [(True, 1), (False, 1), (True, 2), (False, 2)]
    fx["refine_cases"] = np.array(cases, dtype=np.int64)
    fx["refine_params"] = np.array([MEM, CELLS, block[0], block[1], 4, 8, 22], dtype=np.int64)
    fx["refine_frames"] = np.array([0, 6], dtype=np.int64)
    for ci, (same_bank, rounds) in enumerate(cases):
        g = torch.Generator().manual_seed(400 + ci)
        qh = torch.nn.functional.normalize(torch.randn(1, HEADS, N, D, generator=g), dim=-1)
        kh = torch.nn.functional.normalize(torch.randn(1, HEADS, N, D, generator=g) + qh * 0.3,
                                           dim=-1)
        score = qh @ kh.transpose(-1, -2)
        pooled_v = torch.randn(1, HEADS, N, D, generator=g) * 0.5
        rank = score + local[None, None] * 1e6
        sel = torch.sort(rank, dim=-1, descending=True, stable=True).indices[..., :K]
        counts = torch.randint(K - 6, K + 1, (1, HEADS, N), generator=g)
        tr = transport_dict("pooled", 410 + ci, [(0, 6)])
        put_transport(fx, f"refine{ci}_", "pooled", tr)
        tr = dict(tr, attention_spatial_h=block[0], attention_spatial_w=block[1])
        cfg = R.FCPASMSwapRoutingConfig(candidate_multiplier=2, num_swap_rounds=rounds,
                                        swap_eps=1e-6, sketch_groups=16,
                                        require_fc_transport=True, min_transport_affinity=0.5,
                                        same_bank_only=same_bank)
        # refine writes its swaps into the route it is given (the scatter into
        # selected[..., memory:, :] at :950-960), so it gets a copy
        out, rec = Router(cfg).refine(score=score, pooled_value=pooled_v, selected=sel.clone(),
                                      counts=counts, local=local, memory_blocks=MEM,
                                      spatial_shape=block, exact_current_frames=(0, 6),
                                      temporal_group_size=4, current_boundary=8, transport=tr,
                                      layer_index=22)
        assert rec["status"] == "refined" and rec["swap_count"] >= 1, rec
        for key, val in (("score", score), ("pooled_value", pooled_v), ("selected", sel),
                         ("counts", counts), ("out", out)):
            fx[f"refine{ci}_{key}"] = val.numpy()
        fx[f"refine{ci}_swap_count"] = np.int64(rec["swap_count"])
        fx[f"refine{ci}_objective"] = np.array([float(rec["objective_before"]),
                                                float(rec["objective_after"])])
        fx[f"refine{ci}_historical_budget"] = np.array(
            [int(rec["historical_budget_before"]), int(rec["historical_budget_after"])])


# closed loop: CWCA source tiles of 4 frames, 6 spatial worldlines
def provider(curvature, *, offset, block_t, feedback, weight, fixed, layer, responses):
    p = object.__new__(C.MatrixClosedLoopCWCAAttentionCompiler)
    p.mode = "closed_loop"
    p._compact_layer_index = layer
    p._layer_index = layer
    p._curvature_matrix = curvature
    p._current_temporal_offset = offset
    p._block_shape = (block_t, 1, 1)
    p.fixed_query_budget = fixed
    p.response_weight = weight
    p.feedback_form = feedback
    p._responses = responses
    p._call_index = 0
    return p


CL_CASES = [
    # (feedback, weight, layer, fixed, offset, frames (current-local), compact group,
    #  mean, memory rows, peaked); total rows = memory + cells * 6
    ("additive", 0.5, 3, False, 3, list(range(0, 16)), 4, 61, 183, False),
    ("centered_multiplicative", 0.7, 5, False, 3, list(range(0, 16)), 4, 61, 183, False),
    ("centered_inverse", 0.7, 5, False, 3, list(range(0, 16)), 4, 61, 183, False),
    ("additive", 0.5, 0, False, 3, list(range(0, 16)), 4, 61, 183, False),
    ("additive", 0.0, 4, False, 3, list(range(0, 16)), 4, 61, 183, False),
    ("additive", 0.5, 4, True, 3, list(range(0, 16)), 4, 61, 183, False),
    ("centered_inverse", 1.3, 2, False, 1, [0, 2, 5, 6, 7, 9, 12], 3, 40, 24, False),
    ("additive", 0.8, 7, False, 0, [1, 2, 3, 4, 5, 6, 7, 8, 9, 10], 2, 31, 2, True),
]


def closed_loop_cases(fx):
    S = 6
    fx["cl_count"] = np.int64(len(CL_CASES))
    for ci, (form, weight, layer, fixed, offset, frames, cg, mean, memory,
             peaked) in enumerate(CL_CASES):
        g = torch.Generator().manual_seed(500 + ci)
        t_src = 4
        curvature = torch.rand(t_src, S, generator=g) + 0.05
        if peaked:
            curvature[1, 2] = 60.0
        response = torch.rand(t_src, S, generator=g) * 2
        cells = math.ceil(len(frames) / cg)
        total = memory + cells * S
        base = max(7, math.ceil(4 * mean / 5))
        p = provider(curvature, offset=offset, block_t=4, feedback=form, weight=weight,
                     fixed=fixed, layer=layer, responses={layer - 1: response})
        origin = 40
        active = torch.tensor(frames, dtype=torch.long) + origin
        deg, meta = p.compact_closed_loop_degrees(
            layer_index=layer, active_current=active, current_frame_origin=origin,
            temporal_group_size=cg, spatial_blocks=S, mean_degree=mean, base_degree=base,
            total_blocks=total, memory_blocks=memory)
        assert deg.shape == (cells, S) and cells * S == total - memory, (ci, deg.shape)
        pre = f"cl{ci}_"
        fx[pre + "curvature"] = curvature.numpy()
        fx[pre + "response"] = response.numpy()
        fx[pre + "frames"] = np.array(frames, dtype=np.int64)
        fx[pre + "params"] = np.array([layer, int(fixed), offset, 4, cg, mean, base, total,
                                       memory], dtype=np.int64)
        fx[pre + "form"] = np.array(form)
        fx[pre + "weight"] = np.float32(weight)
        fx[pre + "degrees"] = deg.numpy()
        fx[pre + "source"] = np.array(meta["source"])
        fx[pre + "budgets"] = np.array([meta["current_worldline_budget"],
                                        meta["current_edge_budget"], meta["global_edge_budget"],
                                        meta["reference_edge_budget"]], dtype=np.int64)
        cs = meta["curvature"]
        fx[pre + "curvature_stats"] = np.array([cs["min"], cs["max"], cs["mean"], cs["std"]],
                                               dtype=np.float64)
        # the helpers on their own
        normalized = curvature / curvature.mean(dim=0, keepdim=True).clamp_min(
            torch.finfo(curvature.dtype).eps)
        cells_t = C.MatrixControlResponseCWCAAttentionCompiler._compact_time_cells(
            normalized, torch.tensor(frames), cg, 4, offset)
        fx[pre + "time_cells"] = cells_t.numpy()
    # redistribution alone: a column over capacity, a column exactly at it
    deg = torch.tensor([[12, 3, 9], [2, 4, 9], [0, 11, 9]], dtype=torch.long)
    fx["redistribute_in"] = deg.numpy()
    fx["redistribute_out"] = C.MatrixControlResponseCWCAAttentionCompiler \
        ._redistribute_compact_capacity(deg.clone(), capacity=10,
                                        target_per_worldline=18).numpy()


def select_cases(fx):
    """The reference's own select() on a bare compiler instance holding the
    attributes it reads (budgets as set_layer_index would install them)."""
    TABA = Q.MatrixTrajectoryAdaptiveBudgetAttentionCompiler
    for ci, case in enumerate(SELECT_CASES):
        q, k, fp = select_inputs(case)
        nb, degree, rows = select_budgets(case)
        comp = TABA.__new__(TABA)
        comp._block_shape = tuple(case["block_shape"])
        comp._num_blocks = nb
        comp._degree = degree
        comp._row_degrees = torch.tensor(rows, dtype=torch.long)
        comp._ray_motion = torch.linspace(0.1, 1.0, nb)
        comp._first_order_motion = torch.linspace(0.2, 0.8, nb)
        comp.trajectory_complexity_kind = "motion_magnitude"
        B, H = q.shape[:2]
        counts_in = torch.full((B, H, nb), degree, dtype=torch.int32)
        sel, counts, rep = comp.select(
            q, k, geometry_indices=torch.zeros(B, H, nb, degree, dtype=torch.int32),
            geometry_counts=counts_in, latent_hw=(case["height"], case["width"]),
            block_shape=tuple(case["block_shape"]))
        pre = f"select{ci}_"
        fx[pre + "fingerprint"] = np.array(fp, dtype=np.float64)
        fx[pre + "rows"] = np.array(rows, dtype=np.int64)
        fx[pre + "selected"] = sel.numpy()
        fx[pre + "counts"] = counts.numpy()
        fx[pre + "report"] = np.array([rep.mean_selected_qk_cosine, rep.protected_local_edges,
                                       rep.missing_local_edges, rep.budget_min, rep.budget_max,
                                       rep.budget_total], dtype=np.float64)


def apportion_vectors():
    """Weight vectors and totals for TABA._apportion: random weights of mixed
    scales, all-zero and all-equal vectors, negative entries, decimal weights
    whose fp32 fractional parts nearly tie, and peaked weights."""
    g = torch.Generator().manual_seed(500)
    cases = []
    for n, total in ((7, 20), (28, 600), (300, 4096)):
        scale = torch.tensor([1.0, 10.0, 1000.0])[torch.randint(0, 3, (n,), generator=g)]
        cases.append((torch.rand(n, generator=g) * scale, total))
    cases.append((torch.zeros(5), 7))
    cases.append((torch.ones(9), 31))
    w = torch.rand(12, generator=g)
    w[::3] = -torch.rand(4, generator=g)
    cases.append((w, 40))
    cases.append((torch.tensor([0.1, 0.1, 0.1, 0.7]), 10))
    cases.append((torch.tensor([0.1, 0.2, 0.3, 0.4, 0.1, 0.2, 0.3]), 13))
    cases.append((torch.tensor([1.0 / 3.0] * 6 + [2.0 / 3.0] * 5), 17))
    cases.append((torch.rand(853, generator=g) ** 4, 853 * 5))
    # decimal weights whose fp32 quotients tie (or swap) fractional parts that
    # differ in exact arithmetic on the same fp32 inputs
    cases.append((torch.tensor([0.2, 0.7, 0.3]), 30))
    cases.append((torch.tensor([1.0, 4.2, 0.8, 0.3]), 9))
    cases.append((torch.tensor([0.6, 1.35, 2.4, 0.45, 7.2, 0.2, 1.8]), 36))
    return [(w.float(), t) for w, t in cases]


def apportion_matrices():
    """Section matrices and per-section totals for
    MatrixCurvatureTemperedUncertaintyAttentionCompiler._apportion_section_matrix:
    random rows, a zero row, an all-equal row, a row with negatives, a decimal
    row, and decimal rows whose fp32 fractional parts order differently from
    exact arithmetic."""
    g = torch.Generator().manual_seed(501)
    out = []
    for S, n, total in ((6, 7, 23), (5, 40, 300), (4, 260, 1500)):
        w = torch.rand(S, n, generator=g) * torch.tensor([1.0, 10.0, 1000.0])[
            torch.randint(0, 3, (S, n), generator=g)]
        w[1] = 0.0
        w[2] = 1.0
        w[3, ::2] = -1.0
        if S > 4:
            w[4] = torch.tensor([0.1, 0.2, 0.3, 0.4])[torch.arange(n) % 4]
        out.append((w.float(), total))
    out.append((torch.tensor([[3.6, 0.05, 0.45, 4.9, 0.6, 1.05, 0.6],
                              [3.6, 4.9, 0.9, 1.4, 1.2, 1.8, 2.7],
                              [0.3, 0.6, 6.3, 1.4, 6.3, 1.5, 8.1]]), 30))
    return out


def apportion_cases(fx):
    """The reference's largest-remainder apportionments: the 1-D TABA form,
    the row-wise section form, and TABA's motion weights feeding it."""
    TABA = Q.MatrixTrajectoryAdaptiveBudgetAttentionCompiler
    SECT = Q.MatrixCurvatureTemperedUncertaintyAttentionCompiler
    for i, (w, total) in enumerate(apportion_vectors()):
        fx[f"vec{i}_w"] = w.numpy()
        fx[f"vec{i}_total"] = np.array(total, dtype=np.int64)
        fx[f"vec{i}_out"] = TABA._apportion(w.clone(), total).numpy()
    for i, (w, total) in enumerate(apportion_matrices()):
        fx[f"mat{i}_w"] = w.numpy()
        fx[f"mat{i}_total"] = np.array(total, dtype=np.int64)
        fx[f"mat{i}_out"] = SECT._apportion_section_matrix(w.clone(), total).numpy()
    g = torch.Generator().manual_seed(502)
    for i, (n, degree) in enumerate(((30, 7), (330, 21))):
        motion = torch.rand(n, generator=g) ** 2
        weights = TABA._motion_weights(motion)
        fx[f"motion{i}_m"] = motion.numpy()
        fx[f"motion{i}_degree"] = np.array(degree, dtype=np.int64)
        fx[f"motion{i}_w"] = weights.numpy()
        fx[f"motion{i}_out"] = TABA._apportion(weights, n * degree).numpy()


def main():
    torch.manual_seed(0)
    written = []
    if not ONLY or "router" in ONLY:
        fx = {}
        transport_cases(fx)
        objective_cases(fx)
        refine_cases(fx)
        np.savez_compressed(os.path.join(HERE, "ref_router.npz"), **fx)
        written.append(("ref_router.npz", fx))
    if not ONLY or "closed_loop" in ONLY:
        fc = {}
        closed_loop_cases(fc)
        np.savez_compressed(os.path.join(HERE, "ref_closed_loop.npz"), **fc)
        written.append(("ref_closed_loop.npz", fc))
    if not ONLY or "select" in ONLY:
        fs = {}
        select_cases(fs)
        np.savez_compressed(os.path.join(HERE, "ref_select.npz"), **fs)
        written.append(("ref_select.npz", fs))
    if not ONLY or "apportion" in ONLY:
        fa = {}
        apportion_cases(fa)
        np.savez_compressed(os.path.join(HERE, "ref_apportion.npz"), **fa)
        written.append(("ref_apportion.npz", fa))
    for name, d in written:
        size = os.path.getsize(os.path.join(HERE, name))
        print(f"wrote {name}: {len(d)} arrays, {size / 1024:.0f} KiB")


if __name__ == "__main__":
    main()
