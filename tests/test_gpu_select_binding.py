"""The attention-compiler binding of ``taba_select`` (GPU).

CAST's attention compiler is a chain of ``select`` wrappers ending in the
trajectory-adaptive-budget select (P/control_response_cwca_attention.py:
2030-2034 appends the pending budget record; P/qk_uncertainty_tangent_attention.py:
1201-1209 and 1722-1734 add the section and worldline report fields; :988-1082
selects).  Its row budgets change per layer: ``set_layer_index`` re-installs
them (P/control_response_cwca_attention.py:1389-1529) and the select reads them
through ``_runtime_degrees`` (:1040).  These tests build a stand-in of that
chain (no reference import), bind the HIP select one level above its base
class, and check that budgets changed between two calls are followed, that the
wrappers above still run, and that ``_runtime_degrees`` receives the tiles.
"""
from dataclasses import replace

import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPE, HW, T, D = (4, 4, 8), (22, 40), 8, 64
NB = 2 * 6 * 5  # 8 frames / tt 4 = 2 cells, 6 x 5 spatial blocks


class StandInTABA:
    """Attributes of MatrixTrajectoryAdaptiveBudgetAttentionCompiler after compile()."""
    trajectory_complexity_kind = "motion_magnitude"

    def __init__(self, degree):
        self._block_shape, self._num_blocks, self._degree = SHAPE, NB, degree
        self._row_degrees = torch.full((NB,), degree, dtype=torch.long)
        self._ray_motion = torch.linspace(0.0, 1.0, NB)
        self._first_order_motion = self._ray_motion * 0.5
        self.seen_q_blocks = []

    def _runtime_degrees(self, q_blocks):
        self.seen_q_blocks.append(tuple(q_blocks.shape))
        return self._row_degrees

    def select(self, q, k, **kw):
        raise AssertionError("the HIP select must sit above this class")


class StandInSection(StandInTABA):
    """The section-conservative wrapper: report fields added after the select."""

    def select(self, *args, **kwargs):
        selected, counts, report = super().select(*args, **kwargs)
        sec = self._row_degrees.reshape(-1, 30).sum(-1)
        return selected, counts, replace(report, section_budget_min=int(sec.min()),
                                         section_budget_max=int(sec.max()))


class StandInClosedLoop(StandInSection):
    """set_layer_index installs per-layer budgets; select appends the pending record."""

    def __init__(self, degree, budgets):
        super().__init__(degree)
        self._budgets = budgets
        self._budget_records = []
        self._pending_budget_record = None

    def set_layer_index(self, layer):
        self._row_degrees = self._budgets[layer]
        self._pending_budget_record = {"layer": layer,
                                       "global_edge_budget": int(self._row_degrees.sum())}

    def select(self, q, k, **kwargs):
        selected, counts, report = super().select(q, k, **kwargs)
        if self._pending_budget_record is not None:
            self._budget_records.append(self._pending_budget_record)
            self._pending_budget_record = None
        return selected, counts, report


def _bound_class():
    from cast_amd.selector import taba_select

    class HipTABA(StandInTABA):
        def select(self, q, k, **kw):
            return taba_select(self, q, k, **kw)

    class Bound(StandInClosedLoop, HipTABA):
        pass

    mro = [c.__name__ for c in Bound.__mro__]
    assert mro.index("StandInSection") < mro.index("HipTABA") < mro.index("StandInTABA")
    return Bound


def _inputs(seed):
    g = torch.Generator().manual_seed(seed)
    shift = torch.randn(1, 2, T, 1, D, generator=g) * 0.3
    q = (torch.randn(1, 2, T, HW[0] * HW[1], D, generator=g) + shift).reshape(1, 2, -1, D)
    k = (torch.randn(1, 2, T, HW[0] * HW[1], D, generator=g) + shift).reshape(1, 2, -1, D)
    return q, k


def _native(score, rows):
    """Stable descending argsort of score + 1e6 * local, first max(rows) columns."""
    from cast_amd import layout
    local = layout.local_stencil(NB, 6, 5)
    ranking = score + local[None, None].float() * 1e6
    return torch.argsort(ranking, dim=-1, descending=True, stable=True)[..., :int(rows.max())]


def _device_scores(q, k, dev):
    from cast_amd import layout, ops
    lay = layout.compact_layout(range(T), 0, *HW, SHAPE, dev)
    qhat, _, _ = ops.pool_query(ops.pack_tokens(q.to(dev).transpose(1, 2), lay.slot_token),
                                lay.slot_valid, 128)
    khat, _, _, _ = ops.pool_key(ops.pack_tokens(k.to(dev).transpose(1, 2), lay.slot_token),
                                 lay.slot_valid, 128)
    return ops.block_scores(qhat, khat).cpu().reshape(1, 2, NB, NB)


def test_budgets_change_between_calls(dev):
    Bound = _bound_class()
    gen = torch.Generator().manual_seed(3)
    a = torch.full((NB,), 16, dtype=torch.long)
    b = a.clone()
    b[:30] += torch.randint(0, 6, (30,), generator=gen)  # a bigger max in layer 2
    b[30:] = 16 - (b[:30] - 16)                           # same total
    comp = Bound(16, {1: a, 2: b})
    q, k = _inputs(1)
    qd, kd = q.to(dev), k.to(dev)
    gc = torch.full((1, 2, NB), 16, dtype=torch.int32)
    kw = dict(geometry_indices=None, geometry_counts=gc, latent_hw=HW, block_shape=SHAPE)
    score = _device_scores(q, k, dev)
    for layer, rows in ((1, a), (2, b), (1, a)):
        comp.set_layer_index(layer)
        print(f"select layer {layer} max budget {int(rows.max())}", flush=True)
        selected, counts, report = comp.select(qd, kd, **kw)
        torch.cuda.synchronize()
        assert selected.shape == (1, 2, NB, int(rows.max()))
        assert torch.equal(counts.cpu(), rows.int()[None, None].expand(1, 2, -1))
        assert torch.equal(selected.cpu().long(), _native(score, rows))
        assert report.budget_total == int(rows.sum()) and report.budget_max == int(rows.max())
        sec = rows.reshape(-1, 30).sum(-1)
        assert (report.section_budget_min, report.section_budget_max) == \
            (int(sec.min()), int(sec.max()))
        assert report.missing_local_edges == 0 and report.row_duplicate_violations == 0
    assert [r["layer"] for r in comp._budget_records] == [1, 2, 1]
    # _runtime_degrees got the packed tiles [B, H, N, tt*th*tw, D]
    assert comp.seen_q_blocks == [(1, 2, NB, 128, D)] * 3


def test_runtime_degrees_from_tiles(dev):
    """An override that derives budgets from the tiles (the token-cancellation
    uncertainty of P/qk_uncertainty_tangent_attention.py:1266-1302) sees the
    same per-tile statistics as the reference's zero-padded tiles."""
    Bound = _bound_class()

    def uncertainty(q_blocks):
        x = q_blocks.float()
        mean_norm = torch.linalg.vector_norm(x.mean(dim=-2), dim=-1)
        token_norm = torch.linalg.vector_norm(x, dim=-1).mean(dim=-1)
        return (1.0 - mean_norm / token_norm.clamp_min(1e-6)).clamp(0, 1).mean(dim=(0, 1))

    class Adaptive(Bound):
        def _runtime_degrees(self, q_blocks):
            u = uncertainty(q_blocks).cpu()
            return 14 + (u > u.median()).long() * 4  # 14 or 18 edges per row

    q, k = _inputs(2)
    comp = Adaptive(16, {})
    gc = torch.full((1, 2, NB), 16, dtype=torch.int32)
    selected, counts, _ = comp.select(q.to(dev), k.to(dev), geometry_indices=None,
                                      geometry_counts=gc, latent_hw=HW, block_shape=SHAPE)
    torch.cuda.synchronize()
    # the reference's tiles: zero-padded (tt, th, tw) reshape of the grid
    tt, th, tw = SHAPE
    x = torch.nn.functional.pad(q.reshape(1, 2, T, *HW, D), (0, 0, 0, 0, 0, 2))
    x = x.reshape(1, 2, T // tt, tt, 6, th, 5, tw, D).permute(0, 1, 2, 4, 6, 3, 5, 7, 8)
    u_ref = uncertainty(x.reshape(1, 2, NB, 128, D))
    rows = 14 + (u_ref > u_ref.median()).long() * 4
    assert torch.equal(counts[0, 0].cpu(), rows.int())
    assert torch.equal(selected.cpu().long(), _native(_device_scores(q, k, dev), rows))
