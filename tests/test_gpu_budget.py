"""Per-row budgets on the device (rcsa_row_budgets) against the oracle.

Apportionment: exact rational largest remainder on the fp32-rounded weights
(orc.apportion); a result may differ only where two fractional parts lie
within 1e-5 (an fp32 rounding tie, as for the host restatement).  Equal
weights give exact ties, which must go to the lower indices.  Saturation:
orc.saturate on the apportioned rows, bit for bit.
"""
import random

import pytest
import torch

from oracle import rcsa_oracle as orc

pytestmark = pytest.mark.gpu


def _near_tie(w32, total):
    raw = torch.tensor(w32, dtype=torch.float64) * total / sum(w32)
    fr = sorted((raw - raw.floor()).tolist(), reverse=True)
    return any(abs(a - b) < 1e-5 for a, b in zip(fr, fr[1:]))


@pytest.mark.parametrize("n", [7, 28, 300, 853, 4100])
def test_row_budgets_match_oracle(n):
    from cast_amd import ops
    rnd = random.Random(n)
    sections = 6
    w = [[rnd.random() * rnd.choice([1, 10, 1000]) for _ in range(n)] for _ in range(sections)]
    w[2] = [0.0] * n                      # a zero row weighs every entry 1
    w[3] = [1.0] * n                      # exact ties: the lower indices win
    w[4][::3] = [-1.0] * len(w[4][::3])   # negative weights count as 0
    total = rnd.randint(n // 2 + 1, 40 * n)
    print(f"row budgets n {n} total {total}", flush=True)
    wt = torch.tensor(w, dtype=torch.float32)
    got = ops.row_budgets(wt.cuda(), total).cpu().tolist()
    for s in range(sections):
        w32 = wt[s].tolist()
        want = orc.apportion(w32, total)
        assert sum(got[s]) == total
        if got[s] != want:
            pos = [max(x, 0.0) for x in w32]
            assert sum(pos) > 0 and _near_tie(pos, total), f"section {s}"
    assert got[3] == orc.apportion([1.0] * n, total)
    assert got[2] == got[3]


@pytest.mark.parametrize("n", [28, 853])
def test_row_budgets_saturation_matches_oracle(n):
    from cast_amd import ops
    rnd = random.Random(100 + n)
    sections = 5
    cap = max(2, n // 6)
    wt = torch.tensor([[rnd.random() ** 4 for _ in range(n)] for _ in range(sections)],
                      dtype=torch.float32)
    total = cap * n // 2
    for target in (None, total + 7, cap * n + 50):  # the last cannot be met: every row ends at cap
        got = ops.row_budgets(wt.cuda(), total, cap=cap, target_total=target).cpu().tolist()
        plain = ops.row_budgets(wt.cuda(), total).cpu().tolist()
        for s in range(sections):
            want = orc.saturate(plain[s], cap, total if target is None else target)
            assert got[s] == want, (s, target)
            assert max(got[s]) <= cap


def test_row_budgets_rejects_bad_shapes():
    from cast_amd import ops
    w = torch.ones(2, 10, device="cuda")
    with pytest.raises(RuntimeError):
        ops.row_budgets(w, 0)
    with pytest.raises(RuntimeError):
        ops.row_budgets(torch.ones(1, 9000, device="cuda"), 10)
    with pytest.raises(ValueError):
        ops.row_budgets(w.double(), 5)


# ---- the closed-loop allocator of a compact woven layer (rcsa_closed_loop_degrees) ----

def _cl_case(seed, *, S=30, tsrc=4, n_frames=10, feedback=None):
    g = torch.Generator().manual_seed(seed)
    curv = torch.rand(tsrc, S, generator=g) ** 3 * 4 + 1e-3
    frames = sorted(torch.randperm(3 + tsrc * 4, generator=g)[:n_frames].tolist())
    kw = dict(current_temporal_offset=3, source_group=4, compact_group=4)
    cells = -(-n_frames // 4)
    mem = 2 * S
    blocks = mem + cells * S
    mean = max(7, round(0.2 * blocks))
    base = max(7, -(-4 * mean // 5))
    kw.update(mean_degree=mean, base_degree=base, total_blocks=blocks, memory_blocks=mem)
    resp = None
    if feedback is not None:
        resp = torch.rand(tsrc, S, generator=g) * 2
        kw.update(response=resp, response_weight=0.7, feedback_form=feedback)
    return curv, frames, kw


def _cl_near_tie(curv, frames, kw):
    """A worldline whose fp32 weights put two fractional parts within 1e-5."""
    cur = curv.float()
    norm = cur / cur.mean(dim=0, keepdim=True).clamp_min(torch.finfo(torch.float32).eps)
    grp = (kw["compact_group"], kw["source_group"], kw["current_temporal_offset"])
    cells = orc.compact_time_cells(norm, frames, *grp)
    if kw.get("response") is not None:
        resp = orc.compact_time_cells(kw["response"].float(), frames, *grp)
        a = kw["response_weight"]
        if kw["feedback_form"] == "additive":
            cells = cells + a * resp
        else:
            sign = -1.0 if kw["feedback_form"] == "centered_inverse" else 1.0
            cells = cells * torch.exp(sign * a * (resp - 1.0))
    w = 1.0 + torch.log1p(cells)
    total = cells.shape[0] * (kw["mean_degree"] - kw["base_degree"])
    return any(_near_tie(w[:, s].tolist(), total) for s in range(w.shape[1]) if total > 0)


@pytest.mark.parametrize("seed,feedback,n_frames", [(1, None, 10), (2, None, 14), (3, None, 3),
                                                     (4, "additive", 10),
                                                     (5, "centered_multiplicative", 12),
                                                     (6, "centered_inverse", 7)])
def test_closed_loop_degrees_match_oracle(seed, feedback, n_frames):
    from cast_amd import ops
    curv, frames, kw = _cl_case(seed, n_frames=n_frames, feedback=feedback)
    print(f"closed loop seed {seed} feedback {feedback} frames {frames}", flush=True)
    want = orc.closed_loop_degrees(curv, frames, **kw)
    dkw = dict(kw)
    if dkw.get("response") is not None:
        dkw["response"] = dkw["response"].cuda()
    got = ops.closed_loop_degrees(curv.cuda(), frames, **dkw).cpu().long()
    assert int(got.sum()) == kw["total_blocks"] * kw["mean_degree"]
    if not torch.equal(got, want):
        assert _cl_near_tie(curv, frames, kw), (got - want).nonzero().flatten().tolist()
    fixed = ops.closed_loop_degrees(curv.cuda(), frames, fixed_query_budget=True, **dkw).cpu()
    assert torch.all(fixed == kw["mean_degree"])


def test_closed_loop_status_words():
    from cast_amd import ops
    curv, frames, kw = _cl_case(7)
    c = curv.cuda()
    assert len(frames) == 10  # three compact cells, as the row layout of kw expects
    # a profiled frame past the last curvature tile (offset 3 + 4 tiles x 4 frames)
    outside = frames[:-1] + [3 + 16]
    with pytest.raises(RuntimeError, match="outside CWCA frame capacity"):
        ops.closed_loop_degrees(c, outside, **kw)
    with pytest.raises(RuntimeError, match="outside CWCA frame capacity"):
        orc.closed_loop_degrees(curv, outside, **kw)
    # the no-read-back form leaves the bit in the status word
    _, st = ops.closed_loop_degrees(c, outside, check_status=False, **kw)
    assert int(st.item()) & 1
    with pytest.raises(RuntimeError, match="Memory frames"):
        ops.closed_loop_degrees(c, [-1] + frames[1:], **kw)
    # more edges per row than key blocks exist: the worldline budget cannot be placed
    bad = dict(kw, mean_degree=kw["total_blocks"] + 3, base_degree=kw["total_blocks"])
    with pytest.raises(RuntimeError, match="exhausted key capacity"):
        ops.closed_loop_degrees(c, frames, **bad)
    with pytest.raises(RuntimeError, match="exhausted key capacity"):
        orc.closed_loop_degrees(curv, frames, **bad)
