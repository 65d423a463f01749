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
