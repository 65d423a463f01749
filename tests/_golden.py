"""Loading of the committed golden fixtures and of the workloads they were
made from (shared by the CPU and GPU golden tests)."""
import functools
import hashlib
from pathlib import Path

import numpy as np
import torch

from cast_amd import workloads

GOLDEN = Path(__file__).resolve().parent / "golden"
ATTN_QBLOCKS = (0, 27)


def load(name: str) -> dict:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def fingerprint(w) -> str:
    h = hashlib.sha256()
    for t in (w.q, w.k, w.v, w.q_valid, w.k_valid, w.forced):
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        h.update(t.numpy().tobytes())
    return h.hexdigest()


@functools.lru_cache(maxsize=None)
def workload(name: str):
    """The seeded workload behind a fixture (CPU tensors, cached per process)."""
    if name == "c0_plumbing":
        return workloads.plumbing(0)
    if name == "c1_dit_bf16":
        return workloads.matrix_dit(0)
    if name == "c2_dit_int8":
        return workloads.matrix_dit(0, int8=True)
    if name == "c3_selection":
        return workloads.selection_stress(0)
    if name.startswith(("c1_seed", "c2_seed")):  # c1_seed3, c2_seed1, ...
        return workloads.matrix_dit(int(name[len("c1_seed"):]), int8=name.startswith("c2"))
    raise KeyError(name)


def seed_fixture(name: str) -> dict:
    """The per-seed slice of c1_seeds.npz / c2_seeds.npz as a plain dict
    (``c1_seed3`` -> the ``s3_*`` arrays without their prefix)."""
    seed = int(name[len("c1_seed"):])
    fx = load(f"{name[:2]}_seeds")
    pre = f"s{seed}_"
    return {k[len(pre):]: v for k, v in fx.items() if k.startswith(pre)}


def set_equal_where(idx_a, cnt_a, idx_b, cnt_b, rows_mask) -> int:
    """Number of rows in ``rows_mask`` whose selected sets differ."""
    bad = 0
    for r, i in zip(*np.nonzero(rows_mask)):
        ca, cb = int(cnt_a[r, i]), int(cnt_b[r, i])
        if ca != cb or set(idx_a[r, i, :ca].tolist()) != set(idx_b[r, i, :cb].tolist()):
            bad += 1
    return bad
