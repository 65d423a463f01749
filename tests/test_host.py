"""Host-side tests that need no GPU: the C-ABI library loads and exports what
``include/rcsa.h`` declares, the Python wrappers fail loudly off-device, the
synthetic workloads have the shapes and budgets of the benchmark cases, and
bench.py refuses more than one GPU."""
import re
from pathlib import Path

import pytest
import torch

from cast_amd import _lib, ops, workloads

ROOT = Path(__file__).resolve().parents[1]


def _header_functions():
    text = (ROOT / "include" / "rcsa.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(rcsa_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from cast_amd import build
        build.build(verbose=False)
    return _lib.load()


def test_header_and_binding_agree():
    declared = _header_functions()
    assert declared, "no entry points parsed from include/rcsa.h"
    assert sorted(_lib.SIGNATURES) == declared


def test_library_exports_every_declared_symbol(lib):
    for name in _header_functions():
        assert hasattr(lib, name), f"librcsa.so does not export {name}"


def test_status_strings_and_version(lib):
    # host-only entry points: no device work
    assert lib.rcsa_abi_version() == 3 << 16  # gathered attention sources, router
    for code in range(8):
        assert lib.rcsa_status_string(code)
    assert b"unknown" in lib.rcsa_status_string(99).lower()
    with pytest.raises(RuntimeError, match=r"rcsa_demo: .*\(status 2\)"):
        _lib.check(2, "rcsa_demo")


TORCH_OPS = {
    "pool_query_key": "rcsa_pool_query_key",
    "quantize_key_select": "rcsa_quantize_key_select",
    "sparse_attn_bf16": "rcsa_sparse_attn_bf16_split",
    "sparse_attn_int8": "rcsa_sparse_attn_int8_split",
    "quantize_rows_int8": "rcsa_quantize_rows_int8",
    "int8_linear": "rcsa_int8_linear",
}


@pytest.fixture(scope="module")
def rcsa_ops(lib):
    if not _lib.TORCH_OPS_PATH.exists():
        from cast_amd import build
        build.build_torch_ops()
    return _lib.torch_ops()


def test_torch_extension_registers_the_ops(rcsa_ops):
    declared = set(_header_functions())
    for op, entry in TORCH_OPS.items():
        assert entry in declared
        schema = str(getattr(rcsa_ops, op).default._schema)
        assert schema.startswith(f"rcsa::{op}("), schema
        assert schema.endswith("-> ()"), schema  # outputs are written in place
    # outputs are declared mutated, inputs are not
    schema = str(rcsa_ops.int8_linear.default._schema)
    assert "Tensor(a!) out" in schema and "Tensor x_i8," in schema


def test_torch_ops_refuse_host_tensors(rcsa_ops):
    x = torch.zeros(4, 256, dtype=torch.int8)
    xs = torch.ones(4)
    with pytest.raises(RuntimeError, match=r"int8_linear: .* must be a GPU tensor"):
        rcsa_ops.int8_linear(x, xs, x, xs, None, torch.empty(4, 4, dtype=torch.bfloat16))
    q = torch.zeros(1, 1, 128, 128, dtype=torch.bfloat16)
    idx = torch.zeros(1, 1, 1, 1, dtype=torch.int32)
    cnt = torch.ones(1, 1, 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match=r"sparse_attn_bf16: dims needs 8 values"):
        rcsa_ops.sparse_attn_bf16(q, q, q, None, None, 1.0, None, q, idx, cnt, [1], [0] * 18, 1,
                                  None, None, 0, None, 0, None, 0)


def test_ops_refuse_host_tensors():
    q = torch.zeros(1, 1, 128, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.pool_query(q, None, 128)
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.select_topk(torch.zeros(1, 2, 3), 1)
    idx = torch.zeros(1, 1, 1, 1, dtype=torch.int32)
    cnt = torch.ones(1, 1, 1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP device"):
        ops.sparse_attn_bf16(q, q, q, idx, cnt)


def test_plumbing_workload_shape():
    w = workloads.plumbing(0)
    assert tuple(w.q.shape) == (1, 4, 256, 64)
    assert tuple(w.k.shape) == (1, 4, 768, 64) and w.v.shape == w.k.shape
    assert (w.n_qblocks, w.n_kblocks, w.n_hist_blocks, w.k_hist, w.k_total) == (4, 12, 8, 4, 8)
    assert torch.all(w.forced[:, 8:]) and not torch.any(w.forced[:, :8])


def test_matrix_dit_shapes_budget_and_ops():
    w = workloads.matrix_dit(0, heads=1)
    assert tuple(w.q.shape) == (1, 1, 28 * 128, 128)
    assert tuple(w.k.shape) == (1, 1, 303 * 128, 128)
    assert int(w.q_valid.sum()) == 3520 and int(w.k_valid.sum()) == 35200 + 3520
    assert w.q_valid[27 * 128:].sum() == 64          # last query block holds 64 tokens
    assert (w.n_hist_blocks, w.k_hist, w.k_total) == (275, 69, 97)
    assert w.q.dtype == torch.bfloat16
    # 69 history blocks + the 28 current blocks per row: 12,352 keys per query row,
    # 5.3427e11 ops at 24 heads
    idx = torch.cat([torch.arange(69), torch.arange(275, 303)]).int().expand(1, 28, 97)
    cnt = torch.full((1, 28), 97, dtype=torch.int32)
    ops1 = w.attention_ops(idx, cnt)
    assert ops1 == 3520 * 12352 * 2 * 128 * 2
    assert ops1 * 24 == pytest.approx(5.3427e11, rel=1e-4)


def test_int8_workload_outliers():
    w = workloads.matrix_dit(0, heads=1, history_frames=2, int8=True)
    ch = w.meta["outlier_channels"]
    assert len(ch) == 4
    kv = w.k[0, 0, w.k_valid].float()
    rms = kv.pow(2).mean(0).sqrt()
    others = torch.ones(128, dtype=torch.bool)
    others[ch] = False
    assert float(rms[ch].min()) > 5 * float(rms[others].max())


def test_selection_stress_shape_and_forced():
    w = workloads.selection_stress(0, heads=2, history_frames=16)
    nhb = w.n_hist_blocks
    assert nhb == 16 * 880 // 128 and w.k_hist == 64
    hist_forced = w.forced[:, :nhb].sum(1)
    assert torch.all(hist_forced == 8)
    starts = w.meta["anchor_starts"]
    for m in range(w.n_qblocks):
        s = int(starts[m])
        assert torch.all(w.forced[m, s:s + 8])
    assert torch.all(w.forced[:, nhb:])


def test_step_sweep_plan_and_layer_view():
    plan = workloads.step_sweep_plan(0)
    assert len(plan) == 30
    assert {p["fraction"] for p in plan} <= {0.125, 0.25, 0.5}
    assert all(1 <= p["query_frames"] <= 4 for p in plan)
    assert {workloads.budget_blocks(f, 275) for f in (0.125, 0.25, 0.5)} == {34, 69, 138}
    base = workloads.matrix_dit(0, heads=1, history_frames=4, int8=True)
    for nf in (1, 3):
        w = workloads.step_layer_view(base, {"layer": 0, "query_frames": nf, "fraction": 0.5})
        lq = nf * 880
        assert int(w.q_valid.sum()) == lq and w.n_qblocks == -(-lq // 128)
        assert int(w.k_valid[w.n_hist_blocks * 128:].sum()) == lq
        assert torch.all(w.q[:, :, lq:] == 0)


def test_bench_runs_on_one_gpu_only():
    """bench.py --gpus N with N above 1 stops before touching a device, with a
    message that says why (the path shards heads with no exchange)."""
    import subprocess
    import sys
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU" in res.stderr + res.stdout and "--gpus 2" in res.stderr + res.stdout
