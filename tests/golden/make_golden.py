"""Write the golden fixtures of the RCSA path from the pinned CPU oracle.

The reference ships no golden vectors for this path, so these fixtures are
produced by ``oracle/rcsa_oracle.py`` (itself pinned by
tests/test_oracle_pins.py) on the seeded synthetic workloads of
``cast_amd.workloads``.  Each fixture stores a fingerprint of its inputs
(so a drift in the generators is caught) and small slices of the outputs:

  c0_plumbing.npz      C0, H4 D64 bs64: scores, selection, full bf16 and int8
                       layer outputs (stored as fp16), quantiser scales
  c1_dit_bf16.npz      C1, H24 D128 (3520 q x 38720 kv): scores of heads 0-1,
                       selection + margins of every row, attention rows of
                       head 0 for query blocks 0 and 27 (the ragged one)
  c2_dit_int8.npz      C2 (C1 + int8, 4 outlier K channels): scales, key mean,
                       int8 attention rows of head 0, query blocks 0 and 27
  c3_selection.npz     C3 (825 history blocks, k=64 with 8 forced, 10% near
                       ties): selection + margins of every row
  c1_seeds.npz         C1 at seeds 1-4: selection + margins of every row, fp32
  c2_seeds.npz         attention rows of one head (5 * seed mod 24) for query
                       blocks 0 and 27 (C2: the unquantised fp32 rows)

Run from the repository root: ``python tests/golden/make_golden.py``.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from cast_amd import workloads  # noqa: E402
from oracle import rcsa_oracle as orc  # noqa: E402

ATTN_QBLOCKS = (0, 27)


def fingerprint(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            t = t.view(torch.int16)
        h.update(t.numpy().tobytes())
    return h.hexdigest()


def workload_fingerprint(w) -> str:
    return fingerprint(w.q, w.k, w.v, w.q_valid, w.k_valid, w.forced)


def _scores(w, heads=None):
    q, k = w.q, w.k
    if heads is not None:
        q, k = q[:, heads], k[:, heads]
    qhat, _, _ = orc.pool_blocks(q, w.q_valid, w.block_size)
    khat, _, _ = orc.pool_blocks(k, w.k_valid, w.block_size)
    B, H = q.shape[:2]
    return orc.block_scores(qhat, khat).reshape(B * H, qhat.shape[2], khat.shape[2])


def make_c0() -> dict:
    w = workloads.plumbing(0)
    bf = orc.rcsa_layer(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=w.block_size,
                        k_select=w.k_total, forced=w.forced)
    i8 = orc.rcsa_layer(w.q, w.k, w.v, w.q_valid, w.k_valid, block_size=w.block_size,
                        k_select=w.k_total, forced=w.forced, int8=True)
    margin = orc.topk_margin(bf["score"], w.k_total, forced=w.forced)
    return {
        "fingerprint": np.array(workload_fingerprint(w)),
        "score": bf["score"].numpy(), "indices": bf["indices"].numpy(),
        "counts": bf["counts"].numpy(), "margin": margin.numpy(),
        "out_bf16": bf["out"].numpy().astype(np.float16), "lse_bf16": bf["lse"].numpy(),
        "out_int8": i8["out"].numpy().astype(np.float16), "lse_int8": i8["lse"].numpy(),
        "q_scale": i8["q_scale"].numpy(), "k_scale": i8["k_scale"].numpy(),
        "kmean": i8["kmean"].numpy(),
    }


def _selection(w, score):
    idx, cnt = orc.select_topk(score, w.k_total, forced=w.forced)
    margin = orc.topk_margin(score, w.k_total, forced=w.forced)
    return idx, cnt, margin


def make_c1_c2() -> tuple[dict, dict]:
    w = workloads.matrix_dit(0)
    score = _scores(w)
    idx, cnt, margin = _selection(w, score)
    B, H = w.q.shape[:2]
    nqb = w.n_qblocks
    idx4, cnt3 = idx.reshape(B, H, nqb, -1), cnt.reshape(B, H, nqb)
    bs = w.block_size
    out, lse = orc.sparse_attention(w.q, w.k, w.v, idx4, cnt3, w.k_valid, block_m=bs,
                                    block_n=bs, heads=[0], qblocks=list(ATTN_QBLOCKS))
    rows = torch.cat([torch.arange(m * bs, (m + 1) * bs) for m in ATTN_QBLOCKS])
    c1 = {
        "fingerprint": np.array(workload_fingerprint(w)),
        "score_h01": score[:2].numpy(), "indices": idx.numpy().astype(np.int16),
        "counts": cnt.numpy(), "margin": margin.numpy(),
        "attn_rows": rows.numpy(), "out_h0": out[0, 0, rows].numpy(),
        "lse_h0": lse[0, 0, rows].numpy(),
    }
    w8 = workloads.matrix_dit(0, int8=True)
    q8, qs = orc.quantize_query_blocks(w8.q, w8.q_valid, bs)
    km = orc.key_mean(w8.k, w8.k_valid)
    k8, ks = orc.quantize_key_blocks(w8.k, w8.k_valid, bs, km)
    score8 = _scores(w8)
    idx8, cnt8, margin8 = _selection(w8, score8)
    out8, lse8 = orc.sparse_attention_int8(q8, qs, k8, ks, w8.v, idx8.reshape(B, H, nqb, -1),
                                           cnt8.reshape(B, H, nqb), w8.k_valid, block_m=bs,
                                           block_n=bs, heads=[0], qblocks=list(ATTN_QBLOCKS))
    ref_fp, _ = orc.sparse_attention(w8.q, w8.k, w8.v, idx8.reshape(B, H, nqb, -1),
                                     cnt8.reshape(B, H, nqb), w8.k_valid, block_m=bs,
                                     block_n=bs, heads=[0], qblocks=list(ATTN_QBLOCKS))
    c2 = {
        "fingerprint": np.array(workload_fingerprint(w8)),
        "outlier_channels": np.asarray(w8.meta["outlier_channels"]),
        "q_scale": qs.numpy(), "k_scale": ks.numpy(), "kmean": km.numpy(),
        "indices": idx8.numpy().astype(np.int16), "counts": cnt8.numpy(),
        "margin": margin8.numpy(), "attn_rows": rows.numpy(),
        "out_h0": out8[0, 0, rows].numpy(), "lse_h0": lse8[0, 0, rows].numpy(),
        "out_h0_unquantised": ref_fp[0, 0, rows].numpy(),
    }
    return c1, c2


def make_c3() -> dict:
    w = workloads.selection_stress(0)
    score = _scores(w)
    idx, cnt, margin = _selection(w, score)
    return {
        "fingerprint": np.array(workload_fingerprint(w)),
        "indices": idx.numpy().astype(np.int16), "counts": cnt.numpy(),
        "margin": margin.numpy(), "tied_rows": w.meta["tied_rows"].numpy(),
        "anchor_starts": w.meta["anchor_starts"].numpy(),
    }


SEEDS = (1, 2, 3, 4)


def seed_head(seed: int) -> int:
    return (5 * seed) % 24


def make_seeds(int8: bool) -> dict:
    """Selection of every row and fp32 attention rows of one head, per seed."""
    out = {}
    for seed in SEEDS:
        w = workloads.matrix_dit(seed, int8=int8)
        score = _scores(w)
        idx, cnt, margin = _selection(w, score)
        B, H = w.q.shape[:2]
        nqb, bs, h = w.n_qblocks, w.block_size, seed_head(seed)
        o, lse = orc.sparse_attention(w.q, w.k, w.v, idx.reshape(B, H, nqb, -1),
                                      cnt.reshape(B, H, nqb), w.k_valid, block_m=bs,
                                      block_n=bs, heads=[h], qblocks=list(ATTN_QBLOCKS))
        rows = torch.cat([torch.arange(m * bs, (m + 1) * bs) for m in ATTN_QBLOCKS])
        out[f"s{seed}_fingerprint"] = np.array(workload_fingerprint(w))
        out[f"s{seed}_indices"] = idx.numpy().astype(np.int16)
        out[f"s{seed}_counts"] = cnt.numpy()
        out[f"s{seed}_margin"] = margin.numpy()
        out[f"s{seed}_head"] = np.array(h)
        out[f"s{seed}_attn_rows"] = rows.numpy()
        out[f"s{seed}_out"] = o[0, h, rows].numpy()
        out[f"s{seed}_lse"] = lse[0, h, rows].numpy()
        print(f"seed {seed} int8={int8} done", flush=True)
    return out


def main() -> None:
    if sys.argv[1:] == ["seeds"]:  # only the multi-seed fixtures
        torch.set_num_threads(min(8, os.cpu_count() or 1))
        np.savez_compressed(os.path.join(HERE, "c1_seeds.npz"), **make_seeds(False))
        np.savez_compressed(os.path.join(HERE, "c2_seeds.npz"), **make_seeds(True))
        return
    torch.set_num_threads(min(8, os.cpu_count() or 1))
    np.savez_compressed(os.path.join(HERE, "c0_plumbing.npz"), **make_c0())
    c1, c2 = make_c1_c2()
    np.savez_compressed(os.path.join(HERE, "c1_dit_bf16.npz"), **c1)
    np.savez_compressed(os.path.join(HERE, "c2_dit_int8.npz"), **c2)
    np.savez_compressed(os.path.join(HERE, "c3_selection.npz"), **make_c3())
    np.savez_compressed(os.path.join(HERE, "c1_seeds.npz"), **make_seeds(False))
    np.savez_compressed(os.path.join(HERE, "c2_seeds.npz"), **make_seeds(True))
    for name in sorted(os.listdir(HERE)):
        if name.endswith(".npz"):
            print(f"{name}: {os.path.getsize(os.path.join(HERE, name))} bytes")


if __name__ == "__main__":
    main()
