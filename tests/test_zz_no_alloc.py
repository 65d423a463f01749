"""rcsa_sparse_attn_int8_noalloc (static scratch, no allocation) against
rcsa_sparse_attn_int8_split (caller's workspace), through the C ABI.

Two calls in a row on split shapes, the second smaller, each bit-identical to
the split entry point with a torch-allocated workspace; a split that would not
fit the static scratch is refused with RCSA_ERR_SCRATCH before any launch.
"""
import math

import pytest
import torch

pytestmark = pytest.mark.gpu

RCSA_ERR_SCRATCH = 7


def _inputs(seed, H, nqb, nkb, max_k, dev):
    g = torch.Generator().manual_seed(seed)
    bs, D = 128, 128
    q8 = torch.randint(-127, 128, (1, H, nqb * bs, D), generator=g, dtype=torch.int8)
    k8 = torch.randint(-127, 128, (1, H, nkb * bs, D), generator=g, dtype=torch.int8)
    v = (torch.randn(1, H, nkb * bs, D, generator=g) * 0.5).bfloat16()
    qs = torch.rand(H, nqb, generator=g) * 1e-3 + 1e-4
    ks = torch.rand(H, nkb, generator=g) * 1e-3 + 1e-4
    idx = torch.stack([torch.randperm(nkb, generator=g)[:max_k].sort().values
                       for _ in range(H * nqb)]).reshape(1, H, nqb, max_k).int()
    cnt = torch.randint(max_k // 2, max_k + 1, (1, H, nqb), generator=g, dtype=torch.int32)
    return [t.to(dev) for t in (q8, qs, k8, ks, v, idx, cnt)]


def _call(lib, name, q8, qs, k8, ks, v, idx, cnt, n_split, extra):
    B, H, Lq, D = q8.shape
    Lk = k8.shape[2]
    out = torch.full((B, H, Lq, D), float("nan"), dtype=torch.bfloat16, device=q8.device)
    lse = torch.full((B, H, Lq), float("nan"), dtype=torch.float32, device=q8.device)
    fn = getattr(lib, name)
    st = fn(q8.data_ptr(), qs.data_ptr(), qs.shape[1], k8.data_ptr(), ks.data_ptr(),
            ks.shape[1], v.data_ptr(), None, None, 1.0 / math.sqrt(D), lse.data_ptr(),
            out.data_ptr(), idx.data_ptr(), cnt.data_ptr(), *q8.stride()[:3],
            *k8.stride()[:3], *v.stride()[:3], *out.stride()[:3], *idx.stride()[:3],
            *cnt.stride(), B, H, Lq, Lk, D, 128, 128, idx.shape[-1], n_split, *extra,
            None, 0, None, 0, torch.cuda.current_stream().cuda_stream)
    return st, out, lse


def test_noalloc_matches_split_entry_point(dev):
    from cast_amd import _lib
    lib = _lib.load()
    assert lib.rcsa_attn_noalloc_scratch_bytes() == 32 << 20
    # 24 heads x 28 query blocks: 84 items per XCD, two full rounds (the kernel of three
    # workgroups per compute unit) + 20 tail items each; then 12 heads x 28 query
    # blocks: 42 items per XCD -> 32 whole + 10 tail items each; then 2 heads x 20
    # query blocks: 5 items per XCD, all tail items (each call smaller than the last)
    for seed, H, nqb, nkb, max_k, n_split in ((3, 24, 28, 40, 24, 3), (1, 12, 28, 40, 24, 3),
                                              (2, 2, 20, 16, 10, 4)):
        print(f"noalloc H{H} nqb{nqb} nkb{nkb} max_k{max_k} n_split{n_split}", flush=True)
        args = _inputs(seed, H, nqb, nkb, max_k, dev)
        nbytes = int(lib.rcsa_attn_workspace_bytes(1, H, nqb * 128, 128, n_split))
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        st_a, out_a, lse_a = _call(lib, "rcsa_sparse_attn_int8_split", *args, n_split,
                                   (ws.data_ptr(), nbytes))
        st_b, out_b, lse_b = _call(lib, "rcsa_sparse_attn_int8_noalloc", *args, n_split, ())
        torch.cuda.synchronize()
        assert st_a == 0 and st_b == 0, (st_a, st_b)
        assert torch.equal(out_a, out_b) and torch.equal(lse_a, lse_b)
        assert not torch.isnan(out_b.float()).any()


def test_noalloc_refuses_oversized_split(dev):
    """24 heads x 28 query blocks at n_split 8: 160 tail query blocks x 8 shares of
    128 x 128 bf16 partials (42 MB) exceed the 32 MiB scratch."""
    from cast_amd import _lib
    lib = _lib.load()
    args = _inputs(3, 24, 28, 4, 2, dev)
    st, out, _ = _call(lib, "rcsa_sparse_attn_int8_noalloc", *args, 8, ())
    torch.cuda.synchronize()
    assert st == RCSA_ERR_SCRATCH
    assert b"scratch" in lib.rcsa_status_string(st)
    assert torch.isnan(out.float()).all()  # nothing was launched
