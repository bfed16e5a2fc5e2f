"""GPU check of vspec_rocm_paged_decode_step_noalloc, the decode step whose partial
states live in the library's fixed per-GPU scratch array, against
vspec_rocm_paged_decode_step (library or caller workspace) on an identically built pool:
pool bytes (the fused append) and outputs must be equal bit for bit, on two calls in a
row with the second smaller, for f16, int4 and f32 pools.  Plans larger than the scratch
are rejected on the host before any launch."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32, F16, INT4 = 0, 1, 2


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def gpu():
    import torch
    import vspec_rocm

    if not torch.cuda.is_available():
        pytest.fail("no GPU visible for a gpu-marked test")
    vspec_rocm.lib()
    return torch.device("cuda:0")


def _pool_pair(dtype, B, T, Hkv, D, P, seed, dev):
    """Two pools with identical contents (contexts of T - 1 tokens) and one table."""
    import torch
    import vspec_rocm as vr

    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    nblk = (T + P - 1) // P
    nb = B * nblk
    tab = torch.randperm(nb, generator=g, device=dev).to(torch.int32).view(B, nblk).contiguous()
    pools = [vr.PagedPool(dtype, nb, P, Hkv, D, device=dev) for _ in range(2)]
    if dtype == INT4:
        # quantise-on-write appends build the int4 contents (codes, scales, clamp flags)
        k = torch.randn((B, T - 1, Hkv, D), generator=g, device=dev, dtype=torch.float16)
        v = torch.randn((B, T - 1, Hkv, D), generator=g, device=dev, dtype=torch.float16)
        for p in pools:
            vr.kv_append(p, tab, torch.zeros(B, dtype=torch.int32, device=dev), k, v)
    else:
        td = torch.float32 if dtype == F32 else torch.float16
        k = torch.randn(pools[0].k.shape, generator=g, device=dev, dtype=torch.float32).to(td)
        v = torch.randn(pools[0].v.shape, generator=g, device=dev, dtype=torch.float32).to(td)
        for p in pools:
            p.k.copy_(k)
            p.v.copy_(v)
    torch.cuda.synchronize()
    return pools, tab


def _same_bytes(a, b):
    import torch

    for x, y in ((a.k, b.k), (a.v, b.v), (a.ks, b.ks), (a.vs, b.vs), (a.kf, b.kf)):
        if x is not None:
            assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))


@pytest.mark.parametrize("dtype", [F16, INT4, F32])
def test_noalloc_step_matches_decode_step(gpu, dtype):
    import torch
    import vspec_rocm as vr

    L = vr.lib()
    # second call smaller (batch and context); the f32 pool's small batch splits each
    # (sequence, kv head) into partitions, so its combine reads partials from the scratch
    shapes = [(16, 2049, 32, 8, 128, 16), (3, 300, 8, 2, 64, 32)] if dtype != F32 else \
             [(2, 1500, 8, 2, 128, 16), (1, 200, 4, 4, 64, 16)]
    for call, (B, T, Hq, Hkv, D, P) in enumerate(shapes):
        say(f"[noalloc] dtype={dtype} call={call} B={B} T={T} Hq={Hq} Hkv={Hkv} D={D} P={P}")
        (pa, pb), tab = _pool_pair(dtype, B, T, Hkv, D, P, 100 + 10 * dtype + call, gpu)
        g = torch.Generator(device=gpu)
        g.manual_seed(7 + call)
        ctx = torch.full((B,), T, dtype=torch.int32, device=gpu)
        ctx[0] = max(1, T // 3)  # ragged: one shorter context
        q = torch.randn((B, Hq, D), generator=g, device=gpu, dtype=torch.float32)
        kn = torch.randn((B, Hkv, D), generator=g, device=gpu, dtype=torch.float16)
        vn = torch.randn((B, Hkv, D), generator=g, device=gpu, dtype=torch.float16)
        want = torch.full_like(q, float("nan"))
        vr.paged_decode_step(pa, tab, ctx, q, kn, vn, numerics=1, out=want)
        got = torch.full_like(q, float("nan"))
        d = vr.make_decode_desc(pb, tab, ctx, q, got, T, vr.NUMERICS_3BIT)
        ok = L.vspec_rocm_paged_decode_step_noalloc(C.byref(d), kn.data_ptr(), vn.data_ptr(), vr.KV_F16)
        assert ok, vr.last_error()
        torch.cuda.synchronize()
        assert torch.isfinite(want).all()
        assert torch.equal(got, want), float((got - want).abs().max())
        _same_bytes(pa, pb)


def test_noalloc_rejects_plans_beyond_the_scratch(gpu):
    """A chunked split of 16 tokens per workgroup over 64 x 4097 f16 tokens needs far more
    partial states than the scratch holds: rejected on the host, nothing launched."""
    import torch
    import vspec_rocm as vr

    L = vr.lib()
    B, T, Hq, Hkv, D, P = 64, 4097, 32, 8, 128, 16
    pool = vr.PagedPool(F16, 4, P, Hkv, D, device=gpu)
    nblk = (T + P - 1) // P
    tab = torch.zeros((B, nblk), dtype=torch.int32, device=gpu)
    ctx = torch.full((B,), T, dtype=torch.int32, device=gpu)
    q = torch.zeros((B, Hq, D), dtype=torch.float32, device=gpu)
    out = torch.zeros_like(q)
    kn = torch.zeros((B, Hkv, D), dtype=torch.float16, device=gpu)
    d = vr.make_decode_desc(pool, tab, ctx, q, out, T, vr.NUMERICS_PLAIN, partition_tokens=16)
    assert vr.decode_workspace_bytes(d) > (6 << 20)
    assert L.vspec_rocm_paged_decode_step_noalloc(C.byref(d), kn.data_ptr(), kn.data_ptr(), vr.KV_F16) == 0
    assert "scratch" in vr.last_error()
    torch.cuda.synchronize()
    assert torch.count_nonzero(out) == 0  # nothing ran
