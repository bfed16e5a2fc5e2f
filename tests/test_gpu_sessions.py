"""GPU parity of the session layer: the handle API (vspec_py_kv_cache_*) over HBM
against the reference's own paged cache (kv_paged_cache.c compiled into oracle/_ref),
driven through the same seeded operation sequence.  Reads are bit-exact; decode over a
handle's pool through allocator-built block tables matches the reference's GQA
attention over the same tokens to the fp32 bar (1e-4)."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
_f32p = C.POINTER(C.c_float)


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


def _ref_read(ref, c, sid, H, D):
    n = ref.lib.vspec_kv_paged_session_tokens(c, sid)
    k = np.zeros((max(n, 1), H, D), np.float32)
    v = np.zeros_like(k)
    got = ref.lib.vr_paged_read(c, sid, k.ctypes.data_as(_f32p), v.ctypes.data_as(_f32p), 0)
    return k[:got], v[:got]


@pytest.mark.parametrize("P,MAXP,H,D,seed", [(16, 24, 2, 128, 1), (5, 13, 3, 12, 2), (32, 9, 1, 64, 3)])
def test_handles_match_reference_cache(ref, gpu, P, MAXP, H, D, seed):
    from vspec_rocm.sessions import CorePagedKVCache

    say(f"[sessions] P={P} MAXP={MAXP} H={H} D={D} seed={seed}")
    rng = np.random.default_rng(seed)
    cache = CorePagedKVCache(P, MAXP, H, D)
    c = ref.lib.vr_paged_new(P, MAXP, H, D)
    ids = [int(x) for x in rng.integers(0, 7, 10)]
    try:
        for step in range(500):
            op = int(rng.integers(0, 12))
            a, b = int(rng.choice(ids)), int(rng.choice(ids))
            if op <= 7:
                k = rng.standard_normal((H, D)).astype(np.float32)
                v = rng.standard_normal((H, D)).astype(np.float32)
                r1 = cache.append(k, v, session_id=a)
                r2 = ref.lib.vspec_kv_paged_append(c, a, k.ctypes.data_as(_f32p), v.ctypes.data_as(_f32p))
                assert r1 == bool(r2), step
            elif op == 8:
                assert cache.open_session(a) == bool(ref.lib.vspec_kv_paged_open_session(c, a))
            elif op == 9:
                assert cache.close_session(a) == bool(ref.lib.vspec_kv_paged_close_session(c, a))
            else:
                mt = int(rng.integers(0, 3 * P))
                assert cache.reuse_prefix(a, b, mt) == bool(ref.lib.vspec_kv_paged_reuse_prefix(c, a, b, mt))
            if step % 50 == 49 or step == 499:
                for s in sorted(set(ids)):
                    assert cache.session_tokens(s) == ref.lib.vspec_kv_paged_session_tokens(c, s)
                    wk, wv = _ref_read(ref, c, s, H, D)
                    gk, gv = cache.read_tokens(session_id=s)
                    if wk.shape[0] == 0:
                        assert gk is not None and gk.shape[0] == 0
                        continue
                    assert gk.shape == wk.shape
                    assert np.array_equal(gk.view(np.uint32), wk.view(np.uint32)), (step, s)
                    assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), (step, s)
                    # a bounded read returns the prefix
                    m = max(1, wk.shape[0] // 2)
                    pk, _ = cache.read_tokens(max_tokens=m, session_id=s)
                    assert np.array_equal(pk, wk[:m])
        st = cache.stats()
        out = (C.c_uint64 * 6)()
        ref.lib.vr_paged_stats(c, out)
        assert list(st.values()) == list(out)
        say(f"[sessions] stats {st}")
    finally:
        cache.close()
        ref.lib.vr_paged_free(c)


def test_reset_and_handle_table(gpu):
    from vspec_rocm import VspecRocmError, lib
    from vspec_rocm.sessions import CorePagedKVCache

    a = CorePagedKVCache(16, 4, 1, 8, session_id=5)
    x = np.arange(8, dtype=np.float32)
    for _ in range(20):
        assert a.append(x, -x)
    assert a.session_tokens() == 20
    k, v = a.read_tokens()
    assert np.array_equal(k[:, 0], np.tile(x, (20, 1))) and np.array_equal(v[:, 0], np.tile(-x, (20, 1)))
    a.reset()
    assert a.session_tokens() == 0
    k, v = a.read_tokens()
    assert k.shape == (0, 1, 8)
    # 16 handles at most, as in the reference
    extra = []
    try:
        while len(extra) < 20:
            extra.append(CorePagedKVCache(16, 1, 1, 8))
    except VspecRocmError:
        pass
    assert len(extra) == 15
    for e in extra:
        e.close()
    a.close()
    assert lib().vspec_py_kv_cache_append(a.handle, 5, None, None) == 0


@pytest.mark.parametrize("mode", [0, 1])
def test_decode_over_handle_pool(ref, gpu, mode):
    """Sessions filled through the handle API, one sharing a page-aligned prefix;
    block tables from the allocator; decode on the handle's f32 pool."""
    import torch
    import vspec_rocm as vr
    from vspec_rocm.sessions import CorePagedKVCache

    P, H, D, Hq = 16, 2, 64, 8
    rng = np.random.default_rng(7 + mode)
    lens = {1: 173, 2: 64, 3: 300, 4: 1}
    cache = CorePagedKVCache(P, 64, H, D)
    try:
        for sid, n in lens.items():
            for _ in range(n):
                assert cache.append(rng.standard_normal((H, D)), rng.standard_normal((H, D)), session_id=sid)
        # session 5 shares session 3's first 96 tokens (6 full pages), then grows
        assert cache.reuse_prefix(5, 3, 96)
        for _ in range(21):
            assert cache.append(rng.standard_normal((H, D)), rng.standard_normal((H, D)), session_id=5)
        # sharing whole pages up to 40 tokens takes 2 pages; sharing everything takes
        # session 1's partly filled last page, which then sits in the middle of session 7
        assert cache.reuse_prefix(6, 1, 40)
        cache.append(rng.standard_normal((H, D)), rng.standard_normal((H, D)), session_id=6)
        assert cache.block_table(6, 32)[1] == 33
        assert cache.reuse_prefix(7, 1, 0)
        cache.append(rng.standard_normal((H, D)), rng.standard_normal((H, D)), session_id=7)
        assert cache.session_tokens(7) == 174
        # a plain block table cannot express session 7 (its shared page with 13 tokens sits
        # in the middle); the layout with per-block used counts can
        assert cache.block_table(7, 32) is None
        sids = [1, 2, 3, 4, 5]
        tabs, ctx = [], []
        for s in sids:
            t, n = cache.block_table(s, 32)
            tabs.append(t)
            ctx.append(n)
        assert ctx == [173, 64, 300, 1, 117]
        q = rng.standard_normal((len(sids) + 1, Hq, D)).astype(np.float32)
        pool = cache.device_pool()
        out = vr.paged_decode(pool, torch.from_numpy(np.stack(tabs)).to(gpu),
                              torch.tensor(ctx, dtype=torch.int32, device=gpu),
                              torch.from_numpy(q[: len(sids)]).to(gpu), numerics=mode)
        got = out.cpu().numpy()
        for i, s in enumerate(sids):
            k, v = cache.read_tokens(session_id=s)
            want = ref.attention_gqa(mode, q[i], k, v)
            err = float(np.abs(got[i] - want).max())
            assert err <= 2e-5, (s, err)
        # every session through block layouts, session 7 included
        lay = [cache.block_layout(s, 32) for s in sids + [7]]
        assert lay[-1][3] == 174 and lay[-1][2] == 11 * 16 + 1 and (lay[-1][1][:11] < 16).any()
        out = vr.paged_decode(pool, torch.from_numpy(np.stack([l[0] for l in lay])).to(gpu),
                              torch.tensor([l[2] for l in lay], dtype=torch.int32, device=gpu),
                              torch.from_numpy(q).to(gpu), numerics=mode,
                              block_used=torch.from_numpy(np.stack([l[1] for l in lay])).to(gpu))
        got = out.cpu().numpy()
        for i, s in enumerate(sids + [7]):
            k, v = cache.read_tokens(session_id=s)
            want = ref.attention_gqa(mode, q[i], k, v)
            err = float(np.abs(got[i] - want).max())
            assert err <= 2e-5, (s, err)
    finally:
        cache.close()


@pytest.mark.parametrize("dtype", [1, 2])  # f16, int4 pools
def test_continuous_batching_steps(oracle, ref, gpu, dtype):
    """Steps of the reference scheduler (continuous_batch.c) run end to end: the host
    allocator plans each step, one packed append writes the mixed chunked-prefill and
    decode tokens (quantised on write for int4), and the decode-phase items attend over
    their caches.  The pool matches the oracle's bit for bit after every step and the
    outputs match the oracle's attention (4e-3)."""
    import torch
    import vspec_rocm as vr
    from oracle.oracle import HostPool
    from test_paged_meta_cpu import _ref_batcher_steps
    from vspec_rocm.sessions import plan_step

    P, MAXP, Hkv, Hq, D = 16, 96, 2, 8, 128
    m = vr.lib().vspec_rocm_paged_meta_create(P, MAXP, 0, 0)
    pool = vr.PagedPool(dtype, MAXP, P, Hkv, D, device=gpu)
    host = HostPool(dtype, MAXP, P, Hkv, D)
    rng = np.random.default_rng(10 + dtype)
    try:
        for si, step in enumerate(_ref_batcher_steps(ref, 20 + dtype, n_req=5, max_items=6, max_tokens=48,
                                                     prefill_q=24)):
            plan = plan_step(m, step, max_blocks=16)
            n = plan["token_item"].size
            k16 = oracle.f32_to_f16(rng.standard_normal((n, Hkv, D)).astype(np.float32))
            v16 = oracle.f32_to_f16(rng.standard_normal((n, Hkv, D)).astype(np.float32))
            tabs = plan["block_tables"]
            for i, it in enumerate(step):  # oracle: per item, its tokens in order
                sel = np.flatnonzero(plan["token_item"] == i)
                assert oracle.paged_append(host, np.ascontiguousarray(tabs[i:i + 1]), plan["start_pos"][i:i + 1],
                                           np.ascontiguousarray(k16[sel][None]), np.ascontiguousarray(v16[sel][None]))
            dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
            kd = torch.from_numpy(k16.view(np.int16)).to(gpu).view(torch.float16)
            vd = torch.from_numpy(v16.view(np.int16)).to(gpu).view(torch.float16)
            vr.kv_append_tokens(pool, dev(plan["token_item"]), dev(plan["token_pos"]), dev(tabs), kd, vd)
            torch.cuda.synchronize()
            from test_gpu_parity import assert_pools_equal
            assert_pools_equal(host, pool)
            dec = [i for i, it in enumerate(step) if it.phase == 2]
            if dec:
                q = rng.standard_normal((len(dec), Hq, D)).astype(np.float32)
                t_sub = np.ascontiguousarray(tabs[dec])
                c_sub = np.ascontiguousarray(plan["ctx_lens"][dec])
                got = vr.paged_decode(pool, dev(t_sub), dev(c_sub), dev(q), numerics=si % 2).cpu().numpy()
                want = oracle.paged_decode(si % 2, host, t_sub, c_sub, q)
                err = float(np.abs(got - want).max())
                assert err <= 4e-3, (si, err)
        say(f"[cb] dtype={dtype} steps={si + 1}")
    finally:
        vr.lib().vspec_rocm_paged_meta_destroy(m)


def _pool_rows(lib, pool, tab, used, P, dev):
    """A session's rows [n][Hkv][D] as f32 through the row gather, in the order the
    reference's get_token_ptr walk visits them (entry by entry, used slots each)."""
    import ctypes as C
    import torch

    pos = [e * P + s for e in range(len(used)) if tab[e] >= 0 for s in range(int(used[e]))]
    pages = torch.tensor([int(tab[p // P]) for p in pos], dtype=torch.int32, device=dev)
    slots = torch.tensor([p % P for p in pos], dtype=torch.int32, device=dev)
    n = len(pos)
    ok = torch.empty((n, pool.num_kv_heads, pool.head_dim), dtype=torch.float32, device=dev)
    ov = torch.empty_like(ok)
    d = pool.desc()
    assert lib.vspec_rocm_kv_gather_rows(C.byref(d), n, pages.data_ptr(), slots.data_ptr(), ok.data_ptr(),
                                         ov.data_ptr(), None) == 1
    torch.cuda.synchronize()
    return ok.cpu().numpy(), ov.cpu().numpy()


@pytest.mark.parametrize("dtype", [0, 1, 2])  # f32, f16, int4 pools
def test_partial_middle_pages_decode(oracle, ref, gpu, dtype):
    """Prefix reuse of a partly filled page (kv_paged_cache.c:223-234) leaves it in the
    middle of the target and, once the source appends again (a new page: :276), of the
    source.  Steps planned with block_used append through kv_append_tokens at slot-space
    positions, with the reference paged cache appending the same tokens; every session
    then decodes in one batch (block tables, used counts, spans), and a fused decode step
    appends one more token to each.  The pool rows equal the reference cache's walk bit
    for bit (f32, and f16 as its exact f32 values) and the outputs match attention_ref
    over the reference's gathered rows (int4: over the pool's dequantised rows)."""
    import torch
    import vspec_rocm as vr
    from vspec_rocm.sessions import plan_step

    P, MAXP, Hkv, Hq, D, MB = 16, 160, 2, 8, 128, 16
    L = vr.lib()
    m = L.vspec_rocm_paged_meta_create(P, MAXP, 0, 0)
    pool = vr.PagedPool(dtype, MAXP, P, Hkv, D, device=gpu)
    c = ref.lib.vr_paged_new(P, MAXP, Hkv, D)
    rng = np.random.default_rng(40 + dtype)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)

    def tokens(n):
        k = rng.standard_normal((n, Hkv, D)).astype(np.float32)
        v = rng.standard_normal((n, Hkv, D)).astype(np.float32)
        if dtype == 0:
            return k, v, dev(k), dev(v)
        k16, v16 = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
        to16 = lambda h: torch.from_numpy(h.view(np.int16).copy()).view(torch.float16).to(gpu)
        return oracle.f16_to_f32(k16), oracle.f16_to_f32(v16), to16(k16), to16(v16)

    def run(items):
        plan = plan_step(m, items, max_blocks=MB, with_used=True)
        n = plan["token_item"].size
        kf, vf, kd, vd = tokens(n)
        for t in range(n):
            sid = items[int(plan["token_item"][t])][0]
            assert ref.lib.vspec_kv_paged_append(c, sid, kf[t].ctypes.data_as(_f32p), vf[t].ctypes.data_as(_f32p))
        vr.kv_append_tokens(pool, dev(plan["token_item"]), dev(plan["token_pos"]), dev(plan["block_tables"]), kd, vd)
        return plan

    def reuse(t, s_, mt):
        assert L.vspec_rocm_paged_reuse_prefix(m, t, s_, mt) == ref.lib.vspec_kv_paged_reuse_prefix(c, t, s_, mt) == 1

    def layouts(sids):
        tabs, used, spans = [], [], []
        for s_ in sids:
            tb = np.full(MB, -1, np.int32)
            us = np.zeros(MB, np.int32)
            sp, nt = C.c_uint32(), C.c_uint32()
            assert L.vspec_rocm_paged_block_layout(m, s_, tb.ctypes.data_as(C.POINTER(C.c_int32)),
                                                   us.ctypes.data_as(C.POINTER(C.c_int32)), MB, C.byref(sp),
                                                   C.byref(nt))
            assert nt.value == ref.lib.vspec_kv_paged_session_tokens(c, s_)
            tabs.append(tb)
            used.append(us)
            spans.append(sp.value)
        return np.stack(tabs), np.stack(used), np.array(spans, np.int32)

    def expected(mode, sids, tabs, used, q):
        out, vmax = [], 0.0
        for i, s_ in enumerate(sids):
            n = ref.lib.vspec_kv_paged_session_tokens(c, s_)
            rk = np.zeros((n, Hkv, D), np.float32)
            rv = np.zeros_like(rk)
            assert ref.lib.vr_paged_read(c, s_, rk.ctypes.data_as(_f32p), rv.ctypes.data_as(_f32p), 0) == n
            gk, gv = _pool_rows(L, pool, tabs[i], used[i], P, gpu)
            if dtype != 2:
                # the pool holds exactly the reference cache's values, in its walk order
                assert np.array_equal(gk, rk) and np.array_equal(gv, rv), s_
                k, v = rk, rv
            else:
                k, v = gk, gv
            vmax = max(vmax, float(np.abs(v).max()))
            out.append(ref.attention_gqa(mode, q[i], k, v))
        tol = 2e-5 if dtype != 2 else min(4e-3, 2.5e-4 * vmax + 2e-5)
        return np.stack(out), tol

    try:
        say(f"[partial pages] dtype={dtype}")
        run([(1, 1, 37, 0)])                           # 2 full pages + 5 tokens
        run([(2, 1, 16, 0), (3, 1, 50, 0)])
        reuse(5, 1, 0)                                 # shares 1's partly filled page
        reuse(6, 3, 40)                                # two whole pages (32 tokens)
        run([(5, 1, 20, 0), (1, 1, 7, 0), (6, 1, 3, 0)])   # 5 and 1 open pages after it
        reuse(7, 5, 0)
        run([(7, 1, 3, 0), (2, 1, 1, 0)])
        sids = [1, 2, 3, 5, 6, 7]
        tabs, used, spans = layouts(sids)
        npages = (tabs >= 0).sum(1)
        assert any((used[i, : npages[i] - 1] < P).any() for i in range(len(sids)))  # partial middle pages
        q = rng.standard_normal((len(sids), Hq, D)).astype(np.float32)
        for mode in (1, 0):
            got = vr.paged_decode(pool, dev(tabs), dev(spans), dev(q), numerics=mode, block_used=dev(used)).cpu().numpy()
            want, tol = expected(mode, sids, tabs, used, q)
            err = float(np.abs(got - want).max())
            say(f"    decode mode={mode} max-abs {err:.2e} (bound {tol:.1e})")
            assert err <= tol
        # fused decode step: one new token per session at its span (planned with block_used)
        plan = plan_step(m, [(s_, 2, 1, 0) for s_ in sids], max_blocks=MB, with_used=True)
        assert (plan["token_pos"] == plan["ctx_lens"] - 1).all()
        kf, vf, kd, vd = tokens(len(sids))
        for i, s_ in enumerate(sids):
            assert ref.lib.vspec_kv_paged_append(c, s_, kf[i].ctypes.data_as(_f32p), vf[i].ctypes.data_as(_f32p))
        got = vr.paged_decode_step(pool, dev(plan["block_tables"]), dev(plan["ctx_lens"]), dev(q), kd, vd,
                                   numerics=1, block_used=dev(plan["block_used"])).cpu().numpy()
        tabs2, used2, spans2 = layouts(sids)
        assert (tabs2 == plan["block_tables"]).all() and (used2 == plan["block_used"]).all()
        want, tol = expected(1, sids, tabs2, used2, q)
        err = float(np.abs(got - want).max())
        say(f"    decode step max-abs {err:.2e} (bound {tol:.1e})")
        assert err <= tol
    finally:
        L.vspec_rocm_paged_meta_destroy(m)
        ref.lib.vr_paged_free(c)
