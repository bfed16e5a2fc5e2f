"""The host allocator (csrc/paged_meta.c) against the reference's own kv_paged_cache.c
compiled into oracle/_ref: identical return values, page placement, page metadata and
statistics over seeded random operation sequences, plus the known answer of the
reference's profiler driver (tools/profiler/kv_paged_cache_profiler.c).  CPU only."""
import ctypes as C

import numpy as np
import pytest

_f32p = C.POINTER(C.c_float)


@pytest.fixture(scope="module")
def lib():
    import vspec_rocm

    return vspec_rocm.lib()


def _stats(lib, m):
    import vspec_rocm

    st = vspec_rocm.VspecRocmPagedStats()
    lib.vspec_rocm_paged_stats(m, C.byref(st))
    return [st.page_alloc_count, st.page_reuse_count, st.evict_session_count, st.append_token_count,
            st.free_pages, st.active_sessions]


def _ref_stats(ref, c):
    out = (C.c_uint64 * 6)()
    ref.lib.vr_paged_stats(c, out)
    return list(out)


def _ref_locate(ref, c, P, H, D, sid, t):
    """get_token_ptr -> (page, slot) from the returned pointer offset."""
    kp = _f32p()
    vp = _f32p()
    ok = ref.lib.vspec_kv_paged_get_token_ptr(c, sid, t, 0, C.byref(kp), C.byref(vp))
    if not ok:
        return None
    base = C.cast(ref.lib.vr_paged_key_pages(c), C.c_void_p).value
    off = (C.cast(kp, C.c_void_p).value - base) // 4
    page, rem = divmod(off, P * H * D)
    return page, rem // (H * D)


def test_profiler_known_answer(lib):
    """kv_paged_cache_profiler.c: P=32, 128 pages; 1001 appends 120, 1002 reuses a
    64-token prefix then appends 96; probe token 48 lands in page 1 slot 16."""
    m = lib.vspec_rocm_paged_meta_create(32, 128, 0, 0)
    assert m
    u32 = C.c_uint32
    pg, sl = u32(), u32()
    assert lib.vspec_rocm_paged_open_session(m, 1001)
    for _ in range(120):
        assert lib.vspec_rocm_paged_reserve(m, 1001, C.byref(pg), C.byref(sl))
    assert lib.vspec_rocm_paged_open_session(m, 1002)
    assert lib.vspec_rocm_paged_reuse_prefix(m, 1002, 1001, 64)
    for _ in range(96):
        assert lib.vspec_rocm_paged_reserve(m, 1002, C.byref(pg), C.byref(sl))
    assert lib.vspec_rocm_paged_locate(m, 1002, 48, C.byref(pg), C.byref(sl))
    assert (pg.value, sl.value) == (1, 16)
    assert _stats(lib, m) == [7, 2, 0, 216, 121, 2]
    assert lib.vspec_rocm_paged_session_tokens(m, 1001) == 120
    assert lib.vspec_rocm_paged_session_tokens(m, 1002) == 160
    lib.vspec_rocm_paged_meta_destroy(m)


@pytest.mark.parametrize("seed", range(6))
def test_matches_reference_allocator(lib, ref, seed):
    rng = np.random.default_rng(seed)
    P, MAXP, H, D = 4, int(rng.integers(6, 40)), 2, 8
    m = lib.vspec_rocm_paged_meta_create(P, MAXP, 0, 0)
    c = ref.lib.vr_paged_new(P, MAXP, H, D)
    tok = np.zeros(H * D, np.float32)
    u32 = C.c_uint32
    pg, sl = u32(), u32()
    ids = [int(x) for x in rng.integers(0, 9, 12)]  # 0 is an invalid session id
    try:
        for step in range(600):
            op = rng.integers(0, 10)
            a, b = int(rng.choice(ids)), int(rng.choice(ids))
            if op <= 5:
                r1 = lib.vspec_rocm_paged_reserve(m, a, C.byref(pg), C.byref(sl))
                r2 = ref.lib.vspec_kv_paged_append(c, a, tok.ctypes.data_as(_f32p), tok.ctypes.data_as(_f32p))
                assert r1 == r2, step
                if r1:
                    n = lib.vspec_rocm_paged_session_tokens(m, a)
                    assert _ref_locate(ref, c, P, H, D, a, n - 1) == (pg.value, sl.value), step
            elif op == 6:
                assert lib.vspec_rocm_paged_open_session(m, a) == ref.lib.vspec_kv_paged_open_session(c, a)
            elif op == 7:
                assert lib.vspec_rocm_paged_close_session(m, a) == ref.lib.vspec_kv_paged_close_session(c, a)
            elif op == 8:
                mt = int(rng.integers(0, 12))
                assert lib.vspec_rocm_paged_reuse_prefix(m, a, b, mt) == ref.lib.vspec_kv_paged_reuse_prefix(c, a, b, mt)
            assert _stats(lib, m) == _ref_stats(ref, c), step
            for s in set(ids):
                n = lib.vspec_rocm_paged_session_tokens(m, s)
                assert n == ref.lib.vspec_kv_paged_session_tokens(c, s)
                pages = (C.c_uint32 * 1024)()
                rpages = (C.c_uint32 * 1024)()
                k1 = lib.vspec_rocm_paged_session_pages(m, s, pages, 1024)
                k2 = ref.lib.vr_paged_session_pages(c, s, rpages, 1024)
                assert k1 == k2 and list(pages[:k1]) == list(rpages[:k2])
                if n:
                    t = int(rng.integers(0, n))
                    assert lib.vspec_rocm_paged_locate(m, s, t, C.byref(pg), C.byref(sl))
                    assert _ref_locate(ref, c, P, H, D, s, t) == (pg.value, sl.value)
        for p in range(MAXP):
            mine = [C.c_uint32() for _ in range(3)]
            theirs = [C.c_uint32() for _ in range(3)]
            lib.vspec_rocm_paged_page_info(m, p, *[C.byref(x) for x in mine])
            ref.lib.vr_paged_page_meta(c, p, *[C.byref(x) for x in theirs])
            assert [x.value for x in mine] == [x.value for x in theirs]
    finally:
        lib.vspec_rocm_paged_meta_destroy(m)
        ref.lib.vr_paged_free(c)


def test_session_table_eviction_matches_reference(lib, ref):
    """More sessions than the reference's 128 slots: whole-session LRU eviction on open."""
    m = lib.vspec_rocm_paged_meta_create(16, 4096, 0, 0)
    c = ref.lib.vr_paged_new(16, 4096, 1, 8)
    tok = np.zeros(8, np.float32)
    try:
        for sid in range(1, 300):
            assert lib.vspec_rocm_paged_reserve(m, sid, None, None) == ref.lib.vspec_kv_paged_append(
                c, sid, tok.ctypes.data_as(_f32p), tok.ctypes.data_as(_f32p))
            assert _stats(lib, m) == _ref_stats(ref, c)
    finally:
        lib.vspec_rocm_paged_meta_destroy(m)
        ref.lib.vr_paged_free(c)


def test_caps_lifted_beyond_reference(lib):
    """16448 pages (the north-star batch) and 2048 pages per session are accepted."""
    m = lib.vspec_rocm_paged_meta_create(16, 16448, 0, 4096)
    assert m
    for _ in range(2048 * 16):
        assert lib.vspec_rocm_paged_reserve(m, 7, None, None)
    tab = (C.c_int32 * 4096)()
    ctx = C.c_uint32()
    assert lib.vspec_rocm_paged_block_table(m, 7, tab, 4096, C.byref(ctx))
    assert ctx.value == 32768 and list(tab[:3]) == [0, 1, 2]
    lib.vspec_rocm_paged_meta_destroy(m)


def test_block_table_refuses_partial_middle_pages(lib):
    m = lib.vspec_rocm_paged_meta_create(4, 64, 0, 0)
    for _ in range(6):  # 1 full page + a page with 2 tokens
        lib.vspec_rocm_paged_reserve(m, 1, None, None)
    assert lib.vspec_rocm_paged_reuse_prefix(m, 2, 1, 0)  # shares the partial page too
    lib.vspec_rocm_paged_reserve(m, 2, None, None)        # opens a new page after it
    tab = (C.c_int32 * 8)()
    assert not lib.vspec_rocm_paged_block_table(m, 2, tab, 8, None)
    assert lib.vspec_rocm_paged_block_table(m, 1, tab, 8, None)
    lib.vspec_rocm_paged_meta_destroy(m)


def _ref_batcher_steps(ref, seed, n_req=6, max_items=8, max_tokens=64, prefill_q=32):
    """Drive the reference continuous batcher (continuous_batch.c) to completion,
    yielding each step's items and committing them afterwards."""
    import vspec_rocm

    assert ref.lib.vr_batch_item_size() == C.sizeof(vspec_rocm.VspecRocmStepItem)
    rng = np.random.default_rng(seed)
    bt = ref.lib.vr_batcher_new(1 << 40, 16, max_items, max_tokens, prefill_q, 1)
    try:
        rid = C.c_uint64()
        for _ in range(n_req):
            assert ref.lib.vspec_continuous_batch_submit(bt, 1 << 20, int(rng.integers(1, 150)),
                                                         int(rng.integers(1, 12)), 0, C.byref(rid))
        items = (vspec_rocm.VspecRocmStepItem * max_items)()
        for _ in range(400):
            k = ref.lib.vspec_continuous_batch_next_batch(bt, items, max_items)
            if k == 0:
                return
            step = [vspec_rocm.VspecRocmStepItem(items[i].request_id, items[i].phase, items[i].token_quota,
                                                 items[i].prompt_cursor) for i in range(k)]
            yield step
            for it in step:
                if it.phase == 1:
                    assert ref.lib.vspec_continuous_batch_commit_prefill(bt, it.request_id, it.token_quota)
                else:
                    assert ref.lib.vspec_continuous_batch_commit_decode(bt, it.request_id, it.token_quota, 0)
        raise AssertionError("batcher did not drain")
    finally:
        ref.lib.vr_batcher_free(bt)


@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("kept", [False, True])
def test_plan_step_follows_reference_scheduler(lib, ref, seed, kept):
    """Steps of the reference scheduler planned on the host allocator: the packed token
    map, start positions and context lengths are consistent, and every position of every
    item maps through its block table to the page and slot the reference paged cache
    (appending the same tokens) holds it in.  kept: the tables are kept between steps and
    only updated (vspec_rocm_paged_plan_step_update)."""
    from vspec_rocm.sessions import StepPlanner, plan_step

    P, MAXP, H, D = 16, 512, 1, 8
    m = lib.vspec_rocm_paged_meta_create(P, MAXP, 0, 0)
    c = ref.lib.vr_paged_new(P, MAXP, H, D)
    tok = np.zeros(H * D, np.float32)
    nsteps = 0
    planner = StepPlanner(m, max_items=8, max_blocks=64, max_tokens=8 * 64) if kept else None
    try:
        for step in _ref_batcher_steps(ref, seed):
            nsteps += 1
            plan = planner.step(step) if kept else plan_step(m, step, max_blocks=64)
            off = 0
            for i, it in enumerate(step):
                q = int(it.token_quota)
                assert (plan["token_item"][off:off + q] == i).all()
                assert (plan["token_pos"][off:off + q] == plan["start_pos"][i] + np.arange(q)).all()
                assert plan["ctx_lens"][i] == plan["start_pos"][i] + q
                off += q
                for _ in range(q):
                    assert ref.lib.vspec_kv_paged_append(c, it.request_id, tok.ctypes.data_as(_f32p),
                                                         tok.ctypes.data_as(_f32p))
            assert off == plan["token_item"].size
            for i, it in enumerate(step):
                n = int(plan["ctx_lens"][i])
                assert n == ref.lib.vspec_kv_paged_session_tokens(c, it.request_id)
                for t in range(n):
                    want = _ref_locate(ref, c, P, H, D, it.request_id, t)
                    assert want == (int(plan["block_tables"][i, t // P]), t % P), (i, t)
        assert nsteps > 5
    finally:
        lib.vspec_rocm_paged_meta_destroy(m)
        ref.lib.vr_paged_free(c)


def _slot_space(used, P):
    """Table-slot positions of a session's tokens in order: entry e holds used[e] tokens
    at positions e*P .. e*P + used[e] - 1 (the get_token_ptr walk, kv_paged_cache.c:335-347)."""
    return [e * P + s for e in range(len(used)) for s in range(int(used[e]))]


def test_plan_step_partial_middle_pages(lib, ref):
    """Prefix reuse that shares a partly filled page leaves it in the middle of both the
    target and, once the source appends again, the source (kv_paged_cache.c:223-234, 276).
    With block_used the planner still expresses every session: the used counts equal the
    reference pages', the span is the slot-space end, every token maps through the table
    to the (page, slot) the reference cache holds it in, and the new tokens' positions land
    where the reference appends them."""
    from vspec_rocm.sessions import plan_step

    P, MAXP, H, D = 4, 64, 1, 8
    m = lib.vspec_rocm_paged_meta_create(P, MAXP, 0, 0)
    c = ref.lib.vr_paged_new(P, MAXP, H, D)
    tok = np.zeros(H * D, np.float32)
    app = lambda sid: ref.lib.vspec_kv_paged_append(c, sid, tok.ctypes.data_as(_f32p), tok.ctypes.data_as(_f32p))
    steps = [
        ("plan", [(1, 1, 6, 0)]),                          # 1: a full page + 2 tokens
        ("reuse", (2, 1, 0)),                              # 2 shares both, the partial one too
        ("plan", [(1, 2, 3, 0), (2, 2, 2, 0), (3, 1, 5, 0)]),  # 1 and 2 open new pages
        ("reuse", (4, 2, 0)),                              # 4 shares 2's partial middle page
        ("plan", [(4, 2, 1, 0), (2, 2, 7, 0), (1, 2, 1, 0)]),
        ("reuse", (5, 3, 3)),                              # max_tokens 3 < the first page: none
        ("plan", [(5, 1, 9, 0), (4, 2, 4, 0)]),
    ]
    try:
        saw_partial_middle = False
        for kind, arg in steps:
            if kind == "reuse":
                assert lib.vspec_rocm_paged_reuse_prefix(m, *arg) == ref.lib.vspec_kv_paged_reuse_prefix(c, *arg)
                continue
            before = [ref.lib.vspec_kv_paged_session_tokens(c, it[0]) for it in arg]
            plan = plan_step(m, arg, max_blocks=16, with_used=True)
            for it in arg:
                for _ in range(it[2]):
                    assert app(it[0])
            off = 0
            for i, it in enumerate(arg):
                sid, q = it[0], it[2]
                tab, used, span = plan["block_tables"][i], plan["block_used"][i], int(plan["ctx_lens"][i])
                n = ref.lib.vspec_kv_paged_session_tokens(c, sid)
                assert n == before[i] + q == int(used.sum())
                npages = int((tab >= 0).sum())
                assert (tab[:npages] >= 0).all() and (tab[npages:] == -1).all()
                assert span == ((npages - 1) * P + int(used[npages - 1]) if npages else 0)
                saw_partial_middle |= bool((used[: max(npages - 1, 0)] < P).any())
                for e in range(npages):
                    alloc, u, rc = C.c_uint32(), C.c_uint32(), C.c_uint32()
                    ref.lib.vr_paged_page_meta(c, int(tab[e]), C.byref(alloc), C.byref(u), C.byref(rc))
                    assert u.value == used[e], (sid, e)
                pos = _slot_space(used[:npages], P)
                assert len(pos) == n
                for t in range(n):
                    assert _ref_locate(ref, c, P, H, D, sid, t) == (int(tab[pos[t] // P]), pos[t] % P), (sid, t)
                # the packed new tokens are the session's last q, at their slot-space positions
                assert list(plan["token_pos"][off:off + q]) == pos[n - q:]
                assert q == 0 or plan["start_pos"][i] == pos[n - q]
                off += q
        assert saw_partial_middle
    finally:
        lib.vspec_rocm_paged_meta_destroy(m)
        ref.lib.vr_paged_free(c)


def _random_steps(rng, n_steps, n_sessions, max_items, max_quota):
    """Seeded step sequences: items drawn from a small set of sessions in shuffled order
    (rows change hands between steps), mostly decode quotas of 1 with some prefill chunks,
    plus prefix reuses into fresh sessions and closes between steps."""
    next_new = 1000
    for _ in range(n_steps):
        ops = []
        r = rng.random()
        if r < 0.1:
            ops.append(("reuse", next_new, int(rng.integers(1, n_sessions + 1)), int(rng.integers(0, 40))))
            next_new += 1
        elif r < 0.15:
            ops.append(("close", int(rng.integers(1, n_sessions + 1))))
        k = int(rng.integers(1, max_items + 1))
        ids = rng.choice(np.arange(1, n_sessions + 1), size=k, replace=False).tolist()
        if ops and ops[0][0] == "reuse" and rng.random() < 0.7:
            ids[int(rng.integers(0, k))] = ops[0][1]
        items = []
        for sid in ids:
            q = 1 if rng.random() < 0.7 else int(rng.integers(0, max_quota + 1))
            items.append((int(sid), 2 if q == 1 else 1, q, 0))
        yield ops, items


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("with_used", [False, True])
def test_plan_step_update_equals_full_planning(lib, seed, with_used):
    """Two allocators take the same seeded operations; one plans every step into fresh
    tables (vspec_rocm_paged_plan_step), the other updates tables it keeps
    (vspec_rocm_paged_plan_step_update).  Every step gives the same success, block tables,
    used counts, contexts, start positions and packed-token map, through sessions moving
    between rows, prefix reuse (shared, partly filled pages), closes, LRU evictions in a
    small pool, failed steps, and a change of table buffers half way."""
    from vspec_rocm import VspecRocmError
    from vspec_rocm.sessions import StepPlanner, plan_step

    rng = np.random.default_rng(300 + seed)
    P, MAXP, MAXB = 4, int(rng.choice([24, 48, 400])), 32
    a = lib.vspec_rocm_paged_meta_create(P, MAXP, 16, 0)
    b = lib.vspec_rocm_paged_meta_create(P, MAXP, 16, 0)
    planner = StepPlanner(b, max_items=6, max_blocks=MAXB, max_tokens=6 * 9, with_used=with_used)
    fails = updates = 0
    try:
        for n, (ops, items) in enumerate(_random_steps(rng, 300, 10, 6, 9)):
            if n == 150:  # other buffers: every row is written whole again
                planner = StepPlanner(b, max_items=6, max_blocks=MAXB, max_tokens=6 * 9, with_used=with_used)
            for op in ops:
                if op[0] == "reuse":
                    ra = lib.vspec_rocm_paged_reuse_prefix(a, op[1], op[2], op[3])
                    assert ra == lib.vspec_rocm_paged_reuse_prefix(b, op[1], op[2], op[3])
                else:
                    assert lib.vspec_rocm_paged_close_session(a, op[1]) == lib.vspec_rocm_paged_close_session(b, op[1])
            try:
                want = plan_step(a, items, max_blocks=MAXB, with_used=with_used)
            except VspecRocmError:
                want = None
            try:
                got = planner.step(items)
            except VspecRocmError:
                got = None
            assert (want is None) == (got is None), n
            if want is None:
                fails += 1
                continue
            updates += 1
            for key in want:
                assert np.array_equal(want[key], got[key]), (n, key)
            assert _stats(lib, a) == _stats(lib, b)
        # plain tables refuse every step holding a session with a shared, partly filled
        # middle page, which prefix reuse keeps creating here
        assert updates > 50 and (fails < updates or not with_used)
        if MAXP < 100:
            assert fails > 0 or _stats(lib, a)[2] > 0  # small pools do evict
    finally:
        lib.vspec_rocm_paged_meta_destroy(a)
        lib.vspec_rocm_paged_meta_destroy(b)


def test_plan_step_update_writes_only_changed_entries(lib):
    """Steady decode over kept tables: after the first step, a step of one token per
    sequence changes only the entries it must (the last entry's used count, a new page
    every P tokens).  Entries outside them are left untouched, which the test checks by
    planting a marker the planner must not overwrite."""
    from vspec_rocm.sessions import StepPlanner

    P, B = 16, 8
    m = lib.vspec_rocm_paged_meta_create(P, 4096, 0, 0)
    planner = StepPlanner(m, max_items=B, max_blocks=64, max_tokens=B * 100, with_used=True)
    try:
        planner.step([(i + 1, 1, 100, 0) for i in range(B)])  # prefill 100 tokens each
        for t in range(40):
            n_pages = (100 + t) // P  # entries before the current last one
            planner.used[:, : n_pages - 1] = -7   # planted: full pages the update must not touch
            plan = planner.step([(i + 1, 2, 1, 0) for i in range(B)])
            assert (plan["block_used"][:, : n_pages - 1] == -7).all(), t
            assert (plan["ctx_lens"] == 101 + t).all()
            last = (100 + t) // P
            assert (plan["block_used"][:, last] == (100 + t) % P + 1).all()
            planner.used[:, : n_pages - 1] = P
    finally:
        lib.vspec_rocm_paged_meta_destroy(m)


def test_plan_step_rejects_bad_steps(lib):
    from vspec_rocm import VspecRocmError
    from vspec_rocm.sessions import plan_step

    m = lib.vspec_rocm_paged_meta_create(4, 3, 0, 0)
    try:
        with pytest.raises(VspecRocmError):
            plan_step(m, [(7, 2, 1, 0), (7, 2, 1, 0)], max_blocks=4)  # repeated request
        with pytest.raises(VspecRocmError):
            plan_step(m, [(8, 1, 9, 0)], max_blocks=2)  # 9 tokens need 3 pages > 2 columns
        # pool of 3 pages: the second item's pages evict the first item's session
        m2 = lib.vspec_rocm_paged_meta_create(4, 3, 0, 0)
        try:
            with pytest.raises(VspecRocmError):
                plan_step(m2, [(1, 1, 8, 0), (2, 1, 8, 0)], max_blocks=4)
        finally:
            lib.vspec_rocm_paged_meta_destroy(m2)
    finally:
        lib.vspec_rocm_paged_meta_destroy(m)
