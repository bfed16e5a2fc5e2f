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
