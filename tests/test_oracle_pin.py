"""Pin the CPU oracle (oracle/vspec_oracle.c) before trusting it.

Each check is chosen so that a plausible restatement mistake fails it:
  * bit-exact agreement with the reference's own C sources compiled into
    oracle/_ref (attention_ref.c modes P/R, pack.c, int4.c, kv_cache.c int3);
  * the reference drivers' known answers (examples/attention_demo.c,
    examples/quant_pack_demo.c);
  * closed forms and textbook special cases (T=1 -> v0, q=0 -> mean(V),
    clamp-free data -> textbook softmax attention in float64);
  * an independent fp16 implementation (numpy) over every rounding boundary.
"""
import ctypes as C

import numpy as np
import pytest

from oracle.oracle import DTYPE_F16, DTYPE_F32, DTYPE_INT4, HostPool, ptr

_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)


# ----------------------------------------------------------------------------- fp16
def test_half_to_float_exhaustive(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_float_to_half_all_rounding_boundaries(oracle):
    # every finite half, the midpoints between neighbours, and +-1 ulp around them
    h = np.arange(0, 0x7C00, dtype=np.uint32).astype(np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = np.append(lo[1:], 65520.0)  # 65520 is the overflow boundary
    mid = ((lo + hi) / 2).astype(np.float32)
    cands = [lo.astype(np.float32), mid]
    for m in (mid,):
        bits = m.view(np.uint32)
        cands += [(bits + 1).view(np.float32), (bits - 1).view(np.float32)]
    x = np.concatenate(cands)
    x = np.concatenate([x, -x, np.array([np.inf, -np.inf, 1e30, -1e30, 0.0, -0.0, 1e-9, 3e-8, 2.9802322e-08], np.float32)])
    got = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_float_to_half_random(oracle):
    rng = np.random.default_rng(7)
    x = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = x[np.isfinite(x)]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x), want)


# ----------------------------------------------------------------------------- pack / int4
def test_quant_pack_demo_known_answer(oracle):
    """examples/quant_pack_demo.c: round trip equals clip_signed for b in {2,3,4}."""
    src = np.array([-9, -8, -7, -4, -1, 0, 1, 2, 3, 4, 7, 8], np.int8)
    for bits in (2, 3, 4):
        nbytes = oracle.lib.vo_quant_packed_bytes(len(src), bits)
        packed = np.zeros(nbytes, np.uint8)
        out = np.zeros(len(src), np.int8)
        oracle.lib.vo_quant_pack_signed(ptr(src, _i8p), len(src), bits, ptr(packed, _u8p))
        oracle.lib.vo_quant_unpack_signed(ptr(packed, _u8p), len(src), bits, ptr(out, _i8p))
        want = np.clip(src, -(1 << (bits - 1)), (1 << (bits - 1)) - 1)
        assert np.array_equal(out, want), bits


def test_pack_matches_reference(oracle, ref):
    rng = np.random.default_rng(3)
    for bits in (2, 3, 4):
        for n in (1, 2, 7, 64, 127, 128):
            src = rng.integers(-12, 12, size=n).astype(np.int8)
            nb = oracle.lib.vo_quant_packed_bytes(n, bits)
            assert nb == ref.lib.vspec_quant_packed_bytes(n, bits)
            a = np.zeros(nb, np.uint8)
            b = np.zeros(nb, np.uint8)
            oracle.lib.vo_quant_pack_signed(ptr(src, _i8p), n, bits, ptr(a, _u8p))
            ref.lib.vspec_quant_pack_signed(ptr(src, _i8p), n, bits, ptr(b, _u8p))
            assert np.array_equal(a, b)
    for n in (1, 2, 5, 128):
        src = rng.integers(-12, 12, size=n).astype(np.int8)
        a = np.zeros((n + 1) // 2, np.uint8)
        b = np.zeros((n + 1) // 2, np.uint8)
        oracle.lib.vo_int4_pack(ptr(src, _i8p), n, ptr(a, _u8p))
        ref.lib.vspec_int4_pack(ptr(src, _i8p), n, ptr(b, _u8p))
        assert np.array_equal(a, b)
        # pack(bits=4) is the same layout as int4_pack (even element -> low nibble)
        c = np.zeros((n + 1) // 2, np.uint8)
        oracle.lib.vo_quant_pack_signed(ptr(src, _i8p), n, 4, ptr(c, _u8p))
        assert np.array_equal(a, c)
        for i in range(n):
            assert oracle.lib.vo_int4_get(ptr(a, _u8p), i) == ref.lib.vspec_int4_get(ptr(b, _u8p), i)


# ----------------------------------------------------------------------------- KV codecs
@pytest.mark.parametrize("block_size", [16, 32])
def test_int3_codec_matches_reference(oracle, ref, block_size):
    """kv_cache.c:61-126 through the reference's own VspecKVCache int3 path."""
    T, H, D = 5, 3, 64
    x = oracle.normal(11 + block_size, T * H * D).reshape(T, H, D)
    x[0, 0, 3] = 60.0  # outlier: exercises the int8 narrowing quirk (kv_cache.c:100-101)
    x[1, 1, :] = 0.0  # all-zero head: scale 1.0
    v = oracle.normal(99, T * H * D).reshape(T, H, D)
    pb = (3 * D + 7) // 8
    nblk = D // block_size
    rq = np.zeros(T * H * pb, np.uint8)
    rs = np.zeros(T * H * nblk, np.float32)
    rm = np.zeros(T * H * D, np.float32)
    assert ref.lib.vr_int3_append_and_dump(ptr(np.ascontiguousarray(x), _f32p), ptr(np.ascontiguousarray(v), _f32p),
                                           T, H, D, block_size, ptr(rq, _u8p), ptr(rs, _f32p), ptr(rm, _f32p))
    for t in range(T):
        for h in range(H):
            i = t * H + h
            q, s = oracle.int3_quantize_head(x[t, h], block_size)
            assert np.array_equal(q, rq[i * pb:(i + 1) * pb])
            assert np.array_equal(s.view(np.uint32), rs[i * nblk:(i + 1) * nblk].view(np.uint32))
            deq = np.zeros(D, np.float32)
            oracle.lib.vo_int3_dequantize_head(ptr(q, _u8p), ptr(s, _f32p), D, block_size, ptr(deq, _f32p))
            assert np.array_equal(deq.view(np.uint32), rm[i * D:(i + 1) * D].view(np.uint32))


def test_percentile_is_second_largest(oracle):
    rng = np.random.default_rng(5)
    for _ in range(200):
        x = rng.standard_normal(32).astype(np.float32) * rng.uniform(0.01, 100)
        got = oracle.lib.vo_percentile_abs_block(ptr(x, _f32p), 32, C.c_float(99.5))
        assert got == np.sort(np.abs(x))[30]


def _group(vals):
    x = np.zeros(32, np.float32)
    x[: len(vals)] = vals
    return x


def test_int4_codec_closed_forms(oracle):
    def codes_of(c):
        lo = (c & 0xF).astype(np.int8)
        hi = (c >> 4).astype(np.int8)
        out = np.empty(c.size * 2, np.int8)
        out[0::2] = np.where(lo > 7, lo - 16, lo)
        out[1::2] = np.where(hi > 7, hi - 16, hi)
        return out

    # rep (2nd largest |x|) = 8 -> scale = 1.0 exactly: codes are rint(x), saturated
    x = _group([8.0, -8.0, 2.5, 3.5, -2.5, 0.5, 1.5, -0.5, 7.49, 100.0])
    c, s = oracle.int4_quantize_head(np.concatenate([x] * 4))
    assert list(s) == [0x3C00] * 4
    q = codes_of(c)[:32]
    assert list(q[:10]) == [7, -8, 2, 4, -2, 0, 2, 0, 7, 7]
    # all-zero group: rep = 0 -> scale 1.0, codes 0
    c, s = oracle.int4_quantize_head(np.zeros(128, np.float32))
    assert list(s) == [0x3C00] * 4 and not c.any()
    # tiny group: scale floored at 1e-6 and rounded to fp16 (17 * 2^-24)
    c, s = oracle.int4_quantize_head(np.full(128, 1e-7, np.float32))
    assert s[0] == np.float16(1e-6).view(np.uint16) == 17
    # single outlier: rep is the 2nd largest, the outlier saturates at 7
    x = _group([1000.0, 2.0, 1.0])
    c, s = oracle.int4_quantize_head(np.concatenate([x] * 4))
    assert s[0] == np.float16(0.25).view(np.uint16)
    assert list(codes_of(c)[:3]) == [7, 7, 4]
    # scale is fp16(rep/8) and codes use the fp16 scale
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128).astype(np.float32)
    c, s = oracle.int4_quantize_head(x)
    for g in range(4):
        xs = x[g * 32:(g + 1) * 32]
        rep = np.sort(np.abs(xs))[30]
        assert s[g] == np.float16(np.float32(rep) / np.float32(8)).view(np.uint16)
        sc = np.float32(np.float16(s[g].view(np.float16)))
        want = np.clip(np.rint(xs / sc), -8, 7).astype(np.int8)
        assert np.array_equal(codes_of(c)[g * 32:(g + 1) * 32], want)
    # dequantisation is code * float(scale16), exact in fp32
    deq = oracle.int4_dequantize_head(c, s, 128)
    q = codes_of(c).astype(np.float32)
    sc = np.repeat(s.view(np.float16).astype(np.float32), 32)
    assert np.array_equal(deq, q * sc)


# ----------------------------------------------------------------------------- numerics pieces
def test_clamp_std_matches_reference(oracle, ref):
    rng = np.random.default_rng(2)
    for n in (1, 4, 64, 128):
        for scale in (1e-3, 1.0, 50.0):
            x = (rng.standard_normal(n) * scale).astype(np.float32)
            x[rng.integers(0, n)] *= 20
            a = np.zeros(n, np.float32)
            b = np.zeros(n, np.float32)
            oracle.lib.vo_dynamic_clamp_std(ptr(x, _f32p), n, 4.5, ptr(a, _f32p))
            ref.lib.vspec_3bit_dynamic_clamp_std(ptr(x, _f32p), n, 4.5, ptr(b, _f32p))
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ----------------------------------------------------------------------------- attention_ref
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("T,H,D", [(1, 2, 4), (257, 8, 64), (33, 3, 128), (100, 2, 32)])
def test_attention_matches_reference_bitexact(oracle, ref, mode, T, H, D):
    seed = 1000 * T + 10 * H + D
    q = oracle.normal(seed, H * D).reshape(H, D)
    k = oracle.normal(seed + 1, T * H * D).reshape(T, H, D)
    v = oracle.normal(seed + 2, T * H * D).reshape(T, H, D)
    k[T // 2, 0, 1] = 9.0  # fires the std clamp
    q[0, 0] = -7.5
    a = oracle.attention_ref(mode, q, k, v)
    b = ref.attention_mha(mode, q, k, v)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("mode", [0, 1])
def test_attention_large_values_mode_r_paths(oracle, ref, mode):
    """Values large enough that mode R's +-16 input clip and +-24 logit clip fire."""
    T, H, D = 40, 2, 64
    q = oracle.normal(5, H * D).reshape(H, D) * 30
    k = oracle.normal(6, T * H * D).reshape(T, H, D) * 30
    v = oracle.normal(7, T * H * D).reshape(T, H, D)
    a = oracle.attention_ref(mode, q, k, v)
    b = ref.attention_mha(mode, q, k, v)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_attention_demo_known_answer(oracle):
    """examples/attention_demo.c (2 heads, D=4, 2 tokens) printed with %7.4f."""
    k0 = [0.2, 0.1, 0.0, -0.1, 0.1, 0.3, -0.2, 0.4]
    v0 = [0.5, 0.0, 0.1, 0.0, 0.2, 0.3, 0.1, -0.2]
    k1 = [0.0, 0.2, 0.1, 0.3, -0.1, 0.2, 0.2, 0.1]
    v1 = [0.1, 0.2, 0.4, 0.2, 0.0, 0.1, 0.3, 0.2]
    q = np.array([0.3, 0.1, -0.1, 0.0, 0.2, -0.2, 0.3, 0.1], np.float32).reshape(2, 4)
    k = np.array([k0, k1], np.float32).reshape(2, 2, 4)
    v = np.array([v0, v1], np.float32).reshape(2, 2, 4)
    want = np.array([[0.3030, 0.0985, 0.2478, 0.0985], [0.0983, 0.1983, 0.2017, 0.0035]])
    for mode in (0, 1):
        out = oracle.attention_ref(mode, q, k, v)
        assert np.array_equal(np.round(out.astype(np.float64), 4), want), out


def test_attention_closed_forms(oracle):
    D, H = 64, 2
    # T = 1: the single probability is exactly 1 -> out == v0 bit-exactly
    q = oracle.normal(1, H * D).reshape(H, D)
    k = oracle.normal(2, H * D).reshape(1, H, D)
    v = oracle.normal(3, H * D).reshape(1, H, D)
    for mode in (0, 1):
        assert np.array_equal(oracle.attention_ref(mode, q, k, v), v[0])
    # q = 0: clamp threshold 1e-6 keeps q'=0 -> uniform weights -> mean of V
    T = 50
    k = oracle.normal(4, T * H * D).reshape(T, H, D)
    v = oracle.normal(5, T * H * D).reshape(T, H, D)
    for mode in (0, 1):
        out = oracle.attention_ref(mode, np.zeros((H, D), np.float32), k, v)
        np.testing.assert_allclose(out, v.astype(np.float64).mean(0), atol=2e-7)


def test_attention_clamp_free_equals_textbook(oracle):
    """When no element exceeds 4.5 std the reference is plain softmax attention."""
    T, H, D = 300, 4, 128
    rng = np.random.default_rng(9)
    q = rng.uniform(-1, 1, (H, D)).astype(np.float32)
    k = rng.uniform(-1, 1, (T, H, D)).astype(np.float32)  # uniform: max/std = sqrt(3) < 4.5
    v = rng.uniform(-1, 1, (T, H, D)).astype(np.float32)
    for mode in (0, 1):
        out = oracle.attention_ref(mode, q, k, v)
        for h in range(H):
            want = np.zeros(D, np.float64)
            oracle.lib.vo_attention_textbook_f64(ptr(np.ascontiguousarray(q[h]), _f32p),
                                                 ptr(np.ascontiguousarray(k[:, h]), _f32p), D,
                                                 ptr(np.ascontiguousarray(v[:, h]), _f32p), D, T, D,
                                                 want.ctypes.data_as(C.POINTER(C.c_double)))
            # independent numpy float64 restatement as well
            s = (k[:, h].astype(np.float64) @ q[h].astype(np.float64)) / np.sqrt(D)
            p = np.exp(s - s.max())
            np_want = (p / p.sum()) @ v[:, h].astype(np.float64)
            np.testing.assert_allclose(want, np_want, atol=1e-12)
            np.testing.assert_allclose(out[h], np_want, atol=2e-6)


# ----------------------------------------------------------------------------- paged layout
def _tables(oracle, B, nblk, num_blocks, seed):
    perm = oracle.permutation(seed, num_blocks)
    return perm[: B * nblk].reshape(B, nblk).copy()


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_paged_append_gather_roundtrip(oracle, dtype):
    B, H, D, P, T = 3, 2, 64, 16, 37
    nblk = (T + P - 1) // P
    pool = HostPool(dtype, 16, P, H, D)
    bt = _tables(oracle, B, nblk, 16, 5)
    x = oracle.normal(21, B * T * H * D).reshape(B, T, H, D)
    y = oracle.normal(22, B * T * H * D).reshape(B, T, H, D)
    src_k = x if dtype == DTYPE_F32 else oracle.f32_to_f16(x)
    src_v = y if dtype == DTYPE_F32 else oracle.f32_to_f16(y)
    # build the context in two appends (a chunk, then single tokens)
    assert oracle.paged_append(pool, bt, np.zeros(B, np.int32), np.ascontiguousarray(src_k[:, :30]), np.ascontiguousarray(src_v[:, :30]))
    for t in range(30, T):
        assert oracle.paged_append(pool, bt, np.full(B, t, np.int32), np.ascontiguousarray(src_k[:, t:t + 1]), np.ascontiguousarray(src_v[:, t:t + 1]))
    ctx = np.full(B, T, np.int32)
    gk, gv, gks, gvs = oracle.paged_gather(pool, bt, ctx, out_mode=0)
    fk, fv, _, _ = oracle.paged_gather(pool, bt, ctx, out_mode=1)
    if dtype in (DTYPE_F32, DTYPE_F16):
        assert np.array_equal(gk.reshape(B, T, H, D), src_k)
        assert np.array_equal(gv.reshape(B, T, H, D), src_v)
        ref32 = x if dtype == DTYPE_F32 else oracle.f16_to_f32(src_k)
        assert np.array_equal(fk.reshape(B, T, H, D), ref32)
    else:
        src16k = oracle.f16_to_f32(src_k)
        for b in range(B):
            for t in range(T):
                for h in range(H):
                    c, s = oracle.int4_quantize_head(src16k[b, t, h])
                    r = b * T + t
                    assert np.array_equal(gk[r, h], c) and np.array_equal(gks[r, h], s)
                    assert np.array_equal(fk[r, h], oracle.int4_dequantize_head(c, s, D))


@pytest.mark.parametrize("D", [32, 64, 128])
def test_int4_pool_layout_is_a_bijection(oracle, D):
    """Every (block, head, slot, element) of an int4 pool owns exactly one V nibble and
    every (block, head, slot, group) one K scale, inside the pool; a V byte holds the
    two d-tiles of ONE token, so appends of different tokens never share a byte."""
    nb, P, H = 3, 32, 2
    pool = HostPool(DTYPE_INT4, nb, P, H, D)
    desc = pool.desc()
    hi = C.c_int()
    seen = np.zeros((pool.v.size, 2), np.int64) - 1
    for b in range(nb):
        for h in range(H):
            for slot in range(P):
                for d in range(D):
                    at = oracle.lib.vo_int4_v_byte(C.byref(desc), b, h, slot, d, C.byref(hi))
                    assert at < pool.v.size and seen[at, hi.value] < 0
                    seen[at, hi.value] = ((b * H + h) * P + slot)
    assert (seen >= 0).all()
    assert (seen[:, 0] == seen[:, 1]).all()  # one token per byte
    G = D // 32
    idx = sorted(oracle.lib.vo_int4_ks_index(C.byref(desc), b, h, s, c)
                 for b in range(nb) for h in range(H) for s in range(P) for c in range(G))
    assert idx == list(range(pool.ks.size))
    # the low nibble of a byte is an even 16-wide d-tile, the high nibble the next one
    at0 = oracle.lib.vo_int4_v_byte(C.byref(desc), 1, 1, 21, 5, C.byref(hi))
    assert hi.value == 0
    at1 = oracle.lib.vo_int4_v_byte(C.byref(desc), 1, 1, 21, 21, C.byref(hi))
    assert hi.value == 1 and at1 == at0


@pytest.mark.parametrize("D", [64, 128])
def test_f16_v_layout_is_a_bijection(oracle, D):
    """Every (block, head, slot, element) of an f16 V pool owns exactly one half inside the
    pool; a 16-token tile is one contiguous span of 16*D halves; the 4 tokens of a group
    are adjacent for every d (the decode's 8-byte operand); one token's row lies inside
    its group's 4*D halves, every 4th one."""
    nb, P, H = 3, 32, 2
    pool = HostPool(DTYPE_F16, nb, P, H, D)
    desc = pool.desc()
    seen = np.full(pool.v.size, -1, np.int64)
    for b in range(nb):
        for h in range(H):
            for slot in range(P):
                at = [oracle.lib.vo_f16_v_index(C.byref(desc), b, h, slot, d) for d in range(D)]
                assert max(at) < pool.v.size and (seen[at] < 0).all()
                seen[at] = (b * H + h) * P + slot
                g0 = ((b * H + h) * P + slot // 4 * 4) * D
                assert at == [g0 + 4 * d + slot % 4 for d in range(D)]
    assert (seen >= 0).all()
    for b, h, t in ((0, 0, 0), (2, 1, 1)):
        span = sorted(oracle.lib.vo_f16_v_index(C.byref(desc), b, h, 16 * t + s, d) for s in range(16) for d in range(D))
        assert span == list(range(span[0], span[0] + 16 * D))
        quad = [oracle.lib.vo_f16_v_index(C.byref(desc), b, h, 16 * t + 4 + r, 7) for r in range(4)]
        assert quad == list(range(quad[0], quad[0] + 4))


def test_f16_pool_needs_whole_tiles(oracle):
    pool = HostPool(DTYPE_F16, 2, 24, 1, 64)
    x = np.zeros((1, 1, 1, 64), np.float32)
    assert not oracle.paged_append(pool, np.array([[0, 1]], np.int32), np.zeros(1, np.int32), x, x)


def test_int4_pool_needs_whole_tiles(oracle):
    pool = HostPool(DTYPE_INT4, 2, 24, 1, 64)
    x = np.zeros((1, 1, 1, 64), np.float32)
    assert not oracle.paged_append(pool, np.array([[0, 1]], np.int32), np.zeros(1, np.int32), x, x)


def test_paged_gather_equals_reference_read(oracle, ref):
    """The reference pool (token-major pages, capi.c gather) and the build's layout
    hold the same tokens when the block table equals the reference session's pages."""
    P, H, D = 16, 4, 32
    c = ref.lib.vr_paged_new(P, 64, H, D)
    try:
        x = oracle.normal(31, 3 * 70 * H * D).reshape(3, 70, H, D)
        y = oracle.normal(32, 3 * 70 * H * D).reshape(3, 70, H, D)
        for t in range(70):  # interleaved sessions -> interleaved first-fit pages
            for s in range(3):
                assert ref.lib.vspec_kv_paged_append(c, 100 + s, ptr(np.ascontiguousarray(x[s, t]), _f32p), ptr(np.ascontiguousarray(y[s, t]), _f32p))
        pool = HostPool(DTYPE_F32, 64, P, H, D)
        pages = np.zeros((3, 8), np.uint32)
        for s in range(3):
            n = ref.lib.vr_paged_session_pages(c, 100 + s, pages[s].ctypes.data_as(C.POINTER(C.c_uint32)), 8)
            assert n == 5
        bt = pages.astype(np.int32)
        assert not np.array_equal(bt[0], np.arange(8))  # fragmented, not identity
        assert oracle.paged_append(pool, bt, np.zeros(3, np.int32), x, y)
        gk, gv, _, _ = oracle.paged_gather(pool, bt, np.full(3, 70, np.int32))
        for s in range(3):
            rk = np.zeros((70, H, D), np.float32)
            rv = np.zeros((70, H, D), np.float32)
            assert ref.lib.vr_paged_read(c, 100 + s, ptr(rk, _f32p), ptr(rv, _f32p), 0) == 70
            assert np.array_equal(gk[s * 70:(s + 1) * 70], rk)
            assert np.array_equal(gv[s * 70:(s + 1) * 70], rv)
    finally:
        ref.lib.vr_paged_free(c)


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_paged_decode_equals_reference_gqa(oracle, ref, mode, dtype):
    """Paged GQA decode == gather + the reference's attention_ref with kv_h = h // G
    (runtime_inference.py:151), bit-exactly."""
    B, Hq, Hkv, D, P = 2, 8, 2, 128, 16
    ctx = np.array([37, 64], np.int32)
    nblk = 4
    pool = HostPool(dtype, 12, P, Hkv, D)
    bt = _tables(oracle, B, nblk, 12, 8)
    Tm = int(ctx.max())
    x = oracle.normal(41, B * Tm * Hkv * D).reshape(B, Tm, Hkv, D)
    y = oracle.normal(42, B * Tm * Hkv * D).reshape(B, Tm, Hkv, D)
    if dtype != DTYPE_F32:
        x, y = oracle.f32_to_f16(x), oracle.f32_to_f16(y)
    assert oracle.paged_append(pool, bt, np.zeros(B, np.int32), x, y)
    q = oracle.normal(43, B * Hq * D).reshape(B, Hq, D)
    out = oracle.paged_decode(mode, pool, bt, ctx, q)
    fk, fv, _, _ = oracle.paged_gather(pool, bt, ctx, out_mode=1)
    off = 0
    for b in range(B):
        T = int(ctx[b])
        want = ref.attention_gqa(mode, q[b], fk[off:off + T], fv[off:off + T])
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32))
        off += T


def test_paged_compact_moves_blocks(oracle):
    pool = HostPool(DTYPE_INT4, 8, 16, 2, 64)
    rng = np.random.default_rng(4)
    for a in (pool.k, pool.v, pool.ks, pool.vs):
        a[...] = rng.integers(0, 255, a.shape).astype(a.dtype)
    before = [a.copy() for a in (pool.k, pool.v, pool.ks, pool.vs)]
    assert oracle.paged_compact(pool, [5, 6], [0, 1])
    rows = 2 * 16
    for a, b in zip((pool.k, pool.v, pool.ks, pool.vs), before):
        assert np.array_equal(a[0:rows], b[5 * rows:6 * rows])
        assert np.array_equal(a[rows:2 * rows], b[6 * rows:7 * rows])
        assert np.array_equal(a[2 * rows:], b[2 * rows:])


# ----------------------------------------------------------------------------- rotary embedding
def _rope_tables(max_pos, rope_dim, theta=10000.0):
    """cos/sin rows as the reference caches them (runtime_inference.py:1186-1192, 4227):
    float32 inverse frequencies, float32 angles pos * inv_freq, float32 cos/sin."""
    half = rope_dim // 2
    inv = (1.0 / (theta ** (np.arange(half, dtype=np.float32) / max(1, half)))).astype(np.float32)
    ang = np.stack([np.float32(p) * inv for p in range(max_pos)]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def test_rope_row_special_cases(oracle):
    D = 16
    cos, sin = _rope_tables(40, D)
    x = oracle.normal(71, D)
    assert np.array_equal(oracle.rope_row(x, D, cos[0], sin[0]), x)  # position 0: identity
    for i in range(D // 2):  # unit vectors land on (cos_i, sin_i)
        e = np.zeros(D, np.float32)
        e[i] = 1.0
        out = oracle.rope_row(e, D, cos[33], sin[33])
        want = np.zeros(D, np.float32)
        want[i], want[i + D // 2] = cos[33][i], sin[33][i]
        assert np.array_equal(out, want)
    out = oracle.rope_row(x, D, cos[17], sin[17])
    n0 = np.hypot(x[: D // 2], x[D // 2:])
    n1 = np.hypot(out[: D // 2], out[D // 2:])
    np.testing.assert_allclose(n1, n0, rtol=2e-6)  # rotations keep each pair's norm


def test_rope_row_matches_float32_array_arithmetic(oracle):
    """Bit-equal to the reference formula evaluated in numpy float32 (separately rounded
    products and sums), including partial rotary (_apply_partial_rotary)."""
    D = 128
    for rope_dim in (128, 64):
        cos, sin = _rope_tables(300, rope_dim)
        for pos in (1, 7, 255, 299):
            x = oracle.normal(80 + pos, D)
            half = rope_dim // 2
            k1, k2 = x[:half], x[half:rope_dim]
            want = np.concatenate([k1 * cos[pos] - k2 * sin[pos], k1 * sin[pos] + k2 * cos[pos], x[rope_dim:]])
            got = oracle.rope_row(x, rope_dim, cos[pos], sin[pos])
            assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), (rope_dim, pos)


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_paged_append_rope(oracle, dtype):
    """Fused rotary + append == rotate each K row, then the plain append; V untouched."""
    B, H, D, P, T = 2, 2, 64, 16, 21
    cos, sin = _rope_tables(64, D)
    bt = _tables(oracle, B, 2, 8, 9)
    x = oracle.normal(91, B * T * H * D).reshape(B, T, H, D)
    y = oracle.normal(92, B * T * H * D).reshape(B, T, H, D)
    a = HostPool(dtype, 8, P, H, D)
    b = HostPool(dtype, 8, P, H, D)
    start = np.array([3, 11], np.int32)
    assert oracle.paged_append_rope(a, bt, start, x, y, cos, sin, D)
    xr = np.empty_like(x)
    for s_ in range(B):
        for t in range(T):
            for h in range(H):
                p_ = start[s_] + t
                xr[s_, t, h] = oracle.rope_row(x[s_, t, h], D, cos[p_], sin[p_])
    assert oracle.paged_append(b, bt, start, xr, y)
    for u, w in zip((a.k, a.v, a.ks, a.vs), (b.k, b.v, b.ks, b.vs)):
        if u is not None:
            assert np.array_equal(u, w)
    # a position past the tables fails
    assert not oracle.paged_append_rope(HostPool(dtype, 8, P, H, D), bt, np.array([60, 0], np.int32), x, y, cos, sin, D)
