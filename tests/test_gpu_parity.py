"""GPU parity: the HIP path (through the C-ABI) against the CPU oracle on the same
seeded inputs.

Bars:
  * append, gather, compaction and int4 codes/scales: bit-exact;
  * attention, in both reference numerics modes (P: 3-bit module off, R: on): max-abs
    2e-5 with fp32 and fp16 KV, and 2.5e-4 * max|v| + 2e-5 (capped at 4e-3) with int4 KV,
    whose kernel rounds p * scale to fp16 once per token (relative 2^-12).  These are
    tighter than the north-star bars (1e-4 fp32, 4e-3 fp16/int4): at 4k-token contexts a
    single token carries ~2.5e-4 of the softmax weight, so a token dropped or read stale
    by a merge or the fused append would pass the north-star bars unnoticed.
"""
import ctypes as C
import sys

import numpy as np
import pytest

from oracle.oracle import DTYPE_F16, DTYPE_F32, DTYPE_INT4, HostPool, _f32p, _u8p, ptr
from cases import GARBAGE, continuous_c4, fill_garbage, make_case, qwen_c2

pytestmark = pytest.mark.gpu
TOL = {DTYPE_F32: 2e-5, DTYPE_F16: 2e-5, DTYPE_INT4: 4e-3}


def tol_of(dtype, vmax=None):
    """Max-abs bound of a decode against the oracle; int4 scales with max|v| (an upper
    bound of the dequantised values when taken over the source values)."""
    if dtype != DTYPE_INT4 or vmax is None:
        return TOL[dtype]
    return min(4e-3, 2.5e-4 * float(vmax) + 2e-5)


def case_vmax(case):
    v = case.v_tokens
    return float(np.abs(v.view(np.float16) if v.dtype == np.uint16 else v).astype(np.float32).max())


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


@pytest.fixture(params=["plan", "always", "never"])
def flag_gate(request):
    """int4 decode: "plan" lets the host pick the clamp-flag kernel (shares of >= 16 tiles
    per workgroup) or the screen-every-tile one; "always" forces the flag kernel
    (VSPEC_ROCM_DECODE_FLAG_MIN_TILES=0, read on every call), "never" the screen one
    (4096).  Cases of other pool dtypes run once."""
    import os

    dtype = request.node.callspec.params.get("dtype", DTYPE_INT4)
    if request.param != "plan" and dtype != DTYPE_INT4:
        pytest.skip("clamp flags exist for int4 pools only")
    old = os.environ.get("VSPEC_ROCM_DECODE_FLAG_MIN_TILES")
    if request.param != "plan":
        os.environ["VSPEC_ROCM_DECODE_FLAG_MIN_TILES"] = "0" if request.param == "always" else "4096"
    yield request.param
    if old is None:
        os.environ.pop("VSPEC_ROCM_DECODE_FLAG_MIN_TILES", None)
    else:
        os.environ["VSPEC_ROCM_DECODE_FLAG_MIN_TILES"] = old


def _np_to_dev(a, dev):
    import torch

    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.float16).to(dev)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def device_pool(case, dev):
    import torch
    import vspec_rocm as vr

    pool = vr.PagedPool(case.dtype, case.num_blocks, case.P, case.Hkv, case.D, device=dev)
    g, gs = GARBAGE[case.dtype]
    if case.dtype == DTYPE_F32:
        pool.k.view(torch.int32).fill_(int(np.int32(np.uint32(g).view(np.int32))))
        pool.v.view(torch.int32).fill_(int(np.int32(np.uint32(g).view(np.int32))))
    elif case.dtype == DTYPE_F16:
        pool.k.view(torch.int16).fill_(int(np.uint16(g).view(np.int16)))
        pool.v.view(torch.int16).fill_(int(np.uint16(g).view(np.int16)))
    else:
        pool.k.fill_(int(g))
        pool.v.fill_(int(g))
        pool.ks.fill_(int(np.uint16(gs).view(np.int16)))
        pool.vs.fill_(int(np.uint16(gs).view(np.int16)))
    return pool


def pool_bytes(pool):
    """Device pool -> numpy views comparable with HostPool arrays."""
    import torch

    def cv(t, like):
        if t is None:
            return None
        if t.dtype == torch.float16:
            return t.view(torch.int16).cpu().numpy().view(np.uint16)
        if t.dtype == torch.int16:
            return t.cpu().numpy().view(np.uint16)
        return t.cpu().numpy()

    return [cv(pool.k, None), cv(pool.v, None), cv(pool.ks, None), cv(pool.vs, None)]


def assert_pools_equal(host: HostPool, pool):
    got = pool_bytes(pool)
    want = [host.k, host.v, host.ks, host.vs]
    for name, g, w in zip(("k", "v", "k_scales", "v_scales"), got, want):
        if w is None:
            assert g is None
            continue
        ge = np.ascontiguousarray(g).reshape(-1)
        we = np.ascontiguousarray(w).reshape(-1)
        bad = np.flatnonzero(ge.view(np.uint8) != we.view(np.uint8))
        if bad.size:
            el = np.unique(bad // ge.itemsize)[:6]
            detail = ", ".join(f"[{i}] gpu={ge[i]!r} oracle={we[i]!r}" for i in el)
            raise AssertionError(f"{name}: {bad.size} bytes differ; elements {detail}")


def build_both(oracle, case, dev, prefix_split=True):
    """Append the case's token stream on both sides: context minus one token as one
    chunk, then the decode-step token."""
    import torch
    import vspec_rocm as vr

    pool = device_pool(case, dev)
    tab_d = torch.from_numpy(case.tables).to(dev)
    B, T = case.B, case.tmax
    # per-sequence streams are written up to their own ctx: append in uniform chunks
    # over the prefix every sequence shares, then token-by-token for ragged tails
    tmin = int(case.ctx.min())
    first = tmin - 1 if prefix_split and tmin > 1 else tmin
    k_d = _np_to_dev(case.k_tokens, dev)
    v_d = _np_to_dev(case.v_tokens, dev)
    if first > 0:
        kk = np.ascontiguousarray(case.k_tokens[:, :first])
        vv = np.ascontiguousarray(case.v_tokens[:, :first])
        assert oracle.paged_append(case.host, case.tables, np.zeros(B, np.int32), kk, vv)
        vr.kv_append(pool, tab_d, torch.zeros(B, dtype=torch.int32, device=dev),
                     k_d[:, :first].contiguous(), v_d[:, :first].contiguous())
    for t in range(first, T):
        live = np.flatnonzero(case.ctx > t)
        if live.size == 0:
            continue
        kk = np.ascontiguousarray(case.k_tokens[live, t:t + 1])
        vv = np.ascontiguousarray(case.v_tokens[live, t:t + 1])
        sp = np.full(live.size, t, np.int32)
        tabs = np.ascontiguousarray(case.tables[live])
        assert oracle.paged_append(case.host, tabs, sp, kk, vv)
        li = torch.from_numpy(live).to(dev)
        vr.kv_append(pool, torch.from_numpy(tabs).to(dev), torch.from_numpy(sp).to(dev),
                     k_d[li, t:t + 1].contiguous(), v_d[li, t:t + 1].contiguous())
    torch.cuda.synchronize()
    return pool


def run_decode(case, pool, dev, mode, partition_tokens=0):
    import torch
    import vspec_rocm as vr

    q = torch.from_numpy(case.q).to(dev)
    out = vr.paged_decode(pool, torch.from_numpy(case.tables).to(dev), torch.from_numpy(case.ctx).to(dev), q,
                          max_ctx_len=case.tmax, numerics=mode, partition_tokens=partition_tokens)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_attention(oracle, case, got, mode, subset=None):
    idx = np.arange(case.B) if subset is None else np.asarray(subset)
    want = oracle.paged_decode(mode, case.host, case.tables[idx], case.ctx[idx], case.q[idx])
    err = np.abs(got[idx] - want)
    assert np.isfinite(got[idx]).all()
    tol = tol_of(case.dtype, case_vmax(case))
    say(f"    max-abs {err.max():.2e} (bound {tol:.1e}, mode {mode})")
    assert err.max() <= tol, f"max-abs {err.max():.3e} > {tol:.1e} (mode {mode})"
    return float(err.max())


# ----------------------------------------------------------------------------- config 1
@pytest.mark.parametrize("mode", [0, 1])
def test_config1_cpu_reference_shape(oracle, gpu, mode):
    """C1: 1 sequence, MHA 8x64, 256 cached + 1 appended token, P=16, identity table,
    fp32 K/V/Q ~ N(0,1)."""
    say(f"[c1] mode={mode} build")
    case = make_case(oracle, DTYPE_F32, 1, 8, 8, 64, 16, [257], seed=1, table="identity")
    pool = build_both(oracle, case, gpu)
    assert_pools_equal(case.host, pool)
    say("[c1] gather")
    import torch
    import vspec_rocm as vr

    gk, gv, _, _ = vr.kv_gather(pool, torch.from_numpy(case.tables).to(gpu), torch.from_numpy(case.ctx).to(gpu))
    ok_, ov, _, _ = oracle.paged_gather(case.host, case.tables, case.ctx)
    assert np.array_equal(gk.cpu().numpy().view(np.uint32), ok_.view(np.uint32))
    assert np.array_equal(gv.cpu().numpy().view(np.uint32), ov.view(np.uint32))
    assert np.array_equal(ok_.reshape(257, 8, 64), case.k_tokens[0])
    say("[c1] decode")
    got = run_decode(case, pool, gpu, mode)
    check_attention(oracle, case, got, mode)


# ----------------------------------------------------------------------------- append / gather
@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("src16", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_append_gather_bitexact(oracle, gpu, dtype, src16, D):
    import torch
    import vspec_rocm as vr

    say(f"[append] dtype={dtype} src16={src16} D={D}")
    case = make_case(oracle, dtype, 3, 4, 2, D, 32, [45, 1, 70], seed=10 + dtype + 3 * src16 + D,
                     num_blocks=9, src16=src16)
    # tiny and huge values exercise fp16 subnormals/overflow and the int4 scale floor
    case.k_tokens = case.k_tokens.copy()
    if not src16:
        case.k_tokens[0, 3, 0, :5] = [1e-8, -3e-7, 7e4, -1e5, 6.1e-5]
        case.k_tokens[2, 5, 1, :] = 1e-9
    pool = build_both(oracle, case, gpu)
    assert_pools_equal(case.host, pool)
    tab = torch.from_numpy(case.tables).to(gpu)
    ctx = torch.from_numpy(case.ctx).to(gpu)
    for mode in (0, 1):
        say(f"[gather] dtype={dtype} out_mode={mode}")
        gk, gv, gks, gvs = vr.kv_gather(pool, tab, ctx, out_mode=mode)
        wk, wv, wks, wvs = oracle.paged_gather(case.host, case.tables, case.ctx, out_mode=mode)
        for g, w in ((gk, wk), (gv, wv), (gks, wks), (gvs, wvs)):
            if w is None:
                continue
            gb = g.cpu().numpy().view(np.uint8)
            assert np.array_equal(gb, np.ascontiguousarray(w).view(np.uint8))


def test_compact_bitexact(oracle, gpu):
    import torch
    import vspec_rocm as vr

    say("[compact]")
    case = make_case(oracle, DTYPE_INT4, 2, 8, 2, 128, 16, [80, 50], seed=77, num_blocks=16)
    pool = build_both(oracle, case, gpu)
    src = np.concatenate([case.tables[0, 1:5], case.tables[1, 1:4]]).astype(np.int32)
    used = set(case.tables[case.tables >= 0].tolist())
    free = np.array([b for b in range(16) if b not in used], np.int32)
    assert free.size >= src.size
    dst = free[: src.size]
    assert oracle.paged_compact(case.host, src, dst)
    vr.kv_compact(pool, torch.from_numpy(src).to(gpu), torch.from_numpy(dst).to(gpu))
    torch.cuda.synchronize()
    assert_pools_equal(case.host, pool)


@pytest.mark.parametrize("seed", range(12))
def test_append_gather_compact_random(oracle, gpu, seed):
    """Seeded random shapes for the byte-exact part of the path: the appended pool (f32 /
    f16 sources, ragged contexts, block sizes 16-64), the raw and dequantised gathers, and
    a compaction of a random subset of the used blocks into free ones, all equal to the
    oracle's bytes."""
    import torch
    import vspec_rocm as vr

    rng = np.random.default_rng(7000 + seed)
    dtype = [DTYPE_F32, DTYPE_F16, DTYPE_INT4][seed % 3]
    B = int(rng.integers(1, 9))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    D = int(rng.choice([64, 128]))
    P = int(rng.choice([16, 32, 48, 64]))
    src16 = bool(rng.integers(0, 2))
    ctx = rng.integers(0, 400, B).astype(np.int32)
    used_blocks = int(((ctx + P - 1) // P).sum())
    nblk = used_blocks + int(rng.integers(used_blocks // 2 + 1, used_blocks + 3))
    say(f"[bytes {seed}] dtype={dtype} B={B} Hkv={Hkv} D={D} P={P} src16={src16} blocks={nblk} ctx={ctx.tolist()}")
    case = make_case(oracle, dtype, B, Hkv, Hkv, D, P, ctx, seed=400 + seed, num_blocks=nblk, src16=src16)
    pool = build_both(oracle, case, gpu)
    assert_pools_equal(case.host, pool)
    tab = torch.from_numpy(case.tables).to(gpu)
    cl = torch.from_numpy(case.ctx).to(gpu)
    for mode in (vr.GATHER_RAW, vr.GATHER_F32):
        got = vr.kv_gather(pool, tab, cl, out_mode=mode, max_ctx_len=max(case.tmax, 1))
        want = oracle.paged_gather(case.host, case.tables, case.ctx, out_mode=mode)
        for g_, w_ in zip(got, want):
            if w_ is None:
                assert g_ is None
                continue
            g_ = g_.cpu().numpy()
            assert np.array_equal(np.ascontiguousarray(g_).view(np.uint8).reshape(-1),
                                  np.ascontiguousarray(w_).view(np.uint8).reshape(-1))
    used = case.tables[case.tables >= 0]
    if used.size:
        free = np.setdiff1d(np.arange(nblk, dtype=np.int32), used)
        k = int(min(free.size, rng.integers(1, used.size + 1)))
        src = rng.permutation(used)[:k].astype(np.int32)
        dst = rng.permutation(free)[:k].astype(np.int32)
        assert oracle.paged_compact(case.host, src, dst)
        vr.kv_compact(pool, torch.from_numpy(src).to(gpu), torch.from_numpy(dst).to(gpu))
        torch.cuda.synchronize()
        assert_pools_equal(case.host, pool)


# ----------------------------------------------------------------------------- decode edge cases
@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("D,Hq,Hkv", [(64, 8, 8), (128, 8, 4), (128, 16, 4), (128, 16, 2), (64, 6, 2)])
def test_decode_edges(oracle, gpu, flag_gate, dtype, D, Hq, Hkv):
    """Ragged contexts around tile/block edges, GQA groups 1/2/3/4/8, garbage (NaN)
    beyond each context, several partition sizes."""
    ctx = [1, 15, 16, 17, 33, 64, 100, 0]
    say(f"[edges] dtype={dtype} D={D} Hq={Hq} Hkv={Hkv}")
    case = make_case(oracle, dtype, len(ctx), Hq, Hkv, D, 32, ctx, seed=5 * D + Hq + dtype,
                     num_blocks=20)
    pool = build_both(oracle, case, gpu)
    for mode in (0, 1):
        for pt in (0, 16, 48):
            say(f"[edges] mode={mode} partition_tokens={pt}")
            got = run_decode(case, pool, gpu, mode, partition_tokens=pt)
            assert np.all(got[-1] == 0.0)  # empty context -> zeros
            check_attention(oracle, case, got, mode, subset=range(len(ctx) - 1))


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("P", [48, 64])
def test_decode_block_sizes(oracle, gpu, flag_gate, dtype, P):
    """Blocks of 48 and 64 tokens (the kernels' generic block size: several 16-token tiles
    per block) with contexts around block and tile edges: bit-exact pools, attention within
    tolerance in both modes and with fixed-size partitions."""
    import torch
    import vspec_rocm as vr

    ctx = [1, P - 1, P, P + 1, 3 * P + 17, 200, 0]
    say(f"[block sizes] dtype={dtype} P={P}")
    case = make_case(oracle, dtype, len(ctx), 16, 4, 128, P, ctx, seed=3 * P + dtype, num_blocks=24)
    pool = build_both(oracle, case, gpu)
    assert_pools_equal(case.host, pool)
    for mode in (0, 1):
        got = run_decode(case, pool, gpu, mode)
        assert np.all(got[-1] == 0.0)
        check_attention(oracle, case, got, mode, subset=range(len(ctx) - 1))
    got = run_decode(case, pool, gpu, 1, partition_tokens=32)
    check_attention(oracle, case, got, 1, subset=range(len(ctx) - 1))


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_decode_outliers_fire_clamp(oracle, gpu, flag_gate, dtype):
    """Large outliers make the std-clamp (and in mode R the +-16 clip and +-24 logit
    clip) change the result; the GPU must follow the reference there too (the f16 and
    int4 kernels take their exact-score path for these keys)."""
    say(f"[outliers] dtype={dtype}")
    case = make_case(oracle, dtype, 2, 8, 2, 128, 16, [300, 77], seed=91, src16=False)
    k = case.k_tokens.copy()
    k[0, ::7, 0, 3] = 40.0
    k[1, ::5, 1, 100] = -25.0
    k[0, 10, 1, :] *= 20.0
    case.k_tokens = k
    case.q = case.q.copy()
    case.q[0, 0, 7] = 30.0
    case.q[1] *= 8.0
    pool = build_both(oracle, case, gpu)
    for mode in (0, 1):
        got = run_decode(case, pool, gpu, mode)
        check_attention(oracle, case, got, mode)


def test_int4_clamp_flags_are_conservative(oracle, gpu):
    """Every key the append leaves unflagged is one the reference's clamp chain leaves
    alone: the std clamp (alpha 4.5, attention_ref.c:56) returns it unchanged and no
    element reaches the 3-bit input clip of 16, so the decode may score it without
    clamping.  Keys: Gaussian rows, rows with one large element, rows scaled by 20
    (elements beyond 16), constant rows (std 0) and near-constant rows.  The flags are
    also not trivially all set: most Gaussian rows stay clear."""
    import torch

    say("[flags] build")
    case = make_case(oracle, DTYPE_INT4, 3, 8, 2, 128, 16, [300, 77, 160], seed=93, src16=False)
    k = case.k_tokens.copy()
    k[0, ::7, 0, 3] = 40.0
    k[0, 1::7, 1, 5] = 6.5
    k[1, ::5, 1, 100] = -25.0
    k[0, 10, 1, :] *= 20.0
    k[2, :40] *= 20.0
    k[2, 40:60] = 0.75
    k[2, 60:80] = 0.75 + 1e-3 * k[2, 60:80]
    case.k_tokens = k
    pool = build_both(oracle, case, gpu)
    assert_pools_equal(case.host, pool)
    flags = pool.kf.cpu().numpy().view(np.uint32)
    keys, _, _, _ = oracle.paged_gather(case.host, case.tables, case.ctx, out_mode=1)
    H, P = case.Hkv, case.P
    clear = fired = total = 0
    off = 0
    for b in range(case.B):
        for t in range(int(case.ctx[b])):
            phys = int(case.tables[b, t // P])
            for h in range(H):
                word = (phys * H + h) * (P // 16) + (t % P) // 16
                on = bool((flags[word] >> (t % 16)) & 1)
                x = np.ascontiguousarray(keys[off + t, h])
                y = np.empty_like(x)
                oracle.lib.vo_dynamic_clamp_std(ptr(x, _f32p), x.size, 4.5, ptr(y, _f32p))
                moved = not np.array_equal(x, y) or np.abs(x).max() >= 16.0
                total += 1
                fired += moved
                if not on:
                    clear += 1
                    assert not moved, f"unflagged key b={b} t={t} h={h} is changed by the clamp"
        off += int(case.ctx[b])
    say(f"[flags] keys {total} clamped {fired} unflagged {clear}")
    assert fired > 0
    assert clear >= 0.8 * (total - fired)


def _attention_p_f64(q, keys, vals, alpha, scale):
    """Mode P (attention_ref.c:7-88 with the 3-bit module off) in float64 with clamp
    alpha `alpha`: q' = clamp(q), k' = clamp(k) per key, clamp(x) = clip(x, +-max(1e-6,
    alpha * std(x))) around 0 (three_bit_runtime_modules.c:175-203), softmax of
    scale * q'.k', output = p.v.  q [D]; keys, vals [T][D]."""
    def clamp(x):
        th = max(1e-6, alpha * float(np.sqrt(np.mean((x - x.mean()) ** 2))))
        return np.clip(x, -th, th)

    qc = clamp(q.astype(np.float64))
    kc = np.stack([clamp(k) for k in keys.astype(np.float64)])
    sc = (kc @ qc) * scale
    w = np.exp(sc - sc.max())
    return (w / w.sum()) @ vals.astype(np.float64)


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("alpha", [3.0, 6.0])
def test_decode_custom_clamp_alpha(oracle, gpu, flag_gate, dtype, alpha):
    """clamp_alpha other than the reference's 4.5 (mode P), on keys with outliers: below
    4.5 the int4 decode screens every key (the pool's flags are kept for 4.5), above it
    the flags stay a superset of the clamped keys.  Checked against a float64 restatement
    over the pool's (dequantised) keys."""
    import ctypes as C
    import torch
    import vspec_rocm as vr

    say(f"[alpha] dtype={dtype} alpha={alpha}")
    case = make_case(oracle, dtype, 2, 8, 2, 128, 16, [300, 130], seed=97, src16=False)
    k = case.k_tokens.copy()
    # outliers in pairs within one 32-element group, so that int4's scale (the group's
    # second-largest |x|) keeps them
    k[0, ::7, 0, 3:5] = 9.0
    k[0, 1::9, 1, 50:52] = 4.2
    k[1, ::5, 1, 100:102] = -6.0
    k[1, 3, 0, :] *= 12.0
    case.k_tokens = k
    case.q = case.q.copy()
    case.q[0, 2, 7] = 5.0
    pool = build_both(oracle, case, gpu)
    keys, vals, _, _ = oracle.paged_gather(case.host, case.tables, case.ctx, out_mode=1)
    tab = torch.from_numpy(case.tables).to(gpu)
    cl = torch.from_numpy(case.ctx).to(gpu)
    q = torch.from_numpy(case.q).to(gpu)
    out = torch.full_like(q, float("nan"))
    d = vr.make_decode_desc(pool, tab, cl, q, out, case.tmax, vr.NUMERICS_PLAIN)
    d.clamp_alpha = alpha
    assert vr.lib().vspec_rocm_paged_decode_attention(C.byref(d)) == 1, vr.last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    scale = 1.0 / np.sqrt(case.D)
    off, err, moved = 0, 0.0, 0.0
    for b in range(case.B):
        n = int(case.ctx[b])
        for h in range(case.Hq):
            kh = h // (case.Hq // case.Hkv)
            want = _attention_p_f64(case.q[b, h], keys[off: off + n, kh], vals[off: off + n, kh], alpha, scale)
            base = _attention_p_f64(case.q[b, h], keys[off: off + n, kh], vals[off: off + n, kh], 4.5, scale)
            err = max(err, float(np.abs(got[b, h] - want).max()))
            moved = max(moved, float(np.abs(want - base).max()))
        off += n
    say(f"[alpha] max-abs {err:.2e}; alpha moves the result by {moved:.2e}")
    assert moved > 10 * TOL[dtype]  # the case does depend on alpha
    assert err <= tol_of(dtype, case_vmax(case))


# ----------------------------------------------------------------------------- operand ranges
# The matrix-core kernels feed q' (f16 and int4 pools) and, in the int4 kernel, p * V scale to
# fp16 operands.  The reference computes in fp32/double over the whole float range
# (attention_ref.c:50-79, three_bit_runtime_modules.c:175-250), so these cases put the operands
# far outside fp16's range in both directions and compare with the oracle.


def _decode_scaled(case, pool, dev, mode, scale=0.0, partition_tokens=0):
    import torch
    import vspec_rocm as vr

    out = vr.paged_decode(pool, torch.from_numpy(case.tables).to(dev), torch.from_numpy(case.ctx).to(dev),
                          torch.from_numpy(case.q).to(dev), max_ctx_len=case.tmax, numerics=mode, scale=scale,
                          partition_tokens=partition_tokens)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("D", [64, 128])
def test_decode_huge_query_mode_p(oracle, gpu, flag_gate, dtype, D):
    """Mode P has no +-16 clip, so q' = clip(q) * scale * log2(e) is unbounded: std(q) = 2e5
    with a caller scale of 1.0 (D = 64) and std(q) = 3e6 with the default 1/sqrt(D) (D = 128)
    put |q'| near 1e6 and 5e5, beyond fp16's 65504.  The oracle fixes scale = 1/sqrt(D); for
    D = 64 it gets 8q, which the std clamp maps to 8 clip(q) exactly (a power of two scales the
    double mean, variance and threshold exactly), so its scores equal the reference's on q with
    scale 1.0 bit for bit."""
    say(f"[huge q] dtype={dtype} D={D}")
    case = make_case(oracle, dtype, 3, 8, 2, D, 16, [300, 77, 1], seed=131 + D + dtype, src16=False)
    q = case.q.astype(np.float64)
    if D == 64:
        q_gpu = (q * 2e5).astype(np.float32)
        case.q = (q_gpu * np.float32(8.0)).astype(np.float32)
        scale = 1.0
    else:
        case.q = (q * 3e6).astype(np.float32)
        q_gpu, scale = case.q, 0.0
    pool = build_both(oracle, case, gpu)
    want_q = case.q
    case.q = q_gpu
    got = _decode_scaled(case, pool, gpu, 0, scale=scale)
    case.q = want_q
    check_attention(oracle, case, got, 0)


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_decode_tiny_query_large_keys_mode_p(oracle, gpu, flag_gate, dtype):
    """std(q) = 1e-4 against keys of std 1e4 (mode P): |q'| ~ 1e-5 lies in fp16's subnormal
    range while the scores still spread over a few units, so q' must keep its relative
    precision (the kernels shift it by a power of two before the hi + lo split)."""
    say(f"[tiny q] dtype={dtype}")
    case = make_case(oracle, dtype, 2, 16, 4, 128, 16, [400, 129], seed=141 + dtype, src16=False)
    case.k_tokens = (case.k_tokens * np.float32(1e4)).astype(np.float32)
    case.q = (case.q * np.float32(1e-4)).astype(np.float32)
    pool = build_both(oracle, case, gpu)
    got = run_decode(case, pool, gpu, 0)
    # the scores do spread: the result is far from the plain mean of V
    _, vals, _, _ = oracle.paged_gather(case.host, case.tables, case.ctx, out_mode=1)
    mean0 = vals[: int(case.ctx[0]), 0].astype(np.float64).mean(axis=0)
    assert np.abs(got[0, 0] - mean0).max() > 100 * TOL[DTYPE_F16]
    check_attention(oracle, case, got, 0)


@pytest.mark.parametrize("mode", [0, 1])
def test_decode_int4_large_v_scales(oracle, gpu, flag_gate, mode):
    """int4 V groups with |v| ~ 1e4 (scales ~ 800-2000) under scores that climb by ~7.9 per 128
    tokens: each wave of the int4 kernel takes every 8th tile pair of a range, so its lazy
    running max trails its new scores by up to 2^7.9 and p * scale reaches ~4e5, which fp16
    cannot hold.  The bound is relative: the north-star 4e-3 is stated for unit-scale data,
    and the int4 kernel's P' rounding (relative 2^-12) scales with |v| (2.5e-4 max|v|)."""
    say(f"[large v] mode={mode}")
    D, Hq, Hkv = 128, 8, 2
    G = Hq // Hkv
    case = make_case(oracle, DTYPE_INT4, 2, Hq, Hkv, D, 16, [2049, 1500], seed=151, src16=False)
    T = case.k_tokens.shape[1]
    k = case.k_tokens.astype(np.float64)
    t = np.arange(T, dtype=np.float64)
    for b in range(case.B):
        for hk in range(Hkv):
            q0 = case.q[b, G * hk].astype(np.float64)
            th = 4.5 * q0.std()
            qc = np.clip(q0, -th, th)
            u = q0 / np.linalg.norm(q0)
            per_unit = float(u @ qc) / np.sqrt(D) * np.log2(np.e)  # log2 score per unit of a_t
            a = (7.9 / 128.0) * t / per_unit
            k[b, :, hk, :] = a[:, None] * u[None, :] + 0.05 * k[b, :, hk, :]
    case.k_tokens = k.astype(np.float32)
    case.v_tokens = (case.v_tokens * np.float32(3000.0)).astype(np.float32)
    pool = build_both(oracle, case, gpu)
    vmax = case_vmax(case)
    assert vmax > 1e4
    tol = 2.5e-4 * vmax + 2e-5
    for pt in (0, 1024):
        got = _decode_scaled(case, pool, gpu, mode, partition_tokens=pt)
        want = oracle.paged_decode(mode, case.host, case.tables, case.ctx, case.q)
        assert np.isfinite(got).all(), f"non-finite outputs (partition_tokens={pt})"
        err = float(np.abs(got - want).max())
        say(f"    partition_tokens={pt}: max-abs {err:.3e} (bound {tol:.2e}, outputs up to {np.abs(want).max():.1f})")
        assert err <= tol


@pytest.mark.parametrize("seed", range(24))
def test_decode_random_shapes(oracle, gpu, seed):
    """Seeded random shapes against the oracle: pool dtype, batch 1-12, kv heads 1/2/4/8,
    GQA group 1/2/3/4/8, head_dim 64/128, block 16/32/48/64 tokens, ragged contexts of
    0-700 tokens, numerics P/R, and the plain decode (with a random split-K partition
    size and max_ctx_len, the true bound or 0) or the fused decode step (whose appended
    token the oracle appends too)."""
    import torch
    import vspec_rocm as vr

    rng = np.random.default_rng(9000 + seed)
    dtype = [DTYPE_F32, DTYPE_F16, DTYPE_INT4][seed % 3]
    B = int(rng.integers(1, 13))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    grp = int(rng.choice([1, 2, 3, 4, 8]))
    D = int(rng.choice([64, 128]))
    P = int(rng.choice([16, 32, 48, 64]))
    ctx = rng.integers(0, 701, B).astype(np.int32)
    ctx[rng.random(B) < 0.15] = 0
    mode = int(rng.integers(0, 2))
    step = bool(rng.integers(0, 2)) and dtype != DTYPE_F32
    pt = int(rng.choice([0, 0, 16, 32, 48]))       # split-K partition tokens (plain decode)
    cap = bool(rng.integers(0, 2))                  # max_ctx_len 0: the block table's capacity
    say(f"[random {seed}] dtype={dtype} B={B} Hkv={Hkv} group={grp} D={D} P={P} mode={mode} step={step} "
        f"pt={pt} cap={cap} ctx={ctx.tolist()}")
    case = make_case(oracle, dtype, B, Hkv * grp, Hkv, D, P, ctx, seed=300 + seed,
                     num_blocks=int(((ctx + P - 1) // P).sum()) + 3)
    if step:
        # build the pool without each sequence's last token; the decode step appends it
        full_ctx = case.ctx
        case.ctx = np.maximum(full_ctx - 1, 0).astype(np.int32)
        pool = build_both(oracle, case, gpu)
        case.ctx = full_ctx
        last = np.maximum(full_ctx - 1, 0)
        kn = np.ascontiguousarray(case.k_tokens[np.arange(B), last])
        vn = np.ascontiguousarray(case.v_tokens[np.arange(B), last])
        live = np.flatnonzero(full_ctx > 0)
        if live.size:
            assert oracle.paged_append(case.host, np.ascontiguousarray(case.tables[live]),
                                       (full_ctx[live] - 1).astype(np.int32),
                                       np.ascontiguousarray(kn[live][:, None]), np.ascontiguousarray(vn[live][:, None]))
        out = vr.paged_decode_step(pool, torch.from_numpy(case.tables).to(gpu), torch.from_numpy(full_ctx).to(gpu),
                                   torch.from_numpy(case.q).to(gpu), _np_to_dev(kn, gpu), _np_to_dev(vn, gpu),
                                   max_ctx_len=case.tmax, numerics=mode)
        torch.cuda.synchronize()
        assert_pools_equal(case.host, pool)
        got = out.cpu().numpy()
    else:
        pool = build_both(oracle, case, gpu)
        out = vr.paged_decode(pool, torch.from_numpy(case.tables).to(gpu), torch.from_numpy(case.ctx).to(gpu),
                              torch.from_numpy(case.q).to(gpu), max_ctx_len=0 if cap else case.tmax,
                              numerics=mode, partition_tokens=pt)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
    empty = np.flatnonzero(case.ctx == 0)
    assert np.all(got[empty] == 0.0)
    check_attention(oracle, case, got, mode, subset=np.flatnonzero(case.ctx > 0))


# ----------------------------------------------------------------------------- configs 2-4
@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("mode", [0, 1])
def test_config2_3_qwen_decode(oracle, gpu, flag_gate, dtype, mode):
    """C2 (fp16) and C3 (int4 quantize-on-write): B=16, GQA 32/8, D=128, T=2048+1."""
    say(f"[c2/c3] dtype={dtype} mode={mode} build")
    case = qwen_c2(oracle, dtype)
    pool = build_both(oracle, case, gpu)
    assert_pools_equal(case.host, pool)
    say(f"[c2/c3] dtype={dtype} mode={mode} decode")
    got = run_decode(case, pool, gpu, mode)
    err = check_attention(oracle, case, got, mode)
    say(f"[c2/c3] max-abs {err:.2e}")


def test_config4_continuous_batching(oracle, gpu):
    """C4: B=64, context ~ U[128, 8192], fragmented tables from a 1.2x pool (fp16).
    The whole pool (both sides appended token by token) is compared byte for byte; the
    oracle's attention checks 12 sequences including the shortest and the longest."""
    say("[c4] build")
    case = continuous_c4(oracle)
    pool = build_both(oracle, case, gpu, prefix_split=False)
    assert_pools_equal(case.host, pool)
    order = np.argsort(case.ctx)
    subset = sorted(set(order[:4].tolist() + order[-4:].tolist() + [0, 1, 31, 63]))
    for pt in (0, 256):
        say(f"[c4] decode partition_tokens={pt}")
        got = run_decode(case, pool, gpu, 0, partition_tokens=pt)
        check_attention(oracle, case, got, 0, subset=subset)


@pytest.mark.parametrize("dtype,uniform", [(DTYPE_F16, False), (DTYPE_INT4, False), (DTYPE_INT4, True)])
def test_decode_uneven_pair_shares(oracle, gpu, dtype, uniform):
    """With a grid of two workgroups per CU, the balanced split gives the first-half
    workgroup of each pair a larger share of the tiles (the CU's arbiter favours its older
    waves): for ragged f16 batches and for every int4 batch.  Every share the library
    accepts (500..900 per mille, VSPEC_ROCM_DECODE_OLD_PERMILLE / ..._INT4) changes the
    rounding only: the outputs stay within tolerance of the oracle and close to the equal
    split (f16: 1e-5; int4: a fifth of its oracle tolerance, since P' = p * scale is
    rounded to fp16 against each segment's own running max), every row written (int4:
    whether or not the host is told that every context is the same, which decides the
    merge launch from the shares)."""
    import os

    import torch
    import vspec_rocm as vr

    say(f"[pair shares] dtype={dtype} uniform={uniform} build")
    ctx = [4097] * 20 if uniform else oracle.uniform_int(91, 3000, 5200, 20)
    case = make_case(oracle, dtype, 20, 32, 8, 128, 16, ctx, seed=92 + dtype)
    pool = build_both(oracle, case, gpu, prefix_split=False)
    tab = torch.from_numpy(case.tables).to(gpu)
    cl = torch.from_numpy(case.ctx).to(gpu)
    q = torch.from_numpy(case.q).to(gpu)
    outs = {}
    var = "VSPEC_ROCM_DECODE_OLD_PERMILLE_INT4" if dtype == DTYPE_INT4 else "VSPEC_ROCM_DECODE_OLD_PERMILLE"
    old = os.environ.get(var)
    try:
        for pm in (500, 620, 700, 900):
            os.environ[var] = str(pm)
            for hint in ((0, case.tmax) if uniform else (0,)):
                out = torch.full_like(q, float("nan"))
                vr.paged_decode(pool, tab, cl, q, max_ctx_len=case.tmax, numerics=1, out=out, min_ctx_len=hint)
                outs[(pm, hint)] = out.cpu().numpy()
    finally:
        if old is None:
            os.environ.pop(var, None)
        else:
            os.environ[var] = old
    bound = 1e-5 if dtype != DTYPE_INT4 else 0.2 * tol_of(dtype, case_vmax(case))
    for key, o in outs.items():
        assert np.isfinite(o).all(), key
        err = np.abs(o - outs[(500, 0)]).max()
        say(f"    {key}: max-abs vs equal shares {err:.2e} (bound {bound:.1e})")
        assert err < bound, key
    check_attention(oracle, case, outs[(700, 0)], 1, subset=[0, 5, 11, 19])


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_decode_max_ctx_len_zero(oracle, gpu, flag_gate, dtype):
    """max_ctx_len 0 stands for the block table's capacity: the same attention as with the
    true bound (the f16 / int4 split does not depend on it; the f32 partitions do, which
    moves rounding only)."""
    import torch
    import vspec_rocm as vr

    say(f"[max_ctx_len 0] dtype={dtype}")
    case = make_case(oracle, dtype, 3, 8, 2, 128, 16, [300, 75, 1000], seed=61, num_blocks=96)
    pool = build_both(oracle, case, gpu)
    tab = torch.from_numpy(np.pad(case.tables, ((0, 0), (0, 4)), constant_values=-1)).to(gpu)
    cl = torch.from_numpy(case.ctx).to(gpu)
    q = torch.from_numpy(case.q).to(gpu)
    a = vr.paged_decode(pool, tab, cl, q, max_ctx_len=0, numerics=1).cpu().numpy()
    b = vr.paged_decode(pool, tab, cl, q, max_ctx_len=case.tmax, numerics=1).cpu().numpy()
    if dtype == DTYPE_F32:
        assert np.abs(a - b).max() < 1e-5
    else:
        assert np.array_equal(a, b)
    check_attention(oracle, case, a, 1)


def test_decode_partition_invariance(oracle, gpu):
    """Split-K partition size changes rounding only."""
    say("[partitions]")
    case = make_case(oracle, DTYPE_F16, 4, 32, 8, 128, 16, [1000, 2049, 17, 513], seed=33)
    pool = build_both(oracle, case, gpu)
    outs = [run_decode(case, pool, gpu, 0, partition_tokens=pt) for pt in (0, 16, 64, 256, 4096)]
    for o in outs[1:]:
        assert np.abs(o - outs[0]).max() < 1e-5
    check_attention(oracle, case, outs[0], 0)


def test_decode_back_to_back_and_streams(oracle, gpu):
    """Split work items leave partial states in the workspace for the merge launch that
    follows on the same stream: decodes of different shapes and dtypes back to back on one
    stream, then on two streams at once with their own workspaces, must all reproduce the
    first run bit for bit (every output row written: the output is NaN-filled before each
    launch)."""
    import torch
    import vspec_rocm as vr

    say("[back-to-back] build")
    cases = [make_case(oracle, DTYPE_F16, 5, 32, 8, 128, 16, [700, 2049, 33, 1500, 911], seed=51),
             make_case(oracle, DTYPE_INT4, 3, 16, 4, 128, 16, [1777, 64, 1201], seed=52),
             make_case(oracle, DTYPE_F16, 9, 8, 2, 64, 32, [300, 1, 77, 1023, 640, 0, 5, 260, 999], seed=53)]
    pools = [build_both(oracle, c, gpu) for c in cases]
    dev_args = [(torch.from_numpy(c.tables).to(gpu), torch.from_numpy(c.ctx).to(gpu), torch.from_numpy(c.q).to(gpu))
                for c in cases]

    def decode(i, pt=0, stream=None, workspace=None):
        c = cases[i]
        bt, cl, q = dev_args[i]
        out = torch.full_like(q, float("nan"))
        vr.paged_decode(pools[i], bt, cl, q, max_ctx_len=c.tmax, numerics=1, partition_tokens=pt, out=out,
                        stream=stream, workspace=workspace)
        return out

    first = [decode(i).cpu().numpy() for i in range(len(cases))]
    for i, c in enumerate(cases):
        check_attention(oracle, c, first[i], 1)
    say("[back-to-back] alternating shapes")
    for rep in range(4):
        for i in (2, 0, 1, 0, 2, 1):
            got = decode(i).cpu().numpy()
            assert np.array_equal(got, first[i]), f"rep {rep} case {i}: differs from the first run"
    say("[back-to-back] chunked split between balanced launches")
    for i in range(len(cases)):
        # another split moves the lazy running max; int4 rounds p * scale to fp16 once
        # per token (relative 2^-12), so its results move by up to 2.4e-4 * max|v|
        v = cases[i].v_tokens
        vmax = float(np.abs(v.view(np.float16) if v.dtype == np.uint16 else v).astype(np.float32).max())
        tol = 1e-5 if cases[i].dtype == DTYPE_F16 else 2.4e-4 * vmax + 1e-5
        assert np.abs(decode(i, pt=32).cpu().numpy() - first[i]).max() < tol
        assert np.array_equal(decode(i).cpu().numpy(), first[i])
    say("[back-to-back] two streams")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    torch.cuda.synchronize()
    for rep in range(3):
        for i in range(len(cases)):
            bt, cl, q = dev_args[i]
            d = vr.make_decode_desc(pools[i], bt, cl, q, q, cases[i].tmax, 1)
            nbytes = max(vr.decode_workspace_bytes(d), 4)
            for s in (s1, s2):
                ws = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
                with torch.cuda.stream(s):
                    outs.append((i, decode(i, stream=s.cuda_stream, workspace=ws), ws))
    torch.cuda.synchronize()
    for i, o, _ in outs:
        assert np.array_equal(o.cpu().numpy(), first[i])


@pytest.mark.parametrize("dtype,Hq,Hkv,D,P,pt", [
    (DTYPE_F16, 8, 2, 128, 16, 0), (DTYPE_F16, 16, 2, 64, 32, 0), (DTYPE_F16, 32, 8, 128, 16, 32),
    (DTYPE_INT4, 8, 2, 128, 16, 0), (DTYPE_INT4, 16, 2, 64, 32, 32), (DTYPE_F32, 8, 2, 128, 16, 0)])
@pytest.mark.parametrize("src16", [False, True])
def test_decode_step_fused_append(oracle, gpu, flag_gate, dtype, Hq, Hkv, D, P, pt, src16):
    """vspec_rocm_paged_decode_step (append of the decode token at ctx - 1, then attention;
    one launch for f16 / int4 pools) against kv_append + paged_decode on a second pool
    built identically: the same pool bytes and the same outputs bit for bit, both equal to
    the oracle's append (bit-exact) and attention (within tolerance).  Contexts include 0
    (nothing appended) and 1 (the new token alone); GQA group 8 makes two q-head groups
    share each kv head's last tile; P=32 puts two tiles in a block."""
    say(f"[decode-step] dtype={dtype} Hq={Hq} Hkv={Hkv} D={D} P={P} pt={pt} src16={src16}")
    ctx = np.array([1, 17, 40, 0, 100, 33, 16], np.int32)
    _fused_step_case(oracle, gpu, dtype, Hq, Hkv, D, P, pt, src16, ctx, seed=71 + D + P + dtype)


@pytest.mark.parametrize("dtype,D", [(DTYPE_INT4, 128), (DTYPE_INT4, 64), (DTYPE_F16, 128)])
@pytest.mark.parametrize("pt", [64, 256, 0])
def test_decode_step_many_short_items(oracle, gpu, flag_gate, dtype, D, pt):
    """The fused decode step where one workgroup's range ends many work items: 48 sequences
    of 0-48 tokens over ranges of 4 or 16 tiles (partition_tokens 64 / 256) or the balanced
    split, so that each range appends several tokens (in the int4 kernel the range's first
    item through its LDS record, the others written to the pool by all waves before the
    first barrier).  Pool bytes, clamp flags and outputs equal the separate append + decode
    flow, and the oracle."""
    say(f"[decode-step short items] dtype={dtype} D={D} pt={pt}")
    rng = np.random.default_rng(5150 + D + pt)
    ctx = rng.integers(0, 49, 48).astype(np.int32)
    ctx[:3] = [0, 1, 16]
    _fused_step_case(oracle, gpu, dtype, 32, 8, D, 16, pt, True, ctx, seed=91 + D + pt + dtype)


def _fused_step_case(oracle, gpu, dtype, Hq, Hkv, D, P, pt, src16, ctx, seed):
    import copy

    import torch
    import vspec_rocm as vr

    full = make_case(oracle, dtype, len(ctx), Hq, Hkv, D, P, ctx, seed=seed, src16=src16)
    pre = [copy.copy(full) for _ in range(2)]
    pools = []
    for c in pre:
        c.ctx = np.maximum(full.ctx - 1, 0).astype(np.int32)
        c.host = HostPool(dtype, full.num_blocks, P, Hkv, D)
        fill_garbage(c.host)
        pools.append(build_both(oracle, c, gpu))
    host = pre[0].host
    B = len(ctx)
    last = np.maximum(ctx - 1, 0)
    k_new = np.ascontiguousarray(full.k_tokens[np.arange(B), last])  # [B][Hkv][D]
    v_new = np.ascontiguousarray(full.v_tokens[np.arange(B), last])
    live = np.flatnonzero(ctx > 0)
    assert oracle.paged_append(host, np.ascontiguousarray(full.tables[live]), (ctx[live] - 1).astype(np.int32),
                               np.ascontiguousarray(k_new[live][:, None]), np.ascontiguousarray(v_new[live][:, None]))

    tab = torch.from_numpy(full.tables).to(gpu)
    cl = torch.from_numpy(ctx).to(gpu)
    q = torch.from_numpy(full.q).to(gpu)
    kd, vd = _np_to_dev(k_new, gpu), _np_to_dev(v_new, gpu)
    # reference flow: separate append launch, then decode
    vr.kv_append(pools[0], tab, cl - 1, kd[:, None].contiguous(), vd[:, None].contiguous())
    want = vr.paged_decode(pools[0], tab, cl, q, numerics=1, partition_tokens=pt)
    got = torch.full_like(q, float("nan"))
    vr.paged_decode_step(pools[1], tab, cl, q, kd, vd, numerics=1, partition_tokens=pt, out=got)
    torch.cuda.synchronize()
    for a, b in zip(pool_bytes(pools[0]), pool_bytes(pools[1])):
        if a is not None:
            assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))
    if dtype == DTYPE_INT4:
        assert torch.equal(pools[0].kf, pools[1].kf)  # the clamp flags as well
    assert_pools_equal(host, pools[1])
    assert torch.equal(got, want)
    full.host = host
    check_attention(oracle, full, got.cpu().numpy(), 1)


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
def test_decode_step_in_hip_graph(oracle, gpu, flag_gate, dtype):
    """A decode step (fused append + attention) captured into a HIP graph after one eager
    call on the capture stream (which sets up that stream's merge counters and the
    workspace): every replay, with eager decodes of another batch and synchronisations in
    between, equals the eager step bit for bit, and the pool bytes stay those of the eager
    append (every launch returns the counters to zero; no memset is recorded)."""
    import torch
    import vspec_rocm as vr

    say(f"[hip graph] dtype={dtype}")
    ctx = np.array([700, 33, 1501, 2049, 9], np.int32)
    case = make_case(oracle, dtype, len(ctx), 32, 8, 128, 16, ctx, seed=81)
    other = make_case(oracle, DTYPE_F16, 3, 8, 2, 64, 16, [100, 57, 300], seed=82)
    pool = build_both(oracle, case, gpu)
    pool_o = build_both(oracle, other, gpu)
    tab = torch.from_numpy(case.tables).to(gpu)
    cl = torch.from_numpy(case.ctx).to(gpu)
    q = torch.from_numpy(case.q).to(gpu)
    B = len(ctx)
    last = np.maximum(ctx - 1, 0)
    kd = _np_to_dev(np.ascontiguousarray(case.k_tokens[np.arange(B), last]), gpu)
    vd = _np_to_dev(np.ascontiguousarray(case.v_tokens[np.arange(B), last]), gpu)
    ws = torch.empty(1 << 22, dtype=torch.uint8, device=gpu)
    out = torch.full_like(q, float("nan"))
    s = torch.cuda.Stream()

    def step():
        vr.paged_decode_step(pool, tab, cl, q, kd, vd, max_ctx_len=case.tmax, numerics=1, out=out,
                             workspace=ws, stream=s.cuda_stream)

    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()  # eager: counters and workspace exist before capture
    torch.cuda.synchronize()
    want = out.clone()
    want_pool = [None if a is None else a.copy() for a in pool_bytes(pool)]
    check_attention(oracle, case, want.cpu().numpy(), 1)

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    for rep in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
        for a, b in zip(pool_bytes(pool), want_pool):
            if b is not None:
                assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))
        # eager work between replays, on the default stream
        run_decode(other, pool_o, gpu, 1)


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
def test_decode_step_new_token_dominates(oracle, gpu, flag_gate, dtype):
    """Long contexts (4097 tokens, each work item split over several workgroups) where the
    decode step's own token carries almost all of the softmax weight of one query head per
    group: its key is twice that head's query.  Leaving the token out, or reading its tile
    before the fused append's stores, moves that head's output by O(1); the fused step and
    the separate append + decode must both match the oracle within the tight bound."""
    import copy

    import torch
    import vspec_rocm as vr

    say(f"[dominant token] dtype={dtype}")
    B, Hq, Hkv, D, P, T = 8, 32, 8, 128, 16, 4097
    full = make_case(oracle, dtype, B, Hq, Hkv, D, P, [T] * B, seed=303 + dtype)
    grp = Hq // Hkv
    k = full.k_tokens.copy()
    qf = full.q.reshape(B, Hkv, grp, D)[:, :, 0, :]  # first query head of each group
    k[:, T - 1] = oracle.f32_to_f16((2.0 * qf).astype(np.float32))
    full.k_tokens = k
    pre = copy.copy(full)
    pre.ctx = np.full(B, T - 1, np.int32)
    pre.host = HostPool(dtype, full.num_blocks, P, Hkv, D)
    fill_garbage(pre.host)
    pools = [build_both(oracle, pre, gpu)]
    pre2 = copy.copy(pre)
    pre2.host = HostPool(dtype, full.num_blocks, P, Hkv, D)
    fill_garbage(pre2.host)
    pools.append(build_both(oracle, pre2, gpu))
    host = pre.host
    k_new = np.ascontiguousarray(k[:, T - 1])
    v_new = np.ascontiguousarray(full.v_tokens[:, T - 1])
    assert oracle.paged_append(host, full.tables, np.full(B, T - 1, np.int32), np.ascontiguousarray(k_new[:, None]),
                               np.ascontiguousarray(v_new[:, None]))
    full.host = host
    tab = torch.from_numpy(full.tables).to(gpu)
    cl = torch.from_numpy(full.ctx).to(gpu)
    q = torch.from_numpy(full.q).to(gpu)
    kd, vd = _np_to_dev(k_new, gpu), _np_to_dev(v_new, gpu)
    for mode in (1, 0):
        got = vr.paged_decode_step(pools[0], tab, cl, q, kd, vd, max_ctx_len=T, numerics=mode).cpu().numpy()
        check_attention(oracle, full, got, mode)
        # the new token does dominate: without it the first head of each group moves by O(1)
        without = oracle.paged_decode(mode, pre2.host, full.tables, pre.ctx, full.q)
        assert np.abs(got - without).reshape(B, Hkv, grp, D)[:, :, 0].max() > 0.1
    vr.kv_append(pools[1], tab, cl - 1, kd[:, None].contiguous(), vd[:, None].contiguous())
    got = vr.paged_decode(pools[1], tab, cl, q, max_ctx_len=T, numerics=1).cpu().numpy()
    check_attention(oracle, full, got, 1)


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("B,T,pt", [(64, 4097, 0), (16, 2049, 0), (3, 300, 0), (8, 1025, 32), (8, 1024, 64)])
def test_decode_min_ctx_len_hint(gpu, dtype, B, T, pt, monkeypatch):
    """min_ctx_len == max_ctx_len (every context the same) lets the host skip the merge
    launch when no work item spans two workgroups (64 x 4097: each workgroup holds whole
    items) and keeps it otherwise; the decode step's outputs and pool bytes equal those
    without the hint bit for bit, with the balanced and the chunked split.  (The 8-wave
    whole-item kernel, which the hint can also select, splits differently: switched off
    here, tested against the oracle in test_decode_wide_whole_items.)"""
    import ctypes as C

    import torch
    import vspec_rocm as vr

    monkeypatch.setenv("VSPEC_ROCM_DECODE_WIDE", "0")

    say(f"[min_ctx_len] dtype={dtype} B={B} T={T} pt={pt}")
    Hq, Hkv, D, P = 32, 8, 128, 16
    nblk = (T + P - 1) // P
    g = torch.Generator(device=gpu)
    g.manual_seed(B * 131 + T + dtype)
    pools = [vr.PagedPool(dtype, B * nblk, P, Hkv, D, device=gpu) for _ in range(2)]
    tab = torch.randperm(B * nblk, generator=g, device=gpu).to(torch.int32).view(B, nblk).contiguous()
    kk = torch.randn((B, T - 1, Hkv, D), generator=g, device=gpu, dtype=torch.float16)
    vv = torch.randn((B, T - 1, Hkv, D), generator=g, device=gpu, dtype=torch.float16)
    for pl in pools:
        vr.kv_append(pl, tab, torch.zeros(B, dtype=torch.int32, device=gpu), kk, vv)
    ctx = torch.full((B,), T, dtype=torch.int32, device=gpu)
    q = torch.randn((B, Hq, D), generator=g, device=gpu)
    kn = torch.randn((B, Hkv, D), generator=g, device=gpu, dtype=torch.float16)
    vn = torch.randn((B, Hkv, D), generator=g, device=gpu, dtype=torch.float16)
    outs = []
    for i, hint in enumerate((0, T)):
        out = torch.full_like(q, float("nan"))
        d = vr.make_decode_desc(pools[i], tab, ctx, q, out, T, vr.NUMERICS_3BIT, partition_tokens=pt, min_ctx_len=hint)
        assert vr.lib().vspec_rocm_paged_decode_step(C.byref(d), kn.data_ptr(), vn.data_ptr(), vr.KV_F16), vr.last_error()
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])
    for a, b in zip(pool_bytes(pools[0]), pool_bytes(pools[1])):
        if a is not None:
            assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


@pytest.mark.parametrize("D,Hq,Hkv,P,B,T", [
    (128, 32, 8, 16, 32, 2049),   # 256 items of 129 tiles: the default rule picks it
    (128, 32, 8, 16, 16, 2049),   # C2: 128 items
    (128, 32, 8, 16, 1, 1025),    # one sequence, 8 items
    (128, 16, 4, 32, 5, 300),     # GQA 4, 32-token blocks, a partial last tile
    (64, 8, 8, 16, 7, 33),        # MHA, head_dim 64, three tiles per item
    (128, 24, 2, 16, 3, 4100),    # GQA 12 (three q-head groups per kv head), 257 tiles
    (64, 6, 2, 48, 4, 17),        # GQA 3, 48-token blocks, two tiles
])
def test_decode_wide_whole_items(oracle, gpu, D, Hq, Hkv, P, B, T, monkeypatch):
    """f16 batches with every context the same (min_ctx_len == max_ctx_len) and about one
    work item per CU run one whole item per workgroup of 8 waves (no merge launch); forced
    here for smaller batches too (VSPEC_ROCM_DECODE_WIDE=2).  Against the oracle in both
    numerics modes, through the plain decode and the fused decode step (whose appended rows
    are bit-exact)."""
    import torch
    import vspec_rocm as vr

    monkeypatch.setenv("VSPEC_ROCM_DECODE_WIDE", "2")
    say(f"[wide] D={D} Hq={Hq} Hkv={Hkv} P={P} B={B} T={T}")
    ctx = [T] * B
    case = make_case(oracle, DTYPE_F16, B, Hq, Hkv, D, P, ctx, seed=11 * D + Hq + B + T)
    pool = build_both(oracle, case, gpu)
    tab = torch.from_numpy(case.tables).to(gpu)
    cl = torch.from_numpy(case.ctx).to(gpu)
    q = torch.from_numpy(case.q).to(gpu)
    for mode in (0, 1):
        out = vr.paged_decode(pool, tab, cl, q, max_ctx_len=T, numerics=mode, min_ctx_len=T)
        torch.cuda.synchronize()
        check_attention(oracle, case, out.cpu().numpy(), mode)
    # fused step: the same stream minus its last token, which the decode step appends
    import copy

    pre = copy.copy(case)
    pre.ctx = (case.ctx - 1).astype(np.int32)
    pre.host = HostPool(DTYPE_F16, case.num_blocks, P, Hkv, D)
    fill_garbage(pre.host)
    pool2 = build_both(oracle, pre, gpu)
    k_new = np.ascontiguousarray(case.k_tokens[:, T - 1])  # [B][Hkv][D]
    v_new = np.ascontiguousarray(case.v_tokens[:, T - 1])
    assert oracle.paged_append(pre.host, case.tables, pre.ctx, np.ascontiguousarray(k_new[:, None]),
                               np.ascontiguousarray(v_new[:, None]))
    got = vr.paged_decode_step(pool2, tab, cl, q, _np_to_dev(k_new, gpu), _np_to_dev(v_new, gpu), max_ctx_len=T,
                               numerics=1, min_ctx_len=T)
    torch.cuda.synchronize()
    assert_pools_equal(pre.host, pool2)
    check_attention(oracle, case, got.cpu().numpy(), 1)


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("seg_cost", [0, 3, 16, 64])
def test_decode_ragged_segment_cost(oracle, gpu, seg_cost, dtype, monkeypatch):
    """Ragged batches split over a cost axis on which every work item also costs seg_cost
    tiles (VSPEC_ROCM_DECODE_SEGMENT_COST, ..._INT4): workgroup ranges start and end inside
    items' set-up units and inside their tiles, some are empty, items meet many workgroups
    or none.  Many short sequences beside long ones, GQA 4 and 8 (two q-head groups per kv
    head), plain decode and fused decode step: every output against the oracle, the step's
    appended rows bit-exact.  (Unequal pair shares need >= 64 tiles per workgroup: the
    full-size C4 test covers them with the default cost.)"""
    import copy

    import torch
    import vspec_rocm as vr

    monkeypatch.setenv("VSPEC_ROCM_DECODE_SEGMENT_COST" + ("_INT4" if dtype == DTYPE_INT4 else ""), str(seg_cost))
    say(f"[segment cost] dtype={dtype} cost={seg_cost}")
    ctx = np.array([1, 17, 3000, 16, 33, 5, 200, 64, 2, 1500, 48, 129, 7, 4100, 31, 90] * 2, np.int32)
    for Hq in (32, 64):
        case = make_case(oracle, dtype, len(ctx), Hq, 8, 128, 16, ctx, seed=900 + seg_cost + Hq + dtype)
        pre = copy.copy(case)
        pre.ctx = (case.ctx - 1).astype(np.int32)
        pre.host = HostPool(dtype, case.num_blocks, 16, 8, 128)
        fill_garbage(pre.host)
        pool = build_both(oracle, pre, gpu)
        B = len(ctx)
        k_new = np.ascontiguousarray(case.k_tokens[np.arange(B), ctx - 1])
        v_new = np.ascontiguousarray(case.v_tokens[np.arange(B), ctx - 1])
        assert oracle.paged_append(pre.host, case.tables, pre.ctx, np.ascontiguousarray(k_new[:, None]),
                                   np.ascontiguousarray(v_new[:, None]))
        tab = torch.from_numpy(case.tables).to(gpu)
        cl = torch.from_numpy(case.ctx).to(gpu)
        q = torch.from_numpy(case.q).to(gpu)
        got = vr.paged_decode_step(pool, tab, cl, q, _np_to_dev(k_new, gpu), _np_to_dev(v_new, gpu), numerics=1)
        torch.cuda.synchronize()
        assert_pools_equal(pre.host, pool)
        case.host = pre.host
        check_attention(oracle, case, got.cpu().numpy(), 1)
        out = vr.paged_decode(pool, tab, cl, q, numerics=0)
        torch.cuda.synchronize()
        check_attention(oracle, case, out.cpu().numpy(), 0)


def test_graph_replay_survives_workspace_growth(oracle, gpu):
    """A decode captured into a HIP graph with the library's own workspace; then an eager
    decode on the same stream that needs a larger workspace makes the library replace it.
    The replaced buffer is retired, not freed, so later replays of the graph still match
    the eager result bit for bit; the retired buffer is released afterwards."""
    import torch
    import vspec_rocm as vr

    say("[graph + growth] build")
    small = make_case(oracle, DTYPE_F16, 4, 4, 2, 64, 16, [900, 33, 1601, 257], seed=91)
    # head_dim 128 and 4 heads per work item need about four times the small step's
    # partial-state workspace; 600 sequences x 8 kv heads = 4,800 work items to merge
    big = make_case(oracle, DTYPE_F16, 600, 32, 8, 128, 16, [20 + (i % 13) for i in range(600)], seed=92)
    pool_s = build_both(oracle, small, gpu)
    pool_b = build_both(oracle, big, gpu)
    tab = torch.from_numpy(small.tables).to(gpu)
    cl = torch.from_numpy(small.ctx).to(gpu)
    q = torch.from_numpy(small.q).to(gpu)
    out = torch.full_like(q, float("nan"))
    s = torch.cuda.Stream()

    def step():
        vr.paged_decode(pool_s, tab, cl, q, max_ctx_len=small.tmax, numerics=1, out=out, stream=s.cuda_stream)

    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    want = out.clone()
    check_attention(oracle, small, want.cpu().numpy(), 1)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step()
    tab_b = torch.from_numpy(big.tables).to(gpu)
    cl_b = torch.from_numpy(big.ctx).to(gpu)
    q_b = torch.from_numpy(big.q).to(gpu)
    for rep in range(3):
        if rep == 1:
            say("[graph + growth] larger eager decode on the capture stream")
            with torch.cuda.stream(s):
                got_b = vr.paged_decode(pool_b, tab_b, cl_b, q_b, max_ctx_len=big.tmax, numerics=1,
                                        stream=s.cuda_stream)
            torch.cuda.synchronize()
            check_attention(oracle, big, got_b.cpu().numpy(), 1, subset=[0, 1, 299, 599])
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}"
    # the caller may free the retired buffers once no graph that uses them will run again
    del g
    torch.cuda.synchronize()
    assert vr.lib().vspec_rocm_release_retired_workspaces() == 1, vr.last_error()


def test_decode_step_rejects_bad_source(gpu):
    import torch
    import vspec_rocm as vr

    pool = vr.PagedPool(vr.KV_F16, 4, 16, 2, 128, device=gpu)
    d = vr.make_decode_desc(pool, torch.zeros((1, 4), dtype=torch.int32, device=gpu),
                            torch.ones(1, dtype=torch.int32, device=gpu), torch.zeros((1, 2, 128), device=gpu),
                            torch.zeros((1, 2, 128), device=gpu), 1)
    k = torch.zeros((1, 2, 128), device=gpu)
    assert vr.lib().vspec_rocm_paged_decode_step(d, k.data_ptr(), None, vr.KV_F32) == 0
    assert "null" in vr.last_error()
    assert vr.lib().vspec_rocm_paged_decode_step(d, k.data_ptr(), k.data_ptr(), vr.KV_INT4) == 0
    assert "src_dtype" in vr.last_error()


def _oracle_decode_sampled(oracle, kf, vf, ctx, q, mode, P, Hkv, D):
    """Oracle decode of gathered (f32) rows [sum(ctx)][Hkv][D] laid into an fp32 pool."""
    nb = (ctx + P - 1) // P
    host = HostPool(DTYPE_F32, int(nb.sum()), P, Hkv, D)
    tab = np.full((len(ctx), int(nb.max())), -1, np.int32)
    off = 0
    for i, n in enumerate(nb):
        tab[i, :n] = np.arange(off, off + n, dtype=np.int32)
        off += int(n)
    off = 0
    for i, n in enumerate(ctx):
        n = int(n)
        assert oracle.paged_append(host, tab[i: i + 1], np.zeros(1, np.int32), np.ascontiguousarray(kf[off: off + n][None]),
                                   np.ascontiguousarray(vf[off: off + n][None]))
        off += n
    return oracle.paged_decode(mode, host, tab, ctx, q)


@pytest.mark.parametrize("shape,dtype", [("north-star", DTYPE_F16), ("north-star", DTYPE_INT4),
                                         ("c4", DTYPE_F16)])
def test_full_size_sampled_against_oracle(oracle, gpu, shape, dtype):
    """The benchmark shapes at full size: north star (64 sequences x 4097 tokens, GQA
    32/8, D=128; f16 and int4 pools, int4 through the clamp-flag kernel) and C4 (64
    sequences, contexts U[128, 8192]).  The pool is filled on the GPU, the decode step
    appends each sequence's last token and attends (mode R), then a plain decode runs
    in mode P.  Four sampled sequences are gathered back (dequantised for int4), laid into
    an fp32 oracle pool and decoded by the oracle: the GPU rows must agree within the
    tolerance of the pool dtype.  The append is checked on its own as well: the sampled
    sequences' fp16 source rows (context and decode token) go through the oracle's append
    into a pool of their own, whose raw gather must equal the GPU's byte for byte."""
    import torch
    import vspec_rocm as vr

    B, Hq, Hkv, D, P = 64, 32, 8, 128, 16
    if shape == "north-star":
        ctx = np.full(B, 4097, np.int32)
    else:
        ctx = np.random.default_rng(4).integers(128, 8193, B).astype(np.int32)
    nb = (ctx + P - 1) // P
    say(f"[full-size] {shape} dtype={dtype} tokens={int(ctx.sum())}")
    g = torch.Generator(device=gpu)
    g.manual_seed(1234 + dtype)
    pool = vr.PagedPool(dtype, int(nb.sum()), P, Hkv, D, device=gpu)
    perm = torch.randperm(int(nb.sum()), generator=g, device=gpu).to(torch.int32)
    tab = torch.full((B, int(nb.max())), -1, dtype=torch.int32, device=gpu)
    off = 0
    for b in range(B):
        tab[b, : nb[b]] = perm[off: off + nb[b]]
        off += int(nb[b])
    T = int(ctx.max())
    sample = np.array([0, 17, 42, 63])
    src = {}
    for b in range(B):
        # each sequence's context minus the decode token, in one append launch per sequence
        n = int(ctx[b]) - 1
        k = torch.randn((1, n, Hkv, D), generator=g, device=gpu).to(torch.float16)
        v = torch.randn((1, n, Hkv, D), generator=g, device=gpu).to(torch.float16)
        vr.kv_append(pool, tab[b: b + 1], torch.zeros(1, dtype=torch.int32, device=gpu), k, v)
        if b in sample:
            src[b] = (_f16_bits(k), _f16_bits(v))
    kn = torch.randn((B, Hkv, D), generator=g, device=gpu).to(torch.float16)
    vn = torch.randn((B, Hkv, D), generator=g, device=gpu).to(torch.float16)
    q = torch.randn((B, Hq, D), generator=g, device=gpu)
    cl = torch.from_numpy(ctx).to(gpu)
    got = {1: vr.paged_decode_step(pool, tab, cl, q, kn, vn, max_ctx_len=T, numerics=1).cpu().numpy()}
    got[0] = vr.paged_decode(pool, tab, cl, q, max_ctx_len=T, numerics=0).cpu().numpy()
    torch.cuda.synchronize()
    kn_b, vn_b = _f16_bits(kn), _f16_bits(vn)
    for b in sample:
        n = int(ctx[b])
        chunks = [(src[b][0], src[b][1], 0), (kn_b[b][None, None], vn_b[b][None, None], n - 1)]
        _check_raw_gather_against_oracle(oracle, pool, tab[b: b + 1], cl[b: b + 1], dtype, P, Hkv, D, chunks,
                                         np.arange((n + P - 1) // P, dtype=np.int32), n)
    say(f"[full-size] append of sequences {sample.tolist()} byte-exact")
    st = torch.from_numpy(sample).to(gpu)
    kf, vf, _, _ = vr.kv_gather(pool, tab[st], cl[st], out_mode=vr.GATHER_F32, max_ctx_len=T)
    kf, vf = kf.cpu().numpy(), vf.cpu().numpy()
    qs = q.cpu().numpy()[sample]
    for mode in (1, 0):
        want = _oracle_decode_sampled(oracle, kf, vf, ctx[sample], qs, mode, P, Hkv, D)
        err = np.abs(got[mode][sample] - want).max()
        tol = tol_of(dtype, np.abs(vf).max())
        say(f"[full-size] mode={mode} max-abs {err:.2e} (bound {tol:.1e})")
        assert np.isfinite(got[mode]).all()
        assert err <= tol


def _f16_bits(t):
    return t.contiguous().view(__import__("torch").int16).cpu().numpy().view(np.uint16)


def _check_raw_gather_against_oracle(oracle, pool, tab_row, ctx_row, dtype, P, Hkv, D, chunks, table, ctx,
                                     pool_blocks=None):
    """One sequence at full size: the oracle appends `chunks` ((k, v, start) of fp16 bits,
    [1][n][Hkv][D]) into a pool of its own through the identity table, then gathers `ctx`
    tokens through `table`; the GPU's raw gather of the sequence must hold the same bytes."""
    import vspec_rocm as vr

    nblk = pool_blocks if pool_blocks is not None else int(table.size)
    host = HostPool(dtype, nblk, P, Hkv, D)
    ident = np.arange(nblk, dtype=np.int32)[None, :]
    for k, v, start in chunks:
        assert oracle.paged_append(host, ident, np.array([start], np.int32), np.ascontiguousarray(k),
                                   np.ascontiguousarray(v))
    want = oracle.paged_gather(host, table[None, :].astype(np.int32), np.array([ctx], np.int32), out_mode=0)
    got = vr.kv_gather(pool, tab_row, ctx_row, out_mode=vr.GATHER_RAW, max_ctx_len=ctx)
    for name, g_, w_ in zip(("k", "v", "k_scales", "v_scales"), got, want):
        if w_ is None:
            assert g_ is None
            continue
        gb = np.ascontiguousarray(g_.cpu().numpy()).view(np.uint8).reshape(-1)
        wb = np.ascontiguousarray(w_).view(np.uint8).reshape(-1)
        assert gb.size == wb.size, name
        bad = np.flatnonzero(gb != wb)
        assert bad.size == 0, f"{name}: {bad.size} bytes differ (first at byte {bad[0]})"


def test_config5_full_size_sampled(oracle, gpu):
    """C5 at full size (8 int4 contexts of 16k-32k tokens, one 512-token fp16 chunk each,
    oldest 25 % of blocks evicted, survivors compacted, decode in both modes), built on the
    GPU; two sampled sequences are gathered back dequantised and decoded by the oracle."""
    import torch
    import vspec_rocm as vr
    from cases import chunk_evict_c5

    plan = chunk_evict_c5(oracle)
    B, Hq, Hkv, D, P, chunk = 8, 32, 8, 128, 16, 512
    say(f"[c5-full] contexts {plan['L0'].tolist()} -> {plan['new_ctx'].tolist()}")
    g = torch.Generator(device=gpu)
    g.manual_seed(55)
    pool = vr.PagedPool(DTYPE_INT4, plan["num_blocks"], P, Hkv, D, device=gpu)
    tab = torch.from_numpy(plan["tables"]).to(gpu)
    src = {}
    for b in range(B):
        n = int(plan["L0"][b])
        k = torch.randn((1, n, Hkv, D), generator=g, device=gpu).to(torch.float16)
        v = torch.randn((1, n, Hkv, D), generator=g, device=gpu).to(torch.float16)
        vr.kv_append(pool, tab[b: b + 1], torch.zeros(1, dtype=torch.int32, device=gpu), k, v)
        if b in (0, 5):
            src[b] = (_f16_bits(k), _f16_bits(v))
    kc = torch.randn((B, chunk, Hkv, D), generator=g, device=gpu).to(torch.float16)
    vc = torch.randn((B, chunk, Hkv, D), generator=g, device=gpu).to(torch.float16)
    vr.kv_append(pool, tab, torch.from_numpy(plan["L0"]).to(gpu), kc, vc)
    vr.kv_compact(pool, torch.from_numpy(plan["src"]).to(gpu), torch.from_numpy(plan["dst"]).to(gpu))
    ntab = torch.from_numpy(plan["new_tables"]).to(gpu)
    ncl = torch.from_numpy(plan["new_ctx"]).to(gpu)
    q = torch.randn((B, Hq, D), generator=g, device=gpu)
    T = int(plan["new_ctx"].max())
    got = {m: vr.paged_decode(pool, ntab, ncl, q, max_ctx_len=T, numerics=m).cpu().numpy() for m in (1, 0)}
    sample = np.array([0, 5])
    # the sampled sequences' chunk append, eviction and compaction, independently: the oracle
    # appends their source rows into a pool of their own and keeps the surviving blocks
    kc_b, vc_b = _f16_bits(kc), _f16_bits(vc)
    for b in sample:
        L0, nb, ev = int(plan["L0"][b]), int(plan["nb"][b]), int(plan["ev"][b])
        chunks = [(src[b][0], src[b][1], 0), (kc_b[b: b + 1], vc_b[b: b + 1], L0)]
        _check_raw_gather_against_oracle(oracle, pool, ntab[b: b + 1], ncl[b: b + 1], DTYPE_INT4, P, Hkv, D, chunks,
                                         np.arange(ev, nb, dtype=np.int32), int(plan["new_ctx"][b]), pool_blocks=nb)
    say(f"[c5-full] append + eviction + compaction of sequences {sample.tolist()} byte-exact")
    st = torch.from_numpy(sample).to(gpu)
    kf, vf, _, _ = vr.kv_gather(pool, ntab[st], ncl[st], out_mode=vr.GATHER_F32, max_ctx_len=T)
    kf, vf = kf.cpu().numpy(), vf.cpu().numpy()
    for mode in (1, 0):
        want = _oracle_decode_sampled(oracle, kf, vf, plan["new_ctx"][sample], q.cpu().numpy()[sample], mode, P, Hkv, D)
        err = np.abs(got[mode][sample] - want).max()
        tol = tol_of(DTYPE_INT4, np.abs(vf).max())
        say(f"[c5-full] mode={mode} max-abs {err:.2e} (bound {tol:.1e})")
        assert np.isfinite(got[mode]).all()
        assert err <= tol


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
def test_empty_batches_and_bad_arguments(gpu, dtype):
    """Empty inputs are successful no-ops on every entry point (append, gather, compaction,
    decode, decode step), whatever their pointers; bad decode arguments fail with 0 and a
    message and leave the output as it was."""
    import ctypes as C
    import torch
    import vspec_rocm as vr

    say(f"[empty] dtype={dtype}")
    L = vr.lib()
    pool = vr.PagedPool(dtype, 4, 16, 2, 64, device=gpu)
    kv = pool.desc()
    assert L.vspec_rocm_kv_append(C.byref(kv), 0, None, 0, None, 1, None, None, vr.KV_F32, None) == 1
    assert L.vspec_rocm_kv_append(C.byref(kv), 3, None, 0, None, 0, None, None, vr.KV_F32, None) == 1
    assert L.vspec_rocm_kv_gather(C.byref(kv), 0, None, 0, None, 0, None, 0, None, None, None, None, None) == 1
    assert L.vspec_rocm_kv_compact(C.byref(kv), 0, None, None, None) == 1
    tab = torch.zeros((2, 4), dtype=torch.int32, device=gpu)
    cl = torch.tensor([20, 5], dtype=torch.int32, device=gpu)
    q = torch.randn((2, 4, 64), device=gpu)
    out = torch.full_like(q, 7.0)
    d = vr.make_decode_desc(pool, tab, cl, q, out, 20, vr.NUMERICS_3BIT)
    d.batch = 0
    assert L.vspec_rocm_paged_decode_attention(C.byref(d)) == 1
    assert L.vspec_rocm_paged_decode_step(C.byref(d), None, None, vr.KV_F32) == 1
    d.batch = 2
    bad = [("numerics", 5, "numerics"), ("max_ctx_len", 65, "max_ctx_len"), ("num_q_heads", 3, "num_q_heads")]
    for field, value, word in bad:
        good = getattr(d, field)
        setattr(d, field, value)
        assert L.vspec_rocm_paged_decode_attention(C.byref(d)) == 0, field
        assert word in vr.last_error()
        setattr(d, field, good)
    ws_need = vr.decode_workspace_bytes(d)
    if ws_need:
        small = torch.empty(ws_need - 1, dtype=torch.uint8, device=gpu)
        d.workspace, d.workspace_bytes = small.data_ptr(), ws_need - 1
        assert L.vspec_rocm_paged_decode_attention(C.byref(d)) == 0
        assert "workspace" in vr.last_error()
    assert L.vspec_rocm_paged_decode_attention(None) == 0
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())


# ----------------------------------------------------------------------------- config 5
@pytest.mark.parametrize("mode", [0, 1])
def test_config5_chunk_evict_compact(oracle, gpu, flag_gate, mode):
    """C5 at reduced context: int4 contexts, a 512-token fp16 chunk appended with
    quantize-on-write, oldest 25% of blocks evicted, survivors compacted, decode."""
    import torch
    import vspec_rocm as vr
    from cases import chunk_evict_c5

    say(f"[c5] mode={mode} build")
    plan = chunk_evict_c5(oracle, lo=1000, hi=2600, seed=55 + mode)
    B, Hq, Hkv, D, P, chunk = 8, 32, 8, 128, 16, 512
    host = HostPool(DTYPE_INT4, plan["num_blocks"], P, Hkv, D)
    from cases import fill_garbage
    fill_garbage(host)
    case = type("C", (), {})()
    case.dtype, case.num_blocks, case.P, case.Hkv, case.D = DTYPE_INT4, plan["num_blocks"], P, Hkv, D
    pool = device_pool(case, gpu)
    tab_d = torch.from_numpy(plan["tables"]).to(gpu)
    Lmax = int(plan["L0"].max())
    # initial contexts: appended in 512-token chunks (sequences shorter than a chunk
    # boundary append only their own tokens)
    ks = oracle.f32_to_f16(oracle.normal(501 + mode, B * (Lmax + chunk) * Hkv * D).reshape(B, Lmax + chunk, Hkv, D))
    vs = oracle.f32_to_f16(oracle.normal(601 + mode, B * (Lmax + chunk) * Hkv * D).reshape(B, Lmax + chunk, Hkv, D))
    k_d = _np_to_dev(ks, gpu)
    v_d = _np_to_dev(vs, gpu)
    for s0 in range(0, Lmax, chunk):
        live = np.flatnonzero(plan["L0"] >= s0 + chunk)
        if live.size:
            oracle.paged_append(host, np.ascontiguousarray(plan["tables"][live]), np.full(live.size, s0, np.int32),
                                np.ascontiguousarray(ks[live, s0:s0 + chunk]), np.ascontiguousarray(vs[live, s0:s0 + chunk]))
            li = torch.from_numpy(live).to(gpu)
            vr.kv_append(pool, tab_d[li].contiguous(), torch.full((live.size,), s0, dtype=torch.int32, device=gpu),
                         k_d[li, s0:s0 + chunk].contiguous(), v_d[li, s0:s0 + chunk].contiguous())
    for b in range(B):  # ragged remainder of each initial context, one sequence at a time
        s0 = (int(plan["L0"][b]) // chunk) * chunk
        n = int(plan["L0"][b]) - s0
        if n:
            oracle.paged_append(host, np.ascontiguousarray(plan["tables"][b:b + 1]), np.array([s0], np.int32),
                                np.ascontiguousarray(ks[b:b + 1, s0:s0 + n]), np.ascontiguousarray(vs[b:b + 1, s0:s0 + n]))
            vr.kv_append(pool, tab_d[b:b + 1], torch.tensor([s0], dtype=torch.int32, device=gpu),
                         k_d[b:b + 1, s0:s0 + n].contiguous(), v_d[b:b + 1, s0:s0 + n].contiguous())
    torch.cuda.synchronize()
    say("[c5] chunk append")
    # the chunked-prefill append: every sequence appends 512 tokens at its own position
    kc = np.stack([ks[b, plan["L0"][b]: plan["L0"][b] + chunk] for b in range(B)])
    vc = np.stack([vs[b, plan["L0"][b]: plan["L0"][b] + chunk] for b in range(B)])
    assert oracle.paged_append(host, plan["tables"], plan["L0"], np.ascontiguousarray(kc), np.ascontiguousarray(vc))
    vr.kv_append(pool, tab_d, torch.from_numpy(plan["L0"]).to(gpu), _np_to_dev(kc, gpu), _np_to_dev(vc, gpu))
    torch.cuda.synchronize()
    assert_pools_equal(host, pool)
    say("[c5] evict + compact")
    assert oracle.paged_compact(host, plan["src"], plan["dst"])
    vr.kv_compact(pool, torch.from_numpy(plan["src"]).to(gpu), torch.from_numpy(plan["dst"]).to(gpu))
    torch.cuda.synchronize()
    assert_pools_equal(host, pool)
    say("[c5] decode")
    q = oracle.normal(701 + mode, B * Hq * D).reshape(B, Hq, D)
    out = vr.paged_decode(pool, torch.from_numpy(plan["new_tables"]).to(gpu), torch.from_numpy(plan["new_ctx"]).to(gpu),
                          torch.from_numpy(q).to(gpu), max_ctx_len=int(plan["new_ctx"].max()), numerics=mode)
    torch.cuda.synchronize()
    want = oracle.paged_decode(mode, host, plan["new_tables"], plan["new_ctx"], q)
    err = float(np.abs(out.cpu().numpy() - want).max())
    scales = host.vs.view(np.float16).astype(np.float32)
    tol = tol_of(DTYPE_INT4, 8.0 * np.abs(scales[np.isfinite(scales)]).max())  # |code| <= 8
    say(f"[c5] max-abs {err:.2e} (bound {tol:.1e})")
    assert err <= tol, err


# ----------------------------------------------------------------------------- fused rotary + append
@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("src16", [False, True])
@pytest.mark.parametrize("rope_frac", [1, 2])
def test_append_rope_bitexact(oracle, gpu, dtype, src16, rope_frac):
    """Rotary embedding fused into the append: pool bytes and the rotated q rows are
    bit-identical to the oracle (rotate, then the plain append)."""
    import torch
    import vspec_rocm as vr
    from test_oracle_pin import _rope_tables

    B, H, Hq, D, P = 3, 2, 8, 128, 16
    rope_dim = D // rope_frac
    say(f"[rope] dtype={dtype} src16={src16} rope_dim={rope_dim}")
    case = make_case(oracle, dtype, B, Hq, H, D, P, [40, 7, 33], seed=200 + dtype + 3 * src16 + rope_frac,
                     num_blocks=12, src16=src16)
    cos, sin = _rope_tables(64, rope_dim)
    start = np.array([0, 0, 5], np.int32)
    n_new = 7
    kk = np.ascontiguousarray(case.k_tokens[:, :n_new])
    vv = np.ascontiguousarray(case.v_tokens[:, :n_new])
    assert oracle.paged_append_rope(case.host, case.tables, start, kk, vv, cos, sin, rope_dim)
    pool = device_pool(case, gpu)
    q = oracle.normal(301, B * n_new * Hq * D).reshape(B, n_new, Hq, D)
    qo = vr.kv_append_rope(pool, torch.from_numpy(case.tables).to(gpu), torch.from_numpy(start).to(gpu),
                           _np_to_dev(kk, gpu), _np_to_dev(vv, gpu), torch.from_numpy(cos).to(gpu),
                           torch.from_numpy(sin).to(gpu), rope_dim, q=torch.from_numpy(q).to(gpu))
    torch.cuda.synchronize()
    assert_pools_equal(case.host, pool)
    qg = qo.cpu().numpy()
    for b in range(B):
        for i in range(n_new):
            p_ = start[b] + i
            for h in range(Hq):
                want = oracle.rope_row(q[b, i, h], rope_dim, cos[p_], sin[p_])
                assert np.array_equal(qg[b, i, h].view(np.uint32), want.view(np.uint32)), (b, i, h)


# ----------------------------------------------------------------------------- registry entry
def _legacy_launch(q, k, v, mode):
    """vspec_make_rocm_backend().launch_attention with the reference's context convention
    (cpu_backend.c:40-51): input = host q [H][D], weight = VspecKVCache* over host
    [T][H][D] fp32 rows, output = host out; numerics from the same env switch."""
    import ctypes as C
    import os
    import vspec_rocm as vr

    T, H, D = k.shape
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    cache = vr.VspecKVCache()
    cache.key, cache.value = k.ctypes.data, v.ctypes.data
    cache.max_tokens, cache.num_heads, cache.head_dim, cache.current_tokens = T, H, D, T
    return _launch_cache(q, cache, mode)


def _launch_cache(q, cache, mode):
    """launch_attention over a prepared VspecKVCache (host buffers kept alive by the caller)."""
    import ctypes as C
    import os
    import vspec_rocm as vr

    q = np.ascontiguousarray(q, np.float32)
    out = np.full((cache.num_heads, cache.head_dim), 7.0, np.float32)
    ctx = vr.VspecKernelContext()
    ctx.input, ctx.weight, ctx.output = q.ctypes.data, C.cast(C.pointer(cache), C.c_void_p), out.ctypes.data
    if mode:
        os.environ["VSPEC_3BIT_RUNTIME_MODULE"] = "1"
    else:
        os.environ.pop("VSPEC_3BIT_RUNTIME_MODULE", None)
    os.environ.pop("VSPEC_FUSED_BITS", None)
    be = vr.backend()
    be.launch_attention(C.byref(ctx))
    err = vr.last_error()
    return out, err


def test_backend_attention_demo_known_answer(gpu):
    """examples/attention_demo.c through the ROCm registry entry (2 heads, D=4, 2 tokens):
    the demo's printed values, both numerics modes."""
    k0 = [0.2, 0.1, 0.0, -0.1, 0.1, 0.3, -0.2, 0.4]
    v0 = [0.5, 0.0, 0.1, 0.0, 0.2, 0.3, 0.1, -0.2]
    k1 = [0.0, 0.2, 0.1, 0.3, -0.1, 0.2, 0.2, 0.1]
    v1 = [0.1, 0.2, 0.4, 0.2, 0.0, 0.1, 0.3, 0.2]
    q = np.array([0.3, 0.1, -0.1, 0.0, 0.2, -0.2, 0.3, 0.1], np.float32).reshape(2, 4)
    k = np.array([k0, k1], np.float32).reshape(2, 2, 4)
    v = np.array([v0, v1], np.float32).reshape(2, 2, 4)
    want = np.array([[0.3030, 0.0985, 0.2478, 0.0985], [0.0983, 0.1983, 0.2017, 0.0035]])
    for mode in (0, 1):
        out, err = _legacy_launch(q, k, v, mode)
        assert np.array_equal(np.round(out.astype(np.float64), 4), want), (mode, out, err)


@pytest.mark.parametrize("D", [4, 64, 96, 128])
@pytest.mark.parametrize("mode", [0, 1])
def test_backend_legacy_context_matches_oracle(oracle, gpu, D, mode):
    """Any head size through the legacy context path, fp32 KV, against the oracle's
    attention_ref (1e-4), including keys and queries that make the clamps fire."""
    H, T = 3, 150
    q = oracle.normal(400 + D, H * D).reshape(H, D) * 3
    k = oracle.normal(401 + D, T * H * D).reshape(T, H, D)
    v = oracle.normal(402 + D, T * H * D).reshape(T, H, D)
    k = k.copy()
    k[::9, 1, 0] = 30.0
    out, err = _legacy_launch(q, k, v, mode)
    want = oracle.attention_ref(mode, q, k, v)
    assert np.abs(out - want).max() <= 1e-4, (np.abs(out - want).max(), err)


def _int3_cache(oracle, k, v, block_size, mirror):
    """A VspecKVCache with the reference's int3 codec on (kv_cache.c:160-215): codes and
    scales made by the oracle's codec, and the fp32 mirror of the decoded rows on the
    sides named in `mirror` ("k", "v"), NULL on the others.  Returns (cache, buffers,
    decoded k, decoded v)."""
    import vspec_rocm as vr

    T, H, D = k.shape
    pb, nb = (3 * D + 7) // 8, (D + block_size - 1) // block_size
    bufs, dec = [], []
    for x in (k, v):
        codes = np.zeros((T * H, pb), np.uint8)
        scales = np.zeros((T * H, nb), np.float32)
        rows = np.zeros((T * H, D), np.float32)
        for i, row in enumerate(np.asarray(x, np.float32).reshape(T * H, D)):
            codes[i], scales[i] = oracle.int3_quantize_head(row, block_size)
            oracle.lib.vo_int3_dequantize_head(ptr(codes[i], _u8p), ptr(scales[i], _f32p), D, block_size,
                                               ptr(rows[i], _f32p))
        bufs += [codes, scales, rows]
        dec.append(rows.reshape(T, H, D))
    cache = vr.VspecKVCache()
    cache.max_tokens, cache.num_heads, cache.head_dim, cache.current_tokens = T, H, D, T
    cache.int3_compressed = 1
    cache.key_int3, cache.key_scales = bufs[0].ctypes.data, bufs[1].ctypes.data
    cache.value_int3, cache.value_scales = bufs[3].ctypes.data, bufs[4].ctypes.data
    cache.block_size, cache.blocks_per_head, cache.packed_head_bytes = block_size, nb, pb
    cache.key = bufs[2].ctypes.data if "k" in mirror else None
    cache.value = bufs[5].ctypes.data if "v" in mirror else None
    return cache, bufs, dec[0], dec[1]


@pytest.mark.parametrize("D,block_size", [(4, 32), (20, 16), (64, 16), (128, 32)])
@pytest.mark.parametrize("mode", [0, 1])
def test_backend_int3_cache_without_mirror(oracle, gpu, D, block_size, mode):
    """An int3-compressed VspecKVCache with no fp32 mirror, which the reference's
    accessors decode per read (kv_cache.c:296-362): the device decode gives the mirror's
    rows bit for bit, so the result equals the run over the mirror exactly, on either side
    alone and on both; and it matches the oracle's attention_ref over the decoded rows
    within 1e-4.  D=20 has a partial scale block and codes that straddle bytes."""
    H, T = 3, 70
    q = oracle.normal(500 + D, H * D).reshape(H, D) * 2
    k = oracle.normal(501 + D, T * H * D).reshape(T, H, D)
    v = oracle.normal(502 + D, T * H * D).reshape(T, H, D)
    k[::7, 2, 1] = 25.0
    k[3, 0, :] = 0.0  # an all-zero head: scale 1.0
    ref_out = None
    for mirror in ("kv", "", "k", "v"):
        cache, bufs, kd, vd = _int3_cache(oracle, k, v, block_size, mirror)
        out, err = _launch_cache(q, cache, mode)
        assert not np.all(out == 7.0), err
        if ref_out is None:
            ref_out = out
            want = oracle.attention_ref(mode, q, kd, vd)
            assert np.abs(out - want).max() <= 1e-4, np.abs(out - want).max()
        else:
            assert np.array_equal(out.view(np.uint32), ref_out.view(np.uint32)), mirror


@pytest.mark.parametrize("D", [128, 20])
def test_backend_decode_loop_appends_only(oracle, gpu, D):
    """A 64-step decode loop through the registry entry, as vspec_attention_forward
    (runtime.c:641-647) drives it: each step appends one token to the host VspecKVCache
    (kv_cache.c:160-226) and calls launch_attention.  With the append-only upload switched
    on, the device mirror uploads only the appended rows; every step matches the oracle's
    attention_ref over all rows so far.  Then the cache is rewound (current_tokens shrinks)
    and refilled with other rows at the same addresses: the mirror resyncs and the results
    follow the new rows."""
    import ctypes as C
    import vspec_rocm as vr

    was = vr.lib().vspec_rocm_cache_mirror_append_only(1)
    try:
        _legacy_append_loop(oracle, D)
    finally:
        vr.lib().vspec_rocm_cache_mirror_append_only(-1)
    assert was == 0  # off unless the caller or the environment turns it on


@pytest.mark.parametrize("D", [128, 20])
def test_backend_middle_row_rewrite(oracle, gpu, D):
    """The default upload policy sends every row on every call, so a rewrite of rows in the
    middle of a host VspecKVCache, with current_tokens unchanged and the first and last rows
    untouched, is seen by the next launch_attention (the reference copies all rows per call,
    cuda_attention_f32.cu:108-110): both calls match the oracle over the rows as they are."""
    import ctypes as C
    import vspec_rocm as vr

    H, T = 4, 300
    k = np.ascontiguousarray(oracle.normal(610 + D, T * H * D).reshape(T, H, D))
    v = np.ascontiguousarray(oracle.normal(611 + D, T * H * D).reshape(T, H, D))
    q = oracle.normal(612 + D, H * D).reshape(H, D) * 3
    cache = vr.VspecKVCache()
    cache.key, cache.value = k.ctypes.data, v.ctypes.data
    cache.max_tokens, cache.num_heads, cache.head_dim, cache.current_tokens = T, H, D, T
    assert vr.lib().vspec_rocm_cache_mirror_append_only(-1) == 0
    try:
        for mode in (0, 1):
            out, err = _launch_cache(q, cache, mode)
            want = oracle.attention_ref(mode, q, k, v)
            assert np.abs(out - want).max() <= 2e-5, err
            # rows 100-149 point at q (high scores) and carry large values
            k[100:150] = q[None] * 0.5
            v[100:150] *= 10.0
            out2, err = _launch_cache(q, cache, mode)
            want2 = oracle.attention_ref(mode, q, k, v)
            assert np.abs(want2 - want).max() > 0.1  # the rewrite does change the result
            assert np.abs(out2 - want2).max() <= 2e-5 * max(1.0, float(np.abs(want2).max())), err
            k[:] = oracle.normal(610 + D + 17 * (mode + 1), T * H * D).reshape(T, H, D)
    finally:
        assert vr.lib().vspec_rocm_release_cache_mirror(C.cast(C.pointer(cache), C.c_void_p)) == 1


def _legacy_append_loop(oracle, D):
    import ctypes as C
    import vspec_rocm as vr

    H, T0, steps = 8, 700, 64
    cap = T0 + steps
    k = np.ascontiguousarray(oracle.normal(600 + D, cap * H * D).reshape(cap, H, D))
    v = np.ascontiguousarray(oracle.normal(601 + D, cap * H * D).reshape(cap, H, D))
    q_all = oracle.normal(602 + D, steps * H * D).reshape(steps, H, D)
    kb, vb = np.zeros_like(k), np.zeros_like(v)  # the cache's host buffers
    kb[:T0], vb[:T0] = k[:T0], v[:T0]
    cache = vr.VspecKVCache()
    cache.key, cache.value = kb.ctypes.data, vb.ctypes.data
    cache.max_tokens, cache.num_heads, cache.head_dim, cache.current_tokens = cap, H, D, T0
    try:
        worst = 0.0
        for i in range(steps):
            t = T0 + i
            kb[t], vb[t] = k[t], v[t]
            cache.current_tokens = t + 1
            mode = i % 2
            out, err = _launch_cache(q_all[i], cache, mode)
            want = oracle.attention_ref(mode, q_all[i], kb[: t + 1], vb[: t + 1])
            worst = max(worst, float(np.abs(out - want).max()))
            assert np.abs(out - want).max() <= 2e-5, (i, np.abs(out - want).max(), err)
        say(f"[legacy loop] D={D} steps={steps} max-abs {worst:.2e}")
        # rewind and refill the same buffers with other rows
        kb[:] = -k[::-1]
        vb[:] = v[::-1]
        cache.current_tokens = 300
        out, err = _launch_cache(q_all[0], cache, 1)
        want = oracle.attention_ref(1, q_all[0], kb[:300], vb[:300])
        assert np.abs(out - want).max() <= 2e-5, (np.abs(out - want).max(), err)
    finally:
        assert vr.lib().vspec_rocm_release_cache_mirror(C.cast(C.pointer(cache), C.c_void_p)) == 1


@pytest.mark.parametrize("mode", [0, 1])
def test_backend_through_reference_registry(oracle, ref, gpu, mode):
    """The drop-in through the reference's own registry, compiled from its sources into
    oracle/_ref (backend_registry.c:3-11): vspec_set_backend stores the ROCm entry by value
    in the global slot, and vspec_get_backend()->launch_attention, the call
    vspec_attention_forward makes (runtime.c:641-647), reaches it.  Three contexts: a
    legacy fp32 VspecKVCache (D = 128 through the paged kernels, D = 20 through the generic
    one), an int3 cache without its fp32 mirror, and a VSPEC_KCTX_FLAG_PAGED descriptor.
    The registry path equals the direct call bit for bit; for the two host caches the
    reference CPU entry (vspec_make_cpu_backend, installed the same way) gives the
    reference's own result, which the ROCm entry matches within 2e-5 (fp32 rows) and 1e-4
    (int3 rows)."""
    import ctypes as C
    import os
    import torch
    import vspec_rocm as vr

    RL = ref.lib
    RL.vspec_set_backend.argtypes, RL.vspec_set_backend.restype = [vr.VspecBackend], None
    RL.vspec_get_backend.argtypes, RL.vspec_get_backend.restype = [], C.POINTER(vr.VspecBackend)
    RL.vspec_make_cpu_backend.argtypes, RL.vspec_make_cpu_backend.restype = [], vr.VspecBackend
    rocm, cpu = vr.backend(), RL.vspec_make_cpu_backend()
    if mode:
        os.environ["VSPEC_3BIT_RUNTIME_MODULE"] = "1"
    else:
        os.environ.pop("VSPEC_3BIT_RUNTIME_MODULE", None)
    os.environ.pop("VSPEC_FUSED_BITS", None)

    def via_registry(entry, kctx):
        RL.vspec_set_backend(entry)
        slot = RL.vspec_get_backend().contents
        assert slot.name == entry.name
        slot.launch_attention(C.byref(kctx))

    def host_ctx(q, cache):
        out = np.full((cache.num_heads, cache.head_dim), 7.0, np.float32)
        kctx = vr.VspecKernelContext()
        kctx.input, kctx.weight, kctx.output = q.ctypes.data, C.cast(C.pointer(cache), C.c_void_p), out.ctypes.data
        return kctx, out

    try:
        for D in (128, 20):
            H, T = 4, 157
            k = np.ascontiguousarray(oracle.normal(620 + D, T * H * D).reshape(T, H, D))
            v = np.ascontiguousarray(oracle.normal(621 + D, T * H * D).reshape(T, H, D))
            q = np.ascontiguousarray(oracle.normal(622 + D, H * D).reshape(H, D) * 2)
            k[::11, 1, 3] = 30.0  # keys the std clamp moves
            for kind in ("fp32", "int3"):
                if kind == "fp32":
                    cache = vr.VspecKVCache()
                    cache.key, cache.value = k.ctypes.data, v.ctypes.data
                    cache.max_tokens, cache.num_heads, cache.head_dim, cache.current_tokens = T, H, D, T
                    bufs, tol = (k, v), 2e-5
                else:
                    cache, bufs, _, _ = _int3_cache(oracle, k, v, 16, "")
                    scratch = (np.zeros(D, np.float32), np.zeros(D, np.float32))
                    cache.scratch_key_head, cache.scratch_value_head = scratch[0].ctypes.data, scratch[1].ctypes.data
                    tol = 1e-4
                kc, out_reg = host_ctx(q, cache)
                via_registry(rocm, kc)
                err = vr.last_error()
                kd, out_direct = host_ctx(q, cache)
                rocm.launch_attention(C.byref(kd))
                kr, out_cpu = host_ctx(q, cache)
                via_registry(cpu, kr)
                assert not np.all(out_reg == 7.0) and not np.all(out_cpu == 7.0), err
                assert np.array_equal(out_reg.view(np.uint32), out_direct.view(np.uint32)), (D, kind)
                diff = float(np.abs(out_reg - out_cpu).max())
                say(f"[registry] mode={mode} D={D} {kind}: rocm vs reference cpu entry max-abs {diff:.2e}")
                assert diff <= tol, (D, kind, diff)
                assert vr.lib().vspec_rocm_release_cache_mirror(C.cast(C.pointer(cache), C.c_void_p)) == 1
        # the paged descriptor (device pointers) through the same slot
        case = make_case(oracle, DTYPE_F16, 3, 8, 2, 128, 16, [40, 75, 9], seed=45)
        pool = build_both(oracle, case, gpu)
        tab = torch.from_numpy(case.tables).to(gpu)
        ctx_t = torch.from_numpy(case.ctx).to(gpu)
        qd = torch.from_numpy(case.q).to(gpu)
        want = vr.paged_decode(pool, tab, ctx_t, qd, numerics=mode)
        out = torch.zeros_like(qd)
        d = vr.make_decode_desc(pool, tab, ctx_t, qd, out, case.tmax, numerics=mode)
        kp = vr.VspecKernelContext()
        kp.weight = C.cast(C.pointer(d), C.c_void_p)
        kp.config.flags = vr.KCTX_FLAG_PAGED
        via_registry(rocm, kp)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
        check_attention(oracle, case, out.cpu().numpy(), mode)
    finally:
        RL.vspec_set_backend(vr.VspecBackend())


def test_backend_int3_cache_rejects_bad_geometry(oracle, gpu):
    """A codec-only cache whose block_size is 0 or whose code rows are too short for
    head_dim is refused with an error; the output is left as it was."""
    import vspec_rocm as vr

    H, T, D = 2, 5, 64
    k = oracle.normal(7, T * H * D).reshape(T, H, D)
    for field, bad in (("block_size", 0), ("packed_head_bytes", 23), ("blocks_per_head", 1)):
        cache, bufs, _, _ = _int3_cache(oracle, k, k, 32, "")
        setattr(cache, field, bad)
        out, err = _launch_cache(np.ones((H, D), np.float32), cache, 0)
        assert np.all(out == 7.0), field
        assert "int3" in err, (field, err)
    cache, bufs, _, _ = _int3_cache(oracle, k, k, 32, "")
    cache.int3_compressed = 0
    out, err = _launch_cache(np.ones((H, D), np.float32), cache, 0)
    assert np.all(out == 7.0) and "neither" in err, err


def test_backend_paged_flag(oracle, gpu):
    """launch_attention with VSPEC_KCTX_FLAG_PAGED takes a VspecPagedAttnDesc of device
    pointers and equals vspec_rocm_paged_decode_attention."""
    import ctypes as C
    import torch
    import vspec_rocm as vr

    case = make_case(oracle, DTYPE_F16, 3, 8, 2, 128, 16, [40, 75, 9], seed=44)
    pool = build_both(oracle, case, gpu)
    tab = torch.from_numpy(case.tables).to(gpu)
    ctx_t = torch.from_numpy(case.ctx).to(gpu)
    q = torch.from_numpy(case.q).to(gpu)
    want = vr.paged_decode(pool, tab, ctx_t, q, numerics=1)
    out = torch.zeros_like(q)
    d = vr.make_decode_desc(pool, tab, ctx_t, q, out, case.tmax, numerics=1)
    kc = vr.VspecKernelContext()
    kc.weight = C.cast(C.pointer(d), C.c_void_p)
    kc.config.flags = vr.KCTX_FLAG_PAGED
    vr.backend().launch_attention(C.byref(kc))
    torch.cuda.synchronize()
    assert torch.equal(out, want)
