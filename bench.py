#!/usr/bin/env python3
"""Paged decode-attention benchmark on one MI355X (the BASELINE.json metric).

A step is one layer's decode step for the whole batch: append one new K/V token
per sequence into the paged fp16 cache (block-table append), then single-query
GQA attention over the paged context.  By default both run in one launch
(vspec_rocm_paged_decode_step); --separate-append times the two-launch flow
(vspec_rocm_kv_append, then vspec_rocm_paged_decode_attention).  Inputs are
synthetic (seeded N(0,1)) and resident in HBM before timing starts.

Printed JSON (one line on stdout):
  value      whole-step tokens/s = batch * steps / wall seconds
  roofline   the decode kernel: algorithmic bytes per launch (with the fused
             append's bytes) / the average launch time, from one pair of HIP events
             on the launch stream around all timed launches, against 8 TB/s; and
             against the measured ceilings of lib/libvspec_probe.so: a streaming
             copy (copy_gbs) and a read of 4 KB tiles in random order with the
             decode kernels' non-temporal loads (read_tiles_gbs)
  cpu_baseline  the reference's own C path (oracle/_ref: append + capi gather +
             attention_ref) timed on a bounded sample of the same workload

--probe prints the bandwidth probes alone (copy, random and sequential 4 KB tile reads
with ordinary and non-temporal loads).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "vspec-engine_amd" / "python"))

METRIC = "paged decode-attn tokens/s + achieved HBM GB/s (% of peak), Qwen3-8B KV shape"
PEAK_GBS = 8000.0

WORKLOADS = {
    # T: uniform context; ctx_range: seeded U[lo, hi] per sequence with a pool of 1.2x the
    # needed blocks (continuous batching); flow: the chunked-prefill/evict/compact flow
    "qwen3-8b-b64-ctx4k": dict(B=64, T=4097, Hq=32, Hkv=8, D=128, P=16, dtype="f16"),
    "qwen3-8b-b16-ctx2k": dict(B=16, T=2049, Hq=32, Hkv=8, D=128, P=16, dtype="f16"),
    "qwen3-8b-b16-ctx2k-int4": dict(B=16, T=2049, Hq=32, Hkv=8, D=128, P=16, dtype="int4"),
    # the reference cache's own element type (kv_paged_cache.h:7-49): fp32 pools
    "qwen3-8b-b16-ctx2k-f32": dict(B=16, T=2049, Hq=32, Hkv=8, D=128, P=16, dtype="f32"),
    "qwen3-8b-b64-ctx4k-int4": dict(B=64, T=4097, Hq=32, Hkv=8, D=128, P=16, dtype="int4"),
    "qwen3-8b-b64-ctx128-8k": dict(B=64, ctx_range=(128, 8192), Hq=32, Hkv=8, D=128, P=16, dtype="f16"),
    "qwen3-8b-b64-ctx128-8k-int4": dict(B=64, ctx_range=(128, 8192), Hq=32, Hkv=8, D=128, P=16, dtype="int4"),
    "qwen3-8b-b8-chunk512-evict-int4": dict(B=8, flow="c5", Hq=32, Hkv=8, D=128, P=16, dtype="int4"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def step_append_bytes(B, Hkv, D, dtype):
    """The decode step's append: fp16 K and V rows read, pool rows (and int4 scales) written."""
    row = {"f16": 2 * D, "f32": 4 * D, "int4": D // 2 + 2 * (D // 32)}[dtype]
    return B * Hkv * 2 * (2 * D + row)


def algorithmic_bytes(ctx_lens, Hq, Hkv, D, P, dtype):
    per_token_head = {"f16": 2 * D * 2, "f32": 2 * D * 4, "int4": 2 * (D // 2 + 2 * (D // 32))}[dtype]
    kv = sum(int(t) * Hkv * per_token_head for t in ctx_lens)
    tables = sum(((int(t) + P - 1) // P) * 4 for t in ctx_lens)
    qo = len(ctx_lens) * Hq * D * 8
    return kv + tables + qo


def tiles_per_launch(ctx_lens, Hq, Hkv):
    """16-token tiles the decode kernels stream per launch: one per 16 tokens of every
    (sequence, kv head, group of up to 4 query heads) work item."""
    groups = max(1, (Hq // Hkv) // 4)
    return sum(max(1, (int(t) + 15) // 16) for t in ctx_lens) * Hkv * groups


def cpu_baseline(args, wl, pool, tables, ctx, q_all, out_gpu, mode):
    """Time the reference CPU decode step on the first `cpu_seqs` sequences."""
    import numpy as np
    import torch

    import vspec_rocm as vr

    sys.path.insert(0, str(ROOT))
    S = min(args.cpu_seqs, wl["B"])
    Hq, Hkv, D = wl["Hq"], wl["Hkv"], wl["D"]
    lens = [int(t) for t in ctx[:S].cpu().tolist()]
    if len(set(lens)) > 1:
        return cpu_baseline_ragged(wl, pool, tables, ctx, q_all, out_gpu, mode, S, lens)
    T = lens[0]
    k, v, _, _ = vr.kv_gather(pool, tables[:S], ctx[:S], out_mode=vr.GATHER_F32)
    k = k.cpu().numpy().reshape(S, T, Hkv, D)
    v = v.cpu().numpy().reshape(S, T, Hkv, D)
    q = q_all[:S].cpu().numpy()
    res = {}
    try:
        from oracle.oracle import REF_SO, Reference

        if not REF_SO.exists():
            raise FileNotFoundError(REF_SO)
        ref = Reference()
        sec, out = ref.baseline_decode(mode, 1, k, v, q, wl["P"])
        res = {"value": S / sec, "unit": "tokens/s", "cores": 1, "kind": "reference",
               "sample": f"{S} of {wl['B']} sequences x ctx {T}: reference decode step (paged append + "
                         f"capi.c gather + attention_ref, numerics {'R' if mode else 'P'}), gcc -O3, 1 thread"}
        ncores = len(os.sched_getaffinity(0))
        sec_mt, _ = ref.baseline_decode(mode, ncores, k, v, q, wl["P"])
        res["threads_value"] = S / sec_mt
        res["threads"] = ncores
        sec_p, _ = ref.baseline_decode(1 - mode, 1, k, v, q, wl["P"])
        res["other_numerics_value"] = S / sec_p
    except (FileNotFoundError, OSError) as e:
        log(f"reference library unavailable ({e}); timing the C restatement instead")
        from oracle.oracle import DTYPE_F32, HostPool, Oracle

        orc = Oracle()
        nb = (T + wl["P"] - 1) // wl["P"]
        host = HostPool(DTYPE_F32, S * nb, wl["P"], Hkv, D)
        tab = np.arange(S * nb, dtype=np.int32).reshape(S, nb)
        assert orc.paged_append(host, tab, np.zeros(S, np.int32), k, v)
        t0 = time.perf_counter()
        out = orc.paged_decode(mode, host, tab, np.full(S, T, np.int32), q)
        sec = time.perf_counter() - t0
        res = {"value": S / sec, "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"{S} of {wl['B']} sequences x ctx {T}: oracle restatement (gather + attention), 1 thread"}
    err = float(np.abs(out - out_gpu[:S].cpu().numpy()).max())
    res["parity_max_abs_vs_gpu"] = err
    res.update(host_cpu())
    return res


def host_cpu():
    """The host the CPU baseline ran on: the model name lscpu prints (else /proc/cpuinfo's)
    and the usable threads."""
    import subprocess

    model = ""
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if not model:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model = line.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
    return {"cpu_model": model, "nproc": len(os.sched_getaffinity(0))}


PROBE_LIB = ROOT / "vspec-engine_amd" / "lib" / "libvspec_probe.so"


def probe_ceilings(dev, gib=1, reps=10):
    """Measured HBM ceilings from lib/libvspec_probe.so, each timed with one event pair
    around `reps` launches after two warm-up launches on torch's current stream:
      copy_gbs        streaming copy of `gib` GiB (2 x size bytes moved per launch)
      read_tiles_gbs  2 * gib GiB read as 4 KB tiles in a random order, non-temporal loads
                      (the decode kernels' access pattern and load policy)
      read_tiles_cached_gbs  the same with ordinary loads
      read_seq_gbs    the tiles in order, non-temporal loads"""
    import ctypes as C

    import torch

    if not PROBE_LIB.exists():
        raise FileNotFoundError(f"{PROBE_LIB} is missing: build it with __graft_entry__.build()")
    P = C.CDLL(str(PROBE_LIB))
    P.vspec_probe_copy.restype = C.c_int
    P.vspec_probe_copy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
    P.vspec_probe_read_tiles.restype = C.c_int
    P.vspec_probe_read_tiles.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_int,
                                         C.c_void_p]
    P.vspec_probe_read_tiles_grid.restype = C.c_uint32
    stream = torch.cuda.current_stream().cuda_stream

    def timed(launch, nbytes):
        for _ in range(2):
            assert launch()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            assert launch()
        b.record()
        torch.cuda.synchronize()
        return nbytes * reps / (a.elapsed_time(b) / 1e3) / 1e9

    n = gib << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    src.random_(0, 256)
    res = {"copy_gbs": timed(lambda: P.vspec_probe_copy(src.data_ptr(), dst.data_ptr(), n, stream), 2 * n)}
    del src, dst
    tile = 4096
    buf = torch.empty(2 * n, dtype=torch.uint8, device=dev)
    buf.random_(0, 256)
    ntiles = (2 * n) // tile
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    perm = torch.randperm(ntiles, generator=g, device=dev).to(torch.int32)
    seq = torch.arange(ntiles, dtype=torch.int32, device=dev)
    sink = torch.empty(P.vspec_probe_read_tiles_grid() * 256, dtype=torch.int32, device=dev)
    rd = lambda tab, nt: (lambda: P.vspec_probe_read_tiles(buf.data_ptr(), tab.data_ptr(), ntiles, tile,
                                                           sink.data_ptr(), nt, stream))
    res["read_tiles_gbs"] = timed(rd(perm, 1), 2 * n)
    res["read_tiles_cached_gbs"] = timed(rd(perm, 0), 2 * n)
    res["read_seq_gbs"] = timed(rd(seq, 1), 2 * n)
    del buf, perm, seq, sink
    torch.cuda.synchronize()
    res["probe"] = (f"lib/libvspec_probe.so: copy of {gib} GiB; reads of {2 * gib} GiB as 4 KB tiles; "
                    f"{reps} launches per figure between one event pair")
    return res


def cpu_baseline_ragged(wl, pool, tables, ctx, q_all, out_gpu, mode, S, lens):
    """Reference CPU decode step, one sequence at a time (per-sequence context lengths)."""
    import numpy as np

    import vspec_rocm as vr
    from oracle.oracle import REF_SO, Reference

    if not REF_SO.exists():
        return None
    ref = Reference()
    Hkv, D = wl["Hkv"], wl["D"]
    sec, err = 0.0, 0.0
    for b in range(S):
        k, v, _, _ = vr.kv_gather(pool, tables[b:b + 1], ctx[b:b + 1], out_mode=vr.GATHER_F32)
        k = k.cpu().numpy().reshape(1, lens[b], Hkv, D)
        v = v.cpu().numpy().reshape(1, lens[b], Hkv, D)
        s_b, out = ref.baseline_decode(mode, 1, k, v, q_all[b:b + 1].cpu().numpy(), wl["P"])
        sec += s_b
        err = max(err, float(np.abs(out[0] - out_gpu[b].cpu().numpy()).max()))
    return {"value": S / sec, "unit": "tokens/s", "cores": 1, "kind": "reference",
            "sample": f"{S} of {wl['B']} sequences (contexts {min(lens)}..{max(lens)}): reference decode "
                      f"step (paged append + capi.c gather + attention_ref, numerics {'R' if mode else 'P'}), 1 thread",
            "parity_max_abs_vs_gpu": err, **host_cpu()}


def load_traffic(workload):
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        t = json.loads(f.read_text())
        return t.get(workload, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def calibration_copy(args, dev):
    """One device-to-device copy of a known size (--calibration-copy-mib): rocprofv3
    FETCH_SIZE / WRITE_SIZE of this copy scale the counters to bytes."""
    if args.calibration_copy_mib <= 0:
        return
    import torch

    src = torch.empty(args.calibration_copy_mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def run_c5(args, wl, kv_dtype, mode):
    """Config 5: 8 sequences with int4 contexts L0 ~ U[16384, 32256] (seeded) each append a
    512-token fp16 chunk through quantize-on-write, evict the oldest 25 % of their blocks,
    have the survivors compacted into fresh contiguous blocks, then decode.  Each stage is
    timed with HIP events; the whole flow is one step."""
    import ctypes as C

    import torch

    import vspec_rocm as vr

    dev = torch.device("cuda:0")
    B, Hq, Hkv, D, P, chunk = wl["B"], wl["Hq"], wl["Hkv"], wl["D"], wl["P"], 512
    gc = torch.Generator().manual_seed(args.seed)
    L0 = torch.randint(16384, 32256 + 1, (B,), generator=gc)
    total = L0 + chunk
    nb = (total + P - 1) // P
    ev = nb * 25 // 100
    surv = nb - ev
    used = int(nb.sum())
    num_blocks = used + int(surv.sum())
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)
    pool = vr.PagedPool(kv_dtype, num_blocks, P, Hkv, D, device=dev)
    perm = torch.randperm(used, generator=g, device=dev).to(torch.int32)
    tab = torch.full((B, int(nb.max())), -1, dtype=torch.int32, device=dev)
    off = 0
    for b in range(B):
        tab[b, : nb[b]] = perm[off: off + int(nb[b])]
        off += int(nb[b])
    # initial contexts (setup, untimed): quantize-on-write appends in 512-token chunks
    for s0 in range(0, int(L0.max()), chunk):
        live = [b for b in range(B) if int(L0[b]) >= s0 + chunk]
        if live:
            li = torch.tensor(live, device=dev)
            kk = torch.randn((len(live), chunk, Hkv, D), generator=g, device=dev, dtype=torch.float16)
            vv = torch.randn((len(live), chunk, Hkv, D), generator=g, device=dev, dtype=torch.float16)
            vr.kv_append(pool, tab[li].contiguous(), torch.full((len(live),), s0, dtype=torch.int32, device=dev), kk, vv)
    for b in range(B):
        s0 = int(L0[b]) // chunk * chunk
        n = int(L0[b]) - s0
        if n:
            kk = torch.randn((1, n, Hkv, D), generator=g, device=dev, dtype=torch.float16)
            vv = torch.randn((1, n, Hkv, D), generator=g, device=dev, dtype=torch.float16)
            vr.kv_append(pool, tab[b:b + 1], torch.tensor([s0], dtype=torch.int32, device=dev), kk, vv)
    kc = torch.randn((B, chunk, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    vc = torch.randn((B, chunk, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    start = L0.to(torch.int32).to(dev)
    src = torch.cat([tab[b, int(ev[b]): int(nb[b])] for b in range(B)]).contiguous()
    base = used + torch.cat([torch.zeros(1, dtype=torch.int64), torch.cumsum(surv, 0)[:-1]])
    dst = torch.cat([base[b] + torch.arange(int(surv[b])) for b in range(B)]).to(torch.int32).to(dev)
    new_tab = torch.full((B, int(surv.max())), -1, dtype=torch.int32)
    for b in range(B):
        new_tab[b, : surv[b]] = base[b] + torch.arange(int(surv[b]))
    new_tab = new_tab.to(dev)
    new_ctx = (total - ev * P).to(torch.int32).to(dev)
    q = torch.randn((B, Hq, D), generator=g, device=dev, dtype=torch.float32)
    out = torch.empty_like(q)
    desc = vr.make_decode_desc(pool, new_tab, new_ctx, q, out, int(new_ctx.max()), mode)
    ws = torch.empty(max(vr.decode_workspace_bytes(desc), 4), dtype=torch.uint8, device=dev)
    desc.workspace, desc.workspace_bytes = ws.data_ptr(), ws.numel()
    L = vr.lib()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]

    def flow(e):
        if e:
            e[0].record()
        vr.kv_append(pool, tab, start, kc, vc)
        if e:
            e[1].record()
        vr.kv_compact(pool, src, dst)
        if e:
            e[2].record()
        if not L.vspec_rocm_paged_decode_attention(C.byref(desc)):
            raise vr.VspecRocmError(vr.last_error())
        if e:
            e[3].record()

    calibration_copy(args, dev)
    for _ in range(args.warmup):
        flow(None)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        flow(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    stage = [sum(e[k].elapsed_time(e[k + 1]) for e in evs) / args.steps / 1e3 for k in range(3)]
    row = Hkv * (2 * (D // 2 + 2 * (D // 32)))  # K+V int4 bytes per token (codes + scales)
    append_bytes = B * chunk * (Hkv * D * 2 * 2 + row)          # fp16 in, int4 out
    compact_bytes = 2 * int(surv.sum()) * P * row                 # read + write survivors
    ctxs = new_ctx.cpu().tolist()
    decode_bytes = algorithmic_bytes(ctxs, Hq, Hkv, D, P, "int4")
    gbs = lambda n, t: n / t / 1e9
    return {
        "metric": METRIC, "value": B * args.steps / wall, "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: seeded N(0,1) fp16 tokens quantised to int4 on write",
        "config": {"workload": args.workload, "batch": B, "ctx": [min(ctxs), max(ctxs)], "chunk": chunk,
                   "evict": "oldest 25% of blocks", "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
                   "block_tokens": P, "kv_storage": "int4", "numerics": args.numerics, "parallelism": "single-gpu"},
        "stages": {
            "chunk_append": {"ms": stage[0] * 1e3, "GB/s": gbs(append_bytes, stage[0])},
            "compact": {"ms": stage[1] * 1e3, "GB/s": gbs(compact_bytes, stage[1]), "blocks": int(surv.sum())},
            "decode": {"ms": stage[2] * 1e3, "GB/s": gbs(decode_bytes, stage[2]), "tokens_per_s": B / stage[2]},
        },
        "roofline": {"bound": "hbm", "achieved": gbs(decode_bytes, stage[2]), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": gbs(decode_bytes, stage[2]) / PEAK_GBS, "traffic": load_traffic(args.workload),
                     "kernel": "decode_mfma_i4",
                     "algorithmic_bytes_per_launch": decode_bytes,
                     "tiles_per_launch": tiles_per_launch(ctxs, Hq, Hkv)},
    }


def run_legacy(args):
    """The legacy registry path: launch_attention with a host VspecKVCache (fp32 [T][H][D]
    rows, the reference context convention of cpu_backend.c:40-51) in a decode loop that
    appends one token per call, as vspec_attention_forward drives it.  Times the calls with
    the default upload policy (every row uploaded into the persistent device mirror on each
    call), with the opt-in append-only policy (only the new rows uploaded), and with the
    mirror released before every call (device buffers allocated again as well)."""
    import ctypes as C

    import numpy as np

    import vspec_rocm as vr

    T, H, D = args.legacy_tokens, 8, 128
    steps = max(args.steps, 10)
    rng = np.random.default_rng(args.seed)
    cap = T + args.warmup + steps + 2 * max(5, steps // 10) + 2
    kb = rng.standard_normal((cap, H, D)).astype(np.float32)
    vb = rng.standard_normal((cap, H, D)).astype(np.float32)
    q = rng.standard_normal((H, D)).astype(np.float32)
    out = np.zeros((H, D), np.float32)
    cache = vr.VspecKVCache()
    cache.key, cache.value = kb.ctypes.data, vb.ctypes.data
    cache.max_tokens, cache.num_heads, cache.head_dim, cache.current_tokens = cap, H, D, T
    ctx = vr.VspecKernelContext()
    ctx.input, ctx.weight, ctx.output = q.ctypes.data, C.cast(C.pointer(cache), C.c_void_p), out.ctypes.data
    be = vr.backend()
    L = vr.lib()
    cptr = C.cast(C.pointer(cache), C.c_void_p)

    def loop(n, release):
        t0 = time.perf_counter()
        for _ in range(n):
            cache.current_tokens += 1
            if release:
                L.vspec_rocm_release_cache_mirror(cptr)
            out[:] = 7.0
            be.launch_attention(C.byref(ctx))
            if out[0, 0] == 7.0:
                raise vr.VspecRocmError(vr.last_error())
        return (time.perf_counter() - t0) / n

    loop(args.warmup, False)
    every_row = loop(max(5, steps // 10), False)
    L.vspec_rocm_cache_mirror_append_only(1)
    try:
        loop(2, False)
        appends = loop(steps, False)
    finally:
        L.vspec_rocm_cache_mirror_append_only(-1)
    full = loop(max(5, steps // 10), True)
    L.vspec_rocm_release_cache_mirror(cptr)
    return {"metric": "legacy launch_attention latency (host VspecKVCache, one appended token per call)",
            "value": every_row * 1e6, "unit": "us/call", "higher_is_better": False, "n_gpus": 1,
            "config": {"workload": f"legacy-ctx{T}", "tokens": T, "heads": H, "head_dim": D, "kv": "f32 host rows"},
            "every_row_us_per_call": every_row * 1e6, "append_only_us_per_call": appends * 1e6,
            "released_us_per_call": full * 1e6,
            "note": "every_row: default policy, all rows uploaded into the device mirror per call; "
                    "append_only: vspec_rocm_cache_mirror_append_only(1), only the appended rows uploaded; "
                    "released: the mirror is released before each call"}


def run_plan(args):
    """Host step planning for a steady decode batch: 64 sequences at 4k-token contexts in
    16-token pages, one new token each per step.  Times vspec_rocm_paged_plan_step (tables
    written whole every step) against vspec_rocm_paged_plan_step_update (tables kept between
    steps, changed entries only), both with per-entry used counts, one ctypes call per step
    on one host thread.  Needs no GPU."""
    import ctypes as C

    import numpy as np

    import vspec_rocm as vr

    B, T, P = 64, args.ctx or 4096, 16
    steps = max(args.steps, 200)
    n_calls = steps + args.warmup
    max_blocks = (T + n_calls + P - 1) // P + 1
    L = vr.lib()
    p32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))
    out = {}
    for kind, fn in (("whole", L.vspec_rocm_paged_plan_step), ("update", L.vspec_rocm_paged_plan_step_update)):
        m = L.vspec_rocm_paged_meta_create(P, B * max_blocks + 64, 0, max_blocks)
        tables = np.full((B, max_blocks), -1, np.int32)
        used = np.zeros((B, max_blocks), np.int32)
        ctx = np.zeros(B, np.int32)
        start = np.zeros(B, np.int32)
        titem = np.zeros(B * T, np.int32)
        tpos = np.zeros(B * T, np.int32)
        got = C.c_size_t()
        ptrs = [p32(a) for a in (tables, used, ctx, start, titem, tpos)]
        prefill = (vr.VspecRocmStepItem * B)(*[vr.VspecRocmStepItem(i + 1, 1, T - 1, 0) for i in range(B)])
        decode = (vr.VspecRocmStepItem * B)(*[vr.VspecRocmStepItem(i + 1, 2, 1, T - 1) for i in range(B)])
        try:
            assert fn(m, prefill, B, ptrs[0], ptrs[1], max_blocks, ptrs[2], ptrs[3], ptrs[4], ptrs[5], B * T,
                      C.byref(got))
            for _ in range(args.warmup):
                assert fn(m, decode, B, ptrs[0], ptrs[1], max_blocks, ptrs[2], ptrs[3], ptrs[4], ptrs[5], B * T,
                          C.byref(got))
            t0 = time.perf_counter()
            for _ in range(steps):
                fn(m, decode, B, ptrs[0], ptrs[1], max_blocks, ptrs[2], ptrs[3], ptrs[4], ptrs[5], B * T, C.byref(got))
            out[kind] = (time.perf_counter() - t0) / steps * 1e6
            assert int(ctx[0]) == T - 1 + args.warmup + steps
        finally:
            L.vspec_rocm_paged_meta_destroy(m)
    return {"metric": "host step planning, 64-sequence decode step", "value": out["update"], "unit": "us/step",
            "higher_is_better": False, "n_gpus": 0, "steps": steps,
            "config": {"workload": f"plan-b{B}-ctx{T}", "batch": B, "ctx": T, "page_tokens": P,
                       "tables": "block ids + per-entry used counts"},
            "whole_us_per_step": out["whole"], "update_us_per_step": out["update"],
            "note": "whole: vspec_rocm_paged_plan_step writes every row; update: vspec_rocm_paged_plan_step_update "
                    "writes the entries that changed; one ctypes call per step, one host thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="qwen3-8b-b64-ctx4k", choices=sorted(WORKLOADS))
    ap.add_argument("--numerics", default="R", choices=["P", "R"])
    ap.add_argument("--partition-tokens", type=int, default=0)
    ap.add_argument("--cpu-seqs", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--launch-samples", type=int, default=20,
                    help="after the timed steps, time this many single launches between event pairs "
                         "for the per-launch distribution (p10/median/p90; not part of value)")
    ap.add_argument("--probe", action="store_true",
                    help="print the HBM bandwidth probes (copy, random/sequential tile reads) and exit")
    ap.add_argument("--no-probe", action="store_true",
                    help="skip the probe ceilings in the bench line")
    ap.add_argument("--plan", action="store_true",
                    help="time the host step planner (64 sequences, --ctx tokens, default 4096) and exit; no GPU")
    ap.add_argument("--legacy", action="store_true",
                    help="time the legacy registry path (launch_attention over a host VspecKVCache) and exit")
    ap.add_argument("--legacy-tokens", type=int, default=4096)
    ap.add_argument("--separate-append", action="store_true",
                    help="append with its own launch before the decode launch (timed: the decode)")
    ap.add_argument("--batch", type=int, default=0,
                    help="override the workload's batch (uniform-context workloads only)")
    ap.add_argument("--ctx", type=int, default=0,
                    help="override the workload's context, decode token included (uniform only)")
    ap.add_argument("--seed", type=int, default=2026)
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="copy a buffer of this many MiB on the device once before warm-up, so that "
                         "rocprofv3 FETCH_SIZE/WRITE_SIZE of the same run can be scaled to bytes")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the paged decode "
              "path would shard by sequence or kv head, with no exchange between GPUs). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.plan:
        print(json.dumps(run_plan(args)), flush=True)
        return

    import torch

    import vspec_rocm as vr

    vr.lib()
    dev = torch.device("cuda:0")
    if args.legacy:
        print(json.dumps(run_legacy(args)), flush=True)
        return
    if args.probe:
        print(json.dumps({"metric": "HBM bandwidth probes", "unit": "GB/s", "peak": PEAK_GBS,
                          **probe_ceilings(dev), **{"host": host_cpu()}}), flush=True)
        return
    wl = dict(WORKLOADS[args.workload])
    if args.batch or args.ctx:
        if "T" not in wl:
            sys.exit("--batch / --ctx apply to uniform-context workloads only")
        wl["B"] = args.batch or wl["B"]
        wl["T"] = args.ctx or wl["T"]
    kv_dtype = {"f16": vr.KV_F16, "f32": vr.KV_F32, "int4": vr.KV_INT4}[wl["dtype"]]
    mode = vr.NUMERICS_3BIT if args.numerics == "R" else vr.NUMERICS_PLAIN
    if wl.get("flow") == "c5":
        print(json.dumps(run_c5(args, wl, kv_dtype, mode)), flush=True)
        return
    B, Hq, Hkv, D, P = wl["B"], wl["Hq"], wl["Hkv"], wl["D"], wl["P"]
    if "ctx_range" in wl:
        lo, hi = wl["ctx_range"]
        gc = torch.Generator().manual_seed(args.seed)
        lens = torch.randint(lo, hi + 1, (B,), generator=gc).tolist()
    else:
        lens = [wl["T"]] * B
    T = max(lens)
    nblks = [(t + P - 1) // P for t in lens]
    nblk = max(nblks)
    pool_blocks = sum(nblks) if "ctx_range" not in wl else -(-sum(nblks) * 6 // 5)
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)

    # pools smaller than the 256 MB MALL are rotated through >= 4 copies (>= 1 GB total)
    per_pool = vr.lib().vspec_rocm_kv_pool_bytes(kv_dtype, pool_blocks, P, Hkv, D)
    copies = 1 if per_pool >= (1 << 30) else max(4, -(-(1 << 30) // per_pool))
    log(f"workload {args.workload}: B={B} ctx={min(lens)}..{T} GQA {Hq}/{Hkv} D={D} P={P} {wl['dtype']} "
        f"pool {per_pool / 1e9:.3f} GB x {copies}")

    def make_table():
        perm = torch.randperm(pool_blocks, generator=g, device=dev).to(torch.int32)
        tab = torch.full((B, nblk), -1, dtype=torch.int32, device=dev)
        off = 0
        for b in range(B):
            tab[b, : nblks[b]] = perm[off: off + nblks[b]]
            off += nblks[b]
        return tab

    pools, tables_l = [], []
    for c in range(copies):
        pool = vr.PagedPool(kv_dtype, pool_blocks, P, Hkv, D, device=dev)
        if kv_dtype == vr.KV_INT4:
            # build the cache by quantize-on-write appends of fp16 N(0,1) tokens
            tab = make_table()
            chunk = 512
            for s0 in range(0, T, chunk):
                n = min(chunk, T - s0)
                kn = torch.randn((B, n, Hkv, D), generator=g, device=dev, dtype=torch.float16)
                vn = torch.randn((B, n, Hkv, D), generator=g, device=dev, dtype=torch.float16)
                vr.kv_append(pool, tab, torch.full((B,), s0, dtype=torch.int32, device=dev), kn, vn)
        else:
            pool.k.copy_(torch.randn(pool.k.shape, generator=g, device=dev, dtype=torch.float32).to(pool.k.dtype))
            pool.v.copy_(torch.randn(pool.v.shape, generator=g, device=dev, dtype=torch.float32).to(pool.v.dtype))
            tab = make_table()
        pools.append(pool)
        tables_l.append(tab)
    ctx = torch.tensor(lens, dtype=torch.int32, device=dev)
    pos = ctx - 1
    q = torch.randn((B, Hq, D), generator=g, device=dev, dtype=torch.float32)
    k_new = torch.randn((B, 1, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    v_new = torch.randn((B, 1, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    # the host knows the contexts: min_ctx_len lets a uniform batch skip the merge launch
    # when no work item spans two workgroups
    descs = [vr.make_decode_desc(pools[c], tables_l[c], ctx, q, out, T, mode, partition_tokens=args.partition_tokens,
                                 min_ctx_len=min(lens)) for c in range(copies)]
    ws_bytes = max(vr.decode_workspace_bytes(d) for d in descs)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    import ctypes as C

    for d in descs:
        d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel()
    L = vr.lib()

    def step(i, ev=None):
        c = i % copies
        if ev:
            ev[0].record()
        if args.separate_append:
            vr.kv_append(pools[c], tables_l[c], pos, k_new, v_new)
            ok = L.vspec_rocm_paged_decode_attention(C.byref(descs[c]))
        else:
            ok = L.vspec_rocm_paged_decode_step(C.byref(descs[c]), k_new.data_ptr(), v_new.data_ptr(), vr.KV_F16)
        if not ok:
            raise vr.VspecRocmError(vr.last_error())
        if ev:
            ev[1].record()

    # The probes run first: they are untimed work the line needs anyway, and after them the
    # timed steps run in the card's steady state.  Timed straight after the pool set-up, a
    # short run lands in the card's transient at the start of a load (north star: launches of
    # ~166 us, then ~185-190 us for a few ms, then ~170 us), so 20 steps read 3 % slower and
    # vary more between boxes.
    pc = None
    if not args.no_probe:
        log("probe ceilings ...")
        pc = probe_ceilings(dev)
    calibration_copy(args, dev)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    # one event pair on the launch stream (torch's current stream, which the descriptors
    # name) around all timed launches
    span = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
    t0 = time.perf_counter()
    span[0].record()
    for i in range(args.steps):
        step(i)
    span[1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    avg_attn_s = span[0].elapsed_time(span[1]) / args.steps / 1e3
    # per-launch distribution, outside the timed region
    samples = []
    for i in range(max(0, args.launch_samples)):
        ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
        step(i, ev)
        torch.cuda.synchronize()
        samples.append(ev[0].elapsed_time(ev[1]))
    samples.sort()
    pct = lambda f: samples[min(len(samples) - 1, int(f * len(samples)))] if samples else None

    # the step's append bytes count in both modes (fused: the same launch; separate: the
    # append launch sits inside the event span too)
    alg = algorithmic_bytes(lens, Hq, Hkv, D, P, wl["dtype"]) + step_append_bytes(B, Hkv, D, wl["dtype"])
    achieved = alg / avg_attn_s / 1e9
    traffic = load_traffic(args.workload)

    result = {
        "metric": METRIC,
        "value": B * args.steps / wall,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) K/V resident in HBM, random-permutation block tables",
        "config": {"workload": args.workload, "batch": B, "ctx": T if min(lens) == T else [min(lens), T],
                   "q_heads": Hq, "kv_heads": Hkv,
                   "head_dim": D, "block_tokens": P, "kv_storage": wl["dtype"], "numerics": args.numerics,
                   "append": "separate launch" if args.separate_append else "fused into the decode launch",
                   "pool_copies": copies, "parallelism": "single-gpu"},
        "decode_launch": {"timing": f"one event pair around the {args.steps} timed launches",
                          "tokens_per_s": B / avg_attn_s, "avg_ms": avg_attn_s * 1e3,
                          "single_launch_samples": len(samples), "median_ms": pct(0.5), "p10_ms": pct(0.1),
                          "p90_ms": pct(0.9)},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBS, "traffic": traffic,
                     "kernel": ("kv_append + " if args.separate_append else "") +
                               {"f16": "decode_mfma_f16", "int4": "decode_mfma_i4",
                                "f32": "decode_partial" + (" + decode_combine" if ws_bytes else "")}[wl["dtype"]],
                     "algorithmic_bytes_per_launch": alg,
                     "tiles_per_launch": tiles_per_launch(lens, Hq, Hkv)},
    }
    if pc is not None:
        rf = result["roofline"]
        rf["copy_gbs"] = pc["copy_gbs"]
        rf["frac_of_copy"] = achieved / pc["copy_gbs"]
        rf["read_tiles_gbs"] = pc["read_tiles_gbs"]
        rf["frac_of_read_tiles"] = achieved / pc["read_tiles_gbs"]
        rf["probe"] = pc["probe"]
    if (Hq, Hkv, D) == (32, 8, 128):
        # one step covers one layer; Qwen3-8B decodes a token through 36 of them
        result["model_level"] = {"model": "Qwen3-8B", "layers": 36, "tokens_per_s": result["value"] / 36}
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        # the parity spot check compares against pool 0 (the timed loop rotates pools)
        if not L.vspec_rocm_paged_decode_attention(C.byref(descs[0])):
            raise vr.VspecRocmError(vr.last_error())
        torch.cuda.synchronize()
        cb = cpu_baseline(args, wl, pools[0], tables_l[0], ctx, q, out, mode)
        if cb is not None:
            result["cpu_baseline"] = cb
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
