#!/usr/bin/env python3
"""Paged decode-attention benchmark on one MI355X (the BASELINE.json metric).

A step is one layer's decode step for the whole batch: append one new K/V token
per sequence into the paged fp16 cache (block-table append), then single-query
GQA attention over the paged context.  Inputs are synthetic (seeded N(0,1)) and
resident in HBM before timing starts.

Printed JSON (one line on stdout):
  value      whole-step tokens/s = batch * steps / wall seconds
  roofline   the attention kernels: algorithmic bytes per launch / the average
             launch time from HIP events on the launch stream, against 8 TB/s
  cpu_baseline  the reference's own C path (oracle/_ref: append + capi gather +
             attention_ref) timed on a bounded sample of the same workload
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
    # name: (batch, ctx, q_heads, kv_heads, head_dim, block_tokens, kv dtype)
    "qwen3-8b-b64-ctx4k": dict(B=64, T=4097, Hq=32, Hkv=8, D=128, P=16, dtype="f16"),
    "qwen3-8b-b16-ctx2k": dict(B=16, T=2049, Hq=32, Hkv=8, D=128, P=16, dtype="f16"),
    "qwen3-8b-b16-ctx2k-int4": dict(B=16, T=2049, Hq=32, Hkv=8, D=128, P=16, dtype="int4"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(ctx_lens, Hq, Hkv, D, P, dtype):
    per_token_head = {"f16": 2 * D * 2, "f32": 2 * D * 4, "int4": 2 * (D // 2 + 2 * (D // 32))}[dtype]
    kv = sum(int(t) * Hkv * per_token_head for t in ctx_lens)
    tables = sum(((int(t) + P - 1) // P) * 4 for t in ctx_lens)
    qo = len(ctx_lens) * Hq * D * 8
    return kv + tables + qo


def cpu_baseline(args, wl, pool, tables, ctx, q_all, out_gpu, mode):
    """Time the reference CPU decode step on the first `cpu_seqs` sequences."""
    import numpy as np
    import torch

    import vspec_rocm as vr

    sys.path.insert(0, str(ROOT))
    S = min(args.cpu_seqs, wl["B"])
    T, Hq, Hkv, D = wl["T"], wl["Hq"], wl["Hkv"], wl["D"]
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
    return res


def load_traffic(workload):
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    try:
        t = json.loads(f.read_text())
        return t.get(workload, {}).get("hbm_bytes_per_launch")
    except (ValueError, OSError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="qwen3-8b-b64-ctx4k", choices=sorted(WORKLOADS))
    ap.add_argument("--numerics", default="R", choices=["P", "R"])
    ap.add_argument("--partition-tokens", type=int, default=0)
    ap.add_argument("--cpu-seqs", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=2026)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the paged decode "
              "path shards by sequence or kv head with no exchange; see DESIGN.md). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import vspec_rocm as vr

    vr.lib()
    dev = torch.device("cuda:0")
    wl = WORKLOADS[args.workload]
    B, T, Hq, Hkv, D, P = wl["B"], wl["T"], wl["Hq"], wl["Hkv"], wl["D"], wl["P"]
    kv_dtype = {"f16": vr.KV_F16, "f32": vr.KV_F32, "int4": vr.KV_INT4}[wl["dtype"]]
    mode = vr.NUMERICS_3BIT if args.numerics == "R" else vr.NUMERICS_PLAIN
    nblk = (T + P - 1) // P
    g = torch.Generator(device=dev)
    g.manual_seed(args.seed)

    # pools smaller than the 256 MB MALL are rotated through >= 4 copies (>= 1 GB total)
    per_pool = vr.lib().vspec_rocm_kv_pool_bytes(kv_dtype, B * nblk, P, Hkv, D)
    copies = 1 if per_pool >= (1 << 30) else max(4, -(-(1 << 30) // per_pool))
    log(f"workload {args.workload}: B={B} ctx={T} GQA {Hq}/{Hkv} D={D} P={P} {wl['dtype']} "
        f"pool {per_pool / 1e9:.3f} GB x {copies}")

    pools, tables_l = [], []
    for c in range(copies):
        pool = vr.PagedPool(kv_dtype, B * nblk, P, Hkv, D, device=dev)
        if kv_dtype == vr.KV_INT4:
            # build the cache by quantize-on-write appends of fp16 N(0,1) tokens
            tab = torch.randperm(B * nblk, generator=g, device=dev).to(torch.int32).view(B, nblk)
            chunk = 512
            for s0 in range(0, T, chunk):
                n = min(chunk, T - s0)
                kn = torch.randn((B, n, Hkv, D), generator=g, device=dev, dtype=torch.float16)
                vn = torch.randn((B, n, Hkv, D), generator=g, device=dev, dtype=torch.float16)
                vr.kv_append(pool, tab, torch.full((B,), s0, dtype=torch.int32, device=dev), kn, vn)
        else:
            pool.k.copy_(torch.randn(pool.k.shape, generator=g, device=dev, dtype=torch.float32).to(pool.k.dtype))
            pool.v.copy_(torch.randn(pool.v.shape, generator=g, device=dev, dtype=torch.float32).to(pool.v.dtype))
            tab = torch.randperm(B * nblk, generator=g, device=dev).to(torch.int32).view(B, nblk)
        pools.append(pool)
        tables_l.append(tab)
    ctx = torch.full((B,), T, dtype=torch.int32, device=dev)
    pos = torch.full((B,), T - 1, dtype=torch.int32, device=dev)
    q = torch.randn((B, Hq, D), generator=g, device=dev, dtype=torch.float32)
    k_new = torch.randn((B, 1, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    v_new = torch.randn((B, 1, Hkv, D), generator=g, device=dev, dtype=torch.float16)
    out = torch.empty_like(q)
    descs = [vr.make_decode_desc(pools[c], tables_l[c], ctx, q, out, T, mode,
                                 partition_tokens=args.partition_tokens) for c in range(copies)]
    ws_bytes = max(vr.decode_workspace_bytes(d) for d in descs)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    import ctypes as C

    for d in descs:
        d.workspace, d.workspace_bytes = ws.data_ptr(), ws.numel()
    L = vr.lib()

    def step(i):
        c = i % copies
        vr.kv_append(pools[c], tables_l[c], pos, k_new, v_new)
        ev = evs[i] if i >= 0 else None
        if ev:
            ev[0].record()
        if not L.vspec_rocm_paged_decode_attention(C.byref(descs[c])):
            raise vr.VspecRocmError(vr.last_error())
        if ev:
            ev[1].record()

    evs = [None] * 0
    for i in range(args.warmup):
        step(-1 - i)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    attn_ms = [a.elapsed_time(b) for a, b in evs]
    attn_ms.sort()
    avg_attn_s = sum(attn_ms) / len(attn_ms) / 1e3
    med_attn_ms = attn_ms[len(attn_ms) // 2]

    alg = algorithmic_bytes([T] * B, Hq, Hkv, D, P, wl["dtype"])
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
        "config": {"workload": args.workload, "batch": B, "ctx": T, "q_heads": Hq, "kv_heads": Hkv,
                   "head_dim": D, "block_tokens": P, "kv_storage": wl["dtype"], "numerics": args.numerics,
                   "pool_copies": copies, "parallelism": "single-gpu"},
        "attention_only": {"tokens_per_s": B / avg_attn_s, "avg_ms": avg_attn_s * 1e3, "median_ms": med_attn_ms,
                           "p10_ms": attn_ms[len(attn_ms) // 10], "p90_ms": attn_ms[(9 * len(attn_ms)) // 10]},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_GBS, "traffic": traffic,
                     "kernel": ("decode_mfma_f16" if wl["dtype"] == "f16" else "decode_partial")
                               + (" + decode_combine" if ws_bytes else ""),
                     "algorithmic_bytes_per_launch": alg},
    }
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        # the parity spot check compares against pool 0 (the timed loop rotates pools)
        if not L.vspec_rocm_paged_decode_attention(C.byref(descs[0])):
            raise vr.VspecRocmError(vr.last_error())
        torch.cuda.synchronize()
        result["cpu_baseline"] = cpu_baseline(args, wl, pools[0], tables_l[0], ctx, q, out, mode)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
