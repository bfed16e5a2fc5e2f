"""Seeded builders for the BASELINE.json configurations (host side, numpy).

Inputs come from the oracle's splitmix64/Box-Muller generator so the CPU oracle
and the GPU path consume identical bytes (fp16 values are fp32 draws rounded to
nearest-even once, on the host).  Used only by tests/.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from oracle.oracle import DTYPE_F16, DTYPE_F32, DTYPE_INT4, HostPool

# garbage bit patterns for never-written pool memory: NaN for f32/f16, NaN scales for int4
GARBAGE = {DTYPE_F32: (np.uint32(0x7FC00000), None), DTYPE_F16: (np.uint16(0x7E00), None),
           DTYPE_INT4: (np.uint8(0x88), np.uint16(0x7E00))}


@dataclass
class Case:
    dtype: int
    B: int
    Hq: int
    Hkv: int
    D: int
    P: int
    ctx: np.ndarray               # int32 [B] context after the decode-step append
    tables: np.ndarray            # int32 [B][max_blocks]
    num_blocks: int
    k_tokens: np.ndarray          # [B][Tmax][Hkv][D] f32 or f16 bits (the appended stream)
    v_tokens: np.ndarray
    q: np.ndarray                 # [B][Hq][D] f32
    host: HostPool = field(default=None)

    @property
    def tmax(self):
        return int(self.ctx.max())


def fill_garbage(pool: HostPool):
    g, gs = GARBAGE[pool.dtype]
    if pool.dtype == DTYPE_F32:
        pool.k.view(np.uint32)[...] = g
        pool.v.view(np.uint32)[...] = g
    else:
        pool.k[...] = g
        pool.v[...] = g
    if gs is not None:
        pool.ks[...] = gs
        pool.vs[...] = gs


def make_case(oracle, dtype, B, Hq, Hkv, D, P, ctx, seed, num_blocks=None, table="perm", src16=None):
    ctx = np.asarray(ctx, np.int32)
    nblk = np.maximum(1, (ctx + P - 1) // P)
    max_blocks = int(nblk.max())
    need = int(nblk.sum())
    if num_blocks is None:
        num_blocks = need
    if table == "identity":
        assert B == 1
        tables = np.arange(max_blocks, dtype=np.int32)[None, :]
    else:
        perm = oracle.permutation(seed ^ 0x5EED, num_blocks)
        tables = np.full((B, max_blocks), -1, np.int32)
        off = 0
        for b in range(B):
            tables[b, : nblk[b]] = perm[off: off + nblk[b]]
            off += nblk[b]
    tmax = int(ctx.max()) if len(ctx) else 0
    n = B * max(tmax, 1) * Hkv * D
    k = oracle.normal(seed, n).reshape(B, max(tmax, 1), Hkv, D)
    v = oracle.normal(seed + 1, n).reshape(B, max(tmax, 1), Hkv, D)
    if src16 is None:
        src16 = dtype != DTYPE_F32
    if src16:
        k, v = oracle.f32_to_f16(k), oracle.f32_to_f16(v)
    q = oracle.normal(seed + 2, B * Hq * D).reshape(B, Hq, D)
    c = Case(dtype, B, Hq, Hkv, D, P, ctx, tables, num_blocks, k, v, q)
    c.host = HostPool(dtype, num_blocks, P, Hkv, D)
    fill_garbage(c.host)
    return c


def qwen_c2(oracle, dtype=DTYPE_F16, B=16, T=2049, seed=2):
    """Config 2 (and 3 with dtype int4): GQA 32/8, D=128, P=16, uniform context,
    physical blocks from a seeded permutation."""
    return make_case(oracle, dtype, B, 32, 8, 128, 16, [T] * B, seed)


def continuous_c4(oracle, B=64, lo=128, hi=8192, seed=4, dtype=DTYPE_F16):
    """Config 4: per-sequence context ~ U[lo, hi], fragmented tables from a pool of
    1.2x the needed blocks."""
    ctx = oracle.uniform_int(seed, lo, hi, B)
    need = int(((ctx + 15) // 16).sum())
    return make_case(oracle, dtype, B, 32, 8, 128, 16, ctx, seed, num_blocks=int(np.ceil(1.2 * need)))


def chunk_evict_c5(oracle, lo=16384, hi=32256, B=8, chunk=512, seed=5, P=16):
    """Config 5 semantics: each sequence holds an int4 context of L0 ~ U[lo, hi] tokens,
    appends one `chunk`-token fp16 chunk through quantize-on-write, evicts its oldest
    floor(25%) logical blocks, and has its surviving blocks compacted into a fresh
    contiguous run of physical blocks.  Returns the plan (numpy, host side)."""
    L0 = oracle.uniform_int(seed, lo, hi, B)
    total = L0 + chunk
    nb = (total + P - 1) // P
    ev = (nb * 25) // 100
    surv = nb - ev
    # physical blocks: the live cache is a seeded permutation of the first sum(nb) blocks;
    # compaction destinations are a contiguous region after them
    used = int(nb.sum())
    perm = oracle.permutation(seed ^ 0xC5, used)
    tables = np.full((B, int(nb.max())), -1, np.int32)
    off = 0
    for b in range(B):
        tables[b, : nb[b]] = perm[off: off + nb[b]]
        off += nb[b]
    dst_base = used + np.concatenate([[0], np.cumsum(surv)[:-1]]).astype(np.int32)
    src = np.concatenate([tables[b, ev[b]: nb[b]] for b in range(B)]).astype(np.int32)
    dst = np.concatenate([dst_base[b] + np.arange(surv[b]) for b in range(B)]).astype(np.int32)
    new_tables = np.full((B, int(surv.max())), -1, np.int32)
    for b in range(B):
        new_tables[b, : surv[b]] = dst_base[b] + np.arange(surv[b])
    new_ctx = (total - ev * P).astype(np.int32)
    return dict(L0=L0.astype(np.int32), total=total.astype(np.int32), nb=nb, ev=ev, tables=tables,
                num_blocks=used + int(surv.sum()), src=src, dst=dst, new_tables=new_tables,
                new_ctx=new_ctx)
