"""Session-level paged KV cache over the GPU-resident handle API.

`CorePagedKVCache` keeps the method names, argument meaning and return conventions of
the reference's Python wrapper (Vspec-chat/python/runtime_core_bridge.py:479-549):
append one token's [H][D] keys/values, count a session's tokens, read them back as
[T][H][D] float32 arrays.  The token data lives in HBM and moves through the library's
append and row-gather kernels; page placement follows the reference allocator.  Unlike
the reference wrapper, a missing library raises instead of reporting `available=False`:
this package has no CPU path to fall back to.

The extra methods (`reuse_prefix`, `block_table`, `stats`, `device_pool`) expose what a
batched GPU decode step needs from the same cache.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import VspecPagedKV, VspecRocmError, VspecRocmPagedStats, VspecRocmStepItem, last_error, lib

_f32p = C.POINTER(C.c_float)


class HandlePool:
    """A handle's device pool in the shape `paged_decode` expects (`desc()`)."""

    def __init__(self, kv: VspecPagedKV):
        import torch

        self._kv = kv
        self.dtype, self.num_blocks, self.block_tokens = kv.dtype, kv.num_blocks, kv.block_tokens
        self.num_kv_heads, self.head_dim = kv.num_kv_heads, kv.head_dim
        # handle pools live on the device that was current when the handle was created
        self.device = torch.device("cuda", torch.cuda.current_device())

    def desc(self) -> VspecPagedKV:
        return self._kv


class CorePagedKVCache:
    def __init__(self, page_tokens: int, max_pages: int, num_heads: int, head_dim: int, session_id: int = 1) -> None:
        L = lib()
        self.handle = int(L.vspec_py_kv_cache_create(page_tokens, max_pages, num_heads, head_dim))
        if self.handle <= 0:
            raise VspecRocmError(f"vspec_py_kv_cache_create failed: {last_error()}")
        self.session_id = int(session_id)
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.page_tokens = int(page_tokens)

    @property
    def available(self) -> bool:
        return self.handle > 0

    def reset(self) -> None:
        if self.available:
            lib().vspec_py_kv_cache_reset(self.handle)

    def append(self, key_token, value_token, session_id: int | None = None) -> bool:
        if not self.available:
            return False
        k = np.ascontiguousarray(key_token, dtype=np.float32).reshape(-1)
        v = np.ascontiguousarray(value_token, dtype=np.float32).reshape(-1)
        if k.size != self.num_heads * self.head_dim or v.size != k.size:
            raise ValueError(f"append expects {self.num_heads}x{self.head_dim} floats per token")
        sid = self.session_id if session_id is None else int(session_id)
        return bool(lib().vspec_py_kv_cache_append(self.handle, sid, k.ctypes.data_as(_f32p),
                                                   v.ctypes.data_as(_f32p)))

    def session_tokens(self, session_id: int | None = None) -> int:
        if not self.available:
            return 0
        sid = self.session_id if session_id is None else int(session_id)
        return int(lib().vspec_py_kv_cache_session_tokens(self.handle, sid))

    def read_tokens(self, max_tokens: int | None = None, session_id: int | None = None):
        if not self.available:
            return None, None
        sid = self.session_id if session_id is None else int(session_id)
        n = self.session_tokens(sid)
        if max_tokens is not None:
            n = min(n, int(max_tokens))
        shape = (self.num_heads, self.head_dim)
        if n <= 0:
            empty = np.empty((0, *shape), np.float32)
            return empty, empty.copy()
        keys = np.empty((n, *shape), np.float32)
        values = np.empty((n, *shape), np.float32)
        got = int(lib().vspec_py_kv_cache_read(self.handle, sid, keys.ctypes.data_as(_f32p),
                                               values.ctypes.data_as(_f32p), n))
        if got <= 0:
            return None, None
        return keys[:got], values[:got]

    # ---- beyond the reference wrapper: the allocator and the device pool ----
    def _meta(self):
        return lib().vspec_py_kv_cache_meta(self.handle)

    def open_session(self, session_id: int) -> bool:
        return bool(lib().vspec_rocm_paged_open_session(self._meta(), int(session_id)))

    def close_session(self, session_id: int) -> bool:
        return bool(lib().vspec_rocm_paged_close_session(self._meta(), int(session_id)))

    def reuse_prefix(self, target_session: int, source_session: int, max_tokens: int) -> bool:
        return bool(lib().vspec_rocm_paged_reuse_prefix(self._meta(), int(target_session), int(source_session),
                                                         int(max_tokens)))

    def stats(self) -> dict:
        st = VspecRocmPagedStats()
        lib().vspec_rocm_paged_stats(self._meta(), C.byref(st))
        return {name: getattr(st, name) for name, _ in st._fields_}

    def block_table(self, session_id: int, max_blocks: int):
        """(int32 [max_blocks] table padded with -1, context length) or None when a
        shared, partly filled page sits in the middle of the session."""
        tab = np.full(max_blocks, -1, np.int32)
        ctx = C.c_uint32()
        ok = lib().vspec_rocm_paged_block_table(self._meta(), int(session_id),
                                                tab.ctypes.data_as(C.POINTER(C.c_int32)), max_blocks,
                                                C.byref(ctx))
        return (tab, int(ctx.value)) if ok else None

    def block_layout(self, session_id: int, max_blocks: int):
        """Any session as (int32 table [max_blocks] padded with -1, int32 used counts
        [max_blocks], span, tokens): the decode inputs with block_used, which also cover
        shared, partly filled pages in the middle of a session."""
        tab = np.full(max_blocks, -1, np.int32)
        used = np.zeros(max_blocks, np.int32)
        span, tokens = C.c_uint32(), C.c_uint32()
        p32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))
        ok = lib().vspec_rocm_paged_block_layout(self._meta(), int(session_id), p32(tab), p32(used), max_blocks,
                                                 C.byref(span), C.byref(tokens))
        if not ok:
            raise VspecRocmError(f"block_layout: unknown session {session_id} or more than {max_blocks} pages")
        return tab, used, int(span.value), int(tokens.value)

    def device_pool(self) -> HandlePool:
        p = lib().vspec_py_kv_cache_pool(self.handle)
        if not p:
            raise VspecRocmError("handle has no device pool")
        return HandlePool(p.contents)

    def close(self) -> None:
        if self.handle > 0:
            lib().vspec_py_kv_cache_destroy(self.handle)
            self.handle = 0

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


def plan_step(meta, items, max_blocks: int, max_tokens: int | None = None, with_used: bool = False):
    """vspec_rocm_paged_plan_step over a VspecRocmPagedMeta* (e.g. CorePagedKVCache._meta()).

    items: sequence of (request_id, phase, token_quota, prompt_cursor) or VspecRocmStepItem.
    Returns dict(block_tables [n][max_blocks], ctx_lens [n], start_pos [n], token_item [t],
    token_pos [t]) as int32 numpy arrays, positions in table-slot space; with_used adds
    block_used [n][max_blocks] (ctx_lens then hold spans) and accepts sessions with partly
    filled middle pages.  Raises VspecRocmError when the step cannot be planned."""
    n = len(items)
    arr = (VspecRocmStepItem * max(n, 1))()
    for i, it in enumerate(items):
        if isinstance(it, VspecRocmStepItem):
            arr[i] = it
        else:
            arr[i] = VspecRocmStepItem(*[int(x) for x in it])
    total = sum(int(arr[i].token_quota) for i in range(n))
    cap = total if max_tokens is None else int(max_tokens)
    tables = np.full((max(n, 1), max_blocks), -1, np.int32)
    ctx = np.zeros(max(n, 1), np.int32)
    start = np.zeros(max(n, 1), np.int32)
    titem = np.zeros(max(cap, 1), np.int32)
    tpos = np.zeros(max(cap, 1), np.int32)
    used = np.zeros((max(n, 1), max_blocks), np.int32) if with_used else None
    got = C.c_size_t()
    p32 = lambda a: None if a is None else a.ctypes.data_as(C.POINTER(C.c_int32))
    ok = lib().vspec_rocm_paged_plan_step(meta, arr, n, p32(tables), p32(used), max_blocks, p32(ctx), p32(start),
                                          p32(titem), p32(tpos), cap, C.byref(got))
    if not ok:
        raise VspecRocmError("plan_step failed (pool exhausted, eviction of a batch member, repeated request, "
                             "shared partly filled page, or outputs too small)")
    t = int(got.value)
    out = dict(block_tables=tables[:n], ctx_lens=ctx[:n], start_pos=start[:n], token_item=titem[:t],
               token_pos=tpos[:t])
    if with_used:
        out["block_used"] = used[:n]
    return out


class StepPlanner:
    """vspec_rocm_paged_plan_step_update over host tables kept between steps.

    The planner owns block_tables [max_items][max_blocks] (and block_used with with_used),
    ctx_lens, start_pos and the packed-token map; each step() updates only the row entries
    that changed since the previous step and returns views of the first n rows, with the
    same keys as plan_step().  The views are overwritten by the next step."""

    def __init__(self, meta, max_items: int, max_blocks: int, max_tokens: int, with_used: bool = False):
        self.meta, self.max_items, self.max_blocks, self.max_tokens = meta, max_items, max_blocks, max_tokens
        self.tables = np.full((max(max_items, 1), max_blocks), -1, np.int32)
        self.used = np.zeros((max(max_items, 1), max_blocks), np.int32) if with_used else None
        self.ctx = np.zeros(max(max_items, 1), np.int32)
        self.start = np.zeros(max(max_items, 1), np.int32)
        self.titem = np.zeros(max(max_tokens, 1), np.int32)
        self.tpos = np.zeros(max(max_tokens, 1), np.int32)
        self._items = (VspecRocmStepItem * max(max_items, 1))()
        p32 = lambda a: None if a is None else a.ctypes.data_as(C.POINTER(C.c_int32))
        self._p = [p32(a) for a in (self.tables, self.used, self.ctx, self.start, self.titem, self.tpos)]
        self._got = C.c_size_t()

    def step(self, items):
        n = len(items)
        if n > self.max_items:
            raise VspecRocmError(f"step of {n} items exceeds the planner's {self.max_items}")
        for i, it in enumerate(items):
            self._items[i] = it if isinstance(it, VspecRocmStepItem) else VspecRocmStepItem(*[int(x) for x in it])
        pt, pu, pc, ps, pi, pp = self._p
        ok = lib().vspec_rocm_paged_plan_step_update(self.meta, self._items, n, pt, pu, self.max_blocks, pc, ps, pi,
                                                     pp, self.max_tokens, C.byref(self._got))
        if not ok:
            raise VspecRocmError("plan_step_update failed (pool exhausted, eviction of a batch member, repeated "
                                 "request, shared partly filled page, or outputs too small)")
        t = int(self._got.value)
        out = dict(block_tables=self.tables[:n], ctx_lens=self.ctx[:n], start_pos=self.start[:n],
                   token_item=self.titem[:t], token_pos=self.tpos[:t])
        if self.used is not None:
            out["block_used"] = self.used[:n]
        return out

