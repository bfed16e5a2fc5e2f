"""ctypes binding of the MI355X paged KV-cache C-ABI (include/vspec_rocm.h).

This mirrors how the reference reaches its paged cache from Python
(Vspec-chat/python/runtime_core_bridge.py:43-54, 479-549: ctypes prototypes over a
shared library).  torch is used only to own device memory and to name the
stream; every computation runs in lib/libvspec_rocm.so.  There is no CPU
fallback: a missing library raises at import of the first call.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parents[2]
LIB_PATH = Path(os.environ.get("VSPEC_ROCM_LIB", PKG_ROOT / "lib" / "libvspec_rocm.so"))

KV_F32, KV_F16, KV_INT4 = 0, 1, 2
NUMERICS_PLAIN, NUMERICS_3BIT = 0, 1
GATHER_RAW, GATHER_F32 = 0, 1
KCTX_FLAG_PAGED = 1

_vp = C.c_void_p
_i32p = C.c_void_p


class VspecPagedKV(C.Structure):
    _fields_ = [
        ("dtype", C.c_int32),
        ("num_blocks", C.c_uint32),
        ("block_tokens", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("k_data", _vp),
        ("v_data", _vp),
        ("k_scales", _vp),
        ("v_scales", _vp),
        ("k_flags", _vp),
    ]


class VspecPagedAttnDesc(C.Structure):
    _fields_ = [
        ("kv", VspecPagedKV),
        ("batch", C.c_uint32),
        ("num_q_heads", C.c_uint32),
        ("block_tables", _vp),
        ("max_blocks_per_seq", C.c_uint32),
        ("ctx_lens", _vp),
        ("max_ctx_len", C.c_uint32),
        ("q", _vp),
        ("out", _vp),
        ("scale", C.c_float),
        ("numerics", C.c_int32),
        ("clamp_alpha", C.c_float),
        ("partition_tokens", C.c_uint32),
        ("workspace", _vp),
        ("workspace_bytes", C.c_size_t),
        ("stream", _vp),
        ("block_used", _vp),
        ("min_ctx_len", C.c_uint32),
    ]


class VspecQuantMeta(C.Structure):
    _fields_ = [
        ("schema_version", C.c_uint),
        ("type", C.c_int),
        ("scales", _vp),
        ("scale_count", C.c_size_t),
        ("special_format", C.c_int),
        ("special_data", _vp),
    ]


class VspecExecConfig(C.Structure):
    _fields_ = [("m", C.c_size_t), ("n", C.c_size_t), ("k", C.c_size_t), ("flags", C.c_size_t)]


class VspecKernelContext(C.Structure):
    _fields_ = [
        ("input", _vp),
        ("weight", _vp),
        ("output", _vp),
        ("qmeta", VspecQuantMeta),
        ("config", VspecExecConfig),
    ]


_LAUNCH = C.CFUNCTYPE(None, C.POINTER(VspecKernelContext))


class VspecBackend(C.Structure):
    _fields_ = [("name", C.c_char_p), ("launch_linear", _LAUNCH), ("launch_attention", _LAUNCH)]


class VspecKVCache(C.Structure):
    _fields_ = [
        ("key", _vp),
        ("value", _vp),
        ("max_tokens", C.c_size_t),
        ("num_heads", C.c_size_t),
        ("head_dim", C.c_size_t),
        ("current_tokens", C.c_size_t),
        ("int3_compressed", C.c_int),
        ("key_int3", _vp),
        ("value_int3", _vp),
        ("key_scales", _vp),
        ("value_scales", _vp),
        ("block_size", C.c_size_t),
        ("blocks_per_head", C.c_size_t),
        ("packed_head_bytes", C.c_size_t),
        ("scratch_key_head", _vp),
        ("scratch_value_head", _vp),
        ("owns_int3_buffers", C.c_int),
    ]


class VspecRocmPagedStats(C.Structure):
    """Same layout as the reference's VspecKVPagedStats (kv_paged_cache.h:11-18)."""

    _fields_ = [
        ("page_alloc_count", C.c_uint64),
        ("page_reuse_count", C.c_uint64),
        ("evict_session_count", C.c_uint64),
        ("append_token_count", C.c_uint64),
        ("free_pages", C.c_size_t),
        ("active_sessions", C.c_size_t),
    ]


class VspecRocmStepItem(C.Structure):
    """Same layout as the reference's VspecContinuousBatchItem (continuous_batch.h:15-20)."""

    _fields_ = [
        ("request_id", C.c_uint64),
        ("phase", C.c_uint32),
        ("token_quota", C.c_size_t),
        ("prompt_cursor", C.c_size_t),
    ]


_u32p = C.POINTER(C.c_uint32)
_i32p_ = C.POINTER(C.c_int32)
_f32p = C.POINTER(C.c_float)

# Every symbol include/*.h declares, with its ctypes signature.
SIGNATURES = {
    "vspec_rocm_kv_pool_bytes": (C.c_size_t, [C.c_int32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    "vspec_rocm_kv_pool_create": (C.c_int, [C.POINTER(VspecPagedKV), C.c_int32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    "vspec_rocm_kv_pool_destroy": (None, [C.POINTER(VspecPagedKV)]),
    "vspec_rocm_kv_append": (C.c_int, [C.POINTER(VspecPagedKV), C.c_uint32, _vp, C.c_uint32, _vp, C.c_uint32, _vp, _vp, C.c_int32, _vp]),
    "vspec_rocm_kv_append_rope": (C.c_int, [C.POINTER(VspecPagedKV), C.c_uint32, _vp, C.c_uint32, _vp, C.c_uint32, _vp,
                                            _vp, C.c_int32, _vp, _vp, C.c_uint32, C.c_uint32, _vp, _vp, C.c_uint32,
                                            _vp]),
    "vspec_rocm_kv_gather": (C.c_int, [C.POINTER(VspecPagedKV), C.c_uint32, _vp, C.c_uint32, _vp, C.c_uint32, _vp, C.c_int32, _vp, _vp, _vp, _vp, _vp]),
    "vspec_rocm_kv_compact": (C.c_int, [C.POINTER(VspecPagedKV), C.c_uint32, _vp, _vp, _vp]),
    "vspec_rocm_paged_decode_workspace_bytes": (C.c_size_t, [C.POINTER(VspecPagedAttnDesc)]),
    "vspec_rocm_paged_decode_attention": (C.c_int, [C.POINTER(VspecPagedAttnDesc)]),
    "vspec_rocm_paged_decode_step": (C.c_int, [C.POINTER(VspecPagedAttnDesc), _vp, _vp, C.c_int32]),
    "vspec_rocm_paged_decode_step_noalloc": (C.c_int, [C.POINTER(VspecPagedAttnDesc), _vp, _vp, C.c_int32]),
    "vspec_rocm_sync": (C.c_int, [_vp]),
    "vspec_rocm_last_error": (C.c_char_p, []),
    "vspec_rocm_device_count": (C.c_int, []),
    "vspec_rocm_backend_available": (C.c_int, []),
    "vspec_rocm_release_cache_mirror": (C.c_int, [_vp]),
    "vspec_rocm_cache_mirror_append_only": (C.c_int, [C.c_int]),
    "vspec_make_rocm_backend": (VspecBackend, []),
    # include/vspec_rocm_paged.h
    "vspec_rocm_paged_meta_create": (_vp, [C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t]),
    "vspec_rocm_paged_meta_destroy": (None, [_vp]),
    "vspec_rocm_paged_meta_reset": (None, [_vp]),
    "vspec_rocm_paged_open_session": (C.c_int, [_vp, C.c_uint64]),
    "vspec_rocm_paged_close_session": (C.c_int, [_vp, C.c_uint64]),
    "vspec_rocm_paged_reuse_prefix": (C.c_int, [_vp, C.c_uint64, C.c_uint64, C.c_size_t]),
    "vspec_rocm_paged_reserve": (C.c_int, [_vp, C.c_uint64, _u32p, _u32p]),
    "vspec_rocm_paged_locate": (C.c_int, [_vp, C.c_uint64, C.c_size_t, _u32p, _u32p]),
    "vspec_rocm_paged_session_tokens": (C.c_size_t, [_vp, C.c_uint64]),
    "vspec_rocm_paged_stats": (None, [_vp, C.POINTER(VspecRocmPagedStats)]),
    "vspec_rocm_paged_session_pages": (C.c_size_t, [_vp, C.c_uint64, _u32p, C.c_size_t]),
    "vspec_rocm_paged_page_info": (C.c_int, [_vp, C.c_size_t, _u32p, _u32p, _u32p]),
    "vspec_rocm_paged_block_table": (C.c_int, [_vp, C.c_uint64, _i32p_, C.c_size_t, _u32p]),
    "vspec_rocm_paged_block_layout": (C.c_int, [_vp, C.c_uint64, _i32p_, _i32p_, C.c_size_t, _u32p, _u32p]),
    "vspec_py_kv_cache_create": (C.c_int, [C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t]),
    "vspec_py_kv_cache_destroy": (None, [C.c_int]),
    "vspec_py_kv_cache_reset": (C.c_int, [C.c_int]),
    "vspec_py_kv_cache_append": (C.c_int, [C.c_int, C.c_uint64, _f32p, _f32p]),
    "vspec_py_kv_cache_session_tokens": (C.c_size_t, [C.c_int, C.c_uint64]),
    "vspec_py_kv_cache_read": (C.c_size_t, [C.c_int, C.c_uint64, _f32p, _f32p, C.c_size_t]),
    "vspec_py_kv_cache_meta": (_vp, [C.c_int]),
    "vspec_py_kv_cache_pool": (C.POINTER(VspecPagedKV), [C.c_int]),
    "vspec_rocm_kv_gather_rows": (C.c_int, [C.POINTER(VspecPagedKV), C.c_uint32, _vp, _vp, _vp, _vp, _vp]),
    "vspec_rocm_paged_plan_step": (C.c_int, [_vp, C.POINTER(VspecRocmStepItem), C.c_size_t, _i32p_, _i32p_, C.c_size_t,
                                             _i32p_, _i32p_, _i32p_, _i32p_, C.c_size_t, C.POINTER(C.c_size_t)]),
    "vspec_rocm_paged_plan_step_update": (C.c_int, [_vp, C.POINTER(VspecRocmStepItem), C.c_size_t, _i32p_, _i32p_,
                                                    C.c_size_t, _i32p_, _i32p_, _i32p_, _i32p_, C.c_size_t,
                                                    C.POINTER(C.c_size_t)]),
    "vspec_rocm_kv_append_tokens": (C.c_int, [C.POINTER(VspecPagedKV), C.c_uint32, _vp, _vp, _vp, C.c_uint32,
                                              C.c_uint32, _vp, _vp, C.c_int32, _vp]),
    "vspec_rocm_release_retired_workspaces": (C.c_int, []),
}

_LIB = None


class VspecRocmError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load lib/libvspec_rocm.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise VspecRocmError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (make -C vspec-engine_amd)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _LIB = L
    return _LIB


def last_error() -> str:
    e = lib().vspec_rocm_last_error()
    return e.decode() if e else ""


def _check(ok: int, what: str):
    if not ok:
        raise VspecRocmError(f"{what} failed: {last_error()}")


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream=None):
    """The hipStream_t handle for the C-ABI: torch's current stream, a torch stream, or
    a raw handle."""
    import torch

    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def _foreign_stream(stream):
    """The launch stream as a torch stream object when it is not torch's current stream
    (temporaries made on the current stream must then be recorded on it), else None."""
    import torch

    if stream is None:
        return None
    s = stream if isinstance(stream, torch.cuda.Stream) else torch.cuda.ExternalStream(int(stream))
    return None if s.cuda_stream == torch.cuda.current_stream().cuda_stream else s


def _hold(stream, *tensors):
    """Keep the caching allocator from handing the memory of these temporaries (made on
    torch's current stream) to other work before the launch on `stream` has read them."""
    s = _foreign_stream(stream)
    if s is None:
        return
    for t in tensors:
        if t is not None and getattr(t, "is_cuda", False):
            t.record_stream(s)


def _i32(t, device):
    """An index tensor as contiguous int32 on the pool's device (the C-ABI reads int32)."""
    import torch

    out = torch.as_tensor(t).to(device=device, dtype=torch.int32).contiguous()
    if out.device != torch.device(device):
        raise VspecRocmError(f"index tensor on {out.device}, the pool is on {device}")
    return out


class PagedPool:
    """A paged KV pool in HBM, owned by torch tensors, in the layout of
    include/vspec_rocm.h: K/V [num_blocks][H][P][D] (f32/f16) or codes
    [num_blocks][H][P][D/2] plus fp16-bit scales [num_blocks][H][P][D/32] (int4), and for
    int4 the clamp flags [num_blocks][H][P/16] (flags=False: none, the decode screens keys)."""

    def __init__(self, dtype: int, num_blocks: int, block_tokens: int, num_kv_heads: int, head_dim: int, device="cuda",
                 flags=True):
        import torch

        self.dtype, self.num_blocks, self.block_tokens = dtype, num_blocks, block_tokens
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        rows = num_blocks * num_kv_heads * block_tokens
        if dtype == KV_F32:
            shape, td = (rows, head_dim), torch.float32
        elif dtype == KV_F16:
            shape, td = (rows, head_dim), torch.float16
        elif dtype == KV_INT4:
            shape, td = (rows, head_dim // 2), torch.uint8
        else:
            raise ValueError("dtype")
        self.k = torch.zeros(shape, dtype=td, device=device)
        self.v = torch.zeros(shape, dtype=td, device=device)
        if dtype == KV_INT4:
            self.ks = torch.zeros((rows, head_dim // 32), dtype=torch.int16, device=device)
            self.vs = torch.zeros((rows, head_dim // 32), dtype=torch.int16, device=device)
            self.kf = (torch.zeros((num_blocks * num_kv_heads * (block_tokens // 16),), dtype=torch.int32, device=device)
                       if flags else None)
        else:
            self.ks = self.vs = self.kf = None

    @property
    def device(self):
        return self.k.device

    def desc(self) -> VspecPagedKV:
        d = VspecPagedKV()
        d.dtype, d.num_blocks, d.block_tokens = self.dtype, self.num_blocks, self.block_tokens
        d.num_kv_heads, d.head_dim = self.num_kv_heads, self.head_dim
        d.k_data, d.v_data = self.k.data_ptr(), self.v.data_ptr()
        d.k_scales, d.v_scales = _ptr(self.ks), _ptr(self.vs)
        d.k_flags = _ptr(self.kf)
        return d


def kv_append(pool: PagedPool, block_tables, start_pos, k_new, v_new, stream=None):
    """vspec_rocm_kv_append: k_new/v_new [B][n_new][H][D] (float32 or float16, device)."""
    import torch

    assert k_new.is_contiguous() and v_new.is_contiguous() and k_new.shape == v_new.shape
    B, n_new = k_new.shape[0], k_new.shape[1]
    src = KV_F32 if k_new.dtype == torch.float32 else KV_F16
    assert k_new.dtype in (torch.float32, torch.float16)
    dev = pool.device
    bt = _i32(block_tables, dev)
    sp = _i32(start_pos, dev)
    d = pool.desc()
    _check(lib().vspec_rocm_kv_append(C.byref(d), B, bt.data_ptr(), bt.shape[1], sp.data_ptr(), n_new,
                                      k_new.data_ptr(), v_new.data_ptr(), src, _stream(stream)), "kv_append")
    _hold(stream, bt, sp)


def kv_append_rope(pool, block_tables, start_pos, k_new, v_new, rope_cos, rope_sin, rope_dim=None, q=None,
                   stream=None):
    """vspec_rocm_kv_append_rope: kv_append with K (and q [B][n_new][Hq][D] fp32, when
    given) rotated by rows start_pos + i of rope_cos / rope_sin [max_pos][rope_dim/2]
    (fp32, device).  Returns the rotated q (or None)."""
    import torch

    B, n_new = k_new.shape[0], k_new.shape[1]
    assert k_new.is_contiguous() and v_new.is_contiguous()
    assert rope_cos.dtype == torch.float32 and rope_cos.is_contiguous() and rope_sin.is_contiguous()
    src = KV_F16 if k_new.dtype == torch.float16 else KV_F32
    rope_dim = int(rope_dim if rope_dim is not None else 2 * rope_cos.shape[1])
    dev = pool.device
    bt = _i32(block_tables, dev)
    sp = _i32(start_pos, dev)
    q_out = None
    qin = qout = None
    hq = 0
    if q is not None:
        assert q.dtype == torch.float32 and q.is_contiguous()
        q_out = torch.empty_like(q)
        qin, qout, hq = q.data_ptr(), q_out.data_ptr(), q.shape[2]
    kv = pool.desc()
    _check(lib().vspec_rocm_kv_append_rope(C.byref(kv), B, bt.data_ptr(), bt.shape[1], sp.data_ptr(), n_new,
                                           k_new.data_ptr(), v_new.data_ptr(), src, rope_cos.data_ptr(),
                                           rope_sin.data_ptr(), rope_dim, rope_cos.shape[0], qin, qout, hq,
                                           _stream(stream)), "kv_append_rope")
    _hold(stream, bt, sp, q_out)
    return q_out


def kv_append_tokens(pool, token_item, token_pos, block_tables, k_new, v_new, stream=None):
    """vspec_rocm_kv_append_tokens: packed new tokens k_new/v_new [n][H][D] (float32 or
    float16, device); token t goes to position token_pos[t] of block-table row
    token_item[t]."""
    import torch

    n = int(token_item.numel())
    if n == 0:
        return
    assert k_new.is_contiguous() and v_new.is_contiguous() and k_new.shape[0] == n
    assert int(token_pos.numel()) == n
    src = KV_F16 if k_new.dtype == torch.float16 else KV_F32
    dev = pool.device
    ti = _i32(token_item, dev)
    tp = _i32(token_pos, dev)
    bt = _i32(block_tables, dev)
    kv = pool.desc()
    _check(lib().vspec_rocm_kv_append_tokens(C.byref(kv), n, ti.data_ptr(), tp.data_ptr(), bt.data_ptr(),
                                             bt.shape[0], bt.shape[1], k_new.data_ptr(), v_new.data_ptr(), src,
                                             _stream(stream)), "kv_append_tokens")
    _hold(stream, ti, tp, bt)


def kv_gather(pool: PagedPool, block_tables, ctx_lens, out_mode=GATHER_RAW, max_ctx_len=None, stream=None):
    """vspec_rocm_kv_gather -> (k, v, k_scales, v_scales) concatenated [T][H][D]."""
    import torch

    dev = pool.device
    bt = _i32(block_tables, dev)
    cl = _i32(ctx_lens, dev)
    cl_host = cl.cpu()
    offs = torch.zeros(len(cl_host), dtype=torch.int64)
    if len(cl_host) > 1:
        offs[1:] = torch.cumsum(cl_host[:-1].to(torch.int64), 0)
    T = int(cl_host.sum())
    H, D = pool.num_kv_heads, pool.head_dim
    ks = vs = None
    if out_mode == GATHER_F32:
        ok = torch.zeros((T, H, D), dtype=torch.float32, device=dev)
        ov = torch.zeros_like(ok)
    elif pool.dtype == KV_INT4:
        ok = torch.zeros((T, H, D // 2), dtype=torch.uint8, device=dev)
        ov = torch.zeros_like(ok)
        ks = torch.zeros((T, H, D // 32), dtype=torch.int16, device=dev)
        vs = torch.zeros_like(ks)
    else:
        ok = torch.zeros((T, H, D), dtype=pool.k.dtype, device=dev)
        ov = torch.zeros_like(ok)
    offs_d = offs.to(dev)
    mc = int(cl_host.max()) if max_ctx_len is None and len(cl_host) else (max_ctx_len or 0)
    d = pool.desc()
    _check(lib().vspec_rocm_kv_gather(C.byref(d), len(cl_host), bt.data_ptr(), bt.shape[1], cl.data_ptr(), mc,
                                      offs_d.data_ptr(), out_mode, ok.data_ptr(), ov.data_ptr(), _ptr(ks), _ptr(vs),
                                      _stream(stream)), "kv_gather")
    _hold(stream, bt, cl, offs_d, ok, ov, ks, vs)
    return ok, ov, ks, vs


def kv_compact(pool: PagedPool, src_blocks, dst_blocks, stream=None):
    import torch

    s = _i32(src_blocks, pool.device)
    t = _i32(dst_blocks, pool.device)
    d = pool.desc()
    _check(lib().vspec_rocm_kv_compact(C.byref(d), len(s), s.data_ptr(), t.data_ptr(), _stream(stream)), "kv_compact")
    _hold(stream, s, t)


def make_decode_desc(pool: PagedPool, block_tables, ctx_lens, q, out, max_ctx_len, numerics=NUMERICS_PLAIN,
                     scale=0.0, partition_tokens=0, workspace=None, stream=None,
                     block_used=None, min_ctx_len=0) -> VspecPagedAttnDesc:
    B, Hq, D = q.shape
    d = VspecPagedAttnDesc()
    d.kv = pool.desc()
    d.batch, d.num_q_heads = B, Hq
    d.block_tables, d.max_blocks_per_seq = block_tables.data_ptr(), block_tables.shape[1]
    d.ctx_lens, d.max_ctx_len = ctx_lens.data_ptr(), max_ctx_len
    d.q, d.out = q.data_ptr(), out.data_ptr()
    d.scale, d.numerics, d.clamp_alpha = scale, numerics, 0.0
    d.partition_tokens = partition_tokens
    if workspace is not None:
        d.workspace, d.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    d.stream = _stream(stream)
    d.block_used = _ptr(block_used)
    d.min_ctx_len = min_ctx_len
    return d


def decode_workspace_bytes(desc: VspecPagedAttnDesc) -> int:
    return lib().vspec_rocm_paged_decode_workspace_bytes(C.byref(desc))


def paged_decode(pool: PagedPool, block_tables, ctx_lens, q, max_ctx_len=None, numerics=NUMERICS_PLAIN,
                 scale=0.0, partition_tokens=0, out=None, workspace=None, stream=None, block_used=None,
                 min_ctx_len=0):
    """vspec_rocm_paged_decode_attention: q [B][Hq][D] float32 (device) -> out.  With
    block_used ([B][max_blocks], tokens per table entry) ctx_lens holds the spans;
    min_ctx_len: the host's lower bound on ctx_lens (0: none)."""
    import torch

    assert q.dtype == torch.float32 and q.is_contiguous()
    bt = _i32(block_tables, pool.device)
    cl = _i32(ctx_lens, pool.device)
    bu = None if block_used is None else _i32(block_used, pool.device)
    assert bu is None or bu.shape == bt.shape
    if max_ctx_len is None:
        max_ctx_len = int(cl.max().item()) if cl.numel() else 0
    if out is None:
        out = torch.empty_like(q)
    d = make_decode_desc(pool, bt, cl, q, out, max_ctx_len, numerics, scale, partition_tokens, workspace, stream, bu,
                         min_ctx_len)
    _check(lib().vspec_rocm_paged_decode_attention(C.byref(d)), "paged_decode_attention")
    _hold(stream, bt, cl, bu, out)
    return out


def paged_decode_step(pool: PagedPool, block_tables, ctx_lens, q, k_new, v_new, max_ctx_len=None,
                      numerics=NUMERICS_PLAIN, scale=0.0, partition_tokens=0, out=None, workspace=None,
                      stream=None, block_used=None, min_ctx_len=0):
    """vspec_rocm_paged_decode_step: append k_new / v_new [B][Hkv][D] (float32 or float16,
    device) at position ctx_lens[b] - 1, then decode q [B][Hq][D] float32 -> out.
    min_ctx_len: the host's lower bound on ctx_lens (0: none)."""
    import torch

    assert q.dtype == torch.float32 and q.is_contiguous()
    assert k_new.is_contiguous() and v_new.is_contiguous() and k_new.shape == v_new.shape
    assert k_new.dtype in (torch.float32, torch.float16) and v_new.dtype == k_new.dtype
    src = KV_F32 if k_new.dtype == torch.float32 else KV_F16
    bt = _i32(block_tables, pool.device)
    cl = _i32(ctx_lens, pool.device)
    bu = None if block_used is None else _i32(block_used, pool.device)
    assert bu is None or bu.shape == bt.shape
    if max_ctx_len is None:
        max_ctx_len = int(cl.max().item()) if cl.numel() else 0
    if out is None:
        out = torch.empty_like(q)
    d = make_decode_desc(pool, bt, cl, q, out, max_ctx_len, numerics, scale, partition_tokens, workspace, stream, bu,
                         min_ctx_len)
    _check(lib().vspec_rocm_paged_decode_step(C.byref(d), k_new.data_ptr(), v_new.data_ptr(), src),
           "paged_decode_step")
    _hold(stream, bt, cl, bu, out)
    return out


def backend() -> VspecBackend:
    """vspec_make_rocm_backend(): the registry entry a reference build would install."""
    return lib().vspec_make_rocm_backend()
