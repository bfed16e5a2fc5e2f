"""ctypes access to the CPU checker libraries (test infrastructure only).

``Oracle`` wraps ``oracle/liboracle.so`` (the C restatement of the reference
path, vspec_oracle.c).  ``Reference`` wraps ``oracle/_ref/libvspec_ref.so``,
the reference's own hot-path C sources compiled in place by oracle/Makefile.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg may
import this module; it is the checker, never the product.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libvspec_ref.so"

_f32p = C.POINTER(C.c_float)
_u16p = C.POINTER(C.c_uint16)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)
_u32p = C.POINTER(C.c_uint32)
_u64p = C.POINTER(C.c_uint64)
_vp = C.c_void_p
_sz = C.c_size_t

DTYPE_F32, DTYPE_F16, DTYPE_INT4 = 0, 1, 2


def ptr(a: np.ndarray, t=None):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t) if t is not None else C.c_void_p(a.ctypes.data)


class VoPagedKV(C.Structure):
    _fields_ = [
        ("dtype", C.c_int),
        ("num_blocks", C.c_uint32),
        ("block_tokens", C.c_uint32),
        ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("k_data", _vp),
        ("v_data", _vp),
        ("k_scales", _u16p),
        ("v_scales", _u16p),
    ]


class HostPool:
    """A paged pool in host memory in the build's HBM layout (numpy-backed)."""

    def __init__(self, dtype, num_blocks, block_tokens, num_kv_heads, head_dim):
        self.dtype = dtype
        self.num_blocks, self.block_tokens = num_blocks, block_tokens
        self.num_kv_heads, self.head_dim = num_kv_heads, head_dim
        rows = num_blocks * num_kv_heads * block_tokens
        if dtype == DTYPE_F32:
            self.k = np.zeros((rows, head_dim), np.float32)
            self.v = np.zeros((rows, head_dim), np.float32)
            self.ks = self.vs = None
        elif dtype == DTYPE_F16:
            self.k = np.zeros((rows, head_dim), np.uint16)
            self.v = np.zeros((rows, head_dim), np.uint16)
            self.ks = self.vs = None
        else:
            self.k = np.zeros((rows, head_dim // 2), np.uint8)
            self.v = np.zeros((rows, head_dim // 2), np.uint8)
            self.ks = np.zeros((rows, head_dim // 32), np.uint16)
            self.vs = np.zeros((rows, head_dim // 32), np.uint16)

    def desc(self) -> VoPagedKV:
        d = VoPagedKV()
        d.dtype = self.dtype
        d.num_blocks, d.block_tokens = self.num_blocks, self.block_tokens
        d.num_kv_heads, d.head_dim = self.num_kv_heads, self.head_dim
        d.k_data = self.k.ctypes.data
        d.v_data = self.v.ctypes.data
        d.k_scales = ptr(self.ks, _u16p) if self.ks is not None else None
        d.v_scales = ptr(self.vs, _u16p) if self.vs is not None else None
        return d


class Oracle:
    def __init__(self, path: Path = ORACLE_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (run make -C oracle)")
        L = self.lib = C.CDLL(str(path))
        sig = {
            "vo_half_to_float": (C.c_float, [C.c_uint16]),
            "vo_float_to_half": (C.c_uint16, [C.c_float]),
            "vo_f16_to_f32": (None, [_u16p, _f32p, _sz]),
            "vo_f32_to_f16": (None, [_f32p, _u16p, _sz]),
            "vo_fill_normal": (None, [C.c_uint64, _f32p, _sz]),
            "vo_permutation": (None, [C.c_uint64, _i32p, _sz]),
            "vo_uniform_int": (None, [C.c_uint64, C.c_int32, C.c_int32, _i32p, _sz]),
            "vo_quant_packed_bytes": (_sz, [_sz, C.c_uint8]),
            "vo_quant_clip_signed": (C.c_int8, [C.c_int8, C.c_uint8]),
            "vo_quant_pack_signed": (None, [_i8p, _sz, C.c_uint8, _u8p]),
            "vo_quant_get_signed": (C.c_int8, [_u8p, _sz, C.c_uint8]),
            "vo_quant_unpack_signed": (None, [_u8p, _sz, C.c_uint8, _i8p]),
            "vo_int4_packed_bytes": (_sz, [_sz]),
            "vo_int4_pack": (None, [_i8p, _sz, _u8p]),
            "vo_int4_get": (C.c_int8, [_u8p, _sz]),
            "vo_percentile_abs_block": (C.c_float, [_f32p, _sz, C.c_float]),
            "vo_int3_quantize_head": (None, [_f32p, _sz, _sz, _u8p, _f32p]),
            "vo_int3_dequantize_head": (None, [_u8p, _f32p, _sz, _sz, _f32p]),
            "vo_int4_quantize_head": (None, [_f32p, _sz, _u8p, _u16p]),
            "vo_int4_dequantize_head": (None, [_u8p, _u16p, _sz, _f32p]),
            "vo_dynamic_clamp_std": (None, [_f32p, _sz, C.c_float, _f32p]),
            "vo_noise_reduce_vector": (None, [C.c_int, _f32p, _sz, _f32p]),
            "vo_accum_dot_f32": (C.c_float, [C.c_int, _sz, _f32p, _f32p, _sz]),
            "vo_qk_score": (C.c_float, [C.c_int, _sz, _f32p, _f32p, _sz, C.c_float]),
            "vo_softmax_apply": (None, [C.c_int, _f32p, _sz, _f32p]),
            "vo_attention_head": (None, [C.c_int, _sz, _f32p, _f32p, _sz, _f32p, _sz, _sz, _sz, _f32p]),
            "vo_attention_ref_single_query": (None, [C.c_int, _sz, _f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p]),
            "vo_paged_append": (C.c_int, [C.POINTER(VoPagedKV), C.c_uint32, _i32p, C.c_uint32, _i32p, C.c_uint32, _vp, _vp, C.c_int]),
            "vo_paged_gather": (C.c_int, [C.POINTER(VoPagedKV), C.c_uint32, _i32p, C.c_uint32, _i32p, _i64p, C.c_int, _vp, _vp, _u16p, _u16p]),
            "vo_paged_compact": (C.c_int, [C.POINTER(VoPagedKV), C.c_uint32, _i32p, _i32p]),
            "vo_paged_decode_attention": (C.c_int, [C.c_int, _sz, C.POINTER(VoPagedKV), C.c_uint32, C.c_uint32, _i32p, C.c_uint32, _i32p, _f32p, _f32p]),
            "vo_attention_textbook_f64": (None, [_f32p, _f32p, _sz, _f32p, _sz, _sz, _sz, C.POINTER(C.c_double)]),
            "vo_rope_row": (None, [_f32p, _f32p, _sz, _sz, _f32p, _f32p]),
            "vo_paged_append_rope": (C.c_int, [C.POINTER(VoPagedKV), C.c_uint32, _i32p, C.c_uint32, _i32p, C.c_uint32,
                                               _vp, _vp, C.c_int, _f32p, _f32p, _sz, _sz]),
            "vo_int4_ks_index": (_sz, [C.POINTER(VoPagedKV), _sz, _sz, _sz, _sz]),
            "vo_int4_v_byte": (_sz, [C.POINTER(VoPagedKV), _sz, _sz, _sz, _sz, C.POINTER(C.c_int)]),
            "vo_f16_v_index": (_sz, [C.POINTER(VoPagedKV), _sz, _sz, _sz, _sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args

    # ---- generators ----
    def normal(self, seed: int, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        self.lib.vo_fill_normal(seed, ptr(out, _f32p), n)
        return out

    def permutation(self, seed: int, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self.lib.vo_permutation(seed, ptr(out, _i32p), n)
        return out

    def uniform_int(self, seed: int, lo: int, hi: int, n: int) -> np.ndarray:
        out = np.empty(n, np.int32)
        self.lib.vo_uniform_int(seed, lo, hi, ptr(out, _i32p), n)
        return out

    # ---- fp16 ----
    def f32_to_f16(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty(x.shape, np.uint16)
        self.lib.vo_f32_to_f16(ptr(x, _f32p), ptr(out, _u16p), x.size)
        return out

    def f16_to_f32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, np.uint16)
        out = np.empty(h.shape, np.float32)
        self.lib.vo_f16_to_f32(ptr(h, _u16p), ptr(out, _f32p), h.size)
        return out

    # ---- codecs ----
    def int4_quantize_head(self, x: np.ndarray):
        x = np.ascontiguousarray(x, np.float32)
        d = x.size
        codes = np.empty(d // 2, np.uint8)
        scales = np.empty(d // 32, np.uint16)
        self.lib.vo_int4_quantize_head(ptr(x, _f32p), d, ptr(codes, _u8p), ptr(scales, _u16p))
        return codes, scales

    def int4_dequantize_head(self, codes, scales, d):
        out = np.empty(d, np.float32)
        self.lib.vo_int4_dequantize_head(ptr(codes, _u8p), ptr(scales, _u16p), d, ptr(out, _f32p))
        return out

    def int3_quantize_head(self, x: np.ndarray, block_size: int):
        x = np.ascontiguousarray(x, np.float32)
        d = x.size
        packed = np.zeros((3 * d + 7) // 8, np.uint8)
        scales = np.empty((d + block_size - 1) // block_size, np.float32)
        self.lib.vo_int3_quantize_head(ptr(x, _f32p), d, block_size, ptr(packed, _u8p), ptr(scales, _f32p))
        return packed, scales

    # ---- attention ----
    def attention_ref(self, mode, q, k, v, dot_block=64):
        """q [H][D]; k, v [T][H][D] f32 -> out [H][D] (attention_ref.c over a contiguous cache)."""
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        T, H, D = k.shape
        out = np.zeros((H, D), np.float32)
        self.lib.vo_attention_ref_single_query(mode, dot_block, ptr(q, _f32p), ptr(k, _f32p), ptr(v, _f32p), T, H, D, ptr(out, _f32p))
        return out

    def rope_row(self, x, rope_dim, cos_row, sin_row):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self.lib.vo_rope_row(ptr(x, _f32p), ptr(out, _f32p), x.size, rope_dim,
                             ptr(np.ascontiguousarray(cos_row, np.float32), _f32p),
                             ptr(np.ascontiguousarray(sin_row, np.float32), _f32p))
        return out

    def paged_append_rope(self, pool: HostPool, block_tables, start_pos, k_new, v_new, cos, sin, rope_dim):
        """paged_append with K rotated by rows start_pos+i of cos/sin [max_pos][rope_dim/2]."""
        B, n_new = k_new.shape[0], k_new.shape[1]
        bt = np.ascontiguousarray(block_tables, np.int32)
        sp = np.ascontiguousarray(start_pos, np.int32)
        src_dtype = 0 if k_new.dtype == np.float32 else 1
        cos = np.ascontiguousarray(cos, np.float32)
        sin = np.ascontiguousarray(sin, np.float32)
        d = pool.desc()
        return bool(self.lib.vo_paged_append_rope(C.byref(d), B, ptr(bt, _i32p), bt.shape[1], ptr(sp, _i32p), n_new,
                                                  k_new.ctypes.data, v_new.ctypes.data, src_dtype, ptr(cos, _f32p),
                                                  ptr(sin, _f32p), rope_dim, cos.shape[0]))

    def paged_append(self, pool: HostPool, block_tables, start_pos, k_new, v_new):
        B, n_new = k_new.shape[0], k_new.shape[1]
        bt = np.ascontiguousarray(block_tables, np.int32)
        sp = np.ascontiguousarray(start_pos, np.int32)
        src_dtype = 0 if k_new.dtype == np.float32 else 1
        assert k_new.dtype in (np.float32, np.uint16)
        d = pool.desc()
        ok = self.lib.vo_paged_append(C.byref(d), B, ptr(bt, _i32p), bt.shape[1], ptr(sp, _i32p), n_new,
                                      ptr(k_new), ptr(v_new), src_dtype)
        return bool(ok)

    def paged_gather(self, pool: HostPool, block_tables, ctx_lens, out_mode=0):
        bt = np.ascontiguousarray(block_tables, np.int32)
        cl = np.ascontiguousarray(ctx_lens, np.int32)
        offs = np.zeros(len(cl), np.int64)
        offs[1:] = np.cumsum(cl[:-1])
        T = int(cl.sum())
        H, D = pool.num_kv_heads, pool.head_dim
        ks = vs = None
        if out_mode == 1 or pool.dtype == DTYPE_F32:
            ok_ = np.zeros((T, H, D), np.float32)
            ov = np.zeros((T, H, D), np.float32)
        elif pool.dtype == DTYPE_F16:
            ok_ = np.zeros((T, H, D), np.uint16)
            ov = np.zeros((T, H, D), np.uint16)
        else:
            ok_ = np.zeros((T, H, D // 2), np.uint8)
            ov = np.zeros((T, H, D // 2), np.uint8)
            ks = np.zeros((T, H, D // 32), np.uint16)
            vs = np.zeros((T, H, D // 32), np.uint16)
        d = pool.desc()
        r = self.lib.vo_paged_gather(C.byref(d), len(cl), ptr(bt, _i32p), bt.shape[1], ptr(cl, _i32p), ptr(offs, _i64p),
                                     out_mode, ptr(ok_), ptr(ov), ptr(ks, _u16p) if ks is not None else None,
                                     ptr(vs, _u16p) if vs is not None else None)
        assert r == 1
        return ok_, ov, ks, vs

    def paged_compact(self, pool: HostPool, src, dst):
        s = np.ascontiguousarray(src, np.int32)
        t = np.ascontiguousarray(dst, np.int32)
        d = pool.desc()
        return bool(self.lib.vo_paged_compact(C.byref(d), len(s), ptr(s, _i32p), ptr(t, _i32p)))

    def paged_decode(self, mode, pool: HostPool, block_tables, ctx_lens, q, dot_block=64):
        bt = np.ascontiguousarray(block_tables, np.int32)
        cl = np.ascontiguousarray(ctx_lens, np.int32)
        q = np.ascontiguousarray(q, np.float32)
        B, Hq, D = q.shape
        out = np.zeros((B, Hq, D), np.float32)
        d = pool.desc()
        r = self.lib.vo_paged_decode_attention(mode, dot_block, C.byref(d), B, Hq, ptr(bt, _i32p), bt.shape[1],
                                               ptr(cl, _i32p), ptr(q, _f32p), ptr(out, _f32p))
        assert r == 1
        return out


class Reference:
    """The reference's own C path (compiled from its sources into oracle/_ref)."""

    def __init__(self, path: Path = REF_SO):
        if not path.exists():
            raise FileNotFoundError(f"{path} not built (run make -C oracle ref)")
        L = self.lib = C.CDLL(str(path))
        sig = {
            "vr_paged_new": (_vp, [_sz, _sz, _sz, _sz]),
            "vr_paged_free": (None, [_vp]),
            "vr_paged_key_pages": (_f32p, [_vp]),
            "vr_paged_value_pages": (_f32p, [_vp]),
            "vr_paged_session_pages": (_sz, [_vp, C.c_uint64, _u32p, _sz]),
            "vr_paged_page_meta": (None, [_vp, _sz, _u32p, _u32p, _u32p]),
            "vr_paged_stats": (None, [_vp, _u64p]),
            "vr_paged_read": (_sz, [_vp, C.c_uint64, _f32p, _f32p, _sz]),
            "vr_attention_mha": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _f32p]),
            "vr_attention_gqa": (None, [_f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _f32p]),
            "vr_int3_append_and_dump": (C.c_int, [_f32p, _f32p, _sz, _sz, _sz, _sz, _u8p, _f32p, _f32p]),
            "vr_now": (C.c_double, []),
            "vr_baseline_decode": (C.c_double, [C.c_int, _sz, _sz, _sz, _sz, _sz, _sz, _f32p, _f32p, _f32p, _f32p]),
            "vr_batcher_new": (_vp, [_sz, _sz, _sz, _sz, _sz, _sz]),
            "vr_batcher_free": (None, [_vp]),
            "vr_batch_item_size": (_sz, []),
            "vspec_continuous_batch_submit": (C.c_int, [_vp, _sz, _sz, _sz, C.c_uint16, C.POINTER(C.c_uint64)]),
            "vspec_continuous_batch_next_batch": (_sz, [_vp, _vp, _sz]),
            "vspec_continuous_batch_commit_prefill": (C.c_int, [_vp, C.c_uint64, _sz]),
            "vspec_continuous_batch_commit_decode": (C.c_int, [_vp, C.c_uint64, _sz, C.c_int]),
            "vspec_kv_paged_open_session": (C.c_int, [_vp, C.c_uint64]),
            "vspec_kv_paged_close_session": (C.c_int, [_vp, C.c_uint64]),
            "vspec_kv_paged_reuse_prefix": (C.c_int, [_vp, C.c_uint64, C.c_uint64, _sz]),
            "vspec_kv_paged_append": (C.c_int, [_vp, C.c_uint64, _f32p, _f32p]),
            "vspec_kv_paged_get_token_ptr": (C.c_int, [_vp, C.c_uint64, _sz, _sz, C.POINTER(_f32p), C.POINTER(_f32p)]),
            "vspec_kv_paged_session_tokens": (_sz, [_vp, C.c_uint64]),
            "vspec_quant_packed_bytes": (_sz, [_sz, C.c_uint8]),
            "vspec_quant_clip_signed": (C.c_int8, [C.c_int8, C.c_uint8]),
            "vspec_quant_pack_signed": (None, [_i8p, _sz, C.c_uint8, _u8p]),
            "vspec_quant_get_signed": (C.c_int8, [_u8p, _sz, C.c_uint8]),
            "vspec_quant_unpack_signed": (None, [_u8p, _sz, C.c_uint8, _i8p]),
            "vspec_int4_pack": (None, [_i8p, _sz, _u8p]),
            "vspec_int4_get": (C.c_int8, [_u8p, _sz]),
            "vspec_3bit_dynamic_clamp_std": (None, [_f32p, _sz, C.c_float, _f32p]),
            "vspec_memory_pool_init": (C.c_int, [_vp, _vp, _sz]),
            "vspec_memory_pool_alloc": (_vp, [_vp, _sz, _sz]),
            "vspec_arena_init": (C.c_int, [_vp, _vp, _sz]),
            "vspec_arena_alloc": (_vp, [_vp, _sz, _sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args

    @staticmethod
    def set_mode(mode: int):
        """Pin the reference's env-dependent numerics (three_bit_runtime_modules.c:60-66)."""
        os.environ.pop("VSPEC_FUSED_BITS", None)
        os.environ.pop("VSPEC_3BIT_BLOCK_SIZE", None)
        if mode:
            os.environ["VSPEC_3BIT_RUNTIME_MODULE"] = "1"
        else:
            os.environ.pop("VSPEC_3BIT_RUNTIME_MODULE", None)

    def baseline_decode(self, mode, nthreads, k, v, q, block_tokens=16):
        """Time the reference decode step (append + capi gather + GQA attention_ref) over
        sequences k, v [S][T][Hkv][D] f32, q [S][Hq][D].  Returns (seconds, out)."""
        self.set_mode(mode)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        q = np.ascontiguousarray(q, np.float32)
        S, T, Hkv, D = k.shape
        Hq = q.shape[1]
        out = np.zeros((S, Hq, D), np.float32)
        sec = self.lib.vr_baseline_decode(nthreads, S, T, Hq, Hkv, D, block_tokens, ptr(k, _f32p), ptr(v, _f32p),
                                          ptr(q, _f32p), ptr(out, _f32p))
        if sec < 0:
            raise RuntimeError("reference baseline failed")
        return sec, out

    def attention_mha(self, mode, q, k, v):
        self.set_mode(mode)
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        T, H, D = k.shape
        out = np.zeros((H, D), np.float32)
        self.lib.vr_attention_mha(ptr(q, _f32p), ptr(k, _f32p), ptr(v, _f32p), T, H, D, ptr(out, _f32p))
        return out

    def attention_gqa(self, mode, q, k, v):
        self.set_mode(mode)
        q = np.ascontiguousarray(q, np.float32)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        T, Hkv, D = k.shape
        Hq = q.shape[0]
        out = np.zeros((Hq, D), np.float32)
        self.lib.vr_attention_gqa(ptr(q, _f32p), ptr(k, _f32p), ptr(v, _f32p), T, Hq, Hkv, D, ptr(out, _f32p))
        return out
