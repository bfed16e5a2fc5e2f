"""CPU checks of the C-ABI boundary (no GPU calls).

* lib/libvspec_rocm.so loads and exports every function include/*.h declares;
* the ctypes mirrors in vspec_rocm match the C layouts (sizeof / offsetof from gcc);
* the layout-compatible reference types in include/vspec_abi.h have the same
  sizes and offsets as the reference's own headers (when the reference tree is
  present), so a reference build can hand its structs across the boundary.
"""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
INC = ROOT / "include"
REF_INC = Path("/root/reference/include")


def _declared_functions():
    names = set()
    for h in INC.glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(vspec_[a-z0-9_]+)\s*\(", text):
            names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    import vspec_rocm

    L = vspec_rocm.lib()
    declared = _declared_functions()
    assert "vspec_make_rocm_backend" in declared and "vspec_rocm_paged_decode_attention" in declared
    missing = [n for n in sorted(declared) if not hasattr(L, n)]
    assert not missing, missing
    # the Python binding covers the whole public surface
    assert declared <= set(vspec_rocm.SIGNATURES), declared - set(vspec_rocm.SIGNATURES)


def test_pool_bytes_formula():
    import vspec_rocm

    L = vspec_rocm.lib()
    rows = 10 * 8 * 16
    assert L.vspec_rocm_kv_pool_bytes(1, 10, 16, 8, 128) == 2 * rows * 256
    assert L.vspec_rocm_kv_pool_bytes(0, 10, 16, 8, 64) == 2 * rows * 256
    # int4: codes + scales, and one clamp-flag word per 16-token tile of K
    assert L.vspec_rocm_kv_pool_bytes(2, 10, 16, 8, 128) == 2 * rows * (64 + 8) + (rows // 16) * 4


def test_argument_validation_without_gpu():
    """Host-side validation rejects bad descriptors before any device work."""
    import vspec_rocm

    L = vspec_rocm.lib()
    kv = vspec_rocm.VspecPagedKV()
    kv.dtype, kv.num_blocks, kv.block_tokens, kv.num_kv_heads, kv.head_dim = 1, 4, 16, 2, 12
    kv.k_data = kv.v_data = 0x1000
    assert L.vspec_rocm_kv_append(C.byref(kv), 1, 0x1, 1, 0x1, 1, 0x1, 0x1, 1, None) == 0
    assert "head_dim" in vspec_rocm.last_error()
    kv.dtype, kv.head_dim = 2, 48  # int4 rows are whole 32-element groups
    assert L.vspec_rocm_kv_append(C.byref(kv), 1, 0x1, 1, 0x1, 1, 0x1, 0x1, 1, None) == 0
    assert "multiple of 32" in vspec_rocm.last_error()
    kv.dtype = 1
    # f16 pools keep 16-token tiles (V in groups of 4 tokens) for append and gather too
    kv.head_dim, kv.block_tokens = 64, 24
    assert L.vspec_rocm_kv_append(C.byref(kv), 1, 0x1, 1, 0x1, 1, 0x1, 0x1, 1, None) == 0
    assert "f16 pools need block_tokens a multiple of 16" in vspec_rocm.last_error()
    kv.dtype = 0  # f32 pools take any block size: the next error is the null-argument check
    assert L.vspec_rocm_kv_append(C.byref(kv), 1, 0, 1, 0x1, 1, 0x1, 0x1, 0, None) == 0
    assert "block_tokens" not in vspec_rocm.last_error()
    kv.dtype = 1
    # decode needs block_tokens % 16 == 0 and head_dim in {64, 128}
    dd = vspec_rocm.VspecPagedAttnDesc()
    dd.batch, dd.num_q_heads = 1, 4
    dd.kv = kv
    dd.kv.head_dim, dd.kv.block_tokens = 128, 24
    assert L.vspec_rocm_paged_decode_workspace_bytes(C.byref(dd)) == 0
    assert "block_tokens" in vspec_rocm.last_error()
    dd.kv.head_dim, dd.kv.block_tokens = 96, 16
    assert L.vspec_rocm_paged_decode_workspace_bytes(C.byref(dd)) == 0
    assert "64 or 128" in vspec_rocm.last_error()
    kv.head_dim, kv.block_tokens, kv.dtype = 128, 16, 2  # int4 without scales
    assert L.vspec_rocm_kv_gather(C.byref(kv), 1, 0x1, 1, 0x1, 16, 0x1, 0, 0x1, 0x1, None, None, None) == 0
    assert "scales" in vspec_rocm.last_error()
    d = vspec_rocm.VspecPagedAttnDesc()
    d.kv = kv
    d.kv.dtype = 1
    d.batch, d.num_q_heads = 1, 6
    d.kv.num_kv_heads = 4
    assert L.vspec_rocm_paged_decode_workspace_bytes(C.byref(d)) == 0
    assert "multiple" in vspec_rocm.last_error()
    # block indices are int32 table entries and (block, kv head) pairs are indexed in 32 bits
    d.num_q_heads = 8
    d.kv.num_blocks = 0x80000000
    assert L.vspec_rocm_paged_decode_workspace_bytes(C.byref(d)) == 0
    assert "num_blocks" in vspec_rocm.last_error()
    d.kv.num_blocks = 0x40000000  # x 4 kv heads = 2^32
    assert L.vspec_rocm_paged_decode_workspace_bytes(C.byref(d)) == 0
    assert "num_blocks" in vspec_rocm.last_error()
    # the int4 buffer descriptors hold address bits 0..47
    d.kv.num_blocks = 4
    d.kv.k_scales = d.kv.v_scales = 0x1000
    d.kv.k_data = 1 << 47
    assert L.vspec_rocm_paged_decode_workspace_bytes(C.byref(d)) == 0
    assert "2^47" in vspec_rocm.last_error()
    be = L.vspec_make_rocm_backend()
    assert be.name == b"rocm-gfx950"


_PROBE = r"""
#include <stdio.h>
#include <stddef.h>
%s
#define P(T) printf(#T " %%zu\n", sizeof(T))
#define O(T, F) printf(#T "." #F " %%zu\n", offsetof(T, F))
int main(void) {
  P(VspecKVCache); O(VspecKVCache, current_tokens); O(VspecKVCache, int3_compressed);
  O(VspecKVCache, key_scales); O(VspecKVCache, packed_head_bytes); O(VspecKVCache, owns_int3_buffers);
  P(VspecQuantMeta); O(VspecQuantMeta, scales); O(VspecQuantMeta, special_format); O(VspecQuantMeta, special_data);
  P(VspecKernelContext); O(VspecKernelContext, qmeta); O(VspecKernelContext, config);
  P(VspecExecConfig); O(VspecExecConfig, flags);
  P(VspecBackend); O(VspecBackend, launch_attention);
  %s
  return 0;
}
"""

_OURS_EXTRA = r"""
  P(VspecPagedKV); O(VspecPagedKV, k_data); O(VspecPagedKV, v_scales);
  P(VspecPagedAttnDesc); O(VspecPagedAttnDesc, batch); O(VspecPagedAttnDesc, block_tables);
  O(VspecPagedAttnDesc, ctx_lens); O(VspecPagedAttnDesc, q); O(VspecPagedAttnDesc, scale);
  O(VspecPagedAttnDesc, partition_tokens); O(VspecPagedAttnDesc, workspace); O(VspecPagedAttnDesc, stream);
"""


def _probe(includes, extra, incdir, tmp_path, name):
    src = tmp_path / f"{name}.c"
    exe = tmp_path / name
    src.write_text(_PROBE % (includes, extra))
    subprocess.run(["gcc", "-std=gnu11", f"-I{incdir}", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    return dict(line.rsplit(" ", 1) for line in out.strip().splitlines())


def test_ctypes_layout_matches_c(tmp_path):
    import vspec_rocm as vr

    got = _probe('#include "vspec_rocm.h"', _OURS_EXTRA, INC, tmp_path, "ours")
    checks = {
        "VspecPagedKV": C.sizeof(vr.VspecPagedKV),
        "VspecPagedKV.v_scales": vr.VspecPagedKV.v_scales.offset,
        "VspecPagedAttnDesc": C.sizeof(vr.VspecPagedAttnDesc),
        "VspecPagedAttnDesc.block_tables": vr.VspecPagedAttnDesc.block_tables.offset,
        "VspecPagedAttnDesc.scale": vr.VspecPagedAttnDesc.scale.offset,
        "VspecPagedAttnDesc.workspace": vr.VspecPagedAttnDesc.workspace.offset,
        "VspecPagedAttnDesc.stream": vr.VspecPagedAttnDesc.stream.offset,
        "VspecKVCache": C.sizeof(vr.VspecKVCache),
        "VspecKVCache.owns_int3_buffers": vr.VspecKVCache.owns_int3_buffers.offset,
        "VspecKernelContext": C.sizeof(vr.VspecKernelContext),
        "VspecKernelContext.config": vr.VspecKernelContext.config.offset,
        "VspecBackend": C.sizeof(vr.VspecBackend),
    }
    for k, v in checks.items():
        assert int(got[k]) == v, (k, got[k], v)


@pytest.mark.skipif(not REF_INC.exists(), reason="reference headers absent")
def test_abi_types_match_reference_headers(tmp_path):
    ours = _probe('#include "vspec_abi.h"', "", INC, tmp_path, "ours_abi")
    theirs = _probe('#include "vspec/kernel/backend.h"\n#include "vspec/attention/kv_cache.h"', "", REF_INC, tmp_path, "ref_abi")
    assert ours == theirs


def test_missing_library_fails_loudly(tmp_path):
    """With the HIP library absent the binding raises on first use, high-level calls
    included: there is no CPU fallback to run instead."""
    import os
    import sys

    code = (
        "import torch\n"
        "import vspec_rocm as vr\n"
        "pool = vr.PagedPool(vr.KV_F16, 2, 16, 1, 64, device='cpu')\n"
        "tab = torch.zeros((1, 2), dtype=torch.int32)\n"
        "sp = torch.zeros(1, dtype=torch.int32)\n"
        "k = torch.zeros((1, 1, 1, 64), dtype=torch.float16)\n"
        "for f in (vr.lib, lambda: vr.kv_append(pool, tab, sp, k, k)):\n"
        "    try:\n"
        "        f()\n"
        "    except vr.VspecRocmError as e:\n"
        "        assert 'missing' in str(e)\n"
        "    else:\n"
        "        raise SystemExit('no error')\n"
        "print('raised')\n"
    )
    env = dict(os.environ, VSPEC_ROCM_LIB=str(tmp_path / "absent.so"),
               PYTHONPATH=str(ROOT / "vspec-engine_amd" / "python"))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "raised" in r.stdout, r.stderr[-2000:]
