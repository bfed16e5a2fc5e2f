"""CPU emulation of the append kernel (no GPU): the kernel's own per-item code
(vspec-engine_amd/csrc/append_row.h) built for the host with AddressSanitizer
(tests/host_emu/append_emu.cpp) replays the append launches of the GPU tests' cases,
every work item of a launch in forward, reverse and two shuffled orders.

* AddressSanitizer bounds every load and store index the kernel computes by the exact
  extents of the pools, tables and inputs (the run aborts on any access outside them);
* identical pools from every order show that no two work items of a launch write the
  same bytes with different values -- the only way the kernel's result could depend on
  scheduling on the GPU;
* equality with the oracle's append (vo_paged_append, pinned to kv_paged_cache.c:292-303)
  shows the bytes are the reference's.

The cases include the one for which an early GPU run reported an f16 V-pool mismatch
(test_append_gather_bitexact[64-False-1]: f16 pool, f32 source, D=64, P=32, contexts
45/1/70, 9 blocks), with the same launches as that test (uniform chunks, then one token
per launch).  int4 clamp flags need a wave's lanes and are left to the GPU tests."""
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

from cases import make_case
from oracle.oracle import DTYPE_F16, DTYPE_F32, DTYPE_INT4, HostPool

ROOT = Path(__file__).resolve().parent.parent
CLANG = Path("/opt/rocm/llvm/bin/clang++")
ORDERS = (0, 1, 2, 3)


@pytest.fixture(scope="module")
def emu(tmp_path_factory):
    if not CLANG.exists():
        pytest.skip("ROCm clang++ not found")
    out = tmp_path_factory.mktemp("emu") / "append_emu"
    cmd = [str(CLANG), "-std=c++17", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer",
           f"-I{ROOT / 'tests' / 'host_emu'}", f"-I{ROOT / 'include'}", f"-I{ROOT / 'vspec-engine_amd' / 'csrc'}",
           str(ROOT / "tests" / "host_emu" / "append_emu.cpp"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True)
    return out


def _raw(a):
    return np.ascontiguousarray(a).tobytes()


class Recorder:
    """Append launches applied to the oracle pool and written out for the emulator."""

    def __init__(self, oracle, case, d: Path, src_dtype):
        self.oracle, self.case, self.dir, self.n = oracle, case, d, 0
        self.src = src_dtype
        d.mkdir(parents=True, exist_ok=True)
        self.init = [None if a is None else a.copy() for a in (case.host.k, case.host.v, case.host.ks, case.host.vs)]

    def uniform(self, tables, start, k, v):
        assert self.oracle.paged_append(self.case.host, tables, start, k, v)
        self._write(0, tables, k, v, {"start": start.astype(np.int32)}, len(start), k.shape[1], 0)

    def packed(self, tables, item, pos, k, v):
        self._apply_packed(tables, item, pos, k, v)
        self._write(1, tables, k, v, {"item": item.astype(np.int32), "pos": pos.astype(np.int32)}, len(item), 1,
                    tables.shape[0])

    def _apply_packed(self, tables, item, pos, k, v):
        for t in range(len(item)):  # the oracle appends token by token
            assert self.oracle.paged_append(self.case.host, np.ascontiguousarray(tables[item[t]: item[t] + 1]),
                                            pos[t: t + 1].astype(np.int32), np.ascontiguousarray(k[t: t + 1][None]),
                                            np.ascontiguousarray(v[t: t + 1][None]))

    def decode_step(self, tables, ctx, k, v):
        live = np.flatnonzero(ctx > 0)
        assert self.oracle.paged_append(self.case.host, np.ascontiguousarray(tables[live]),
                                        (ctx[live] - 1).astype(np.int32), np.ascontiguousarray(k[live][:, None]),
                                        np.ascontiguousarray(v[live][:, None]))
        self._write(2, tables, k, v, {"ctx": ctx.astype(np.int32)}, len(ctx), 1, 0)

    def _write(self, mode, tables, k, v, extra, batch, n_new, n_items):
        pre = self.dir / f"L{self.n}"
        pre.with_suffix(".txt").write_text(f"{mode} {batch} {n_new} {tables.shape[1]} {n_items} 0 0\n")
        (self.dir / f"L{self.n}_tables.bin").write_bytes(_raw(tables.astype(np.int32)))
        (self.dir / f"L{self.n}_k.bin").write_bytes(_raw(k))
        (self.dir / f"L{self.n}_v.bin").write_bytes(_raw(v))
        for name, a in extra.items():
            (self.dir / f"L{self.n}_{name}.bin").write_bytes(_raw(a))
        self.n += 1

    def run(self, emu):
        c = self.case
        (self.dir / "meta.txt").write_text(f"{c.dtype} {self.src} {c.num_blocks} {c.P} {c.Hkv} {c.D} {self.n}\n")
        for name, a in zip(("k", "v", "ks", "vs"), self.init):
            if a is not None:
                (self.dir / f"pool_{name}.bin").write_bytes(_raw(a))
        want = [a for a in (c.host.k, c.host.v, c.host.ks, c.host.vs)]
        for order in ORDERS:
            r = subprocess.run([str(emu), str(self.dir), str(order)], capture_output=True, text=True,
                               env={"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0"})
            assert r.returncode == 0, f"order {order}: {r.stderr[-3000:]}"
            for name, w in zip(("k", "v", "ks", "vs"), want):
                if w is None:
                    continue
                got = np.frombuffer((self.dir / f"out{order}_{name}.bin").read_bytes(), np.uint8)
                bad = np.flatnonzero(got != np.ascontiguousarray(w).view(np.uint8).reshape(-1))
                assert bad.size == 0, f"order {order} {name}: {bad.size} bytes differ from the oracle, first {bad[:8]}"
        shutil.rmtree(self.dir)


def _build_launches(rec, case, prefix_split=True):
    """The launch sequence of tests/test_gpu_parity.py build_both: the prefix every
    sequence shares in one uniform launch, then one launch per position for the ragged
    tails (the sequences still live at that position)."""
    B = case.B
    tmin = int(case.ctx.min())
    first = tmin - 1 if prefix_split and tmin > 1 else tmin
    if first > 0:
        rec.uniform(case.tables, np.zeros(B, np.int32), np.ascontiguousarray(case.k_tokens[:, :first]),
                    np.ascontiguousarray(case.v_tokens[:, :first]))
    for t in range(first, case.tmax):
        live = np.flatnonzero(case.ctx > t)
        if live.size:
            rec.uniform(np.ascontiguousarray(case.tables[live]), np.full(live.size, t, np.int32),
                        np.ascontiguousarray(case.k_tokens[live, t:t + 1]),
                        np.ascontiguousarray(case.v_tokens[live, t:t + 1]))


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("src16", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_append_emulation_bitexact_case(oracle, emu, tmp_path, dtype, src16, D):
    """The cases of test_append_gather_bitexact (the recorded mismatch was D=64,
    src16=False, f16), same seeds, planted values and launches."""
    case = make_case(oracle, dtype, 3, 4, 2, D, 32, [45, 1, 70], seed=10 + dtype + 3 * src16 + D, num_blocks=9,
                     src16=src16)
    case.k_tokens = case.k_tokens.copy()
    if not src16:
        case.k_tokens[0, 3, 0, :5] = [1e-8, -3e-7, 7e4, -1e5, 6.1e-5]
        case.k_tokens[2, 5, 1, :] = 1e-9
    rec = Recorder(oracle, case, tmp_path / "case", 1 if src16 else 0)
    _build_launches(rec, case)
    rec.run(emu)


@pytest.mark.parametrize("dtype", [DTYPE_F32, DTYPE_F16, DTYPE_INT4])
@pytest.mark.parametrize("P", [16, 48])
def test_append_emulation_ragged_launches(oracle, emu, tmp_path, dtype, P):
    """Ragged contexts around block edges with multi-token uniform launches (every launch
    writes many rows of one block), invalid table entries past each context, subnormal and
    overflowing fp16 sources."""
    ctx = [1, 15, 16, 17, 33, 64, 100, 47]
    case = make_case(oracle, dtype, len(ctx), 8, 4, 64, P, ctx, seed=900 + P + dtype, num_blocks=40, src16=False)
    case.k_tokens = case.k_tokens.copy()
    case.k_tokens[3, 2, 1, :4] = [3e-8, -7e-6, 8e4, 6.0e-5]
    rec = Recorder(oracle, case, tmp_path / "case", 0)
    _build_launches(rec, case, prefix_split=False)
    rec.run(emu)


@pytest.mark.parametrize("dtype", [DTYPE_F16, DTYPE_INT4])
def test_append_emulation_packed_and_decode_step(oracle, emu, tmp_path, dtype):
    """Packed-token launches (a continuous-batching step: chunked prefill and decode
    tokens of several sequences, token_pos / token_item) and the decode step's append at
    ctx - 1, including a context of 0 (nothing written)."""
    rng = np.random.default_rng(5 + dtype)
    B, Hkv, D, P = 4, 2, 128, 16
    case = make_case(oracle, dtype, B, 8, Hkv, D, P, [60, 33, 1, 90], seed=77 + dtype, num_blocks=24)
    rec = Recorder(oracle, case, tmp_path / "case", 1)
    f16 = lambda a: oracle.f32_to_f16(a.astype(np.float32))
    lens = np.zeros(B, np.int64)
    for step in range(6):
        quota = rng.integers(0, 12, B)
        item = np.repeat(np.arange(B), quota).astype(np.int32)
        pos = np.concatenate([lens[b] + np.arange(quota[b]) for b in range(B)]).astype(np.int32)
        keep = pos < case.ctx[item] - 1  # stay inside each sequence's blocks, before the decode token
        item, pos = item[keep], pos[keep]
        n = item.size
        if n:
            rec.packed(case.tables, item, pos, f16(rng.standard_normal((n, Hkv, D))),
                       f16(rng.standard_normal((n, Hkv, D))))
            for b in range(B):
                lens[b] = max(lens[b], pos[item == b].max() + 1) if (item == b).any() else lens[b]
    ctx = case.ctx.copy()
    ctx[2] = 0
    rec.decode_step(case.tables, ctx, f16(rng.standard_normal((B, Hkv, D))), f16(rng.standard_normal((B, Hkv, D))))
    rec.run(emu)
