"""libkvv.so loads on a CPU-only host, exports what include/kvv.h declares, and its
structs have the layout the ctypes binding assumes.  No compute call is made here."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from kernelverse_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kvv.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"KVV_API\s+[\w\s\*]+?\b(kvv_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert names, "no KVV_API declarations found"
    assert set(names) == set(_lib.EXPORTED)
    for name in names:
        assert hasattr(lib, name), name
    assert lib.kvv_abi_version() == 1


def _c_layout(struct: str, fields):
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
           f'printf("size %zu\\n", sizeof({struct}));']
    for f in fields:
        src.append(f'printf("{f} %zu\\n", offsetof({struct}, {f}));')
    src.append("return 0;}")
    return "\n".join(src)


@pytest.mark.parametrize("cls,cname", [(_lib.KvvTensor, "kvv_tensor"), (_lib.KvvPolicy, "kvv_policy"),
                                       (_lib.KvvResult, "kvv_result")])
def test_struct_layout_matches_header(tmp_path, cls, cname):
    fields = [f for f, _ in cls._fields_]
    c = tmp_path / "probe.c"
    c.write_text(_c_layout(cname, fields))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-o", str(exe), str(c)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = dict(line.split() for line in out if line)
    assert int(got["size"]) == ctypes.sizeof(cls)
    for f in fields:
        assert int(got[f]) == getattr(cls, f).offset, f


def _tensor(shape, strides, dtype=_lib.F32, ptr=4096):
    t = _lib.KvvTensor()
    t.data = ptr
    t.dtype = dtype
    t.ndim = len(shape)
    for i, (s, st) in enumerate(zip(shape, strides)):
        t.sizes[i] = s
        t.strides[i] = st
    return t


def _policy(**kw):
    p = _lib.KvvPolicy()
    p.mode = kw.get("mode", _lib.MODE_ISCLOSE)
    p.rtol = kw.get("rtol", 1e-5)
    p.atol = kw.get("atol", 1e-5)
    p.max_abs_diff = kw.get("max_abs_diff", 0)
    p.max_samples = kw.get("max_samples", 1_000_000)
    p.flags = kw.get("flags", 0)
    return p


def test_planning_rejects_bad_arguments():
    lib = _lib.load()
    size = ctypes.c_size_t()
    ok = lib.kvv_workspace_size(_tensor((4, 5), (5, 1)), _tensor((4, 5), (5, 1)), _policy(), ctypes.byref(size))
    assert ok == 0 and size.value >= 256
    assert lib.kvv_workspace_size(_tensor((4, 5), (5, 1)), _tensor((5, 4), (4, 1)), _policy(), ctypes.byref(size)) == -1
    assert b"shapes differ" in lib.kvv_last_error()
    assert lib.kvv_workspace_size(_tensor((4,), (1,), _lib.F16), _tensor((4,), (1,)), _policy(), ctypes.byref(size)) == -1
    assert lib.kvv_workspace_size(_tensor((4,), (1,), 99), _tensor((4,), (1,), 99), _policy(), ctypes.byref(size)) == -1
    assert lib.kvv_workspace_size(_tensor((4,), (1,)), _tensor((4,), (1,)), _policy(max_samples=1),
                                  ctypes.byref(size)) == -1
    assert lib.kvv_workspace_size(_tensor((4,), (1,)), _tensor((4,), (1,)),
                                  _policy(mode=_lib.MODE_MAX_ABS_DIFF, max_abs_diff=2**31), ctypes.byref(size)) == -1
    assert lib.kvv_workspace_size(_tensor((2**21, 2**20), (2**20, 1)), _tensor((2**21, 2**20), (2**20, 1)),
                                  _policy(), ctypes.byref(size)) == -4
    assert lib.kvv_workspace_size(_tensor((4,), (1,), ptr=0), _tensor((4,), (1,)), _policy(),
                                  ctypes.byref(size)) == -1


def test_workspace_grows_with_samples_and_near_zero():
    lib = _lib.load()
    a, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    t = _tensor((1 << 22,), (1,), _lib.BF16)
    lib.kvv_workspace_size(t, t, _policy(max_samples=1000), ctypes.byref(a))
    lib.kvv_workspace_size(t, t, _policy(), ctypes.byref(b))
    lib.kvv_workspace_size(t, t, _policy(flags=_lib.FLAG_NEAR_ZERO), ctypes.byref(c))
    assert a.value < b.value < c.value


def test_many_group_batch_reserves_input_select_state():
    """A batch with more large contiguous pairs than the device has CUs selects
    their p99 from the inputs: its workspace holds 16,640 bytes of state per
    such pair (plus the segment list, the capture pass's chunk work list, the
    per-chunk sampled sums and the fallback's segment list), which the same batch with
    transposed pairs (selected from sample arrays) does not."""
    lib = _lib.load()
    count = 300  # above any device's CU count (no device here: the planner assumes 256)
    GA, PA = _lib.KvvTensor * count, _lib.KvvPolicy * count
    pols = PA(*[_policy() for _ in range(count)])
    contig = GA(*[_tensor((100, 100), (100, 1), ptr=4096 * (1 + i)) for i in range(count)])
    transposed = GA(*[_tensor((100, 100), (1, 100), ptr=4096 * (1 + i)) for i in range(count)])
    a, b = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.kvv_batch_workspace_size(count, contig, contig, pols, ctypes.byref(a)) == 0
    assert lib.kvv_batch_workspace_size(count, transposed, transposed, pols, ctypes.byref(b)) == 0
    state = count * 16_640
    lists = 256 * (2 * -(-count * 4 // 256) + -(-count * 8 // 256) + -(-count * 24 // 256))  # one chunk per pair
    assert a.value - b.value == state + lists


def test_noalloc_rejects_beyond_its_scratch_without_a_device():
    """kvv_verdict_noalloc plans first and refuses a verdict whose workspace exceeds its fixed
    scratch array before touching the device (no device here: nothing may be launched)."""
    lib = _lib.load()
    n = 1 << 23  # 8 Mi bf16 samples of abs and rel: 64 MiB of sample arrays
    t = _tensor((n,), (1,), _lib.BF16)
    size = ctypes.c_size_t()
    assert lib.kvv_workspace_size(t, t, _policy(max_samples=n), ctypes.byref(size)) == 0
    assert size.value > _lib.NOALLOC_SCRATCH_BYTES
    out = ctypes.create_string_buffer(ctypes.sizeof(_lib.KvvResult))
    assert lib.kvv_verdict_noalloc(t, t, _policy(max_samples=n), out, None) == -2
    assert f"holds {_lib.NOALLOC_SCRATCH_BYTES}".encode() in lib.kvv_last_error()
