"""select_final's candidate bounds on the host (no GPU).

The final read-off of a large select group reads, for each select round, the
keys of one cell: [round * 8192 + lo, round * 8192 + lo + len), with lo and
len taken from the round's candidate table.  kvv::cell_span
(csrc/kvv_bounds.h, the function the kernel calls) clamps both to the round's
own sample count, so the reads stay inside the group's samples whatever the
table words hold -- stale or uninitialised workspace included.  The header is
plain C++; this test builds it with g++ and feeds it arbitrary words.
"""

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest

CSRC = Path(__file__).resolve().parents[1] / "kernelverse_amd" / "csrc"
CHUNK = 8192

HARNESS = r"""
#include "kvv_bounds.h"
extern "C" void spans(int n, const uint32_t* tlo, const uint32_t* thi, const int64_t* count, const int64_t* round,
                      int64_t chunk, uint32_t* lo, uint32_t* len) {
  for (int i = 0; i < n; ++i) {
    const kvv::CellSpan s = kvv::cell_span(tlo[i], thi[i], count[i], round[i], chunk);
    lo[i] = s.lo;
    len[i] = s.len;
  }
}
"""


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    d = tmp_path_factory.mktemp("bounds")
    src = d / "h.cpp"
    src.write_text(HARNESS)
    so = d / "h.so"
    subprocess.run(["g++", "-O2", "-shared", "-fPIC", f"-I{CSRC}", str(src), "-o", str(so)], check=True)
    return ctypes.CDLL(str(so))


def _spans(lib, tlo, thi, count, rnd, chunk=CHUNK):
    n = tlo.size
    tlo, thi = tlo.astype(np.uint32), thi.astype(np.uint32)
    count, rnd = count.astype(np.int64), rnd.astype(np.int64)
    lo, ln = np.zeros(n, np.uint32), np.zeros(n, np.uint32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    lib.spans(ctypes.c_int(n), p(tlo), p(thi), p(count), p(rnd), ctypes.c_int64(chunk), p(lo), p(ln))
    return lo, ln


def _round_size(count, rnd):
    return np.clip(count - rnd * CHUNK, 0, CHUNK)


def test_arbitrary_table_words_stay_inside_the_round(lib):
    rng = np.random.default_rng(11)
    n = 400_000
    count = rng.integers(8193, 1 << 24, size=n)
    nsub = (count + CHUNK - 1) // CHUNK
    rnd = rng.integers(0, nsub)
    # the table holds u16 words; any value, in any order (a stale or unwritten table)
    tlo = rng.integers(0, 1 << 16, size=n)
    thi = rng.integers(0, 1 << 16, size=n)
    lo, ln = _spans(lib, tlo, thi, count, rnd)
    rsz = _round_size(count, rnd)
    end = rnd * CHUNK + lo.astype(np.int64) + ln.astype(np.int64)
    assert np.all(lo <= rsz)
    assert np.all(lo.astype(np.int64) + ln <= rsz)
    assert np.all(end <= count)


def test_sane_tables_pass_through(lib):
    rng = np.random.default_rng(12)
    n = 200_000
    count = rng.integers(8193, 1 << 24, size=n)
    rnd = rng.integers(0, (count + CHUNK - 1) // CHUNK)
    rsz = _round_size(count, rnd)
    a = rng.integers(0, rsz + 1)
    b = rng.integers(0, rsz + 1)
    tlo, thi = np.minimum(a, b), np.maximum(a, b)
    lo, ln = _spans(lib, tlo, thi, count, rnd)
    assert np.array_equal(lo, tlo) and np.array_equal(ln, thi - tlo)


@pytest.mark.parametrize("t_lo,t_hi,count,rnd,want", [
    (0, 8192, 3 * CHUNK + 5, 3, (0, 5)),          # the group's last, partial round
    (7, 3, 2 * CHUNK, 1, (7, CHUNK - 7)),          # words out of order: the wrapped length is cut
    (65535, 65535, 2 * CHUNK, 0, (CHUNK, 0)),      # start past the round: nothing read
    (100, 200, 2 * CHUNK, 5, (0, 0)),              # a round beyond the group: nothing read
    (0, 65535, CHUNK + 1, 1, (0, 1)),
])
def test_edges(lib, t_lo, t_hi, count, rnd, want):
    lo, ln = _spans(lib, np.array([t_lo]), np.array([t_hi]), np.array([count]), np.array([rnd]))
    assert (int(lo[0]), int(ln[0])) == want
