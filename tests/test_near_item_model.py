"""Host model of the main pass's near-zero element mask (csrc/kvv_kernels.h, near_item).

A wave's item is 64 lanes x 4 vectors of 8 sixteen-bit codes.  A single pair too
small to give every wave of the grid two full items takes smaller items (512 or
1024 elements for bf16/fp16), so a lane's later vectors lie past the item's end
even when the item itself is full.  load_item leaves such absent vectors zero
(`full` has their bit clear), and a zero code is a near-zero value
(|+0| <= near_zero_abs).  near_item therefore masks every lane whose `full` is
not all ones by the elements that lie inside the item.

The model restates that mask bit for bit (mask bit u*4+j for element 2j of
vector u, bit 16+u*4+j for element 2j+1) and counts the near-zero elements of
whole tensors with it.  It also restates a dropped form that skipped the mask
with a wave-uniform test "the item has item_elems elements": on shrunk items
that form counts the absent vectors' zero codes, i.e. 1 + 3/f times the true
count for a near-zero fraction f on 512-element items -- the 4x to 31x
miscount that form gave on the GPU (f = 1 to about 0.1).  No GPU needed.
"""

import numpy as np
import pytest

UNROLL, LANES, V = 4, 64, 8


def _near_code(dtype_bits_bf16=True, t=0.25):
    """Largest bf16 magnitude code whose value is <= t."""
    codes = np.arange(0x7F80, dtype=np.uint32)
    vals = (codes << 16).view(np.float32)
    return int(codes[vals <= np.float32(t)].max())


def _item_mask(codes_item, L0, L1, nz_code, dropped, item_elems):
    """(64 lanes,) near-zero counts of one item, per the kernel's mask logic."""
    lane = np.arange(LANES)
    count = np.zeros(LANES, dtype=np.int64)
    full = np.zeros(LANES, dtype=np.int64)
    vecs = []
    for u in range(UNROLL):
        v = L0 + (u * LANES + lane) * V
        present = v + V <= L1
        full |= present.astype(np.int64) << u
        # the item's codes as loaded: full vectors read, the rest zero (a partial
        # vector's elements past L1 stay zero; its elements before L1 are patched in)
        vec = np.zeros((LANES, V), dtype=np.uint32)
        for e in range(V):
            idx = v + e
            inside = idx < L1
            vec[inside, e] = codes_item[idx[inside] - L0]
        vecs.append(vec)
    # per-element flags: |code| <= nz_code, in the slow-mask bit layout
    mask = np.zeros(LANES, dtype=np.int64)
    for u in range(UNROLL):
        for j in range(4):
            lo = (vecs[u][:, 2 * j] & 0x7FFF) <= nz_code
            hi = (vecs[u][:, 2 * j + 1] & 0x7FFF) <= nz_code
            mask |= lo.astype(np.int64) << (u * 4 + j)
            mask |= hi.astype(np.int64) << (16 + u * 4 + j)
    if dropped and L1 - L0 == item_elems:
        valid = np.full(LANES, 0xFFFFFFFF, dtype=np.int64)
    else:
        valid = np.where(full == 0xF, 0xFFFFFFFF, 0)
        for u in range(UNROLL):
            left = L1 - (L0 + (u * LANES + lane) * V)
            lo = np.where(left >= 7, 0xF, np.where(left > 0, (1 << ((left + 1) >> 1)) - 1, 0))
            hi = np.where(left >= 8, 0xF, np.where(left > 1, (1 << (left >> 1)) - 1, 0))
            part = np.where((full >> u) & 1, 0x000F000F << (u * 4), (lo << (u * 4)) | (hi << (16 + u * 4)))
            valid = np.where(full == 0xF, valid, valid | part)
    m = mask & valid
    for b in range(32):
        count += (m >> b) & 1
    return int(count.sum())


def _tensor_count(codes, item_elems, nz_code, dropped):
    n = codes.size
    total = 0
    for L0 in range(0, n, item_elems):
        L1 = min(L0 + item_elems, n)
        total += _item_mask(codes[L0:L1], L0, L1, nz_code, dropped, item_elems)
    return total


def _codes(n, near_frac, seed):
    rng = np.random.default_rng(seed)
    big = rng.uniform(1.0, 4.0, size=n) * rng.choice([-1.0, 1.0], size=n)
    small = rng.uniform(-0.25, 0.25, size=n)
    x = np.where(rng.random(n) < near_frac, small, big).astype(np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint32)  # bf16 codes by truncation


@pytest.mark.parametrize("n,item_elems", [(4096, 512), (5000, 512), (4096, 1024), (6150, 1024), (8192, 2048),
                                          (9001, 2048), (3, 512)])
def test_kept_mask_counts_exactly(n, item_elems):
    nz = _near_code()
    codes = _codes(n, 0.3, n + item_elems)
    want = int(((codes & 0x7FFF) <= nz).sum())
    assert _tensor_count(codes, item_elems, nz, dropped=False) == want


@pytest.mark.parametrize("near_frac,ratio", [(1.0, 4.0), (0.1, 31.0)])
def test_dropped_form_overcounts_on_shrunk_items(near_frac, ratio):
    """512-element items, every item full: the dropped form adds 3 x 512 zero codes per item."""
    nz = _near_code()
    n = 512 * 16
    codes = _codes(n, near_frac, 7)
    true = int(((codes & 0x7FFF) <= nz).sum())
    got = _tensor_count(codes, 512, nz, dropped=True)
    assert got == true + 3 * n
    assert abs(got / true - ratio) / ratio < 0.15, got / true
    # full-size items (2048 elements: all four vectors of every lane present) are unaffected
    assert _tensor_count(codes, 2048, nz, dropped=True) == true
