"""The XCD-sliced decode kernel's placement assumption, decided on the host.

At dmh_create the library launches one workgroup per CU that records the XCD
it ran on (read from the hardware), and plans the XCD-sliced form of the
fused decode kernel only when that placement is a rotation: workgroup b on
XCD (b + r) % n for a single r, with n dividing the grid.  The kernel then
reads its own XCD at run time and numbers itself b / n inside it, so the
rotation's r may change from launch to launch, but the count n per XCD must
hold.  dmh_xcd_rotation is that decision on a recorded placement; these
tests drive it with synthetic placements (no GPU)."""
import ctypes as C

import numpy as np
import pytest

from dismoen._lib import lib


def rot(placement):
    a = np.ascontiguousarray(placement, dtype=np.uint32)
    return lib().dmh_xcd_rotation(a.ctypes.data if a.size else None, int(a.size))


@pytest.mark.parametrize("r", range(8))
def test_mi355x_rotation_any_start(r):
    b = np.arange(256)
    assert rot((b + r) % 8) == 8


@pytest.mark.parametrize("n", [1, 2, 4, 8])
def test_other_xcd_counts(n):
    b = np.arange(64)
    assert rot((b + 1) % n) == n


def test_not_a_rotation():
    b = np.arange(256)
    p = (b % 8).copy()
    p[[5, 6]] = p[[6, 5]]          # two workgroups swapped
    assert rot(p) == 0
    assert rot(b // 32) == 0       # contiguous blocks per XCD
    assert rot((7 - b) % 8) == 0   # descending order
    p = (b % 8).copy()
    p[255] = 3                     # one workgroup elsewhere
    assert rot(p) == 0


def test_count_must_divide_the_grid():
    b = np.arange(250)
    assert rot(b % 8) == 0
    assert rot(np.arange(256) % 5) == 0
    assert rot(np.arange(255) % 5) == 5


def test_degenerate_inputs():
    assert rot([]) == 0
    assert lib().dmh_xcd_rotation(None, 256) == 0
    assert rot(np.full(256, 70)) == 0       # not an XCD number
    assert rot(np.zeros(256)) == 1          # a single XCD: every hand-off is local
