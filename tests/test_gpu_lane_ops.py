"""The wave lane exchanges under every reduction in the kernels, checked directly.

eb_launch_selftest_lane_ops applies the 16- and 32-lane swaps, the DPP row rotations and
mirrors, and the reductions built from them (eyebrowse_amd/csrc/eb_common.h) to known lane
patterns; each row is compared with its definition evaluated in numpy. The inputs are
small integers, so every sum is exact in any order and the comparison is bit for bit. A
compiler that mishandles one of these exchanges (ROCm 7.2 folds the f32 add of a swap's
two results into an add of the first to itself) fails here by name, not only through an
attention output.
"""
import numpy as np
import pytest

import eyebrowse_amd as eb
from tests._gpu import note, upload

pytestmark = pytest.mark.gpu


def _expected(a, b):
    lanes = np.arange(64)
    rows = [a[lanes ^ 16], a[lanes ^ 32]]
    for f in (1, 2, 4, 8, 16, 32):
        rows.append(np.array([a[lanes % f == l % f].sum() for l in lanes], np.float32))
    for f in (1, 8):
        rows.append(np.array([a[lanes % f == l % f].max() for l in lanes], np.float32))
    s32 = np.where(lanes < 32, a + a[lanes ^ 32], b + b[lanes ^ 32])
    odd_row = (lanes >> 4) & 1
    s16 = np.where(odd_row == 0, a + a[lanes ^ 16], b + b[lanes ^ 16])
    rows += [s32, s16]
    for n in (4, 16):
        rows.append(np.array([a[(l // n) * n:(l // n) * n + n].sum() for l in lanes], np.float32))
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_lane_ops_match_their_definitions(dev, seed):
    note(f"lane ops seed={seed}")
    rng = np.random.default_rng(seed)
    a = rng.integers(-1000, 1000, 64).astype(np.float32)
    b = rng.integers(-1000, 1000, 64).astype(np.float32)
    if seed == 2:  # lane-distinct powers of two plus the lane: every partial sum is an
        # integer below 2^24 (exact), and a lane dropped or counted twice changes it
        lanes = np.arange(64)
        a = (2.0 ** (lanes % 18) + lanes).astype(np.float32)
        b = -a[::-1].copy()
    inp = upload(dev, np.concatenate([a, b]))
    out = eb.Tensor.empty(dev, (eb.LANE_OPS_ROWS, 64))
    eb.launch_selftest_lane_ops(dev.stream, inp.data_ptr, out.data_ptr)
    dev.synchronize()
    got = out.to_f32().reshape(eb.LANE_OPS_ROWS, 64)
    want = _expected(a, b)
    names = ["xor16", "xor32", "sum/1", "sum/2", "sum/4", "sum/8", "sum/16", "sum/32",
             "max/1", "max/8", "swap_sum32", "swap_sum16", "group4", "group16"]
    assert len(names) == eb.LANE_OPS_ROWS
    for i, name in enumerate(names):
        np.testing.assert_array_equal(got[i].view(np.uint32), want[i].view(np.uint32),
                                      err_msg=name)
