"""The test-input generator of the reference's Rust tests (refgen.rand_vec):
the block-stepped LCG equals the one-step-at-a-time definition
(tests/metal_qmm_4bit_parity.rs:14-24) across block boundaries."""
import numpy as np
import pytest

from refgen import _A, _BLOCK, _C, _M, rand_vec


def rand_vec_scalar(n, seed):
    s = (seed * _A + _C) & _M
    out = np.empty(n, np.uint32)
    for i in range(n):
        s = (s * _A + _C) & _M
        out[i] = (s >> 33) & 0xFFFFFFFF
    return (out.astype(np.float32) / np.float32(4294967295.0)) - np.float32(0.5)


@pytest.mark.parametrize("n,seed", [(0, 1), (1, 3), (5, 11), (_BLOCK, 7), (_BLOCK + 1, 9), (3 * _BLOCK - 1, 0x1234),
                                    (2 * _BLOCK + 77, (1 << 40) + 5)])
def test_rand_vec_matches_scalar_lcg(n, seed):
    assert np.array_equal(rand_vec(n, seed), rand_vec_scalar(n, seed))
