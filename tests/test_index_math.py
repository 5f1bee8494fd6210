"""The decode kernels' small floor division (mi_moe_device.hpp div_small):
floor(i / d) as (float)(i + 0.5) * fl(1 / d), truncated.  Claimed exact for
0 <= i < 2^21 and d >= 1; checked here in fp32 arithmetic (numpy float32,
round-to-nearest like the device) over that whole range of i for the
divisors the kernels use (top-k K, blocks per row H/32 and I/32) and more."""
import numpy as np
import pytest


@pytest.mark.parametrize("d", list(range(1, 17)) + [24, 32, 48, 64, 96, 128, 192, 256, 384, 512, 1000])
def test_div_small_exact(d):
    i = np.arange(1 << 21, dtype=np.int64)
    rd = np.float32(1.0) / np.float32(d)
    q = ((i.astype(np.float32) + np.float32(0.5)) * rd).astype(np.int64)   # fp32 ops, truncation
    assert np.array_equal(q, i // d)
