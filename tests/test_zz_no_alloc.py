"""The allocation-free greedy pick (sml_hip_argmax_noalloc, include/sml-hip.h)
against the allocating one (sml_hip_argmax): the same index, bit for bit, on
two calls in a row -- the second with a smaller input -- through the C ABI,
for inputs that take the two-stage pick over the library's device scratch
and for a one-workgroup input; out-of-range sizes are refused."""
import numpy as np
import pytest

import sheep_amd as sa

pytestmark = pytest.mark.gpu


def pick(fn, lg):
    d = sa.DevBuf.of(lg)
    t = sa.DevBuf.of(np.array([-1], np.int32))
    assert fn(d.ptr, len(lg), t.ptr) == 0, sa.lib().sml_hip_last_error()
    sa.sync()
    return int(t.read(np.int32)[0])


@pytest.mark.parametrize("sizes", [(151936, 128256), (5_000_003, 9000), (128256, 1000)])
def test_noalloc_argmax_equals_argmax(sizes):
    sa.init(0)
    rng = np.random.default_rng(sizes[0])
    for n in sizes:
        lg = rng.standard_normal(n).astype(np.float32)
        lg[n // 3] = lg[n - 1] = lg.max() + 1.0          # a tie: the first index wins
        a = pick(sa.lib().sml_hip_argmax, lg)
        b = pick(sa.lib().sml_hip_argmax_noalloc, lg)
        assert a == b == n // 3, (n, a, b)


def test_noalloc_argmax_refuses_sizes():
    sa.init(0)
    d = sa.DevBuf(16)
    t = sa.DevBuf(4)
    assert sa.lib().sml_hip_argmax_noalloc(d.ptr, 0, t.ptr) == -1
    assert sa.lib().sml_hip_argmax_noalloc(d.ptr, (1 << 30) + 1, t.ptr) == -1
    assert b"argmax_noalloc" in sa.lib().sml_hip_last_error()
