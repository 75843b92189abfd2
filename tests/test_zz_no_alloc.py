"""mk_group_norm_noalloc (the entry point that allocates nothing: its scratch is a fixed array of the library) against
mk_group_norm through the C ABI: bit-identical outputs on two calls in a row, the second smaller, and the size limit
refused before any work."""
import numpy as np
import pytest

import mkimage as M

pytestmark = pytest.mark.gpu


def _norms(x, c, groups, fn, rng_w):
    batch, rows, _ = x.shape
    g = M.Dev.from_array((1 + 0.1 * rng_w.standard_normal(c)).astype(np.float32))
    b = M.Dev.from_array((0.1 * rng_w.standard_normal(c)).astype(np.float32))
    xd = M.Dev.from_array(x)
    y = M.Dev(x.size * 2)
    M.call(fn, xd.p, batch, rows, c, groups, g.p, b.p, 1e-6, y.p, None)
    M.sync()
    return y.to_array(np.uint16, x.shape)


@pytest.mark.parametrize("shape", [((2, 4096, 640), 32), ((1, 1000, 1280), 32)])
def test_group_norm_noalloc_equals_group_norm(gpu, shape):
    (batch, rows, c), groups = shape
    x = np.random.default_rng(rows).standard_normal((batch, rows, c)).astype(np.float32) * 3 + 1
    want = _norms(x, c, groups, "mk_group_norm", np.random.default_rng(7))
    got = _norms(x, c, groups, "mk_group_norm_noalloc", np.random.default_rng(7))
    assert np.array_equal(got, want)


def test_group_norm_noalloc_two_calls_in_a_row(gpu):
    # the second call, smaller, on the array the first left behind
    rng = np.random.default_rng(3)
    for batch, rows, c, groups in ((2, 4096, 640, 32), (1, 77, 256, 8)):
        x = rng.standard_normal((batch, rows, c)).astype(np.float32)
        want = _norms(x, c, groups, "mk_group_norm", np.random.default_rng(batch))
        got = _norms(x, c, groups, "mk_group_norm_noalloc", np.random.default_rng(batch))
        assert np.array_equal(got, want)


def test_group_norm_noalloc_refuses_more_than_its_scratch(gpu):
    z = M.Dev(64)
    # 2 x 4096 chunks x 1024 groups x 16 bytes = 128 MiB of partials: refused on the host, nothing launched
    st = M.lib().mk_group_norm_noalloc(z.p, 2, 65536, 4096, 1024, z.p, z.p, 1e-6, z.p, None)
    assert st == 1 and b"scratch" in M.lib().mk_last_error()
