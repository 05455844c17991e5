"""The allocation-free matrix operator (ls_matmul_noalloc) against the allocating one (ls_matmul),
through the C ABI on an MI355X: the same bits for every format, two calls in a row on the same
scratch (the second smaller, so it runs over what the first left behind), the second also with a
split K; and a call that needs more than the static scratch is refused before any work.
"""
import sys

import numpy as np
import pytest

import layerstream_amd as LS
import tinymodels as T
from hipmem import DeviceArray, hip

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def weights(f, rows, cols, rng):
    w = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    if f[0] == 16:
        return T.bf16_trunc_bytes(w.reshape(-1))
    return np.concatenate([LS.quantize_row(f, r)[0] for r in w])


def product(fn, f, dw, rows, cols, x):
    t = x.shape[0]
    dx, dy = DeviceArray(x), DeviceArray(np.full(t * rows, np.nan, np.float32))
    LS._check(fn(LS.fmt(*f), dw.p, rows, cols, dx.p, t, dy.p, None))
    assert hip().hipDeviceSynchronize() == 0
    return dy.to_host(np.zeros(t * rows, np.float32))


@pytest.mark.parametrize("f", [(16, 0), (8, 64), (4, 32), (4, 16)])
def test_noalloc_matmul_equals_the_allocating_one_on_two_calls_in_a_row(f):
    rng = np.random.default_rng(11)
    L = LS.lib()
    # first call: wide K (5 split-K pieces) over 33 inputs (3 token tiles); second: smaller
    for rows, cols, t in [(600, 4864, 33), (150, 896, 5)]:
        say("noalloc", f, rows, cols, t)
        dw = DeviceArray(weights(f, rows, cols, rng))
        x = rng.standard_normal((t, cols)).astype(np.float32)
        want = product(L.ls_matmul, f, dw, rows, cols, x)
        got = product(L.ls_matmul_noalloc, f, dw, rows, cols, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (f, rows, cols, t)


def test_noalloc_matmul_refuses_what_does_not_fit_its_scratch():
    L = LS.lib()
    dw, dx, dy = DeviceArray(np.zeros(16, np.uint8)), DeviceArray(np.zeros(16, np.float32)), DeviceArray(np.zeros(16, np.float32))
    # 8192 x 8192 int8: a 64 MiB tile copy, above the 32 MiB array (nothing is read before the check)
    rc = L.ls_matmul_noalloc(LS.fmt(8, 64), dw.p, 8192, 8192, dx.p, 1, dy.p, None)
    assert rc == -1 and b"static limit" in L.ls_last_error()
