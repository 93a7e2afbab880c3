"""openmini_qmm_linear_host_noalloc (the entry point that allocates nothing) against
openmini_qmm_linear_host, through the C-ABI.

Both run the same GEMV kernels on the same inputs, so the outputs must be bitwise
identical; each is also checked against the fp64 oracle (model.rs:1050-1064, 1e-3).
Two calls in a row share the library's staging array: the second, smaller call must
not see the first call's data.  A call past the staging size is rejected."""
import ctypes

import numpy as np
import pytest

from openmini_qmm import _native, synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _both(qmm, w, x):
    L = _native.lib()
    m = x.shape[0]
    y_ref = np.full((m, w.n_rows), np.nan, np.float32)
    y = np.full((m, w.n_rows), np.nan, np.float32)
    _native.check(L.openmini_qmm_linear_host(w.handle, _ptr(x), _ptr(y_ref), m))
    _native.check(L.openmini_qmm_linear_host_noalloc(w.handle, _ptr(x), _ptr(y), m))
    return y, y_ref


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_noalloc_matches_linear_host(qmm, orc, qtype):
    # first call: 9 rows (batched kernel) of a 4096 x 4096 weight; second call: 3 rows
    # (single-row kernel) of a smaller 1000 x 2080 weight, with the first call's data
    # still in the staging array
    for N, K, m, seed in ((4096, 4096, 9, 0xA10), (1000, 2080, 3, 0xA20)):
        print(f"noalloc type={qtype} N={N} K={K} m={m}", flush=True)
        blocks = synth.weight_blocks(qtype, N, K, seed=seed)
        w = qmm.QuantizedWeight(qtype, blocks, N, K)
        x = synth.normal(seed + 1, (m, K), 1.0)
        y, y_ref = _both(qmm, w, x)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} K={K} m={m}")


def test_noalloc_rejects_past_staging(qmm):
    L = _native.lib()
    N, K = 8192, 8192
    blocks = synth.weight_blocks(Q4_0, N, K, seed=0xA30)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    rows_max = ((16 << 20) - 256) // ((N + K) * 4)  # 255 rows of x[8192] and y[8192]
    m = rows_max + 1
    x = np.zeros((m, K), np.float32)
    y = np.full((m, N), 7.0, np.float32)
    assert L.openmini_qmm_linear_host_noalloc(w.handle, _ptr(x), _ptr(y), m) == _native.ERR_INVALID_PARAM
    assert b"staging" in L.openmini_qmm_last_error()
    assert np.all(y == 7.0)  # nothing written
    # the largest accepted call runs and matches the allocating path
    xs = synth.normal(0xA31, (rows_max, K), 1.0)
    ys, ys_ref = _both(qmm, w, xs)
    assert np.array_equal(ys.view(np.uint32), ys_ref.view(np.uint32))
