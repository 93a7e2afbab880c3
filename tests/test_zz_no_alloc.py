"""openmini_qmm_linear_host_noalloc (the entry point that allocates nothing) against
openmini_qmm_linear_host, through the C-ABI.

Both run the same kernels on the same inputs, so the outputs must be bitwise
identical; each is also checked against the fp64 oracle (model.rs:1050-1064, 1e-3).
Calls in a row share the library's staging array: a later, smaller call must not see
an earlier call's data.  A call past the staging size is rejected.""" 
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
    # first call: 150 rows (fp32 prefill GEMM) of a 1000 x 2080 weight; then 9 rows
    # (batched kernel) of a 4096 x 4096 weight; then 3 rows (single-row kernel) of the
    # first weight's shape, each with the previous call's data still in the staging array
    for N, K, m, seed in ((1000, 2080, 150, 0xA00), (4096, 4096, 9, 0xA10), (1000, 2080, 3, 0xA20)):
        print(f"noalloc type={qtype} N={N} K={K} m={m}", flush=True)
        blocks = synth.weight_blocks(qtype, N, K, seed=seed)
        w = qmm.QuantizedWeight(qtype, blocks, N, K)
        x = synth.normal(seed + 1, (m, K), 1.0)
        y, y_ref = _both(qmm, w, x)
        assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32))
        assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} K={K} m={m}")


def _staged_bytes(rows, N, K, t):
    """The staging the entry point needs for `rows` rows: x, from the weight's
    gemm_min_rows() = t rows on the fp32 GEMM's workspace (split x and one exponent per
    row), then y, each from a 256-byte boundary."""
    def up(v):
        return (v + 255) // 256 * 256
    work = up(rows * K * 4) + rows * 4 if rows >= t else 0
    return up(rows * K * 4) + work + rows * N * 4


def test_noalloc_rejects_past_staging(qmm):
    L = _native.lib()
    N, K = 8192, 8192
    blocks = synth.weight_blocks(Q4_0, N, K, seed=0xA30)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    t = w.gemm_min_rows()
    rows_max = max(r for r in range(1, 600) if _staged_bytes(r, N, K, t) <= 16 << 20)
    assert rows_max >= t  # the largest call runs the fp32 GEMM
    m = rows_max + 1
    x = np.zeros((m, K), np.float32)
    y = np.full((m, N), 7.0, np.float32)
    assert L.openmini_qmm_linear_host_noalloc(w.handle, _ptr(x), _ptr(y), m) == _native.ERR_INVALID_PARAM
    assert b"staging" in L.openmini_qmm_last_error()
    assert f"at most {rows_max} rows".encode() in L.openmini_qmm_last_error()
    assert np.all(y == 7.0)  # nothing written
    # the largest accepted call runs and matches the allocating path
    xs = synth.normal(0xA31, (rows_max, K), 1.0)
    ys, ys_ref = _both(qmm, w, xs)
    assert np.array_equal(ys.view(np.uint32), ys_ref.view(np.uint32))


def test_noalloc_concurrent_threads(qmm):
    """Four host threads call the entry point at once, each on its own weight (both
    kernels, a K-split weight among them).  The library serialises the shared staging
    array per device, so every result must equal the single-threaded linear_host
    result for the same inputs, bit for bit."""
    import threading
    L = _native.lib()
    cases = [(Q4_0, 4096, 4096, 9, 0xA40), (Q8_0, 1000, 2080, 3, 0xA41), (Q4_0, 2048, 8192, 16, 0xA42),
             (Q8_0, 3000, 1024, 1, 0xA43)]
    work = []
    for qtype, N, K, m, seed in cases:
        w = qmm.QuantizedWeight(qtype, synth.weight_blocks(qtype, N, K, seed=seed), N, K)
        xs = [synth.normal(seed + 1 + r, (m, K), 1.0) for r in range(6)]
        refs = []
        for x in xs:
            y = np.full((m, N), np.nan, np.float32)
            _native.check(L.openmini_qmm_linear_host(w.handle, _ptr(x), _ptr(y), m))
            refs.append(y)
        work.append((w, xs, refs))
    errors = []

    def run(i):
        w, xs, refs = work[i]
        try:
            for r, (x, ref) in enumerate(zip(xs, refs)):
                y = np.full_like(ref, np.nan)
                rc = L.openmini_qmm_linear_host_noalloc(w.handle, _ptr(x), _ptr(y), x.shape[0])
                if rc != 0:
                    errors.append((i, r, rc, L.openmini_qmm_last_error()))
                elif not np.array_equal(y.view(np.uint32), ref.view(np.uint32)):
                    errors.append((i, r, "differs from linear_host"))
        except Exception as e:  # reported below, on the main thread
            errors.append((i, repr(e)))

    print("noalloc: 4 threads x 6 calls", flush=True)
    threads = [threading.Thread(target=run, args=(i,)) for i in range(len(work))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_noalloc_leaves_device_memory_unchanged(qmm):
    """After a warm-up call, further calls leave the device's free memory where it
    was (hipMemGetInfo): the staging array is static, nothing is allocated or kept."""
    import ctypes as C
    from openmini_qmm import hip_runtime as hipr
    H = hipr.hip()
    H.hipMemGetInfo.restype = C.c_int
    H.hipMemGetInfo.argtypes = [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
    L = _native.lib()
    N, K, m = 4096, 4096, 12
    w = qmm.QuantizedWeight(Q4_0, synth.weight_blocks(Q4_0, N, K, seed=0xA50), N, K)
    x = synth.normal(0xA51, (m, K), 1.0)
    y = np.empty((m, N), np.float32)
    _native.check(L.openmini_qmm_linear_host_noalloc(w.handle, _ptr(x), _ptr(y), m))
    free0, total = C.c_size_t(), C.c_size_t()
    assert H.hipMemGetInfo(C.byref(free0), C.byref(total)) == 0
    for _ in range(5):
        _native.check(L.openmini_qmm_linear_host_noalloc(w.handle, _ptr(x), _ptr(y), m))
    free1 = C.c_size_t()
    assert H.hipMemGetInfo(C.byref(free1), C.byref(total)) == 0
    assert free1.value == free0.value, (free0.value, free1.value)
