"""Batched decode GEMV (four or more activation rows: one pass over W on fp16 MFMA)
against the fp64 oracle (model.rs:1050-1064 semantics: y = x . W^T), tolerance from
tests/parity.py (1e-3 normwise and elementwise)."""
import numpy as np
import pytest

from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def run_gemv(qmm, w, x):
    B = x.shape[0]
    dx = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x))
    dy = qmm.DeviceBuffer(B * w.n_rows * 4)
    w.gemv(dx, dy, B)
    return dy.download(np.float32, (B, w.n_rows))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("N,K", [(1, 32), (37, 96), (130, 2080), (255, 4064), (1000, 4000), (4096, 4096)])
@pytest.mark.parametrize("B", [4, 5, 8, 16, 21, 36])
def test_batch_parity(qmm, orc, qtype, N, K, B):
    print(f"gemv batch type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = synth.weight_blocks(qtype, N, K, seed=0xB000 + N + K + B)
    x = synth.normal(0xB001 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    assert_parity(run_gemv(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} K={K} B={B}")


@pytest.mark.parametrize("qtype,N,K,B", [
    (Q8_0, 11008, 4096, 8),     # BASELINE config 1, batch 8
    (Q8_0, 4096, 11008, 8),
    (Q4_0, 8192, 8192, 16),     # config 4, 70B q-proj, batch 16
    (Q4_0, 1024, 28672, 16),    # a slice of the 70B down-proj's K
])
def test_batch_baseline_shapes(qmm, orc, qtype, N, K, B):
    print(f"gemv batch type={qtype} N={N} K={K} B={B}", flush=True)
    sigma = 0.015 if K >= 8192 else 0.02
    blocks = synth.weight_blocks(qtype, N, K, seed=0xB100 + N + B, sigma=sigma)
    x = synth.normal(0xB101 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    print(assert_parity(run_gemv(qmm, w, x), orc.linear_f64(qtype, blocks, N, K, x), TOL, "baseline"))


@pytest.mark.parametrize("qtype,N,K,B", [
    (Q4_0, 16 * 700, 1024, 8),     # 700 row tiles: 3 per workgroup
    (Q4_0, 16 * 1100, 512, 16),    # 5 per workgroup, one wave (K < 8 groups)
    (Q4_0, 16 * 1400, 1024, 6),    # 6
    (Q4_0, 16 * 1700, 1024, 16),   # 7
    (Q4_0, 16 * 2000 + 5, 1024, 9),  # 8, ragged last tile
    (Q8_0, 16 * 700 + 3, 1024, 8),   # 3 (Q8_0 stops at 4)
    (Q8_0, 16 * 1500, 1024, 16),   # 4
    (12, 16 * 1100, 1024, 8),      # Q4_K, 5
    (14, 16 * 700, 1024, 8),       # Q6_K, 3
])
def test_batch_tiles_per_workgroup(qmm, orc, qtype, N, K, B):
    """Every tiles-per-workgroup count the launch rule picks (ceil(tiles / 256), at
    most 8 or 4) against the oracle on all N outputs; y is NaN-filled first, so a
    tile the kernel skips fails."""
    print(f"gemv batch tiles type={qtype} N={N} K={K} B={B}", flush=True)
    blocks = (synth.kquant_blocks(qtype, N, K, seed=0xB500 + N) if qtype in (12, 14)
              else synth.weight_blocks(qtype, N, K, seed=0xB500 + N))
    x = synth.normal(0xB501 + B, (B, K), 1.0)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    dx, dy = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(B * N * 4)
    dy.fill(0xFF)
    w.gemv(dx, dy, B)
    assert_parity(dy.download(np.float32, (B, N)), orc.linear_f64(qtype, blocks, N, K, x), TOL, f"N={N} B={B}")


@pytest.mark.parametrize("qtype,N,K", [
    (Q4_0, 1024, 8192),        # 64 tiles, 64 groups: 4 K splits of 1 tile
    (Q4_0, 1030, 8192),        # 65 tiles (ragged): 2 splits of 1 tile
    (Q8_0, 2000, 4096),        # 125 tiles, 32 groups: 2 splits of 1 tile
    (12, 4096, 4096),          # Q4_K, 256 tiles: 2 splits of 2 tiles
    (14, 4096, 4096),          # Q6_K, the same
    (Q8_0, 8192, 4096),        # 512 tiles: 2 splits of 4 tiles
    (Q4_0, 1024, 3968),        # 31 groups: no split
    (Q8_0, 2000, 16384),       # 2 splits of 1 tile, 64 groups each: eight waves
    (14, 4096, 16384),         # Q6_K, 2 splits of 2 tiles, eight waves
    (12, 9600, 8192),          # Q4_K, 600 tiles (3 per workgroup), no split, eight waves
    (Q4_0, 8192, 8192),        # 2 splits of 4 tiles, 64 groups; at 4 rows one workgroup of 8 waves
    (Q8_0, 4096, 11008),       # 2 splits of 2 tiles, 86 groups (43 per split); the same at 4 rows
    (Q4_0, 4112, 8192),        # 257 tiles (ragged): 2 splits of 4 tiles; the same at 4 rows
])
def test_batch_k_split(qmm, orc, qtype, N, K):
    """The K-split launches (two or four workgroups per tile group, each over a part
    of K; the last to finish adds the parts in split order; the group's arrival
    counter only grows, by the split count per call), and the eight-wave workgroups
    of 64+ K groups.  Every call is checked on all outputs, y NaN-filled first:
    against the oracle at 4, 7 and 16 rows, and bit for bit against a repeat of the
    same call and against the 16-row call's rows (the split depends on the shape
    only; at 4 rows a two-way split of 64-127 groups runs as one eight-wave workgroup
    per tile group, which must give the split's bits).  The calls run back to back on one weight, so each starts from the count
    its predecessors left (0, splits, 2 splits, ...): a wrong choice of last
    workgroup would leave outputs unwritten (NaN) or half-summed."""
    blocks = (synth.kquant_blocks(qtype, N, K, seed=0xB700 + N) if qtype in (12, 14)
              else synth.weight_blocks(qtype, N, K, seed=0xB700 + N))
    x16 = synth.normal(0xB701 + N, (16, K), 1.0)
    x16[3] *= 1e4
    w = qmm.QuantizedWeight(qtype, blocks, N, K)

    def call(x):
        B = x.shape[0]
        dx, dy = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x)), qmm.DeviceBuffer(B * N * 4)
        dy.fill(0xFF)
        w.gemv(dx, dy, B)
        return dy.download(np.float32, (B, N))

    y16 = call(x16)
    for B in (4, 7, 16):
        print(f"gemv batch k-split type={qtype} N={N} K={K} B={B}", flush=True)
        y = call(x16[:B])
        assert_parity(y, orc.linear_f64(qtype, blocks, N, K, x16[:B]), TOL, f"N={N} K={K} B={B}")
        assert np.array_equal(y.view(np.uint32), call(x16[:B]).view(np.uint32)), "repeat call differs"
        assert np.array_equal(y.view(np.uint32), y16[:B].view(np.uint32)), f"B={B} rows differ from B=16"


def test_k_split_graph_replays_match_eager(qmm):
    """K-split batched GEMVs captured in a HIP graph, as a serving loop replays a
    decode step.  Every replay must equal the eager result bit for bit. Eager calls
    on the same weights run between the replays: each call, captured or not, must
    leave the split counters at a multiple of the split count for the next. No
    memset node is involved; the counters are only ever incremented by the kernels."""
    from openmini_qmm import hip_runtime as hipr
    cases = [(Q4_0, 1024, 8192, 16), (Q8_0, 4096, 8192, 8), (Q4_0, 4096, 4096, 4)]
    st = qmm.Stream()
    sh = st.handle
    runs = []
    for qtype, N, K, B in cases:
        blocks = synth.weight_blocks(qtype, N, K, seed=0xB900 + N + K)
        w = qmm.QuantizedWeight(qtype, blocks, N, K)
        dx = qmm.DeviceBuffer.from_numpy(synth.normal(0xB901 + N, (B, K), 1.0))
        dx2 = qmm.DeviceBuffer.from_numpy(synth.normal(0xB902 + N, (B, K), 1.0))
        dy, dy2 = qmm.DeviceBuffer(B * N * 4), qmm.DeviceBuffer(B * N * 4)
        w.gemv(dx, dy, B, sh)
        st.synchronize()
        runs.append((w, dx, dx2, dy, dy2, B, N, dy.download(np.float32, (B, N))))
    print("gemv batch k-split graph: capture", flush=True)
    graph = hipr.Graph(sh, lambda s: [w.gemv(dx, dy, B, s) for w, dx, _, dy, _, B, _, _ in runs])
    for rep in range(3):
        print(f"gemv batch k-split graph: replay {rep}", flush=True)
        for r in runs:
            r[3].fill(0xFF, sh)
        graph.launch(sh)
        st.synchronize()
        for w, dx, dx2, dy, dy2, B, N, want in runs:
            got = dy.download(np.float32, (B, N))
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"replay {rep} N={N} B={B}"
            w.gemv(dx2, dy2, B, sh)  # eager work on the same weight between replays
        st.synchronize()


def test_engine_matmul_threads_share_a_split_weight(qmm):
    """The engine's matmul (openmini_qmm_linear_host) on one K-split weight from four
    host threads at once, 8 rows each (the batched kernel).  The calls run on the
    null stream, shared by all host threads, and the library also serialises them
    per weight; every thread's result must equal the single-threaded one bit for
    bit."""
    import threading
    N, K = 1024, 8192  # 4 K splits
    blocks = synth.weight_blocks(Q4_0, N, K, seed=0xB800)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    eng = qmm.get_gemm_engine()
    xs = [synth.normal(0xB801 + t, (8, K), 1.0) for t in range(4)]
    want = [eng.matmul(x, w) for x in xs]
    got = [[] for _ in xs]

    def worker(t):
        for _ in range(6):
            got[t].append(eng.matmul(xs[t], w))

    print("gemv batch engine threads N=1024 K=8192 B=8", flush=True)
    threads = [threading.Thread(target=worker, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    for t in range(4):
        assert len(got[t]) == 6
        for y in got[t]:
            assert np.array_equal(y.view(np.uint32), want[t].view(np.uint32)), f"thread {t} differs"


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0, 12, 14])
def test_batch_rows_independent(qmm, qtype):
    """A row's result depends neither on the other rows of the batch (each MFMA row
    and each range scale belongs to one activation row) nor on the batch size: batches
    of up to 8 and up to 4 rows split each row's activations over 2 and 4 lanes, and
    their results must equal the 16-row kernel's bit for bit.  Rows 8..15 of a 16-row
    call equal an 8-row call of the same rows, rows 0..3 a 4-row call, rows 4..9 a
    6-row call; a repeated call is bitwise identical."""
    N, K = 777, 2048
    blocks = (synth.kquant_blocks(qtype, N, K, seed=0xB200) if qtype in (12, 14)
              else synth.weight_blocks(qtype, N, K, seed=0xB200))
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(0xB201, (16, K), 1.0)
    x[3] *= 1e6  # a loud neighbour must not change the quiet rows
    x[9, 100] = np.float32(1e-41)
    y16 = run_gemv(qmm, w, x)
    for lo, hi in ((8, 16), (0, 4), (4, 10), (12, 16)):
        print(f"rows {lo}..{hi - 1} of 16 vs a {hi - lo}-row call", flush=True)
        assert np.array_equal(y16[lo:hi].view(np.uint32), run_gemv(qmm, w, x[lo:hi]).view(np.uint32)), (lo, hi)
    assert np.array_equal(y16.view(np.uint32), run_gemv(qmm, w, x).view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_batch_activation_dynamic_range(qmm, orc, qtype):
    """Per (row, group) range scales: outliers (x1e4), tiny rows (x1e-30 with
    subnormals), huge rows (x1e30), zero rows and zero blocks stay within the contract."""
    N, K = 512, 4096
    blocks = synth.weight_blocks(qtype, N, K, seed=0xB300)
    x = synth.normal(0xB301, (8, K), 1.0)
    x[0, 5] *= 1e4
    x[0, 1000:1032] *= 1e-6
    x[0, 2048:2080] = 0.0
    x[1, :] *= 1e-30
    x[1, 100:110] = np.float32(1e-41)  # subnormal
    x[2, :] *= 1e30
    x[3, :] = 0.0
    x[4, ::64] *= 1e-20
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    y = run_gemv(qmm, w, x)
    ref = orc.linear_f64(qtype, blocks, N, K, x)
    for r in range(8):
        if r == 3:
            assert np.all(y[3] == 0.0)
            continue
        assert_parity(y[r:r + 1], ref[r:r + 1], TOL, f"row {r}")


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_batch_nonfinite_row_stays_in_its_row(qmm, orc, qtype):
    N, K = 96, 512
    blocks = synth.weight_blocks(qtype, N, K, seed=0xB400)
    w = qmm.QuantizedWeight(qtype, blocks, N, K)
    x = synth.normal(0xB401, (8, K), 1.0)
    x[1, 300] = np.nan
    x[3, 0] = -np.inf
    x[6, 511] = np.inf
    y = run_gemv(qmm, w, x)
    for r in (1, 3, 6):
        assert not np.any(np.isfinite(y[r])), r
    for r in (0, 2, 4, 5, 7):
        assert_parity(y[r:r + 1], orc.linear_f64(qtype, blocks, N, K, x[r:r + 1]), TOL, f"row {r}")


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("N,K,B", [(11008, 4096, 8), (1000, 2080, 16), (40, 96, 5)])
def test_batch_ffn_gate_up(qmm, orc, qtype, N, K, B):
    """FFN hidden state silu(x . Wg^T) * (x . Wu^T) (model.rs:713-735) for a batch: the
    pair kernel's gate and up sums are the single-weight batched GEMV's bit for bit."""
    print(f"ffn_gate_up batch type={qtype} N={N} K={K} B={B}", flush=True)
    bg = synth.weight_blocks(qtype, N, K, seed=0xB500 + N)
    bu = synth.weight_blocks(qtype, N, K, seed=0xB501 + N)
    wg, wu = qmm.QuantizedWeight(qtype, bg, N, K), qmm.QuantizedWeight(qtype, bu, N, K)
    x = synth.normal(0xB502 + B, (B, K), 1.0)
    dx, dh = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(B * N * 4)
    qmm.ffn_gate_up(wg, wu, dx, dh, B)
    h = dh.download(np.float32, (B, N))
    assert_parity(h, orc.ffn_hidden_f64(qtype, bg, bu, N, K, x), TOL, "hidden")
    g = run_gemv(qmm, wg, x).astype(np.float64)
    u = run_gemv(qmm, wu, x).astype(np.float64)
    np.testing.assert_allclose(h, orc.silu_f64(g) * u, rtol=1e-5, atol=1e-6 * float(np.max(np.abs(h))))


@pytest.mark.parametrize("qtype,N,K,B", [
    (Q4_0, 16 * 1100, 1024, 16),     # 4 tiles per workgroup (the pair cap)
    (Q4_0, 16 * 600 + 7, 512, 8),    # 3, one wave, ragged last tile
    (Q8_0, 16 * 700, 1024, 8),       # 3 (the pair cap for Q8_0 / Q6_K)
    (12, 16 * 600, 1024, 8),         # Q4_K, 3
    (14, 16 * 700 + 5, 1024, 6),     # Q6_K, 3, ragged
])
def test_batch_ffn_gate_up_tiles(qmm, orc, qtype, N, K, B):
    """The pair kernel with several row tiles per workgroup, on all N outputs of a
    NaN-filled h."""
    print(f"ffn_gate_up batch tiles type={qtype} N={N} K={K} B={B}", flush=True)
    make = (lambda sd: synth.kquant_blocks(qtype, N, K, sd)) if qtype in (12, 14) else \
        (lambda sd: synth.weight_blocks(qtype, N, K, seed=sd))
    bg, bu = make(0xB600 + N), make(0xB601 + N)
    wg, wu = qmm.QuantizedWeight(qtype, bg, N, K), qmm.QuantizedWeight(qtype, bu, N, K)
    x = synth.normal(0xB602 + B, (B, K), 1.0)
    dx, dh = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(B * N * 4)
    dh.fill(0xFF)
    qmm.ffn_gate_up(wg, wu, dx, dh, B)
    assert_parity(dh.download(np.float32, (B, N)), orc.ffn_hidden_f64(qtype, bg, bu, N, K, x), TOL, "hidden")


def test_batch_gemv_multi(qmm, orc):
    """gemv_multi with a batch runs one batched pass per weight."""
    shapes = ((4096, 4096), (1024, 4096), (1024, 4096))
    B = 12
    ws, blocks = [], []
    for i, (n, k) in enumerate(shapes):
        b = synth.weight_blocks(Q4_0, n, k, seed=0xB600 + i)
        blocks.append(b)
        ws.append(qmm.QuantizedWeight(Q4_0, b, n, k))
    x = synth.normal(0xB610, (B, 4096), 1.0)
    dx = qmm.DeviceBuffer.from_numpy(x)
    dys = [qmm.DeviceBuffer(B * w.n_rows * 4) for w in ws]
    qmm.gemv_multi(ws, dx, dys, B)
    for i, (w, b, dy) in enumerate(zip(ws, blocks, dys)):
        y = dy.download(np.float32, (B, w.n_rows))
        assert_parity(y, orc.linear_f64(Q4_0, b, w.n_rows, 4096, x), TOL, f"weight {i}")
        assert np.array_equal(y.view(np.uint32), run_gemv(qmm, w, x).view(np.uint32))


def test_batch_linearity_full_size(qmm):
    """Size-independent property at the 70B gate shape with 16 rows: y(2 x1 + x2) =
    2 y(x1) + y(x2) within fp32 reassociation, and zero rows give exact zeros."""
    N, K = 28672, 8192
    print(f"gemv batch linearity N={N} K={K}", flush=True)
    blocks = synth.weight_blocks(Q4_0, N, K, seed=0xB700, sigma=0.015)
    w = qmm.QuantizedWeight(Q4_0, blocks, N, K)
    x1 = synth.normal(0xB701, (16, K), 1.0)
    x2 = synth.normal(0xB702, (16, K), 1.0)
    y1, y2 = run_gemv(qmm, w, x1), run_gemv(qmm, w, x2)
    y12 = run_gemv(qmm, w, (np.float32(2.0) * x1 + x2).astype(np.float32))
    p = assert_parity(y12, 2.0 * y1.astype(np.float64) + y2, TOL, "linearity")
    assert p["normwise"] <= 2e-6, p
    assert np.all(run_gemv(qmm, w, np.zeros((16, K), np.float32)) == 0.0)
