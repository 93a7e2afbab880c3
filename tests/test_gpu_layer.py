"""The projections of one layer on the GPU: grouped q/k/v GEMV (prepare_qkv,
model.rs:1392-1394) and the FFN's silu(gate) * up (FFNWeights::forward,
model.rs:713-735), against the fp64 oracle at the tolerance of tests/parity.py
(1e-3 normwise and elementwise), plus exact agreement with the single-weight GEMV
that shares their kernel."""
import numpy as np
import pytest

from openmini_qmm import synth
from parity import TOL, assert_parity

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def _gemv(qmm, w, x):
    dx = qmm.DeviceBuffer.from_numpy(x)
    dy = qmm.DeviceBuffer(x.shape[0] * w.n_rows * 4)
    w.gemv(dx, dy, x.shape[0])
    return dy.download(np.float32, (x.shape[0], w.n_rows))


def _weights(qmm, qtype, shapes, seed, sigma=0.02):
    out = []
    for i, (n, k) in enumerate(shapes):
        blocks = synth.weight_blocks(qtype, n, k, seed=seed + 7 * i, sigma=sigma)
        out.append((qmm.QuantizedWeight(qtype, blocks, n, k), blocks))
    return out


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("shapes,B", [
    (((4096, 4096), (4096, 4096), (4096, 4096)), 1),   # Llama-7B q / k / v
    (((4096, 4096), (1024, 4096), (1024, 4096)), 3),   # grouped-query k / v
    (((1000, 96), (37, 96), (5, 96), (130, 96)), 4),   # ragged N, four weights, small K
    (((300, 2080),), 7),                               # one weight, batch sliced by 4
    (((16, 8192), (48, 8192)), 2),                     # few tiles, long K
])
def test_gemv_multi(qmm, orc, qtype, shapes, B):
    print(f"gemv_multi type={qtype} shapes={shapes} B={B}", flush=True)
    K = shapes[0][1]
    ws = _weights(qmm, qtype, shapes, seed=0x9100 + B + len(shapes))
    x = synth.normal(0x9200 + B, (B, K), 1.0)
    dx = qmm.DeviceBuffer.from_numpy(x)
    dys = [qmm.DeviceBuffer(B * w.n_rows * 4) for w, _ in ws]
    qmm.gemv_multi([w for w, _ in ws], dx, dys, B)
    for i, ((w, blocks), dy) in enumerate(zip(ws, dys)):
        y = dy.download(np.float32, (B, w.n_rows))
        assert_parity(y, orc.linear_f64(qtype, blocks, w.n_rows, K, x), TOL, f"weight {i}")
        # the same kernel per tile: identical to the single-weight launch bit for bit
        assert np.array_equal(y.view(np.uint32), _gemv(qmm, w, x).view(np.uint32)), f"weight {i}"


def test_attention_project_qkv(qmm, orc):
    ws = _weights(qmm, Q4_0, ((4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096)), seed=0x9300)
    attn = qmm.AttentionWeights(*[w for w, _ in ws])
    x = synth.normal(0x9301, (2, 4096), 1.0)
    outs = attn.project_qkv(x)
    for (w, blocks), y in zip(ws[:3], outs):
        assert_parity(y, orc.linear_f64(Q4_0, blocks, w.n_rows, 4096, x), TOL, "qkv")
    o = attn.project_o(x)
    assert_parity(o, orc.linear_f64(Q4_0, ws[3][1], 4096, 4096, x), TOL, "o_proj")


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("N,K,B", [(11008, 4096, 1), (11008, 4096, 4), (1000, 2080, 6), (5, 64, 1)])
def test_ffn_gate_up_gemv(qmm, orc, qtype, N, K, B):
    print(f"ffn_gate_up type={qtype} N={N} K={K} B={B}", flush=True)
    (wg, bg), (wu, bu) = _weights(qmm, qtype, ((N, K), (N, K)), seed=0x9400 + N + B)
    x = synth.normal(0x9401 + B, (B, K), 1.0)
    dx, dh = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(B * N * 4)
    qmm.ffn_gate_up(wg, wu, dx, dh, B)
    h = dh.download(np.float32, (B, N))
    assert_parity(h, orc.ffn_hidden_f64(qtype, bg, bu, N, K, x), TOL, "hidden")
    # composition: silu(g) * u from the two single GEMVs, fp32 epilogue vs fp64 here
    g, u = _gemv(qmm, wg, x).astype(np.float64), _gemv(qmm, wu, x).astype(np.float64)
    np.testing.assert_allclose(h, orc.silu_f64(g) * u, rtol=1e-5,
                               atol=1e-6 * float(np.max(np.abs(h))))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
@pytest.mark.parametrize("N,K,M", [(11008, 4096, 128), (11008, 4096, 512), (1000, 2080, 77), (48, 96, 300)])
def test_ffn_gate_up_bf16(qmm, orc, qtype, N, K, M):
    """Prefill FFN hidden state through the GEMM's SwiGLU epilogue.  At the full
    Llama-7B sizes the fp64 oracle runs on a sample of rows (first, last and random
    ones; a row of h depends only on its own x row); every row is still checked
    against the composition of the two plain GEMMs below."""
    print(f"ffn_gate_up_bf16 type={qtype} N={N} K={K} M={M}", flush=True)
    (wg, bg), (wu, bu) = _weights(qmm, qtype, ((N, K), (N, K)), seed=0x9500 + N + M)
    xb = synth.to_bf16_bits(synth.normal(0x9501 + M, (M, K), 1.0))
    dx, dh = qmm.DeviceBuffer.from_numpy(xb), qmm.DeviceBuffer(M * N * 4)
    qmm.ffn_gate_up_bf16(wg, wu, dx, dh, M)
    h = dh.download(np.float32, (M, N))
    rows = np.arange(M)
    if M * N * K > (1 << 31):
        rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M + N).integers(0, M, 6)]))
    assert_parity(h[rows], orc.ffn_hidden_bf16x_f64(qtype, bg, bu, N, K, xb[rows]), TOL, "hidden bf16")
    # composition against the plain GEMM of each weight
    dg = qmm.DeviceBuffer(M * N * 4)
    wg.gemm_bf16(dx, dg, M)
    wu.gemm_bf16(dx, dh, M)
    g = dg.download(np.float32, (M, N)).astype(np.float64)
    u = dh.download(np.float32, (M, N)).astype(np.float64)
    np.testing.assert_allclose(h, orc.silu_f64(g) * u, rtol=1e-5,
                               atol=1e-6 * float(np.max(np.abs(h))))


@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_ffn_forward_llama7b(qmm, orc, qtype):
    """FFNWeights::forward at Llama-7B shape: hidden 4096, intermediate 11008."""
    H, I = 4096, 11008
    print(f"ffn forward type={qtype}", flush=True)
    (wg, bg), (wu, bu), (wd, bd) = _weights(qmm, qtype, ((I, H), (I, H), (H, I)), seed=0x9600 + qtype)
    ffn = qmm.FFNWeights(wg, wu, wd)
    x = synth.normal(0x9601, (3, H), 1.0)
    out = ffn.forward(x)
    h_ref = orc.ffn_hidden_f64(qtype, bg, bu, I, H, x)
    assert_parity(ffn.hidden(x), h_ref, TOL, "hidden")
    # the down projection consumes the kernel's own fp32 hidden state; its oracle is
    # fed the same state, and the whole chain against the fp64 chain is also gated
    h = ffn.hidden(x)
    assert_parity(out, orc.linear_f64(qtype, bd, H, I, h), TOL, "down")
    assert_parity(out, orc.linear_f64(qtype, bd, H, I, h_ref.astype(np.float32)), TOL, "chain")


def test_layer_prefill_rows(qmm, orc):
    """The host-array layer methods at prefill sizes (from GEMM_MIN_ROWS rows on they run
    the fp32-activation GEMMs): FFNWeights.forward / hidden and AttentionWeights
    project_qkv / project_o at 160 rows of a 1024-hidden, 2816-intermediate layer."""
    H, I, M = 1024, 2816, 160
    assert M >= qmm.GEMM_MIN_ROWS
    print(f"layer prefill rows M={M}", flush=True)
    (wg, bg), (wu, bu), (wd, bd) = _weights(qmm, Q4_0, ((I, H), (I, H), (H, I)), seed=0x9650)
    ffn = qmm.FFNWeights(wg, wu, wd)
    x = synth.normal(0x9651, (M, H), 1.0)
    h = ffn.hidden(x)
    assert_parity(h, orc.ffn_hidden_f64(Q4_0, bg, bu, I, H, x), TOL, "hidden")
    out = ffn.forward(x)
    assert_parity(out, orc.linear_f64(Q4_0, bd, H, I, h), TOL, "down")
    ws = _weights(qmm, Q8_0, ((H, H), (256, H), (256, H), (H, H)), seed=0x9652)
    attn = qmm.AttentionWeights(*[w for w, _ in ws])
    for (w, blocks), y in zip(ws[:3], attn.project_qkv(x)):
        assert_parity(y, orc.linear_f64(Q8_0, blocks, w.n_rows, H, x), TOL, "qkv")
    assert_parity(attn.project_o(x), orc.linear_f64(Q8_0, ws[3][1], H, H, x), TOL, "o_proj")


@pytest.mark.parametrize("M", [64, 100])
def test_layer_mixed_routing(qmm, orc, M):
    """Gate / up of 10240 rows over a short K take the fp32 GEMM from GEMM_MIN_ROWS_LOW
    rows, the down projection (few rows, long K) keeps the decode GEMVs below
    GEMM_MIN_ROWS: between the two, FFNWeights.forward runs the GEMM pair and then the
    down GEMV on its hidden state, and both halves meet the oracle."""
    H, I = 512, 10240
    print(f"layer mixed routing M={M}", flush=True)
    (wg, bg), (wu, bu), (wd, bd) = _weights(qmm, Q4_0, ((I, H), (I, H), (H, I)), seed=0x9660)
    assert wg.prefill_gemm(M) and not wd.prefill_gemm(M)
    ffn = qmm.FFNWeights(wg, wu, wd)
    x = synth.normal(0x9661 + M, (M, H), 1.0)
    h = ffn.hidden(x)
    assert_parity(h, orc.ffn_hidden_f64(Q4_0, bg, bu, I, H, x), TOL, "hidden")
    out = ffn.forward(x)
    assert np.all(np.isfinite(out))
    assert_parity(out, orc.linear_f64(Q4_0, bd, H, I, h), TOL, "down")


def test_ffn_gate_up_rejects_mismatched_pair(qmm):
    (wg, _), (wu, _) = _weights(qmm, Q4_0, ((64, 128), (48, 128)), seed=0x9700)
    dx, dh = qmm.DeviceBuffer(128 * 4), qmm.DeviceBuffer(64 * 4)
    with pytest.raises(qmm.QmmError) as e:
        qmm.ffn_gate_up(wg, wu, dx, dh, 1)
    assert e.value.status == -2
    (w8, _), = _weights(qmm, Q8_0, ((64, 128),), seed=0x9701)
    with pytest.raises(qmm.QmmError):
        qmm.ffn_gate_up(wg, w8, dx, dh, 1)
    with pytest.raises(qmm.QmmError):
        qmm.gemv_multi([wg, w8], dx, [dh, dh], 1)
    (wk, _), = _weights(qmm, Q4_0, ((64, 256),), seed=0x9702)
    with pytest.raises(qmm.QmmError):
        qmm.gemv_multi([wg, wk], dx, [dh, dh], 1)
    with pytest.raises(qmm.QmmError):
        qmm.gemv_multi([wg] * 5, dx, [dh] * 5, 1)


def test_ffn_gate_up_non_finite_activation(qmm):
    """A non-finite activation row gives a non-finite hidden row; other rows stay finite."""
    (wg, _), (wu, _) = _weights(qmm, Q4_0, ((64, 128), (64, 128)), seed=0x9800)
    x = synth.normal(0x9801, (2, 128), 1.0)
    x[1, 5] = np.inf
    dx, dh = qmm.DeviceBuffer.from_numpy(x), qmm.DeviceBuffer(2 * 64 * 4)
    qmm.ffn_gate_up(wg, wu, dx, dh, 2)
    h = dh.download(np.float32, (2, 64))
    assert np.all(np.isfinite(h[0])) and not np.any(np.isfinite(h[1]))
