"""The loader's raw-block path on the GPU: projections read from GGUF files (both
dialects) are uploaded without dequantization and must give exactly what the same
blocks give through openmini_qmm_upload; get_tensor_data_by_ref on the GPU is
bit-identical to the reference's dequantization (gguf.rs:2062-2110)."""
import numpy as np
import pytest

import gguf_fixtures as fx
from openmini_qmm import gguf as G
from openmini_qmm import synth

pytestmark = pytest.mark.gpu
Q4_0, Q8_0 = 2, 7


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("dialect", ["reference", "standard"])
@pytest.mark.parametrize("qtype", [Q4_0, Q8_0])
def test_projection_from_file_matches_direct_upload(qmm, orc, tmp_path, dialect, qtype):
    N, K = 304, 4096 + 96
    blocks = synth.weight_blocks(qtype, N, K, seed=11 + qtype)
    path = tmp_path / "layer.gguf"
    path.write_bytes(fx.build([("general.architecture", fx.STRING, "llama")],
                              [("model.layers.0.ffn.up_proj", [K, N], qtype, blocks.tobytes())], dialect))
    print(f"gguf upload type={qtype} dialect={dialect}", flush=True)
    g = G.GgufFile(str(path))
    w_file = g.upload_weight("model.layers.0.ffn.up_proj")
    w_direct = qmm.QuantizedWeight(qtype, blocks, N, K)
    assert (w_file.n_rows, w_file.k_cols) == (N, K)
    assert np.array_equal(bits(w_file.dequantize()), bits(orc.dequantize(qtype, blocks, N * K).reshape(N, K)))
    x = synth.normal(5, (3, K), 1.0)
    dx = qmm.DeviceBuffer.from_numpy(x)
    y1, y2 = qmm.DeviceBuffer(3 * N * 4), qmm.DeviceBuffer(3 * N * 4)
    w_file.gemv(dx, y1, 3)
    w_direct.gemv(dx, y2, 3)
    assert np.array_equal(y1.download(np.float32, (3, N)), y2.download(np.float32, (3, N)))


def test_tensor_by_ref_every_layout(qmm, orc, tmp_path):
    rng = np.random.default_rng(3)
    layouts = {0: 4, 1: 2, 2: 18, 3: 20, 7: 34, 10: 68, 11: 162, 12: 144, 13: 176, 14: 210, 15: 258}
    tensors = []
    for t, bpb in layouts.items():
        bs = 1 if t < 2 else 32 if t < 10 else 256
        nblk = 40
        raw = rng.integers(0, 256, nblk * bpb, dtype=np.uint8)
        if t == 0:
            raw = rng.standard_normal(nblk).astype(np.float32).view(np.uint8)
        elif t == 1:
            raw = rng.standard_normal(nblk).astype(np.float16).view(np.uint8)
        else:
            for f in ((0, 2) if t in (3, 10, 12, 13) else (0,)):
                raw[f + 1::bpb] &= 0x7B
        tensors.append((f"t{t}", [nblk * bs], t, raw.tobytes()))
    path = tmp_path / "all.gguf"
    path.write_bytes(fx.build([], tensors, "reference"))
    g = G.GgufFile(str(path))
    for name, dims, t, raw in tensors:
        got = g.get_tensor_data_by_ref(g.tensors[name])
        ref = orc.dequantize(t, np.frombuffer(raw, np.uint8), dims[0])
        assert np.array_equal(bits(got), bits(ref)), name
    with pytest.raises(G.GgufError):  # a 1-D tensor is not a linear weight
        g.upload_weight("t12")


def test_loader_layer(qmm, orc, tmp_path):
    """QuantizedWeightLoader.load_attention_weights / load_ffn_weights over one small
    Llama-shaped layer (quant_loader.rs:95-138), weights staying quantized."""
    H, F = 256, 704
    shapes = {"attention.q_proj": (H, H), "attention.k_proj": (H, H), "attention.v_proj": (H, H),
              "attention.o_proj": (H, H), "ffn.gate_proj": (F, H), "ffn.up_proj": (F, H), "ffn.down_proj": (H, F)}
    blocks = {k: synth.weight_blocks(Q4_0, n, kk, seed=i) for i, (k, (n, kk)) in enumerate(shapes.items())}
    path = tmp_path / "llama_layer.gguf"
    path.write_bytes(fx.build([("general.architecture", fx.STRING, "llama")],
                              [(f"model.layers.0.{k}", [kk, n], Q4_0, blocks[k].tobytes())
                               for k, (n, kk) in shapes.items()], "standard"))
    loader = G.QuantizedWeightLoader.open(str(path))
    attn, ffn = loader.load_attention_weights(0), loader.load_ffn_weights(0)
    x = synth.normal(9, (1, H), 1.0)
    for name, w in list(attn.items()) + list(ffn.items()):
        key = ("attention." if name in attn else "ffn.") + name
        n, kk = shapes[key]
        assert (w.n_rows, w.k_cols) == (n, kk)
        xi = x if kk == H else synth.normal(10, (1, kk), 1.0)
        y = qmm.linear(xi, w)
        ref = orc.linear_f64(Q4_0, blocks[key], n, kk, xi)
        assert np.max(np.abs(y - ref)) <= 1e-3 * np.max(np.abs(ref))
    with pytest.raises(G.GgufError, match="Tensor not found"):
        loader.load_tensor("model.layers.1.ffn.up_proj")


@pytest.mark.parametrize("ttype,shift,ok", [(0, 0, True), (0, 2, False), (0, 4, True),
                                           (1, 0, True), (1, 1, False), (1, 2, True)])
def test_tensor_by_ref_f32_f16_alignment(qmm, tmp_path, ttype, shift, ok):
    """get_tensor_data_by_ref casts F32 / F16 data in place and refuses a start that is
    not 4- / 2-byte aligned in the file ("F32 data is not properly aligned",
    gguf.rs:2076-2078, 2090-2092); the reference dialect places data anywhere."""
    vals = np.array([0.5, -1.25, 3.0, 1e-3], np.float32)
    raw = vals.tobytes() if ttype == 0 else vals.astype(np.float16).tobytes()
    path = tmp_path / "plain.gguf"
    path.write_bytes(fx.build([], [("t", [4], ttype, raw)], "reference", data_shift=shift))
    g = G.GgufFile(str(path), G.REFERENCE)
    if ok:
        got = g.get_tensor_data_by_ref(g.tensors["t"])
        want = vals if ttype == 0 else vals.astype(np.float16).astype(np.float32)
        assert np.array_equal(bits(got), bits(want))
    else:
        name = "F32" if ttype == 0 else "F16"
        with pytest.raises(G.GgufError, match=f"{name} data is not properly aligned"):
            g.get_tensor_data_by_ref(g.tensors["t"])


@pytest.mark.parametrize("dialect", ["reference", "standard"])
def test_load_layer(qmm, orc, tmp_path, dialect):
    """QuantizedModelLoader::load_layer (quant_loader.rs:439-484) on a one-layer file:
    the seven projections by the reference's names come back as GPU weights that equal
    direct uploads of the same blocks (dequantized bit for bit, and a GEMV against the
    oracle), the two norm vectors as f32 bit-identical to the reference's
    dequantization (one stored F32, one F16); MLA / MoE tensors are reported, not
    loaded; a missing norm is "Tensor not found"."""
    H, I = 256, 704
    rng = np.random.default_rng(21)
    shapes = {"attention.q_proj": (H, H), "attention.k_proj": (64, H), "attention.v_proj": (64, H),
              "attention.o_proj": (H, H), "ffn.gate_proj": (I, H), "ffn.up_proj": (I, H),
              "ffn.down_proj": (H, I)}
    qtypes = {name: (Q4_0 if i % 2 == 0 else Q8_0) for i, name in enumerate(shapes)}
    blocks = {name: synth.weight_blocks(qtypes[name], n, k, seed=0x1A00 + i)
              for i, (name, (n, k)) in enumerate(shapes.items())}
    ln_in = rng.standard_normal(H).astype(np.float32)
    ln_post = rng.standard_normal(H).astype(np.float16)
    tensors = [(f"model.layers.0.{name}", [k, n], qtypes[name], blocks[name].tobytes())
               for name, (n, k) in shapes.items()]
    tensors += [("model.layers.0.input_layernorm", [H], 0, ln_in.tobytes()),
                ("model.layers.0.post_attention_layernorm", [H], 1, ln_post.tobytes()),
                ("model.layers.0.moe.router", [H], 0, ln_in.tobytes())]
    path = tmp_path / "one_layer.gguf"
    path.write_bytes(fx.build([("general.architecture", fx.STRING, "llama")], tensors, dialect))
    print(f"load_layer dialect={dialect}", flush=True)
    loader = G.QuantizedWeightLoader.open(str(path))
    layer = loader.load_layer(0)
    assert sorted(layer.attention) == ["k_proj", "o_proj", "q_proj", "v_proj"]
    assert sorted(layer.ffn) == ["down_proj", "gate_proj", "up_proj"]
    x = synth.normal(0x1A10, (2, I), 1.0)
    for group, part in (("attention", layer.attention), ("ffn", layer.ffn)):
        for p, w in part.items():
            name = f"{group}.{p}"
            n, k = shapes[name]
            assert (w.n_rows, w.k_cols, int(w.tensor_type)) == (n, k, qtypes[name])
            assert np.array_equal(bits(w.dequantize()),
                                  bits(orc.dequantize(qtypes[name], blocks[name], n * k).reshape(n, k)))
            dx, dy = qmm.DeviceBuffer.from_numpy(np.ascontiguousarray(x[:, :k])), qmm.DeviceBuffer(2 * n * 4)
            w.gemv(dx, dy, 2)
            ref = orc.linear_f64(qtypes[name], blocks[name], n, k, x[:, :k])
            assert np.max(np.abs(dy.download(np.float32, (2, n)) - ref)) <= 1e-3 * np.max(np.abs(ref))
    assert np.array_equal(bits(layer.input_layernorm), bits(ln_in))
    assert np.array_equal(bits(layer.post_attention_layernorm), bits(ln_post.astype(np.float32)))
    assert layer.has_moe and not layer.has_mla
    with pytest.raises(G.GgufError, match="Tensor not found"):
        loader.load_layer(1)
