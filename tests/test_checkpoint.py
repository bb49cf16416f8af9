"""The HuggingFace-layout checkpoint importer (loom_amd/checkpoint.py) on the
host: tensor routing (decodeHFPrefixRouting, poly/prefix_safetensor.go:195-250),
config parsing (ParseHFDecoderDims, poly/hf_import.go:130-178), global-tensor
patterns (poly/prefix_safetensor.go:14-76) and the safetensors reader with
loom's dtype decodes (poly/safetensors.go:624-781), the reader pinned against
the safetensors library's own writer and torch's bf16 conversion."""
import json

import numpy as np
import pytest

from loom_amd import checkpoint as ck


@pytest.mark.parametrize("name,want", [
    ("model.layers.0.input_layernorm.weight", (0, 0, "")),
    ("model.layers.3.post_attention_layernorm.weight", (3, 2, "")),
    ("model.layers.1.self_attn.q_proj.weight", (1, 1, "q")),
    ("model.layers.1.self_attn.k_proj.weight", (1, 1, "k")),
    ("model.layers.1.self_attn.v_proj.weight_scale", (1, 1, "v_scale")),
    ("model.layers.12.self_attn.o_proj.weight", (12, 1, "o")),
    ("model.layers.2.self_attn.attn_sub_norm.weight", (2, 1, "inner_norm")),
    ("model.layers.2.self_attn.q_norm.weight", (2, 1, "qn")),
    ("model.layers.2.self_attn.k_norm.weight", (2, 1, "kn")),
    ("model.layers.2.self_attn.rotary_emb.inv_freq", (2, 1, "")),
    ("model.layers.4.mlp.gate_proj.weight", (4, 3, "g")),
    ("model.layers.4.mlp.up_proj.weight_scale", (4, 3, "u_scale")),
    ("model.layers.4.mlp.down_proj.weight", (4, 3, "d")),
    ("model.layers.4.mlp.ffn_sub_norm.weight", (4, 3, "inner_norm")),
    ("transformer.h.7.ln_1.weight", (7, 0, "")),
    ("transformer.h.7.ln_2.weight", (7, 2, "")),
    ("transformer.h.7.attn.c_attn.weight", (7, 1, "")),
    ("transformer.h.7.mlp.w1.weight", (7, 3, "g")),
    ("transformer.h.7.mlp.w3.weight", (7, 3, "u")),
    ("transformer.h.7.mlp.w2.weight", (7, 3, "d")),
    ("model.embed_tokens.weight", None),
    ("model.norm.weight", None),
    ("model.layers.x.mlp.up_proj.weight", None),
    ("model.layers.5.something_else.weight", None),
])
def test_route(name, want):
    assert ck.route(name) == want


def test_decoder_dims():
    cfg = {"num_attention_heads": 20, "num_key_value_heads": 5, "hidden_size": 2560,
           "intermediate_size": 6912, "num_hidden_layers": 30, "hidden_act": "relu2",
           "rms_norm_eps": 1e-5, "rope_theta": 500000.0}
    d = ck.decoder_dims(cfg)
    assert (d.layers, d.hidden, d.heads, d.kv_heads, d.head_dim, d.inter) == (30, 2560, 20, 5, 128, 6912)
    assert (d.rms_eps, d.theta, d.activation) == (1e-5, 500000.0, ck.ACT_RELU2)
    # defaults: kv = heads, SiLU, eps 1e-6, theta 10000; layer count from the tensor names
    d = ck.decoder_dims({"num_attention_heads": 4, "hidden_size": 256, "intermediate_size": 512,
                         "hidden_act": "silu", "head_dim": 32},
                        ["model.layers.0.mlp.up_proj.weight", "model.layers.6.input_layernorm.weight"])
    assert (d.layers, d.kv_heads, d.head_dim, d.activation, d.rms_eps, d.theta) == \
        (7, 4, 32, ck.ACT_SILU, 1e-6, 10000.0)
    with pytest.raises(ValueError):
        ck.decoder_dims({"hidden_size": 256, "intermediate_size": 512})
    with pytest.raises(ValueError):
        ck.decoder_dims({"num_attention_heads": 4, "hidden_size": 256, "intermediate_size": 512})


def test_find_global_exact_then_suffix():
    t = lambda: ck.StoredTensor("F32", (1,), np.zeros(4, np.uint8))  # noqa: E731
    a, b, c = t(), t(), t()
    assert ck.find_global({"model.embed_tokens.weight": a, "x.embed_tokens.weight": b}, "embeddings") is a
    assert ck.find_global({"foo.model.embed_tokens.weight": b}, "embeddings") is b
    assert ck.find_global({"transformer.ln_f.weight": c}, "final_norm") is c
    assert ck.find_global({"model.embed_tokens.weight": a}, "lm_head") is None


def test_reader_matches_safetensors_library(tmp_path):
    from safetensors.numpy import save_file
    rng = np.random.default_rng(5)
    ref = {"a": rng.standard_normal((3, 5)).astype(np.float32),
           "b": rng.standard_normal(7).astype(np.float16),
           "c": rng.integers(0, 256, (4, 6)).astype(np.uint8),
           "d": rng.integers(-2 ** 31, 2 ** 31, 9).astype(np.int32),
           "e": rng.standard_normal(4).astype(np.float64)}
    p = str(tmp_path / "t.safetensors")
    save_file(ref, p)
    got = ck.read_safetensors(p)
    assert set(got) == set(ref)
    assert got["a"].dtype == "F32" and got["a"].shape == (3, 5)
    np.testing.assert_array_equal(got["a"].to_float32().reshape(3, 5), ref["a"])
    np.testing.assert_array_equal(got["b"].to_float32(), ref["b"].astype(np.float32))
    np.testing.assert_array_equal(got["c"].as_bytes().reshape(4, 6), ref["c"])
    np.testing.assert_array_equal(got["d"].to_float32(), ref["d"].astype(np.float32))
    np.testing.assert_array_equal(got["e"].to_float32(), ref["e"].astype(np.float32))


def test_reader_bf16_matches_torch(tmp_path):
    torch = pytest.importorskip("torch")
    from safetensors.torch import save_file
    x = torch.randn(257, dtype=torch.float32) * 1e3
    x[0], x[1], x[2] = float("inf"), 0.0, -0.0
    xb = x.to(torch.bfloat16)
    p = str(tmp_path / "b.safetensors")
    save_file({"w": xb}, p)
    got = ck.read_safetensors(p)["w"]
    assert got.dtype == "BF16"
    want = xb.to(torch.float32).numpy()
    assert np.array_equal(got.to_float32().view(np.uint32), want.view(np.uint32))


def test_writer_round_trip(tmp_path):
    rng = np.random.default_rng(9)
    bf = rng.integers(0, 2 ** 16, 10).astype(np.uint16)
    u8 = rng.integers(0, 256, (2, 3)).astype(np.uint8)
    p = str(tmp_path / "w.safetensors")
    ck.write_safetensors(p, {"x": ("BF16", (10,), bf), "y": ("U8", (2, 3), u8)})
    torch = pytest.importorskip("torch")
    from safetensors import safe_open
    with safe_open(p, framework="pt") as f:
        np.testing.assert_array_equal(f.get_tensor("y").numpy(), u8)
        xt = f.get_tensor("x").to(torch.float32).numpy()
    got = ck.read_safetensors(p)
    want = bf.astype(np.uint32) << 16
    assert np.array_equal(got["x"].to_float32().view(np.uint32), want)
    assert np.array_equal(xt.view(np.uint32), want)


def test_reader_rejects_bad_ranges(tmp_path):
    p = tmp_path / "bad.safetensors"
    h = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}).encode()
    p.write_bytes(len(h).to_bytes(8, "little") + h + b"\0" * 12)
    with pytest.raises(ValueError):
        ck.read_safetensors(str(p))
