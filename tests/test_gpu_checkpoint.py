"""A BitNet checkpoint in the HuggingFace layout through loom_amd.checkpoint
(ImportHFCheckpointDir, poly/hf_import.go:185-260) equals the same model built
directly from the same arrays: the importer's routing, scales, norm epsilons
and dtype decodes put every tensor where the block expects it.

The checkpoint is synthetic (no network here): microsoft offline U8
projections with BF16 weight_scale tensors, BF16 norms and embeddings, as the
BitNet-b1.58-2B-4T files store them, plus a dense F32 projection (absmean
packed on import) and an untied F32 LM head in the second case."""
import json

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H, HEADS, KV, HD, INTER, LAYERS, VOCAB = 256, 4, 2, 64, 512, 2, 300
THETA, RMS_EPS = 500000.0, 1e-6


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    from loom_amd import _lib
    assert _lib.lib().loom_amd_device_count() >= 1, "no gfx950 device visible to the library"
    return torch


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (round to nearest even), as a checkpoint stores them."""
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).view(torch.int16) \
        .numpy().view(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def ms_bytes(rng, rows: int, cols: int) -> np.ndarray:
    f = rng.integers(0, 3, (4, rows // 4, cols))
    return (f[0] | (f[1] << 2) | (f[2] << 4) | (f[3] << 6)).astype(np.uint8)


def build(tmp_path, rng, dense_o: bool, untied: bool):
    """Write the checkpoint; return its directory and the arrays it holds."""
    q, kv = HEADS * HD, KV * HD
    shapes = {"q_proj": (q, H), "k_proj": (kv, H), "v_proj": (kv, H), "o_proj": (H, q),
              "gate_proj": (INTER, H), "up_proj": (INTER, H), "down_proj": (H, INTER)}
    t, ref = {}, {"layers": []}
    emb = bf16_bits(rng.standard_normal((VOCAB, H)) * 0.05)
    t["model.embed_tokens.weight"] = ("BF16", emb.shape, emb)
    ref["emb"] = bf16_value(emb)
    fn = bf16_bits(rng.uniform(0.5, 1.5, H))
    t["model.norm.weight"] = ("BF16", fn.shape, fn)
    ref["fnorm"] = bf16_value(fn)
    if untied:
        lm = (rng.standard_normal((VOCAB, H)) * 0.05).astype(np.float32)
        t["lm_head.weight"] = ("F32", lm.shape, lm)
        ref["lm"] = lm
    for li in range(LAYERS):
        L = {}
        for nm, (rows, cols) in shapes.items():
            grp = "self_attn" if nm[0] in "qkvo" else "mlp"
            key = f"model.layers.{li}.{grp}.{nm}"
            if dense_o and li == 1 and nm == "o_proj":
                w = (rng.integers(-1, 2, (rows, cols)) * 0.0125).astype(np.float32)
                t[key + ".weight"] = ("F32", w.shape, w)
                L[nm] = ("dense", w)
                continue
            b = ms_bytes(rng, rows, cols)
            s = bf16_bits(np.array([rng.uniform(0.5, 2.0)]))
            t[key + ".weight"] = ("U8", b.shape, b)
            t[key + ".weight_scale"] = ("BF16", (1,), s)
            L[nm] = ("ms", b, float(bf16_value(s)[0]))
        for nm, n in (("input_layernorm", H), ("post_attention_layernorm", H),
                      ("self_attn.attn_sub_norm", q), ("mlp.ffn_sub_norm", INTER)):
            v = bf16_bits(rng.uniform(0.5, 1.5, n))
            t[f"model.layers.{li}.{nm}.weight"] = ("BF16", v.shape, v)
            L[nm] = bf16_value(v)
        ref["layers"].append(L)
    config = {"architectures": ["BitNetForCausalLM"], "model_type": "bitnet", "hidden_size": H,
              "num_attention_heads": HEADS, "num_key_value_heads": KV, "intermediate_size": INTER,
              "num_hidden_layers": LAYERS, "hidden_act": "relu2", "rms_norm_eps": RMS_EPS,
              "rope_theta": THETA, "vocab_size": VOCAB}
    d = tmp_path / ("dense" if dense_o else "ms") / ("untied" if untied else "tied")
    d.mkdir(parents=True)
    (d / "config.json").write_text(json.dumps(config))
    from loom_amd import checkpoint as ck
    names = sorted(t)
    half = len(names) // 2  # two shard files, as large checkpoints come
    ck.write_safetensors(str(d / "model-00001-of-00002.safetensors"), {n: t[n] for n in names[:half]})
    ck.write_safetensors(str(d / "model-00002-of-00002.safetensors"), {n: t[n] for n in names[half:]})
    return str(d), ref


def direct_model(ref, norm: str, msl: int, attn_eps: float = 1e-5, qk: bool = True):
    from loom_amd import transformer as tf
    from loom_amd.bitnet import TernaryMatrix
    q = HEADS * HD
    layers = []
    for L in ref["layers"]:
        m = {}
        for nm in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
            rows = {"q_proj": q, "k_proj": KV * HD, "v_proj": KV * HD, "o_proj": H,
                    "gate_proj": INTER, "up_proj": INTER, "down_proj": H}[nm]
            cols = {"o_proj": q, "down_proj": INTER}.get(nm, H)
            e = L[nm]
            m[nm] = (TernaryMatrix.from_float32(e[1], rows, cols) if e[0] == "dense"
                     else TernaryMatrix.from_ms_offline(e[1], rows, cols, e[2]))
        layers.append(tf.BlockWeights(m["q_proj"], m["k_proj"], m["v_proj"], m["o_proj"], m["gate_proj"],
                                      m["up_proj"], m["down_proj"], L["input_layernorm"],
                                      L["post_attention_layernorm"], L["self_attn.attn_sub_norm"],
                                      L["mlp.ffn_sub_norm"],
                                      q_norm=L.get("q_norm") if qk else None,
                                      k_norm=L.get("k_norm") if qk else None))
    cfg = tf.BlockConfig(H, HEADS, KV, HD, INTER, max_seq_len=msl, rope_theta=THETA, norm_eps=RMS_EPS,
                         attn_eps=attn_eps, ffn_eps=1e-5, ffn_activation=6, norm=norm)
    return tf.Transformer(cfg, layers, ref["emb"], ref["fnorm"], lm_head=ref.get("lm"), vocab=VOCAB,
                          final_norm_eps=1e-6)


@pytest.mark.parametrize("dense_o,untied,norm", [(False, False, "strict"), (True, True, "strict"),
                                                 (False, True, "fast")])
def test_hf_checkpoint_equals_direct_model(torch_dev, tmp_path, dense_o, untied, norm):
    from loom_amd import checkpoint as ck
    rng = np.random.default_rng(4242 + 2 * dense_o + untied)
    path, ref = build(tmp_path, rng, dense_o, untied)
    msl = 96
    got, dims = ck.load_hf_checkpoint(path, norm=norm, max_seq_len=msl)
    assert (dims.layers, dims.hidden, dims.heads, dims.kv_heads, dims.head_dim, dims.inter,
            dims.activation) == (LAYERS, H, HEADS, KV, HD, INTER, 6)
    want = direct_model(ref, norm, msl)
    ids = rng.integers(0, VOCAB, (1, 40)).astype(np.int32)
    la = got.prefill(ids, logits=True)
    lb = want.prefill(ids, logits=True)
    torch_dev.cuda.synchronize()
    assert la.cpu().numpy().tobytes() == lb.cpu().numpy().tobytes()
    ta = got.generate(ids, 12)
    tb = want.generate(ids, 12)
    assert np.array_equal(ta, tb), (ta, tb)
    got.release()
    want.release()


@pytest.mark.parametrize("norm", ["strict", "fast"])
def test_hf_checkpoint_qk_norm(torch_dev, tmp_path, norm):
    # q_norm / k_norm tensors become the layers' QNormWeight / KNormWeight
    # (poly/prefix_safetensor.go:240-244, 425-434), applied with eps 1e-6: the
    # import leaves the MHA layer's RMSNormEps unset (poly/hf_decoder.go:43-51,
    # poly/mha.go:19-24).  The model equals the directly built one with the
    # same norms and attn_eps 0 (both defaults), and differs from it without
    # them.
    from loom_amd import checkpoint as ck
    rng = np.random.default_rng(7)
    path, ref = build(tmp_path, rng, False, False)
    import glob
    import os
    f = sorted(glob.glob(os.path.join(path, "*.safetensors")))[0]
    t = {n: (s.dtype, s.shape, np.array(s.raw)) for n, s in ck.read_safetensors(f).items()}
    qn = [bf16_bits(rng.uniform(0.5, 1.5, HD)) for _ in range(LAYERS)]
    kn = [bf16_bits(rng.uniform(0.5, 1.5, KV * HD)) for _ in range(LAYERS)]
    for li in range(LAYERS):
        t[f"model.layers.{li}.self_attn.q_norm.weight"] = ("BF16", qn[li].shape, qn[li])
        t[f"model.layers.{li}.self_attn.k_norm.weight"] = ("BF16", kn[li].shape, kn[li])
    ck.write_safetensors(f, t)
    msl = 96
    got, _ = ck.load_hf_checkpoint(path, norm=norm, max_seq_len=msl)
    for li in range(LAYERS):
        ref["layers"][li]["q_norm"] = bf16_value(qn[li])
        ref["layers"][li]["k_norm"] = bf16_value(kn[li])
    want = direct_model(ref, norm, msl, attn_eps=0.0)
    plain = direct_model(ref, norm, msl, attn_eps=0.0, qk=False)
    ids = rng.integers(0, VOCAB, (1, 30)).astype(np.int32)
    la = got.prefill(ids, logits=True)
    lb = want.prefill(ids, logits=True)
    lc = plain.prefill(ids, logits=True)
    torch_dev.cuda.synchronize()
    assert la.cpu().numpy().tobytes() == lb.cpu().numpy().tobytes()
    assert la.cpu().numpy().tobytes() != lc.cpu().numpy().tobytes()
    assert np.array_equal(got.generate(ids, 8), want.generate(ids, 8))
    for m in (got, want, plain):
        m.release()
