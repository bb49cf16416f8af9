"""BitNet checkpoints in the HuggingFace layout, loaded onto the device.

This follows loom's importer of a HuggingFace snapshot directory
(config.json + *.safetensors):

- ``ImportHFCheckpointDir`` (poly/hf_import.go:185-260): globals first, then
  the decoder blocks;
- ``ParseHFDecoderDims`` (poly/hf_import.go:130-178): the block shape from
  config.json (``hidden_act`` "relu2" selects ReLU^2, anything else SiLU;
  ``rms_norm_eps`` defaults to 1e-6, ``rope_theta`` to 10000);
- ``InitHFDecoderBlocks`` (poly/hf_decoder.go:20-67): ``rms_norm_eps`` goes to
  the two block RMSNorms only; the MHA and SwiGLU inner norms keep eps 0, for
  which loom's norms use 1e-5 (``bitNetRMSNormFloat64Weighted`` and
  ``bitNetRMSNormTensorRowWeighted``, poly/bitnet_cpu.go:868-900);
- ``NewPrefixWeightMapper`` / ``MapWeights`` (poly/prefix_safetensor.go:14-122):
  embeddings, final norm and LM head by name (exact, then suffix match), the
  head tied to the embeddings when the checkpoint has none;
- ``decodeHFPrefixRouting`` and ``copyWeights`` (poly/prefix_safetensor.go:
  195-345): each ``layers.<i>`` tensor to its block slot and role; a projection
  whose element count is rows*cols/4 is the microsoft/bitnet-b1.58 offline U8
  layout (``SetMicrosoftBitNetPackedMatrix``, poly/bitnet_cpu.go:1005-1026,
  scale from the matching ``weight_scale`` tensor, 1 when absent or zero:
  poly/bitnet_cpu.go:979-1003), any other a dense fp32 master packed by the
  absmean rule;
- the final norm's eps is 1e-6 (poly/transformer.go:97-108).

The safetensors files are read here (8-byte header length, JSON header, raw
payloads; memory-mapped), with loom's dtype decodes (poly/safetensors.go:
624-781): BF16 is the 16 high bits of an fp32, F16 widens exactly, F64 and the
integer types round to the nearest fp32.  Nothing in a file is executed.

Per-head Q/K RMSNorm weights (``q_norm`` / ``k_norm``) become the block's
QNormWeight / KNormWeight as loom stores them (any length,
poly/prefix_safetensor.go:425-434); the block applies them before RoPE
(poly/mha.go:285-290) with eps 1e-6, since the import leaves the MHA layer's
RMSNormEps unset (mhaQKNormEpsilon, poly/mha.go:19-24; InitHFDecoderBlocks,
poly/hf_decoder.go:43-51).
"""
from __future__ import annotations

import dataclasses
import glob
import json
import os
import re

import numpy as np

from . import transformer as tf
from .bitnet import TernaryMatrix

ACT_SILU, ACT_RELU2 = 1, 6

_DTYPES = {
    "F64": (np.float64, 8), "F32": (np.float32, 4), "F16": (np.float16, 2), "BF16": (np.uint16, 2),
    "I64": (np.int64, 8), "I32": (np.int32, 4), "I16": (np.int16, 2), "I8": (np.int8, 1),
    "U64": (np.uint64, 8), "U32": (np.uint32, 4), "U16": (np.uint16, 2), "U8": (np.uint8, 1),
}


@dataclasses.dataclass
class StoredTensor:
    """One tensor of a safetensors file: dtype string, shape and its raw
    little-endian payload (a view into the memory-mapped file)."""
    dtype: str
    shape: tuple
    raw: np.ndarray  # uint8

    @property
    def size(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    def to_float32(self) -> np.ndarray:
        """loom's decodeTensorData (poly/safetensors.go:624-750)."""
        if self.dtype not in _DTYPES:
            raise ValueError(f"unsupported safetensors dtype {self.dtype}")
        np_t, _ = _DTYPES[self.dtype]
        v = self.raw.view(np.dtype(np_t).newbyteorder("<"))
        if self.dtype == "BF16":
            return (v.astype(np.uint32) << 16).view(np.float32)
        return v.astype(np.float32)

    def as_bytes(self) -> np.ndarray:
        if self.dtype not in ("U8", "I8"):
            raise ValueError(f"expected a byte tensor, got {self.dtype}")
        return self.raw


def read_safetensors(path: str) -> dict[str, StoredTensor]:
    """Every tensor of one safetensors file, memory-mapped (no copy until a
    tensor is decoded)."""
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise ValueError(f"{path}: not a safetensors file (short header)")
        n = int.from_bytes(head, "little")
        if n > 256 << 20:
            raise ValueError(f"{path}: safetensors header size unreasonable: {n}")
        header = json.loads(f.read(n))
    data = np.memmap(path, np.uint8, mode="r", offset=8 + n) if os.path.getsize(path) > 8 + n \
        else np.zeros(0, np.uint8)
    out = {}
    for name, meta in header.items():
        if name == "__metadata__":
            continue
        dtype, shape = meta["dtype"], tuple(meta["shape"])
        b0, b1 = meta["data_offsets"]
        if dtype not in _DTYPES:
            raise ValueError(f"{path}: tensor {name}: unsupported dtype {dtype}")
        t = StoredTensor(dtype, shape, data[b0:b1])
        if b1 - b0 != t.size * _DTYPES[dtype][1] or b1 > data.size:
            raise ValueError(f"{path}: tensor {name}: byte range {b0}..{b1} does not hold "
                             f"{t.size} x {dtype}")
        out[name] = t
    return out


def write_safetensors(path: str, tensors: dict[str, tuple[str, tuple, np.ndarray]]) -> None:
    """Write {name: (dtype, shape, raw payload)} as a safetensors file (used to
    build checkpoints for tests; BF16 payloads are uint16 arrays)."""
    header, blobs, off = {}, [], 0
    for name, (dtype, shape, arr) in tensors.items():
        b = np.ascontiguousarray(arr).view(np.uint8).reshape(-1)
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + b.size]}
        blobs.append(b)
        off += b.size
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b.tobytes())


@dataclasses.dataclass
class DecoderDims:
    """ParseHFDecoderDims (poly/hf_import.go:130-178)."""
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    inter: int
    rms_eps: float
    theta: float
    activation: int

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


def _layer_index(name: str) -> int:
    parts = name.split(".")
    for i, p in enumerate(parts):
        if p in ("layers", "h") and i + 1 < len(parts):
            m = re.match(r"-?\d+", parts[i + 1])
            return int(m.group(0)) if m else -1
    return -1


def decoder_dims(config: dict, tensor_names=()) -> DecoderDims:
    heads = int(config.get("num_attention_heads") or 0)
    if heads <= 0:
        raise ValueError("config missing num_attention_heads")
    kv = int(config.get("num_key_value_heads") or 0) or heads
    hidden = int(config.get("hidden_size") or 0)
    if hidden <= 0:
        raise ValueError("config missing hidden_size")
    inter = int(config.get("intermediate_size") or 0)
    if inter <= 0:
        raise ValueError("config missing intermediate_size")
    layers = int(config.get("num_hidden_layers") or 0)
    if layers <= 0:
        top = max((_layer_index(n) for n in tensor_names), default=-1)
        if top < 0:
            raise ValueError("could not determine num_hidden_layers")
        layers = top + 1
    head_dim = int(config.get("head_dim") or 0) or hidden // heads
    act = ACT_RELU2 if str(config.get("hidden_act", "")).lower() == "relu2" else ACT_SILU
    return DecoderDims(layers, hidden, heads, kv, head_dim, inter,
                       float(config.get("rms_norm_eps", 1e-6)), float(config.get("rope_theta", 10000.0)),
                       act)


def route(name: str):
    """decodeHFPrefixRouting (poly/prefix_safetensor.go:195-245): (layer,
    slot, role) of a block tensor, or None.  Slots: 0 RMSNorm1, 1 MHA, 2
    RMSNorm2, 3 SwiGLU; roles q/k/v/o/g/u/d (+ "_scale"), inner_norm, qn/kn,
    and "" for a norm's weight."""
    li = _layer_index(name)
    if li < 0:
        return None
    role = ""
    if "inner_attn_ln" in name or "attn_sub_norm" in name:
        slot, role = 1, "inner_norm"
    elif "ffn_layernorm" in name or "ffn_sub_norm" in name:
        slot, role = 3, "inner_norm"
    elif "input_layernorm" in name or "ln_1" in name:
        slot = 0
    elif "self_attn" in name or "attn" in name:
        slot = 1
        for key, r in (("q_proj", "q"), ("k_proj", "k"), ("v_proj", "v"), ("o_proj", "o")):
            if key in name:
                role = r
        if "weight_scale" in name and role:
            role += "_scale"
        if "q_norm" in name:
            role = "qn"
        if "k_norm" in name:
            role = "kn"
    elif "post_attention_layernorm" in name or "ln_2" in name:
        slot = 2
    elif "mlp" in name:
        slot = 3
        for keys, r in ((("gate_proj", "w1"), "g"), (("up_proj", "w3"), "u"), (("down_proj", "w2"), "d")):
            if any(k in name for k in keys):
                role = r
        if "weight_scale" in name and role:
            role += "_scale"
    else:
        return None
    return li, slot, role


_GLOBALS = {
    "embeddings": ("model.embed_tokens.weight", "transformer.wte.weight", "embeddings.weight",
                   "embed_tokens.weight"),
    "final_norm": ("model.norm.weight", "transformer.ln_f.weight", "ln_f.weight", "norm.weight"),
    "lm_head": ("lm_head.weight", "output.weight"),
}


def find_global(tensors: dict[str, StoredTensor], role: str):
    """PrefixWeightMapper.Find: the first pattern that matches a name
    exactly, else the first name ending in a pattern (patterns in order)."""
    for pat in _GLOBALS[role]:
        if pat in tensors:
            return tensors[pat]
        for k in sorted(tensors):
            if k.endswith(pat):
                return tensors[k]
    return None


def _matrix(t: StoredTensor, rows: int, cols: int, scale: float, device: int) -> TernaryMatrix:
    # copyWeights: a packed slab holds rows*cols/4 cells, a dense master rows*cols
    if rows % 4 == 0 and t.size * 4 == rows * cols:
        if t.dtype in ("U8", "I8"):
            packed = t.as_bytes()
        else:  # byte values stored in another dtype (SetMicrosoftBitNetPackedMatrix's float slots)
            packed = t.to_float32().astype(np.int64).astype(np.uint8)
        return TernaryMatrix.from_ms_offline(packed, rows, cols, scale, device=device)
    if t.size == rows * cols:
        return TernaryMatrix.from_float32(t.to_float32(), rows, cols, device=device)
    raise ValueError(f"projection of {t.shape} {t.dtype} fits neither {rows}x{cols} nor its packed form")


def load_blocks(tensors: dict[str, StoredTensor], dims: DecoderDims, device: int = 0):
    """The decoder blocks of a checkpoint as BlockWeights (the device copies
    of the ternary matrices are made here)."""
    per = [dict() for _ in range(dims.layers)]
    for name, t in tensors.items():
        r = route(name)
        if r is None:
            continue
        li, slot, role = r
        if li >= dims.layers:
            continue
        per[li][(slot, role)] = t
    h, q, kv, inter = dims.hidden, dims.q_dim, dims.kv_dim, dims.inter
    shapes = {(1, "q"): (q, h), (1, "k"): (kv, h), (1, "v"): (kv, h), (1, "o"): (h, q),
              (3, "g"): (inter, h), (3, "u"): (inter, h), (3, "d"): (h, inter)}
    out = []
    for li, d in enumerate(per):
        mats = {}
        for key, (rows, cols) in shapes.items():
            t = d.get(key)
            if t is None:
                raise ValueError(f"layer {li}: missing {key[1]} projection")
            st = d.get((key[0], key[1] + "_scale"))
            scale = float(st.to_float32().reshape(-1)[0]) if st is not None and st.size else 1.0
            if scale == 0.0:
                scale = 1.0
            mats[key[1]] = _matrix(t, rows, cols, scale, device)

        def vec(key, n):
            t = d.get(key)
            if t is None:
                return None
            v = t.to_float32().reshape(-1)
            if v.size != n:
                raise ValueError(f"layer {li}: {key} holds {v.size} values, expected {n}")
            return v

        norm1, norm2 = vec((0, ""), h), vec((2, ""), h)
        if norm1 is None or norm2 is None:
            raise ValueError(f"layer {li}: missing input_layernorm / post_attention_layernorm")
        def raw(key):  # QNormWeight / KNormWeight keep whatever length the tensor has
            t = d.get(key)
            return None if t is None else t.to_float32().reshape(-1)

        out.append(tf.BlockWeights(mats["q"], mats["k"], mats["v"], mats["o"], mats["g"], mats["u"],
                                   mats["d"], norm1, norm2, vec((1, "inner_norm"), q),
                                   vec((3, "inner_norm"), inter),
                                   q_norm=raw((1, "qn")), k_norm=raw((1, "kn"))))
    return out


def block_config(dims: DecoderDims, norm: str = "strict", max_seq_len: int = 2048,
                 max_batch: int = 1) -> tf.BlockConfig:
    # the import leaves the MHA and SwiGLU layers' RMSNormEps unset
    # (poly/hf_decoder.go:43-66): their inner norms take loom's default 1e-5,
    # the per-head Q/K norms 1e-6 (attn_eps 0 selects both defaults)
    return tf.BlockConfig(dims.hidden, dims.heads, dims.kv_heads, dims.head_dim, dims.inter,
                          max_seq_len=max_seq_len, max_batch=max_batch, rope_theta=dims.theta,
                          norm_eps=dims.rms_eps, attn_eps=0.0, ffn_eps=1e-5,
                          ffn_activation=dims.activation, norm=norm)


def load_hf_checkpoint(model_dir: str, norm: str = "strict", max_seq_len: int = 2048,
                       max_batch: int = 1, max_tokens: int | None = None, max_prefill: int = 0,
                       device: int = 0, simd_forward: bool = True):
    """ImportHFCheckpointDir: a Transformer on `device` and its DecoderDims."""
    with open(os.path.join(model_dir, "config.json")) as f:
        config = json.load(f)
    files = sorted(glob.glob(os.path.join(model_dir, "*.safetensors")))
    if not files:
        raise FileNotFoundError(f"no .safetensors in {model_dir}")
    tensors: dict[str, StoredTensor] = {}
    for p in files:
        tensors.update(read_safetensors(p))
    dims = decoder_dims(config, tensors.keys())
    emb_t = find_global(tensors, "embeddings")
    if emb_t is None:
        raise ValueError("checkpoint has no embeddings")
    emb = emb_t.to_float32().reshape(-1, dims.hidden)
    fn_t = find_global(tensors, "final_norm")
    lm_t = find_global(tensors, "lm_head")
    lm = None if lm_t is None else lm_t.to_float32().reshape(-1, dims.hidden)
    layers = load_blocks(tensors, dims, device)
    cfg = block_config(dims, norm, max_seq_len, max_batch)
    model = tf.Transformer(cfg, layers, emb, None if fn_t is None else fn_t.to_float32().reshape(-1),
                           lm_head=lm, vocab=emb.shape[0], final_norm_eps=1e-6,
                           max_tokens=max_tokens, max_prefill=max_prefill, device=device,
                           simd_forward=simd_forward)
    return model, dims
