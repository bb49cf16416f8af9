"""BitNet decoder block and greedy decode loop on gfx950: the host-side mirror
of loom's Transformer CPU path, running on libloom_accel_amd.so.

=====================================================  ==============================
loom (poly/)                                           here
=====================================================  ==============================
forwardOnCPUNormal block body                          ``BitNetBlock.forward``
  (transformer_forward.go:228-245): RMSNorm, packed
  ternary MHA (mha.go:204-371), residual, RMSNorm,
  packed ternary SwiGLU, residual
KVOffset / mhaPrepareKVForForward (mha_layout.go:62)   ``BitNetBlock.kv_offset``
Transformer.Generate greedy (transformer.go:330-520)   ``Transformer.generate``
  prefill: TokensToTensor + ForwardFull + ApplyLMHead  ``Transformer.prefill``
  decode: getEmbedding + forwardOne + ApplyLMHead +    ``Transformer.decode``
  SampleTopK(k<=1)
=====================================================  ==============================

Weights are loom BitNetTernaryMatrix words (``TernaryMatrix``) and fp32 host
arrays; activations are torch CUDA tensors (torch provides device memory and
the stream only).  There is no CPU fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import check
from .bitnet import ACT_SILU, NORM_STRICT, TernaryMatrix, _norm_mode, _stream, _torch


@dataclass
class BlockConfig:
    hidden: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    intermediate: int
    max_seq_len: int = 512
    max_batch: int = 1
    rope_theta: float = 10000.0
    norm_eps: float = 1e-6
    attn_eps: float = 1e-5
    ffn_eps: float = 1e-5
    ffn_activation: int = ACT_SILU
    norm: str | int = "strict"

    def desc(self) -> _lib.BlockDesc:
        return _lib.BlockDesc(self.hidden, self.num_heads, self.num_kv_heads, self.head_dim,
                              self.intermediate, self.max_seq_len, self.max_batch,
                              self.rope_theta, self.norm_eps, self.attn_eps, self.ffn_eps,
                              self.ffn_activation, _norm_mode(self.norm))

    @property
    def q_dim(self) -> int:
        return self.num_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return (self.num_kv_heads or self.num_heads) * self.head_dim


@dataclass
class BlockWeights:
    """Ternary matrices and fp32 host vectors of one decoder block."""
    q: TernaryMatrix
    k: TernaryMatrix
    v: TernaryMatrix
    o: TernaryMatrix
    gate: TernaryMatrix
    up: TernaryMatrix
    down: TernaryMatrix
    norm1: np.ndarray
    norm2: np.ndarray
    attn_inner_norm: np.ndarray | None = None
    ffn_inner_norm: np.ndarray | None = None
    bias_q: np.ndarray | None = None
    bias_k: np.ndarray | None = None
    bias_v: np.ndarray | None = None
    bias_o: np.ndarray | None = None
    # per-head Q / K RMSNorm weights (loom's QNormWeight / KNormWeight,
    # poly/mha.go:285-290): None or empty applies none; eps from attn_eps
    # (mhaQKNormEpsilon: RMSNormEps, else 1e-6)
    q_norm: np.ndarray | None = None
    k_norm: np.ndarray | None = None

    def struct(self, keep: list) -> _lib.BlockWeights:
        def host(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a, np.float32)
            keep.append(a)
            return a.ctypes.data_as(C.c_void_p)

        return _lib.BlockWeights(self.q.handle, self.k.handle, self.v.handle, self.o.handle,
                                 self.gate.handle, self.up.handle, self.down.handle,
                                 host(self.norm1), host(self.norm2), host(self.attn_inner_norm),
                                 host(self.ffn_inner_norm), host(self.bias_q), host(self.bias_k),
                                 host(self.bias_v), host(self.bias_o),
                                 host(self.q_norm), _length(self.q_norm),
                                 host(self.k_norm), _length(self.k_norm))


def _length(a) -> int:
    return 0 if a is None else int(np.asarray(a).size)


@dataclass
class BlockTaps:
    """Device copies of one block call's intermediates (loom_amd_block_taps).
    Requesting them does not change which kernels run."""
    y1: object = None         # rows x hidden fp32: RMSNorm1 output
    q: object = None          # rows x q_dim fp64: Q after bias and RoPE
    attn: object = None       # rows x q_dim fp64: attention before the inner norm
    mid: object = None        # rows x hidden fp32: x after the attention residual
    xq1: object = None        # rows x hidden int8: quantized RMSNorm1 rows
    amax1: object = None      # rows fp32
    attn_norm: object = None  # rows x q_dim fp64: attention after the inner norm
    aq: object = None         # rows x q_dim int8
    aamax: object = None      # rows fp32
    y2: object = None         # rows x hidden fp32: RMSNorm2 output
    xq2: object = None        # rows x hidden int8
    amax2: object = None      # rows fp32
    h: object = None          # rows x inter fp32: gate product before the inner norm
    hn: object = None         # rows x inter fp32: after the inner norm
    hq: object = None         # rows x inter int8
    hamax: object = None      # rows fp32

    FIELDS = ("y1", "q", "attn", "mid", "xq1", "amax1", "attn_norm", "aq", "aamax", "y2", "xq2",
              "amax2", "h", "hn", "hq", "hamax")

    def numpy(self) -> dict:
        return {f: getattr(self, f).cpu().numpy() for f in self.FIELDS}


class BitNetBlock:
    """One BitNet decoder block with its KV ring caches, on one device."""

    def __init__(self, cfg: BlockConfig, w: BlockWeights, device: int = 0):
        self.cfg = cfg
        self.device = device
        keep: list = []
        ws = w.struct(keep)
        desc = cfg.desc()
        out = C.c_void_p()
        check(_lib.lib().loom_amd_block_create(device, C.byref(desc), C.byref(ws), C.byref(out)),
              "block_create")
        self._h = out

    @property
    def kv_offset(self) -> int:
        return _lib.lib().loom_amd_block_kv_offset(self._h)

    def forward(self, x, taps: bool = False, shared_timeline: bool = False):
        """In place on x (torch float32 CUDA tensor, [seq, hidden] or
        [batch, seq, hidden]); returns (x, BlockTaps or None).

        A 3-D batch runs as separate sequences, each with its own KV ring.
        shared_timeline=True gives loom's semantics for a 3-D input instead
        (poly/mha.go:251-371): the batch's sequences form one KV timeline from
        position 0, sequence b at positions b*seq .., each attending to every
        earlier position of the timeline -- the batch's rows run as one
        sequence of batch*seq tokens."""
        torch = _torch()
        if x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous():
            raise ValueError("x must be a contiguous float32 device tensor")
        if x.dim() == 2:
            batch, seq = 1, x.shape[0]
        elif x.dim() == 3:
            batch, seq = x.shape[0], x.shape[1]
        else:
            raise ValueError("x must be [seq, hidden] or [batch, seq, hidden]")
        if shared_timeline:
            batch, seq = 1, batch * seq
        if x.shape[-1] != self.cfg.hidden:
            raise ValueError(f"hidden is {x.shape[-1]}, block expects {self.cfg.hidden}")
        rows = batch * seq
        t = None
        tp = None
        if taps:
            dev = x.device
            H, Q, I = self.cfg.hidden, self.cfg.q_dim, self.cfg.intermediate

            def e(*shape, dt=torch.float32):
                return torch.empty(*shape, dtype=dt, device=dev)

            f64, i8 = torch.float64, torch.int8
            t = BlockTaps(y1=e(rows, H), q=e(rows, Q, dt=f64), attn=e(rows, Q, dt=f64),
                          mid=e(rows, H), xq1=e(rows, H, dt=i8), amax1=e(rows),
                          attn_norm=e(rows, Q, dt=f64), aq=e(rows, Q, dt=i8), aamax=e(rows),
                          y2=e(rows, H), xq2=e(rows, H, dt=i8), amax2=e(rows),
                          h=e(rows, I), hn=e(rows, I), hq=e(rows, I, dt=i8), hamax=e(rows))
            tp = C.byref(_lib.BlockTaps(*(getattr(t, f).data_ptr() for f in BlockTaps.FIELDS)))
        check(_lib.lib().loom_amd_block_forward(self._h, C.c_void_p(x.data_ptr()), batch, seq, tp,
                                                _stream(self.device)), "block_forward")
        return x, t

    def kv_cache(self, slot: int = 0):
        """(K, V) ring of one sequence slot as torch views [max_seq_len, kv_dim]."""
        k, v = C.c_void_p(), C.c_void_p()
        check(_lib.lib().loom_amd_block_kv_cache(self._h, slot, C.byref(k), C.byref(v)),
              "block_kv_cache")
        shape = (self.cfg.max_seq_len, self.cfg.kv_dim)
        return tuple(_clone_device(p, shape, self.device) for p in (k.value, v.value))

    def release(self) -> None:
        if self._h is not None:
            _lib.lib().loom_amd_block_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


class _DeviceView:
    """__cuda_array_interface__ of a raw device pointer (read-only view)."""

    def __init__(self, ptr: int, shape: tuple, typestr: str):
        self.__cuda_array_interface__ = {"shape": shape, "typestr": typestr,
                                         "data": (ptr, False), "version": 2, "strides": None}


def _clone_device(ptr: int, shape: tuple, device: int, typestr: str = "<f4"):
    """Copy of device memory at ptr into a new torch tensor."""
    torch = _torch()
    torch.cuda.synchronize(device)
    return torch.as_tensor(_DeviceView(ptr, shape, typestr), device=f"cuda:{device}").clone()


def lm_head(table, x, sequential: bool = False):
    """applyFP32LMHeadRows on device: table [vocab, hidden], x [rows, hidden]
    float32 device tensors -> logits [rows, vocab], in simd.DotTile's order
    (SIMD forward on) or, with sequential, the scalar loop's."""
    torch = _torch()
    for t in (table, x):
        if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous():
            raise ValueError("table and x must be contiguous float32 device tensors")
    x2 = x.reshape(-1, x.shape[-1])
    vocab, hidden = table.shape
    if x2.shape[1] != hidden:
        raise ValueError("hidden sizes differ")
    out = torch.empty(x2.shape[0], vocab, dtype=torch.float32, device=x.device)
    fn = _lib.lib().loom_amd_lm_head_sequential if sequential else _lib.lib().loom_amd_lm_head
    check(fn(C.c_void_p(table.data_ptr()), vocab, hidden, C.c_void_p(x2.data_ptr()), x2.shape[0],
             C.c_void_p(out.data_ptr()), _stream(x.device.index or 0)), "lm_head")
    return out


def lm_head_sequential(table, x):
    """applyFP32LMHeadRows with SIMD forward off (one sequential fp64 sum per
    logit) on device; arguments as for lm_head."""
    return lm_head(table, x, sequential=True)


def greedy_sample(logits):
    """SampleTopK with k <= 1 per row of a float32 device tensor -> int32 ids."""
    torch = _torch()
    lg = logits.reshape(-1, logits.shape[-1])
    if lg.dtype != torch.float32 or not lg.is_cuda or not lg.is_contiguous():
        raise ValueError("logits must be a contiguous float32 device tensor")
    ids = torch.empty(lg.shape[0], dtype=torch.int32, device=lg.device)
    check(_lib.lib().loom_amd_greedy_sample(C.c_void_p(lg.data_ptr()), lg.shape[1], lg.shape[0],
                                            C.c_void_p(ids.data_ptr()),
                                            _stream(lg.device.index or 0)), "greedy_sample")
    return ids


class Transformer:
    """A stack of BitNet blocks with fp32 embeddings, final RMSNorm and LM head
    (tied to the embeddings when lm_head is None), decoding greedily.  An fp32
    head sums in simd.DotTile's order, or loom's scalar order when
    simd_forward is False (Network.UseSimdForward)."""

    def __init__(self, cfg: BlockConfig, layers: list[BlockWeights], embeddings: np.ndarray,
                 final_norm: np.ndarray | None, lm_head: np.ndarray | None = None,
                 vocab: int | None = None, final_norm_eps: float = 1e-6,
                 max_tokens: int | None = None, max_prefill: int = 0, device: int = 0,
                 simd_forward: bool = True):
        self.cfg = cfg
        self.device = device
        emb = np.ascontiguousarray(embeddings, np.float32)
        self.vocab = vocab or emb.size // cfg.hidden
        keep: list = []
        arr = (_lib.BlockWeights * max(1, len(layers)))()
        for i, w in enumerate(layers):
            arr[i] = w.struct(keep)
        self.max_tokens = max_tokens or cfg.max_seq_len + 1
        desc = _lib.ModelDesc(cfg.desc(), len(layers), self.vocab, final_norm_eps,
                              self.max_tokens, max_prefill, 0 if simd_forward else 1)
        fn = None if final_norm is None else np.ascontiguousarray(final_norm, np.float32)
        lm = None if lm_head is None else np.ascontiguousarray(lm_head, np.float32)
        out = C.c_void_p()
        check(_lib.lib().loom_amd_model_create(
            device, C.byref(desc), arr, emb.ctypes.data_as(C.c_void_p),
            None if fn is None else fn.ctypes.data_as(C.c_void_p),
            None if lm is None else lm.ctypes.data_as(C.c_void_p), C.byref(out)), "model_create")
        self._h = out
        self.batch = 0

    @property
    def position(self) -> int:
        return _lib.lib().loom_amd_model_position(self._h)

    def prefill(self, ids, logits: bool = False):
        """Restart with prompt ids ([n] or [batch, n]); returns the logits of
        each sequence's last position (torch [batch, vocab]) when asked."""
        torch = _torch()
        ids = np.ascontiguousarray(np.atleast_2d(np.asarray(ids)), np.int32)
        batch, n = ids.shape
        out = (torch.empty(batch, self.vocab, dtype=torch.float32, device=f"cuda:{self.device}")
               if logits else None)
        check(_lib.lib().loom_amd_model_prefill(self._h, ids.ctypes.data_as(C.c_void_p), batch, n,
                                                None if out is None else C.c_void_p(out.data_ptr()),
                                                _stream(self.device)), "model_prefill")
        self.batch = batch
        return out

    def decode(self, steps: int, use_graph: bool = True, logits: bool = False):
        torch = _torch()
        out = (torch.empty(self.batch, self.vocab, dtype=torch.float32,
                           device=f"cuda:{self.device}") if logits else None)
        check(_lib.lib().loom_amd_model_decode(self._h, steps, int(use_graph),
                                               None if out is None else C.c_void_p(out.data_ptr()),
                                               _stream(self.device)), "model_decode")
        return out

    def tokens(self) -> np.ndarray:
        """Prompt + generated ids of every sequence, [batch, position + 1]."""
        count = self.position + 1
        out = np.empty((max(1, self.batch), count), np.int32)
        check(_lib.lib().loom_amd_model_tokens(self._h, out.ctypes.data_as(C.c_void_p), count,
                                               _stream(self.device)), "model_tokens")
        return out

    def generate(self, prompt_ids, max_tokens: int, use_graph: bool = True) -> np.ndarray:
        """Greedy Generate without EOS stop: max_tokens new ids per sequence."""
        self.prefill(prompt_ids)
        if max_tokens > 1:
            self.decode(max_tokens - 1, use_graph=use_graph)
        toks = self.tokens()
        n = np.atleast_2d(np.asarray(prompt_ids)).shape[1]
        return toks[:, n:n + max_tokens]

    def last_hidden(self):
        """Each sequence's last row after the final norm (torch [batch, hidden])."""
        p = _lib.lib().loom_amd_model_last_hidden(self._h)
        return _clone_device(p, (self.batch, self.cfg.hidden), self.device)

    def release(self) -> None:
        if self._h is not None:
            _lib.lib().loom_amd_model_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.release()
        except Exception:
            pass


__all__ = ["BlockConfig", "BlockWeights", "BlockTaps", "BitNetBlock", "Transformer", "NORM_STRICT",
           "lm_head", "lm_head_sequential", "greedy_sample"]
