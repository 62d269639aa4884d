"""Host-side model description and the decode engine handle.

``HostModel`` holds a model's tensors in host memory -- either drawn from a
seeded synthetic configuration or memory-mapped from a GGUF file -- and turns
them into the ``lg_model_desc`` of include/ligguf_hip.h, i.e. the fields of
the reference's gguf_model / trans_block (fast/lil_gguf.h:126-219) plus the
RoPE table of model_state::allocate (fast/common.cpp:38-39).

``Engine`` owns one ``lg_ctx`` (one device, one stream) and exposes the
per-token step of inference() (fast/ligguf_fast_qk.cpp:24-144).
"""
from __future__ import annotations

import ctypes as C
import ctypes.util
import zlib
from dataclasses import dataclass

import numpy as np

from . import encode
from .gguf import GARRAY, GFLOAT32, GSTRING, GUINT32, read_gguf, write_gguf
from .lib import (ARCH_LLAMA, ARCH_QWEN3, BLOCK, F32, Q1_0, Q1_G, Q4_K, Q6_K, Q8_0, LgLayerDesc, LgModelDesc,
                  LgWeight, check, load, row_size)


@dataclass(frozen=True)
class ModelConfig:
    name: str
    arch: int
    n_layers: int
    n_embed: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    n_ff: int
    vocab: int
    n_context: int
    rope_theta: float
    rms_eps: float
    layer_type: int
    embd_type: int
    out_type: int
    sigma: float = 0.02
    q1_direct: bool = False   # 1-bit layers drawn as Bernoulli signs + |N(0,sigma)| scales
    seed: int = 1234
    # per-tensor types that replace layer_type, in every layer ("attn_v") or
    # in one ("attn_v.3", taking precedence), e.g. (("attn_v", Q6_K),
    # ("ffn_down", Q6_K)) for a Q4_K_M-style mix
    overrides: tuple = ()

    def tensor_type(self, tensor: str, layer: int = None) -> int:
        """The type of layer tensor `tensor` ("attn_q" .. "ffn_down") in
        layer `layer` (None: the type every layer has without a per-layer
        override)."""
        o = dict(self.overrides)
        if layer is not None and f"{tensor}.{layer}" in o:
            return o[f"{tensor}.{layer}"]
        return o.get(tensor, self.layer_type)

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def rope_dim(self) -> int:
        return self.head_dim

    def with_(self, **kw) -> "ModelConfig":
        d = dict(self.__dict__)
        d.update(kw)
        return ModelConfig(**d)

    def weight_bytes(self) -> int:
        """Bytes read per decode token: every layer weight, the output head,
        the norms and one embedding row."""
        ne, kv, ff = self.n_embed, self.kv_dim, self.n_ff
        total = 0
        for l in range(self.n_layers):
            def tt(t):
                return self.tensor_type(t, l)
            total += (ne * row_size(tt("attn_q"), ne) + kv * row_size(tt("attn_k"), ne) +
                      kv * row_size(tt("attn_v"), ne) + ne * row_size(tt("attn_output"), ne) +
                      ff * row_size(tt("ffn_up"), ne) + ff * row_size(tt("ffn_gate"), ne) +
                      ne * row_size(tt("ffn_down"), ff) + 2 * ne * 4)
            if self.arch == ARCH_QWEN3:
                total += 2 * self.head_dim * 4
        return total + self.vocab * row_size(self.out_type, ne) + ne * 4 + row_size(self.embd_type, ne)

    def kv_bytes(self, pos: int) -> int:
        """fp16 K and V bytes the attention reads at position pos (all layers)."""
        return self.n_layers * (pos + 1) * self.kv_dim * 2 * 2


# Tiny llama, Q8_0 everywhere (dim 288, FFN 768, 6 layers, 6/6 heads, hd 48)
TINY = ModelConfig("tiny-llama-q8_0", ARCH_LLAMA, 6, 288, 6, 6, 48, 768, 32000, 256, 1e4, 1e-5, Q8_0, Q8_0, Q8_0)
# Qwen3-8B shape, Q4_K layers and embedding, Q6_K output
QWEN3_8B_Q4K = ModelConfig("qwen3-8b-shape-q4_k", ARCH_QWEN3, 36, 4096, 32, 8, 128, 12288, 151936, 1024, 1e6, 1e-6,
                           Q4_K, Q4_K, Q6_K)
# Qwen3-8B shape, 1-bit Q1_G layers, Q8_0 embedding and output
QWEN3_8B_Q1G = ModelConfig("qwen3-8b-shape-q1_g", ARCH_QWEN3, 36, 4096, 32, 8, 128, 12288, 151936, 8704, 1e6, 1e-6,
                           Q1_G, Q8_0, Q8_0, q1_direct=True)

_libm = C.CDLL(ctypes.util.find_library("m"))
_libm.powf.restype = C.c_float
_libm.powf.argtypes = [C.c_float, C.c_float]


def rope_freq_table(base: float, rope_dim: int) -> np.ndarray:
    """powf(base, -2i/rope_dim) with fp32 exponent arithmetic, the formula of
    model_state::allocate (fast/common.cpp:38-39), through the C library's
    scalar powf.  (The reference's -Ofast build may vectorise that loop with
    libmvec; callers that need its exact table pass it in.)"""
    out = np.empty(rope_dim // 2, np.float32)
    for i in range(rope_dim // 2):
        e = np.float32(-2.0) * np.float32(i) / np.float32(rope_dim)
        out[i] = _libm.powf(np.float32(base), e)
    return out


LAYER_TENSORS = ["attn_q", "attn_k", "attn_v", "attn_output", "ffn_up", "ffn_gate", "ffn_down"]


class HostModel:
    """Tensors of one model in host memory (numpy arrays, possibly memmaps)."""

    def __init__(self, cfg: ModelConfig):
        self.cfg = cfg
        self.weights = {}    # name -> (type, rows, cols, uint8 ndarray)
        self.norms = {}      # name -> float32 ndarray
        self.rope_freq = rope_freq_table(cfg.rope_theta, cfg.rope_dim)
        self._keep = []

    # ---- construction
    @classmethod
    def synthetic(cls, cfg: ModelConfig) -> "HostModel":
        """Weights N(0, sigma) encoded to the configured types, norms 1.0; 1-bit
        layers optionally drawn directly (Bernoulli signs, |N| scales)."""
        m = cls(cfg)
        ne, kv, ff = cfg.n_embed, cfg.kv_dim, cfg.n_ff

        def draw(name, t, rows, cols):
            stream = zlib.crc32(name.encode())
            if t in (Q1_0, Q1_G) and cfg.q1_direct:
                data = encode.random_q1(t, cfg.seed, stream, rows, cols, cfg.sigma)
            else:
                data = encode.random_tensor(t, cfg.seed, stream, rows, cols, cfg.sigma)
            m.weights[name] = (t, rows, cols, data)

        draw("token_embd.weight", cfg.embd_type, cfg.vocab, ne)
        draw("output.weight", cfg.out_type, cfg.vocab, ne)
        m.norms["output_norm.weight"] = np.ones(ne, np.float32)
        shapes = {"attn_q": (ne, ne), "attn_k": (kv, ne), "attn_v": (kv, ne), "attn_output": (ne, ne),
                  "ffn_up": (ff, ne), "ffn_gate": (ff, ne), "ffn_down": (ne, ff)}
        for l in range(cfg.n_layers):
            for t in LAYER_TENSORS:
                draw(f"blk.{l}.{t}.weight", cfg.tensor_type(t, l), *shapes[t])
            m.norms[f"blk.{l}.attn_norm.weight"] = np.ones(ne, np.float32)
            m.norms[f"blk.{l}.ffn_norm.weight"] = np.ones(ne, np.float32)
            if cfg.arch == ARCH_QWEN3:
                m.norms[f"blk.{l}.attn_q_norm.weight"] = np.ones(cfg.head_dim, np.float32)
                m.norms[f"blk.{l}.attn_k_norm.weight"] = np.ones(cfg.head_dim, np.float32)
        return m

    @classmethod
    def from_gguf(cls, path: str, n_context: int = 0) -> "HostModel":
        """Memory-map a llama/qwen3 GGUF the way read_llama/read_qwen3 read it
        (fast/lil_gguf.cpp:397-499)."""
        g = read_gguf(path)
        arch = g.kv["general.architecture"]
        if arch == "llama":
            p = "llama."
            ne = int(g.kv[p + "embedding_length"])
            nh = int(g.kv[p + "attention.head_count"])
            hd = ne // nh
            cfg_arch = ARCH_LLAMA
            vocab = int(g.kv[p + "vocab_size"])
        elif arch == "qwen3":
            p = "qwen3."
            ne = int(g.kv[p + "embedding_length"])
            nh = int(g.kv[p + "attention.head_count"])
            hd = int(g.kv[p + "attention.key_length"])
            cfg_arch = ARCH_QWEN3
            vocab = int(g.tensors["token_embd.weight"].dims[1])
        else:
            raise ValueError(f"architecture {arch} is not on the decode path")
        nkv = int(g.kv[p + "attention.head_count_kv"])
        ctx = int(g.kv[p + "context_length"])
        if 0 < n_context <= ctx:
            ctx = n_context
        lt = g.tensors["blk.0.attn_q.weight"].type
        cfg = ModelConfig(f"gguf:{path}", cfg_arch, int(g.kv[p + "block_count"]), ne, nh, nkv, hd,
                          int(g.kv[p + "feed_forward_length"]), vocab, ctx, float(g.kv[p + "rope.freq_base"]),
                          float(g.kv[p + "attention.layer_norm_rms_epsilon"]), lt,
                          g.tensors["token_embd.weight"].type, g.tensors["output.weight"].type)
        m = cls(cfg)
        if arch == "llama":
            rd = int(g.kv[p + "rope.dimension_count"])
            m.rope_freq = rope_freq_table(cfg.rope_theta, rd)
            m._rope_dim = rd
        for name, t in g.tensors.items():
            if name.endswith("norm.weight"):
                m.norms[name] = np.frombuffer(t.data, np.float32)
            else:
                m.weights[name] = (t.type, t.rows, int(t.dims[0]), t.data)
        m._gguf = g
        return m

    # ---- export
    def write_gguf(self, path: str, byte_tokens: bool = False) -> None:
        """A GGUF v3 file the reference loader reads (fast/lil_gguf.cpp:328-499).
        The tokenizer vocabulary is placeholder strings; with byte_tokens the
        first 256 are the byte tokens <0x00>..<0xFF>, so the reference's
        fallback tokenizer (fast/tokenize.cpp:68-104) can encode any text."""
        c = self.cfg
        if c.arch == ARCH_LLAMA:
            p = "llama."
            kv = [("general.architecture", GSTRING, "llama"),
                  (p + "vocab_size", GUINT32, c.vocab), (p + "context_length", GUINT32, c.n_context),
                  (p + "embedding_length", GUINT32, c.n_embed), (p + "attention.head_count", GUINT32, c.n_heads),
                  (p + "attention.head_count_kv", GUINT32, c.n_kv_heads), (p + "block_count", GUINT32, c.n_layers),
                  (p + "attention.layer_norm_rms_epsilon", GFLOAT32, c.rms_eps),
                  (p + "rope.freq_base", GFLOAT32, c.rope_theta), (p + "rope.dimension_count", GUINT32, c.rope_dim),
                  (p + "feed_forward_length", GUINT32, c.n_ff)]
        else:
            p = "qwen3."
            kv = [("general.architecture", GSTRING, "qwen3"),
                  (p + "block_count", GUINT32, c.n_layers), (p + "context_length", GUINT32, c.n_context),
                  (p + "embedding_length", GUINT32, c.n_embed), (p + "attention.head_count", GUINT32, c.n_heads),
                  (p + "attention.head_count_kv", GUINT32, c.n_kv_heads),
                  (p + "attention.layer_norm_rms_epsilon", GFLOAT32, c.rms_eps),
                  (p + "rope.freq_base", GFLOAT32, c.rope_theta), (p + "attention.key_length", GUINT32, c.head_dim),
                  (p + "attention.value_length", GUINT32, c.head_dim), (p + "feed_forward_length", GUINT32, c.n_ff)]
        names = [f"<0x{i:02X}>" if byte_tokens and i < 256 else f"<t{i}>" for i in range(c.vocab)]
        kv.append(("tokenizer.ggml.tokens", GARRAY, (GSTRING, names)))
        tensors = []
        for name, (t, rows, cols, data) in self.weights.items():
            tensors.append((name, t, [cols, rows], data))
        for name, arr in self.norms.items():
            tensors.append((name, F32, [arr.size], arr.view(np.uint8)))
        write_gguf(path, kv, tensors)

    def _w(self, struct_cls, name):
        t, rows, cols, data = self.weights[name]
        arr = np.ascontiguousarray(data)
        self._keep.append(arr)
        return struct_cls(arr.ctypes.data, t, row_size(t, cols), rows, cols)

    def _f(self, name):
        a = np.ascontiguousarray(self.norms[name], dtype=np.float32)
        self._keep.append(a)
        return a.ctypes.data

    def fill_desc(self, model_cls=LgModelDesc, layer_cls=LgLayerDesc, weight_cls=LgWeight):
        """The lg_model_desc (or the oracle's identically laid out or_model)."""
        c = self.cfg
        layers = (layer_cls * c.n_layers)()
        for l in range(c.n_layers):
            b = f"blk.{l}."
            L = layers[l]
            L.att_norm = self._f(b + "attn_norm.weight")
            L.att_q = self._w(weight_cls, b + "attn_q.weight")
            L.att_k = self._w(weight_cls, b + "attn_k.weight")
            L.att_v = self._w(weight_cls, b + "attn_v.weight")
            L.att_out = self._w(weight_cls, b + "attn_output.weight")
            if c.arch == ARCH_QWEN3:
                L.att_q_norm = self._f(b + "attn_q_norm.weight")
                L.att_k_norm = self._f(b + "attn_k_norm.weight")
            L.ffn_norm = self._f(b + "ffn_norm.weight")
            L.ffn_up = self._w(weight_cls, b + "ffn_up.weight")
            L.ffn_down = self._w(weight_cls, b + "ffn_down.weight")
            L.ffn_gate = self._w(weight_cls, b + "ffn_gate.weight")
        self._keep.append(layers)
        freq = np.ascontiguousarray(self.rope_freq, dtype=np.float32)
        self._keep.append(freq)
        rope_dim = getattr(self, "_rope_dim", c.rope_dim)
        d = model_cls(c.arch, c.n_layers, c.n_embed, c.n_heads, c.n_kv_heads, c.head_dim, c.kv_dim, c.n_ff, c.vocab,
                      c.n_context, rope_dim, c.rms_eps, freq.ctypes.data, self._w(weight_cls, "token_embd.weight"),
                      self._w(weight_cls, "output.weight"), self._f("output_norm.weight"),
                      C.cast(layers, C.c_void_p))
        self._keep.append(d)
        return d


class Engine:
    """One lg_ctx: a device, a stream and an uploaded model."""

    def __init__(self, device: int = 0):
        self.lib = load()
        self.ctx = C.c_void_p()
        check(self.lib.lg_create(device, C.byref(self.ctx)))
        self.vocab = 0
        self.cfg = None

    def load(self, hm: HostModel) -> None:
        desc = hm.fill_desc()
        check(self.lib.lg_load_model(self.ctx, C.byref(desc)), self.ctx)
        self.vocab = hm.cfg.vocab
        self.cfg = hm.cfg

    def set_path(self, path: int) -> None:
        """lg_set_decode_path: PATH_AUTO, PATH_FUSED, PATH_PERSISTENT or PATH_MULTI."""
        check(self.lib.lg_set_decode_path(self.ctx, path), self.ctx)

    def path(self) -> int:
        """The decode path the next step takes (PATH_FUSED / PATH_PERSISTENT / PATH_MULTI)."""
        return int(self.lib.lg_decode_path(self.ctx))

    def time_phase(self, phase: int, layer0: int = 0, iters: int = 100) -> float:
        """lg_time_fused_phase: mean microseconds per launch of one fused-step
        kernel (0 QKV, 1 attention, 2 att_out, 3 up|gate, 4 down, 5 output),
        at layers layer0, layer0+1, ... (mod n_layers)."""
        us = C.c_float()
        check(self.lib.lg_time_fused_phase(self.ctx, phase, layer0, iters, C.byref(us)), self.ctx)
        return float(us.value)

    def decode(self, tok: int, pos: int, want_logits: bool = True):
        if want_logits:
            out = np.empty(self.vocab, np.float32)
            check(self.lib.lg_decode_step(self.ctx, tok, pos, out.ctypes.data), self.ctx)
            return out
        check(self.lib.lg_decode_step(self.ctx, tok, pos, None), self.ctx)
        return None

    def decode_traced(self, tok: int, pos: int):
        """lg_decode_step with lg_trace_acts_next_step: (logits, [4L+1][stride]
        uint8 quantized activations of the step).  Device memory from torch."""
        import torch
        n = int(self.lib.lg_trace_acts_size(self.ctx))
        buf = torch.zeros(n, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()          # the fill runs on torch's stream, the step on the context's
        check(self.lib.lg_trace_acts_next_step(self.ctx, C.c_void_p(buf.data_ptr())), self.ctx)
        logits = self.decode(tok, pos)
        tr = buf.cpu().numpy().reshape(4 * self.cfg.n_layers + 1, -1)
        return logits, tr

    def prefill_traced(self, toks, pos0: int = 0):
        """lg_prefill with lg_trace_acts_next_prefill: (logits, [n][4L+1][stride]
        uint8 quantized activations of every token; the output head's slot
        for the last token only).  The prompt must run batched."""
        import torch
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        n1 = int(self.lib.lg_trace_acts_size(self.ctx))
        buf = torch.zeros(len(toks) * n1, dtype=torch.uint8, device="cuda")
        torch.cuda.synchronize()
        check(self.lib.lg_trace_acts_next_prefill(self.ctx, C.c_void_p(buf.data_ptr())), self.ctx)
        logits = self.prefill(toks, pos0)
        tr = buf.cpu().numpy().reshape(len(toks), 4 * self.cfg.n_layers + 1, -1)
        return logits, tr

    def state_save(self, path: str, pos: int) -> None:
        """lg_state_save: the reference's state file of cache rows [0, pos)
        and the last step's logits."""
        check(self.lib.lg_state_save(self.ctx, path.encode(), pos), self.ctx)

    def state_load(self, path: str):
        """lg_state_load: (pos, logits) of a reference state file."""
        pos = C.c_int()
        out = np.empty(self.vocab, np.float32)
        check(self.lib.lg_state_load(self.ctx, path.encode(), C.byref(pos), out.ctypes.data), self.ctx)
        return int(pos.value), out

    def decode_async(self, tok: int, pos: int) -> None:
        check(self.lib.lg_decode_step_async(self.ctx, tok, pos), self.ctx)

    def sync(self) -> None:
        check(self.lib.lg_sync(self.ctx), self.ctx)

    def argmax(self) -> int:
        t = C.c_int()
        check(self.lib.lg_argmax(self.ctx, C.byref(t)), self.ctx)
        return int(t.value)

    def decode_greedy(self, tok: int, pos: int, n: int) -> np.ndarray:
        """lg_decode_greedy: n greedy steps from (tok, pos) queued back to
        back; the greedy token of each step."""
        out = np.zeros(n, dtype=np.int32)
        check(self.lib.lg_decode_greedy(self.ctx, tok, pos, n, out.ctypes.data_as(C.POINTER(C.c_int))), self.ctx)
        return out

    def sample_topp(self, temp: float, topp: float, topk: int, r01: float) -> int:
        """lg_sample_topp: the reference's sampler_topp over the device logits,
        r01 = (float)rand() / (float)RAND_MAX drawn by the caller."""
        t = C.c_int()
        check(self.lib.lg_sample_topp(self.ctx, temp, topp, topk, r01, C.byref(t)), self.ctx)
        return int(t.value)

    def set_prefill_path(self, path: int) -> None:
        """lg_set_prefill_path: PREFILL_AUTO, PREFILL_STEPS or PREFILL_BATCHED."""
        check(self.lib.lg_set_prefill_path(self.ctx, path), self.ctx)

    def prefill_path(self) -> int:
        return int(self.lib.lg_prefill_path(self.ctx))

    def prefill(self, toks, pos0: int, want_logits: bool = True):
        arr = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty(self.vocab, np.float32) if want_logits else None
        check(self.lib.lg_prefill(self.ctx, arr.ctypes.data, arr.size, pos0,
                                  out.ctypes.data if out is not None else None), self.ctx)
        return out

    def kv_read(self, layer0: int, nlayers: int, pos0: int, npos: int):
        kvd = self.cfg.kv_dim
        k = np.empty(nlayers * npos * kvd, np.uint16)
        v = np.empty_like(k)
        check(self.lib.lg_kv_read(self.ctx, layer0, nlayers, pos0, npos, k.ctypes.data, v.ctypes.data), self.ctx)
        return k, v

    def kv_write(self, layer0: int, nlayers: int, pos0: int, npos: int, k: np.ndarray, v: np.ndarray) -> None:
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        check(self.lib.lg_kv_write(self.ctx, layer0, nlayers, pos0, npos, k.ctypes.data, v.ctypes.data), self.ctx)

    def close(self) -> None:
        if self.ctx:
            self.lib.lg_destroy(self.ctx)
            self.ctx = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
