"""ctypes bindings of the CPU checkers (oracle/lg_oracle.c and the reference
engine build under oracle/_ref).  TEST INFRASTRUCTURE ONLY."""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(ORACLE_DIR, "liblg_oracle.so")
REF_SO = os.path.join(ORACLE_DIR, "_ref", "libligguf_ref.so")
REF_SRC = "/root/reference/fast"

_fp = C.POINTER(C.c_float)
_vp = C.c_void_p


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def build_reference() -> bool:
    """Compile the reference engine from its sources when they are present
    (only in the build container; the built .so travels with the tree)."""
    if not os.path.isdir(REF_SRC):
        return False
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "ref", "-j8"], check=True)
    # the reference's own driver, as is and with the LG_HIP patch (needs libligguf_hip.so built)
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "driver"], check=True)
    return True


def reference_available() -> bool:
    return os.path.exists(REF_SO)


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_fp)


class OrWeight(C.Structure):
    _fields_ = [("data", _vp), ("type", C.c_int32), ("rsz", C.c_uint32), ("rows", C.c_int32), ("cols", C.c_int32)]


class OrLayer(C.Structure):
    _fields_ = [("att_norm", _vp), ("att_q", OrWeight), ("att_k", OrWeight), ("att_v", OrWeight),
                ("att_out", OrWeight), ("att_q_norm", _vp), ("att_k_norm", _vp), ("ffn_norm", _vp),
                ("ffn_up", OrWeight), ("ffn_down", OrWeight), ("ffn_gate", OrWeight)]


class OrModel(C.Structure):
    _fields_ = [("arch", C.c_int32), ("n_layers", C.c_int32), ("n_embed", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("kv_dim", C.c_int32), ("n_ff", C.c_int32),
                ("vocab_size", C.c_int32), ("n_context", C.c_int32), ("rope_dim", C.c_int32),
                ("rms_epsilon", C.c_float), ("rope_freq", _vp), ("token_embd", OrWeight), ("output", OrWeight),
                ("output_norm", _vp), ("layers", _vp)]


class OrBertLayer(C.Structure):
    _fields_ = [("attn_q", OrWeight), ("attn_k", OrWeight), ("attn_v", OrWeight), ("attn_out", OrWeight),
                ("attn_q_bias", _vp), ("attn_k_bias", _vp), ("attn_v_bias", _vp), ("attn_out_bias", _vp),
                ("attn_norm_w", _vp), ("attn_norm_b", _vp), ("ffn_up", OrWeight), ("ffn_down", OrWeight),
                ("ffn_up_bias", _vp), ("ffn_down_bias", _vp), ("ffn_norm_w", _vp), ("ffn_norm_b", _vp)]


class OrBert(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("n_embed", C.c_int32), ("n_heads", C.c_int32), ("n_ff", C.c_int32),
                ("n_context", C.c_int32), ("vocab_size", C.c_int32), ("tok_cls", C.c_int32), ("tok_sep", C.c_int32),
                ("eps", C.c_float), ("tok_embd", OrWeight), ("pos_embd", OrWeight), ("tok_types", OrWeight),
                ("emb_norm_w", _vp), ("emb_norm_b", _vp), ("layers", _vp)]


class Oracle:
    """The plain-C restatement."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build_oracle()
        L = C.CDLL(path)
        self.L = L
        L.or_fp16_to_fp32.restype = C.c_float
        L.or_fp16_to_fp32.argtypes = [C.c_uint16]
        L.or_fp32_to_fp16.restype = C.c_uint16
        L.or_fp32_to_fp16.argtypes = [C.c_float]
        L.or_f32_to_f16_row.argtypes = [_fp, _vp, C.c_int64]
        L.or_row_size.restype = C.c_int64
        L.or_row_size.argtypes = [C.c_int, C.c_int64]
        L.or_dequantize_row.argtypes = [C.c_int, _vp, _fp, C.c_int64]
        L.or_quantize_q8_0.argtypes = [_fp, C.c_int64, _vp]
        L.or_quantize_q8_K.argtypes = [_fp, C.c_int64, _vp]
        L.or_matvec_q.argtypes = [C.c_int, _vp, C.c_uint32, C.c_int, C.c_int, _vp, _fp, _fp]
        L.or_matvec.argtypes = [C.c_int, _vp, C.c_uint32, C.c_int, C.c_int, _fp, _fp]
        L.or_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        L.or_rope.argtypes = [_fp, C.c_int, C.c_int, C.c_int, C.c_int, _fp]
        L.or_swiglu.argtypes = [_fp, _fp, C.c_int]
        L.or_attention.argtypes = [_fp, _fp, _fp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _fp]
        L.or_state_new.restype = _vp
        L.or_state_new.argtypes = [C.POINTER(OrModel)]
        L.or_state_free.argtypes = [_vp]
        L.or_state_pos.argtypes = [_vp]
        L.or_state_set_pos.argtypes = [_vp, C.c_int]
        L.or_inference.argtypes = [_vp, C.c_int, _fp]
        L.or_state_trace.argtypes = [_vp, _fp]
        L.or_state_force.argtypes = [_vp, _vp, C.c_size_t, _vp]
        L.or_state_kv.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]
        L.or_state_kv_write.argtypes = [_vp, C.c_int, C.c_int, C.c_int, _vp, _vp]
        L.or_argmax.argtypes = [_fp, C.c_int]
        L.or_sampler_topp.argtypes = [_fp, C.c_int, C.c_float, C.c_float, C.c_int, C.c_float]
        L.or_layernorm.argtypes = [_fp, _fp, _fp, _fp, C.c_int, C.c_float]
        L.or_bert_embed.argtypes = [C.POINTER(OrBert), _vp, C.c_int, _fp]
        L.or_bert_embed_traced.argtypes = [C.POINTER(OrBert), _vp, C.c_int, _fp, _fp]
        L.or_vdb_search.argtypes = [_vp, C.c_int, C.c_int, _fp, C.c_float, C.c_int, _vp, _fp]

    # --- scalar helpers
    def fp16_to_fp32(self, h: np.ndarray) -> np.ndarray:
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.size, np.float32)
        self.L.or_dequantize_row(1, h.ctypes.data, out.ctypes.data_as(_fp), h.size)
        return out

    def fp32_to_fp16(self, x: np.ndarray) -> np.ndarray:
        x, px = _f32(x)
        out = np.empty(x.size, np.uint16)
        self.L.or_f32_to_f16_row(px, out.ctypes.data, x.size)
        return out

    def row_size(self, t: int, n: int) -> int:
        return int(self.L.or_row_size(t, n))

    def dequantize_row(self, t: int, data: np.ndarray, n: int) -> np.ndarray:
        data = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.empty(n, np.float32)
        rc = self.L.or_dequantize_row(t, data.ctypes.data, out.ctypes.data_as(_fp), n)
        assert rc == 0
        return out

    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        x, px = _f32(x)
        out = np.empty(x.size // 32 * 34, np.uint8)
        self.L.or_quantize_q8_0(px, x.size, out.ctypes.data)
        return out

    def quantize_q8_K(self, x: np.ndarray) -> np.ndarray:
        x, px = _f32(x)
        out = np.empty(x.size // 256 * 292, np.uint8)
        self.L.or_quantize_q8_K(px, x.size, out.ctypes.data)
        return out

    def matvec_q(self, t: int, w: np.ndarray, rsz: int, n: int, d: int, xq: np.ndarray, want_abs=False):
        w = np.ascontiguousarray(w)
        xq = np.ascontiguousarray(xq)
        out = np.empty(d, np.float32)
        ab = np.empty(d, np.float32)
        rc = self.L.or_matvec_q(t, w.ctypes.data, rsz, n, d, xq.ctypes.data, out.ctypes.data_as(_fp),
                                ab.ctypes.data_as(_fp))
        assert rc == 0
        return (out, ab) if want_abs else out

    def matvec(self, t: int, w: np.ndarray, rsz: int, n: int, d: int, x: np.ndarray) -> np.ndarray:
        w = np.ascontiguousarray(w)
        x, px = _f32(x)
        out = np.empty(d, np.float32)
        assert self.L.or_matvec(t, w.ctypes.data, rsz, n, d, px, out.ctypes.data_as(_fp)) == 0
        return out

    def rmsnorm(self, x, w, eps):
        x, px = _f32(x)
        w, pw = _f32(w)
        out = np.empty(x.size, np.float32)
        self.L.or_rmsnorm(out.ctypes.data_as(_fp), px, pw, x.size, eps)
        return out

    def rope(self, x, n_heads, head_dim, rope_dim, pos, freq):
        x = np.array(x, dtype=np.float32, copy=True)
        freq, pf = _f32(freq)
        self.L.or_rope(x.ctypes.data_as(_fp), n_heads, head_dim, rope_dim, pos, pf)
        return x

    def swiglu(self, hb, hb2):
        hb = np.array(hb, dtype=np.float32, copy=True)
        hb2, p2 = _f32(hb2)
        self.L.or_swiglu(hb.ctypes.data_as(_fp), p2, hb.size)
        return hb

    def attention(self, q, k, v, kc, vc, n_heads, n_kv_heads, head_dim, pos):
        q, pq = _f32(q)
        k, pk = _f32(k)
        v, pv = _f32(v)
        kc = np.ascontiguousarray(kc, dtype=np.uint16)
        vc = np.ascontiguousarray(vc, dtype=np.uint16)
        out = np.empty(n_heads * head_dim, np.float32)
        self.L.or_attention(pq, pk, pv, kc.ctypes.data, vc.ctypes.data, n_heads, n_kv_heads, head_dim, pos,
                            out.ctypes.data_as(_fp))
        return out

    def argmax(self, x) -> int:
        x, px = _f32(x)
        return int(self.L.or_argmax(px, x.size))

    def sampler_topp(self, logits, temp: float, topp: float, topk: int, r01: float) -> int:
        x, px = _f32(logits)
        return int(self.L.or_sampler_topp(px, x.size, temp, topp, topk, r01))

    # --- BERT / vector memory
    def layernorm(self, x, w, b, eps):
        x, px = _f32(x)
        w, pw = _f32(w)
        b, pb = _f32(b)
        out = np.empty(x.size, np.float32)
        self.L.or_layernorm(out.ctypes.data_as(_fp), px, pw, pb, x.size, eps)
        return out

    def bert_embed(self, hb, toks) -> np.ndarray:
        """or_bert_embed of a HostBert (ligguf_amd.bert) for bert_tokenize's ids"""
        d = hb.fill_desc(OrBert, OrBertLayer, OrWeight)
        a = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty(hb.cfg.n_embed, np.float32)
        assert self.L.or_bert_embed(C.byref(d), a.ctypes.data, a.size, out.ctypes.data_as(_fp)) == 0
        return out

    def bert_embed_traced(self, hb, toks):
        """(embedding, trace [n_layers][4][T][max(n_embed, n_ff)]): the float
        vectors at the four quantization points of each block"""
        c = hb.cfg
        d = hb.fill_desc(OrBert, OrBertLayer, OrWeight)
        a = np.ascontiguousarray(toks, dtype=np.int32)
        T = min(a.size, c.n_context - 2) + 2
        tr = np.zeros((c.n_layers, 4, T, max(c.n_embed, c.n_ff)), np.float32)
        out = np.empty(c.n_embed, np.float32)
        assert self.L.or_bert_embed_traced(C.byref(d), a.ctypes.data, a.size, out.ctypes.data_as(_fp),
                                           tr.ctypes.data_as(_fp)) == 0
        return out, tr

    def vdb_search(self, vecs, emb, thr: float, k: int):
        v = np.ascontiguousarray(vecs, dtype=np.uint16)
        e, pe = _f32(emb)
        idx = np.empty(k, np.int32)
        sim = np.empty(k, np.float32)
        n = self.L.or_vdb_search(v.ctypes.data, v.shape[0] if v.ndim == 2 else v.size // e.size, e.size, pe, thr, k,
                                 idx.ctypes.data, sim.ctypes.data_as(_fp))
        return idx[:n].copy(), sim[:n].copy()

    # --- whole engine
    def new_state(self, model_struct: OrModel):
        self._keep = model_struct
        return self.L.or_state_new(C.byref(model_struct))

    def free_state(self, st):
        self.L.or_state_free(st)

    def inference(self, st, tok: int, vocab: int) -> np.ndarray:
        out = np.empty(vocab, np.float32)
        rc = self.L.or_inference(st, tok, out.ctypes.data_as(_fp))
        assert rc == 0
        return out

    def inference_traced(self, st, tok: int, cfg):
        """inference() plus the float vector before each of its 4 n_layers + 1
        activation quantizations: (logits, trace [4 L + 1][max(n_embed, n_ff)])."""
        wide = max(cfg.n_embed, cfg.n_ff)
        tr = np.zeros((4 * cfg.n_layers + 1, wide), np.float32)
        self.L.or_state_trace(st, tr.ctypes.data_as(_fp))
        out = self.inference(st, tok, cfg.vocab)
        return out, tr

    def inference_forced(self, st, tok: int, cfg, acts: np.ndarray, forms):
        """inference_traced() with the quantized activations of `acts`
        ([4 L + 1][stride] bytes, block_q8_K / block_q8_0) in place of the
        step's own at every point whose form in `forms` is Q8_K or Q8_0
        (None / 0: the step quantizes its own): (logits, trace)."""
        acts = np.ascontiguousarray(acts, dtype=np.uint8)
        fm = np.array([f or 0 for f in forms], np.int32)
        assert acts.ndim == 2 and acts.shape[0] == len(fm) == 4 * cfg.n_layers + 1
        self.L.or_state_force(st, acts.ctypes.data, acts.shape[1], fm.ctypes.data)
        return self.inference_traced(st, tok, cfg)

    def state_kv_write(self, st, layer, p0, np_, k, v):
        k = np.ascontiguousarray(k, dtype=np.uint16)
        v = np.ascontiguousarray(v, dtype=np.uint16)
        self.L.or_state_kv_write(st, layer, p0, np_, k.ctypes.data, v.ctypes.data)

    def state_kv(self, st, layer, p0, np_, kv_dim):
        k = np.empty(np_ * kv_dim, np.uint16)
        v = np.empty(np_ * kv_dim, np.uint16)
        self.L.or_state_kv(st, layer, p0, np_, k.ctypes.data, v.ctypes.data)
        return k, v


class RefWeight(C.Structure):
    _fields_ = [("ptr", _vp), ("type", C.c_int32), ("rsz", C.c_uint32)]


class RefLayer(C.Structure):
    _fields_ = [("att_norm", _vp), ("att_q", RefWeight), ("att_k", RefWeight), ("att_v", RefWeight),
                ("att_out", RefWeight), ("att_q_norm", _vp), ("att_k_norm", _vp), ("ffn_norm", _vp),
                ("ffn_up", RefWeight), ("ffn_down", RefWeight), ("ffn_gate", RefWeight)]


class RefModel(C.Structure):
    _fields_ = [("qwen3", C.c_int32), ("n_layers", C.c_int32), ("n_embed", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("kv_dim", C.c_int32), ("n_ff", C.c_int32),
                ("vocab_size", C.c_int32), ("n_context", C.c_int32), ("rope_dim", C.c_int32),
                ("rms_epsilon", C.c_float), ("rope_base", C.c_float), ("embed", RefWeight), ("output", RefWeight),
                ("output_norm", _vp), ("layers", _vp)]


class Reference:
    """The reference FAST engine, built from its own sources (oracle/_ref).

    Loading it also loads the -Ofast start-up code that sets flush-to-zero in
    the loading thread, as it does in the reference binary."""

    def __init__(self, path: str = REF_SO):
        L = C.CDLL(path)
        self.L = L
        L.ref_init.argtypes = []
        L.ref_fp16_to_fp32.restype = C.c_float
        L.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        L.ref_f32_to_f16_row.argtypes = [_fp, _vp, C.c_int]
        L.ref_f16_to_f32_row.argtypes = [_vp, _fp, C.c_int]
        L.ref_dequantize_row.argtypes = [C.c_int, _vp, _fp, C.c_int64]
        L.ref_quantize_q8_0.argtypes = [_fp, C.c_int, _vp]
        L.ref_quantize_q8_K.argtypes = [_fp, C.c_int, _vp]
        L.ref_bert_open.argtypes = [C.c_char_p]
        L.ref_bert_n_embed.argtypes = []
        L.ref_bert_tokenize.argtypes = [C.c_char_p, _vp, C.c_int]
        L.ref_bert_embed.argtypes = [C.c_char_p, _fp, C.c_int]
        L.ref_vdb_create.argtypes = [C.c_char_p]
        L.ref_vdb_entry.argtypes = [C.c_int, _vp, _vp, C.c_int]
        L.ref_vdb_query.argtypes = [C.c_char_p, _vp, C.c_int]
        L.ref_matmul.argtypes = [C.c_int, _vp, C.c_uint32, C.c_int, C.c_int, _fp, _fp]
        L.ref_matmul_q.argtypes = [C.c_int, _vp, C.c_uint32, C.c_int, C.c_int, _vp, _fp]
        L.ref_rmsnorm.argtypes = [_fp, _fp, _fp, C.c_int, C.c_float]
        L.ref_rmsnorm_inplace.argtypes = [_fp, _fp, C.c_int, C.c_float]
        L.ref_softmax.argtypes = [_fp, C.c_int]
        L.ref_rope.argtypes = [_fp, C.c_int, C.c_int, C.c_int, C.c_int, _fp, C.c_int]
        L.ref_rope_freq.argtypes = [C.c_float, C.c_int, _fp]
        L.ref_attention.argtypes = [_fp, _fp, _fp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _fp, _fp]
        L.ref_model_open.argtypes = [C.c_char_p, C.c_int]
        L.ref_model_bind.argtypes = [C.POINTER(RefModel)]
        L.ref_model_info.argtypes = [_vp]
        L.ref_rope_freq_table.restype = _fp
        L.ref_inference.argtypes = [C.c_int, _fp]
        L.ref_get_pos.restype = C.c_int
        L.ref_set_pos.argtypes = [C.c_int]
        L.ref_kv_rows.argtypes = [C.c_int, C.c_int, C.c_int, _vp, _vp]
        L.ref_kv_write_rows.argtypes = [C.c_int, C.c_int, C.c_int, _vp, _vp]
        L.ref_state_save.argtypes = [C.c_char_p]
        L.ref_state_load.argtypes = [C.c_char_p]
        L.ref_logits.argtypes = [_fp]
        L.ref_sampler_greedy.restype = C.c_int
        L.ref_sampler_topp.restype = C.c_int
        L.ref_sampler_topp.argtypes = [_fp, C.c_int, C.c_float, C.c_float, C.c_int, C.c_uint]
        L.ref_init()

    def sampler_topp(self, logits, temp: float, topp: float, topk: int, seed: int) -> int:
        """the reference's sampler_topp over these logits after srand(seed)"""
        x, px = _f32(logits)
        return int(self.L.ref_sampler_topp(px, x.size, temp, topp, topk, seed))

    def fp16_to_fp32(self, h):
        h = np.ascontiguousarray(h, dtype=np.uint16)
        out = np.empty(h.size, np.float32)
        self.L.ref_f16_to_f32_row(h.ctypes.data, out.ctypes.data_as(_fp), h.size)
        return out

    def fp32_to_fp16(self, x):
        x, px = _f32(x)
        out = np.empty(x.size, np.uint16)
        self.L.ref_f32_to_f16_row(px, out.ctypes.data, x.size)
        return out

    def dequantize_row(self, t, data, n):
        data = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.empty(n, np.float32)
        self.L.ref_dequantize_row(t, data.ctypes.data, out.ctypes.data_as(_fp), n)
        return out

    def quantize_q8_0(self, x):
        x, px = _f32(x)
        out = np.empty(x.size // 32 * 34, np.uint8)
        self.L.ref_quantize_q8_0(px, x.size, out.ctypes.data)
        return out

    def quantize_q8_K(self, x):
        x, px = _f32(x)
        out = np.empty(x.size // 256 * 292, np.uint8)
        self.L.ref_quantize_q8_K(px, x.size, out.ctypes.data)
        return out

    def matmul(self, t, w, rsz, n, d, x):
        w = np.ascontiguousarray(w)
        x, px = _f32(x)
        out = np.empty(d, np.float32)
        self.L.ref_matmul(t, w.ctypes.data, rsz, n, d, px, out.ctypes.data_as(_fp))
        return out

    def matmul_q(self, t, w, rsz, n, d, xq):
        w = np.ascontiguousarray(w)
        xq = np.ascontiguousarray(xq)
        out = np.empty(d, np.float32)
        self.L.ref_matmul_q(t, w.ctypes.data, rsz, n, d, xq.ctypes.data, out.ctypes.data_as(_fp))
        return out

    def rmsnorm(self, x, w, eps):
        x, px = _f32(x)
        w, pw = _f32(w)
        out = np.empty(x.size, np.float32)
        self.L.ref_rmsnorm(out.ctypes.data_as(_fp), px, pw, x.size, eps)
        return out

    def rmsnorm_inplace(self, x, w, eps):
        x = np.array(x, dtype=np.float32, copy=True)
        w, pw = _f32(w)
        self.L.ref_rmsnorm_inplace(x.ctypes.data_as(_fp), pw, x.size, eps)
        return x

    def softmax(self, x):
        x = np.array(x, dtype=np.float32, copy=True)
        self.L.ref_softmax(x.ctypes.data_as(_fp), x.size)
        return x

    def rope(self, x, n_heads, head_dim, rope_dim, pos, freq):
        x = np.array(x, dtype=np.float32, copy=True)
        freq, pf = _f32(freq)
        self.L.ref_rope(x.ctypes.data_as(_fp), n_heads, head_dim, rope_dim, pos, pf, freq.size)
        return x

    def rope_freq(self, base, rope_dim):
        out = np.empty(rope_dim // 2, np.float32)
        self.L.ref_rope_freq(base, rope_dim, out.ctypes.data_as(_fp))
        return out

    def attention(self, q, k, v, kc, vc, n_heads, n_kv_heads, head_dim, pos):
        q, pq = _f32(q)
        k, pk = _f32(k)
        v, pv = _f32(v)
        kc = np.ascontiguousarray(kc, dtype=np.uint16)
        vc = np.ascontiguousarray(vc, dtype=np.uint16)
        out = np.empty(n_heads * head_dim, np.float32)
        scratch = np.empty(n_heads * (pos + 1), np.float32)
        self.L.ref_attention(pq, pk, pv, kc.ctypes.data, vc.ctypes.data, n_heads, n_kv_heads, head_dim, pos,
                             out.ctypes.data_as(_fp), scratch.ctypes.data_as(_fp))
        return out

    def model_open(self, path: str, n_ctx: int = 0) -> None:
        rc = self.L.ref_model_open(path.encode(), n_ctx)
        if rc != 0:
            raise RuntimeError(f"reference could not open {path}: {rc}")

    def model_bind(self, m: RefModel) -> None:
        self._keep = m
        assert self.L.ref_model_bind(C.byref(m)) == 0

    def model_info(self) -> dict:
        o = np.zeros(13, np.int32)
        self.L.ref_model_info(o.ctypes.data)
        keys = ["n_layers", "n_embed", "n_heads", "n_kv_heads", "head_dim", "kv_dim", "n_ff", "vocab_size",
                "n_context", "rope_dim", "qwen3", "tok_eos", "pos"]
        return dict(zip(keys, (int(v) for v in o)))

    def rope_freq_table(self, rope_dim: int) -> np.ndarray:
        p = self.L.ref_rope_freq_table()
        return np.ctypeslib.as_array(p, shape=(rope_dim // 2,)).copy()

    def inference(self, tok: int, vocab: int) -> np.ndarray:
        out = np.empty(vocab, np.float32)
        self.L.ref_inference(tok, out.ctypes.data_as(_fp))
        return out

    def set_pos(self, pos: int) -> None:
        self.L.ref_set_pos(pos)

    def get_pos(self) -> int:
        return int(self.L.ref_get_pos())

    def state_save(self, path: str) -> None:
        assert self.L.ref_state_save(path.encode()) == 0, path

    def state_load(self, path: str) -> None:
        assert self.L.ref_state_load(path.encode()) == 0, path

    def logits(self, vocab: int) -> np.ndarray:
        out = np.empty(vocab, np.float32)
        self.L.ref_logits(out.ctypes.data_as(_fp))
        return out

    # --- BERT / vector memory (fast/vdb.cpp, through oracle/ref_bert.cpp)
    def bert_open(self, path: str) -> int:
        """vdb_set_model + ensure_bert; returns n_embed"""
        assert self.L.ref_bert_open(path.encode()) == 0, path
        return int(self.L.ref_bert_n_embed())

    def bert_tokenize(self, text: bytes) -> list:
        cap = 4 * len(text) + 16
        out = np.empty(cap, np.int32)
        n = self.L.ref_bert_tokenize(text, out.ctypes.data, cap)
        return [int(x) for x in out[:n]]

    def bert_embed(self, text: bytes) -> np.ndarray:
        ne = int(self.L.ref_bert_n_embed())
        out = np.empty(ne, np.float32)
        assert self.L.ref_bert_embed(text, out.ctypes.data_as(_fp), ne) == ne
        return out

    def vdb_create(self, log: bytes) -> int:
        return int(self.L.ref_vdb_create(log))

    def vdb_entry(self, i: int):
        ne = int(self.L.ref_bert_n_embed())
        ts = C.c_uint32()
        vec = np.empty(ne, np.uint16)
        assert self.L.ref_vdb_entry(i, C.byref(ts), vec.ctypes.data, ne) == ne
        return int(ts.value), vec

    def vdb_query(self, text: bytes) -> list:
        idx = np.empty(16, np.int32)
        n = self.L.ref_vdb_query(text, idx.ctypes.data, 16)
        return [int(x) for x in idx[:n]]

    def kv_rows(self, layer, p0, np_, kv_dim):
        k = np.empty(np_ * kv_dim, np.uint16)
        v = np.empty(np_ * kv_dim, np.uint16)
        self.L.ref_kv_rows(layer, p0, np_, k.ctypes.data, v.ctypes.data)
        return k, v


_oracle = None
_ref = None


def load_oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def load_reference() -> Reference:
    global _ref
    if _ref is None:
        _ref = Reference()
    return _ref
