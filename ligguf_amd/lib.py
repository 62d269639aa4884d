"""ctypes binding of libligguf_hip.so (include/ligguf_hip.h).

The library is loaded from this package directory only; there is no fallback
path: when it is missing or fails to load, every call raises.
"""
from __future__ import annotations

import ctypes as C
import os

PKG = os.path.dirname(os.path.abspath(__file__))
HIP_SO = os.path.join(PKG, "libligguf_hip.so")

LG_OK = 0
ERRORS = {-1: "LG_ERR_ARG", -2: "LG_ERR_TYPE", -3: "LG_ERR_HIP", -4: "LG_ERR_STATE", -5: "LG_ERR_NOMEM"}

# gguf_type codes (fast/lil_gguf.h:26-43)
F32, F16, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K, Q1_0, Q1_G = 0, 1, 8, 10, 11, 12, 13, 14, 15, 40, 41
TYPE_NAMES = {F32: "F32", F16: "F16", Q8_0: "Q8_0", Q2_K: "Q2_K", Q3_K: "Q3_K", Q4_K: "Q4_K", Q5_K: "Q5_K",
              Q6_K: "Q6_K", Q8_K: "Q8_K", Q1_0: "Q1_0", Q1_G: "Q1_G"}
BLOCK = {F32: (1, 4), F16: (1, 2), Q8_0: (32, 34), Q1_0: (32, 6), Q1_G: (128, 18), Q2_K: (256, 84),
         Q3_K: (256, 110), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210), Q8_K: (256, 292)}

ARCH_LLAMA, ARCH_QWEN3 = 0, 1
PATH_AUTO, PATH_PERSISTENT, PATH_MULTI, PATH_FUSED = 0, 1, 2, 3
PREFILL_AUTO, PREFILL_STEPS, PREFILL_BATCHED = 0, 1, 2

_vp = C.c_void_p


class LgError(RuntimeError):
    pass


class LgWeight(C.Structure):
    _fields_ = [("data", _vp), ("type", C.c_int32), ("rsz", C.c_uint32), ("rows", C.c_int32), ("cols", C.c_int32)]


class LgLayerDesc(C.Structure):
    _fields_ = [("att_norm", _vp), ("att_q", LgWeight), ("att_k", LgWeight), ("att_v", LgWeight),
                ("att_out", LgWeight), ("att_q_norm", _vp), ("att_k_norm", _vp), ("ffn_norm", _vp),
                ("ffn_up", LgWeight), ("ffn_down", LgWeight), ("ffn_gate", LgWeight)]


class LgModelDesc(C.Structure):
    _fields_ = [("arch", C.c_int32), ("n_layers", C.c_int32), ("n_embed", C.c_int32), ("n_heads", C.c_int32),
                ("n_kv_heads", C.c_int32), ("head_dim", C.c_int32), ("kv_dim", C.c_int32), ("n_ff", C.c_int32),
                ("vocab_size", C.c_int32), ("n_context", C.c_int32), ("rope_dim", C.c_int32),
                ("rms_epsilon", C.c_float), ("rope_freq", _vp), ("token_embd", LgWeight), ("output", LgWeight),
                ("output_norm", _vp), ("layers", _vp)]


class LgBertLayerDesc(C.Structure):
    _fields_ = [("attn_q", LgWeight), ("attn_k", LgWeight), ("attn_v", LgWeight), ("attn_out", LgWeight),
                ("attn_q_bias", _vp), ("attn_k_bias", _vp), ("attn_v_bias", _vp), ("attn_out_bias", _vp),
                ("attn_norm_w", _vp), ("attn_norm_b", _vp), ("ffn_up", LgWeight), ("ffn_down", LgWeight),
                ("ffn_up_bias", _vp), ("ffn_down_bias", _vp), ("ffn_norm_w", _vp), ("ffn_norm_b", _vp)]


class LgBertDesc(C.Structure):
    _fields_ = [("n_layers", C.c_int32), ("n_embed", C.c_int32), ("n_heads", C.c_int32), ("n_ff", C.c_int32),
                ("n_context", C.c_int32), ("vocab_size", C.c_int32), ("tok_cls", C.c_int32), ("tok_sep", C.c_int32),
                ("eps", C.c_float), ("tok_embd", LgWeight), ("pos_embd", LgWeight), ("tok_types", LgWeight),
                ("emb_norm_w", _vp), ("emb_norm_b", _vp), ("layers", _vp)]


# Every exported symbol of include/ligguf_hip.h with its ctypes signature.
SIGNATURES = {
    "lg_row_size": (C.c_int64, [C.c_int, C.c_int64]),
    "lg_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "lg_destroy": (C.c_int, [_vp]),
    "lg_last_error": (C.c_char_p, [_vp]),
    "lg_load_model": (C.c_int, [_vp, C.POINTER(LgModelDesc)]),
    "lg_decode_step": (C.c_int, [_vp, C.c_int, C.c_int, _vp]),
    "lg_decode_step_async": (C.c_int, [_vp, C.c_int, C.c_int]),
    "lg_sync": (C.c_int, [_vp]),
    "lg_logits_device": (_vp, [_vp]),
    "lg_argmax": (C.c_int, [_vp, C.POINTER(C.c_int)]),
    "lg_decode_greedy": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int)]),
    "lg_sample_topp": (C.c_int, [_vp, C.c_float, C.c_float, C.c_int, C.c_float, C.POINTER(C.c_int)]),
    "lg_sample_topp_device": (C.c_int, [_vp, C.c_int, C.c_float, C.c_float, C.c_int, C.c_float, C.POINTER(C.c_int)]),
    "lg_set_decode_path": (C.c_int, [_vp, C.c_int]),
    "lg_decode_path": (C.c_int, [_vp]),
    "lg_trace_next_step": (C.c_int, [_vp, _vp]),
    "lg_trace_size": (C.c_size_t, [_vp]),
    "lg_trace_acts_next_step": (C.c_int, [_vp, _vp]),
    "lg_trace_acts_next_prefill": (C.c_int, [_vp, _vp]),
    "lg_trace_acts_size": (C.c_size_t, [_vp]),
    "lg_time_fused_phase": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_float)]),
    "lg_hbm_read_probe": (C.c_int, [_vp, C.c_size_t, C.c_int, C.POINTER(C.c_float), _vp]),
    "lg_prefill": (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp]),
    "lg_set_prefill_path": (C.c_int, [_vp, C.c_int]),
    "lg_prefill_path": (C.c_int, [_vp]),
    "lg_kv_read": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "lg_kv_write": (C.c_int, [_vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "lg_state_save": (C.c_int, [_vp, C.c_char_p, C.c_int]),
    "lg_state_load": (C.c_int, [_vp, C.c_char_p, C.POINTER(C.c_int), _vp]),
    "lg_dequantize_row": (C.c_int, [C.c_int, _vp, _vp, C.c_int64, _vp]),
    "lg_quantize_q8_0": (C.c_int, [_vp, C.c_int64, _vp, _vp]),
    "lg_quantize_q8_K": (C.c_int, [_vp, C.c_int64, _vp, _vp]),
    "lg_matvec": (C.c_int, [C.c_int, _vp, C.c_uint32, C.c_int, C.c_int, _vp, _vp, C.c_int, _vp]),
    "lg_matmul_tokens": (C.c_int, [C.c_int, _vp, C.c_uint32, C.c_int, C.c_int, _vp, C.c_int, _vp, _vp]),
    "lg_rmsnorm_quant": (C.c_int, [_vp, _vp, C.c_int, C.c_float, C.c_int, _vp, _vp, _vp]),
    "lg_qk_norm_rope_kv": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, _vp,
                                     C.c_float, _vp, _vp, _vp]),
    "lg_attn_workspace_size": (C.c_size_t, [C.c_int, C.c_int, C.c_int]),
    "lg_attn_decode": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp,
                                 C.c_size_t, _vp]),
    "lg_attn_scratch_bytes": (C.c_size_t, []),
    "lg_attn_decode_noalloc": (C.c_int, [_vp, _vp, _vp, _vp, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp, _vp]),
    "lg_swiglu_quant": (C.c_int, [_vp, _vp, C.c_int, C.c_int, _vp, _vp]),
    "lg_bert_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "lg_bert_destroy": (C.c_int, [_vp]),
    "lg_bert_last_error": (C.c_char_p, [_vp]),
    "lg_bert_load": (C.c_int, [_vp, C.POINTER(LgBertDesc), C.c_int]),
    "lg_bert_embed": (C.c_int, [_vp, _vp, C.c_int, _vp]),
    "lg_bert_embed_batch": (C.c_int, [_vp, _vp, _vp, C.c_int, _vp]),
    "lg_bert_trace_size": (C.c_size_t, [_vp]),
    "lg_bert_trace_next": (C.c_int, [_vp, _vp]),
    "lg_bert_vdb_set": (C.c_int, [_vp, _vp, C.c_int, C.c_int]),
    "lg_bert_vdb_append": (C.c_int, [_vp, _vp, C.c_int, C.c_int]),
    "lg_bert_vdb_size": (C.c_int, [_vp]),
    "lg_bert_vdb_query": (C.c_int, [_vp, _vp, C.c_int, C.c_float, C.c_int, _vp, _vp]),
    "lg_bert_query": (C.c_int, [_vp, _vp, C.c_int, C.c_float, C.c_int, _vp, _vp, _vp]),
}

_lib = None


def load(path: str = HIP_SO) -> C.CDLL:
    """Load the in-tree HIP library (raises when it is missing)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LgError(f"{path} is not built: run `python -m ligguf_amd.build` (no CPU fallback exists)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int, ctx=None) -> None:
    if rc != LG_OK:
        lib = load()
        msg = lib.lg_last_error(ctx)
        raise LgError(f"{ERRORS.get(rc, rc)}: {msg.decode() if msg else ''}")


def row_size(t: int, n: int) -> int:
    qk, bs = BLOCK[t]
    if n % qk:
        return -1
    return n // qk * bs


def sample_topp_device(logits_ptr: int, n: int, temp: float, topp: float, topk: int, r01: float) -> int:
    """lg_sample_topp_device over n device floats at logits_ptr (e.g. a torch
    tensor's data_ptr()): the reference's sampler_topp on the device."""
    t = C.c_int()
    check(load().lg_sample_topp_device(C.c_void_p(logits_ptr), n, temp, topp, topk, r01, C.byref(t)))
    return int(t.value)
