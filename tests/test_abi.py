"""The C-ABI library: loads, exports every symbol the headers declare, and
rejects bad arguments with a status code (no GPU needed for these paths)."""
import ctypes as C
import os
import re

import pytest

from conftest import ROOT
from ligguf_amd import lib as L


def declared(header):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(lg[e]?_[A-Za-z0-9_]+)\s*\(", src)))


def test_hip_library_exports_every_declared_symbol():
    lib = L.load()
    names = declared("ligguf_hip.h")
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding covers all of them with signatures
    assert set(names) == set(L.SIGNATURES), set(names) ^ set(L.SIGNATURES)


def test_encode_library_exports_every_declared_symbol():
    from ligguf_amd import encode
    e = encode.load()
    missing = [n for n in declared("ligguf_encode.h") if not hasattr(e, n)]
    assert not missing, missing


def test_row_size_matches_reference_table():
    lib = L.load()
    for t, (qk, bs) in L.BLOCK.items():
        assert lib.lg_row_size(t, 4096) == 4096 // qk * bs
        if qk > 1:
            assert lib.lg_row_size(t, qk + 1) == -1
    assert lib.lg_row_size(99, 256) == -1


@pytest.mark.parametrize("call", [
    lambda lib: lib.lg_matvec(99, 1, 0, 256, 1, 1, 1, 0, None),          # unknown type
    lambda lib: lib.lg_matvec(L.Q4_K, 1, 144, 300, 1, 1, 1, 0, None),     # n not a block multiple
    lambda lib: lib.lg_matvec(L.Q4_K, 1, 100, 256, 1, 1, 1, 0, None),     # row size too small
    lambda lib: lib.lg_quantize_q8_K(1, 100, 1, None),                    # n % 256
    lambda lib: lib.lg_quantize_q8_0(1, 33, 1, None),                     # n % 32
    lambda lib: lib.lg_dequantize_row(L.Q8_K, 1, 1, 256, None),           # activation type
    lambda lib: lib.lg_rmsnorm_quant(1, 1, 300, 1e-6, L.Q8_K, 1, None, None),
    lambda lib: lib.lg_attn_decode(1, 1, 1, 1, 1, 6, 4, 128, 3, 1, 1, 1 << 20, None),   # heads not divisible
    lambda lib: lib.lg_attn_decode(1, 1, 1, 1, 1, 8, 2, 128, 3, 1, 1, 8, None),         # workspace too small
    lambda lib: lib.lg_attn_decode(1, 1, 1, 1, 1, 8, 2, 96, 3, 1, 1, 1 << 20, None),    # head_dim
    lambda lib: lib.lg_qk_norm_rope_kv(1, 1, 1, None, None, 4, 2, 6, 6, 0, 1, 1e-6, None, None, None),
    # partials beyond the fixed scratch area (checked before any device call)
    lambda lib: lib.lg_attn_decode_noalloc(1, 1, 1, 1, 1, 64, 8, 256, 1 << 20, 1, None),
])
def test_bad_arguments_return_errors(call):
    lib = L.load()
    rc = call(lib)
    assert rc in (L.ERRORS.keys()), rc
    assert lib.lg_last_error(None)


def test_null_context_errors():
    lib = L.load()
    assert lib.lg_decode_step(None, 0, 0, None) == -1
    assert lib.lg_load_model(None, None) == -1
    assert lib.lg_kv_read(None, 0, 1, 0, 1, None, None) == -1
    assert lib.lg_destroy(None) == 0
    t = C.c_int()
    assert lib.lg_argmax(None, C.byref(t)) == -1
    toks = (C.c_int * 4)()
    assert lib.lg_decode_greedy(None, 1, 0, 4, toks) == -1
    us = C.c_float()
    assert lib.lg_hbm_read_probe(None, 1 << 20, 1, C.byref(us), None) == -1      # no buffer
    assert lib.lg_hbm_read_probe(C.c_void_p(16), 1 << 20, 0, C.byref(us), None) == -1   # no passes
