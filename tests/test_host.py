"""Host-side pieces: weight encoders, synthetic models, GGUF files (read back
by our reader and by the reference loader when it is built)."""
import os

import numpy as np
import pytest

from ligguf_amd import encode
from ligguf_amd.lib import BLOCK, F16, F32, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, row_size
from ligguf_amd.model import QWEN3_8B_Q4K, TINY, HostModel, ModelConfig

# rms error of encode -> dequant relative to the signal, per format (min/max fits)
MAX_REL_ERR = {F32: 0, F16: 1e-3, Q8_0: 0.01, Q6_K: 0.03, Q5_K: 0.06, Q4_K: 0.12, Q3_K: 0.25, Q2_K: 0.45}


@pytest.mark.parametrize("t", list(MAX_REL_ERR))
def test_encoder_roundtrip(oracle, t):
    rows, cols = 32, 1024
    x = encode.normal(9, 3, rows * cols, 0.02)
    q = encode.quantize(t, x, rows, cols)
    rsz = row_size(t, cols)
    y = np.concatenate([oracle.dequantize_row(t, q[r * rsz:(r + 1) * rsz], cols) for r in range(rows)])
    err = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert err <= MAX_REL_ERR[t], err


@pytest.mark.parametrize("t", [Q1_0, Q1_G])
def test_one_bit_encoders(oracle, t):
    rows, cols = 8, 512
    x = encode.normal(9, 4, rows * cols, 0.02)
    q = encode.quantize(t, x, rows, cols)
    rsz = row_size(t, cols)
    y = np.concatenate([oracle.dequantize_row(t, q[r * rsz:(r + 1) * rsz], cols) for r in range(rows)])
    assert np.array_equal(np.sign(y), np.where(x >= 0, 1.0, -1.0))
    r = encode.random_q1(t, 1, 2, rows, cols, 0.02)
    assert r.size == rows * rsz
    yr = oracle.dequantize_row(t, r[:rsz], cols)
    assert np.all(np.abs(yr) > 0) and 0.3 < np.mean(yr > 0) < 0.7


def test_random_tensor_is_deterministic_and_thread_independent():
    a = encode.random_tensor(Q4_K, 5, 7, 64, 512)
    b = encode.random_tensor(Q4_K, 5, 7, 64, 512)
    c = encode.random_tensor(Q4_K, 5, 8, 64, 512)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    x = encode.normal(5, 7, 64 * 512, 0.02)
    assert np.array_equal(a, encode.quantize(Q4_K, x, 64, 512))


def test_weight_bytes_per_token_qwen3_8b():
    # 36 layers x 108.53 MB of Q4_K + Q6_K head + norms + one embedding row
    assert QWEN3_8B_Q4K.weight_bytes() == 4_418_734_336
    assert QWEN3_8B_Q4K.kv_bytes(511) == 512 * 147_456


def test_gguf_roundtrip(tmp_path):
    cfg = TINY.with_(n_layers=2, vocab=512, name="t2")
    hm = HostModel.synthetic(cfg)
    p = str(tmp_path / "m.gguf")
    hm.write_gguf(p)
    back = HostModel.from_gguf(p)
    assert back.cfg.n_layers == 2 and back.cfg.vocab == 512 and back.cfg.n_embed == cfg.n_embed
    for name, (t, rows, cols, data) in hm.weights.items():
        t2, r2, c2, d2 = back.weights[name]
        assert (t, rows, cols) == (t2, r2, c2) and np.array_equal(np.asarray(d2), data)
    assert np.array_equal(back.rope_freq, hm.rope_freq)


@pytest.mark.parametrize("cfg", [TINY.with_(n_layers=2, vocab=512, name="l2"),
                                 ModelConfig("q2", 1, 2, 256, 4, 2, 64, 512, 300, 64, 1e6, 1e-6, Q4_K, Q4_K, Q6_K)])
def test_reference_loader_reads_our_gguf(tmp_path, reference, oracle, cfg):
    """The reference's own mmap loader (read_gguf/read_llama/read_qwen3)
    accepts the file, and its first inference equals the oracle's."""
    from oracle.binding import OrLayer, OrModel, OrWeight
    hm = HostModel.synthetic(cfg)
    p = str(tmp_path / "m.gguf")
    hm.write_gguf(p)
    reference.model_open(p, 0)
    info = reference.model_info()
    assert info["n_layers"] == cfg.n_layers and info["n_embed"] == cfg.n_embed
    assert info["vocab_size"] == cfg.vocab and info["kv_dim"] == cfg.kv_dim and info["qwen3"] == cfg.arch
    hm.rope_freq = reference.rope_freq_table(cfg.rope_dim)
    st = oracle.new_state(hm.fill_desc(OrModel, OrLayer, OrWeight))
    a = oracle.inference(st, 3, cfg.vocab)
    b = reference.inference(3, cfg.vocab)
    assert np.linalg.norm(a - b) / np.linalg.norm(b) < 1e-5
    oracle.free_state(st)
