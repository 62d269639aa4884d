"""The reference's state file (save_model_state / load_model_state,
fast/ligguf_fast_qk.cpp:216-302) written and read by the device cache
(lg_state_save / lg_state_load), exchanged with the reference engine in both
directions, and a GGUF file taken end to end through the host loader to the
device (HostModel.from_gguf -> lg_load_model -> bit-exact dequantization)."""
import os

import numpy as np
import pytest

from conftest import golden
from ligguf_amd import ops
from ligguf_amd.lib import PATH_FUSED, PATH_MULTI, LgError
from ligguf_amd.model import TINY, Engine, HostModel
from test_gpu_decode import rel
from test_gpu_ops import dev, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny_state(gpu, tmp_path_factory):
    g = golden("tiny_decode.npz")
    hm = HostModel.synthetic(TINY)
    hm.rope_freq = g["rope_freq"]
    d = tmp_path_factory.mktemp("state")
    path = str(d / "tiny.gguf")
    hm.write_gguf(path)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng, g, d, path
    eng.close()


def test_state_roundtrip_on_device(tiny_state):
    """Save after 20 steps, load into a second context: cache rows, logits and
    the next step equal bit for bit."""
    hm, eng, g, d, _ = tiny_state
    toks = np.concatenate([g["prompt"], g["greedy"][:4]])
    for p, t in enumerate(toks):
        lg = eng.decode(int(t), p)
    fn = str(d / "gpu.state")
    eng.state_save(fn, len(toks))
    assert os.path.getsize(fn) == 24 + 2 * TINY.n_layers * len(toks) * TINY.kv_dim * 2 + TINY.vocab * 4
    other = Engine(0)
    other.load(hm)
    pos, lg2 = other.state_load(fn)
    assert pos == len(toks) and np.array_equal(lg2, lg)
    k1, v1 = eng.kv_read(0, TINY.n_layers, 0, pos)
    k2, v2 = other.kv_read(0, TINY.n_layers, 0, pos)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    assert other.argmax() == int(np.argmax(lg))        # greedy over the loaded logits
    nxt = int(g["greedy"][4])
    assert np.array_equal(eng.decode(nxt, pos), other.decode(nxt, pos))
    other.close()


def test_state_device_to_reference(tiny_state, reference):
    """The reference loads the device's file, saves it again byte for byte,
    and its next step agrees with the device's."""
    hm, eng, g, d, path = tiny_state
    toks = g["prompt"]
    for p, t in enumerate(toks):
        lg = eng.decode(int(t), p)
    fn, back = str(d / "to_ref.state"), str(d / "ref_again.state")
    eng.state_save(fn, len(toks))
    reference.model_open(path, 0)
    reference.state_load(fn)
    assert reference.get_pos() == len(toks)
    assert np.array_equal(reference.logits(TINY.vocab), lg)
    reference.state_save(back)
    assert open(fn, "rb").read() == open(back, "rb").read()
    nxt = int(g["greedy"][0])
    a = eng.decode(nxt, len(toks))
    b = reference.inference(nxt, TINY.vocab)
    print(f"\nnext step after the reference loaded the device state: rel-L2 {rel(a, b):.2e}")
    assert rel(a, b) <= 3e-2 and int(np.argmax(a)) == int(np.argmax(b))


def test_state_reference_to_device(tiny_state, reference):
    """The device loads the reference's file: rows and logits bit for bit,
    then the next step on the fused-or-multi path agrees with the
    reference's."""
    hm, eng, g, d, path = tiny_state
    reference.model_open(path, 0)
    toks = np.concatenate([g["prompt"], g["greedy"][:8]])
    for t in toks:
        ref_lg = reference.inference(int(t), TINY.vocab)
    fn = str(d / "from_ref.state")
    reference.state_save(fn)
    pos, lg = eng.state_load(fn)
    assert pos == len(toks)
    assert np.array_equal(lg, ref_lg)
    for l in range(TINY.n_layers):
        k, v = reference.kv_rows(l, 0, pos, TINY.kv_dim)
        k2, v2 = eng.kv_read(l, 1, 0, pos)
        assert np.array_equal(k, k2) and np.array_equal(v, v2)
    nxt = int(g["greedy"][8])
    a = eng.decode(nxt, pos)
    b = reference.inference(nxt, TINY.vocab)
    assert rel(a, b) <= 3e-2 and int(np.argmax(a)) == int(np.argmax(b))


def test_state_rejects_bad_files(tiny_state):
    hm, eng, g, d, _ = tiny_state
    eng.decode(1, 0)
    with pytest.raises(LgError):
        eng.state_save(str(d / "empty.state"), 0)                 # an empty state, as the reference refuses
    fn = str(d / "ok.state")
    eng.state_save(fn, 1)
    raw = open(fn, "rb").read()
    bad = str(d / "bad.state")
    with open(bad, "wb") as f:
        f.write(raw[:100])                                        # truncated
    with pytest.raises(LgError):
        eng.state_load(bad)
    # a file cut inside the V blocks: rejected before any block reaches the
    # cache, as load_model_state keeps the old state on a failed read
    k0, v0 = eng.kv_read(0, TINY.n_layers, 0, 1)
    other = str(d / "other.state")
    eng.decode(2, 0)                                              # another row 0 ...
    eng.state_save(other, 1)
    eng.kv_write(0, TINY.n_layers, 0, 1, k0, v0)                  # ... and back
    raw2 = open(other, "rb").read()
    with open(bad, "wb") as f:
        f.write(raw2[:len(raw2) - TINY.vocab * 4 - 8])
    with pytest.raises(LgError, match="truncated"):
        eng.state_load(bad)
    k1, v1 = eng.kv_read(0, TINY.n_layers, 0, 1)
    assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
    hdr = bytearray(raw)
    hdr[8:16] = (12345).to_bytes(8, "little")                     # kv_size of another model
    with open(bad, "wb") as f:
        f.write(bytes(hdr))
    with pytest.raises(LgError):
        eng.state_load(bad)
    with pytest.raises(LgError):
        eng.state_load(str(d / "missing.state"))


def test_gguf_file_to_device(gpu, tmp_path):
    """A GGUF written by the reference-compatible writer and read back through
    the host loader (HostModel.from_gguf, which maps the file as
    read_llama / read_qwen3 do, fast/lil_gguf.cpp:397-499), uploaded with
    lg_load_model: every tensor's rows dequantize on the device to the host
    oracle's values bit for bit, and the first step matches a context loaded
    from the synthetic tensors directly."""
    from ligguf_amd.model import ModelConfig
    from ligguf_amd.lib import Q4_K, Q6_K, Q8_0
    from oracle import load_oracle
    oracle = load_oracle()
    cfg = ModelConfig("qwen3-gguf-rt", 1, 2, 512, 8, 2, 64, 1024, 1000, 256, 1e6, 1e-6, Q4_K, Q8_0, Q6_K)
    hm = HostModel.synthetic(cfg)
    path = str(tmp_path / "m.gguf")
    hm.write_gguf(path)
    hf = HostModel.from_gguf(path)
    assert hf.cfg.n_layers == 2 and hf.cfg.vocab == 1000 and hf.cfg.layer_type == Q4_K
    for name, (t, rows, cols, data) in hf.weights.items():
        t0, r0, c0, d0 = hm.weights[name]
        assert (t, rows, cols) == (t0, r0, c0)
        raw = np.frombuffer(data, np.uint8)
        assert np.array_equal(raw, np.asarray(d0, np.uint8).ravel()), name
        rsz = raw.size // rows
        for r in (0, rows - 1):
            row = np.ascontiguousarray(raw[r * rsz:(r + 1) * rsz])
            got = host(ops.dequantize_row(t, dev(row, gpu), cols))
            assert np.array_equal(got.view(np.uint32), oracle.dequantize_row(t, row, cols).view(np.uint32)), name
    a, b = Engine(0), Engine(0)
    a.load(hf)
    b.load(hm)
    for e in (a, b):
        e.set_path(PATH_MULTI)
    assert np.array_equal(a.decode(5, 0), b.decode(5, 0))
    a.close()
    b.close()
