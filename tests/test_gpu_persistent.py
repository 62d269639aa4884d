"""The persistent one-launch-per-token decode kernel (LG_PATH_PERSISTENT)
against the oracle and against the multi-kernel path.

Both GPU paths compute the matvecs, norms and quantizers with the same slot
order and lane reductions; attention differs in fp32 order only (the
persistent kernel runs one online-softmax pass per unit, the multi-kernel
path a three-pass softmax per chunk).  So on the same KV state their logits
agree to ~1e-7 except where that rounding moves one activation across an
int8 rounding boundary (see test_gpu_decode.py): the bounds below are the
one-step parity bounds used against the oracle."""
import numpy as np
import pytest

from ligguf_amd.lib import PATH_MULTI, PATH_PERSISTENT, Q1_G, Q4_K, Q5_K, Q6_K, Q8_0
from ligguf_amd.model import Engine, HostModel, ModelConfig
from test_gpu_decode import one_step_errors, rel

pytestmark = pytest.mark.gpu

# two-layer models at the Qwen3-8B widths the persistent kernel is built for
PK_MODELS = [
    ModelConfig("qwen3-w4096-q4k", 1, 2, 4096, 32, 8, 128, 12288, 2048, 4096, 1e6, 1e-6, Q4_K, Q4_K, Q6_K),
    ModelConfig("qwen3-w4096-q1g", 1, 2, 4096, 32, 8, 128, 12288, 2048, 4096, 1e6, 1e-6, Q1_G, Q8_0, Q8_0,
                q1_direct=True),
    ModelConfig("llama-w4096-q5k", 0, 1, 4096, 32, 32, 128, 12288, 1024, 1024, 1e4, 1e-5, Q5_K, Q8_0, Q4_K),
]


@pytest.fixture(scope="module", params=PK_MODELS, ids=lambda c: c.name)
def pk_model(request, gpu):
    cfg = request.param
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng
    eng.close()


def test_persistent_path_available(pk_model):
    hm, eng = pk_model
    eng.set_path(PATH_PERSISTENT)
    assert eng.path() == PATH_PERSISTENT
    eng.set_path(PATH_MULTI)
    assert eng.path() == PATH_MULTI


def test_persistent_one_step_parity_with_oracle(pk_model, oracle):
    hm, eng = pk_model
    eng.set_path(PATH_PERSISTENT)
    toks = np.random.default_rng(5).integers(1, hm.cfg.vocab, 6)
    errs, agree = one_step_errors(eng, oracle, hm, toks)
    print(f"\n{hm.cfg.name}: median {np.median(errs):.2e} max {errs.max():.2e}")
    assert np.median(errs) <= 1e-5
    assert errs.max() <= 2e-2
    assert agree.mean() >= 0.8


def run_both(eng, toks, pos0=0):
    """Greedy-free replay of toks on each path from a zeroed cache: logits of
    every step and the in-kernel argmax."""
    out = {}
    for path in (PATH_MULTI, PATH_PERSISTENT):
        eng.set_path(path)
        logits, am = [], []
        for i, t in enumerate(toks):
            logits.append(eng.decode(int(t), pos0 + i))
            am.append(eng.argmax())
        out[path] = (np.array(logits), am)
    return out


def test_persistent_matches_multikernel(pk_model):
    hm, eng = pk_model
    toks = np.random.default_rng(11).integers(1, hm.cfg.vocab, 12)
    out = run_both(eng, toks)
    lm, am = out[PATH_MULTI]
    lp, ap = out[PATH_PERSISTENT]
    errs = np.array([rel(a, b) for a, b in zip(lp, lm)])
    print(f"\n{hm.cfg.name}: persistent vs multi median {np.median(errs):.2e} max {errs.max():.2e}")
    assert np.median(errs) <= 1e-6
    assert errs.max() <= 2e-2
    assert np.mean(np.array(ap) == np.array(am)) >= 0.9
    # the in-kernel greedy reduction is exactly sampler_greedy on its own logits
    assert ap == [int(np.argmax(v)) for v in lp]


def test_persistent_long_context_attention(pk_model):
    """Decode at a long position over a random fp16 cache: the persistent
    split (one unit per workgroup, chunks up to 512) against the multi-kernel
    split (about 64 chunks), from the same cache rows."""
    hm, eng = pk_model
    cfg = hm.cfg
    pos = min(cfg.n_context - 1, 3001)
    rng = np.random.default_rng(2)
    for l in range(cfg.n_layers):
        k = rng.standard_normal(pos * cfg.kv_dim).astype(np.float16).view(np.uint16)
        v = rng.standard_normal(pos * cfg.kv_dim).astype(np.float16).view(np.uint16)
        eng.kv_write(l, 1, 0, pos, k, v)
    res = {}
    for path in (PATH_MULTI, PATH_PERSISTENT):
        eng.set_path(path)
        res[path] = eng.decode(7, pos)
        eng.set_path(PATH_MULTI)
    e = rel(res[PATH_PERSISTENT], res[PATH_MULTI])
    print(f"\n{cfg.name}: pos {pos} persistent vs multi {e:.2e}")
    assert e <= 2e-2


def test_persistent_prefill_equals_sequential_and_greedy(pk_model):
    """lg_prefill on the persistent path equals the same tokens fed one
    lg_decode_step at a time, bit for bit (feed_text's prompt loop,
    fast/ligguf_fast_qk.cpp:340-356), and the in-kernel greedy token of every
    step of a free-running loop is sampler_greedy of that step's logits."""
    hm, eng = pk_model
    eng.set_path(PATH_PERSISTENT)
    prompt = np.random.default_rng(9).integers(1, hm.cfg.vocab, 20)
    lg_prefill = eng.prefill(prompt, 0)
    for i, t in enumerate(prompt):
        lg_seq = eng.decode(int(t), i)
    assert np.array_equal(lg_prefill.view(np.uint32), lg_seq.view(np.uint32))
    tok, pos = int(np.argmax(lg_prefill)), len(prompt)
    for _ in range(12):
        lg = eng.decode(tok, pos)
        nxt = eng.argmax()
        assert nxt == int(np.argmax(lg))
        tok, pos = nxt, pos + 1
