"""The two full-size workloads on the GPU: the Qwen3-8B shape with Q4_K
layers and a Q6_K output head (36 layers, vocab 151936; 512-token prefill then
greedy decode -- the benchmark's workload) and the same shape with 1-bit
Q1_G layers and Q8_0 embedding/output at an 8192-token context.

Each checks, at its real size: the batched prefill against the
token-by-token one (within the distance between two correct token-by-token
paths that sum in different orders: over 36 layers the int8 rounding flips
that enter the KV caches of any two such paths grow to ~1e-1 in the logits); the fused and persistent whole-step kernels bit for bit
over a run of greedy steps; the in-kernel greedy token against
sampler_greedy of the step's logits (fast/ligguf_fast_qk.cpp:146-160, first
index wins); and single steps against the oracle from the GPU's own KV
state, every quantized activation compared (tests/parity.py) -- at 8200
positions that includes the long-context attention's output against the
oracle's exact attention.  Over 36 layers one flip moves the logits by up to
~5e-2 (against ~1e-2 over the two layers of the smaller models), so a step
whose first differing activation is a flip is held to FLIP_STEP_36."""
import numpy as np
import pytest

from ligguf_amd.lib import PATH_FUSED, PATH_MULTI, PATH_PERSISTENT, PREFILL_BATCHED, PREFILL_STEPS
from ligguf_amd.model import QWEN3_8B_Q1G, QWEN3_8B_Q4K, Engine, HostModel
from parity import EXACT_STEP, step_flips
from test_gpu_decode import oracle_state, rel

pytestmark = pytest.mark.gpu

# logits rel-L2 of a 36-layer step whose first differing activation is a
# rounding flip (5.0e-2 seen at position 512 of the Q4_K model)
FLIP_STEP_36 = 0.15


def prefill(eng, mode, prompt, pos0=0):
    eng.set_prefill_path(mode)
    return eng.prefill(prompt, pos0)


def oracle_check(eng, oracle, hm, pos, tok):
    """One traced step at pos on the GPU and in the oracle over the GPU's KV
    rows 0..pos-1 (all layers): (first differing activation, unexplained
    differences, logits rel-L2)."""
    cfg = hm.cfg
    st = oracle_state(oracle, hm)
    for l in range(cfg.n_layers):
        k, v = eng.kv_read(l, 1, 0, pos)
        oracle.state_kv_write(st, l, 0, pos, k, v)
    oracle.L.or_state_set_pos(st, pos)
    g, gtr = eng.decode_traced(tok, pos)
    o, otr = oracle.inference_traced(st, tok, cfg)
    oracle.free_state(st)
    first, bad = step_flips(gtr, otr, cfg)
    return first, bad, rel(g, o)


def greedy_run(eng, path, tok, pos, n):
    """n greedy steps from (tok, pos): tokens, logits, in-kernel argmax."""
    eng.set_path(path)
    toks, logits, am = [], [], []
    for i in range(n):
        lg = eng.decode(tok, pos + i)
        nxt = eng.argmax()
        logits.append(lg)
        am.append(nxt)
        toks.append(tok)
        tok = nxt
    return toks, np.array(logits), am


@pytest.fixture(scope="module")
def qwen_q4k(gpu):
    cfg = QWEN3_8B_Q4K.with_(n_context=1024)
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng
    eng.close()


def test_q4k_prefill_batched_vs_steps(qwen_q4k):
    """512 random ids: batched (int8 MFMA GEMMs) against token by token."""
    hm, eng = qwen_q4k
    cfg = hm.cfg
    prompt = np.random.default_rng(0).integers(1, cfg.vocab, 512).astype(np.int32)
    eng.set_path(PATH_MULTI)
    lg_m = prefill(eng, PREFILL_STEPS, prompt)
    eng.set_path(PATH_FUSED)
    lg_s = prefill(eng, PREFILL_STEPS, prompt)
    k_s, v_s = eng.kv_read(0, 1, 0, 512)
    lg_b = prefill(eng, PREFILL_BATCHED, prompt)
    k_b, v_b = eng.kv_read(0, 1, 0, 512)
    e, e_paths = rel(lg_b, lg_s), rel(lg_m, lg_s)
    eq0 = min(np.mean(k_s == k_b), np.mean(v_s == v_b))
    print(f"\nQwen3-8B Q4_K 512-token prefill: batched vs steps logits {e:.2e} (two step paths: {e_paths:.2e}), "
          f"layer-0 KV equal {eq0:.4f}")
    assert eq0 >= 0.99
    assert e <= max(2.0 * e_paths, 3e-2)


def test_q4k_decode_paths_and_oracle(qwen_q4k, oracle):
    """After the batched prefill: 16 greedy steps on the fused and the
    persistent kernels bit for bit, the in-kernel argmax = sampler_greedy of
    the logits, and the steps at 512 and 700 against the oracle."""
    hm, eng = qwen_q4k
    cfg = hm.cfg
    prompt = np.random.default_rng(0).integers(1, cfg.vocab, 512).astype(np.int32)
    lg = prefill(eng, PREFILL_BATCHED, prompt)
    tok0 = int(np.argmax(lg))
    runs = {}
    for path in (PATH_FUSED, PATH_PERSISTENT):
        prefill(eng, PREFILL_BATCHED, prompt)
        runs[path] = greedy_run(eng, path, tok0, 512, 16)
    tf, lf, af = runs[PATH_FUSED]
    tp, lp, ap = runs[PATH_PERSISTENT]
    assert np.array_equal(lf.view(np.uint32), lp.view(np.uint32))
    assert tf == tp and af == ap
    assert af == [int(np.argmax(v)) for v in lf]
    # one step against the oracle at 512 (over the prefilled cache) and at 700
    eng.set_path(PATH_FUSED)
    prefill(eng, PREFILL_BATCHED, prompt)
    res = [oracle_check(eng, oracle, hm, 512, tok0)]
    tok, pos = eng.argmax(), 513
    while pos < 700:
        eng.decode_async(tok, pos)
        tok = eng.argmax()
        pos += 1
    res.append(oracle_check(eng, oracle, hm, 700, tok))
    for (first, bad, e), p in zip(res, (512, 700)):
        print(f"\nQwen3-8B Q4_K step at {p} vs oracle: rel-L2 {e:.2e}, first int8 difference at activation {first}")
        assert not bad, bad[:5]
        assert e <= (EXACT_STEP if first < 0 else FLIP_STEP_36)


@pytest.fixture(scope="module")
def qwen_q1g(gpu):
    cfg = QWEN3_8B_Q1G.with_(n_context=8704)
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng
    eng.close()


def test_q1g_8k_context(qwen_q1g, oracle):
    """An 8192-token batched prefill, then 8 greedy steps (fused = persistent
    bit for bit, in-kernel argmax = sampler_greedy), then the step at 8200
    against the oracle: at that length the whole-step attention takes the
    long-context units merged in groups."""
    hm, eng = qwen_q1g
    cfg = hm.cfg
    prompt = np.random.default_rng(1).integers(1, cfg.vocab, 8192).astype(np.int32)
    assert eng.prefill_path() == PREFILL_BATCHED
    lg = prefill(eng, PREFILL_BATCHED, prompt)
    assert np.all(np.isfinite(lg))
    tok0 = int(np.argmax(lg))
    tf, lf, af = greedy_run(eng, PATH_FUSED, tok0, 8192, 8)
    # the persistent kernel over the same cache (rows 8192.. are rewritten identically)
    tp, lp, ap = greedy_run(eng, PATH_PERSISTENT, tok0, 8192, 8)
    assert np.array_equal(lf.view(np.uint32), lp.view(np.uint32))
    assert af == ap == [int(np.argmax(v)) for v in lf]
    eng.set_path(PATH_FUSED)
    first, bad, e = oracle_check(eng, oracle, hm, 8200, af[-1])
    print(f"\nQwen3-8B Q1_G step at 8200 vs oracle: rel-L2 {e:.2e}, first int8 difference at activation {first}")
    assert not bad, bad[:5]
    assert e <= (EXACT_STEP if first < 0 else FLIP_STEP_36)
    # and against the multi-kernel path from the same cache
    eng.set_path(PATH_MULTI)
    m = eng.decode(af[-1], 8200)
    eng.set_path(PATH_FUSED)
    f = eng.decode(af[-1], 8200)
    assert rel(f, m) <= FLIP_STEP_36
