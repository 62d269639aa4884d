"""The batched prefill: lg_matmul_tokens (the int8 MFMA GEMMs of T tokens)
against the oracle's matvec of every token, and lg_prefill with
LG_PREFILL_BATCHED against the token-by-token prefill (LG_PREFILL_STEPS,
itself bit-equal to sequential decode steps) and against the oracle, for
models of every quantized layer type the GEMMs take (Q2_K..Q6_K, Q8_0,
Q1_0, Q1_G, F16, F32), a Q4_K_M-style mix and head_dim 48 / 64 / 128.

The GEMMs reproduce the integer (sub-)block sums of the reference's dots
exactly (fast/lil_math.cpp:411-739) and combine them in fp32 per block, so
each output is held to the matvec bar: within 2e-6 of the row's sum of
|terms|.  A whole prompt is held to the flip-explained bar
(tests/parity.py, prefill_flips): every quantized activation of every token
the pass builds before any difference can reach it equals the oracle's
token-by-token value or differs by a rounding flip, and a prompt without
any difference matches the oracle's logits to fp32 noise."""
import numpy as np
import pytest

from ligguf_amd import encode, ops
from ligguf_amd.lib import (F16, F32, PATH_AUTO, PATH_FUSED, PATH_MULTI, PREFILL_AUTO, PREFILL_BATCHED, PREFILL_STEPS,
                            Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, TYPE_NAMES, LgError, row_size)
from ligguf_amd.model import TINY, Engine, HostModel, ModelConfig
from parity import EXACT_STEP, prefill_flips, slot_formats
from test_gpu_decode import oracle_state, rel
from test_gpu_ops import MATVEC_TOL, dev, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,n,T", [(200, 512, 37), (130, 256, 1), (384, 12288, 5), (4096, 4096, 64),
                                   (6144, 4096, 100)])
def test_matmul_tokens_vs_oracle(gpu, oracle, d, n, T):
    rng = np.random.default_rng(d + T)
    w = encode.random_tensor(Q4_K, d + n, Q4_K, d, n)
    x = rng.standard_normal((T, n)).astype(np.float32)
    rsz = row_size(Q4_K, n)
    y = host(ops.matmul_tokens(Q4_K, dev(w, gpu), rsz, n, d, dev(x, gpu)))
    toks = range(T) if T <= 40 else rng.choice(T, 12, replace=False)
    for t in toks:
        ref, ab = oracle.matvec_q(Q4_K, w, rsz, n, d, oracle.quantize_q8_K(x[t]), want_abs=True)
        err = np.abs(y[t] - ref) / np.maximum(ab, 1e-30)
        assert np.all(err <= MATVEC_TOL), (t, float(err.max()))


@pytest.mark.parametrize("d,n,T", [(200, 512, 37), (130, 256, 1), (384, 12288, 5), (4096, 4096, 64)])
def test_matmul_tokens_q1g_vs_oracle(gpu, oracle, d, n, T):
    """The Q1_G x Q8_0 GEMM (one int8 MFMA per 32-value block) against the
    oracle's matvec of each token's Q8_0 activation."""
    rng = np.random.default_rng(d + T + 1)
    w = encode.random_tensor(Q1_G, d + n + 1, Q1_G, d, n)
    x = rng.standard_normal((T, n)).astype(np.float32)
    rsz = row_size(Q1_G, n)
    y = host(ops.matmul_tokens(Q1_G, dev(w, gpu), rsz, n, d, dev(x, gpu)))
    toks = range(T) if T <= 40 else rng.choice(T, 12, replace=False)
    for t in toks:
        ref, ab = oracle.matvec_q(Q1_G, w, rsz, n, d, oracle.quantize_q8_0(x[t]), want_abs=True)
        err = np.abs(y[t] - ref) / np.maximum(ab, 1e-30)
        assert np.all(err <= MATVEC_TOL), (t, float(err.max()))


# fp32 sums of n products in two orders differ by ~sqrt(n) 2^-24 of the sum of |terms| (3.8e-6 at 4096)
FLOAT_GEMM_TOL = 2e-5

GEMM_CASES = [(t, d, n, T) for t in (Q2_K, Q3_K, Q5_K, Q6_K)
              for d, n, T in [(200, 512, 37), (130, 256, 1), (4096, 4096, 64)]] + \
             [(t, d, n, T) for t in (Q8_0, Q1_0, F16, F32)
              for d, n, T in [(200, 288, 37), (130, 32, 1), (100, 1376, 70), (4096, 4096, 64)]]


@pytest.mark.parametrize("wt,d,n,T", GEMM_CASES,
                         ids=[f"{TYPE_NAMES[t]}-{d}x{n}-T{T}" for t, d, n, T in GEMM_CASES])
def test_matmul_tokens_types_vs_oracle(gpu, oracle, wt, d, n, T):
    """The K-quant GEMM (one int8 MFMA per 16- or 32-value sub-block, the
    sub-block scales in int32), the Q8_0 / Q1_0 GEMM (one per 32-value
    block, widths any multiple of 32) and the F16 / F32 GEMM (fp32 MFMA on
    the unquantized activation) against the oracle's matvec of each token."""
    rng = np.random.default_rng(d + n + T + wt)
    w = encode.random_tensor(wt, d + n + wt, wt, d, n)
    x = rng.standard_normal((T, n)).astype(np.float32)
    rsz = row_size(wt, n)
    y = host(ops.matmul_tokens(wt, dev(w, gpu), rsz, n, d, dev(x, gpu)))
    kq = wt in (Q2_K, Q3_K, Q5_K, Q6_K)
    toks = range(T) if T <= 40 else rng.choice(T, 12, replace=False)
    for t in toks:
        if wt in (F16, F32):
            ref = oracle.matvec(wt, w, rsz, n, d, x[t])
            wf = np.frombuffer(np.asarray(w, np.uint8).tobytes()[:d * rsz], np.float16 if wt == F16 else np.float32)
            ab = np.abs(wf.reshape(d, n).astype(np.float64)) @ np.abs(x[t].astype(np.float64))
            tol = FLOAT_GEMM_TOL
        else:
            xq = oracle.quantize_q8_K(x[t]) if kq else oracle.quantize_q8_0(x[t])
            ref, ab = oracle.matvec_q(wt, w, rsz, n, d, xq, want_abs=True)
            tol = MATVEC_TOL
        err = np.abs(y[t] - ref) / np.maximum(ab, 1e-30)
        assert np.all(err <= tol), (t, float(err.max()))


def test_matmul_tokens_rejects_other_types(gpu):
    x = dev(np.zeros((2, 256), np.float32), gpu)
    w = dev(np.zeros(row_size(Q8_0, 256) * 4, np.uint8), gpu)
    with pytest.raises(LgError):                 # Q8_K is an activation form, not a weight type
        ops.matmul_tokens(15, w, row_size(Q8_0, 256), 256, 4, x)
    with pytest.raises(LgError):                 # a K-quant row is a whole number of 256-value blocks
        ops.matmul_tokens(Q4_K, w, row_size(Q4_K, 256), 288, 4, dev(np.zeros((2, 288), np.float32), gpu))


BATCHED_MODELS = [
    ModelConfig("qwen3-w4096-q4k", 1, 2, 4096, 32, 8, 128, 12288, 2048, 4096, 1e6, 1e-6, Q4_K, Q4_K, Q6_K),
    ModelConfig("llama-w4096-q4k-nrep1", 0, 1, 4096, 32, 32, 128, 12288, 1024, 1024, 1e4, 1e-5, Q4_K, Q8_0, Q4_K),
    # the other query-head ratios of the prefill attention kernel: 2 (16/8 heads) and 8 (32/4)
    ModelConfig("qwen3-w2048-q4k-nrep2", 1, 1, 2048, 16, 8, 128, 6144, 1024, 1024, 1e6, 1e-6, Q4_K, Q4_K, Q6_K),
    ModelConfig("llama-w4096-q4k-nrep8", 0, 1, 4096, 32, 4, 128, 12288, 1024, 1024, 1e4, 1e-5, Q4_K, Q4_K, Q6_K),
    # Qwen3-14B widths: 5 query heads per KV head (40/8), FFN 17408
    ModelConfig("qwen3-w5120-q4k-nrep5", 1, 1, 5120, 40, 8, 128, 17408, 1024, 1024, 1e6, 1e-6, Q4_K, Q4_K, Q6_K),
    # Q1_G layers (Q1_G x Q8_0 GEMM), Q8_0 embedding and output
    ModelConfig("qwen3-w4096-q1g", 1, 2, 4096, 32, 8, 128, 12288, 2048, 4096, 1e6, 1e-6, Q1_G, Q8_0, Q8_0),
    # the tiny parity config: Q8_0 throughout, width 288 (no multiple of 256), head_dim 48
    TINY.with_(name="tiny-q8_0-hd48", n_context=1024),
    # Q4_K_M-style: Q6_K attn_v and ffn_down among Q4_K matrices (Q|K|V not stacked), head_dim 64
    ModelConfig("llama-w2048-q4k_m-hd64", 0, 2, 2048, 32, 8, 64, 5632, 1024, 1024, 1e4, 1e-5, Q4_K, Q4_K, Q6_K,
                overrides=(("attn_v", Q6_K), ("ffn_down", Q6_K))),
    # one K-quant type throughout each (a Q4_K embedding: a Q6_K one puts 60-80 of every 1024 first
    # activations on exact rounding ties, which end the flip walk at its first activation)
    ModelConfig("qwen3-w1024-q6k", 1, 2, 1024, 16, 8, 64, 2816, 1024, 1024, 1e6, 1e-6, Q6_K, Q4_K, Q6_K),
    ModelConfig("llama-w1024-q5k", 0, 2, 1024, 8, 8, 128, 2816, 1024, 1024, 1e4, 1e-5, Q5_K, Q5_K, Q6_K),
    ModelConfig("llama-w1024-q3k", 0, 2, 1024, 16, 4, 64, 2816, 1024, 1024, 1e4, 1e-5, Q3_K, Q4_K, Q6_K),
    ModelConfig("llama-w1024-q2k", 0, 2, 1024, 16, 4, 64, 2816, 1024, 1024, 1e4, 1e-5, Q2_K, Q4_K, Q6_K),
    # Q1_0 layers, and a mix of the two activation forms (Q8_0 ffn_down under Q4_K up|gate)
    ModelConfig("llama-w1024-q1_0", 0, 2, 1024, 16, 16, 64, 2816, 1024, 1024, 1e4, 1e-5, Q1_0, Q8_0, Q8_0),
    ModelConfig("qwen3-w1024-q4k-q8down", 1, 2, 1024, 8, 2, 128, 2816, 1024, 1024, 1e6, 1e-6, Q4_K, Q4_K, Q8_0,
                overrides=(("ffn_down", Q8_0), ("attn_output", Q8_0))),
    # unquantized layers (fp32 MFMA on the fp32 activations), one with a K-quant among them
    ModelConfig("llama-w1024-f16", 0, 2, 1024, 16, 4, 64, 2816, 1024, 1024, 1e4, 1e-5, F16, Q8_0, Q8_0),
    ModelConfig("llama-w512-f32-q4kdown", 0, 2, 512, 8, 8, 64, 1536, 1024, 1024, 1e4, 1e-5, F32, Q8_0, Q8_0,
                overrides=(("ffn_down", Q4_K),)),
]


@pytest.fixture(scope="module", params=BATCHED_MODELS, ids=lambda c: c.name)
def pf_model(request, gpu):
    cfg = request.param
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng
    eng.close()


def run_prefill(eng, path, prompt, pos0=0):
    eng.set_prefill_path(path)
    lg = eng.prefill(prompt, pos0)
    return lg, eng.argmax()


def test_prefill_path_selection(pf_model):
    hm, eng = pf_model
    eng.set_prefill_path(PREFILL_AUTO)
    assert eng.prefill_path() == PREFILL_BATCHED
    eng.set_prefill_path(PREFILL_STEPS)
    assert eng.prefill_path() == PREFILL_STEPS
    eng.set_prefill_path(PREFILL_AUTO)


def near_best(lg, tok, tol=3e-2):
    """tok is the argmax of lg, or within the flip tolerance of it (a near tie)"""
    return tok == int(np.argmax(lg)) or lg[tok] >= lg.max() - tol * np.abs(lg).max()


@pytest.mark.parametrize("n", [2, 33, 200])
def test_batched_equals_steps(pf_model, n):
    """Against the token-by-token prefill, beside the distance between the two
    token-by-token paths (fused kernels and one kernel per op) on the same
    prompt: an int8 flip moves a whole later-layer KV row, for every path
    pair alike.  Layer 0's K/V depend on their own token only, so they agree
    to fp16 rounding."""
    hm, eng = pf_model
    cfg = hm.cfg
    prompt = np.random.default_rng(n).integers(1, cfg.vocab, n)
    lg_s, tok_s = run_prefill(eng, PREFILL_STEPS, prompt)
    k_s, v_s = eng.kv_read(0, cfg.n_layers, 0, n)
    eng.set_path(PATH_MULTI)
    lg_m, _ = run_prefill(eng, PREFILL_STEPS, prompt)
    eng.set_path(PATH_AUTO)
    lg_b, tok_b = run_prefill(eng, PREFILL_BATCHED, prompt)
    k_b, v_b = eng.kv_read(0, cfg.n_layers, 0, n)
    e, e_paths = rel(lg_b, lg_s), rel(lg_m, lg_s)
    L, kvd = cfg.n_layers, cfg.kv_dim
    k_s, k_b, v_s, v_b = (a.reshape(L, n, kvd) for a in (k_s, k_b, v_s, v_b))
    eq0 = min(np.mean(k_s[0] == k_b[0]), np.mean(v_s[0] == v_b[0]))

    def maxrel(a, b):
        fa, fb = a.view(np.float16).astype(np.float32), b.view(np.float16).astype(np.float32)
        return float(np.max(np.abs(fa - fb)) / np.max(np.abs(fa)))
    kv_err = max(maxrel(k_s, k_b), maxrel(v_s, v_b))
    print(f"\n{cfg.name} n={n}: logits batched-vs-steps {e:.2e} (multi-vs-fused steps {e_paths:.2e}); "
          f"layer-0 KV equal {eq0:.4f}; KV max rel diff {kv_err:.1e}")
    assert e <= 3e-2
    assert eq0 >= 0.99
    assert kv_err <= 5e-2
    assert near_best(lg_s, tok_b)
    # the next step reads the batched KV state as it reads the sequential one
    a = eng.decode(int(tok_s), n)
    assert np.array_equal(a, eng.decode(int(tok_s), n))


def test_batched_prefill_vs_oracle(pf_model, oracle):
    """The last token's logits of a 24-token prompt against the oracle's
    sequential inference() over the same prompt."""
    hm, eng = pf_model
    cfg = hm.cfg
    prompt = np.random.default_rng(77).integers(1, cfg.vocab, 24)
    st = oracle_state(oracle, hm)
    for t in prompt:
        ref = oracle.inference(st, int(t), cfg.vocab)
    oracle.free_state(st)
    lg_b, tok_b = run_prefill(eng, PREFILL_BATCHED, prompt)
    e = rel(lg_b, ref)
    print(f"\n{cfg.name}: batched prefill vs oracle {e:.2e}")
    assert e <= 3e-2
    assert near_best(ref, tok_b)


def test_batched_prefill_in_several_passes(pf_model):
    """A prompt longer than one pass (512 tokens) continues the KV cache across
    passes; at pos0 > 0 the pass reads the rows before it."""
    hm, eng = pf_model
    cfg = hm.cfg
    n = min(600, cfg.n_context - 8)
    prompt = np.random.default_rng(5).integers(1, cfg.vocab, n)
    lg_s, tok_s = run_prefill(eng, PREFILL_STEPS, prompt)
    lg_b, tok_b = run_prefill(eng, PREFILL_BATCHED, prompt)
    e = rel(lg_b, lg_s)
    # a second prompt appended at pos0 = n on top of each state
    more = np.random.default_rng(6).integers(1, cfg.vocab, 5)
    run_prefill(eng, PREFILL_STEPS, prompt)
    lg_s2, _ = run_prefill(eng, PREFILL_STEPS, more, n)
    run_prefill(eng, PREFILL_BATCHED, prompt)
    lg_b2, _ = run_prefill(eng, PREFILL_BATCHED, more, n)
    e2 = rel(lg_b2, lg_s2)
    print(f"\n{cfg.name}: n={n} rel {e:.2e}; +5 at pos {n} rel {e2:.2e}")
    assert e <= 3e-2 and e2 <= 3e-2
    assert near_best(lg_s, tok_b)


def test_batched_prefill_flips_explained(pf_model, oracle):
    """Every quantized activation of a 24-token batched prefill against the
    oracle's token-by-token run (prefill_flips): no difference that is not a
    rounding flip, and the last token's logits to fp32 noise when no
    difference reached it, within a flip's reach otherwise."""
    hm, eng = pf_model
    cfg = hm.cfg
    prompt = np.random.default_rng(77).integers(1, cfg.vocab, 24)
    st = oracle_state(oracle, hm)
    otr = []
    for t in prompt:
        ref, tr = oracle.inference_traced(st, int(t), cfg)
        otr.append(tr)
    oracle.free_state(st)
    eng.set_prefill_path(PREFILL_BATCHED)
    lg_b, gtr = eng.prefill_traced(prompt)
    compared, differing, bad, clean = prefill_flips(gtr, otr, cfg)
    e = rel(lg_b, ref)
    print(f"\n{cfg.name}: {compared} token activations compared, {differing} with rounding flips, "
          f"{len(bad)} unexplained; last token {'clean' if clean else 'after a flip'}; logits vs oracle {e:.2e}")
    assert not bad, bad[:5]
    quantized = sum(1 for qt, _ in slot_formats(cfg) if qt is not None)
    assert compared >= quantized                            # at least the first token all the way
    assert e <= (EXACT_STEP if clean else 5e-2)
    assert near_best(ref, int(np.argmax(lg_b)))


def test_batched_prefill_unavailable_for_other_shapes(gpu):
    """head_dim 256 has no prefill attention kernel: the prompt runs token by token."""
    cfg = ModelConfig("llama-w1024-hd256", 0, 1, 1024, 4, 4, 256, 2816, 1024, 1024, 1e4, 1e-5, Q4_K, Q8_0, Q4_K)
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    try:
        assert eng.prefill_path() == PREFILL_STEPS
        with pytest.raises(LgError):
            eng.set_prefill_path(PREFILL_BATCHED)
        lg = eng.prefill(np.arange(1, 9), 0)       # AUTO falls back to steps
        assert np.all(np.isfinite(lg))
    finally:
        eng.close()
