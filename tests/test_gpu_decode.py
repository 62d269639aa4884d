"""GPU decode step (lg_decode_step) against the oracle and the reference.

The models here quantize every activation to int8 (Q8_0 / Q8_K) before each
matvec, as the reference does.  Two correct fp32 implementations that sum in
different orders therefore agree to ~1e-7 until some activation lands within
that noise of a rounding boundary of the quantizer; there they differ by one
int8 step in one element (a "flip"), which these random-weight models amplify
to ~1e-3..1e-2 in the logits.  The reference itself is not immune: its
rmsnorm and SwiGLU use the approximate rsqrtss/rcpps instructions, whose bits
differ between CPU vendors, and the oracle (double sums) leaves the
reference's own greedy sequence at token 38 of 128 for exactly this reason.
The tests therefore check
  * one-step parity with every difference explained: GPU and oracle run the
    same token from the SAME KV state (the oracle's, written into the GPU
    cache); each step's quantized activations are compared with the oracle's
    (tests/parity.py): a step without any differing int8 must match the
    oracle's logits to EXACT_STEP, and the first differing activation of a
    step may differ only by rounding flips;
  * teacher-forced greedy on the tiny config: fed the reference's greedy
    sequence from its own KV state, the GPU picks the reference's token at
    every step whose reference top-2 gap exceeds the measured flip noise, and
    its logits stay within that noise of the reference's;
  * free-running greedy: the GPU's sequence equals the reference's up to a
    first divergence, which must fall on such a near-tie and no earlier
    than the oracle's own (token 38); teacher-forced, the GPU keeps the
    reference's token on at least 124 of 128 steps.
"""
import numpy as np
import pytest

from conftest import golden
from ligguf_amd.lib import Q4_K, Q5_K, Q6_K, Q8_0, Q3_K, Q2_K, Q1_G
from ligguf_amd.model import TINY, Engine, HostModel, ModelConfig
from parity import EXACT_STEP, FORCED_STEP, flip_summary, forced_flips, slot_formats, step_flips

# what this build achieves on the tiny run, held so that a regression shows:
# the oracle's own free run (double sums) leaves the reference's greedy
# sequence at token 38, so a correct engine does at least that well; the
# oracle misses the reference's token on 5 of the 128 teacher-forced steps
FREE_RUN_MIN = 38
TEACHER_MIN = 124
# largest logit difference allowed between two correct engines fed the same
# tokens once a flip has entered their KV caches: the oracle (double sums)
# against the reference on the tiny teacher-forced run peaks at 0.0177
# (tests/golden/tiny_teacher.npz oracle_maxdiff); 0.03 keeps a margin
FLIP_NOISE = 0.03

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


def oracle_state(oracle, hm):
    from oracle.binding import OrLayer, OrModel, OrWeight
    return oracle.new_state(hm.fill_desc(OrModel, OrLayer, OrWeight))


def one_step_flips(eng, oracle, hm, toks):
    """Each token on the GPU and in the oracle from the oracle's KV state,
    with both steps' quantized activations: rows (first differing
    activation or -1, unexplained differences, logits rel-L2, argmax agree).
    Each step also runs in the oracle with the GPU's quantized activations
    forced in (or_state_force): every activation of the step is compared
    (forced_flips) and the logits held to FORCED_STEP; what fails there is
    listed among the step's unexplained differences, tagged "forced"."""
    cfg = hm.cfg
    forms = [f for f, _ in slot_formats(cfg)]
    st = oracle_state(oracle, hm)
    rows, nf, worst, worst_rel = [], 0, 0.0, 0.0
    for pos, t in enumerate(toks):
        if pos:
            for l in range(cfg.n_layers):
                k, v = oracle.state_kv(st, l, 0, pos, cfg.kv_dim)
                eng.kv_write(l, 1, 0, pos, k, v)
        g, gtr = eng.decode_traced(int(t), pos)
        o, otr = oracle.inference_traced(st, int(t), cfg)
        first, bad = step_flips(gtr, otr, cfg)
        oracle.L.or_state_set_pos(st, pos)
        fo, ftr = oracle.inference_forced(st, int(t), cfg, gtr, forms)
        compared, differing, fbad, dist = forced_flips(gtr, ftr, cfg)
        frel = rel(g, fo)
        bad = bad + [("forced",) + b for b in fbad]
        if frel > FORCED_STEP:
            bad.append(("forced", "logits", frel))
        nf += compared
        worst, worst_rel = max(worst, dist), max(worst_rel, frel)
        rows.append((first, bad, rel(g, o), int(np.argmax(g)) == int(np.argmax(o))))
    oracle.free_state(st)
    print(f"\nactivations forced: {nf} compared over {len(toks)} steps, largest boundary distance of a "
          f"differing int8 {worst:.1e}, largest logits rel-L2 {worst_rel:.1e}")
    return rows


def assert_flips_explained(rows, name, max_flip_rel=5e-2):
    """No unexplained int8 difference; steps without one exact to fp32 noise;
    steps with a flip within the reach of one flip."""
    print(f"\n{name}: " + flip_summary([(f, len(b), r) for f, b, r, _ in rows]))
    for i, (first, bad, r, _) in enumerate(rows):
        assert not bad, f"step {i}: int8 differences that are not rounding flips: {bad[:5]}"
        if first < 0:
            assert r <= EXACT_STEP, f"step {i}: no int8 difference yet logits rel-L2 {r:.2e}"
        else:
            assert r <= max_flip_rel, f"step {i}: flip at activation {first}, logits rel-L2 {r:.2e}"


def one_step_errors(eng, oracle, hm, toks):
    """Run each token on the GPU and in the oracle from the oracle's KV state."""
    cfg = hm.cfg
    st = oracle_state(oracle, hm)
    errs, agree = [], []
    for pos, t in enumerate(toks):
        if pos:
            for l in range(cfg.n_layers):
                k, v = oracle.state_kv(st, l, 0, pos, cfg.kv_dim)
                eng.kv_write(l, 1, 0, pos, k, v)
        g = eng.decode(int(t), pos)
        o = oracle.inference(st, int(t), cfg.vocab)
        errs.append(rel(g, o))
        agree.append(int(np.argmax(g)) == int(np.argmax(o)))
    oracle.free_state(st)
    return np.array(errs), np.array(agree)


@pytest.fixture(scope="module")
def tiny(gpu):
    g = golden("tiny_decode.npz")
    hm = HostModel.synthetic(TINY)
    hm.rope_freq = g["rope_freq"]     # the reference's own table (fast/common.cpp:38-39)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng, g
    eng.close()


def test_tiny_first_step_matches_reference(tiny):
    hm, eng, g = tiny
    lg = eng.decode(int(g["prompt"][0]), 0)
    assert rel(lg, g["logits_step0"]) < 2e-2
    assert int(np.argmax(lg)) == int(np.argmax(g["logits_step0"]))


def test_tiny_one_step_vs_live_reference(tiny, reference, tmp_path):
    """GPU and the reference engine (built from its own sources, running on
    this host's CPU) each run a token of the reference's greedy trajectory
    from the reference's KV state.  The reference's internal activations are
    not observable, so flips are explained against the oracle
    (test_tiny_one_step_flips_explained); here most steps must agree to fp32
    noise and none by more than one flip."""
    hm, eng, g = tiny
    path = str(tmp_path / "tiny.gguf")
    hm.write_gguf(path)
    reference.model_open(path, 0)
    toks = np.concatenate([g["prompt"], g["greedy"][:48]])
    errs, agree = [], []
    for pos, t in enumerate(toks):
        if pos:
            for l in range(TINY.n_layers):
                k, v = reference.kv_rows(l, 0, pos, TINY.kv_dim)
                eng.kv_write(l, 1, 0, pos, k, v)
        a = eng.decode(int(t), pos)
        b = reference.inference(int(t), TINY.vocab)
        errs.append(rel(a, b))
        agree.append(int(np.argmax(a)) == int(np.argmax(b)))
    errs = np.array(errs)
    print(f"\nGPU vs live reference one-step: median {np.median(errs):.2e} p90 {np.quantile(errs, 0.9):.2e}"
          f" max {errs.max():.2e}; steps within 1e-5: {np.mean(errs <= 1e-5):.3f} argmax agree {np.mean(agree):.3f}")
    assert np.median(errs) <= 1e-5
    assert np.mean(errs <= 1e-5) >= 0.8
    assert errs.max() <= 3e-2
    assert np.mean(agree) >= 0.95


def test_tiny_one_step_flips_explained(tiny, oracle):
    hm, eng, g = tiny
    toks = np.concatenate([g["prompt"], g["greedy"][:80]])
    rows = one_step_flips(eng, oracle, hm, toks)
    assert_flips_explained(rows, "tiny, GPU vs oracle one-step")
    assert np.mean([a for *_, a in rows]) >= 0.95


def test_tiny_teacher_forced_greedy(tiny):
    """The reference's 128-token greedy sequence fed to the GPU (own KV
    state): the GPU's greedy token equals the reference's at every step whose
    top-2 gap exceeds FLIP_NOISE and on at least TEACHER_MIN of the 128, and
    its logits stay within FLIP_NOISE of the reference's 32 largest
    (tests/golden/tiny_teacher.npz)."""
    hm, eng, g = tiny
    tt = golden("tiny_teacher.npz")
    toks = np.concatenate([g["prompt"], g["greedy"]])
    n0 = len(g["prompt"]) - 1
    miss, worst = [], 0.0
    for pos in range(len(toks) - 1):
        lg = eng.decode(int(toks[pos]), pos)
        if pos < n0:
            continue
        j = pos - n0
        d = float(np.max(np.abs(lg[tt["top_ids"][j]] - tt["top_vals"][j])))
        worst = max(worst, d)
        assert d <= FLIP_NOISE, f"step {j}: logits {d:.3e} from the reference's"
        if int(np.argmax(lg)) != int(g["greedy"][j]):
            miss.append((j, float(tt["gap"][j])))
    print(f"\nteacher-forced: GPU greedy equals the reference's on {128 - len(miss)} of 128 steps; "
          f"largest logit difference {worst:.2e}; near-tie steps that differ {miss} "
          f"(the oracle differs on {int(np.sum(tt['oracle_tok'] != tt['top_ids'][:, 0]))})")
    for j, gap in miss:
        assert gap < FLIP_NOISE, f"step {j}: the GPU left the reference's token at a top-2 gap of {gap:.3e}"
    assert 128 - len(miss) >= TEACHER_MIN


def test_tiny_greedy_free_running(tiny):
    """Free-running greedy decode of the 16-token prompt + 128 tokens: equal
    to the reference's sequence up to the first divergence, which comes no
    earlier than FREE_RUN_MIN and falls on a step whose reference top-2 gap
    is below FLIP_NOISE (until then both engines saw the same tokens)."""
    hm, eng, g = tiny
    tt = golden("tiny_teacher.npz")
    toks = []
    logits = None
    for pos, t in enumerate(g["prompt"]):
        logits = eng.decode(int(t), pos)
    pos = len(g["prompt"])
    for j in range(128):
        nxt = int(np.argmax(logits))
        toks.append(nxt)
        if j == 127:
            break
        logits = eng.decode(nxt, pos)
        pos += 1
    ref = g["greedy"].tolist()
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, ref)) if a != b), len(ref))
    same = sum(a == b for a, b in zip(toks, ref))
    print(f"\nGPU greedy equals the reference's first {first_diff} of 128 tokens ({same} equal overall); "
          f"the oracle's free run leaves it at token 38")
    assert toks[0] == ref[0]
    assert first_diff >= FREE_RUN_MIN
    if first_diff < len(ref):
        assert float(tt["gap"][first_diff]) < FLIP_NOISE, \
            f"diverged at {first_diff} where the reference's top-2 gap is {float(tt['gap'][first_diff]):.3e}"


def test_tiny_decode_deterministic_and_async(tiny):
    hm, eng, g = tiny
    a = [eng.decode(int(t), p) for p, t in enumerate(g["prompt"][:6])]
    b = [eng.decode(int(t), p) for p, t in enumerate(g["prompt"][:6])]
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    for p, t in enumerate(g["prompt"][:6]):
        eng.decode_async(int(t), p)
    eng.sync()
    assert eng.argmax() == int(np.argmax(a[-1]))


def test_prefill_equals_sequential(tiny):
    """Token by token the prefill is the step loop bit for bit; AUTO takes the
    batched prefill on this config (test_gpu_prefill.py holds it to the
    oracle activation by activation)."""
    from ligguf_amd.lib import PREFILL_AUTO, PREFILL_BATCHED, PREFILL_STEPS
    hm, eng, g = tiny
    seq = [eng.decode(int(t), p) for p, t in enumerate(g["prompt"])][-1]
    k1, v1 = eng.kv_read(0, TINY.n_layers, 0, 16)
    eng.set_prefill_path(PREFILL_STEPS)
    pre = eng.prefill(g["prompt"], 0)
    k2, v2 = eng.kv_read(0, TINY.n_layers, 0, 16)
    eng.set_prefill_path(PREFILL_AUTO)
    assert np.array_equal(pre, seq)
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    assert eng.prefill_path() == PREFILL_BATCHED
    bat = eng.prefill(g["prompt"], 0)
    assert int(np.argmax(bat)) == int(np.argmax(seq))


def test_kv_roundtrip_and_errors(tiny):
    hm, eng, g = tiny
    from ligguf_amd.lib import LgError
    rng = np.random.default_rng(1)
    k = rng.integers(0, 65535, 3 * 5 * TINY.kv_dim, dtype=np.uint16)
    v = rng.integers(0, 65535, 3 * 5 * TINY.kv_dim, dtype=np.uint16)
    eng.kv_write(2, 3, 40, 5, k, v)
    k2, v2 = eng.kv_read(2, 3, 40, 5)
    assert np.array_equal(k, k2) and np.array_equal(v, v2)
    with pytest.raises(LgError):
        eng.decode(1, TINY.n_context)        # position beyond the context
    with pytest.raises(LgError):
        eng.decode(TINY.vocab, 0)            # token beyond the vocabulary
    with pytest.raises(LgError):
        eng.kv_read(0, TINY.n_layers + 1, 0, 1)


QWEN_SMALL = [
    ModelConfig("qwen3-small-q4k", 1, 3, 512, 8, 2, 64, 1024, 2048, 128, 1e6, 1e-6, Q4_K, Q4_K, Q6_K),
    ModelConfig("qwen3-small-mixed", 1, 2, 512, 4, 4, 128, 768, 1024, 128, 1e6, 1e-6, Q5_K, Q3_K, Q2_K),
    ModelConfig("llama-small-q1g", 0, 2, 512, 8, 4, 64, 1024, 1024, 128, 1e4, 1e-5, Q1_G, Q8_0, Q8_0,
                q1_direct=True),
]


@pytest.mark.parametrize("cfg", QWEN_SMALL, ids=lambda c: c.name)
def test_small_models_one_step(gpu, oracle, cfg):
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    toks = np.random.default_rng(3).integers(1, cfg.vocab, 24)
    rows = one_step_flips(eng, oracle, hm, toks)
    assert_flips_explained(rows, cfg.name)
    assert np.mean([a for *_, a in rows]) >= 0.9
    eng.close()
