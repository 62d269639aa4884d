"""The fused whole-step decode kernels (LG_PATH_FUSED) at widths other than
the Qwen3-8B shape: runtime n_embed / n_ff (the kernels come in width
classes, slots and activation chunks past the model's widths masked) and
head_dim 128, 64 and 48 (48 laid out as 64 with zero lanes).  Every model is
held to the flip-explained one-step bar against the oracle (tests/parity.py)
on the fused and the multi-kernel path, the two paths must agree as on the
4096-wide models, and attention is checked past the short-context split (the
long-context units with their 8-lane position groups) against the oracle's
exact attention over the same fp16 cache.  The tiny parity config T runs
its own tests (tests/test_gpu_decode.py) on the path AUTO picks, which is
this one.  A model mixing V and down types per layer (Q4_K_M-style) runs the
same tests on the fused path's mixed-layer kernels, and F16 and F32 models
on the kernels that hold the fp32 activations in LDS."""
import numpy as np
import pytest

from ligguf_amd.lib import (F16, F32, PATH_FUSED, PATH_MULTI, PATH_PERSISTENT, PREFILL_AUTO, PREFILL_STEPS, Q1_0, Q1_G, Q2_K,
                            Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, LgError)
from ligguf_amd.model import TINY, Engine, HostModel, ModelConfig
from parity import step_flips
from test_gpu_decode import assert_flips_explained, one_step_flips, oracle_state, rel
from test_gpu_persistent import oracle_step_from_cache

pytestmark = pytest.mark.gpu

SHAPES = [
    # Llama-3-8B widths: FFN 14336 (224 Q4_K slots per row: four per lane, the last one masked)
    ModelConfig("llama3-w4096-ff14336-q4k", 0, 2, 4096, 32, 8, 128, 14336, 2048, 2048, 5e5, 1e-5, Q4_K, Q4_K, Q6_K),
    # TinyLlama-1.1B widths: head_dim 64, 8 query heads per KV head, FFN 5632 (2.75 chunks per wave)
    ModelConfig("tinyllama-w2048-hd64-q8", 0, 2, 2048, 32, 4, 64, 5632, 2048, 2048, 1e4, 1e-5, Q8_0, Q8_0, Q8_0),
    # widths that are no multiple of 256: Q8_0 blocks in a partial chunk
    ModelConfig("small-w576-ff1376-hd64-q8", 0, 2, 576, 9, 9, 64, 1376, 1024, 2048, 1e4, 1e-5, Q8_0, Q8_0, Q8_0),
    # the tiny config's shape (head_dim 48) with a context long enough for the long-context units
    TINY.with_(name="tiny-ctx2048", n_context=2048),
    # Q4_K_M / Q4_K_S-style layers: Q6_K attn_v and ffn_down in layer 0, none in layer 1, Q5_K in layer 2
    # (Q|K one matrix, V on its own; the persistent kernel takes uniform layers only)
    ModelConfig("qwen3-w4096-q4k-mixed", 1, 3, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q4_K, Q4_K, Q6_K,
                overrides=(("attn_v.0", Q6_K), ("ffn_down.0", Q6_K), ("attn_v.2", Q5_K), ("ffn_down.2", Q5_K))),
    # Q3_K and Q2_K layers (Q6_K output head)
    ModelConfig("qwen3-w4096-q3k", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q3_K, Q4_K, Q6_K),
    ModelConfig("qwen3-w4096-q2k", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q2_K, Q4_K, Q6_K),
    # Q1_0 layers (32-value sign blocks) with a Q8_0 output head
    ModelConfig("qwen3-w4096-q1_0", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q1_0, Q8_0, Q8_0),
    # Q1_G layers (128-value sign blocks; regrouped for the fused step and the batched prefill)
    ModelConfig("qwen3-w4096-q1g", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q1_G, Q8_0, Q8_0),
    # Q8_0 layers with a Q6_K output head
    ModelConfig("qwen3-w4096-q8_0-q6khead", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q8_0, Q4_K, Q6_K),
    # Qwen3-14B widths: 40 query heads on 8 KV heads (5 per group), FFN 17408
    ModelConfig("qwen3-w5120-ff17408-40x8-q4k", 1, 2, 5120, 40, 8, 128, 17408, 2048, 2048, 1e6, 1e-6, Q4_K, Q4_K,
                Q6_K),
    # Q5_K layers with 8 query heads per KV head
    ModelConfig("qwen3-w4096-q5k-nrep8", 1, 2, 4096, 32, 4, 128, 12288, 2048, 2048, 1e6, 1e-6, Q5_K, Q4_K, Q6_K),
    # F16 / F32 layers, embedding and output head: the fp32 activations stay in LDS, nothing is quantized
    ModelConfig("qwen3-w4096-f16", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, F16, F16, F16),
    ModelConfig("qwen3-w4096-f32", 1, 1, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, F32, F32, F32),
    # Q5_K_M-style: Q5_K layers, Q6_K attn_v and ffn_down in layer 1
    ModelConfig("qwen3-w4096-q5k-mixed", 1, 2, 4096, 32, 8, 128, 12288, 2048, 2048, 1e6, 1e-6, Q5_K, Q4_K, Q6_K,
                overrides=(("attn_v.1", Q6_K), ("ffn_down.1", Q6_K))),
]


@pytest.fixture(scope="module", params=SHAPES, ids=lambda c: c.name)
def shape_model(request, gpu):
    cfg = request.param
    print(f"model {cfg.name}: n_embed {cfg.n_embed} n_ff {cfg.n_ff} head_dim {cfg.head_dim}", flush=True)
    hm = HostModel.synthetic(cfg)
    eng = Engine(0)
    eng.load(hm)
    yield hm, eng
    eng.close()


def test_auto_takes_fused(shape_model):
    hm, eng = shape_model
    cfg = hm.cfg
    eng.set_path(0)
    assert eng.path() == PATH_FUSED
    # the persistent kernel keeps its one width class (4096 / 12288, one type for every layer matrix)
    if cfg.n_embed == 4096 and cfg.n_ff == 12288 and not cfg.overrides:
        try:
            eng.set_path(PATH_PERSISTENT)
        except LgError:
            pass                              # no persistent variant for this type
    else:
        with pytest.raises(LgError):
            eng.set_path(PATH_PERSISTENT)
    eng.set_path(PATH_MULTI)
    assert eng.path() == PATH_MULTI
    eng.set_path(PATH_FUSED)


@pytest.mark.parametrize("path", [PATH_FUSED, PATH_MULTI], ids=["fused", "multi"])
def test_one_step_flips_explained(shape_model, oracle, path):
    hm, eng = shape_model
    eng.set_path(path)
    toks = np.random.default_rng(5).integers(1, hm.cfg.vocab, 12)
    rows = one_step_flips(eng, oracle, hm, toks)
    assert_flips_explained(rows, f"{hm.cfg.name} path {path}")
    assert np.mean([a for *_, a in rows]) >= 0.8


def test_fused_matches_multikernel(shape_model, oracle):
    """Both paths stepped from the same KV state (the oracle's rows) agree to
    fp32 noise on most steps; a free replay on each path's own cache would
    part at the first int8 rounding flip either path takes (both stay within
    flip distance of the oracle, test_one_step_flips_explained)."""
    hm, eng = shape_model
    cfg = hm.cfg
    toks = np.random.default_rng(11).integers(1, cfg.vocab, 12)
    st = oracle_state(oracle, hm)
    errs, am = [], []
    for pos, t in enumerate(toks):
        res = {}
        for p in (PATH_MULTI, PATH_FUSED):
            eng.set_path(p)
            if pos:
                for l in range(cfg.n_layers):
                    k, v = oracle.state_kv(st, l, 0, pos, cfg.kv_dim)
                    eng.kv_write(l, 1, 0, pos, k, v)
            res[p] = (eng.decode(int(t), pos), eng.argmax())
        oracle.inference(st, int(t), cfg.vocab)
        errs.append(rel(res[PATH_FUSED][0], res[PATH_MULTI][0]))
        am.append(res[PATH_FUSED][1] == int(np.argmax(res[PATH_FUSED][0])))
    oracle.free_state(st)
    errs = np.array(errs)
    print(f"\n{cfg.name} fused vs multi on the same KV state: median {np.median(errs):.2e} max {errs.max():.2e}")
    assert np.median(errs) <= 1e-6
    assert errs.max() <= 5e-2
    assert all(am)       # the in-kernel greedy reduction is sampler_greedy on its own logits


def test_prefill_steps_equal_sequential(shape_model):
    hm, eng = shape_model
    eng.set_path(PATH_FUSED)
    eng.set_prefill_path(PREFILL_STEPS)
    prompt = np.random.default_rng(9).integers(1, hm.cfg.vocab, 16)
    pre = eng.prefill(prompt, 0)
    eng.set_prefill_path(PREFILL_AUTO)
    for i, t in enumerate(prompt):
        seq = eng.decode(int(t), i)
    assert np.array_equal(pre.view(np.uint32), seq.view(np.uint32))


@pytest.mark.parametrize("want_pos", [200, 1500], ids=["short-units", "long-units"])
def test_attention_past_the_short_split(shape_model, oracle, want_pos):
    """A step at a late position over a random fp16 cache against the
    oracle's exact attention, every quantized activation compared."""
    hm, eng = shape_model
    cfg = hm.cfg
    pos = min(cfg.n_context - 1, want_pos)
    rng = np.random.default_rng(2)
    ks, vs = [], []
    for l in range(cfg.n_layers):
        k = rng.standard_normal(pos * cfg.kv_dim).astype(np.float16).view(np.uint16)
        v = rng.standard_normal(pos * cfg.kv_dim).astype(np.float16).view(np.uint16)
        eng.kv_write(l, 1, 0, pos, k, v)
        ks.append(k)
        vs.append(v)
    eng.set_path(PATH_MULTI)
    multi = eng.decode(7, pos)
    eng.set_path(PATH_FUSED)
    g, gtr = eng.decode_traced(7, pos)
    o, otr = oracle_step_from_cache(oracle, hm, ks, vs, pos, 7)
    first, bad = step_flips(gtr, otr, cfg)
    e, em = rel(g, o), rel(g, multi)
    print(f"\n{cfg.name}: pos {pos} vs oracle {e:.2e} (first int8 difference at activation {first}), "
          f"vs multi {em:.2e}")
    assert not bad, bad[:5]
    assert e <= (1e-5 if first < 0 else 5e-2)
    assert em <= 5e-2


def test_regrouped_copies_equal_gguf_rows(shape_model, monkeypatch):
    """Where the fused step reads regrouped copies (Q8_0, Q6_K, Q1_G, Q3_K,
    Q1_0 matrices in whole 8-block groups) -- and the batched prefill those
    of uniform Q8_0 / Q1_0 layers --, LG_NO_REGROUP=1 reads the GGUF rows:
    the same logits bit for bit."""
    hm, eng = shape_model
    toks = np.random.default_rng(17).integers(1, hm.cfg.vocab, 3)
    prompt = np.random.default_rng(18).integers(1, hm.cfg.vocab, 40)
    eng.set_path(PATH_FUSED)
    a = [eng.decode(int(t), i) for i, t in enumerate(toks)]
    eng.set_prefill_path(PREFILL_AUTO)
    pa = eng.prefill(prompt, 0)
    monkeypatch.setenv("LG_NO_REGROUP", "1")
    other = Engine(0)
    try:
        other.load(hm)
        other.set_path(PATH_FUSED)
        b = [other.decode(int(t), i) for i, t in enumerate(toks)]
        pb = other.prefill(prompt, 0)
    finally:
        other.close()
    assert all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(a, b))
    assert np.array_equal(pa.view(np.uint32), pb.view(np.uint32))
