"""The flip-explained parity helper (tests/parity.py) against the oracle's own
quantizers: its float32 restatement of quantize_q8_K / quantize_q8_0 must give
the oracle's int8 values bit for bit (the oracle itself is pinned to the
reference's golden vectors in test_oracle.py), and a planted off-boundary
difference must be reported."""
import numpy as np
import pytest

from conftest import golden
from ligguf_amd.lib import Q8_0, Q8_K
from ligguf_amd.model import TINY
from parity import boundary_dist, forced_flips, parse_q, prefill_flips, quantize_ref, slot_formats, step_flips


def _vectors():
    rng = np.random.default_rng(42)
    vs = [golden("quant.npz")["x"]] if "x" in golden("quant.npz").files else []
    for s in (1e-3, 0.02, 1.0, 30.0):
        vs.append((rng.standard_normal(4096) * s).astype(np.float32))
    b = np.linspace(-127.5, 127.5, 512).astype(np.float32)      # values on .5 boundaries
    vs.append(b)
    return vs


def test_quantize_ref_matches_oracle(oracle):
    for x in _vectors():
        n = x.size // 256 * 256
        x = x[:n]
        qk = oracle.quantize_q8_K(x)
        q, _ = quantize_ref(x, Q8_K)
        qo, _ = parse_q(qk, Q8_K, n)
        assert np.array_equal(q, qo)
        q0 = oracle.quantize_q8_0(x)
        q, _ = quantize_ref(x, Q8_0)
        qo, _ = parse_q(q0, Q8_0, n)
        assert np.array_equal(q, qo)


def test_step_flips_reports_planted_differences(oracle):
    cfg = TINY.with_(n_layers=1)
    rng = np.random.default_rng(3)
    wide = max(cfg.n_embed, cfg.n_ff)
    ot = (rng.standard_normal((4 * cfg.n_layers + 1, wide)) * 0.5).astype(np.float32)
    stride = 1024
    gt = np.zeros((4 * cfg.n_layers + 1, stride), np.uint8)
    for k, (qt, n) in enumerate(slot_formats(cfg)):
        b = oracle.quantize_q8_0(ot[k][:n])
        gt[k][:b.size] = b
    assert step_flips(gt, ot, cfg) == (-1, [])
    # a one-step change at a value far from a rounding boundary is not a flip
    _, v = quantize_ref(ot[2][:cfg.n_embed], Q8_0)
    i = int(np.argmax(boundary_dist(v)))
    blk, j = divmod(i, 32)
    gt[2][blk * 34 + 2 + j] = np.uint8((int(gt[2][blk * 34 + 2 + j].view(np.int8)) + 1) & 255)
    first, bad = step_flips(gt, ot, cfg)
    assert first == 2 and len(bad) == 1 and bad[0][1] == i


def _prefill_traces(oracle, cfg, n, seed):
    rng = np.random.default_rng(seed)
    wide = max(cfg.n_embed, cfg.n_ff)
    nk = 4 * cfg.n_layers + 1
    ots = [(rng.standard_normal((nk, wide)) * 0.5).astype(np.float32) for _ in range(n)]
    gt = np.zeros((n, nk, 1024), np.uint8)
    for t in range(n):
        for k, (qt, w) in enumerate(slot_formats(cfg)):
            b = oracle.quantize_q8_0(ots[t][k][:w])
            gt[t, k, :b.size] = b
    return gt, ots


def _bump(gt, t, k, i):
    blk, j = divmod(i, 32)
    gt[t, k, blk * 34 + 2 + j] = np.uint8((int(gt[t, k, blk * 34 + 2 + j].view(np.int8)) + 1) & 255)


def test_prefill_flips_walk(oracle):
    """The causal walk of prefill_flips: a difference at (token t, activation
    k) stops the comparisons of tokens >= t past k, not those of earlier
    tokens; an off-boundary one is reported, a near-boundary one is a flip."""
    cfg = TINY.with_(n_layers=2)
    n, nk = 4, 9
    gt, ots = _prefill_traces(oracle, cfg, n, 8)
    full = n * (nk - 1) + 1
    assert prefill_flips(gt, ots, cfg) == (full, 0, [], True)
    # an off-boundary one-step change at token 2, activation 1
    _, v = quantize_ref(ots[2][1][:cfg.n_embed], Q8_0)
    far = int(np.argmax(boundary_dist(v)))
    g2 = gt.copy()
    _bump(g2, 2, 1, far)
    compared, differing, bad, clean = prefill_flips(g2, ots, cfg)
    assert differing == 1 and len(bad) == 1 and bad[0][:3] == (2, 1, far) and not clean
    # tokens 2, 3 stop after activation 1; tokens 0, 1 run to the end
    assert compared == full - 2 * (nk - 3) - 1
    # a value planted on a rounding boundary differing by one step is a flip
    g3 = gt.copy()
    x = ots[0][3][:cfg.n_embed].copy()
    amax = np.abs(x[:32]).max()
    x[5] = np.float32((10.5 / 127.0) * amax)             # v = 10.5 exactly: roundf gives 11
    ots3 = [o.copy() for o in ots]
    ots3[0][3][:cfg.n_embed] = x
    b = oracle.quantize_q8_0(x)
    g3[0, 3, :b.size] = b
    g3[0, 3, 2 + 5] = np.uint8(10)                       # the other side of the boundary
    compared, differing, bad, clean = prefill_flips(g3, ots3, cfg)
    assert differing == 1 and bad == [] and not clean
    assert compared == full - n * (nk - 5) - 1


def test_ties_do_not_count_against_the_cap(oracle):
    """Values on exact halves (as a Q6_K embedding makes them) may all round
    either way; flips at larger boundary distances stay capped."""
    cfg = TINY.with_(n_layers=1)
    n = cfg.n_embed
    rng = np.random.default_rng(4)
    x = np.clip(rng.standard_normal(n) * 0.3, -0.9, 0.9).astype(np.float32)
    x[0::32] = 1.0                                           # each block's maximum
    ties = [b * 32 + j for b in range(n // 32) for j in (3, 7, 11)]
    x[ties] = np.float32(63.5 / 127.0)                        # v = 63.5: a tie, roundf gives 64
    ot = np.zeros((4 * cfg.n_layers + 1, max(n, cfg.n_ff)), np.float32)
    ot[0][:n] = x
    gt = np.zeros((4 * cfg.n_layers + 1, 1024), np.uint8)
    for k, (qt, w) in enumerate(slot_formats(cfg)):
        b = oracle.quantize_q8_0(ot[k][:w])
        gt[k][:b.size] = b
    _, v = quantize_ref(x, Q8_0)
    assert np.all(boundary_dist(v[ties]) < 1e-4) and len(ties) > 20
    g = gt.copy()
    for i in ties:
        blk, j = divmod(i, 32)
        g[0][blk * 34 + 2 + j] = np.uint8(63)
    assert step_flips(g, ot, cfg) == (0, [])
    # the same number of one-step changes at distance ~0.01 exceed the cap
    x2 = x.copy()
    x2[ties] = np.float32(63.49 / 127.0)
    ot2 = ot.copy()
    ot2[0][:n] = x2
    g2 = gt.copy()
    b = oracle.quantize_q8_0(x2)
    g2[0][:b.size] = b
    for i in ties:
        blk, j = divmod(i, 32)
        g2[0][blk * 34 + 2 + j] = np.uint8(64)
    first, bad = step_flips(g2, ot2, cfg)
    assert first == 0 and bad and bad[0][1] == -1


def test_scale_flips(oracle):
    """A Q8_0 block scale one fp16 ulp off is a flip when amax / 127 lies on an
    fp16 rounding tie, and unexplained off a tie or more than one ulp off."""
    cfg = TINY.with_(n_layers=1)
    n = cfg.n_embed
    rng = np.random.default_rng(5)
    ulp = 2.0 ** -16                       # fp16 spacing in [2^-6, 2^-5)
    x = (rng.standard_normal(n) * 0.2).astype(np.float32)
    x = np.clip(x, -1.0, 1.0)

    def run(m, planted):
        xs = x.copy()
        xs[64] = np.float32(127 * m * ulp)            # block 2's maximum: amax / 127 = m fp16 ulps exactly
        assert np.float32(xs[64]) / np.float32(127) == np.float32(m * ulp)
        ot = np.zeros((4 * cfg.n_layers + 1, max(n, cfg.n_ff)), np.float32)
        ot[0][:n] = xs
        gt = np.zeros((4 * cfg.n_layers + 1, 1024), np.uint8)
        for k, (qt, w) in enumerate(slot_formats(cfg)):
            b = oracle.quantize_q8_0(ot[k][:w])
            gt[k][:b.size] = b
        assert step_flips(gt, ot, cfg) == (-1, [])
        gt[0][2 * 34:2 * 34 + 2] = np.frombuffer(np.float16(planted * ulp).tobytes(), np.uint8)
        return step_flips(gt, ot, cfg)

    # 1171.5 ulps: a tie, fp16 rounds to the even 1172; 1171 is the other side
    assert run(1171.5, 1171) == (0, [])
    # 1171.25 ulps rounds to 1171 with no tie near: 1172 is no flip
    first, bad = run(1171.25, 1172)
    assert first == 0 and bad and bad[0][1] == -2 and bad[0][2] == 2
    # two ulps off a tie is no flip either
    first, bad = run(1171.5, 1170)
    assert first == 0 and bad and bad[0][5] == 1.0


# ---------------- forced activations (or_state_force) ----------------
def _k_model():
    """Small K-quant model with a Q8_0 consumer beside Q4_K ones in the
    attention input (that activation is recorded in the Q8_K form; the
    Q8_0 matvec quantizes its own)."""
    from ligguf_amd.lib import ARCH_QWEN3, Q4_K, Q6_K
    from ligguf_amd.model import ModelConfig
    return ModelConfig("k-mix", ARCH_QWEN3, 3, 256, 4, 2, 64, 512, 700, 32, 1e6, 1e-6, Q4_K, Q4_K, Q6_K,
                       overrides=(("attn_v", Q8_0), ("ffn_down", Q6_K)))


def _quantized(oracle, cfg, tr):
    """[4L+1][stride] blocks: each traced float vector through the oracle's
    own quantizer in its recorded form."""
    fm = slot_formats(cfg)
    stride = max(n // 256 * 292 for _, n in fm)
    acts = np.zeros((len(fm), stride), np.uint8)
    for k, (qt, n) in enumerate(fm):
        if qt is not None:
            b = (oracle.quantize_q8_K if qt == Q8_K else oracle.quantize_q8_0)(tr[k][:n])
            acts[k, :b.size] = b
    return acts


def _forced_state(oracle, cfg, npos):
    """An oracle state after npos unforced steps (with the host model whose
    arrays it points into), the next token, its logits and trace."""
    from oracle.binding import OrLayer, OrModel, OrWeight
    from ligguf_amd.model import HostModel
    hm = HostModel.synthetic(cfg)
    st = oracle.new_state(hm.fill_desc(OrModel, OrLayer, OrWeight))
    toks = np.random.default_rng(5).integers(1, cfg.vocab, npos + 1)
    for t in toks[:npos]:
        oracle.inference(st, int(t), cfg.vocab)
    lg, tr = oracle.inference_traced(st, int(toks[npos]), cfg)
    return (hm, st), int(toks[npos]), lg, tr


def _forced(oracle, st, cfg, pos, tok, acts):
    oracle.L.or_state_set_pos(st, pos)
    return oracle.inference_forced(st, tok, cfg, acts, [f for f, _ in slot_formats(cfg)])


def _bump_q(acts, k, qt, i):
    """one int8 of activation k one step up (or down at 127)"""
    qk, bs = (256, 292) if qt == Q8_K else (32, 34)
    blk, j = divmod(i, qk)
    off = blk * bs + (4 if qt == Q8_K else 2) + j
    q = int(acts[k, off].view(np.int8))
    acts[k, off] = np.uint8((q + (1 if q < 127 else -1)) & 255)


def _consistent(oracle, st, cfg, pos, tok, acts, k):
    """acts with every activation after k re-quantized from a forced step
    over acts (repeated until stable): what a GPU step whose activation k
    went wrong would record after it."""
    for _ in range(len(slot_formats(cfg))):
        _, tr = _forced(oracle, st, cfg, pos, tok, acts)
        nxt = _quantized(oracle, cfg, tr)
        new = acts.copy()
        new[k + 1:] = nxt[k + 1:]
        if np.array_equal(new, acts):
            return acts
        acts = new
    raise AssertionError("forced re-quantization did not settle")


@pytest.mark.parametrize("which", ["tiny", "kmix"])
def test_forced_step_reproduces_own_activations(oracle, which):
    """Forcing a step's own quantized activations back into it changes
    nothing: logits and every traced vector bit for bit, every activation
    compared and equal.  A wrong slot offset, form or block layout in the
    forced path would break this."""
    cfg = TINY.with_(n_context=16) if which == "tiny" else _k_model()
    (hm, st), tok, lg, tr = _forced_state(oracle, cfg, 5)
    acts = _quantized(oracle, cfg, tr)
    lg2, tr2 = _forced(oracle, st, cfg, 5, tok, acts)
    assert np.array_equal(lg.view(np.uint32), lg2.view(np.uint32))
    assert np.array_equal(tr.view(np.uint32), tr2.view(np.uint32))
    nq = sum(1 for f, _ in slot_formats(cfg) if f is not None)
    assert nq == 4 * cfg.n_layers + 1
    assert forced_flips(acts, tr2, cfg) == (nq, 0, [], 0.0)
    # the Q8_K bsums are recomputed from the quants, not read
    if which == "kmix":
        a2 = acts.copy()
        a2[0, 260:292] = 0x55
        lg3, _ = _forced(oracle, st, cfg, 5, tok, a2)
        assert np.array_equal(lg.view(np.uint32), lg3.view(np.uint32))
    oracle.free_state(st)


@pytest.mark.parametrize("which", ["tiny", "kmix"])
def test_forced_flips_localise_planted_differences(oracle, which):
    """A one-step int8 change far from a rounding boundary at one activation
    -- the attention output of layer 0, the SwiGLU output of the last layer,
    the output head's input -- is reported at that activation and nowhere
    else once the activations after it follow from it; the changed value is
    read (the next activation, or the logits, move)."""
    cfg = TINY.with_(n_context=16) if which == "tiny" else _k_model()
    (hm, st), tok, lg, tr = _forced_state(oracle, cfg, 5)
    base = _quantized(oracle, cfg, tr)
    fm = slot_formats(cfg)
    nq = len(fm)
    for k in (1, 4 * cfg.n_layers - 1, 4 * cfg.n_layers):
        qt, n = fm[k]
        _, v = quantize_ref(tr[k][:n], qt)
        far = int(np.argmax(boundary_dist(v)))
        acts = base.copy()
        _bump_q(acts, k, qt, far)
        acts = _consistent(oracle, st, cfg, 5, tok, acts, k)
        lg2, tr2 = _forced(oracle, st, cfg, 5, tok, acts)
        if k < nq - 1:
            assert not np.array_equal(tr[k + 1], tr2[k + 1])     # the next activation reads it
        else:
            assert not np.array_equal(lg, lg2)                   # the logits read the head's input
        compared, differing, bad, _ = forced_flips(acts, tr2, cfg)
        assert compared == nq and differing == 1
        assert len(bad) == 1 and bad[0][:2] == (k, far), bad
    oracle.free_state(st)
