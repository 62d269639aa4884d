"""Pin the CPU oracle (oracle/lg_oracle.c) before trusting it as the checker.

Each function is checked against the golden vectors the reference engine
wrote (tests/golden/make_golden.py), against what the mathematics fixes
(IEEE conversion, invariants of the quantizers, dot == sum of dequantized
products, brute-force attention), and, where the reference build is present,
against the live reference on fresh random inputs.
"""
import numpy as np
import pytest

from conftest import golden, sampler_agree
from ligguf_amd.lib import BLOCK, F16, F32, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0

WEIGHT_TYPES = [Q8_0, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]


# ---------------- A1 fp16 ----------------
def test_fp16_to_fp32_all_halves(oracle):
    g = golden("fp16.npz")
    h = np.arange(65536, dtype=np.uint16)
    a = oracle.fp16_to_fp32(h)
    assert np.array_equal(a.view(np.uint32), g["h2f"].view(np.uint32))
    # and IEEE (numpy) for every non-NaN half
    fin = ~np.isnan(h.view(np.float16))
    assert np.array_equal(a[fin], h.view(np.float16)[fin].astype(np.float32))


def test_fp32_to_fp16_golden_and_ieee(oracle):
    g = golden("fp16.npz")
    assert np.array_equal(oracle.fp32_to_fp16(g["f32_in"]), g["f2h"])
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    f = u.view(np.float32)
    ok = np.isfinite(f) & (np.abs(f) < 65504)
    assert np.array_equal(oracle.fp32_to_fp16(f[ok]), f[ok].astype(np.float16).view(np.uint16))


# ---------------- A3 dequant ----------------
@pytest.mark.parametrize("t", WEIGHT_TYPES)
def test_dequant_golden(oracle, t):
    g = golden("dequant.npz")
    data = g[f"in_{t}"]
    ref = g[f"out_{t}"]
    out = oracle.dequantize_row(t, data, ref.size)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def test_dequant_closed_forms(oracle):
    # Q8_0: value = qs * d ; Q1_0: +-d by bit
    rng = np.random.default_rng(2)
    blk = np.zeros((4, 34), np.uint8)
    d = np.array([0.5, -0.25, 2.0 ** -20, 3.0], np.float16)
    blk[:, :2] = d.view(np.uint8).reshape(4, 2)
    qs = rng.integers(-127, 128, (4, 32)).astype(np.int8)
    blk[:, 2:] = qs.view(np.uint8)
    out = oracle.dequantize_row(Q8_0, blk.reshape(-1), 128).reshape(4, 32)
    assert np.array_equal(out, qs.astype(np.float32) * d.astype(np.float32)[:, None])
    b1 = np.zeros(6, np.uint8)
    b1[:2] = np.array([0.125], np.float16).view(np.uint8)
    b1[2:] = [0b10100101, 0xFF, 0, 0x0F]
    out = oracle.dequantize_row(Q1_0, b1, 32)
    bits = np.unpackbits(b1[2:], bitorder="little")
    assert np.array_equal(out, np.where(bits == 1, 0.125, -0.125).astype(np.float32))


# ---------------- A2 quantizers ----------------
def test_quantizers_golden(oracle):
    g = golden("quant.npz")
    assert np.array_equal(oracle.quantize_q8_0(g["x"]), g["q8_0"])
    assert np.array_equal(oracle.quantize_q8_K(g["x"]), g["q8_K"])


def test_q8k_invariants(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256 * 64) * rng.uniform(1e-3, 10, 64).repeat(256)).astype(np.float32)
    q = oracle.quantize_q8_K(x).reshape(64, 292)
    d = q[:, :4].copy().view(np.float32)[:, 0]
    qs = q[:, 4:260].view(np.int8).astype(np.int32)
    bs = q[:, 260:292].copy().view(np.int16)
    xb = x.reshape(64, 256)
    # bsums are the 16-value sums of qs
    assert np.array_equal(bs, qs.reshape(64, 16, 16).sum(-1))
    # the first largest-magnitude value maps to -127 and d*q reconstructs within d/2
    i = np.argmax(np.abs(xb), axis=1)
    assert np.all(qs[np.arange(64), i] == -127)
    assert np.all(np.abs(d[:, None] * qs - xb) <= np.abs(d)[:, None] * 0.5 + 1e-6 * np.abs(xb))


# ---------------- A4/A5 matvec ----------------
@pytest.mark.parametrize("t", WEIGHT_TYPES + [F16, F32])
def test_matmul_golden(oracle, t):
    g = golden("matmul.npz")
    qk, bs = BLOCK[t]
    n, d = 1024, 48
    w, ref = g[f"w_{t}"], g[f"y_{t}"]
    y = oracle.matvec(t, w, n // qk * bs, n, d, g["x"])
    if t in (F16, F32):
        xq = g["x"]
    elif t in (Q8_0, Q1_0, Q1_G):
        xq = oracle.quantize_q8_0(g["x"])
    else:
        xq = oracle.quantize_q8_K(g["x"])
    _, ab = oracle.matvec_q(t, w, n // qk * bs, n, d, xq, want_abs=True)
    # the reference sums in fp32: within a few ulps of sum |terms|
    assert np.all(np.abs(y - ref) <= 1e-6 * ab + 1e-30)


@pytest.mark.parametrize("t", WEIGHT_TYPES)
def test_matvec_equals_dequantized_dot(oracle, t):
    """sum over the row of dequant(w) * dequant(activation) in float64 equals the
    oracle's integer decomposition (two independent paths through the data)."""
    g = golden("dequant.npz")
    qk, bs = BLOCK[t]
    data = g[f"in_{t}"]
    n = 1024 if qk <= 256 else qk
    rows = data.size // (n // qk * bs)
    rsz = n // qk * bs
    rng = np.random.default_rng(4)
    x = rng.standard_normal(n).astype(np.float32)
    if t in (Q8_0, Q1_0, Q1_G):
        xq = oracle.quantize_q8_0(x)
        xd = oracle.dequantize_row(Q8_0, xq, n).astype(np.float64)
    else:
        xq = oracle.quantize_q8_K(x).reshape(-1, 292)
        dd = xq[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
        xd = (xq[:, 4:260].view(np.int8).astype(np.float64) * dd[:, None]).reshape(-1)
        xq = xq.reshape(-1)
    y, ab = oracle.matvec_q(t, data[:rows * rsz], rsz, n, rows, xq, want_abs=True)
    W = np.stack([oracle.dequantize_row(t, data[r * rsz:(r + 1) * rsz], n) for r in range(rows)]).astype(np.float64)
    exact = W @ xd
    assert np.all(np.abs(y - exact) <= 1e-6 * ab + 1e-30)


# ---------------- A6/A7/A9/A10 ----------------
def test_rmsnorm_golden(oracle):
    g = golden("ops.npz")
    y = oracle.rmsnorm(g["rms_x"], g["rms_w"], 1e-6)
    assert np.max(np.abs(y - g["rms_out"]) / (np.abs(g["rms_out"]) + 1e-6)) < 1e-5
    y = oracle.rmsnorm(g["rmsi_x"], g["rmsi_w"], 1e-6)
    assert np.max(np.abs(y - g["rmsi_out"]) / (np.abs(g["rmsi_out"]) + 1e-6)) < 1e-5


@pytest.mark.parametrize("pos", [0, 1, 517, 32767])
def test_rope_golden(oracle, pos):
    g = golden("ops.npz")
    y = oracle.rope(g["rope_x"], 32, 128, 128, pos, g["freq_q"])
    ref = g[f"rope_out_{pos}"]
    assert np.max(np.abs(y - ref)) < 2e-6 * np.max(np.abs(ref))
    if pos == 0:
        assert np.array_equal(y, g["rope_x"])
    # rotation keeps every pair's norm
    p = y.reshape(-1, 2)
    p0 = g["rope_x"].reshape(-1, 2)
    assert np.allclose(np.hypot(p[:, 0], p[:, 1]), np.hypot(p0[:, 0], p0[:, 1]), rtol=1e-5)


def test_attention_golden_and_bruteforce(oracle):
    g = golden("ops.npz")
    nh, nkv, hd, pos = 8, 2, 128, int(g["att_pos"])
    out = oracle.attention(g["att_q"], g["att_k"], g["att_v"], g["att_kc"], g["att_vc"], nh, nkv, hd, pos)
    ref = g["att_out"]
    assert np.max(np.abs(out - ref)) < 1e-5 * np.max(np.abs(ref))
    # brute force softmax(q K^T / sqrt(hd)) V in float64
    K = g["att_kc"].view(np.float16).astype(np.float64).reshape(pos + 1, nkv, hd)
    V = g["att_vc"].view(np.float16).astype(np.float64).reshape(pos + 1, nkv, hd)
    K[pos] = g["att_k"].reshape(nkv, hd)
    V[pos] = g["att_v"].reshape(nkv, hd)
    q = g["att_q"].astype(np.float64).reshape(nh, hd)
    bf = np.empty((nh, hd))
    for h in range(nh):
        s = K[:, h // (nh // nkv)] @ q[h] * np.float32(1 / np.sqrt(np.float32(hd)))
        p = np.exp(s - s.max())
        bf[h] = (p / p.sum()) @ V[:, h // (nh // nkv)]
    assert np.max(np.abs(out - bf.reshape(-1))) < 1e-6 * np.max(np.abs(bf))


def test_attention_pos0_returns_v(oracle):
    rng = np.random.default_rng(5)
    q = rng.standard_normal(4 * 64).astype(np.float32)
    k = rng.standard_normal(2 * 64).astype(np.float32)
    v = rng.standard_normal(2 * 64).astype(np.float32)
    out = oracle.attention(q, k, v, np.zeros(0, np.uint16), np.zeros(0, np.uint16), 4, 2, 64, 0)
    assert np.array_equal(out.reshape(4, 64), np.repeat(v.reshape(2, 64), 2, axis=0))


def test_swiglu_special_values(oracle):
    g = np.array([0.0, 1.0, -1.0, 20.0, -20.0], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0], np.float32)
    y = oracle.swiglu(u, g)
    expect = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(y, expect, rtol=1e-7, atol=0)
    assert y[0] == 0.0


# ---------------- A12 whole step against the reference's tiny run ----------------
def _tiny_model(g):
    from ligguf_amd.model import TINY, HostModel
    hm = HostModel.synthetic(TINY)
    wsum = np.array([int(np.sum(hm.weights[nm][3], dtype=np.uint64) % (1 << 61)) for nm in sorted(hm.weights)],
                    np.uint64)
    assert np.array_equal(wsum, g["weight_sums"]), "synthetic weights changed: regenerate the golden vectors"
    hm.rope_freq = g["rope_freq"]
    return hm


def test_tiny_step0_golden(oracle):
    """Step 0 of the reference's tiny Q8_0 run.  A step can hold one
    activation-quantization flip (roundf(x*127/amax) landing on the other
    side of .5 under fp32 noise), worth up to ~1e-2 here, so this golden-only
    check is loose; the one-step test against the live reference is tight."""
    from oracle.binding import OrLayer, OrModel, OrWeight
    from ligguf_amd.model import TINY
    g = golden("tiny_decode.npz")
    hm = _tiny_model(g)
    st = oracle.new_state(hm.fill_desc(OrModel, OrLayer, OrWeight))
    lg = oracle.inference(st, int(g["prompt"][0]), TINY.vocab)
    ref = g["logits_step0"]
    assert np.linalg.norm(lg - ref) / np.linalg.norm(ref) < 2e-2
    assert int(np.argmax(lg)) == int(np.argmax(ref))
    oracle.free_state(st)


def test_tiny_one_step_vs_reference(oracle, reference, tmp_path):
    """Oracle and reference run each token of the reference's greedy run from
    the reference's own KV state: most steps agree to fp32 noise, the rest by
    at most one activation-quantization flip."""
    from oracle.binding import OrLayer, OrModel, OrWeight
    from ligguf_amd.model import TINY
    g = golden("tiny_decode.npz")
    hm = _tiny_model(g)
    path = str(tmp_path / "tiny.gguf")
    hm.write_gguf(path)
    reference.model_open(path, 0)
    st = oracle.new_state(hm.fill_desc(OrModel, OrLayer, OrWeight))
    toks = np.concatenate([g["prompt"], g["greedy"][:48]])
    errs, agree = [], []
    for pos, t in enumerate(toks):
        if pos:
            for l in range(TINY.n_layers):
                k, v = reference.kv_rows(l, 0, pos, TINY.kv_dim)
                oracle.state_kv_write(st, l, 0, pos, k, v)
        a = oracle.inference(st, int(t), TINY.vocab)
        b = reference.inference(int(t), TINY.vocab)
        errs.append(np.linalg.norm(a - b) / np.linalg.norm(b))
        agree.append(np.argmax(a) == np.argmax(b))
    errs = np.array(errs)
    oracle.free_state(st)
    assert np.median(errs) <= 1e-6
    assert np.mean(errs <= 1e-5) >= 0.7
    assert errs.max() <= 5e-2
    assert np.mean(agree) >= 0.95


# ---------------- next: top-p / top-k sampling ----------------
def _libc_draw(seed: int) -> float:
    """(float)rand() / (float)RAND_MAX after srand(seed), as the reference draws it"""
    import ctypes
    libc = ctypes.CDLL(None)
    libc.srand(ctypes.c_uint(seed))
    return float(np.float32(libc.rand()) / np.float32(2147483647))


def test_sampler_topp_closed_forms(oracle):
    rng = np.random.default_rng(11)
    lg = rng.normal(0, 2, 1000).astype(np.float32)
    lg[[17, 503]] = lg.max() + 1.0            # two equal maxima: the first wins
    assert oracle.sampler_topp(lg, 0.0, 0.9, 0, 0.5) == 17    # temp <= 0: greedy
    assert oracle.sampler_topp(lg, 0.8, 0.9, 1, 0.99) == 17   # top-1
    assert oracle.sampler_topp(lg, 0.8, 0.0, 0, 0.99) == 17   # topp <= 0: the first entry's p
    assert oracle.sampler_topp(lg, 0.8, 0.9, 2, 1.0) == 503   # the tie's second entry
    # hand-made distribution: p = 0.4, 0.3, 0.2, 0.1 at tokens 3, 0, 2, 1
    p = np.array([0.3, 0.1, 0.2, 0.4])
    lg4 = np.log(p).astype(np.float32)
    order = [3, 0, 2, 1]
    cum = np.cumsum(p[order])
    for i, tok in enumerate(order):
        lo = cum[i - 1] if i else 0.0
        r = (lo + cum[i]) / 2                 # the middle of entry i's interval
        assert oracle.sampler_topp(lg4, 1.0, 1.0, 0, float(r)) == tok
    # top-p 0.65 cuts after two entries (0.4 + 0.3 >= 0.65): r01 scales their 0.7
    assert oracle.sampler_topp(lg4, 1.0, 0.65, 0, 0.55) == 3    # 0.385 < 0.4
    assert oracle.sampler_topp(lg4, 1.0, 0.65, 0, 0.60) == 0    # 0.42 > 0.4
    assert oracle.sampler_topp(lg4, 1.0, 0.65, 0, 1.0) == 0     # never past the cutoff
    # top-k 3 with top-p 1: the cutoff is the third entry
    assert oracle.sampler_topp(lg4, 1.0, 1.0, 3, 1.0) == 2


@pytest.mark.parametrize("n,temp,topp,topk", [(1000, 1.0, 0.9, 0), (151936, 0.7, 0.95, 40), (151936, 2.0, 0.9, 0),
                                              (5000, 1.0, 0.0, 0), (5000, 1.5, 1.5, 5001), (4096, 0.5, 0.5, 3)])
def test_sampler_topp_vs_reference(oracle, reference, n, temp, topp, topk):
    rng = np.random.default_rng(n + topk)
    for seed in range(6):
        lg = (rng.normal(0, 3, n)).astype(np.float32)
        lg[rng.integers(0, n, n // 10)] = lg[0]          # ties
        want = reference.sampler_topp(lg, temp, topp, topk, seed)
        r01 = _libc_draw(seed)
        got = oracle.sampler_topp(lg, temp, topp, topk, r01)
        # the reference's -Ofast build sums and divides in its own order
        assert sampler_agree(lg, temp, topp, topk, r01, got, want), (seed, got, want)
