"""GPU per-op parity through the C-ABI against the oracle and the golden
vectors.  Bars: bit-exact for dequantization and the activation quantizers;
matvec within 2e-6 of the sum of |terms| of each row (the reference's own
fp32 summation sits at ~2e-7 of it); float ops within the stated relative
tolerances."""
import numpy as np
import pytest
import torch

from conftest import golden
from ligguf_amd import encode, ops
from ligguf_amd.lib import BLOCK, F16, F32, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0, Q8_K, row_size

pytestmark = pytest.mark.gpu

WEIGHT_TYPES = [Q8_0, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]
MATVEC_TOL = 2e-6


def dev(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


# ---------------- quantizers (bit-exact) ----------------
def test_quantizers_golden(gpu):
    g = golden("quant.npz")
    x = dev(g["x"], gpu)
    assert np.array_equal(host(ops.quantize_q8_0(x)), g["q8_0"])
    assert np.array_equal(host(ops.quantize_q8_K(x)), g["q8_K"])


@pytest.mark.parametrize("n", [288, 768, 4096, 12288, 14336])
def test_quantizers_random(gpu, oracle, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * rng.choice([1e-3, 0.05, 3.0])).astype(np.float32)
    assert np.array_equal(host(ops.quantize_q8_0(dev(x, gpu))), oracle.quantize_q8_0(x))
    if n % 256 == 0:
        assert np.array_equal(host(ops.quantize_q8_K(dev(x, gpu))), oracle.quantize_q8_K(x))


# ---------------- dequant (bit-exact) ----------------
@pytest.mark.parametrize("t", WEIGHT_TYPES)
def test_dequant_golden(gpu, t):
    g = golden("dequant.npz")
    ref = g[f"out_{t}"]
    y = host(ops.dequantize_row(t, dev(g[f"in_{t}"], gpu), ref.size))
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("t", WEIGHT_TYPES + [F16, F32])
def test_dequant_random_tensor(gpu, oracle, t):
    rows, cols = 96, 4096
    w = encode.random_tensor(t, 11, t, rows, cols, 0.02)
    y = host(ops.dequantize_row(t, dev(w, gpu), rows * cols))
    rsz = row_size(t, cols)
    ref = np.concatenate([oracle.dequantize_row(t, w[r * rsz:(r + 1) * rsz], cols) for r in range(rows)])
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


# ---------------- matvec ----------------
def _act(t, x, gpu, oracle):
    if t in (F16, F32):
        return dev(x, gpu), x
    if t in (Q8_0, Q1_0, Q1_G):
        return ops.quantize_q8_0(dev(x, gpu)), oracle.quantize_q8_0(x)
    return ops.quantize_q8_K(dev(x, gpu)), oracle.quantize_q8_K(x)


def _check_matvec(gpu, oracle, t, n, d, w=None, seed=0):
    rng = np.random.default_rng(seed)
    if w is None:
        w = encode.random_q1(t, seed, t, d, n) if t in (Q1_0, Q1_G) else encode.random_tensor(t, seed, t, d, n)
    x = rng.standard_normal(n).astype(np.float32)
    xq_d, xq_h = _act(t, x, gpu, oracle)
    rsz = row_size(t, n)
    y = host(ops.matvec(t, dev(w, gpu), rsz, n, d, xq_d))
    ref, ab = oracle.matvec_q(t, w, rsz, n, d, xq_h, want_abs=True)
    err = np.abs(y - ref) / np.maximum(ab, 1e-30)
    assert np.all(err <= MATVEC_TOL), (t, n, d, float(err.max()))
    return w, xq_d, y


@pytest.mark.parametrize("t", WEIGHT_TYPES + [F16, F32])
@pytest.mark.parametrize("n", [256 * 1, 288, 768, 4096, 12288])
def test_matvec_formats_widths(gpu, oracle, t, n):
    qk, _ = BLOCK[t]
    if n % qk or (t in (Q2_K, Q3_K, Q4_K, Q5_K, Q6_K) and n % 256):
        pytest.skip("width not a block multiple")
    _check_matvec(gpu, oracle, t, n, 200, seed=n)


def test_matvec_golden(gpu):
    g = golden("matmul.npz")
    n, d = 1024, 48
    for t in WEIGHT_TYPES + [F16, F32]:
        qk, bs = BLOCK[t]
        x = dev(g["x"], gpu)
        xq = x if t in (F16, F32) else (ops.quantize_q8_0(x) if t in (Q8_0, Q1_0, Q1_G) else ops.quantize_q8_K(x))
        y = host(ops.matvec(t, dev(g[f"w_{t}"], gpu), n // qk * bs, n, d, xq))
        ref = g[f"y_{t}"]
        assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref)), t


def test_matvec_accumulate(gpu, oracle):
    w, xq, y = _check_matvec(gpu, oracle, Q4_K, 4096, 512, seed=3)
    base = torch.arange(512, dtype=torch.float32, device=gpu)
    out = base.clone()
    ops.matvec(Q4_K, dev(w, gpu), row_size(Q4_K, 4096), 4096, 512, xq, out=out, accumulate=True)
    assert np.allclose(host(out), host(base) + y, rtol=0, atol=1e-5)


@pytest.mark.parametrize("t,d,n", [(Q4_K, 4096, 4096), (Q4_K, 14336, 4096), (Q6_K, 128256, 4096)])
def test_matvec_isolated_workload_shapes(gpu, oracle, t, d, n):
    """The isolated matvec shapes (Q4_K 4096x4096, 14336x4096, Q6_K 128256x4096):
    every row against the oracle."""
    _check_matvec(gpu, oracle, t, n, d, seed=d)


# ---------------- fused norms / rope / swiglu ----------------
@pytest.mark.parametrize("n", [288, 4096])
def test_rmsnorm_quant(gpu, oracle, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    f = host(ops.rmsnorm_quant(dev(x, gpu), dev(w, gpu), 1e-5, F32))
    ref = oracle.rmsnorm(x, w, 1e-5)
    assert np.max(np.abs(f - ref) / (np.abs(ref) + 1e-3)) < 2e-6
    # the quantized form is the quantizer applied to the GPU's own float output
    q, f2 = ops.rmsnorm_quant(dev(x, gpu), dev(w, gpu), 1e-5, Q8_0, want_float=True)
    assert np.array_equal(host(q), oracle.quantize_q8_0(host(f2)))
    if n % 256 == 0:
        q = ops.rmsnorm_quant(dev(x, gpu), dev(w, gpu), 1e-5, Q8_K)
        assert np.array_equal(host(q), oracle.quantize_q8_K(f))


@pytest.mark.parametrize("nh,nkv,hd,pos,qk", [(6, 6, 48, 37, False), (32, 8, 128, 517, True),
                                             (32, 8, 128, 32767, True), (4, 2, 64, 0, True)])
def test_qk_norm_rope_kv(gpu, oracle, nh, nkv, hd, pos, qk):
    rng = np.random.default_rng(pos)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    freq = golden("ops.npz")["freq_q"] if hd == 128 else (10000.0 ** (-2 * np.arange(hd // 2) / hd)).astype(np.float32)
    qd, kd, vd = dev(q, gpu), dev(k, gpu), dev(v, gpu)
    kc = torch.zeros(nkv * hd, dtype=torch.int16, device=gpu)
    vc = torch.zeros(nkv * hd, dtype=torch.int16, device=gpu)
    ops.qk_norm_rope_kv(qd, kd, vd, dev(qw, gpu) if qk else None, dev(kw, gpu) if qk else None, nh, nkv, hd, hd, pos,
                        dev(freq, gpu), 1e-6, kc, vc)
    rq, rk = q.copy(), k.copy()
    if qk:
        rq = np.concatenate([oracle.rmsnorm(rq[h * hd:(h + 1) * hd], qw, 1e-6) for h in range(nh)])
        rk = np.concatenate([oracle.rmsnorm(rk[h * hd:(h + 1) * hd], kw, 1e-6) for h in range(nkv)])
    rq = oracle.rope(rq, nh, hd, hd, pos, freq)
    rk = oracle.rope(rk, nkv, hd, hd, pos, freq)
    assert np.max(np.abs(host(qd) - rq)) < 1e-5 * np.max(np.abs(rq))
    assert np.max(np.abs(host(kd) - rk)) < 1e-5 * np.max(np.abs(rk))
    kh = host(kc).view(np.uint16)
    # fp16 of the GPU's own rotated k, and within one half-ulp step of the oracle's
    assert np.array_equal(kh, oracle.fp32_to_fp16(host(kd)))
    assert np.array_equal(host(vc).view(np.uint16), oracle.fp32_to_fp16(v))
    assert np.max(np.abs(kh.view(np.float16).astype(np.float32) - rk)) <= 2 ** -10 * np.max(np.abs(rk))


def test_swiglu_quant(gpu, oracle):
    rng = np.random.default_rng(7)
    u = rng.standard_normal(12288).astype(np.float32)
    g = (rng.standard_normal(12288) * 3).astype(np.float32)
    ud = dev(u, gpu)
    q = ops.swiglu_quant(ud, dev(g, gpu), Q8_K)
    out = host(ud)
    ref = oracle.swiglu(u, g)
    assert np.max(np.abs(out - ref) / (np.abs(ref) + 1e-3)) < 2e-6
    assert np.array_equal(host(q), oracle.quantize_q8_K(out))


# ---------------- attention ----------------
def _attn_case(gpu, oracle, nh, nkv, hd, pos, seed):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    kc = rng.standard_normal(max(pos, 1) * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(max(pos, 1) * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    out = host(ops.attention(dev(q, gpu), dev(k, gpu), dev(v, gpu), dev(kc, gpu), dev(vc, gpu), nh, nkv, hd, pos))
    ref = oracle.attention(q, k, v, kc, vc, nh, nkv, hd, pos)
    return out, ref


@pytest.mark.parametrize("nh,nkv,hd,pos", [(32, 8, 128, 511), (32, 8, 128, 4095), (32, 8, 128, 32767),
                                           (6, 6, 48, 200), (8, 4, 64, 1000), (16, 2, 128, 77), (32, 8, 128, 0),
                                           (32, 8, 128, 1), (16, 4, 256, 700), (8, 8, 64, 33), (32, 8, 128, 300000)])
def test_attention(gpu, oracle, nh, nkv, hd, pos):
    out, ref = _attn_case(gpu, oracle, nh, nkv, hd, pos, pos + hd)
    assert np.max(np.abs(out - ref)) <= 2e-6 * max(1.0, float(np.max(np.abs(ref)))), float(np.max(np.abs(out - ref)))


def test_attention_golden(gpu):
    g = golden("ops.npz")
    pos = int(g["att_pos"])
    out = host(ops.attention(dev(g["att_q"], gpu), dev(g["att_k"], gpu), dev(g["att_v"], gpu),
                             dev(g["att_kc"], gpu), dev(g["att_vc"], gpu), 8, 2, 128, pos))
    assert np.max(np.abs(out - g["att_out"])) < 1e-5 * np.max(np.abs(g["att_out"]))


def test_hbm_read_probe(gpu):
    """lg_hbm_read_probe reads its buffer: a 1 GiB pass takes at least the
    time 8 TB/s allows (a rate above the peak would mean loads were dropped)."""
    import ctypes as C
    from ligguf_amd import lib as L
    n = 1 << 30
    buf = torch.ones(n // 4, dtype=torch.float32, device=gpu)
    us = C.c_float()
    L.check(L.load().lg_hbm_read_probe(C.c_void_p(buf.data_ptr()), n, 3, C.byref(us),
                                       C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    gbs = n / (us.value * 1e-6) / 1e9
    print(f"\nread probe: {gbs:.0f} GB/s over 1 GiB")
    assert 1000.0 < gbs < 8100.0
