"""The flip-explained parity helper (tests/parity.py) against the oracle's own
quantizers: its float32 restatement of quantize_q8_K / quantize_q8_0 must give
the oracle's int8 values bit for bit (the oracle itself is pinned to the
reference's golden vectors in test_oracle.py), and a planted off-boundary
difference must be reported."""
import numpy as np

from conftest import golden
from ligguf_amd.lib import Q8_0, Q8_K
from ligguf_amd.model import TINY
from parity import boundary_dist, parse_q, quantize_ref, slot_formats, step_flips


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
