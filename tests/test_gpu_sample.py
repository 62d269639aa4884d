"""On-device top-p / top-k sampling (lg_sample_topp, lg_sample_topp_device)
against the oracle's sampler_topp (fast/ligguf_fast_qk.cpp:172-214).

The device sums probabilities as trees, the oracle (like the reference
source) sequentially: tokens must be identical unless the draw or top-p lies
within float rounding of a cumulative probability (conftest.sampler_agree),
and identical in most trials of every case.
"""
import numpy as np
import pytest
import torch

from conftest import sampler_agree
from ligguf_amd.lib import LgError, sample_topp_device
from ligguf_amd.model import TINY, Engine, HostModel

pytestmark = pytest.mark.gpu

# (n, temp, topp, topk, identical trials of 8 at least): top-p over all of a
# 151936-entry vocabulary normalises by a sum of 151936 terms, which the
# oracle's sequential float sum gets wrong by ~5e-4 relative -- several
# entries' widths at the cutoff -- so only the tolerance holds there
CASES = [(151936, 0.8, 0.9, 0, 0), (151936, 0.7, 0.95, 40, 6), (151936, 2.0, 0.9, 0, 0), (151936, 1.0, 0.0, 0, 6),
         (151936, 1.0, 1.5, 0, 0), (151936, 0.5, 0.5, 3, 6), (1000, 1.0, 0.9, 0, 6), (1, 1.0, 0.9, 0, 8),
         (2049, 1.3, 0.99, 2056, 6)]


@pytest.mark.parametrize("n,temp,topp,topk,min_exact", CASES)
def test_sample_topp_device_vs_oracle(gpu, oracle, n, temp, topp, topk, min_exact):
    print(f"sample n={n} temp={temp} topp={topp} topk={topk}", flush=True)
    rng = np.random.default_rng(n * 7 + topk)
    exact = 0
    for trial in range(8):
        lg = rng.normal(0, 3, n).astype(np.float32)
        if n > 10:
            lg[rng.integers(0, n, n // 10)] = lg[0]      # ties
        r01 = 1.0 if trial == 0 else 0.0 if trial == 1 else float(np.float32(rng.random()))
        t = torch.from_numpy(lg).to("cuda:0")
        got = sample_topp_device(t.data_ptr(), n, temp, topp, topk, r01)
        want = oracle.sampler_topp(lg, temp, topp, topk, r01)
        assert sampler_agree(lg, temp, topp, topk, r01, got, want), (trial, got, want)
        exact += got == want
    assert exact >= min_exact, exact


def test_sample_topp_ties_take_lower_token(gpu):
    """Equal logits: every p is 1/n, the order is by token, so the draw in the
    middle of entry i's interval picks token i (cmp_sampler_ent_desc,
    fast/ligguf_fast_qk.cpp:162-170)."""
    n = 5000
    t = torch.zeros(n, dtype=torch.float32, device="cuda:0")
    for i in (0, 1, 17, 2500, 4998, 4999):
        assert sample_topp_device(t.data_ptr(), n, 1.0, 1.0, 0, (i + 0.5) / n) == i
    # top-k 100 scales the draw to the first 100 entries
    assert sample_topp_device(t.data_ptr(), n, 1.0, 1.0, 100, 0.505) == 50
    # temp <= 0: greedy, the first maximum
    t[[40, 7]] = 1.0
    assert sample_topp_device(t.data_ptr(), n, 0.0, 0.9, 0, 0.3) == 7


def test_sample_topp_rejects_bad_draw(gpu):
    t = torch.zeros(16, dtype=torch.float32, device="cuda:0")
    with pytest.raises(LgError):
        sample_topp_device(t.data_ptr(), 16, 1.0, 0.9, 0, 1.5)


def test_engine_sample_topp_after_decode(gpu, oracle):
    """lg_sample_topp over the logits a decode step left on the device, the
    same draw through the oracle on their host copy; the second context size
    check reuses the workspace."""
    hm = HostModel.synthetic(TINY)
    eng = Engine(0)
    try:
        eng.load(hm)
        rng = np.random.default_rng(5)
        tok = 1
        for pos in range(4):
            lg = eng.decode(tok, pos)
            for temp, topp, topk in ((0.8, 0.9, 0), (1.0, 0.5, 5), (0.0, 0.9, 0)):
                r01 = float(np.float32(rng.random()))
                got = eng.sample_topp(temp, topp, topk, r01)
                want = oracle.sampler_topp(lg, temp, topp, topk, r01)
                assert sampler_agree(lg, temp, topp, topk, r01, got, want), (pos, temp, got, want)
            tok = got
    finally:
        eng.close()
