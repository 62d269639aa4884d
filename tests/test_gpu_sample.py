"""On-device top-p / top-k sampling (lg_sample_topp, lg_sample_topp_device)
against sampler_topp (fast/ligguf_fast_qk.cpp:172-214) evaluated in float64.

The device computes p = expf((l - max) / temp) in float32 and sums as trees;
its normalising sum and cumulative sums are within ~1e-6 of exact.  The
float64 restatement (sampler64) takes the same float32 exponentials and sums
them exactly enough, so the device must return its token unless the draw or
top-p lies within DEVICE_TOL of a cumulative probability (then a token within
DEVICE_TOL plus one entry of it), and must return exactly its token in at
least 6 of 8 trials of every case.  (The oracle's or_sampler_topp sums
sequentially in float, as the reference does, and is compared with the
reference in tests/test_oracle.py under the looser float-sum bound.)
"""
import numpy as np
import pytest
import torch

from ligguf_amd.lib import LgError, sample_topp_device
from ligguf_amd.model import TINY, Engine, HostModel

pytestmark = pytest.mark.gpu

# cumulative-probability distance within which two correct samplers may
# disagree: the device's float32 tree sums of up to 151936 terms are within
# ~1e-6 of exact; 1e-5 keeps a margin
DEVICE_TOL = 1e-5

CASES = [(151936, 0.8, 0.9, 0), (151936, 0.7, 0.95, 40), (151936, 2.0, 0.9, 0), (151936, 1.0, 0.0, 0),
         (151936, 1.0, 1.5, 0), (151936, 0.5, 0.5, 3), (1000, 1.0, 0.9, 0), (1, 1.0, 0.9, 0),
         (2049, 1.3, 0.99, 2056)]


def sampler64(lg, temp, topp, topk, r01):
    """sampler_topp with the float32 exponentials of the device and float64
    sums: (token, cumulative sums in sorted order, cutoff, r, order)."""
    lg = np.asarray(lg, np.float32)
    imax = int(np.argmax(lg))
    inv = np.float32(1.0) / np.float32(temp)
    e = np.exp(((lg - lg[imax]).astype(np.float32) * inv).astype(np.float32)).astype(np.float64)
    p = e / e.sum()
    order = np.lexsort((np.arange(p.size), -p))        # p descending, token ascending
    cum = np.cumsum(p[order])
    top = min(p[order[0]] if topp <= 0 else topp, 1.0)
    k = p.size if topk <= 0 or topk > p.size else topk
    cut = min(int(np.searchsorted(cum, top)), k - 1)
    r = r01 * cum[cut]
    pick = min(int(np.searchsorted(cum[:cut + 1], r)), cut)
    return int(order[pick]), cum, cut, r, order, top


def device_agrees(lg, temp, topp, topk, r01, got):
    want, cum, cut, r, order, top = sampler64(lg, temp, topp, topk, r01)
    if got == want:
        return True, True
    near = abs(cum[cut] - top) <= DEVICE_TOL or np.min(np.abs(cum[:cut + 1] - r)) <= DEVICE_TOL
    rank = np.empty(order.size, np.int64)
    rank[order] = np.arange(order.size)
    p = np.diff(np.concatenate([[0.0], cum]))
    far = abs(cum[rank[got]] - cum[rank[want]]) - max(p[rank[got]], p[rank[want]])
    return bool(near) and far <= DEVICE_TOL, False


@pytest.mark.parametrize("n,temp,topp,topk", CASES)
def test_sample_topp_device_vs_float64(gpu, n, temp, topp, topk):
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
        ok, same = device_agrees(lg, temp, topp, topk, r01, got)
        assert ok, (trial, got, sampler64(lg, temp, topp, topk, r01)[0])
        exact += same
    print(f"  identical in {exact} of 8 trials")
    assert exact >= 6, exact


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


def test_sample_topp_large_buckets(gpu):
    """Leading-digit buckets holding more entries than the select pass keeps
    in LDS (12288): the selections read every block's slice from global
    memory.  40000 equal logits (one bucket, every pick a tie broken by
    token, ranks past 0 taking the token selection), and a near-flat
    151936-entry vocabulary against sampler64."""
    n = 40000
    t = torch.zeros(n, dtype=torch.float32, device="cuda:0")
    for i in (0, 1, 12287, 12288, 20000, 39999):
        assert sample_topp_device(t.data_ptr(), n, 1.0, 1.0, 0, (i + 0.5) / n) == i
    # top-k 30000: the draw scaled to the first 30000, mid-way through entry 15000
    assert sample_topp_device(t.data_ptr(), n, 1.0, 1.0, 30000, 15000.5 / 30000) == 15000
    rng = np.random.default_rng(11)
    exact = 0
    for trial in range(8):
        lg = rng.normal(0, 0.02, 151936).astype(np.float32)
        r01 = float(np.float32(rng.random()))
        x = torch.from_numpy(lg).to("cuda:0")
        got = sample_topp_device(x.data_ptr(), lg.size, 1.0, 0.9, 0, r01)
        ok, same = device_agrees(lg, 1.0, 0.9, 0, r01, got)
        assert ok, (trial, got, sampler64(lg, 1.0, 0.9, 0, r01)[0])
        exact += same
    print(f"  near-flat: identical in {exact} of 8 trials")
    assert exact >= 6


def test_sample_topp_rejects_bad_draw(gpu):
    t = torch.zeros(16, dtype=torch.float32, device="cuda:0")
    with pytest.raises(LgError):
        sample_topp_device(t.data_ptr(), 16, 1.0, 0.9, 0, 1.5)


def test_engine_sample_topp_after_decode(gpu):
    """lg_sample_topp over the logits a decode step left on the device, the
    same draw through sampler64 on their host copy; the second context size
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
                if temp > 0:
                    assert device_agrees(lg, temp, topp, topk, r01, got)[0], (pos, temp, got)
                else:
                    assert got == int(np.argmax(lg))
            tok = got
    finally:
        eng.close()
