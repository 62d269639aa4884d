import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running case")


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name))


@pytest.fixture(scope="session")
def oracle():
    from oracle import load_oracle
    return load_oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import load_reference, reference_available
    if not reference_available():
        pytest.skip("reference engine (oracle/_ref) not built here")
    return load_reference()


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from ligguf_amd import lib
    lib.load()   # raises when the HIP library is missing: no fallback
    return torch.device("cuda:0")


def sampler_agree(logits, temp, topp, topk, r01, tok_a, tok_b, margin=1e-4):
    """Two top-p samples of the same logits and draw agree: the same token
    when r01 * cum and top lie farther than tol from every cumulative
    probability up to the cutoff (probabilities sum to 1), else tokens whose
    cumulative probabilities (order by p descending, token ascending) differ
    by at most tol plus the larger entry.  tol = margin + 2 (n + cut + 1)
    2^-24: float sums taken in another order (sequential, tree, vectorised)
    move by up to (terms) 2^-24 relative -- the normalising sum of all n
    entries scales every p, the running sum of cut + 1 entries moves the
    cutoff and r."""
    if tok_a == tok_b:
        return True
    lg = np.asarray(logits, np.float64)
    p = np.exp((lg - lg.max()) / temp)
    p /= p.sum()
    order = np.lexsort((np.arange(p.size), -p))
    cum = np.cumsum(p[order])
    top = min(p[order[0]] if topp <= 0 else topp, 1.0)
    k = p.size if topk <= 0 or topk > p.size else topk
    cut = min(int(np.searchsorted(cum, top)), k - 1)
    r = r01 * cum[cut]
    tol = margin + 2.0 * (p.size + cut + 1) * 2.0 ** -24
    near = abs(cum[cut] - top) <= tol or np.min(np.abs(cum[:cut + 1] - r)) <= tol
    rank = np.empty(p.size, np.int64)
    rank[order] = np.arange(p.size)
    far = abs(cum[rank[tok_a]] - cum[rank[tok_b]]) - max(p[tok_a], p[tok_b])
    return bool(near) and far <= tol
