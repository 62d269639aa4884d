"""Flip-explained parity: the quantized activations of a GPU step against the
oracle's, element by element.

inference() quantizes 4 n_layers + 1 activations per token
(fast/ligguf_fast_qk.cpp:39,108,116,126,140) with quantize_q8_K or
quantize_q8_0 (fast/lil_math.cpp:329-394).  Two correct implementations that
round their fp32 sums in different orders produce int8 values that agree
except where an activation lies within that rounding noise of a rounding
boundary (x * 127/amax = k + 1/2).  Such a "flip" moves one int8 by one step
and, on these random-weight models, the logits by ~1e-3..1e-2.

``step_flips`` walks the quantized activations of one step in execution order
and compares the GPU's int8 values (lg_trace_acts_next_step) with the int8
values the as-compiled quantizer gives for the oracle's float vector at the
same point (or_state_trace).  The first activation that differs must differ
only by flips: every differing value one step away, and the oracle's
pre-rounding value within FLIP_TOL of k + 1/2.  Everything after it in the
step depends on the flipped value, so the walk stops there.  A step with no
differing int8 at all must match the oracle's logits to fp32 noise.

``forced_flips`` compares every activation of a step instead: the oracle
step takes the GPU's quantized activations as the inputs of its matvecs
(or_state_force), so activation k is formed from the same quantized
activations < k on both sides, a flip does not propagate, and each of the
4 n_layers + 1 activations is held to the flip rule on its own.  The logits
of such a step are then a function of the same quantized head input on both
sides and must agree to fp32 noise.

Q8_0 blocks also carry an fp16 scale, fp16(amax / 127), which the next matvec
multiplies in: when amax / 127 lies on an fp16 rounding tie, an amax one fp32
ulp apart rounds the scale one fp16 ulp (~1e-3) the other way with every int8
equal.  A differing Q8_0 scale is therefore a difference of its activation
too, a flip when the oracle's amax / 127 is within SCALE_TIE_TOL fp16 ulps of
a tie.
"""
from __future__ import annotations

import numpy as np

from ligguf_amd.lib import BLOCK, F16, F32, Q1_0, Q1_G, Q8_0, Q8_K

# distance of the oracle's scaled value v = x * 127/amax from k + 1/2 below
# which a one-step difference counts as a rounding flip.  Matvec outputs are
# exact only to ~2e-6 of the row's sum of |terms| (the fp32 combination of
# exact integer block sums), so a value formed by cancelling terms, then
# normalised and scaled to v, differs between the GPU and the oracle by up to
# ~1e-2 of a quantization step (largest seen: 0.0117 on the tiny model).
# 0.05 keeps a 4x margin; a differing value that is no flip lands this close to
# a boundary with probability 0.1, and MAX_FLIPS bounds how many may differ.
FLIP_TOL = 0.05
# differing int8 values allowed in the first differing activation of a step:
# when a block's largest value itself moves by the noise above, every value of
# the block shifts with it, so several flips can share one block (9 of 768
# seen on the tiny model); a fraction of the width bounds them
MAX_FLIP_FRAC = 0.02
# values this close to a boundary are ties at fp32 resolution (|v| <= 127.5,
# so fp32 rounding alone moves v by ~1e-5): any reordering rounds them either
# way, and they do not count against MAX_FLIP_FRAC.  Quantized tables make
# many: a Q6_K embedding row is integers times per-16 scales, so values of
# the block holding the maximum scale to exact halves (127 q / 32 for q = 16)
# -- 60-80 of 1024 per token on the synthetic Q6_K models.
TIE_TOL = 1e-4
# distance (in fp16 ulps) of a Q8_0 block's amax / 127 from an fp16 rounding
# tie below which a scale one fp16 ulp off counts as a flip: amax moves by
# ~1e-7..1e-5 relative between two correct paths (1e-4..1e-2 of an fp16 ulp)
SCALE_TIE_TOL = 0.1
# logits rel-L2 of a step whose int8 activations all agree with the oracle's
EXACT_STEP = 1e-5
# with the GPU's quantized activations forced into the oracle step every
# activation is formed from identical quantized inputs: a differing int8 is
# then within fp32 noise of a boundary (at most 3.1e-5 from it over every
# step measured: the 36-layer Qwen3-8B-shape Q4_K and Q1_G models at 13
# positions and the small models of the GPU suite), so a one-step
# difference farther than 1e-3 is no flip; the logits, one matvec of the same
# head input, agree to ~8e-8 (at most 8.4e-8 measured)
FORCED_FLIP_TOL = 1e-3
FORCED_STEP = 1e-6

K_FAMILY = {10, 11, 12, 13, 14}   # Q2_K..Q6_K read Q8_K activations


def slot_formats(cfg):
    """(quantized form, width) of each of the 4 n_layers + 1 activations of a
    step, as lg_trace_acts_next_step records them (None: float activation)."""
    def form(*types):
        # the Q8_K form when any consumer is a K-quant, as the step records it
        if any(t in K_FAMILY for t in types):
            return Q8_K
        if any(t in (Q8_0, Q1_0, Q1_G) for t in types):
            return Q8_0
        return None
    out = []
    for l in range(cfg.n_layers):
        def tt(t):
            return cfg.tensor_type(t, l)
        out += [(form(tt("attn_q"), tt("attn_k"), tt("attn_v")), cfg.n_embed), (form(tt("attn_output")), cfg.n_embed),
                (form(tt("ffn_up"), tt("ffn_gate")), cfg.n_embed), (form(tt("ffn_down")), cfg.n_ff)]
    out.append((form(cfg.out_type), cfg.n_embed))
    return out


def parse_q(buf: np.ndarray, qtype: int, n: int):
    """int8 quants and float scales of n values in block_q8_K / block_q8_0."""
    qk, bs = BLOCK[qtype]
    nb = n // qk
    blk = np.asarray(buf[:nb * bs], np.uint8).reshape(nb, bs)
    if qtype == Q8_K:
        d = blk[:, 0:4].copy().view(np.float32).ravel()
        qs = blk[:, 4:260].copy().view(np.int8).ravel()
    else:
        d = blk[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
        qs = blk[:, 2:34].copy().view(np.int8).ravel()
    return qs, d


def quantize_ref(x: np.ndarray, qtype: int):
    """quantize_q8_K / quantize_q8_0 as the reference compiles them, in
    float32 arithmetic (the oracle's or_quantize_*): (int8 quants, the scaled
    values v they round)."""
    x = np.asarray(x, np.float32)
    if qtype == Q8_0:
        b = x.reshape(-1, 32)
        amax = np.abs(b).max(axis=1)
        idv = np.where(amax != 0, np.float32(127.0) / np.where(amax != 0, amax, np.float32(1)), np.float32(0))
        v = (b * idv[:, None].astype(np.float32)).astype(np.float32)
        t = np.trunc(v)
        q = t + np.sign(v) * (np.abs(v - t) >= np.float32(0.5))     # roundf: half away from zero
        return q.astype(np.int8).ravel(), v.ravel()
    b = x.reshape(-1, 256)
    ia = np.argmax(np.abs(b), axis=1)                                # first index of the largest magnitude
    mx = b[np.arange(b.shape[0]), ia]
    isc = np.where(mx != 0, np.float32(-127.0) / np.where(mx != 0, mx, np.float32(1)), np.float32(0))
    v = (b * isc[:, None].astype(np.float32)).astype(np.float32)
    r = np.where(v < 0, v - np.float32(0.5), v + np.float32(0.5)).astype(np.float32)   # nearest_int as compiled
    q = np.minimum(np.trunc(r), 127)
    return q.astype(np.int8).ravel(), v.ravel()


def boundary_dist(v: np.ndarray) -> np.ndarray:
    a = np.abs(v.astype(np.float64))
    return np.abs(a - np.floor(a) - 0.5)


def scale_diffs(buf: np.ndarray, x: np.ndarray, qtype: int, n: int):
    """Q8_0 blocks whose fp16 scale in `buf` differs from fp16(amax / 127) of
    the oracle's values x (quantize_q8_0, fast/lil_math.cpp:363-394): the
    blocks and, per block, the distance of amax / 127 from an fp16 rounding
    tie in fp16 ulps -- or 1.0 when the two scales are not neighbours.
    Empty for other forms."""
    if qtype != Q8_0:
        return np.zeros(0, np.int64), np.zeros(0)
    _, dg = parse_q(buf, qtype, n)
    amax = np.abs(np.asarray(x[:n], np.float32).reshape(-1, 32)).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    d16 = d.astype(np.float16).astype(np.float32)
    diff = np.nonzero(dg != d16)[0]
    dd = d[diff].astype(np.float64)
    e = np.maximum(np.floor(np.log2(np.where(dd > 0, dd, 1.0))), -14.0)   # fp16 subnormals: ulp 2^-24
    ulp = 2.0 ** (e - 10)
    f = dd / ulp
    dist = np.abs(f - np.floor(f) - 0.5)
    neighbours = np.abs(dg[diff].astype(np.float64) - d16[diff]) <= ulp * 1.0000001
    return diff, np.where(neighbours, dist, 1.0)


def slot_check(gbuf: np.ndarray, x: np.ndarray, qt: int, n: int, tag=(), flip_tol=FLIP_TOL):
    """One quantized activation: the GPU's blocks `gbuf` against the
    as-compiled quantizer applied to the oracle's float vector x at the same
    point.  Returns (differs, unexplained): every differing int8 must be one
    step away with the oracle's pre-rounding value within FLIP_TOL of k + 1/2,
    at most max(8, MAX_FLIP_FRAC n) of them off exact ties, and every
    differing Q8_0 scale must sit within SCALE_TIE_TOL of an fp16 tie.
    Returns (differs, unexplained, largest boundary distance of a differing
    int8); entries of `unexplained` start with `tag`."""
    qg, _ = parse_q(gbuf, qt, n)
    qo, v = quantize_ref(x[:n], qt)
    diff = np.nonzero(qg != qo)[0]
    sdiff, sdist = scale_diffs(gbuf, x, qt, n)
    if diff.size == 0 and sdiff.size == 0:
        return False, [], 0.0
    bad = []
    dists = boundary_dist(v[diff])
    nties = int(np.sum(dists < TIE_TOL))
    if diff.size - nties > max(8, int(MAX_FLIP_FRAC * n)):
        bad.append(tag + (-1, int(diff.size), n, 0.0, 1.0))
    for i in diff:
        step = abs(int(qg[i]) - int(qo[i]))
        dist = float(boundary_dist(v[i:i + 1])[0])
        if step != 1 or dist > flip_tol:
            bad.append(tag + (int(i), int(qg[i]), int(qo[i]), float(v[i]), dist))
    for b, dist in zip(sdiff, sdist):
        if dist > SCALE_TIE_TOL:
            bad.append(tag + (-2, int(b), 0, 0.0, float(dist)))     # a scale off an fp16 tie
    return True, bad, float(dists.max()) if diff.size else 0.0


def step_flips(gpu_trace: np.ndarray, oracle_trace: np.ndarray, cfg):
    """(first differing activation or -1, list of unexplained differences).

    gpu_trace: [4L+1][stride] bytes from lg_trace_acts_next_step;
    oracle_trace: [4L+1][max(n_embed, n_ff)] floats from or_state_trace."""
    for k, (qt, n) in enumerate(slot_formats(cfg)):
        if qt is None:
            continue
        differs, bad, _ = slot_check(gpu_trace[k], oracle_trace[k], qt, n, (k,))
        if differs:
            return k, bad
    return -1, []


def forced_flips(gpu_trace: np.ndarray, oracle_trace: np.ndarray, cfg, flip_tol=FORCED_FLIP_TOL):
    """Every quantized activation of a step against an oracle step that took
    the GPU's quantized activations as its inputs (or_state_force): there each
    activation k is computed from the same quantized activations < k on both
    sides, so no flip propagates and every one of the 4 L + 1 points is
    compared, with differing values held to flip_tol.  Returns (compared, differing, unexplained, largest boundary
    distance of a differing int8)."""
    compared, differing, bad, worst = 0, 0, [], 0.0
    for k, (qt, n) in enumerate(slot_formats(cfg)):
        if qt is None:
            continue
        differs, b, d = slot_check(gpu_trace[k], oracle_trace[k], qt, n, (k,), flip_tol)
        compared += 1
        differing += int(differs)
        bad += b
        worst = max(worst, d)
    return compared, differing, bad, worst


def prefill_flips(gpu_trace: np.ndarray, oracle_traces, cfg):
    """The quantized activations of a batched prefill of n tokens against the
    oracle's token-by-token run of the same prompt.

    gpu_trace: [n][4L+1][stride] (lg_trace_acts_next_prefill); oracle_traces:
    n arrays [4L+1][wide] (or_state_trace per step).  A pass computes
    activation k of every token before activation k+1 of any, and token t's
    activation k depends on activations < k of tokens <= t only (its own
    stream and, through the KV rows, the earlier tokens').  So (token t,
    activation k) is compared while no token <= t differed at an activation
    < k; every difference found there must be a rounding flip as in
    step_flips.  Returns (compared, differing, unexplained list, last token
    clean through every activation)."""
    fm = slot_formats(cfg)
    n, nk = len(oracle_traces), len(fm)
    first = np.full(n, nk + 1)          # first differing activation of each token
    compared, differing, bad = 0, 0, []
    for k in range(nk):
        qt, w = fm[k]
        if qt is None:
            continue
        toks = [n - 1] if k == nk - 1 else range(n)      # the output head's input: the last token only
        for t in toks:
            if first[:t + 1].min() < k:
                continue
            qg, _ = parse_q(gpu_trace[t][k], qt, w)
            qo, v = quantize_ref(oracle_traces[t][k][:w], qt)
            compared += 1
            diff = np.nonzero(qg != qo)[0]
            sdiff, sdist = scale_diffs(gpu_trace[t][k], oracle_traces[t][k], qt, w)
            if diff.size == 0 and sdiff.size == 0:
                continue
            differing += 1
            first[t] = k
            nties = int(np.sum(boundary_dist(v[diff]) < TIE_TOL))
            if diff.size - nties > max(8, int(MAX_FLIP_FRAC * w)):
                bad.append((t, k, -1, int(diff.size), w, 0.0, 1.0))
            for i in diff:
                step = abs(int(qg[i]) - int(qo[i]))
                dist = float(boundary_dist(v[i:i + 1])[0])
                if step != 1 or dist > FLIP_TOL:
                    bad.append((t, k, int(i), int(qg[i]), int(qo[i]), float(v[i]), dist))
            for b, dist in zip(sdiff, sdist):
                if dist > SCALE_TIE_TOL:
                    bad.append((t, k, -2, int(b), 0, 0.0, float(dist)))
    return compared, differing, bad, bool(first.min() > nk)


def flip_summary(rows):
    """rows: (first_slot, n_bad, rel) per step -> printable counts."""
    exact = sum(1 for f, b, r in rows if f < 0)
    flips = sum(1 for f, b, r in rows if f >= 0 and b == 0)
    bad = sum(1 for f, b, r in rows if b)
    worst_exact = max([r for f, b, r in rows if f < 0] or [0.0])
    return f"{len(rows)} steps: {exact} without int8 differences (max rel-L2 {worst_exact:.1e}), " \
           f"{flips} with rounding flips only, {bad} unexplained"


__all__ = ["FLIP_TOL", "MAX_FLIP_FRAC", "TIE_TOL", "SCALE_TIE_TOL", "EXACT_STEP", "FORCED_FLIP_TOL", "FORCED_STEP", "slot_formats", "parse_q",
           "quantize_ref", "scale_diffs", "slot_check", "step_flips", "forced_flips", "prefill_flips", "flip_summary",
           "F16", "F32"]
