"""Write the golden vectors of the decode path from the reference engine.

Runs in the build container only: it needs oracle/_ref/libligguf_ref.so,
compiled from the reference's own sources (``make -C oracle ref``).  The
outputs are small .npz fixtures next to this script; tests compare the oracle
(and through it the GPU path) against them on machines without the
reference.

    python tests/golden/make_golden.py                  # everything
    python tests/golden/make_golden.py --teacher-only   # tiny_teacher.npz alone
    python tests/golden/make_golden.py --bert-only      # bert.npz alone
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from ligguf_amd import encode  # noqa: E402
from ligguf_amd.lib import BLOCK, F16, F32, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_0  # noqa: E402
from ligguf_amd.model import TINY, HostModel  # noqa: E402
from oracle.binding import OrLayer, OrModel, OrWeight, RefLayer, RefModel, RefWeight, load_oracle, load_reference  # noqa: E402

WEIGHT_TYPES = [Q8_0, Q1_0, Q1_G, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K]
# block field offsets of the fp16 scales (fast/lil_gguf.h:64-113)
D_OFFS = {Q8_0: [0], Q1_0: [0], Q1_G: [0], Q2_K: [80, 82], Q3_K: [108], Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208]}


def random_blocks(rng, t, nb):
    """Random block bytes with finite fp16 scales of moderate size; Q8_0
    quants kept in [-127, 127] as quantize_q8_0 produces them."""
    qk, bs = BLOCK[t]
    if t == Q8_0:
        blk = rng.integers(-127, 128, size=(nb, bs)).astype(np.int8).view(np.uint8)
    else:
        blk = rng.integers(0, 256, size=(nb, bs), dtype=np.uint8)
    for off in D_OFFS[t]:
        d = (rng.uniform(2.0 ** -14, 2.0 ** -6, nb) * rng.choice([-1.0, 1.0], nb)).astype(np.float16)
        blk[:, off:off + 2] = d.view(np.uint8).reshape(nb, 2)
    return np.ascontiguousarray(blk).reshape(-1)


def quant_inputs(rng):
    """Activation vectors that exercise the quantizers: several magnitudes,
    exact zeros, an all-zero block, sign ties of the largest magnitude and
    values on rounding boundaries."""
    parts = []
    for s in (1e-3, 0.02, 1.0, 50.0):
        parts.append((rng.standard_normal(1024) * s).astype(np.float32))
    z = np.zeros(256, np.float32)
    tie = (rng.standard_normal(256) * 0.1).astype(np.float32)
    tie[10], tie[200] = 0.75, -0.75       # |x| tie: first index wins
    bound = np.linspace(-127.5, 127.5, 256).astype(np.float32)   # .5 boundaries
    sparse = np.zeros(256, np.float32)
    sparse[::37] = rng.standard_normal(7).astype(np.float32)
    parts += [z, tie, bound, sparse]
    return np.concatenate(parts)


def main():
    R = load_reference()
    rng = np.random.default_rng(20260101)
    out = {}

    # ---- A1 fp16: all 65536 halves -> float; chosen floats -> half
    h = np.arange(65536, dtype=np.uint16)
    f16 = R.fp16_to_fp32(h)
    edge = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 6.1035156e-05, 6.0975552e-05, 5.9604645e-08,
                     2.9802322e-08, 2.9802326e-08, 1.0009766, 1.0004883, 1.0014648, 0.33333334, -2.5e-06], np.float32)
    rnd = (rng.standard_normal(4096) * np.exp(rng.uniform(-12, 10, 4096))).astype(np.float32)
    rnd = rnd[np.abs(rnd) < 65504]
    f32in = np.concatenate([edge, rnd])
    np.savez_compressed(os.path.join(HERE, "fp16.npz"), h2f=f16, f32_in=f32in, f2h=R.fp32_to_fp16(f32in))

    # ---- A3 dequant: 64 random blocks per format
    dq = {}
    for t in WEIGHT_TYPES:
        qk, bs = BLOCK[t]
        nb = 64
        data = random_blocks(rng, t, nb)
        dq[f"in_{t}"] = data
        dq[f"out_{t}"] = R.dequantize_row(t, data, nb * qk)
    np.savez_compressed(os.path.join(HERE, "dequant.npz"), **dq)

    # ---- A2 quantizers
    x = quant_inputs(rng)
    np.savez_compressed(os.path.join(HERE, "quant.npz"), x=x, q8_0=R.quantize_q8_0(x), q8_K=R.quantize_q8_K(x))

    # ---- A4/A5 matmul: 48 rows x 1024 per format, float activation in,
    # quantized the way inference() does it
    mm = {}
    n, d = 1024, 48
    xa = rng.standard_normal(n).astype(np.float32)
    mm["x"] = xa
    for t in WEIGHT_TYPES + [F16, F32]:
        qk, bs = BLOCK[t]
        if t in (F16, F32):
            w = encode.quantize(t, (rng.standard_normal(d * n) * 0.02).astype(np.float32), d, n)
        else:
            w = random_blocks(rng, t, d * n // qk)
        rsz = n // qk * bs
        mm[f"w_{t}"] = w
        mm[f"y_{t}"] = R.matmul(t, w, rsz, n, d, xa)
    np.savez_compressed(os.path.join(HERE, "matmul.npz"), **mm)

    # ---- A6/A7/A9/softmax
    ops = {}
    xn = rng.standard_normal(4096).astype(np.float32)
    wn = (1.0 + 0.1 * rng.standard_normal(4096)).astype(np.float32)
    ops["rms_x"], ops["rms_w"] = xn, wn
    ops["rms_out"] = R.rmsnorm(xn, wn, 1e-6)
    qh = rng.standard_normal(128).astype(np.float32)
    ops["rmsi_x"], ops["rmsi_w"] = qh, wn[:128]
    ops["rmsi_out"] = R.rmsnorm_inplace(qh, wn[:128], 1e-6)
    sm = (rng.standard_normal(777) * 3).astype(np.float32)
    ops["softmax_x"], ops["softmax_out"] = sm, R.softmax(sm)
    for base, rd, tag in ((1e4, 48, "t"), (1e6, 128, "q"), (5e5, 128, "a")):
        ops[f"freq_{tag}"] = R.rope_freq(base, rd)
    xr = rng.standard_normal(32 * 128).astype(np.float32)
    ops["rope_x"] = xr
    for pos in (0, 1, 517, 32767):
        ops[f"rope_out_{pos}"] = R.rope(xr, 32, 128, 128, pos, ops["freq_q"])
    # attention: 8 query heads, 2 KV heads, hd 128, pos 300
    nh, nkv, hd, pos = 8, 2, 128, 300
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    kc = R.fp32_to_fp16(rng.standard_normal((pos + 1) * nkv * hd).astype(np.float32))
    vc = R.fp32_to_fp16(rng.standard_normal((pos + 1) * nkv * hd).astype(np.float32))
    ops.update(att_q=q, att_k=k, att_v=v, att_kc=kc, att_vc=vc, att_pos=np.int32(pos),
               att_out=R.attention(q, k, v, kc, vc, nh, nkv, hd, pos))
    np.savez_compressed(os.path.join(HERE, "ops.npz"), **ops)

    # ---- A12 tiny model: 16 random prompt ids, then 128 greedy tokens
    hm = HostModel.synthetic(TINY)
    path = os.path.join("/tmp", "ligguf_tiny_golden.gguf")
    hm.write_gguf(path)
    R.model_open(path, 0)
    info = R.model_info()
    assert info["n_embed"] == TINY.n_embed and info["vocab_size"] == TINY.vocab, info
    freq = R.rope_freq_table(TINY.rope_dim)
    prompt = rng.integers(1, TINY.vocab, 16).astype(np.int32)
    toks = []
    keep = {}
    logits = None
    for i, t in enumerate(prompt):
        logits = R.inference(int(t), TINY.vocab)
        if i in (0, 15):
            keep[i] = logits.copy()
    for j in range(128):
        nxt = int(np.argmax(logits))   # sampler_greedy: first max index
        toks.append(nxt)
        if j == 127:
            break
        logits = R.inference(nxt, TINY.vocab)
    keep[16 + 126] = logits.copy()
    wsum = np.array([int(np.sum(hm.weights[nm][3], dtype=np.uint64) % (1 << 61)) for nm in sorted(hm.weights)],
                    np.uint64)
    np.savez_compressed(os.path.join(HERE, "tiny_decode.npz"), prompt=prompt, greedy=np.array(toks, np.int32),
                        logits_step0=keep[0], logits_step15=keep[15], logits_step142=keep[142], rope_freq=freq,
                        weight_sums=wsum)
    os.unlink(path)
    print("golden vectors written to", HERE)


def tiny_teacher():
    """tiny_teacher.npz: for each of the 128 generated steps of the tiny greedy
    run (tiny_decode.npz), the reference's 32 largest logits (ids, values)
    and top-2 gap, and -- the reference and the oracle each fed the same
    tokens from its own KV state -- the oracle's largest absolute logit
    difference from the reference and its argmax: the spread that separates
    two correct engines once an int8 rounding flip has entered their caches."""
    R = load_reference()
    O = load_oracle()
    g = np.load(os.path.join(HERE, "tiny_decode.npz"))
    hm = HostModel.synthetic(TINY)
    hm.rope_freq = g["rope_freq"]
    path = os.path.join("/tmp", "ligguf_tiny_teacher.gguf")
    hm.write_gguf(path)
    R.model_open(path, 0)
    st = O.new_state(hm.fill_desc(OrModel, OrLayer, OrWeight))
    toks = np.concatenate([g["prompt"], g["greedy"]])
    ids, vals, gap, diff, otok = [], [], [], [], []
    for pos in range(len(toks) - 1):
        a = R.inference(int(toks[pos]), TINY.vocab)
        b = O.inference(st, int(toks[pos]), TINY.vocab)
        if pos >= len(g["prompt"]) - 1:
            top = np.argsort(-a, kind="stable")[:32]
            assert int(top[0]) == int(g["greedy"][pos - len(g["prompt"]) + 1])
            ids.append(top.astype(np.int32))
            vals.append(a[top])
            gap.append(a[top[0]] - a[top[1]])
            diff.append(float(np.max(np.abs(a - b))))
            otok.append(int(np.argmax(b)))
    O.free_state(st)
    os.unlink(path)
    np.savez_compressed(os.path.join(HERE, "tiny_teacher.npz"), top_ids=np.array(ids), top_vals=np.array(vals),
                        gap=np.array(gap, np.float32), oracle_maxdiff=np.array(diff, np.float32),
                        oracle_tok=np.array(otok, np.int32))
    print("tiny_teacher.npz written to", HERE)


BERT_TEXTS = [b"Hello world, the cat sat on the mat!", b"What is the WEATHER like in Paris on Monday?",
              b"", b"xyzzy quux", b"caf\xc3\xa9 \xe2\x82\xac42 coffee", b"(a)[b]{c}", b"python code " * 40]
BERT_LOG = (b"@@1700000000\n<<<<<<<\nthe cat sat on the mat\n>>>>>>>\nnice cat\n"
            b"@@1700000100\n<<<<<<<\nwhat is the weather in paris\n>>>>>>>\nsunny and warm\n"
            b"@@1700000200\n<<<<<<<\nI like pizza for dinner\nand coffee\n>>>>>>>\nme too\n"
            b"@@1700000300\n<<<<<<<\nthe cat sat on the mat\n>>>>>>>\nagain?\n"
            b"@@1700000400\n<<<<<<<\npython code search\n>>>>>>>\nok")
BERT_QUERIES = [b"the cat sat on the mat", b"weather in paris", b"pizza dinner coffee", b"river mountain tree"]
BERT_TYPES = [(F32, F16), (F16, F16), (Q8_0, Q8_0), (Q1_G, F32)]


def bert_golden():
    """bert.npz: the reference's bert_tokenize ids and bert_embed vectors
    (fast/vdb.cpp:75-245) for BERT_TEXTS on the tiny synthetic encoder in four
    weight types, and for its vector memory (vdb_create over BERT_LOG, then
    vdb_query) the entries' timestamps and fp16 vectors and the indices found
    for each of BERT_QUERIES."""
    from ligguf_amd.bert import BERT_TINY, HostBert
    R = load_reference()
    out = {}
    for lt, et in BERT_TYPES:
        hb = HostBert.synthetic(BERT_TINY.with_(layer_type=lt, embd_type=et))
        path = os.path.join("/tmp", f"ligguf_bert_{lt}.gguf")
        hb.write_gguf(path)
        R.bert_open(path)
        key = f"t{lt}_{et}"
        out[key + "_wsum"] = np.array([int(np.sum(hb.weights[nm][3], dtype=np.uint64) % (1 << 61))
                                       for nm in sorted(hb.weights)], np.uint64)
        for i, t in enumerate(BERT_TEXTS):
            out[f"{key}_tok{i}"] = np.array(R.bert_tokenize(t), np.int32)
            out[f"{key}_emb{i}"] = R.bert_embed(t)
        n = R.vdb_create(BERT_LOG)
        ents = [R.vdb_entry(i) for i in range(n)]
        out[key + "_vdb_ts"] = np.array([e[0] for e in ents], np.uint32)
        out[key + "_vdb_vec"] = np.stack([e[1] for e in ents])
        for i, q in enumerate(BERT_QUERIES):
            out[f"{key}_q{i}_emb"] = R.bert_embed(q)
            out[f"{key}_q{i}_idx"] = np.array(R.vdb_query(q), np.int32)
        os.unlink(path)
    np.savez_compressed(os.path.join(HERE, "bert.npz"), **out)
    print("bert.npz written to", HERE)


if __name__ == "__main__":
    if "--teacher-only" in sys.argv:
        tiny_teacher()
    elif "--bert-only" in sys.argv:
        bert_golden()
    else:
        main()
        tiny_teacher()
        bert_golden()
