"""BERT embedding and vector-memory search on the GPU (lg_bert_*, the
bert_embed / vdb_query path of fast/vdb.cpp:123-245,337-377) against the
reference's own outputs (tests/golden/bert.npz), the oracle (or_bert_embed,
or_vdb_search) and, where oracle/_ref is present, the live reference.

Bars.  F32/F16 matrices: relative L2 of the embedding <= 2e-5 (fp32
products, only summation orders differ; measured ~1e-7 .. 1e-6).  Q8_0/Q1
matrices quantize their activations (quantize_q8_0), and an activation within
fp32 noise of a rounding boundary can take the other int8 value on either
side; so these passes run with lg_bert_trace_next and are checked as the
decode step is (tests/parity.py): where every int8 equals the oracle's the
embedding must match to 2e-5, and the first point where some differ must
differ only by one-step flips of values within FLIP_TOL of k + 1/2 (then the
embedding within 1e-2).  Against the reference's vectors (no trace) the Q8
bar is 1e-2.  Searches must return the oracle's rows exactly, except where
two similarities lie within 1e-6 of each other or of the threshold."""
import os
import tempfile
import zlib

import numpy as np
import pytest

from conftest import golden
from parity import FLIP_TOL, MAX_FLIP_FRAC, boundary_dist, quantize_ref
from ligguf_amd import encode
from ligguf_amd.bert import BERT_TINY, MINILM_L6, Bert, HostBert, parse_chat_log
from ligguf_amd.lib import F16, F32, Q1_0, Q1_G, Q4_K, Q8_0, LgError

pytestmark = pytest.mark.gpu

BERT_TEXTS = [b"Hello world, the cat sat on the mat!", b"What is the WEATHER like in Paris on Monday?",
              b"", b"xyzzy quux", b"caf\xc3\xa9 \xe2\x82\xac42 coffee", b"(a)[b]{c}", b"python code " * 40]
BERT_LOG = (b"@@1700000000\n<<<<<<<\nthe cat sat on the mat\n>>>>>>>\nnice cat\n"
            b"@@1700000100\n<<<<<<<\nwhat is the weather in paris\n>>>>>>>\nsunny and warm\n"
            b"@@1700000200\n<<<<<<<\nI like pizza for dinner\nand coffee\n>>>>>>>\nme too\n"
            b"@@1700000300\n<<<<<<<\nthe cat sat on the mat\n>>>>>>>\nagain?\n"
            b"@@1700000400\n<<<<<<<\npython code search\n>>>>>>>\nok")
BERT_QUERIES = [b"the cat sat on the mat", b"weather in paris", b"pizza dinner coffee", b"river mountain tree"]
BERT_TYPES = [(F32, F16), (F16, F16), (Q8_0, Q8_0), (Q1_G, F32)]
SIM_TOL = 1e-6
EXACT = 2e-5          # no int8 difference from the oracle
FLIP_REL = 1e-2       # after a rounding flip
Q8_CLASS = (Q8_0, Q1_0, Q1_G)


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(np.asarray(b, np.float64)))


def bar(lt):
    return EXACT if lt in (F32, F16) else FLIP_REL


def q8_points(hb):
    """(layer, point) pairs whose activation a Q8_0/Q1 matrix consumes"""
    out = []
    for l in range(hb.cfg.n_layers):
        b = f"blk.{l}."
        mats = [["attn_q", "attn_k", "attn_v"], ["attn_output"], ["ffn_up"], ["ffn_down"]]
        for s, names in enumerate(mats):
            if any(hb.weights[b + n + ".weight"][0] in Q8_CLASS for n in names):
                out.append((l, s))
    return out


def check_embed(dev, oracle, hb, toks, label=""):
    """The GPU embedding of toks against the oracle's, flip-explained when the
    encoder has Q8_0/Q1 matrices; returns the GPU vector."""
    pts = q8_points(hb)
    if not pts:
        e = dev.embed(toks)
        r = rel(e, oracle.bert_embed(hb, toks))
        print(f"  {label} {len(toks)} tokens: {r:.2e}")
        assert r < EXACT, (label, r)
        return e
    e, gtr = dev.embed_traced(toks)
    oe, otr = oracle.bert_embed_traced(hb, toks)
    r = rel(e, oe)
    T = otr.shape[2]
    for (l, s) in pts:
        K = hb.cfg.n_ff if s == 3 else hb.cfg.n_embed
        qg, dg = gtr[(l, s)]
        xo = otr[l, s, :, :K].reshape(-1)
        qo, v = quantize_ref(xo, Q8_0)
        # block scales: fp16(amax / 127) as the quantizer stores them; one
        # fp16 step apart where amax / 127 sits on an fp16 rounding boundary
        do = (np.abs(xo.reshape(-1, 32)).max(axis=1) * np.float32(1.0 / 127.0)).astype(np.float16)
        dgh = dg.T.reshape(-1).astype(np.float16)
        dd = np.nonzero(dgh != do)[0]
        if dd.size:
            ulps = np.abs(dgh[dd].view(np.int16).astype(np.int32) - do[dd].view(np.int16).astype(np.int32))
            print(f"  {label}: {dd.size} block scales one fp16 step apart at layer {l} point {s}")
            assert np.all(ulps == 1) and dd.size <= max(4, int(MAX_FLIP_FRAC * T * K / 32)), (label, l, s, dd[:5])
        diff = np.nonzero(qg.reshape(-1) != qo)[0]
        if diff.size == 0:
            if dd.size:
                assert r < FLIP_REL, (label, r)
                return e
            continue
        steps = np.abs(qg.reshape(-1)[diff].astype(np.int32) - qo[diff].astype(np.int32))
        dist = boundary_dist(v[diff])
        print(f"  {label} {len(toks)} tokens: {diff.size} int8 flips first at layer {l} point {s} "
              f"(max boundary distance {dist.max():.3f}), rel-L2 {r:.2e}")
        assert diff.size <= max(8, int(MAX_FLIP_FRAC * T * K)), (label, l, s, diff.size)
        assert np.all(steps == 1) and np.all(dist <= FLIP_TOL), (label, l, s, list(zip(diff[:5], dist[:5])))
        assert r < FLIP_REL, (label, r)
        return e
    print(f"  {label} {len(toks)} tokens: no int8 differences, rel-L2 {r:.2e}")
    assert r < EXACT, (label, r)
    return e


@pytest.fixture(scope="module")
def dev(gpu):
    b = Bert(0)
    yield b
    b.close()


def load(dev, hb, max_tokens=0):
    print(f"bert load {hb.cfg.name} layers={hb.cfg.n_layers} ne={hb.cfg.n_embed} type={hb.cfg.layer_type}", flush=True)
    dev.load(hb, max_tokens)
    return hb


@pytest.mark.parametrize("lt,et", BERT_TYPES)
def test_bert_embed_golden(dev, oracle, lt, et):
    """the reference's bert_embed vectors (golden) and the oracle's"""
    hb = load(dev, HostBert.synthetic(BERT_TINY.with_(layer_type=lt, embd_type=et)))
    g = golden("bert.npz")
    key = f"t{lt}_{et}"
    for i in range(len(BERT_TEXTS)):
        toks = g[f"{key}_tok{i}"]
        e = check_embed(dev, oracle, hb, toks, f"text {i}")
        r_ref = rel(e, g[f"{key}_emb{i}"])
        print(f"    vs the reference's vector {r_ref:.2e}")
        assert r_ref < bar(lt), (i, r_ref)


@pytest.mark.parametrize("lt,et", [(Q1_0, Q8_0), (F16, Q1_0), (F32, F32)])
def test_bert_embed_oracle_more_types(dev, oracle, lt, et):
    hb = load(dev, HostBert.synthetic(BERT_TINY.with_(layer_type=lt, embd_type=et, seed=99)))
    rng = np.random.default_rng(lt * 7 + et)
    for n in (0, 1, 17, 126):
        check_embed(dev, oracle, hb, rng.integers(5, hb.cfg.vocab, n))


def test_bert_mixed_matrix_types(dev, oracle):
    """q, k, v of three forms (three GEMMs instead of one stacked), Q8_0
    att_out and F32 FFN down -- matmul3 / matmul take any mix
    (fast/lil_math.cpp:748-899)"""
    hb = HostBert.synthetic(BERT_TINY)
    c = hb.cfg
    for name, t in (("blk.0.attn_k.weight", Q8_0), ("blk.0.attn_v.weight", F32), ("blk.1.attn_output.weight", Q8_0),
                    ("blk.1.ffn_down.weight", F32), ("blk.1.attn_q.weight", Q1_0)):
        _, rows, cols, _ = hb.weights[name]
        hb.weights[name] = (t, rows, cols, encode.random_tensor(t, c.seed, zlib.crc32(name.encode()) + 1, rows, cols,
                                                                c.sigma))
    load(dev, hb)
    rng = np.random.default_rng(8)
    for n in (5, 100):
        check_embed(dev, oracle, hb, rng.integers(5, c.vocab, n), "mixed")


def test_bert_batch_equals_single_and_truncation(dev):
    """a batch gives each sequence exactly its single-sequence vector (per-token
    arithmetic, per-sequence attention and pooling); tokens past
    n_context - 2 are dropped (fast/vdb.cpp:135)"""
    hb = load(dev, HostBert.synthetic(BERT_TINY.with_(layer_type=Q8_0, embd_type=F16)))
    rng = np.random.default_rng(9)
    seqs = [rng.integers(5, hb.cfg.vocab, n) for n in (0, 3, 126, 127, 300, 1, 64)]
    single = np.stack([dev.embed(s) for s in seqs])
    batch = dev.embed_batch(seqs)
    assert np.array_equal(batch.view(np.uint32), single.view(np.uint32))
    nmax = hb.cfg.n_context - 2
    assert np.array_equal(single[3], dev.embed(seqs[3][:nmax]))
    assert np.array_equal(single[4], dev.embed(seqs[4][:nmax]))


def test_bert_batch_spans_several_passes(dev):
    """more tokens than one pass holds: the batch is cut at sequence
    boundaries into passes of at most max_tokens"""
    hb = load(dev, HostBert.synthetic(BERT_TINY), max_tokens=256)
    rng = np.random.default_rng(10)
    seqs = [rng.integers(5, hb.cfg.vocab, int(n)) for n in rng.integers(0, 140, 25)]
    single = np.stack([dev.embed(s) for s in seqs])
    assert np.array_equal(dev.embed_batch(seqs).view(np.uint32), single.view(np.uint32))


def test_bert_minilm_shape(dev, oracle):
    """all-MiniLM-L6-v2 shape (6 blocks, 384 wide, 12 heads of 32, FFN 1536,
    30522 pieces), F16 matrices, a 510-token sequence and a short one"""
    hb = load(dev, HostBert.synthetic(MINILM_L6))
    rng = np.random.default_rng(11)
    for n in (510, 12):
        check_embed(dev, oracle, hb, rng.integers(5, hb.cfg.vocab, n), "MiniLM shape")


def test_bert_long_sequences(dev, oracle):
    """the attention variants by sequence length: up to 512 and up to 1024
    positions on MFMA with the score rows in LDS, longer ones on the
    vector-ALU kernel with fewer queries per block; a batch mixing them"""
    hb = load(dev, HostBert.synthetic(BERT_TINY.with_(n_context=2048, seed=21)))
    rng = np.random.default_rng(12)
    seqs = [rng.integers(5, hb.cfg.vocab, n) for n in (300, 700, 1500, 2046)]
    single = [check_embed(dev, oracle, hb, s, "long") for s in seqs]
    batch = dev.embed_batch(seqs)
    for i in range(len(seqs)):
        assert rel(batch[i], single[i]) < EXACT


def test_bert_live_reference(dev, reference):
    """text in, vector out: the reference's bert_tokenize + bert_embed on its
    own GGUF load against the GPU fed the same ids"""
    for lt, et in ((F16, F16), (Q8_0, F32)):
        hb = HostBert.synthetic(BERT_TINY.with_(layer_type=lt, embd_type=et, seed=5))
        with tempfile.TemporaryDirectory() as d:
            fn = os.path.join(d, "b.gguf")
            hb.write_gguf(fn)
            reference.bert_open(fn)
            hg = load(dev, HostBert.from_gguf(fn))
            for text in (b"The quick brown fox, jumps!", b"memory " * 90):
                toks = reference.bert_tokenize(text)
                assert toks == hg.tokenize(text)
                r = rel(dev.embed(toks), reference.bert_embed(text))
                print(f"  type {lt}: {r:.2e}")
                assert r < bar(lt)
            del hg


def check_search(got_idx, got_sim, want_idx, sims, thr):
    """got equals want, or differs only among rows whose similarities tie
    within SIM_TOL (or sit within SIM_TOL of the threshold)"""
    if list(got_idx) == list(want_idx):
        return
    near = lambda i: abs(sims[i] - thr) <= SIM_TOL
    assert len(got_idx) == len(want_idx) or any(near(i) for i in set(got_idx) ^ set(want_idx))
    for a, b in zip(got_idx, want_idx):
        assert a == b or abs(sims[a] - sims[b]) <= SIM_TOL or near(a) or near(b), (got_idx, want_idx)
    assert np.allclose(got_sim, sims[got_idx], atol=SIM_TOL)


@pytest.mark.parametrize("n,dim", [(1, 128), (5000, 128), (70000, 384)])
def test_vdb_query_vs_oracle(dev, oracle, n, dim):
    hb = load(dev, HostBert.synthetic(BERT_TINY.with_(n_embed=dim, n_heads=dim // 32, n_layers=1)))
    rng = np.random.default_rng(n)
    v = rng.normal(0, 1, (n, dim))
    v /= np.linalg.norm(v, axis=1, keepdims=True)
    emb = rng.normal(0, 1, dim)
    emb /= np.linalg.norm(emb)
    v[n // 2] = 0.9 * emb + 0.1 * v[n // 2]               # a near match
    if n > 10:
        v[n - 1] = v[n // 2]                              # and its exact twin (the lower row first)
        v[3] = np.nan                                     # a NaN row never qualifies
    vh = v.astype(np.float16)
    emb = emb.astype(np.float32)
    dev.vdb_set(vh.view(np.uint16))
    assert dev.vdb_size() == n
    sims = (np.nan_to_num(vh.astype(np.float64), nan=0.0) @ emb).astype(np.float32)
    for thr, k in ((0.75, 3), (-2.0, 8), (0.05, 5), (2.0, 3), (-2.0, 1)):
        idx, sim = dev.vdb_query(emb, thr, k)
        want_idx, _ = oracle.vdb_search(vh.view(np.uint16), emb, thr, k)
        check_search(idx, sim, want_idx, sims, thr)
        assert 3 not in idx or n <= 10


def test_vdb_append_and_golden_memory(dev, oracle):
    """the golden vector memory in pieces (append grows the device table past
    its first capacity), the golden query vectors find the reference's
    entries; then end to end: the log parsed on the host, every user turn
    embedded on the GPU in one batch, stored as fp16 (the reference's
    f32_to_f16_row, fast/vdb.cpp:258), queried from tokens"""
    g = golden("bert.npz")
    for lt, et in BERT_TYPES:
        key = f"t{lt}_{et}"
        hb = load(dev, HostBert.synthetic(BERT_TINY.with_(layer_type=lt, embd_type=et)))
        vecs = g[key + "_vdb_vec"]
        filler = np.full((1500, hb.cfg.n_embed), 0, np.uint16)   # zero rows: similarity 0, below 0.75
        dev.vdb_set(vecs[:2])
        dev.vdb_append(filler)
        dev.vdb_append(vecs[2:])
        order = np.r_[0, 1, np.arange(1502, 1502 + len(vecs) - 2)]
        for i in range(len(BERT_QUERIES)):
            idx, _ = dev.vdb_query(g[f"{key}_q{i}_emb"])
            assert [int(np.nonzero(order == j)[0][0]) for j in idx] == g[f"{key}_q{i}_idx"].tolist()
        ents = parse_chat_log(BERT_LOG.decode())
        embs = dev.embed_batch([hb.tokenize(e.user_text) for e in ents])
        dev.vdb_set(np.stack([oracle.fp32_to_fp16(e) for e in embs]))
        for i, q in enumerate(BERT_QUERIES):
            check_embed(dev, oracle, hb, hb.tokenize(q), f"{key} query {i}")
            idx, sim, emb = dev.query(hb.tokenize(q))
            assert rel(emb, g[f"{key}_q{i}_emb"]) < bar(lt)
            print(f"  {key} query {i}: {idx.tolist()} {np.round(sim, 4).tolist()}")
            assert idx.tolist() == g[f"{key}_q{i}_idx"].tolist()


def test_bert_errors(dev):
    hb = HostBert.synthetic(BERT_TINY)
    bad = HostBert.synthetic(BERT_TINY)
    _, rows, cols, _ = bad.weights["blk.0.ffn_down.weight"]       # 512 columns: two Q4_K blocks a row
    bad.weights["blk.0.ffn_down.weight"] = (Q4_K, rows, cols, encode.random_tensor(Q4_K, 1, 2, rows, cols, 0.02))
    with pytest.raises(LgError, match="LG_ERR_TYPE"):
        dev.load(bad)
    with pytest.raises(LgError, match="LG_ERR_STATE"):
        dev.embed([5, 6])
    load(dev, hb)
    with pytest.raises(LgError, match="LG_ERR_ARG"):
        dev.embed([5, hb.cfg.vocab])
    with pytest.raises(LgError, match="LG_ERR_ARG"):
        dev.vdb_query(np.zeros(hb.cfg.n_embed + 32, np.float32))
    dev.vdb_set(np.zeros((4, hb.cfg.n_embed), np.uint16))
    with pytest.raises(LgError, match="LG_ERR_ARG"):
        dev.vdb_query(np.zeros(hb.cfg.n_embed, np.float32), 0.5, 9)
    assert dev.embed([5, 6]).shape == (hb.cfg.n_embed,)   # the handle still works
