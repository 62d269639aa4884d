#!/usr/bin/env python3
"""Batch-1 decode throughput of a Qwen3-8B-shaped Q4_K model on one MI355X.

Workload (one "step" = one greedy decode token, batch 1):
  Qwen3-8B shape -- 36 layers, dim 4096, 32 query / 8 KV heads of 128,
  per-head QK RMSNorm, SwiGLU FFN 12288, vocab 151936, RoPE theta 1e6 --
  with synthetic N(0, 0.02) weights encoded to Q4_K (attention, FFN,
  embedding) and Q6_K (output head), norms 1.0.  A 512-token random-id
  prompt is prefilled first, then W warm-up and K timed greedy tokens run
  through lg_decode_greedy: the reference's inference() + sampler_greedy
  loop (fast/ligguf_fast_qk.cpp:368-382) with each step's greedy token fed
  to the next on the device, the steps queued back to back.  The same K
  steps with the token read back to the host every step (lg_decode_step_async
  + lg_argmax) are reported beside it.

Prints one JSON line.  `value` is decode tokens/s with weights and KV
resident in HBM.  `roofline` is for the dominant kernel of the step, the
fused rmsnorm + up|gate (2 x 12288 x 4096 Q4_K) + SwiGLU kernel, launched
on its own through lg_time_fused_phase over all 36 layers in turn (2 GB of
distinct weights, far above the 256 MB Infinity Cache) and timed with HIP
events on the stream it runs on; `cpu_baseline` is the reference FAST engine
(built from its own sources, AVX2) decoding the same model on this host's
cores at the GPU's positions, from the state the GPU saved after its
prefill.  `hbm_practical` holds two measured bounds: a read-only pass over
2 GiB (lg_hbm_read_probe) and a device copy.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# the CPU baseline's OpenMP threads stay on their cores (set before any
# OpenMP runtime starts in this process)
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")
USABLE_CPUS = len(os.sched_getaffinity(0))      # before any OpenMP runtime pins this thread

HBM_PEAK = 8.0e12          # MI355X HBM3E, bytes/s


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


UG_KERNEL = "k_f_ug Q4_K (x + att_out group partials, rmsnorm + up|gate 24576x4096 + SwiGLU)"


def dominant_kernel_roofline(eng, cfg, passes: int = 5):
    """Mean duration of the fused up|gate kernel over `passes` sweeps of all
    layers (lg_time_fused_phase: HIP events on the engine's stream), against
    its algorithmic bytes: the two Q4_K matrices; the fp32 residual input, the
    8 att_out partials of the KV groups (summed into xm by its build) and the
    rmsnorm weights it reads; the fp32 SwiGLU output and xm it writes."""
    from ligguf_amd.lib import Q4_K, row_size
    iters = passes * cfg.n_layers
    eng.time_phase(3, 0, cfg.n_layers)             # warm-up sweep
    avg_us = eng.time_phase(3, 0, iters)
    alg = (2 * cfg.n_ff * row_size(Q4_K, cfg.n_embed) + (1 + 8 + 1) * cfg.n_embed * 4 + cfg.n_ff * 4 +
           cfg.n_embed * 4)
    avg_s = avg_us * 1e-6
    return {"bound": "hbm", "achieved": round(alg / avg_s / 1e9, 1), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": round(alg / avg_s / HBM_PEAK, 4), "traffic": measured_traffic(UG_KERNEL),
            "kernel": UG_KERNEL, "avg_us": round(avg_us, 3), "bytes_per_launch": alg, "launches": iters}


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE and WRITE_SIZE runs, each scaled by the same counter's
    reading for a copy of known size), or None when no summary covers it."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f).get(kernel)
    except (OSError, ValueError):
        return None
    return int(rec["traffic_bytes"]) if rec else None


def plain_copy(torch, nbytes: int = 256 << 20, reps: int = 20):
    """A plain device copy of a known size (read nbytes, write nbytes): the
    calibration kernel for the FETCH_SIZE / WRITE_SIZE counters."""
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        dst.copy_(src)
    e1.record(s)
    torch.cuda.synchronize()
    avg_s = e0.elapsed_time(e1) / 1e3 / reps
    del src, dst
    torch.cuda.empty_cache()
    return {"bytes_each_way": nbytes, "avg_us": round(avg_s * 1e6, 2), "GB/s": round(2 * nbytes / avg_s / 1e9, 1)}


def plain_read(torch, nbytes: int = 2 << 30, iters: int = 10):
    """lg_hbm_read_probe over a buffer of nbytes (8x the 256 MiB last-level
    cache): the practical read-only HBM rate, the bound a decode step that
    only reads weights and cache rows can reach."""
    import ctypes as C
    from ligguf_amd import lib as L
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    torch.cuda.synchronize()
    us = C.c_float()
    L.check(L.load().lg_hbm_read_probe(C.c_void_p(buf.data_ptr()), nbytes, iters, C.byref(us),
                                       C.c_void_p(torch.cuda.current_stream().cuda_stream)))
    del buf
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "avg_us": round(us.value, 2), "GB/s": round(nbytes / (us.value * 1e-6) / 1e9, 1)}


MFMA_INT8_PEAK = 5.0e15    # MI355X dense int8, ops/s


def prefill_report(cfg, tokens: int, seconds: float, path: int):
    """Prefill throughput against two bounds: the HBM roofline of one pass
    (every layer matrix read once per pass of <= 512 tokens) and the int8
    MFMA peak for the pass's GEMM work (2 ops per weight x token)."""
    from ligguf_amd.lib import PREFILL_BATCHED, row_size
    passes = (tokens + 511) // 512
    head = cfg.vocab * row_size(cfg.out_type, cfg.n_embed)      # the output head, once (last token)
    hbm = passes * (cfg.weight_bytes() - head) + head
    macs = cfg.n_layers * (cfg.n_embed + 2 * cfg.kv_dim + cfg.n_embed + 2 * cfg.n_ff + cfg.n_ff) * cfg.n_embed
    ops = 2.0 * macs * tokens
    return {"tok_s": round(tokens / seconds, 1), "tokens": tokens, "ms": round(seconds * 1e3, 2),
            "path": "batched" if path == PREFILL_BATCHED else "steps",
            "hbm_roofline_frac": round(hbm / seconds / HBM_PEAK, 4),
            "gemm_int8_tops": round(ops / seconds / 1e12, 1),
            "mfma_frac": round(ops / seconds / MFMA_INT8_PEAK, 4)}


_SLEEP_CYCLES_PER_MS = None


def _time_launches(torch, fn, reps: int) -> float:
    """Mean GPU time of fn() over reps back-to-back launches, microseconds:
    HIP events on the current stream around the launches, which are queued
    behind a GPU spin (torch.cuda._sleep) long enough for the host to
    enqueue them all -- so the time is the kernels' and their launch gaps',
    not the host's per-call overhead."""
    global _SLEEP_CYCLES_PER_MS
    fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if _SLEEP_CYCLES_PER_MS is None:
        e0.record()
        torch.cuda._sleep(1 << 24)
        e1.record()
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = (1 << 24) / max(e0.elapsed_time(e1), 1e-3)
    t0 = time.perf_counter()
    for _ in range(min(reps, 20)):
        fn()
    torch.cuda.synchronize()
    host_ms = (time.perf_counter() - t0) / min(reps, 20) * 1e3
    torch.cuda._sleep(int(_SLEEP_CYCLES_PER_MS * (2.0 * host_ms * reps + 2.0)))
    e0.record()
    for _ in range(reps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


ROTATE_BYTES = 512 << 20    # distinct buffers cycled per isolated kernel: twice the 256 MB Infinity Cache


def isolated_kernels(torch, np):
    """The isolated-kernel workloads: batch-1 quantized matvec (k_matvec)
    for Q4_K 4096x4096, Q4_K 14336x4096 and Q6_K 128256x4096 (weights N(0,
    0.02) through the reference quantizers, activation N(0,1) as Q8_K); and
    GQA decode attention (lg_attn_decode: 32 query / 8 KV heads of 128, fp16
    cache, the reference's KV format) at 512, 4096 and 32768 positions.  Each
    launch takes the next of enough distinct weight copies / KV caches to
    cover at least 512 MiB, so no launch finds its bytes in the 256 MB
    Infinity Cache.  Rates are algorithmic bytes (weights + activation +
    output; K and V rows read) per launch over the launch time."""
    from ligguf_amd import ops
    from ligguf_amd.encode import random_tensor
    from ligguf_amd.lib import Q4_K, Q6_K, row_size
    dev = "cuda:0"
    out = {"matvec": [], "attention": []}
    for t, name, rows, cols in ((Q4_K, "Q4_K", 4096, 4096), (Q4_K, "Q4_K", 14336, 4096), (Q6_K, "Q6_K", 128256, 4096)):
        rsz = row_size(t, cols)
        mbytes = rows * rsz
        copies = max(2, -(-ROTATE_BYTES // mbytes))
        w0 = torch.from_numpy(random_tensor(t, 7, 0, rows, cols)).to(dev)
        ws = [w0] + [w0.clone() for _ in range(copies - 1)]
        x = torch.from_numpy(np.random.default_rng(3).standard_normal(cols).astype(np.float32)).to(dev)
        xq = ops.quantize_q8_K(x)
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        k = [0]

        def mv():
            ops.matvec(t, ws[k[0] % copies], rsz, cols, rows, xq, y)
            k[0] += 1
        us = _time_launches(torch, mv, 10 * copies)
        alg = mbytes + xq.numel() + 4 * rows
        out["matvec"].append({"type": name, "shape": [rows, cols], "us": round(us, 2),
                              "GB/s": round(alg / us / 1e3, 1), "frac": round(alg / (us * 1e-6) / HBM_PEAK, 4),
                              "copies": copies})
        del ws, w0
    torch.cuda.empty_cache()
    nh, nkv, hd = 32, 8, 128
    rng = np.random.default_rng(5)
    for ctx in (512, 4096, 32768):
        kvd = nkv * hd
        cache_bytes = 2 * ctx * kvd * 2
        ncache = max(2, -(-ROTATE_BYTES // cache_bytes))
        base = torch.from_numpy(rng.standard_normal(2 * ctx * kvd).astype(np.float16).view(np.uint16)).to(dev)
        caches = [base] + [base.clone() for _ in range(ncache - 1)]
        q = torch.from_numpy(rng.standard_normal(nh * hd).astype(np.float32)).to(dev)
        kk = torch.from_numpy(rng.standard_normal(kvd).astype(np.float32)).to(dev)
        vv = torch.from_numpy(rng.standard_normal(kvd).astype(np.float32)).to(dev)
        pos = ctx - 1
        wsz = max(16, ops.load().lg_attn_workspace_size(nh, hd, pos))
        ws = torch.empty(wsz, dtype=torch.uint8, device=dev)
        k = [0]

        def att():
            c = caches[k[0] % ncache]
            ops.attention(q, kk, vv, c[:ctx * kvd], c[ctx * kvd:], nh, nkv, hd, pos, ws)
            k[0] += 1
        us = _time_launches(torch, att, max(50, 4 * ncache))
        alg = pos * kvd * 2 * 2 + (nh * hd + 2 * kvd) * 4 + nh * hd * 4
        out["attention"].append({"ctx": ctx, "us": round(us, 2), "GB/s": round(alg / us / 1e3, 1),
                                 "frac": round(alg / (us * 1e-6) / HBM_PEAK, 4), "caches": ncache})
        del caches, base
    torch.cuda.empty_cache()
    log(f"isolated: {out}")
    return out


FP32_MFMA_PEAK = 157.3e12   # MI355X dense fp32 matrix, flop/s


def bert_report(torch, np, cpu_seconds: float = 0.0):
    """BERT sentence embedding and vector-memory search (lg_bert_*, the
    bert_embed / vdb_query path of fast/vdb.cpp:123-245,337-377) on the
    all-MiniLM-L6-v2 shape (6 blocks, 384 wide, 12 heads of 32, FFN 1536, 512
    positions, 30522 pieces), synthetic F16 matrices:
      - one 510-piece text (512 positions with CLS/SEP), embeddings/s of
        synchronous lg_bert_embed calls (host tables, upload of the ids and
        download of the vector included);
      - 64 texts of 126 pieces in lg_bert_embed_batch calls (a chat log's
        turns, as vdb_create embeds them);
      - a 2^20-row fp16 memory of 384-wide vectors: lg_bert_vdb_query (top 3
        at threshold 0, so every row is a candidate) per synchronous call.
    TFLOP/s count the layer matrices and attention products (BertConfig.flops)
    against the 157.3 TFLOP/s dense fp32 MFMA peak the F16 x fp32 products run
    on; the search counts the rows' bytes against 8 TB/s.  cpu_baseline: the
    reference's bert_embed (oracle/_ref, OpenMP over matrix rows) on a
    510-word text of the same encoder, a bounded number of calls."""
    from ligguf_amd.bert import MINILM_L6, Bert, HostBert
    cfg = MINILM_L6
    hb = HostBert.synthetic(cfg)
    b = Bert(0)
    b.load(hb)
    rng = np.random.default_rng(0)
    out = {"workload": "minilm-l6-shape F16 (6x384, 12 heads of 32, FFN 1536, vocab 30522)"}
    toks = rng.integers(5, cfg.vocab, 510)
    for _ in range(3):
        b.embed(toks)
    reps = 30
    t0 = time.perf_counter()
    for _ in range(reps):
        b.embed(toks)
    dt = (time.perf_counter() - t0) / reps
    fl = cfg.flops(512)
    out["single_512"] = {"ms": round(dt * 1e3, 3), "emb_per_s": round(1 / dt, 1), "TFLOP/s": round(fl / dt / 1e12, 2),
                         "frac_fp32_mfma": round(fl / dt / FP32_MFMA_PEAK, 4)}
    seqs = [rng.integers(5, cfg.vocab, 126) for _ in range(64)]
    b.embed_batch(seqs)
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        b.embed_batch(seqs)
    dt = (time.perf_counter() - t0) / reps
    fl = 64 * cfg.flops(128)
    out["batch_64x128"] = {"ms": round(dt * 1e3, 3), "emb_per_s": round(64 / dt, 1), "tok_per_s": round(64 * 128 / dt),
                           "TFLOP/s": round(fl / dt / 1e12, 2), "frac_fp32_mfma": round(fl / dt / FP32_MFMA_PEAK, 4)}
    n, dim = 1 << 20, cfg.n_embed
    vecs = (rng.standard_normal((n, dim), dtype=np.float32) / np.float32(dim ** 0.5)).astype(np.float16)
    b.vdb_set(vecs.view(np.uint16))
    del vecs
    emb = rng.standard_normal(dim).astype(np.float32)
    emb /= np.linalg.norm(emb)
    for _ in range(3):
        b.vdb_query(emb, 0.0, 3)
    reps = 30
    t0 = time.perf_counter()
    for _ in range(reps):
        b.vdb_query(emb, 0.0, 3)
    dt = (time.perf_counter() - t0) / reps
    out["vdb_search"] = {"rows": n, "dim": dim, "us": round(dt * 1e6, 1), "GB/s": round(n * dim * 2 / dt / 1e9, 1),
                         "frac": round(n * dim * 2 / dt / HBM_PEAK, 4)}
    b.close()
    if cpu_seconds > 0:
        from oracle import load_reference, reference_available
        if reference_available():
            import tempfile
            R = load_reference()
            words = [w for w in hb.tokens if w.isalpha() and w.islower() and len(w) > 1]
            text = " ".join(rng.choice(words, 510)).encode()
            assert len(hb.tokenize(text)) == 510
            with tempfile.TemporaryDirectory() as d:
                fn = os.path.join(d, "bert.gguf")
                hb.write_gguf(fn)
                with _stdout_to_stderr():
                    R.bert_open(fn)
                    R.bert_embed(text)
                    calls, t0 = 0, time.perf_counter()
                    while time.perf_counter() - t0 < cpu_seconds and calls < 200:
                        R.bert_embed(text)
                        calls += 1
                    dt = (time.perf_counter() - t0) / calls
            info = cpu_info()
            out["cpu_baseline"] = {"value": round(1 / dt, 2), "unit": "embeddings/s (512 positions)",
                                   "ms": round(dt * 1e3, 2), "cores": info.get("omp_threads"), "kind": "reference",
                                   "sample": f"{calls} bert_embed calls of a 510-word text"}
    log(f"bert: {out}")
    return out


def q1g_context(torch, np, ctx: int = 8192, steps: int = 128, warmup: int = 8, cpu_seconds: float = 0.0):
    """The 1-bit workload: Qwen3-8B shape with Q1_G layers (group 128, sign
    bits, fp16 group scales |N(0,0.02)|) and Q8_0 embedding/output, an
    8192-token prompt of random ids fed through lg_prefill (batched: 16 layer
    passes of 512 tokens on the Q1_G x Q8_0 GEMM), then greedy decode at
    positions 8192.. .  Reports prefill and decode tok/s and the decode
    token roofline (weight + KV bytes per token over the time)."""
    from ligguf_amd.model import QWEN3_8B_Q1G, Engine, HostModel
    cfg = QWEN3_8B_Q1G.with_(n_context=ctx + warmup + steps + 1)
    t0 = time.perf_counter()
    hm = HostModel.synthetic(cfg)
    log(f"synthetic {cfg.name} built in {time.perf_counter() - t0:.1f}s")
    eng = Engine(0)
    eng.load(hm)
    prompt = np.random.default_rng(1).integers(1, cfg.vocab, ctx).astype(np.int32)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = eng.prefill(prompt, 0)
    pf_s = time.perf_counter() - t0
    state = None
    if cpu_seconds > 0:
        import tempfile
        state = os.path.join(tempfile.mkdtemp(prefix="lg_q1g_"), "ctx.state")
        eng.state_save(state, ctx)
    tok, pos = int(np.argmax(logits)), ctx
    if warmup:
        tok = int(eng.decode_greedy(tok, pos, warmup)[-1])
        pos += warmup
    torch.cuda.synchronize()
    p_first = pos
    t0 = time.perf_counter()
    eng.decode_greedy(tok, pos, steps)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    pos += steps
    path = {1: "persistent", 2: "multi-kernel", 3: "fused-graph"}.get(eng.path(), "?")
    eng.close()
    mean_bytes = cfg.weight_bytes() + np.mean([cfg.kv_bytes(p) for p in range(p_first, pos)])
    out = {"workload": f"qwen3-8b-shape Q1_G layers, Q8_0 embedding/output, {ctx}-token prompt then greedy decode",
           "prefill_tok_s": round(ctx / pf_s, 1), "decode_tok_s": round(steps / dt, 1),
           "ms_per_token": round(dt / steps * 1e3, 4), "positions": [p_first, pos - 1],
           "bytes_per_token": int(mean_bytes), "hbm_roofline_frac_token": round(mean_bytes / (dt / steps) / HBM_PEAK, 4),
           "decode_path": path}
    if state:
        with _stdout_to_stderr():
            out["cpu_baseline"] = cpu_baseline_q1g(hm, state, cpu_seconds)
        os.unlink(state)
    log(f"q1g: {out}")
    return out


def sampler_report(eng, np, tok: int, pos: int, reps: int = 50):
    """lg_sample_topp (softmax, sort and cutoff on the device, one token back
    to the host, synchronous) over the decode step's vocabulary logits, per
    call, against the reference's sampler_topp (qsort of the vocabulary, one
    host thread) on the same logits."""
    lg = eng.decode(tok, pos)
    rng = np.random.default_rng(0)
    out = {"vocab": int(lg.size)}
    for name, topk in (("topp0.9_us", 0), ("topp0.9_topk40_us", 40)):
        eng.sample_topp(0.8, 0.9, topk, 0.5)
        t0 = time.perf_counter()
        for _ in range(reps):
            eng.sample_topp(0.8, 0.9, topk, float(rng.random()))
        out[name] = round((time.perf_counter() - t0) / reps * 1e6, 1)
    from oracle import binding
    if binding.reference_available():
        R = binding.load_reference()
        t0 = time.perf_counter()
        for s in range(5):
            R.sampler_topp(lg, 0.8, 0.9, 0, s)
        out["reference_host_topp0.9_us"] = round((time.perf_counter() - t0) / 5 * 1e6, 1)
        out["reference_cores"] = 1
    log(f"sampler: {out}")
    return out


def cpu_info():
    """The host CPU as lscpu reports it and the OpenMP threads the reference
    runs with."""
    import ctypes as C
    import subprocess
    info = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        kv = dict(line.split(":", 1) for line in txt.splitlines() if ":" in line)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        info["model"] = kv.get("Model name")
        sockets = int(kv.get("Socket(s)", "1"))
        info["physical_cores"] = sockets * int(kv.get("Core(s) per socket", "0"))
        info["logical_cpus"] = int(kv.get("CPU(s)", "0"))
    except Exception as e:          # lscpu missing: report what is known
        info["lscpu_error"] = str(e)
    try:
        gomp = C.CDLL("libgomp.so.1")
        info["omp_threads"] = int(gomp.omp_get_max_threads())
    except OSError:
        info["omp_threads"] = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    info["OMP_PROC_BIND"] = os.environ.get("OMP_PROC_BIND")
    info["usable_cpus"] = USABLE_CPUS
    return info


class _stdout_to_stderr:
    """The reference prints progress to stdout (its DBG lines); the bench's
    stdout carries only the JSON line, so C-level stdout goes to stderr
    meanwhile."""

    def __enter__(self):
        sys.stdout.flush()
        self.saved = os.dup(1)
        os.dup2(2, 1)
        return self

    def __exit__(self, *exc):
        import ctypes as C
        C.CDLL(None).fflush(None)
        os.dup2(self.saved, 1)
        os.close(self.saved)
        return False


def _ref_bind(R, hm):
    """Bind a host model's tensors into the reference engine's g_m."""
    import ctypes as C
    import numpy as np
    from ligguf_amd.lib import row_size
    from oracle import binding
    c = hm.cfg
    layers = (binding.RefLayer * c.n_layers)()

    def w(name):
        t, rows, cols, data = hm.weights[name]
        return binding.RefWeight(np.asarray(data).ctypes.data, t, row_size(t, cols))

    def f(name):
        return np.asarray(hm.norms[name]).ctypes.data

    for l in range(c.n_layers):
        b = f"blk.{l}."
        L = layers[l]
        L.att_norm, L.ffn_norm = f(b + "attn_norm.weight"), f(b + "ffn_norm.weight")
        L.att_q, L.att_k, L.att_v = w(b + "attn_q.weight"), w(b + "attn_k.weight"), w(b + "attn_v.weight")
        L.att_out = w(b + "attn_output.weight")
        L.att_q_norm, L.att_k_norm = f(b + "attn_q_norm.weight"), f(b + "attn_k_norm.weight")
        L.ffn_up, L.ffn_down, L.ffn_gate = w(b + "ffn_up.weight"), w(b + "ffn_down.weight"), w(b + "ffn_gate.weight")
    m = binding.RefModel(c.arch, c.n_layers, c.n_embed, c.n_heads, c.n_kv_heads, c.head_dim, c.kv_dim, c.n_ff,
                         c.vocab, c.n_context, c.rope_dim, c.rms_eps, c.rope_theta, w("token_embd.weight"),
                         w("output.weight"), f("output_norm.weight"), C.cast(layers, C.c_void_p))
    R.model_bind(m)


def cpu_baseline(hm, state_path: str, last_pos: int, prompt_tokens: int = 64):
    """The reference FAST engine (oracle/_ref, AVX2, OpenMP) on the same host
    model, decoding the GPU's positions: it loads the state the GPU saved
    after its 512-token prefill (the reference's own state-file format,
    load_model_state, fast/ligguf_fast_qk.cpp:216-263) and decodes greedily
    from there through `last_pos`, the GPU's last timed position.  Its
    prefill rate (feed_text: one inference() per prompt token,
    fast/ligguf_fast_qk.cpp:340-356) is timed on `prompt_tokens` random ids
    beforehand."""
    import numpy as np
    from oracle import binding
    if not binding.reference_available():
        return None
    R = binding.load_reference()
    c = hm.cfg
    _ref_bind(R, hm)
    rng = np.random.default_rng(1)
    R.inference(int(rng.integers(1, c.vocab)), c.vocab)      # untimed: faults pages in, warms caches
    R.set_pos(0)
    prompt = rng.integers(1, c.vocab, prompt_tokens)
    t0 = time.perf_counter()
    for t in prompt:
        R.inference(int(t), c.vocab)
    pf_s = time.perf_counter() - t0
    R.state_load(state_path)
    pos0 = R.get_pos()
    tok = int(np.argmax(R.logits(c.vocab)))
    n, t0 = 0, time.perf_counter()
    while pos0 + n <= last_pos:
        logits = R.inference(tok, c.vocab)
        tok = int(np.argmax(logits))
        n += 1
    dt = time.perf_counter() - t0
    ci = cpu_info()
    threads = ci.get("omp_threads")
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
            "prefill_tok_s": round(prompt_tokens / pf_s, 3), "cpu": ci,
            "sample": f"{n} greedy decode tokens at positions {pos0}..{pos0 + n - 1} from the state the GPU saved "
                      f"after its {pos0}-token prefill, the GPU's timed positions among them (reference FAST engine, "
                      f"AVX2 build, {threads} OpenMP threads); prefill rate from {prompt_tokens} random ids fed "
                      f"token by token, as feed_text"}


def cpu_baseline_q1g(hm, state_path: str, seconds: float, max_tokens: int = 64):
    """The reference on the Q1_G model, decoding from the 8192-token state
    the GPU saved in the reference's own state-file format (load_model_state,
    fast/ligguf_fast_qk.cpp:216-263): an 8192-token prefill on the CPU would
    take hours, so the baseline starts from the file, as the -L option does."""
    import numpy as np
    from oracle import binding
    if not binding.reference_available():
        return None
    R = binding.load_reference()
    c = hm.cfg
    _ref_bind(R, hm)
    R.state_load(state_path)
    pos0 = R.get_pos()
    tok = int(np.argmax(R.logits(c.vocab)))
    logits = R.inference(tok, c.vocab)                     # untimed: faults the weights in
    tok = int(np.argmax(logits))
    n, t0 = 0, time.perf_counter()
    while n < max_tokens and (time.perf_counter() - t0 < seconds or n < 2):
        logits = R.inference(tok, c.vocab)
        tok = int(np.argmax(logits))
        n += 1
    dt = time.perf_counter() - t0
    threads = cpu_info().get("omp_threads")
    return {"value": round(n / dt, 3), "unit": "tok/s", "cores": threads, "kind": "reference",
            "sample": f"{n} greedy decode tokens at positions {pos0 + 1}..{pos0 + n} from the GPU's state file "
                      f"(reference FAST engine, AVX2 build, {threads} OpenMP threads)"}


def layer_type_config(cfg, name: str):
    """The headline shape with its layer matrices of another type (or mix)."""
    from ligguf_amd.lib import TYPE_NAMES, Q6_K
    if name == "Q4_K":
        return cfg
    if name == "Q4_K_M":
        return cfg.with_(name=cfg.name + "_m", overrides=(("attn_v", Q6_K), ("ffn_down", Q6_K)))
    if name == "Q4_K_Mx":
        # llama.cpp's Q4_K_M choice of layers for the larger attn_v / ffn_down type: the first and last
        # eighth of the layers and every third one between them
        n = cfg.n_layers
        more = [l for l in range(n) if l < n // 8 or l >= 7 * n // 8 or (l - n // 8) % 3 == 2]
        return cfg.with_(name=cfg.name + "_mx", overrides=tuple((f"{t}.{l}", Q6_K) for l in more
                                                                 for t in ("attn_v", "ffn_down")))
    lt = {v: k for k, v in TYPE_NAMES.items()}[name]
    return cfg.with_(name=cfg.name.replace("q4_k", name.lower()), layer_type=lt)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prefill", type=int, default=512)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-kernel", action="store_true")
    ap.add_argument("--no-isolated", action="store_true", help="skip the isolated matvec/attention lines")
    ap.add_argument("--isolated-only", action="store_true", help="only the isolated matvec/attention lines")
    ap.add_argument("--no-q1g", action="store_true", help="skip the Q1_G 8192-context workload")
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the dominant-kernel timing plus a plain copy of known size (for PMC runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only the prefill: the prompt twice, the second timed (for MFMA counter runs)")
    ap.add_argument("--layer-type", default="Q4_K",
                    help="with --prefill-only / --decode-only: the layer matrices' type (Q2_K..Q6_K, Q8_0, Q1_0, "
                         "Q1_G; Q4_K_M: Q4_K with Q6_K attn_v and ffn_down; Q4_K_Mx: Q6_K attn_v and ffn_down in "
                         "the layers where llama.cpp's Q4_K_M mix puts them, Q4_K elsewhere)")
    ap.add_argument("--decode-only", action="store_true",
                    help="only the prefill and greedy decode of the --layer-type model, one JSON record")
    ap.add_argument("--q1g-only", action="store_true",
                    help="run only the Q1_G long-context workload and print its line (profiling)")
    ap.add_argument("--q1g-ctx", type=int, default=8192, help="prompt length of the Q1_G workload")
    ap.add_argument("--no-bert", action="store_true", help="skip the BERT embedding / vector-memory lines")
    ap.add_argument("--bert-only", action="store_true",
                    help="run only the BERT embedding / vector-memory workloads and print their line (profiling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU: the decode path here is single-GPU (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch
    from ligguf_amd.model import QWEN3_8B_Q4K, Engine, HostModel

    cfg = QWEN3_8B_Q4K.with_(n_context=max(1024, args.prefill + args.warmup + 2 * args.steps + 1))
    if args.kernel_only:
        hm = HostModel.synthetic(cfg)
        eng = Engine(0)
        eng.load(hm)
        eng.decode(1, 0, want_logits=False)           # a known device step record
        copy_gbs = plain_copy(torch)
        roof = dominant_kernel_roofline(eng, cfg)
        eng.close()
        print(json.dumps({"roofline": roof, "copy": copy_gbs}), flush=True)
        return 0

    if args.q1g_only:
        print(json.dumps({"q1g": q1g_context(torch, np, ctx=args.q1g_ctx)}), flush=True)
        return 0

    if args.bert_only:
        print(json.dumps({"bert": bert_report(torch, np, 0.0 if args.no_cpu else args.cpu_seconds)}), flush=True)
        return 0

    if args.prefill_only or args.decode_only:
        cfg = layer_type_config(cfg, args.layer_type)
    if args.decode_only:
        hm = HostModel.synthetic(cfg)
        eng = Engine(0)
        eng.load(hm)
        prompt = np.random.default_rng(0).integers(1, cfg.vocab, args.prefill).astype(np.int32)
        logits = eng.prefill(prompt, 0)
        tok, pos = int(np.argmax(logits)), args.prefill
        if args.warmup:
            tok = int(eng.decode_greedy(tok, pos, args.warmup)[-1])
            pos += args.warmup
        torch.cuda.synchronize()
        p_first, t0 = pos, time.perf_counter()
        eng.decode_greedy(tok, pos, args.steps)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        pos += args.steps
        mean_bytes = cfg.weight_bytes() + np.mean([cfg.kv_bytes(p) for p in range(p_first, pos)])
        rep = {"model": cfg.name, "tok_s": round(args.steps / dt, 2), "ms_per_token": round(dt / args.steps * 1e3, 4),
               "bytes_per_token": int(mean_bytes), "hbm_roofline_frac_token": round(mean_bytes / (dt / args.steps) /
                                                                                   HBM_PEAK, 4),
               "decode_path": {1: "persistent", 2: "multi-kernel", 3: "fused-graph"}.get(eng.path(), "?"),
               "positions": [p_first, pos - 1]}
        eng.close()
        print(json.dumps({"decode": rep}), flush=True)
        return 0

    if args.isolated_only:
        print(json.dumps({"isolated": isolated_kernels(torch, np)}), flush=True)
        return 0

    if args.prefill_only:
        hm = HostModel.synthetic(cfg)
        eng = Engine(0)
        eng.load(hm)
        prompt = np.random.default_rng(0).integers(1, cfg.vocab, args.prefill).astype(np.int32)
        eng.prefill(prompt, 0)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        eng.prefill(prompt, 0)
        seconds = time.perf_counter() - t0
        rep = prefill_report(cfg, args.prefill, seconds, eng.prefill_path())
        rep["model"] = cfg.name
        eng.close()
        print(json.dumps({"prefill": rep}), flush=True)
        return 0

    t0 = time.perf_counter()
    hm = HostModel.synthetic(cfg)
    log(f"synthetic {cfg.name}: {cfg.weight_bytes() / 1e9:.3f} GB of weights read per token, "
        f"built in {time.perf_counter() - t0:.1f}s")
    eng = Engine(0)
    t0 = time.perf_counter()
    eng.load(hm)
    path_name = {1: "persistent", 2: "multi-kernel", 3: "fused-graph"}.get(eng.path(), "?")
    log(f"uploaded in {time.perf_counter() - t0:.1f}s; decode path {path_name}")

    rng = np.random.default_rng(0)
    prompt = rng.integers(1, cfg.vocab, args.prefill).astype(np.int32)
    eng.prefill(prompt, 0)                         # warm-up: first-use buffers and code objects
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    logits = eng.prefill(prompt, 0)                # the same rows again (KV positions 0.. rewritten)
    prefill_s = time.perf_counter() - t0
    log(f"prefill {args.prefill} tokens: {args.prefill / prefill_s:.1f} tok/s")
    prefill = prefill_report(cfg, args.prefill, prefill_s, eng.prefill_path())
    state = None
    if not args.no_cpu:
        import tempfile
        state = os.path.join(tempfile.mkdtemp(prefix="lg_q4k_"), "prefill.state")
        eng.state_save(state, args.prefill)        # the CPU baseline decodes from here

    pos = args.prefill
    tok = int(np.argmax(logits))
    if args.warmup:
        tok = int(eng.decode_greedy(tok, pos, args.warmup)[-1])   # greedy steps queued back to back
        pos += args.warmup
    torch.cuda.synchronize()
    p_first = pos
    t0 = time.perf_counter()
    toks = eng.decode_greedy(tok, pos, args.steps)   # returns after the last step's token is on the host
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tok = int(toks[-1])
    pos += args.steps
    ms = dt / args.steps * 1e3
    tps = args.steps / dt
    mean_bytes = cfg.weight_bytes() + np.mean([cfg.kv_bytes(p) for p in range(p_first, pos)])
    log(f"decode: {tps:.1f} tok/s, {ms:.3f} ms/token, {mean_bytes / (dt / args.steps) / 1e9:.0f} GB/s per token")
    # the same steps with the greedy token read back to the host each step (lg_decode_step_async + lg_argmax)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.decode_async(tok, pos)
        tok = eng.argmax()
        pos += 1
    torch.cuda.synchronize()
    host_loop_tps = args.steps / (time.perf_counter() - t0)
    log(f"decode with a host round trip per token: {host_loop_tps:.1f} tok/s")

    isolated = None if args.no_isolated else isolated_kernels(torch, np)
    sampler = None if args.no_isolated else sampler_report(eng, np, tok, pos)

    roof = None
    if not args.no_kernel and path_name == "fused-graph":
        roof = dominant_kernel_roofline(eng, cfg)
        log(f"dominant kernel: {roof['avg_us']} us, {roof['achieved']} GB/s ({roof['frac'] * 100:.1f}% of HBM peak)")
    eng.close()

    copy = plain_copy(torch)
    log(f"plain copy: {copy}")
    read = plain_read(torch)
    log(f"plain read: {read}")
    q1g = None if args.no_q1g else q1g_context(torch, np, ctx=args.q1g_ctx,
                                               cpu_seconds=0.0 if args.no_cpu else args.cpu_seconds)
    bert = None if args.no_bert else bert_report(torch, np, 0.0 if args.no_cpu else min(args.cpu_seconds, 10.0))

    cpu = None
    if not args.no_cpu:
        t0 = time.perf_counter()
        with _stdout_to_stderr():
            cpu = cpu_baseline(hm, state, p_first + args.steps - 1)
        log(f"cpu baseline: {cpu} ({time.perf_counter() - t0:.1f}s)")

    out = {
        "metric": "batch-1 decode tok/s (Qwen3-8B-shape Q4_K) + % of HBM roofline",
        "value": round(tps, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-8b-shape Q4_K/Q6_K batch-1 greedy decode after a 512-token prefill",
            "layers": cfg.n_layers, "dim": cfg.n_embed, "heads": f"{cfg.n_heads}/{cfg.n_kv_heads}x{cfg.head_dim}",
            "ffn": cfg.n_ff, "vocab": cfg.vocab, "weights": "Q4_K layers+embedding, Q6_K output",
            "prefill_tokens": args.prefill, "positions": [p_first, pos - 1],
            "bytes_per_token": int(mean_bytes), "decode_path": path_name,
            "decode_loop": "lg_decode_greedy: greedy steps queued back to back, argmax fed forward on the device",
        },
        "decode_host_loop_tok_s": round(host_loop_tps, 1),
        "hbm_roofline_frac_token": round(mean_bytes / (dt / args.steps) / HBM_PEAK, 4),
        "hbm_practical": {"read_GB/s": read["GB/s"], "read_bytes": read["bytes"],
                          "read_frac_of_peak": round(read["GB/s"] * 1e9 / HBM_PEAK, 4),
                          "token_frac_of_read": round(mean_bytes / (dt / args.steps) / (read["GB/s"] * 1e9), 4),
                          "copy_GB/s": copy["GB/s"], "bytes_each_way": copy["bytes_each_way"],
                          "frac_of_peak": round(copy["GB/s"] * 1e9 / HBM_PEAK, 4),
                          "token_frac_of_practical": round(mean_bytes / (dt / args.steps) / (copy["GB/s"] * 1e9), 4)},
        "prefill_tok_s": round(args.prefill / prefill_s, 1),
        "prefill": prefill,
        "roofline": roof,
        "cpu_baseline": cpu,
        "isolated": isolated,
        "sampler": sampler,
        "q1g_8k": q1g,
        "bert": bert,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
