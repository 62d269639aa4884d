"""lg_attn_decode_noalloc (the attention entry point that allocates nothing)
against lg_attn_decode on the same inputs: two calls in a row, the second
smaller, each bit-identical to the workspace entry point (same kernels) and
within the attention bar of the oracle; position 0; the size limit at its
boundary; and a call captured into a HIP graph, replayed several times."""
import ctypes as C

import numpy as np
import pytest

from ligguf_amd import lib as L

pytestmark = pytest.mark.gpu


def _inputs(rng, nh, nkv, hd, pos):
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(nkv * hd).astype(np.float32)
    v = rng.standard_normal(nkv * hd).astype(np.float32)
    kc = rng.standard_normal(max(pos, 1) * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    vc = rng.standard_normal(max(pos, 1) * nkv * hd).astype(np.float32).astype(np.float16).view(np.uint16)
    return q, k, v, kc, vc


def test_attn_noalloc_matches_workspace_entry(gpu, oracle):
    import torch
    lib = L.load()
    assert lib.lg_attn_scratch_bytes() == 8 << 20
    rng = np.random.default_rng(7)
    stream = torch.cuda.current_stream().cuda_stream
    # second call smaller in every dimension: fewer heads, shorter context, narrower heads
    for nh, nkv, hd, pos in [(32, 8, 128, 20000), (8, 4, 64, 300)]:
        print(f"noalloc attention: heads {nh}/{nkv} head_dim {hd} pos {pos}", flush=True)
        q, k, v, kc, vc = (torch.from_numpy(a).to(gpu) for a in _inputs(rng, nh, nkv, hd, pos))
        need = lib.lg_attn_workspace_size(nh, hd, pos)
        assert 0 < need <= lib.lg_attn_scratch_bytes()
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        a = torch.empty(nh * hd, dtype=torch.float32, device=gpu)
        b = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device=gpu)
        L.check(lib.lg_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), nh, nkv,
                                   hd, pos, a.data_ptr(), ws.data_ptr(), need, C.c_void_p(stream)))
        L.check(lib.lg_attn_decode_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                                           nh, nkv, hd, pos, b.data_ptr(), C.c_void_p(stream)))
        torch.cuda.synchronize()
        a_h, b_h = a.cpu().numpy(), b.cpu().numpy()
        assert np.array_equal(a_h, b_h), float(np.nanmax(np.abs(a_h - b_h)))
        ref = oracle.attention(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), kc.cpu().numpy(),
                               vc.cpu().numpy(), nh, nkv, hd, pos)
        assert np.max(np.abs(b_h - ref)) <= 2e-6 * max(1.0, float(np.max(np.abs(ref))))


def _call(lib, fn, t, nh, nkv, hd, pos, out, stream, *ws):
    q, k, v, kc, vc = t
    return fn(q.data_ptr(), k.data_ptr(), v.data_ptr(), kc.data_ptr(), vc.data_ptr(), nh, nkv, hd, pos,
              out.data_ptr(), *ws, C.c_void_p(stream))


def test_attn_noalloc_rejects_oversize(gpu):
    lib = L.load()
    cap = lib.lg_attn_scratch_bytes()
    # the limit at its boundary: 32 heads of 128 up to position 2064383 (504
    # chunks of 4096 keys), 64 heads of 256 up to 520191 (127 chunks)
    assert lib.lg_attn_workspace_size(32, 128, 2064383) <= cap < lib.lg_attn_workspace_size(32, 128, 2064384)
    assert lib.lg_attn_workspace_size(64, 256, 520191) <= cap < lib.lg_attn_workspace_size(64, 256, 520192)
    # position 0 takes one chunk of the three-pass kernel
    assert lib.lg_attn_workspace_size(32, 128, 0) == 32 * 130 * 4
    for nh, nkv, hd, pos in [(32, 8, 128, 2064384), (64, 8, 256, 520192), (64, 8, 256, 1 << 20)]:
        rc = lib.lg_attn_decode_noalloc(None, None, None, None, None, nh, nkv, hd, pos, None, None)
        assert rc == -1
        assert b"scratch" in lib.lg_last_error(None)


def test_attn_noalloc_position0(gpu):
    """Position 0 (the current k/v only) with the workspace entry point given
    exactly lg_attn_workspace_size bytes: both results are v, head by head."""
    import torch
    lib = L.load()
    rng = np.random.default_rng(9)
    stream = torch.cuda.current_stream().cuda_stream
    nh, nkv, hd = 32, 8, 128
    t = [torch.from_numpy(a).to(gpu) for a in _inputs(rng, nh, nkv, hd, 0)]
    need = lib.lg_attn_workspace_size(nh, hd, 0)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    a = torch.empty(nh * hd, dtype=torch.float32, device=gpu)
    b = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device=gpu)
    L.check(_call(lib, lib.lg_attn_decode, t, nh, nkv, hd, 0, a, stream, ws.data_ptr(), need))
    L.check(_call(lib, lib.lg_attn_decode_noalloc, t, nh, nkv, hd, 0, b, stream))
    torch.cuda.synchronize()
    v = t[2].cpu().numpy().reshape(nkv, 1, hd)
    want = np.repeat(v, nh // nkv, axis=1).ravel()
    assert np.array_equal(a.cpu().numpy(), b.cpu().numpy())
    assert np.max(np.abs(b.cpu().numpy() - want)) <= 1e-6 * np.max(np.abs(want))


def test_attn_noalloc_graph_capture(gpu):
    """lg_attn_decode_noalloc captured into a HIP graph (the scratch area of
    the device set up beforehand by lg_create) and replayed three times with
    new queries written eagerly in between: every replay equals an eager
    lg_attn_decode of the same inputs bit for bit."""
    import torch
    from ligguf_amd.model import Engine
    lib = L.load()
    eng = Engine(0)                      # lg_create: looks up the device's scratch address
    rng = np.random.default_rng(11)
    nh, nkv, hd, pos = 16, 4, 128, 3000
    t = [torch.from_numpy(a).to(gpu) for a in _inputs(rng, nh, nkv, hd, pos)]
    need = lib.lg_attn_workspace_size(nh, hd, pos)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    ref = torch.empty(nh * hd, dtype=torch.float32, device=gpu)
    out = torch.full((nh * hd,), float("nan"), dtype=torch.float32, device=gpu)
    cur = torch.cuda.current_stream().cuda_stream
    L.check(_call(lib, lib.lg_attn_decode, t, nh, nkv, hd, pos, ref, cur, ws.data_ptr(), need))   # kernels loaded
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=side):
        L.check(_call(lib, lib.lg_attn_decode_noalloc, t, nh, nkv, hd, pos, out,
                      torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    for i in range(3):
        print(f"graph replay {i}", flush=True)
        t[0].copy_(torch.from_numpy(rng.standard_normal(nh * hd).astype(np.float32)))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        L.check(_call(lib, lib.lg_attn_decode, t, nh, nkv, hd, pos, ref, cur, ws.data_ptr(), need))
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), ref.cpu().numpy()), i
    del g
    eng.close()
