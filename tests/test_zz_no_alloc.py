"""lg_attn_decode_noalloc (the attention entry point that allocates nothing)
against lg_attn_decode on the same inputs: two calls in a row, the second
smaller, each bit-identical to the workspace entry point (same kernels) and
within the attention bar of the oracle."""
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


def test_attn_noalloc_rejects_oversize(gpu):
    lib = L.load()
    # 64 heads of 256 at 2^20 positions need more partials than the scratch area holds
    assert lib.lg_attn_workspace_size(64, 256, 1 << 20) > lib.lg_attn_scratch_bytes()
    rc = lib.lg_attn_decode_noalloc(None, None, None, None, None, 64, 8, 256, 1 << 20, None, None)
    assert rc == -1
    assert b"scratch" in lib.lg_last_error(None)
