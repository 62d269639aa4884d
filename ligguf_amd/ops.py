"""Per-op calls of the C-ABI on torch device tensors.

Names follow the reference's math layer (fast/lil_math.h:5-39).  torch only
supplies device memory and the stream: every call goes to libligguf_hip.so
and raises LgError on failure; there is no CPU path.
"""
from __future__ import annotations

import torch

from .lib import BLOCK, F32, Q8_0, Q8_K, check, load


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _p(t):
    if t is None:
        return None
    assert t.is_cuda and t.is_contiguous(), "device tensors must be contiguous CUDA tensors"
    return t.data_ptr()


def dequantize_row(t: int, x: torch.Tensor, n: int) -> torch.Tensor:
    y = torch.empty(n, dtype=torch.float32, device=x.device)
    check(load().lg_dequantize_row(t, _p(x), _p(y), n, _stream()))
    return y


def quantize_q8_0(x: torch.Tensor) -> torch.Tensor:
    n = x.numel()
    y = torch.empty(n // 32 * 34, dtype=torch.uint8, device=x.device)
    check(load().lg_quantize_q8_0(_p(x), n, _p(y), _stream()))
    return y


def quantize_q8_K(x: torch.Tensor) -> torch.Tensor:
    n = x.numel()
    y = torch.empty(n // 256 * 292, dtype=torch.uint8, device=x.device)
    check(load().lg_quantize_q8_K(_p(x), n, _p(y), _stream()))
    return y


def matvec(t: int, w: torch.Tensor, rsz: int, n: int, d: int, xq: torch.Tensor, out: torch.Tensor = None,
           accumulate: bool = False) -> torch.Tensor:
    if out is None:
        out = torch.empty(d, dtype=torch.float32, device=w.device)
    check(load().lg_matvec(t, _p(w), rsz, n, d, _p(xq), _p(out), 1 if accumulate else 0, _stream()))
    return out


def matmul_tokens(t: int, w: torch.Tensor, rsz: int, n: int, d: int, x: torch.Tensor) -> torch.Tensor:
    """lg_matmul_tokens: x [T, n] fp32 -> [T, d], each row quantized to the
    activation form of weight type t (Q8_K for the K-quants, else Q8_0)."""
    T = x.shape[0]
    out = torch.empty((T, d), dtype=torch.float32, device=w.device)
    check(load().lg_matmul_tokens(t, _p(w), rsz, n, d, _p(x), T, _p(out), _stream()))
    return out


def rmsnorm_quant(x: torch.Tensor, w: torch.Tensor, eps: float, qtype: int, want_float: bool = False):
    n = x.numel()
    if qtype == F32:
        q = None
        f = torch.empty(n, dtype=torch.float32, device=x.device)
        check(load().lg_rmsnorm_quant(_p(x), _p(w), n, eps, qtype, None, _p(f), _stream()))
        return f
    qk, bs = BLOCK[qtype]
    q = torch.empty((n + qk - 1) // qk * bs, dtype=torch.uint8, device=x.device)
    f = torch.empty(n, dtype=torch.float32, device=x.device) if want_float else None
    check(load().lg_rmsnorm_quant(_p(x), _p(w), n, eps, qtype, _p(q), _p(f), _stream()))
    return (q, f) if want_float else q


def qk_norm_rope_kv(q, k, v, qw, kw, n_heads, n_kv_heads, head_dim, rope_dim, pos, freq, eps, kc_row=None,
                    vc_row=None) -> None:
    check(load().lg_qk_norm_rope_kv(_p(q), _p(k), _p(v), _p(qw), _p(kw), n_heads, n_kv_heads, head_dim, rope_dim,
                                    pos, _p(freq), eps, _p(kc_row), _p(vc_row), _stream()))


def attention(q, k, v, kc, vc, n_heads, n_kv_heads, head_dim, pos, workspace: torch.Tensor = None) -> torch.Tensor:
    lib = load()
    need = lib.lg_attn_workspace_size(n_heads, head_dim, pos)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    out = torch.empty(n_heads * head_dim, dtype=torch.float32, device=q.device)
    check(lib.lg_attn_decode(_p(q), _p(k), _p(v), _p(kc), _p(vc), n_heads, n_kv_heads, head_dim, pos, _p(out),
                             _p(workspace), workspace.numel(), _stream()))
    return out


def swiglu_quant(hb: torch.Tensor, hb2: torch.Tensor, qtype: int = Q8_K):
    n = hb.numel()
    if qtype == F32:
        check(load().lg_swiglu_quant(_p(hb), _p(hb2), n, qtype, None, _stream()))
        return None
    qk, bs = BLOCK[qtype]
    q = torch.empty((n + qk - 1) // qk * bs, dtype=torch.uint8, device=hb.device)
    check(load().lg_swiglu_quant(_p(hb), _p(hb2), n, qtype, _p(q), _stream()))
    return q


__all__ = ["dequantize_row", "quantize_q8_0", "quantize_q8_K", "matvec", "rmsnorm_quant", "qk_norm_rope_kv",
           "attention", "swiglu_quant", "Q8_0", "Q8_K", "F32"]
