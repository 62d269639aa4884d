/* lg_rope.h -- Qwen3 QK RMSNorm + adjacent-pair RoPE + fp16 KV write of one
 * head, one wave per head (the decode step's k_qk_norm_rope_kv and the
 * batched prefill's per-token form). */
#pragma once

#include <math.h>

#include "lg_common.h"

/* head `wave`: waves 0..n_heads-1 take the Q heads, the next n_kv_heads the
 * K heads (which also copy their V slice into the fp16 cache).  Lane l holds
 * elements 4l..4l+3 of the head (head_dim <= 256, multiple of 4), so each
 * RoPE pair (2i, 2i+1) sits in one lane (fast/ligguf_fast_qk.cpp:42-62,
 * fast/lil_math.cpp:901-920). */
__device__ __forceinline__ void lg_qk_norm_rope_kv_wave(int wave, float* __restrict__ q, float* __restrict__ k,
                                                         const float* __restrict__ v, const float* __restrict__ qw,
                                                         const float* __restrict__ kw, int n_heads, int n_kv_heads,
                                                         int hd, int rope_dim, int pos,
                                                         const float* __restrict__ freq, float eps,
                                                         uint16_t* __restrict__ kc_row, uint16_t* __restrict__ vc_row)
{
    const int lane = threadIdx.x & 63;
    if (wave >= n_heads + n_kv_heads) return;
    const bool is_q = wave < n_heads;
    const int h = is_q ? wave : wave - n_heads;
    float* p = (is_q ? q : k) + (size_t)h * hd;
    const float* nw = is_q ? qw : kw;
    const bool act = 4 * lane < hd;
    float e[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
        const float4 t = *(const float4*)(p + 4 * lane);
        e[0] = t.x; e[1] = t.y; e[2] = t.z; e[3] = t.w;
    }
    if (nw) {
        float ss = lg_sq4(make_float4(e[0], e[1], e[2], e[3]));
        ss = lg_group_sum<64>(ss);
        const float sc = 1.0f / sqrtf(ss / (float)hd + eps);
        if (act) {
            const float4 g = *(const float4*)(nw + 4 * lane);
            e[0] = e[0] * sc * g.x; e[1] = e[1] * sc * g.y; e[2] = e[2] * sc * g.z; e[3] = e[3] * sc * g.w;
        }
    }
    int rd = rope_dim < hd ? rope_dim : hd;
    rd &= ~1;
    if (act) {
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
            const int i = 4 * lane + j;
            if (i < rd) {
                const float ang = (float)pos * freq[i >> 1];
                float s, c;
                sincosf(ang, &s, &c);
                const float x0 = e[j], x1 = e[j + 1];
                e[j] = lg_fma2(x0, c, -x1, s);
                e[j + 1] = lg_fma2(x0, s, x1, c);
            }
        }
        *(float4*)(p + 4 * lane) = make_float4(e[0], e[1], e[2], e[3]);
        if (!is_q) {
            const size_t o = (size_t)h * hd + 4 * lane;
            if (kc_row) {
                const uint32_t lo = (uint32_t)lg_f2h(e[0]) | ((uint32_t)lg_f2h(e[1]) << 16);
                const uint32_t hi = (uint32_t)lg_f2h(e[2]) | ((uint32_t)lg_f2h(e[3]) << 16);
                *(uint2*)(kc_row + o) = make_uint2(lo, hi);
            }
            if (vc_row) {
                const float4 t = *(const float4*)(v + o);
                const uint32_t lo = (uint32_t)lg_f2h(t.x) | ((uint32_t)lg_f2h(t.y) << 16);
                const uint32_t hi = (uint32_t)lg_f2h(t.z) | ((uint32_t)lg_f2h(t.w) << 16);
                *(uint2*)(vc_row + o) = make_uint2(lo, hi);
            }
        }
    }
}

