// attention.hip -- single-query causal attention over the KV cache (gfx950).
//
// Replaces LlmModel::attention_core (reference csrc/src/llm.cpp:189-217) for one
// query per head: s_p = (q . k_p) * 0.125, softmax over p < n, o = sum_p w_p v_p.
//
// KV layout (per layer): K[heads][ctx_stride][64] and V likewise, fp16 (or
// fp32), so one head's keys are contiguous 128-byte rows.  Split-KV: workgroup
// (split s, head h) owns positions [s*chunk, (s+1)*chunk); it writes the
// unnormalised o_s = sum_p exp(s_p - m_s) v_p plus (m_s, l_s).  The consumer
// (a standalone merge, or the proj GEMV prologue) combines the splits with a
// log-sum-exp merge.  The grid is sized for the cache capacity; splits past the
// live key count exit immediately, so a captured graph stays valid as n grows.
#include "mh_ops.h"

namespace mh {
namespace {

template <int KV>
__device__ __forceinline__ void load_row8(const void *base, size_t idx, float (&f)[8]) {
    if constexpr (KV == KV_F16) {
        const uint4 raw = *(const uint4 *)((const __half *)base + idx);
        const __half2 *h = (const __half2 *)&raw;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 t = __half22float2(h[i]);
            f[2 * i] = t.x;
            f[2 * i + 1] = t.y;
        }
    } else {
        const float4 a = *(const float4 *)((const float *)base + idx);
        const float4 b = *(const float4 *)((const float *)base + idx + 4);
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
}

template <int KV>
__device__ __forceinline__ float4 load4(const void *base, size_t idx) {
    if constexpr (KV == KV_F16) {
        const uint2 raw = *(const uint2 *)((const __half *)base + idx);
        const __half2 *h = (const __half2 *)&raw;
        const float2 a = __half22float2(h[0]), b = __half22float2(h[1]);
        return make_float4(a.x, a.y, b.x, b.y);
    } else {
        return *(const float4 *)((const float *)base + idx);
    }
}

template <int KV, int PPL>  // PPL = positions per lane in the score phase (chunk = 64 * PPL)
__global__ __launch_bounds__(64) void attn_split_kernel(AttnArgs a) {
    __shared__ float qs[kHeadDim];
    __shared__ float sc[64 * PPL];
    if (a.state != nullptr && a.state->stop) return;
    const int s = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const int n = (a.pos_ptr ? *a.pos_ptr : a.pos_const) + 1;
    const int chunk = 64 * PPL;
    const int p0 = s * chunk;
    if (p0 >= n) return;
    const int cnt = min(chunk, n - p0);
    qs[lane] = a.q[h * kHeadDim + lane];
    __syncthreads();

    const size_t head_base = (size_t)h * a.ctx_stride * kHeadDim;
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
        const int pi = lane + 64 * i;
        float dot = -INFINITY;
        if (pi < cnt) {
            const size_t row = head_base + (size_t)(p0 + pi) * kHeadDim;
            dot = 0.0f;
#pragma unroll
            for (int c = 0; c < kHeadDim; c += 8) {
                float kf[8];
                load_row8<KV>(a.k_cache, row + c, kf);
#pragma unroll
                for (int e = 0; e < 8; ++e) dot = fmaf(qs[c + e], kf[e], dot);
            }
            dot *= 0.125f;  // 1/sqrt(64), applied after the dot as llm.cpp:200 does
        }
        sc[pi] = dot;
        m = fmaxf(m, dot);
    }
    m = wave_max(m);
    float l = 0.0f;
#pragma unroll
    for (int i = 0; i < PPL; ++i) {
        const int pi = lane + 64 * i;
        const float e = pi < cnt ? expf(sc[pi] - m) : 0.0f;
        sc[pi] = e;
        l += e;
    }
    l = wave_sum(l);
    __syncthreads();

    // o[d] = sum_p e_p v_p[d]: lane = 16*pg + dg covers dims 4dg..4dg+3 of every 4th position.
    const int pg = lane >> 4, dg = lane & 15;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = pg; i < cnt; i += 4) {
        const float e = sc[i];
        const float4 v = load4<KV>(a.v_cache, head_base + (size_t)(p0 + i) * kHeadDim + 4 * dg);
        o.x = fmaf(e, v.x, o.x);
        o.y = fmaf(e, v.y, o.y);
        o.z = fmaf(e, v.z, o.z);
        o.w = fmaf(e, v.w, o.w);
    }
#pragma unroll
    for (int off = 16; off < 64; off <<= 1) {
        o.x += __shfl_xor(o.x, off);
        o.y += __shfl_xor(o.y, off);
        o.z += __shfl_xor(o.z, off);
        o.w += __shfl_xor(o.w, off);
    }
    const size_t slot = (size_t)h * a.max_splits + s;
    if (lane < 16) ((float4 *)(a.part_o + slot * kHeadDim))[dg] = o;
    if (lane == 0) {
        a.part_ml[2 * slot] = m;
        a.part_ml[2 * slot + 1] = l;
    }
}

__global__ __launch_bounds__(64) void attn_merge_kernel(AttnArgs a, void *out, int out_f16) {
    const int h = blockIdx.x, d = threadIdx.x;
    const int n = (a.pos_ptr ? *a.pos_ptr : a.pos_const) + 1;
    const int nsplit = (n + a.chunk - 1) / a.chunk;
    const float *ml = a.part_ml + (size_t)h * a.max_splits * 2;
    const float *po = a.part_o + (size_t)h * a.max_splits * kHeadDim + d;
    float m = -INFINITY;
    for (int s = 0; s < nsplit; ++s) m = fmaxf(m, ml[2 * s]);
    float l = 0.0f, o = 0.0f;
    for (int s = 0; s < nsplit; ++s) {
        const float w = expf(ml[2 * s] - m);
        l = fmaf(ml[2 * s + 1], w, l);
        o = fmaf(po[(size_t)s * kHeadDim], w, o);
    }
    const float r = o / l;
    if (out_f16)
        ((__half *)out)[h * kHeadDim + d] = __float2half_rn(r);
    else
        ((float *)out)[h * kHeadDim + d] = r;
}

}  // namespace

hipError_t launch_attn_split(const AttnArgs &a, KvType kv, hipStream_t s) {
    if (a.chunk % 64 != 0 || a.chunk < 64 || a.chunk > 256 || a.max_splits <= 0 || a.heads <= 0)
        return hipErrorInvalidValue;
    const dim3 grid(a.max_splits, a.heads);
    const int ppl = a.chunk / 64;
#define MH_ATTN(KVT, P) hipLaunchKernelGGL((attn_split_kernel<KVT, P>), grid, dim3(64), 0, s, a)
    if (kv == KV_F16) {
        if (ppl == 1) MH_ATTN(KV_F16, 1);
        else if (ppl == 2) MH_ATTN(KV_F16, 2);
        else if (ppl == 3) MH_ATTN(KV_F16, 3);
        else MH_ATTN(KV_F16, 4);
    } else {
        if (ppl == 1) MH_ATTN(KV_F32, 1);
        else if (ppl == 2) MH_ATTN(KV_F32, 2);
        else if (ppl == 3) MH_ATTN(KV_F32, 3);
        else MH_ATTN(KV_F32, 4);
    }
#undef MH_ATTN
    return hipGetLastError();
}

hipError_t launch_attn_merge(const AttnArgs &a, void *out, int out_f16, hipStream_t s) {
    hipLaunchKernelGGL(attn_merge_kernel, dim3(a.heads), dim3(64), 0, s, a, out, out_f16);
    return hipGetLastError();
}

}  // namespace mh
