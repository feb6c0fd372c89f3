// attention.hip -- single-query causal attention over the KV cache (gfx950).
//
// Replaces LlmModel::attention_core (reference csrc/src/llm.cpp:189-217) for one
// query per head: s_p = (q . k_p) * 0.125, softmax over p < n, o = sum_p w_p v_p.
//
// KV layout (per layer): K[heads][ctx_stride][64] and V likewise, fp16 (or
// fp32), so one head's keys are contiguous 128-byte rows.
//
// One workgroup per head, NW wavefronts: wave w owns positions
// [w*64*PPL, (w+1)*64*PPL) (PPL positions per lane), computes its scores, its
// local max m_w and sum l_w and the unnormalised o_w = sum exp(s_p - m_w) v_p;
// the waves are then merged through LDS with a log-sum-exp combine (split-KV
// inside the workgroup: no cross-workgroup traffic, no fences).  Every K/V load
// is unconditional -- rows past the live count are clamped to a live row and
// weighted 0 -- so each lane has all its loads in flight at once.  NW*64*PPL
// bounds the key count; waves without live keys skip the work.
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

template <int KV, int PPL, int NW>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(AttnArgs a) {
    constexpr int SPAN = 64 * PPL;  // positions per wave
    __shared__ float qs[kHeadDim];
    __shared__ float sc[NW][SPAN];
    __shared__ float4 po[NW][16];
    __shared__ float pm[NW], pl[NW];
    if (a.state != nullptr && a.state->stop) return;
    const int h = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = (a.pos_ptr ? *a.pos_ptr : a.pos_const) + 1;
    if (threadIdx.x < kHeadDim) qs[threadIdx.x] = a.q[h * kHeadDim + threadIdx.x];
    __syncthreads();

    const int p0 = w * SPAN;
    const int cnt = min(SPAN, n - p0);  // <= 0: this wave has no keys
    const size_t head_base = (size_t)h * a.ctx_stride * kHeadDim;
    float m = -INFINITY, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    const int pg = lane >> 4, dg = lane & 15;
    if (cnt > 0) {
        float dots[PPL];
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            const int pi = min(lane + 64 * i, cnt - 1);
            const size_t row = head_base + (size_t)(p0 + pi) * kHeadDim;
            float kf[8][8];
#pragma unroll
            for (int c = 0; c < 8; ++c) load_row8<KV>(a.k_cache, row + 8 * c, kf[c]);
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int e = 0; e < 8; ++e) dot = fmaf(qs[8 * c + e], kf[c][e], dot);
            dots[i] = dot * 0.125f;  // 1/sqrt(64), applied after the dot as llm.cpp:200 does
        }
#pragma unroll
        for (int i = 0; i < PPL; ++i)
            if (lane + 64 * i < cnt) m = fmaxf(m, dots[i]);
        m = wave_max(m);
#pragma unroll
        for (int i = 0; i < PPL; ++i) {
            const float e = lane + 64 * i < cnt ? expf(dots[i] - m) : 0.0f;
            sc[w][lane + 64 * i] = e;
            l += e;
        }
        l = wave_sum(l);
        // sc[w][*] is written and read by different lanes of this one wave
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        // o[d] = sum_p e_p v_p[d]: lane = 16*pg + dg covers dims 4dg..4dg+3 of every 4th position.
#pragma unroll
        for (int t = 0; t < 16 * PPL; ++t) {
            const int i = pg + 4 * t;
            const int ic = min(i, cnt - 1);
            const float4 v = load4<KV>(a.v_cache, head_base + (size_t)(p0 + ic) * kHeadDim + 4 * dg);
            const float e = sc[w][i];
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
    }
    if (NW == 1) {
        if (lane < 16) {
            const float inv = 1.0f / l;
            const int base = h * kHeadDim + 4 * dg;
            const float r[4] = {o.x * inv, o.y * inv, o.z * inv, o.w * inv};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (a.out_f16)
                    ((__half *)a.out)[base + k] = __float2half_rn(r[k]);
                else
                    ((float *)a.out)[base + k] = r[k];
            }
        }
        return;
    }
    if (lane < 16) po[w][dg] = o;
    if (lane == 0) {
        pm[w] = m;
        pl[w] = l;
    }
    __syncthreads();
    if (w != 0) return;
    // log-sum-exp merge of the live waves, lane d = output dimension
    const int live = min(NW, (n + SPAN - 1) / SPAN);
    float M = -INFINITY;
    for (int t = 0; t < live; ++t) M = fmaxf(M, pm[t]);
    float L = 0.0f, O = 0.0f;
    for (int t = 0; t < live; ++t) {
        const float s = expf(pm[t] - M);
        L = fmaf(pl[t], s, L);
        O = fmaf(((const float *)&po[t][0])[lane], s, O);
    }
    const float r = O / L;
    if (a.out_f16)
        ((__half *)a.out)[h * kHeadDim + lane] = __float2half_rn(r);
    else
        ((float *)a.out)[h * kHeadDim + lane] = r;
}

template <int KV, int NW>
hipError_t launch_ppl(const AttnArgs &a, int ppl, hipStream_t s) {
    const dim3 grid(a.heads), block(64 * NW);
    switch (ppl) {
        case 1: hipLaunchKernelGGL((attn_decode_kernel<KV, 1, NW>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((attn_decode_kernel<KV, 2, NW>), grid, block, 0, s, a); break;
        case 3: hipLaunchKernelGGL((attn_decode_kernel<KV, 3, NW>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((attn_decode_kernel<KV, 4, NW>), grid, block, 0, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

int attn_max_keys() { return 16 * 64 * 4; }

hipError_t launch_attn_decode(const AttnArgs &a, KvType kv, hipStream_t s) {
    if (a.heads <= 0 || a.max_keys <= 0 || a.max_keys > attn_max_keys() || !a.out) return hipErrorInvalidValue;
    // capacity-based shape (fixed for a captured graph): one wave for <= 64 keys,
    // else 16 waves with ceil(max_keys / 1024) positions per lane.
    if (a.max_keys <= 64) return kv == KV_F16 ? launch_ppl<KV_F16, 1>(a, 1, s) : launch_ppl<KV_F32, 1>(a, 1, s);
    const int ppl = (a.max_keys + 1023) / 1024;
    return kv == KV_F16 ? launch_ppl<KV_F16, 16>(a, ppl, s) : launch_ppl<KV_F32, 16>(a, ppl, s);
}

}  // namespace mh
