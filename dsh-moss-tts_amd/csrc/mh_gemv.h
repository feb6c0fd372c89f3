// mh_gemv.h -- per-wavefront building blocks of the Q8_0_4X4 GEMV (gfx950),
// shared by the one-GEMV-per-launch kernels and the fused decode-layer kernel.
//
// A 4-row group is one contiguous run of nb*136 bytes, 8-byte aligned blocks of
// 17 qwords (qword 0 = the 4 fp16 scales, qwords 1+4k+j = row k, columns
// 8j..8j+7).  Lane = 16*bl + 4*k + j of a wave reads qword 1+4k+j of block
// b = first + bl (+4 per batch step), plus its row's fp16 scale, and accumulates
// acc += d * (8-term fp32 dot) in block order -- the per-row arithmetic of
// row_dot_q8_4x4_actf32 (reference csrc/src/gemv_avx2.cpp:123-150).
#pragma once
#include "mh_device.h"
#include "moss_hip.h"  // MOSS_HIP_CAP_* (quantiser capture layout)

namespace mh {

// Up to NB blocks per lane are in flight at once: all loads of a batch are
// issued before the first is consumed.  Loads are unconditional (the block
// index is clamped to the wave's last block, so every address is valid):
// guarded loads would make the compiler wait on each one in turn.
template <int NB>
__device__ __forceinline__ void load_batch(const uint8_t *grp, int first_b, int b1, int u, int kk, uint2 (&qv)[NB],
                                           uint16_t (&dh)[NB]) {
#pragma unroll
    for (int it = 0; it < NB; ++it) {
        const int b = min(first_b + 4 * it, b1 - 1);
        const uint8_t *blk = grp + (size_t)b * kBlockBytes;
        const uint64_t raw = __builtin_nontemporal_load((const uint64_t *)(blk + 8 + 8 * u));
        qv[it] = make_uint2((uint32_t)raw, (uint32_t)(raw >> 32));
        dh[it] = *(const uint16_t *)(blk + 2 * kk);
    }
}

// A8: act holds the W8A8 activation (integers as floats, see quant_act_lds) and
// da its fp32 block scales: the 8-term sum is then an exact integer, and it is
// scaled by fp32(d_w * d_a), the per-block factor of row_dot_q8_4x4 (reference
// csrc/src/gemv_avx2.cpp:105-121); only the fp32 summation order differs.
template <int NB, bool A8 = false>
__device__ __forceinline__ float dot_batch(const float *act, int first_b, int b1, int j, const uint2 (&qv)[NB],
                                           const uint16_t (&dh)[NB], float acc, const float *da = nullptr) {
#pragma unroll
    for (int it = 0; it < NB; ++it) {
        const int b = first_b + 4 * it;
        if (b < b1) {
            const float4 x0 = *(const float4 *)(act + b * 32 + 8 * j);
            const float4 x1 = *(const float4 *)(act + b * 32 + 8 * j + 4);
            const uint2 q = qv[it];
            float s = (float)(int8_t)(q.x) * x0.x;
            s = fmaf((float)(int8_t)(q.x >> 8), x0.y, s);
            s = fmaf((float)(int8_t)(q.x >> 16), x0.z, s);
            s = fmaf((float)(int8_t)(q.x >> 24), x0.w, s);
            s = fmaf((float)(int8_t)(q.y), x1.x, s);
            s = fmaf((float)(int8_t)(q.y >> 8), x1.y, s);
            s = fmaf((float)(int8_t)(q.y >> 16), x1.z, s);
            s = fmaf((float)(int8_t)(q.y >> 24), x1.w, s);
            if constexpr (A8) {
                const float scale = h2f(dh[it]) * da[b];
                acc = fmaf(s, scale, acc);
            } else {
                acc = fmaf(s, h2f(dh[it]), acc);
            }
        }
    }
    return acc;
}

// The W8A8 activation (quantize_row_q8_0_scaled, reference csrc/src/quant.cpp:28-54,
// via quantize_activation, quant.cpp:45) in place: act[0, K) becomes its int8 values
// (as floats, exact) and da[K / 32] the fp32 block scales d = amax / 127.  Called
// by all 256 threads of the workgroup between two barriers; K % 256 == 0.
//
// For a K known at compile time: quant_block32's arithmetic on runs of 8 consecutive values
// (4 threads per block of 32; thread t takes runs t, t + 256, ...), in registers: a block's
// amax from the run's 8 values and two lane exchanges (every lane of the 4 ends with it),
// then d = amax / 127 and 1 / d in those 4 lanes (not in all 32 lanes of the block), then
// the 8 values scaled and written back.  No barrier inside: the caller's barriers before
// and after order it, and a copy of act made just before it (the capture) needs a barrier
// of its own.  A stage's quantiser measured 0.7 -> ~0.2 us at K = 768 and 2.6 -> ~0.5 us at
// K = 3072 against the loop form below (an LDS round trip per value, 5 exchanges and 2
// divisions per value).
// NT threads (t = 0 .. NT - 1) share the vector: the whole workgroup by default, one
// wave (NT = 64, t = its lane) for a K slice that wave alone reads.
template <int K, int NT = 256>
__device__ __forceinline__ void quant_act_lds_k(float *act, float *da, int t = tix()) {
#pragma clang fp contract(off)
    static_assert(K % NT == 0 && NT % 64 == 0, "whole waves");
    constexpr int R = K / 8, N = (R + NT - 1) / NT;  // runs of 8, runs per thread
    float4 x[N][2];
#pragma unroll
    for (int j = 0; j < N; ++j)
        if (t + NT * j < R) {
            const float4 *p = (const float4 *)(act + 8 * (t + NT * j));
            x[j][0] = p[0];
            x[j][1] = p[1];
        }
    auto qv = [](float v, float id) {
        int q = (int)rintf(v * id);
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        return (float)q;
    };
#pragma unroll
    for (int j = 0; j < N; ++j) {
        const int g = t + NT * j;
        // R is a multiple of 4: the run test holds for whole 4-lane groups, so the
        // exchanges stay inside active groups
        if (g < R) {
            float amax = fmaxf(fmaxf(fabsf(x[j][0].x), fabsf(x[j][0].y)), fmaxf(fabsf(x[j][0].z), fabsf(x[j][0].w)));
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(x[j][1].x), fabsf(x[j][1].y)), fmaxf(fabsf(x[j][1].z), fabsf(x[j][1].w))));
            amax = fmaxf(amax, xshfl<1>(amax));
            amax = fmaxf(amax, xshfl<2>(amax));
            const float d = amax / 127.0f;
            const float id = d > 0.0f ? 1.0f / d : 0.0f;
            float4 *p = (float4 *)(act + 8 * g);
            p[0] = make_float4(qv(x[j][0].x, id), qv(x[j][0].y, id), qv(x[j][0].z, id), qv(x[j][0].w, id));
            p[1] = make_float4(qv(x[j][1].x, id), qv(x[j][1].y, id), qv(x[j][1].z, id), qv(x[j][1].w, id));
            if ((g & 3) == 0) da[g >> 2] = d;
        }
    }
}

// Any K (the GEMV operators): the compile-time forms for the model's widths, else a loop
// of quant_block32.  K is the same for every thread of the workgroup.
__device__ __forceinline__ void quant_act_lds(float *act, float *da, int K) {
    if (K == 768) {
        quant_act_lds_k<768>(act, da);
        return;
    }
    if (K == 3072) {
        quant_act_lds_k<3072>(act, da);
        return;
    }
    for (int i = tix(); i < K; i += 256) {
        float d;
        const int q = quant_block32(act[i], &d);
        act[i] = (float)q;
        if ((i & 31) == 0) da[i >> 5] = d;
    }
}

// Quantiser capture (tests only, moss_hip_llm_capture): the workgroup's 256 threads
// copy n values of an LDS vector to dst.  A copy made just before quant_act_lds_k needs a
// barrier between them (the quantiser rewrites runs other threads copy).
__device__ __forceinline__ void cap_copy(float *dst, const float *src, int n) {
    for (int i = tix(); i < n; i += 256) dst[i] = src[i];
}

// Sum of a row's 16 lanes (lanes 16*bl + 4*kk + j for the row kk): every lane
// of the row ends with the row's total.
__device__ __forceinline__ float row_lane_sum(float acc) {
    acc += xshfl<1>(acc);
    acc += xshfl<2>(acc);
    acc += xshfl<16>(acc);
    acc += xshfl<32>(acc);
    return acc;
}

// A GEMV stage of a fused launch whose weights wait in LDS: GemvStage's rows,
// lanes and summation order, but the workgroup's rows of the stage (one contiguous
// run of 4-row groups, kBytes) are copied into LDS by direct DMA (global_load_lds,
// 16 bytes per lane), issued by one wave a stage or more ahead.  Loads complete in
// issue order per wave, so a gather by the other waves never waits behind the
// copy; the copy must follow a workgroup barrier after the previous use's dot, and
// dot() a __syncthreads() after the copy (its s_waitcnt vmcnt(0) completes it).
template <int NB, int K>
struct LdsGemvStage {
    static constexpr int nb = K / 32, per = nb;
    static constexpr int kGroupBytes = nb * kBlockBytes;
    static constexpr int kBytes = 4 * kGroupBytes;  // a group per wave
    static_assert(per <= 4 * NB && kGroupBytes % 16 == 0, "one batch per wave, whole chunks");
    const uint8_t *base;
    int g;

    // the rows of workgroup b of w (16-byte aligned) into lds (kBytes, 16-byte aligned),
    // by the calling wave alone
    static __device__ __forceinline__ void issue_wave(const uint8_t *w, int b, uint8_t *lds) {
        constexpr int chunks = kBytes / 16;
        const int lane = tix() & 63;
        const uint8_t *src = w + (size_t)b * kBytes;
#pragma unroll
        for (int i = 0; i < (chunks + 63) / 64; ++i)
            if (64 * i + lane < chunks)
                __builtin_amdgcn_global_load_lds((const void *)(src + 16 * (64 * i + lane)), (lds_ptr)(lds + 1024 * i), 16,
                                                 0, 0);
    }
    __device__ __forceinline__ void setup(int b, const uint8_t *lds) {
        const int wave = tix() >> 6;
        g = 4 * b + wave;
        base = lds + wave * kGroupBytes;
    }
    __device__ __forceinline__ int row() const { return 4 * g + ((tix() & 15) >> 2); }
    __device__ __forceinline__ bool storer() const {
        const int lane = tix() & 63;
        return lane < 16 && (lane & 3) == 0;
    }
    // GemvStage<1, NB, K>::dot with the weights read from LDS (same order)
    template <bool A8 = false>
    __device__ __forceinline__ float dot(const float *act, const float *da = nullptr) const {
        const int lane = tix() & 63, u = lane & 15, kk = u >> 2, j = u & 3;
        const int first = lane >> 4;
        float acc = 0.0f;
#pragma unroll
        for (int it = 0; it < NB; ++it) {
            const int b = first + 4 * it;
            if (b < per) {
                const uint8_t *blk = base + b * kBlockBytes;
                const uint2 q = *(const uint2 *)(blk + 8 + 8 * u);
                const float dw = h2f(*(const uint16_t *)(blk + 2 * kk));
                const float4 x0 = *(const float4 *)(act + b * 32 + 8 * j);
                const float4 x1 = *(const float4 *)(act + b * 32 + 8 * j + 4);
                float s = (float)(int8_t)(q.x) * x0.x;
                s = fmaf((float)(int8_t)(q.x >> 8), x0.y, s);
                s = fmaf((float)(int8_t)(q.x >> 16), x0.z, s);
                s = fmaf((float)(int8_t)(q.x >> 24), x0.w, s);
                s = fmaf((float)(int8_t)(q.y), x1.x, s);
                s = fmaf((float)(int8_t)(q.y >> 8), x1.y, s);
                s = fmaf((float)(int8_t)(q.y >> 16), x1.z, s);
                s = fmaf((float)(int8_t)(q.y >> 24), x1.w, s);
                if constexpr (A8) {
                    const float scale = dw * da[b];
                    acc = fmaf(s, scale, acc);
                } else {
                    acc = fmaf(s, dw, acc);
                }
            }
        }
        return row_lane_sum(acc);
    }
};

// QKV epilogue of row r at position pos (llm.cpp:234-236): bias, then RoPE on
// the q and k sections, which pairs row r with its neighbour r ^ 1 (the
// partner's raw sum comes from the caller).  load() before the dot, apply()
// after it.
struct QkvEpi {
    float b0 = 0.f, b1 = 0.f, c = 0.f, s = 0.f;
    __device__ __forceinline__ void load(const float *bias, const float *cosv, const float *sinv, int r, int pos) {
        const int sec = r / kHidden, d = (r - sec * kHidden) & 63;
        b0 = bias[r];
        if (sec < 2) {
            b1 = bias[r ^ 1];
            c = cosv[pos * kRopeHalf + (d >> 1)];
            s = sinv[pos * kRopeHalf + (d >> 1)];
        }
    }
    __device__ __forceinline__ float apply(int r, float v, float partner) const {
#pragma clang fp contract(off)
        const float val = v + b0;
        const int sec = r / kHidden, d = (r - sec * kHidden) & 63;
        if (sec == 2) return val;
        const float pv = partner + b1;
        // (x0, x1) -> (x0 c - x1 s, x1 c + x0 s)   (llm.cpp:181-184)
        const float p0 = val * c, p1 = pv * s;
        return (d & 1) == 0 ? p0 - p1 : p0 + p1;
    }
};

}  // namespace mh
