// gemv_q8x4.hip -- W8A16 GEMV over the native Q8_0_4X4 layout (gfx950).
//
// Replaces gemv_par (reference csrc/include/moss/gemv.h:48, csrc/src/gemv.cpp:245-274)
// in its MOSS_A16 mode, whose per-row kernel is row_dot_q8_4x4_actf32
// (csrc/src/gemv_avx2.cpp:123-150):  y[r] = sum_b fp32(d[r,b]) * sum_i q[r,b,i] * x[32b+i].
//
// Mapping.  A 4-row group is one contiguous run of nb*136 bytes, 8-byte aligned
// blocks of 17 qwords (qword 0 = the 4 fp16 scales, qwords 1+4k+j = row k,
// columns 8j..8j+7).  A wavefront handles a group: lane = 16*bl + 4*k + j reads
// qword 1+4k+j of block b = b0+bl (64 lanes = 4 blocks = 512 contiguous bytes
// minus the scale qwords, one global_load_dwordx2 each), plus its row's fp16
// scale (same cache lines).  Activations sit in LDS as fp32.  Each lane
// accumulates acc += d * (8-term fp32 dot); a 4-step xor shuffle sums the 16
// lanes of a row.  SPLIT waves may share one group (split-K), reduced through
// LDS in a fixed order, so results never depend on the launch shape's timing.
//
// Prologues stage the activation: plain fp32/fp16, LayerNorm (llm.cpp:159-171)
// or the split-KV attention merge; epilogues fuse what block_forward
// (llm.cpp:230-246) does next to each GEMV: bias + RoPE + KV write (QKV),
// residual add (proj, fc_out), bias + gelu_new (fc_in).
#include "mh_ops.h"

namespace mh {
namespace {

template <int PRO>
__device__ __forceinline__ void stage_activation(const GemvArgs &a, float *act, float *red) {
    const int t = threadIdx.x;
    const int K = a.cols;
    if constexpr (PRO == PRO_F32) {
        const float4 *x4 = (const float4 *)a.x;
        for (int i = t; i < (K >> 2); i += 256) ((float4 *)act)[i] = x4[i];
    } else if constexpr (PRO == PRO_F16) {
        const __half2 *x2 = (const __half2 *)a.x;
        for (int i = t; i < (K >> 1); i += 256) {
            const float2 f = __half22float2(x2[i]);
            act[2 * i] = f.x;
            act[2 * i + 1] = f.y;
        }
    } else if constexpr (PRO == PRO_LN) {
        const float *x = (const float *)a.x;
        float v[3], o[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) v[i] = x[t + 256 * i];
        layernorm_768(v, a.ln_w, a.ln_b, o, red);
#pragma unroll
        for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
    } else {  // PRO_MERGE: K = heads * 64
        const int n = (a.pos_ptr ? *a.pos_ptr : a.pos_const) + 1;
        const int nsplit = (n + a.chunk - 1) / a.chunk;
        for (int e = t; e < K; e += 256) {
            const int h = e >> 6, d = e & 63;
            const float *ml = a.part_ml + (size_t)h * a.max_splits * 2;
            const float *po = a.part_o + (size_t)h * a.max_splits * 64 + d;
            float m = -INFINITY;
            for (int s = 0; s < nsplit; ++s) m = fmaxf(m, ml[2 * s]);
            float l = 0.0f, o = 0.0f;
            for (int s = 0; s < nsplit; ++s) {
                const float w = expf(ml[2 * s] - m);
                l = fmaf(ml[2 * s + 1], w, l);
                o = fmaf(po[(size_t)s * 64], w, o);
            }
            act[e] = o / l;
        }
    }
}

template <int EPI, int KV>
__device__ __forceinline__ void finish_row(const GemvArgs &a, int r, float v, float partner) {
#pragma clang fp contract(off)
    if constexpr (EPI == EPI_F32) {
        ((float *)a.y)[r] = v;
    } else if constexpr (EPI == EPI_F16) {
        ((__half *)a.y)[r] = __float2half_rn(v);
    } else if constexpr (EPI == EPI_RESID) {
        float *y = (float *)a.y;
        const float *xin = a.resid_in != nullptr ? a.resid_in : y;
        y[r] = xin[r] + (v + a.bias[r]);
    } else if constexpr (EPI == EPI_GELU) {
        ((float *)a.y)[r] = gelu_new(v + a.bias[r]);
    } else {  // EPI_QKV (llm.cpp:234-236 then the KV write of llm.cpp:224-225)
        const float val = v + a.bias[r];
        const int sec = r / kHidden, within = r - sec * kHidden;
        const int h = within >> 6, d = within & 63;
        const int pos = a.pos_ptr ? *a.pos_ptr : a.pos_const;
        float out = val;
        if (sec < 2) {
            const float pv = partner + a.bias[r ^ 1];
            const float c = a.rope_cos[pos * kRopeHalf + (d >> 1)];
            const float s = a.rope_sin[pos * kRopeHalf + (d >> 1)];
            // (x0, x1) -> (x0 c - x1 s, x1 c + x0 s)   (llm.cpp:181-184)
            if ((d & 1) == 0) {
                const float p0 = val * c, p1 = pv * s;
                out = p0 - p1;
            } else {
                const float p0 = val * c, p1 = pv * s;
                out = p0 + p1;
            }
        }
        if (sec == 0) {
            a.q_out[within] = out;
        } else {
            const size_t idx = ((size_t)h * a.ctx_stride + pos) * kHeadDim + d;
            void *cache = sec == 1 ? a.k_cache : a.v_cache;
            if constexpr (KV == KV_F16)
                ((__half *)cache)[idx] = __float2half_rn(out);
            else
                ((float *)cache)[idx] = out;
        }
    }
}

template <int PRO, int EPI, int SPLIT, int KV>
__global__ __launch_bounds__(256) void gemv_q8x4_kernel(GemvArgs a) {
    extern __shared__ float act[];
    __shared__ float red[4];
    __shared__ float part[4][4];
    if (a.state != nullptr && a.state->stop) return;

    stage_activation<PRO>(a, act, red);
    __syncthreads();

    constexpr int GPW = 4 / SPLIT;  // groups per workgroup pass
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gslot = wave / SPLIT, ks = wave % SPLIT;
    const int nb = a.cols >> 5;
    const int ngroups = a.rows >> 2;
    const int bl = lane >> 4, u = lane & 15, kk = u >> 2, j = u & 3;
    const int per = (nb + SPLIT - 1) / SPLIT;
    const int b0 = ks * per, b1 = min(nb, b0 + per);

    for (int gb = blockIdx.x * GPW; gb < ngroups; gb += gridDim.x * GPW) {
        const int g = gb + gslot;
        const bool valid = g < ngroups;
        float acc = 0.0f;
        if (valid) {
            const uint8_t *grp = a.w + (size_t)g * nb * kBlockBytes;
#pragma unroll 4
            for (int b = b0 + bl; b < b1; b += 4) {
                const uint8_t *blk = grp + (size_t)b * kBlockBytes;
                const uint2 qv = *(const uint2 *)(blk + 8 + 8 * u);
                const float d = h2f(*(const uint16_t *)(blk + 2 * kk));
                const float4 x0 = *(const float4 *)(act + b * 32 + 8 * j);
                const float4 x1 = *(const float4 *)(act + b * 32 + 8 * j + 4);
                float s = (float)(int8_t)(qv.x) * x0.x;
                s = fmaf((float)(int8_t)(qv.x >> 8), x0.y, s);
                s = fmaf((float)(int8_t)(qv.x >> 16), x0.z, s);
                s = fmaf((float)(int8_t)(qv.x >> 24), x0.w, s);
                s = fmaf((float)(int8_t)(qv.y), x1.x, s);
                s = fmaf((float)(int8_t)(qv.y >> 8), x1.y, s);
                s = fmaf((float)(int8_t)(qv.y >> 16), x1.z, s);
                s = fmaf((float)(int8_t)(qv.y >> 24), x1.w, s);
                acc = fmaf(s, d, acc);
            }
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        float yv = acc;
        if constexpr (SPLIT > 1) {
            if (lane < 16 && j == 0) part[wave][kk] = acc;
            __syncthreads();
            yv = part[gslot * SPLIT][kk];
#pragma unroll
            for (int s2 = 1; s2 < SPLIT; ++s2) yv += part[gslot * SPLIT + s2][kk];
            __syncthreads();
        }
        const float partner = __shfl_xor(yv, 4);
        if (ks == 0 && valid && lane < 16 && j == 0) finish_row<EPI, KV>(a, 4 * g + kk, yv, partner);
    }
}

template <int PRO, int EPI, int KV>
hipError_t launch_split(const GemvArgs &a, int split, hipStream_t s) {
    const int ngroups = a.rows / 4;
    const size_t lds = (size_t)a.cols * sizeof(float);
    auto grid_for = [&](int gpw) {
        int g = (ngroups + gpw - 1) / gpw;
        return g > 4096 ? 4096 : g;
    };
    switch (split) {
        case 4:
            hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, 4, KV>), dim3(grid_for(1)), dim3(256), lds, s, a);
            break;
        case 2:
            hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, 2, KV>), dim3(grid_for(2)), dim3(256), lds, s, a);
            break;
        default:
            hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, 1, KV>), dim3(grid_for(4)), dim3(256), lds, s, a);
            break;
    }
    return hipGetLastError();
}

// Waves per 4-row group: enough workgroups to cover the 256 CUs at small N,
// whole-K waves (and a persistent-style grid) at large N.
int pick_split(int rows, int cols) {
    const int groups = rows / 4;
    const int nb = cols / 32;
    if (nb < 16) return 1;
    if (groups >= 2048) return 1;
    if (groups >= 512) return 2;
    return 4;
}

}  // namespace

hipError_t launch_gemv(const GemvArgs &a, Prologue pro, Epilogue epi, KvType kv, hipStream_t s) {
    if (a.rows % 4 != 0 || a.cols % 128 != 0 || a.cols > 4096 || a.rows <= 0) return hipErrorInvalidValue;
    if ((pro == PRO_LN || pro == PRO_MERGE) && a.cols != kHidden) return hipErrorInvalidValue;
    if (epi == EPI_QKV && a.rows != 3 * kHidden) return hipErrorInvalidValue;
    const int split = pick_split(a.rows, a.cols);
#define MH_CASE(P, E)                                                                         \
    if (pro == P && epi == E) {                                                               \
        if (E == EPI_QKV && kv == KV_F32) return launch_split<P, E, KV_F32>(a, split, s);  \
        return launch_split<P, E, KV_F16>(a, split, s);                                   \
    }
    MH_CASE(PRO_F32, EPI_F32)
    MH_CASE(PRO_F16, EPI_F16)
    MH_CASE(PRO_F16, EPI_F32)
    MH_CASE(PRO_F32, EPI_F16)
    MH_CASE(PRO_LN, EPI_QKV)
    MH_CASE(PRO_MERGE, EPI_RESID)
    MH_CASE(PRO_LN, EPI_GELU)
    MH_CASE(PRO_F32, EPI_RESID)
    MH_CASE(PRO_LN, EPI_F32)
#undef MH_CASE
    return hipErrorInvalidValue;
}

}  // namespace mh
