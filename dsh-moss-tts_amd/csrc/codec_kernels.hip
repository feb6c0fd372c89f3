// codec_kernels.hip -- gfx950 kernels of the audio codec decoder.
//
// Every matrix product runs on v_mfma_f32_16x16x4_f32: fp32 activations times the file's
// weights widened to fp32 (exact for fp16), fp32 accumulation -- the arithmetic of the
// reference's gemm_par on F16/F32 matrices (csrc/src/gemv.cpp:343-363) in another
// summation order.
//
// v_mfma_f32_16x16x4_f32 lane layout: lane l gives A[l%16][k] and B[k][l%16] for the
// k = l/16 of the step, and holds D[4(l/16)+i][l%16], i = 0..3.  Which 4 values of
// the contraction index form a step is free as long as A and B agree; here lane group
// g = l/16 walks 8 (GEMM) or 16 (attention) consecutive indices of its own, so every
// operand is read with 16-byte vector loads.
#include <math.h>

#include "codec.h"
#include "mh_device.h"

namespace mh {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp_f(float x) {  // e^x; e^-inf = 0
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

constexpr int KC = 256;       // contraction columns staged per pass
constexpr int AST = KC + 4;   // LDS row stride (floats): rows start 4 banks apart

// 8 consecutive weights of one row, raw (fp16: one 16-byte load; fp32: two).
template <int WF32>
struct W8 {
    uint4 r[WF32 ? 2 : 1];
    __device__ __forceinline__ void load(const void *w, size_t off) {
        if constexpr (WF32) {
            const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const float *>(w) + off);
            r[0] = p[0];
            r[1] = p[1];
        } else {
            r[0] = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(w) + off);
        }
    }
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < (WF32 ? 2 : 1); ++i) r[i] = make_uint4(0, 0, 0, 0);
    }
    __device__ __forceinline__ float get(int s) const {
        if constexpr (WF32) {
            const uint32_t u = s < 4 ? (&r[0].x)[s] : (&r[1].x)[s - 4];
            return __uint_as_float(u);
        } else {
            const uint32_t u = (&r[0].x)[s >> 1];
            return h2f((uint16_t)((s & 1) ? (u >> 16) : (u & 0xffffu)));
        }
    }
};

// Stage rows m0..m0+15 of the activation source, columns k0..k0+kn, into As (zeros
// past row M).
template <int PRO>
__device__ __forceinline__ void stage_a(const CodecGemmArgs &g, float *As, int m0, int k0, int kn, int t) {
    if constexpr (PRO == CPRO_ROWS) {
        const int q4 = kn >> 2;
        for (int i = t; i < 16 * q4; i += 256) {
            const int r = i / q4, c4 = i - r * q4, m = m0 + r;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < g.M) v = *reinterpret_cast<const float4 *>(g.a + (size_t)m * g.lda + k0 + 4 * c4);
            *reinterpret_cast<float4 *>(As + r * AST + 4 * c4) = v;
        }
    } else if constexpr (PRO == CPRO_LN) {
        // audio_layernorm (audio_layer.cpp:17-28): two-pass mean / variance over 256, eps 1e-5
        const int lane = t & 63, wave = t >> 6;
        const float4 w = *reinterpret_cast<const float4 *>(g.ln_w + 4 * lane);
        const float4 b = *reinterpret_cast<const float4 *>(g.ln_b + 4 * lane);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = 4 * wave + j, m = m0 + r;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < g.M) {  // uniform over the wave
                const float4 x = *reinterpret_cast<const float4 *>(g.a + (size_t)m * g.lda + 4 * lane);
                const float mean = wave_sum((x.x + x.y) + (x.z + x.w)) / 256.0f;
                const float d0 = x.x - mean, d1 = x.y - mean, d2 = x.z - mean, d3 = x.w - mean;
                const float var = wave_sum((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3)) / 256.0f;
                const float inv = 1.0f / sqrtf(var + 1e-5f);
                o = make_float4(d0 * inv * w.x + b.x, d1 * inv * w.y + b.y, d2 * inv * w.z + b.z, d3 * inv * w.w + b.w);
            }
            *reinterpret_cast<float4 *>(As + r * AST + 4 * lane) = o;
        }
    } else {
        // merge of the split-KV partials: sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s
        for (int i = t; i < 16 * 64; i += 256) {
            const int r = i >> 6, c4 = i & 63, h = c4 >> 4, m = m0 + r;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m < g.M) {
                float mx = -INFINITY;
                for (int s = 0; s < g.splits; ++s) mx = fmaxf(mx, g.st[((size_t)s * g.M + m) * kCodecHeads + h].x);
                float den = 0.f;
                for (int s = 0; s < g.splits; ++s) {
                    const float2 st = g.st[((size_t)s * g.M + m) * kCodecHeads + h];
                    const float f = exp_f(st.x - mx);
                    den += f * st.y;
                    const float4 o = *reinterpret_cast<const float4 *>(g.o + ((size_t)s * g.M + m) * kCodecDModel + 4 * c4);
                    v.x += f * o.x;
                    v.y += f * o.y;
                    v.z += f * o.z;
                    v.w += f * o.w;
                }
                const float inv = 1.0f / den;
                v = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
            }
            *reinterpret_cast<float4 *>(As + r * AST + 4 * c4) = v;
        }
    }
}

// Y[m][n] = sum_k A[m][k] W[n][k] over a 16-row x 64-column tile: wave w owns columns
// 16w..16w+15 over the whole contraction, A comes from LDS, W from global memory
// (a pass's 8 chunks of 32 columns are all in flight before its A is staged).
template <int PRO, int EPI, int WF32>
__global__ __launch_bounds__(256) void codec_gemm_kernel(const CodecGemmArgs g) {
    __shared__ __align__(16) float As[16 * AST];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, col = lane & 15, grp = lane >> 4;
    const int m0 = blockIdx.y * 16;
    const int n = blockIdx.x * 64 + wave * 16 + col;
    const bool nvalid = n < g.N;  // N % 16 == 0: whole waves are in or out
    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < g.K; k0 += KC) {
        const int kn = min(KC, g.K - k0);  // multiple of 32
        const int nch = kn >> 5;
        W8<WF32> wr[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (nvalid && c < nch)
                wr[c].load(g.w, (size_t)n * g.K + k0 + 32 * c + 8 * grp);
            else
                wr[c].zero();
        }
        stage_a<PRO>(g, As, m0, k0, kn, t);
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (c < nch) {
                const float4 a0 = *reinterpret_cast<const float4 *>(As + col * AST + 32 * c + 8 * grp);
                const float4 a1 = *reinterpret_cast<const float4 *>(As + col * AST + 32 * c + 8 * grp + 4);
                acc0 = mfma4(a0.x, wr[c].get(0), acc0);
                acc1 = mfma4(a0.y, wr[c].get(1), acc1);
                acc0 = mfma4(a0.z, wr[c].get(2), acc0);
                acc1 = mfma4(a0.w, wr[c].get(3), acc1);
                acc0 = mfma4(a1.x, wr[c].get(4), acc0);
                acc1 = mfma4(a1.y, wr[c].get(5), acc1);
                acc0 = mfma4(a1.z, wr[c].get(6), acc0);
                acc1 = mfma4(a1.w, wr[c].get(7), acc1);
            }
        }
        __syncthreads();
    }
    const floatx4 acc = acc0 + acc1;

    if constexpr (EPI == CEPI_QKV) {
        // RoPE pairs (2i, 2i+1) are adjacent columns, held by lanes l and l ^ 1
        float partner[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) partner[i] = xshfl<1>(acc[i]);
        if (!nvalid) return;
        const int region = n / kCodecDModel, c = n - region * kCodecDModel;
        const int pos0 = *g.pos0;
        const float fr = g.freq[(c & (kCodecHeadDim - 1)) >> 1];
        float *dst = region == 0 ? g.q : (region == 1 ? g.kc : g.vc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + 4 * grp + i;
            if (m >= g.M) break;
            const int pos = pos0 + m;
            float v = acc[i];
            if (region < 2) {
                // audio_rope (audio_layer.cpp:30-44): angle = float(pos) * freq in fp32
                const float ang = (float)pos * fr;
                float sn, cs;
                sincosf(ang, &sn, &cs);
                v = (c & 1) ? partner[i] * sn + v * cs : v * cs - partner[i] * sn;
            }
            const size_t row = region == 0 ? (size_t)m : (size_t)(pos % g.ring);
            dst[row * kCodecDModel + c] = v;
        }
    } else {
        if (!nvalid) return;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + 4 * grp + i;
            if (m >= g.M) break;
            const float v = acc[i];
            if constexpr (EPI == CEPI_STORE) {
                const int p = g.patch;
                const int pr = n % p;
                g.y[((size_t)m * p + pr) * g.ldy + n / p] = g.bias ? v + g.bias[n] : v;
            } else if constexpr (EPI == CEPI_GELU) {
                // audio_gelu (audio_layer.cpp:46)
                g.y[(size_t)m * g.ldy + n] = 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
            } else {
                float *y = g.y + (size_t)m * g.ldy + n;
                *y = *y + g.ls[n] * v;
            }
        }
    }
}

// Windowed causal attention of 16 query rows x one head over the ring's keys
// (attention_window_avx2, attn_avx2.cpp:93-204): key position kp is visible to the
// query at position qp iff 0 <= qp - kp < window.  Grid (row tiles, heads, splits):
// split z takes a contiguous share of the tile's 16-key blocks, its 4 waves every 4th
// block of it, each with a running max / sum (online softmax); the waves merge in LDS
// and the split writes its unnormalised output and (max, sum) for the proj GEMM's
// merge prologue.
//   S^T = K Q^T: A = K[key kb + l%16][16g + t], B = Q[q l%16][16g + t], t = 0..15
//   O^T = V^T P^T per 4-column group j: A = V[key kb + 4g + s][4(l%16) + j], B = P[q][kb + 4g + s]
// so the lane with q = l%16 holds S^T for keys kb + 4g + i and O for columns 16g..16g+15.
__global__ __launch_bounds__(256) void codec_attn_kernel(const CodecAttnArgs a) {
    __shared__ float red[4][16 * 64 + 32];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, col = lane & 15, grp = lane >> 4;
    const int m0 = blockIdx.x * 16, h = blockIdx.y, split = blockIdx.z;
    const int P0 = *a.pos0;
    const int mlast = min(m0 + 15, a.M - 1);
    const int klo = max(0, P0 + m0 - a.window + 1), khi = P0 + mlast;
    const int nkb = (khi - klo + 16) >> 4;
    const int per = (nkb + a.splits - 1) / a.splits;
    const int b0 = split * per, b1 = min(nkb, b0 + per);
    const int mq = m0 + col, qpos = P0 + mq;
    const bool qvalid = mq < a.M;
    const int hoff = h * kCodecHeadDim;

    float qv[16];
    {
        const float4 *src = reinterpret_cast<const float4 *>(a.q + (size_t)(qvalid ? mq : 0) * kCodecDModel + hoff + 16 * grp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = qvalid ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            qv[4 * i] = v.x;
            qv[4 * i + 1] = v.y;
            qv[4 * i + 2] = v.z;
            qv[4 * i + 3] = v.w;
        }
    }
    float mrun = -INFINITY, lrun = 0.f;
    floatx4 o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int b = b0 + wave; b < b1; b += 4) {
        const int kb = klo + 16 * b;
        float kv[16];
        {
            const int kp = kb + col;
            const bool ok = kp <= khi;
            const float4 *src = reinterpret_cast<const float4 *>(a.kc + (size_t)((ok ? kp : klo) % a.ring) * kCodecDModel + hoff + 16 * grp);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = ok ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
                kv[4 * i] = v.x;
                kv[4 * i + 1] = v.y;
                kv[4 * i + 2] = v.z;
                kv[4 * i + 3] = v.w;
            }
        }
        float4 vv[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kp = kb + 4 * grp + s;
            vv[s] = kp <= khi ? *reinterpret_cast<const float4 *>(a.vc + (size_t)(kp % a.ring) * kCodecDModel + hoff + 4 * col)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        floatx4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; ++i) sc = mfma4(kv[i], qv[i], sc);
        float p[4], bmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kp = kb + 4 * grp + i;
            const bool vis = qvalid && kp <= qpos && qpos - kp < a.window;
            p[i] = vis ? sc[i] * 0.125f : -INFINITY;  // 1/sqrt(64)
            bmax = fmaxf(bmax, p[i]);
        }
        bmax = fmaxf(bmax, xshfl<16>(bmax));
        bmax = fmaxf(bmax, xshfl<32>(bmax));
        const float mnew = fmaxf(mrun, bmax);
        const float msafe = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = exp_f(mrun - msafe);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = exp_f(p[i] - msafe);
        lrun = lrun * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        mrun = mnew;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] *= alpha;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            o[0] = mfma4(vv[s].x, p[s], o[0]);
            o[1] = mfma4(vv[s].y, p[s], o[1]);
            o[2] = mfma4(vv[s].z, p[s], o[2]);
            o[3] = mfma4(vv[s].w, p[s], o[3]);
        }
    }
    lrun += xshfl<16>(lrun);
    lrun += xshfl<32>(lrun);
    // lane (grp, col) holds O[q col][16 grp + 4 i + j] = o[j][i]
    float *R = red[wave];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) R[(16 * grp + 4 * i + j) * 16 + col] = o[j][i];
    if (grp == 0) {
        R[1024 + col] = mrun;
        R[1040 + col] = lrun;
    }
    __syncthreads();
    const int q = t >> 4, d4 = t & 15, m = m0 + q;
    if (m >= a.M) return;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, red[w][1024 + q]);
    const float msafe = mx == -INFINITY ? 0.f : mx;
    float l = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float f = exp_f(red[w][1024 + q] - msafe);
        l += f * red[w][1040 + q];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += f * red[w][(4 * d4 + e) * 16 + q];
    }
    const size_t row = (size_t)split * a.M + m;
    *reinterpret_cast<float4 *>(a.o + row * kCodecDModel + hoff + 4 * d4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    if (d4 == 0) a.st[row * kCodecHeads + h] = make_float2(mx, l);
}

// z[t][r] = sum_i (b_i[r] + sum_k W_i[r][k] cb_i[code_it][k])   (decoder.cpp:224-240)
__global__ __launch_bounds__(512) void codec_front_kernel(const CodecFrontArgs a) {
    const int t = blockIdx.x, r = threadIdx.x;
    float z = 0.f;
    for (int i = 0; i < kCodecNq; ++i) {
        const int code = a.codes[i * a.frames + t];
        const float4 *e = reinterpret_cast<const float4 *>(a.cb[i] + (size_t)code * kCodecCbDim);
        const float4 *w = reinterpret_cast<const float4 *>(a.cw[i] + (size_t)r * kCodecCbDim);
        const float4 e0 = e[0], e1 = e[1], w0 = w[0], w1 = w[1];
        float acc = a.cbias[i][r];
        acc += w0.x * e0.x;
        acc += w0.y * e0.y;
        acc += w0.z * e0.z;
        acc += w0.w * e0.w;
        acc += w1.x * e1.x;
        acc += w1.y * e1.y;
        acc += w1.z * e1.z;
        acc += w1.w * e1.w;
        z += acc;
    }
    a.z[(size_t)t * kCodecZ + r] = z;
}

struct Rows4 {
    int r[kCodecStages];
};

__global__ void codec_advance_kernel(int *pos0, Rows4 rows) {
    if (threadIdx.x < kCodecStages) pos0[threadIdx.x] += rows.r[threadIdx.x];
}

template <int PRO, int EPI>
int launch_w(const CodecGemmArgs &g, hipStream_t s) {
    const dim3 grid((g.N + 63) / 64, (g.M + 15) / 16);
    if (g.w_f32)
        hipLaunchKernelGGL((codec_gemm_kernel<PRO, EPI, 1>), grid, dim3(256), 0, s, g);
    else
        hipLaunchKernelGGL((codec_gemm_kernel<PRO, EPI, 0>), grid, dim3(256), 0, s, g);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

}  // namespace

int codec_gemm_launch(int pro, int epi, const CodecGemmArgs &g, hipStream_t s) {
    if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.N % 16 || g.K % 32 || (!g.a && pro != CPRO_MERGE) || !g.w)
        return MOSS_HIP_EINVAL;
    if ((pro == CPRO_LN || pro == CPRO_MERGE) && g.K != kCodecDModel) return MOSS_HIP_EINVAL;
    if (pro == CPRO_ROWS && (g.lda % 4 || g.lda < g.K)) return MOSS_HIP_EINVAL;
    if (pro == CPRO_MERGE && (!g.o || !g.st || g.splits < 1)) return MOSS_HIP_EINVAL;
    if (epi == CEPI_QKV && (g.N != 3 * kCodecDModel || !g.q || !g.kc || !g.vc || g.ring <= 0 || !g.pos0 || !g.freq))
        return MOSS_HIP_EINVAL;
    if (epi == CEPI_STORE && (g.patch < 1 || g.N % g.patch)) return MOSS_HIP_EINVAL;
    if (epi == CEPI_RESID && !g.ls) return MOSS_HIP_EINVAL;
    switch (pro * 4 + epi) {
        case CPRO_ROWS * 4 + CEPI_STORE: return launch_w<CPRO_ROWS, CEPI_STORE>(g, s);
        case CPRO_ROWS * 4 + CEPI_RESID: return launch_w<CPRO_ROWS, CEPI_RESID>(g, s);
        case CPRO_LN * 4 + CEPI_QKV: return launch_w<CPRO_LN, CEPI_QKV>(g, s);
        case CPRO_LN * 4 + CEPI_GELU: return launch_w<CPRO_LN, CEPI_GELU>(g, s);
        case CPRO_MERGE * 4 + CEPI_RESID: return launch_w<CPRO_MERGE, CEPI_RESID>(g, s);
        default: return MOSS_HIP_EUNSUPPORTED;
    }
}

int codec_attn_launch(const CodecAttnArgs &a, hipStream_t s) {
    if (a.M <= 0 || a.splits < 1 || a.window <= 0 || a.ring <= 0 || !a.q || !a.kc || !a.vc || !a.pos0 || !a.o || !a.st)
        return MOSS_HIP_EINVAL;
    const dim3 grid((a.M + 15) / 16, kCodecHeads, a.splits);
    hipLaunchKernelGGL(codec_attn_kernel, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

int codec_front_launch(const CodecFrontArgs &a, hipStream_t s) {
    if (a.frames <= 0 || !a.codes || !a.z) return MOSS_HIP_EINVAL;
    hipLaunchKernelGGL(codec_front_kernel, dim3(a.frames), dim3(kCodecZ), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

int codec_advance_launch(int *pos0, const int *rows, hipStream_t s) {
    Rows4 r;
    for (int i = 0; i < kCodecStages; ++i) r.r[i] = rows[i];
    hipLaunchKernelGGL(codec_advance_kernel, dim3(1), dim3(64), 0, s, pos0, r);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

}  // namespace mh
