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

// Y[m][n] = sum_k A[m][k] W[n][k] over a 16-row x 16-column tile.  The contraction is
// cut into chunks of 32 columns; wave w takes chunks [w nch/4, (w+1) nch/4) of every
// round of 1024 columns and reads its A and W straight from global memory (each lane
// 8 consecutive columns of one A row and one W row per chunk, all of the wave's chunks in
// flight before the first MFMA); the 4 partial tiles are summed in LDS and thread t
// finishes element (t / 16, t % 16).  Prologues transform A as it is loaded:
// CPRO_LN with per-row (mean, 1/std) from LDS, CPRO_MERGE with wave w = head w.
constexpr int kWaveChunks = 8;  // chunks of 32 per wave per round (rounds of 1024 columns)

template <int PRO, int EPI, int WF32>
__global__ __launch_bounds__(256) void codec_gemm_kernel(const CodecGemmArgs g) {
    __shared__ float red[4][256];
    __shared__ float2 rowst[16];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, col = lane & 15, grp = lane >> 4;
    const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
    const int am = m0 + col;        // A row this lane feeds
    const bool avalid = am < g.M;
    const int n = n0 + col;          // W row this lane feeds (N % 16 == 0: always valid)

    // CPRO_MERGE: this lane's (row am, head = wave) split weights e^(m_s - M) / sum_s e^(m_s - M) l_s
    float mx = 0.f, inv_den = 0.f;
    if constexpr (PRO == CPRO_MERGE) {
        if (avalid) {
            mx = -INFINITY;
            for (int s = 0; s < g.splits; ++s) mx = fmaxf(mx, g.st[((size_t)s * g.M + am) * kCodecHeads + wave].x);
            float den = 0.f;
            for (int s = 0; s < g.splits; ++s) {
                const float2 st = g.st[((size_t)s * g.M + am) * kCodecHeads + wave];
                den += exp_f(st.x - mx) * st.y;
            }
            inv_den = 1.0f / den;
        }
    }

    floatx4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < g.K; k0 += 32 * 4 * kWaveChunks) {
        const int nch = min(4 * kWaveChunks, (g.K - k0) >> 5);
        const int c0 = wave * nch / 4, c1 = (wave + 1) * nch / 4;
        float4 av[kWaveChunks][2];
        W8<WF32> wr[kWaveChunks];
#pragma unroll
        for (int c = 0; c < kWaveChunks; ++c) {
            const int kk = k0 + 32 * (c0 + c) + 8 * grp;
            if (c0 + c < c1) {
                wr[c].load(g.w, (size_t)n * g.K + kk);
                if constexpr (PRO == CPRO_MERGE) {
                    av[c][0] = av[c][1] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (avalid) {
                        for (int s = 0; s < g.splits; ++s) {
                            const float2 st = g.st[((size_t)s * g.M + am) * kCodecHeads + wave];
                            const float f = exp_f(st.x - mx);
                            const float4 *o = reinterpret_cast<const float4 *>(g.o + ((size_t)s * g.M + am) * kCodecDModel + kk);
                            const float4 o0 = o[0], o1 = o[1];
                            av[c][0].x += f * o0.x;
                            av[c][0].y += f * o0.y;
                            av[c][0].z += f * o0.z;
                            av[c][0].w += f * o0.w;
                            av[c][1].x += f * o1.x;
                            av[c][1].y += f * o1.y;
                            av[c][1].z += f * o1.z;
                            av[c][1].w += f * o1.w;
                        }
                    }
                } else {
                    const float4 *src = reinterpret_cast<const float4 *>(g.a + (size_t)(avalid ? am : 0) * g.lda + kk);
                    av[c][0] = avalid ? src[0] : make_float4(0.f, 0.f, 0.f, 0.f);
                    av[c][1] = avalid ? src[1] : make_float4(0.f, 0.f, 0.f, 0.f);
                }
            } else {
                wr[c].zero();
                av[c][0] = av[c][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        if constexpr (PRO == CPRO_LN) {  // K == 256: one round; the loads above are in flight
            // audio_layernorm (audio_layer.cpp:17-28): two-pass mean / variance over 256, eps 1e-5
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = 4 * wave + j, m = m0 + r;
                if (m < g.M) {  // uniform over the wave
                    const float4 x = *reinterpret_cast<const float4 *>(g.a + (size_t)m * g.lda + 4 * lane);
                    const float mean = wave_sum((x.x + x.y) + (x.z + x.w)) / 256.0f;
                    const float d0 = x.x - mean, d1 = x.y - mean, d2 = x.z - mean, d3 = x.w - mean;
                    const float var = wave_sum((d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3)) / 256.0f;
                    if (lane == 0) rowst[r] = make_float2(mean, 1.0f / sqrtf(var + 1e-5f));
                } else if (lane == 0) {
                    rowst[r] = make_float2(0.f, 0.f);
                }
            }
            __syncthreads();
        }
#pragma unroll
        for (int c = 0; c < kWaveChunks; ++c) {
            if (c0 + c < c1) {
                float a[8] = {av[c][0].x, av[c][0].y, av[c][0].z, av[c][0].w,
                              av[c][1].x, av[c][1].y, av[c][1].z, av[c][1].w};
                if constexpr (PRO == CPRO_LN) {
                    const int kk = k0 + 32 * (c0 + c) + 8 * grp;
                    const float2 rs = rowst[col];
                    const float4 w0 = *reinterpret_cast<const float4 *>(g.ln_w + kk);
                    const float4 w1 = *reinterpret_cast<const float4 *>(g.ln_w + kk + 4);
                    const float4 b0 = *reinterpret_cast<const float4 *>(g.ln_b + kk);
                    const float4 b1 = *reinterpret_cast<const float4 *>(g.ln_b + kk + 4);
                    const float lw[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                    const float lb[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
#pragma unroll
                    for (int i = 0; i < 8; ++i) a[i] = avalid ? (a[i] - rs.x) * rs.y * lw[i] + lb[i] : 0.f;
                } else if constexpr (PRO == CPRO_MERGE) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) a[i] *= inv_den;
                }
                acc0 = mfma4(a[0], wr[c].get(0), acc0);
                acc1 = mfma4(a[1], wr[c].get(1), acc1);
                acc0 = mfma4(a[2], wr[c].get(2), acc0);
                acc1 = mfma4(a[3], wr[c].get(3), acc1);
                acc0 = mfma4(a[4], wr[c].get(4), acc0);
                acc1 = mfma4(a[5], wr[c].get(5), acc1);
                acc0 = mfma4(a[6], wr[c].get(6), acc0);
                acc1 = mfma4(a[7], wr[c].get(7), acc1);
            }
        }
    }
    const floatx4 acc = acc0 + acc1;
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][(4 * grp + i) * 16 + col] = acc[i];
    __syncthreads();
    const int r = t >> 4, cn = t & 15, m = m0 + r, nn = n0 + cn;
    const float v = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
    if (m >= g.M) return;

    if constexpr (EPI == CEPI_QKV) {
        const int region = nn / kCodecDModel, c = nn - region * kCodecDModel;
        const int pos = *g.pos0 + m;
        float out = v;
        if (region < 2) {
            // audio_rope (audio_layer.cpp:30-44): pairs (2i, 2i+1), angle = float(pos) * freq in fp32
            const int tp = t ^ 1;
            const float partner = (red[0][tp] + red[1][tp]) + (red[2][tp] + red[3][tp]);
            const float ang = (float)pos * g.freq[(c & (kCodecHeadDim - 1)) >> 1];
            float sn, cs;
            sincosf(ang, &sn, &cs);
            out = (c & 1) ? partner * sn + v * cs : v * cs - partner * sn;
        }
        float *dst = region == 0 ? g.q : (region == 1 ? g.kc : g.vc);
        const size_t row = region == 0 ? (size_t)m : (size_t)(pos % g.ring);
        dst[row * kCodecDModel + c] = out;
    } else if constexpr (EPI == CEPI_STORE) {
        const int p = g.patch;
        g.y[((size_t)m * p + nn % p) * g.ldy + nn / p] = g.bias ? v + g.bias[nn] : v;
    } else if constexpr (EPI == CEPI_GELU) {
        // audio_gelu (audio_layer.cpp:46)
        g.y[(size_t)m * g.ldy + nn] = 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
    } else {
        float *y = g.y + (size_t)m * g.ldy + nn;
        *y = *y + g.ls[nn] * v;
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

    // block b's operands: K rows kb + l%16 (this lane's 16 columns of the head), V rows
    // kb + 4g + s (4 columns); keys past khi read as zeros (their scores are masked)
    auto load_block = [&](int b, float (&kv)[16], float4 (&vv)[4]) {
        const int kb = klo + 16 * b;
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
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kq = kb + 4 * grp + s;
            vv[s] = kq <= khi ? *reinterpret_cast<const float4 *>(a.vc + (size_t)(kq % a.ring) * kCodecDModel + hoff + 4 * col)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    float kv[16];
    float4 vv[4];
    if (b0 + wave < b1) load_block(b0 + wave, kv, vv);
    for (int b = b0 + wave; b < b1; b += 4) {
        const int kb = klo + 16 * b;
        // the wave's next block is in flight while this one is computed
        float kn[16];
        float4 vn[4];
        const bool more = b + 4 < b1;
        if (more) load_block(b + 4, kn, vn);
        floatx4 sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            sc0 = mfma4(kv[i], qv[i], sc0);
            sc1 = mfma4(kv[i + 1], qv[i + 1], sc1);
        }
        const floatx4 sc = sc0 + sc1;
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
        if (more) {
#pragma unroll
            for (int i = 0; i < 16; ++i) kv[i] = kn[i];
#pragma unroll
            for (int i = 0; i < 4; ++i) vv[i] = vn[i];
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
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    const dim3 grid(g.N / 16, (g.M + 15) / 16);
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
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (a.M <= 0 || a.splits < 1 || a.window <= 0 || a.ring <= 0 || !a.q || !a.kc || !a.vc || !a.pos0 || !a.o || !a.st)
        return MOSS_HIP_EINVAL;
    const dim3 grid((a.M + 15) / 16, kCodecHeads, a.splits);
    hipLaunchKernelGGL(codec_attn_kernel, grid, dim3(256), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

int codec_front_launch(const CodecFrontArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (a.frames <= 0 || !a.codes || !a.z) return MOSS_HIP_EINVAL;
    hipLaunchKernelGGL(codec_front_kernel, dim3(a.frames), dim3(kCodecZ), 0, s, a);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

int codec_advance_launch(int *pos0, const int *rows, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    Rows4 r;
    for (int i = 0; i < kCodecStages; ++i) r.r[i] = rows[i];
    hipLaunchKernelGGL(codec_advance_kernel, dim3(1), dim3(64), 0, s, pos0, r);
    return hipGetLastError() == hipSuccess ? 0 : MOSS_HIP_EDEVICE;
}

}  // namespace mh
