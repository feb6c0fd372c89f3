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
// Prologues stage the activation: plain fp32/fp16 or LayerNorm (llm.cpp:159-171);
// epilogues fuse what block_forward
// (llm.cpp:230-246) does next to each GEMV: bias + RoPE + KV write (QKV),
// residual add (proj, fc_out), bias + gelu_new (fc_in).
#include "mh_gemv.h"
#include "mh_ops.h"

namespace mh {
namespace {

// Local attention (llm.cpp:189-217 over the local cache, at most 17 keys),
// computed by every workgroup of the consuming GEMV into its activation, in
// the reference's order: thread (h, p) forms score s_p = (q_h . k_p) * 0.125;
// thread (h, p) then e_p = exp(s_p - max), the in-order sum and w_p = e_p *
// (1 / sum); thread (h, d) finally sums w_p v_p[d] over p in order.  Every
// global load (q, k, and the V values a thread will need) is issued up front;
// keys past the live count are clamped to a live key and weighted 0.
__device__ __forceinline__ void local_attention(const GemvArgs &a, float *act) {
#pragma clang fp contract(off)
    __shared__ float sc[kHeads][kLocalLen + 1];
    const int t = threadIdx.x;
    const int n = (a.pos_ptr ? *a.pos_ptr : a.pos_const) + 1;
    const float *q = (const float *)a.x;
    const float *K = (const float *)a.k_cache, *V = (const float *)a.v_cache;
    float vv[3][kLocalLen];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = t + 256 * k, h = i >> 6, d = i & 63;
#pragma unroll
        for (int p = 0; p < kLocalLen; ++p) vv[k][p] = V[((size_t)h * a.ctx_stride + min(p, n - 1)) * kHeadDim + d];
    }
    const int hp = t / kLocalLen, pp = t - hp * kLocalLen;  // (head, key) of this thread's score
    const bool scorer = t < kHeads * kLocalLen;
    float dot = 0.0f;  // sequential over d, unfused, as llm.cpp:196-198
    if (scorer) {
        const float *kr = K + ((size_t)hp * a.ctx_stride + min(pp, n - 1)) * kHeadDim;
        const float *qh = q + hp * kHeadDim;
#pragma unroll
        for (int c = 0; c < kHeadDim; c += 4) {
            const float4 kv = *(const float4 *)(kr + c);
            const float4 qv = *(const float4 *)(qh + c);
            dot = dot + qv.x * kv.x;
            dot = dot + qv.y * kv.y;
            dot = dot + qv.z * kv.z;
            dot = dot + qv.w * kv.w;
        }
        dot *= 0.125f;
        sc[hp][pp] = dot;
    }
    __syncthreads();
    float e = 0.0f;
    if (scorer && pp < n) {
        float mx = -1e30f;
        for (int p = 0; p < n; ++p) mx = fmaxf(mx, sc[hp][p]);
        e = expf(dot - mx);
    }
    __syncthreads();
    if (scorer) sc[hp][pp] = e;
    __syncthreads();
    float wgt = 0.0f;  // 0 for keys past n
    if (scorer) {
        float sum = 0.0f;
        for (int p = 0; p < n; ++p) sum += sc[hp][p];
        wgt = e * (1.0f / sum);
    }
    __syncthreads();
    if (scorer) sc[hp][pp] = wgt;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = t + 256 * k, h = i >> 6;
        float o = 0.0f;
#pragma unroll
        for (int p = 0; p < kLocalLen; ++p) o = o + sc[h][p] * vv[k][p];
        act[i] = o;
    }
}

// Log-sum-exp merge of split-KV partials (o, m, l per 64-key span) into the
// attention output: o = sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s.  The
// partial o values a thread needs are loaded up front (spans clamped to the
// live ones and weighted 0).
constexpr int kMaxMergeSplits = 16;  // PRO_AMERGE serves key capacities up to 1024
__device__ __forceinline__ void merge_attention(const GemvArgs &a, float *act) {
    __shared__ float pm[kHeads][kMaxMergeSplits], pl[kHeads][kMaxMergeSplits];
    const int t = threadIdx.x;
    const int n = (a.pos_ptr ? *a.pos_ptr : a.pos_const) + 1;
    const int live = (n + 63) / 64;
    const int S = a.attn_splits;
    float ov[3][kMaxMergeSplits];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = t + 256 * k, h = i >> 6, d = i & 63;
#pragma unroll
        for (int sp = 0; sp < kMaxMergeSplits; ++sp)
            ov[k][sp] = a.attn_part[((size_t)h * S + min(sp, live - 1)) * kPartStride + d];
    }
    const int hs = t / kMaxMergeSplits, ss = t - hs * kMaxMergeSplits;
    float m = -INFINITY, l = 0.0f;
    if (hs < kHeads && ss < live) {
        const float *pp = a.attn_part + ((size_t)hs * S + ss) * kPartStride;
        m = pp[64];
        l = pp[65];
    }
    if (hs < kHeads) pm[hs][ss] = m;
    __syncthreads();
    float sw = 0.0f;
    if (hs < kHeads) {
        float M = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < kMaxMergeSplits; ++sp) M = fmaxf(M, pm[hs][sp]);
        sw = ss < live ? expf(m - M) : 0.0f;
    }
    __syncthreads();
    if (hs < kHeads) {
        pm[hs][ss] = sw;
        pl[hs][ss] = sw * l;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = t + 256 * k, h = i >> 6;
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int sp = 0; sp < kMaxMergeSplits; ++sp) {
            L += pl[h][sp];
            O = fmaf(ov[k][sp], pm[h][sp], O);
        }
        act[i] = O / L;
    }
}

// Greedy pick of the previous channel (sampler.cpp:13-28 as llm.cpp:689-697
// calls it) done by every workgroup of the next local step's QKV GEMV:
// penalised argmax (lowest index on ties, 0 if all NaN), the used code
// (forced under teacher forcing), its aemb row, LayerNorm.  Workgroup 0 records
// the pick; the count of the used code is added at the end of the frame.
__device__ __forceinline__ void pick_input(const GemvArgs &a, float *act, float *red) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const int t = threadIdx.x;
    const DevState *st = a.pick_state;
    int idx = greedy_pick_1024(a.pick_logits, a.pick_counts, st->rep_penalty, bv, bi);
    if (idx >= kCodebook) idx = 0;
    const int used = st->forced_on ? a.pick_forced[st->frame * kNVq + a.pick_ch] : idx;
    if (blockIdx.x == 0 && t == 0) {
        a.pick_state->codes[a.pick_ch] = idx;
        a.pick_state->row[a.pick_ch + 1] = used;
    }
    float v[3], o[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = q8x4_elem(a.pick_aemb, kHidden / 32, used, t + 256 * i);
    if (blockIdx.x == 0)
#pragma unroll
        for (int i = 0; i < 3; ++i) a.pick_raw[t + 256 * i] = v[i];
    layernorm_768(v, a.ln_w, a.ln_b, o, red);
#pragma unroll
    for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
}

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
    } else if constexpr (PRO == PRO_LATTN) {
        local_attention(a, act);
    } else if constexpr (PRO == PRO_AMERGE) {
        merge_attention(a, act);
    } else if constexpr (PRO == PRO_PICK) {
        pick_input(a, act, red);
    }
}

// The epilogue's operands (bias, residual, RoPE factors) are loaded before the
// dot product so their latency overlaps it: epi_load at the start of a group,
// epi_store once the row's sum is known.
struct EpiIn {
    float b0 = 0.f, b1 = 0.f, res = 0.f, c = 0.f, s = 0.f;
    int pos = 0;
};

template <int EPI>
__device__ __forceinline__ EpiIn epi_load(const GemvArgs &a, int r) {
    EpiIn e;
    if constexpr (EPI == EPI_RESID) {
        const float *xin = a.resid_in != nullptr ? a.resid_in : (const float *)a.y;
        e.b0 = a.bias[r];
        e.res = xin[r];
    } else if constexpr (EPI == EPI_GELU) {
        e.b0 = a.bias[r];
    } else if constexpr (EPI == EPI_QKV) {
        e.b0 = a.bias[r];
        e.pos = a.pos_ptr ? *a.pos_ptr : a.pos_const;
        const int sec = r / kHidden, d = (r - sec * kHidden) & 63;
        if (sec < 2) {
            e.b1 = a.bias[r ^ 1];
            e.c = a.rope_cos[e.pos * kRopeHalf + (d >> 1)];
            e.s = a.rope_sin[e.pos * kRopeHalf + (d >> 1)];
        }
    }
    return e;
}

template <int EPI, int KV>
__device__ __forceinline__ void epi_store(const GemvArgs &a, int r, float v, float partner, const EpiIn &e) {
#pragma clang fp contract(off)
    if constexpr (EPI == EPI_F32) {
        ((float *)a.y)[r] = v;
    } else if constexpr (EPI == EPI_F16) {
        ((__half *)a.y)[r] = __float2half_rn(v);
    } else if constexpr (EPI == EPI_RESID) {
        ((float *)a.y)[r] = e.res + (v + e.b0);
    } else if constexpr (EPI == EPI_GELU) {
        ((float *)a.y)[r] = gelu_new(v + e.b0);
    } else {  // EPI_QKV (llm.cpp:234-236 then the KV write of llm.cpp:224-225)
        const float val = v + e.b0;
        const int sec = r / kHidden, within = r - sec * kHidden;
        const int h = within >> 6, d = within & 63;
        float out = val;
        if (sec < 2) {
            const float pv = partner + e.b1;
            // (x0, x1) -> (x0 c - x1 s, x1 c + x0 s)   (llm.cpp:181-184)
            if ((d & 1) == 0) {
                const float p0 = val * e.c, p1 = pv * e.s;
                out = p0 - p1;
            } else {
                const float p0 = val * e.c, p1 = pv * e.s;
                out = p0 + p1;
            }
        }
        if (sec == 0) {
            a.q_out[within] = out;
        } else {
            const size_t idx = ((size_t)h * a.ctx_stride + e.pos) * kHeadDim + d;
            void *cache = sec == 1 ? a.k_cache : a.v_cache;
            if constexpr (KV == KV_F16)
                ((__half *)cache)[idx] = __float2half_rn(out);
            else
                ((float *)cache)[idx] = out;
        }
    }
}

template <int EPI, int KV>
__device__ __forceinline__ void finish_row(const GemvArgs &a, int r, float v, float partner) {
    epi_store<EPI, KV>(a, r, v, partner, epi_load<EPI>(a, r));
}

// A8: W8A8 rows -- the staged activation is quantised per 32-block in LDS
// (quant_act_lds) and every block sum scaled by fp32(d_w * d_a), as the
// reference's decode with MOSS_A16 unset (csrc/src/gemv.cpp:229-274).
template <int PRO, int EPI, int SPLIT, int KV, int NB, bool A8>
__global__ __launch_bounds__(256) void gemv_q8x4_kernel(GemvArgs a) {
    extern __shared__ float act[];
    __shared__ float red[4];
    __shared__ float part[4][4];
    __shared__ float da[4096 / 32];  // block scales of act (A8)
    // A frame that has ended (state->stop) makes this a no-op.  The flag is read
    // here but tested after the prologue, so its load overlaps the weight and
    // activation loads instead of delaying them (the prologue only writes
    // per-frame scratch).
    const bool stopped = a.state != nullptr && a.state->stop;

    constexpr int GPW = 4 / SPLIT;  // groups per workgroup pass
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int gslot = wave / SPLIT, ks = wave % SPLIT;
    const int nb = a.cols >> 5;
    const int ngroups = a.rows >> 2;
    const int bl = lane >> 4, u = lane & 15, kk = u >> 2, j = u & 3;
    const int per = (nb + SPLIT - 1) / SPLIT;
    const int b0 = ks * per, b1 = min(nb, b0 + per);
    const int gfirst = blockIdx.x * GPW;

    // The weights do not depend on the activation: start streaming this wave's
    // first batch before the prologue (activation load, LayerNorm) runs.
    uint2 qv[NB];
    uint16_t dh[NB];
    if (gfirst + gslot < ngroups) load_batch<NB>(a.w + (size_t)(gfirst + gslot) * nb * kBlockBytes, b0 + bl, b1, u, kk, qv, dh);
    const bool storer = ks == 0 && lane < 16 && (u & 3) == 0;  // the lane that finishes row 4g + kk
    EpiIn pre;
    if (storer && gfirst + gslot < ngroups) pre = epi_load<EPI>(a, 4 * (gfirst + gslot) + kk);

    stage_activation<PRO>(a, act, red);
    __syncthreads();
    if (stopped) return;
    if constexpr (A8) {
        quant_act_lds(act, da, a.cols);
        __syncthreads();
    }

    for (int gb = gfirst; gb < ngroups; gb += gridDim.x * GPW) {
        const int g = gb + gslot;
        const bool valid = g < ngroups;
        if (gb != gfirst && storer && valid) pre = epi_load<EPI>(a, 4 * g + kk);
        float acc = 0.0f;
        if (valid) {
            const uint8_t *grp = a.w + (size_t)g * nb * kBlockBytes;
            for (int base = b0; base < b1; base += 4 * NB) {
                if (base != b0 || gb != gfirst) load_batch<NB>(grp, base + bl, b1, u, kk, qv, dh);
                acc = dot_batch<NB, A8>(act, base + bl, b1, j, qv, dh, acc, da);
            }
        }
        acc = row_lane_sum(acc);
        float yv = acc;
        if constexpr (SPLIT > 1) {
            if (lane < 16 && j == 0) part[wave][kk] = acc;
            __syncthreads();
            yv = part[gslot * SPLIT][kk];
#pragma unroll
            for (int s2 = 1; s2 < SPLIT; ++s2) yv += part[gslot * SPLIT + s2][kk];
            __syncthreads();
        }
        const float partner = xshfl<4>(yv);
        if (storer && valid) epi_store<EPI, KV>(a, 4 * g + kk, yv, partner, pre);
    }
}

template <int PRO, int EPI, int SPLIT, int KV, bool A8>
hipError_t launch_nb(const GemvArgs &a, int nbatch, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    const int ngroups = a.rows / 4;
    constexpr int GPW = 4 / SPLIT;
    int grid = (ngroups + GPW - 1) / GPW;
    grid = grid > 4096 ? 4096 : grid;
    const size_t lds = (size_t)a.cols * sizeof(float);
    switch (nbatch) {
        case 2: hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, SPLIT, KV, 2, A8>), dim3(grid), dim3(256), lds, s, a); break;
        case 3: hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, SPLIT, KV, 3, A8>), dim3(grid), dim3(256), lds, s, a); break;
        case 6: hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, SPLIT, KV, 6, A8>), dim3(grid), dim3(256), lds, s, a); break;
        default: hipLaunchKernelGGL((gemv_q8x4_kernel<PRO, EPI, SPLIT, KV, 8, A8>), dim3(grid), dim3(256), lds, s, a); break;
    }
    return hipGetLastError();
}

template <int PRO, int EPI, int KV, bool A8>
hipError_t launch_split(const GemvArgs &a, int split, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    // blocks per wave -> batch size (iterations of 4 blocks), one of 2, 3, 6, 8
    const int per = (a.cols / 32 + split - 1) / split;
    const int its = (per + 3) / 4;
    const int nbatch = its <= 2 ? 2 : its <= 3 ? 3 : its <= 6 ? 6 : 8;
    switch (split) {
        case 4: return launch_nb<PRO, EPI, 4, KV, A8>(a, nbatch, s);
        case 2: return launch_nb<PRO, EPI, 2, KV, A8>(a, nbatch, s);
        default: return launch_nb<PRO, EPI, 1, KV, A8>(a, nbatch, s);
    }
}

// ---- large-N streaming GEMV: weights stream HBM -> LDS by direct DMA
// (global_load_lds_dwordx4), several units in flight per wave.
//
// A unit is 24 consecutive blocks (3264 contiguous bytes) of one 4-row group:
// the whole group at K = 768, one of P = nb / 24 slices at K = 1536 / 3072
// (the wave accumulates a group's slices one after the other, so no
// cross-wave reduction is needed).  Each wave owns a ring of kStreamStages LDS
// slots; a unit takes 4 DMA instructions of 64 x 16 B (the 4th has 12 active
// lanes), so a wave keeps kStreamStages - 1 units in flight without holding
// them in registers.  The math from LDS is the register kernel's: lane
// 16*bl + 4*k + j takes qword j of row k of block 4*it + bl.
constexpr int kUnitBlocks = 24;
constexpr int kUnitBytes = kUnitBlocks * kBlockBytes;  // 3264
constexpr int kUnitChunks = kUnitBytes / 16;           // 204 = 3 x 64 + 12
#ifndef MH_STREAM_STAGES
#define MH_STREAM_STAGES 2
#endif
#ifndef MH_STREAM_WG_PER_CU
#define MH_STREAM_WG_PER_CU 4
#endif
// 2 slots x 4 waves x 3264 B + the activation: four workgroups per CU (16
// waves) measured 74-75 % of 8 TB/s cold, against 70-71 % for three slots with
// three workgroups and 68-73 % for the other ring/occupancy pairs tried
constexpr int kStreamStages = MH_STREAM_STAGES;

// s_waitcnt with only the vector-memory count constrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

#ifndef MH_STREAM_CPOL
#define MH_STREAM_CPOL 2  // non-temporal: the weights are read once per pass
#endif
__device__ __forceinline__ void issue_unit(const uint8_t *src, uint8_t *slot, int lane) {
#pragma unroll
    for (int i = 0; i < 3; ++i)
        __builtin_amdgcn_global_load_lds((const void *)(src + 16 * (64 * i + lane)), (lds_ptr)(slot + 1024 * i), 16,
                                         0, MH_STREAM_CPOL);
    if (lane < kUnitChunks - 192)
        __builtin_amdgcn_global_load_lds((const void *)(src + 16 * (192 + lane)), (lds_ptr)(slot + 3072), 16, 0,
                                         MH_STREAM_CPOL);
}

// Partial dot of one unit (24 blocks x 4 rows) from LDS (A8: ds = the unit's block scales).
template <bool A8>
__device__ __forceinline__ float unit_dot(const uint8_t *slot, const float *xs, int bl, int u, int kk, int j,
                                          float acc, const float *ds) {
#pragma unroll
    for (int it = 0; it < kUnitBlocks / 4; ++it) {
        const int b = 4 * it + bl;
        const uint8_t *blk = slot + b * kBlockBytes;
        const uint2 q = *(const uint2 *)(blk + 8 + 8 * u);
        const float d = h2f(*(const uint16_t *)(blk + 2 * kk));
        const float4 x0 = *(const float4 *)(xs + b * 32 + 8 * j);
        const float4 x1 = *(const float4 *)(xs + b * 32 + 8 * j + 4);
        float sm = (float)(int8_t)(q.x) * x0.x;
        sm = fmaf((float)(int8_t)(q.x >> 8), x0.y, sm);
        sm = fmaf((float)(int8_t)(q.x >> 16), x0.z, sm);
        sm = fmaf((float)(int8_t)(q.x >> 24), x0.w, sm);
        sm = fmaf((float)(int8_t)(q.y), x1.x, sm);
        sm = fmaf((float)(int8_t)(q.y >> 8), x1.y, sm);
        sm = fmaf((float)(int8_t)(q.y >> 16), x1.z, sm);
        sm = fmaf((float)(int8_t)(q.y >> 24), x1.w, sm);
        if constexpr (A8) {
            const float scale = d * ds[b];
            acc = fmaf(sm, scale, acc);
        } else {
            acc = fmaf(sm, d, acc);
        }
    }
    return acc;
}

// One step of a wave's stream: refill `refill` (the slot consumed last step)
// with unit t + stages - 1, wait for unit t in `cur`, accumulate it, and on a
// group's last slice reduce and store.  The restrict-qualified slots let the
// compiler keep the DMA into `refill` in flight while it reads `cur`.
template <int EPI, int KV, bool A8>
__device__ __forceinline__ void stream_step(const GemvArgs &a, const float *act, const float *da, int t, int units, int P,
                                            const uint8_t *next_src, uint8_t *__restrict__ refill,
                                            const uint8_t *__restrict__ cur, int g, int ngroups, float &acc) {
    const int lane = threadIdx.x & 63;
    const int bl = lane >> 4, u = lane & 15, kk = u >> 2, j = u & 3;
    if (t + kStreamStages - 1 < units) {
        issue_unit(next_src, refill, lane);
        wait_vmcnt<4 * (kStreamStages - 1)>();
    } else {
        wait_vmcnt<0>();
    }
    const int slice = t % P;
    acc = unit_dot<A8>(cur, act + slice * kUnitBlocks * 32, bl, u, kk, j, acc, da + slice * kUnitBlocks);
    if (slice == P - 1) {
        float yv = acc;
        yv = row_lane_sum(yv);
        const float partner = xshfl<4>(yv);
        if (g < ngroups && lane < 16 && j == 0) finish_row<EPI, KV>(a, 4 * g + kk, yv, partner);
        acc = 0.0f;
    }
}

template <int PRO, int EPI, int KV, bool A8>
__global__ __launch_bounds__(256) void gemv_stream_kernel(GemvArgs a) {
    constexpr int S = kStreamStages;
    __shared__ __attribute__((aligned(16))) uint8_t ring[S][4][kUnitBytes];
    extern __shared__ float act[];
    __shared__ float red[4];
    __shared__ float da[4096 / 32];  // block scales of act (A8)
    if (a.state != nullptr && a.state->stop) return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nb = a.cols >> 5;
    const int P = nb / kUnitBlocks;
    const int ngroups = a.rows >> 2;
    const int gfirst = blockIdx.x * 4 + wave, gstride = gridDim.x * 4;
    // units per wave, uniform over the workgroup (a wave past the end repeats a valid unit and stores nothing)
    const int units = P * ((ngroups - blockIdx.x * 4 + gstride - 1) / gstride);
    auto src = [&](int t) {
        const int g = min(gfirst + (t / P) * gstride, ngroups - 1);
        return a.w + ((size_t)g * nb + (t % P) * kUnitBlocks) * kBlockBytes;
    };
#pragma unroll
    for (int t = 0; t < S - 1; ++t) issue_unit(src(t), ring[t][wave], lane);

    stage_activation<PRO>(a, act, red);
    __syncthreads();
    if constexpr (A8) {
        quant_act_lds(act, da, a.cols);
        __syncthreads();
    }

    float acc = 0.0f;
    // unrolled by the ring size so every step names its two slots statically
    for (int t = 0; t < units; t += S) {
#pragma unroll
        for (int r = 0; r < S; ++r) {
            if (t + r >= units) break;
            stream_step<EPI, KV, A8>(a, act, da, t + r, units, P, src(t + r + S - 1), ring[(r + S - 1) % S][wave],
                                 ring[r][wave], gfirst + ((t + r) / P) * gstride, ngroups, acc);
        }
    }
}

template <int PRO, int EPI, int KV, bool A8>
hipError_t launch_stream(const GemvArgs &a, hipStream_t s) {
    const int ngroups = a.rows / 4;
    const size_t lds = (size_t)a.cols * sizeof(float);
    int grid = (ngroups + 3) / 4;
    grid = grid > 256 * MH_STREAM_WG_PER_CU ? 256 * MH_STREAM_WG_PER_CU : grid;  // MH_STREAM_WG_PER_CU 4-wave workgroups per CU
    hipLaunchKernelGGL((gemv_stream_kernel<PRO, EPI, KV, A8>), dim3(grid), dim3(256), lds, s, a);
    return hipGetLastError();
}

// The streaming kernel serves large N at K = 768, 1536 or 3072.
bool use_stream(int rows, int cols) {
    const int nb = cols / 32;
    return rows / 4 >= 2048 && (nb == 24 || nb == 48 || nb == 96);
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
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (a.rows % 4 != 0 || a.cols % 128 != 0 || a.cols > 4096 || a.rows <= 0) return hipErrorInvalidValue;
    if ((pro == PRO_LN || pro == PRO_LATTN || pro == PRO_AMERGE || pro == PRO_PICK) && a.cols != kHidden)
        return hipErrorInvalidValue;
    if (pro == PRO_PICK && (!a.pick_logits || !a.pick_counts || !a.pick_aemb || !a.pick_forced || !a.pick_state ||
                            !a.pick_raw || a.pick_ch < 0 || a.pick_ch >= kNVq))
        return hipErrorInvalidValue;
    if (pro == PRO_LATTN && (!a.k_cache || !a.v_cache || a.ctx_stride < kLocalLen)) return hipErrorInvalidValue;
    if (pro == PRO_AMERGE && (!a.attn_part || a.attn_splits <= 0 || a.attn_splits > kMaxMergeSplits))
        return hipErrorInvalidValue;
    if (epi == EPI_QKV && a.rows != 3 * kHidden) return hipErrorInvalidValue;
    if (a.a8 && a.cols % 256 != 0) return hipErrorInvalidValue;  // quant_act_lds: whole waves per block
    const int split = pick_split(a.rows, a.cols);
    const bool stream = use_stream(a.rows, a.cols);
#define MH_LAUNCH(P, E, A8)                                                                     \
    do {                                                                                        \
        if (stream) {                                                                           \
            if (E == EPI_QKV && kv == KV_F32) return launch_stream<P, E, KV_F32, A8>(a, s);    \
            return launch_stream<P, E, KV_F16, A8>(a, s);                                       \
        }                                                                                       \
        if (E == EPI_QKV && kv == KV_F32) return launch_split<P, E, KV_F32, A8>(a, split, s);  \
        return launch_split<P, E, KV_F16, A8>(a, split, s);                                     \
    } while (0)
// combinations served in W8A16 only
#define MH_CASE(P, E)                                                                           \
    if (pro == P && epi == E) {                                                                 \
        if (a.a8) return hipErrorInvalidValue;                                                  \
        MH_LAUNCH(P, E, false);                                                                 \
    }
// combinations served in W8A16 or W8A8 (the decode's, and the operator layer's fp32 GEMV)
#define MH_CASE_A8(P, E)                                                                        \
    if (pro == P && epi == E) {                                                                 \
        if (a.a8) MH_LAUNCH(P, E, true);                                                        \
        MH_LAUNCH(P, E, false);                                                                 \
    }
    MH_CASE_A8(PRO_F32, EPI_F32)
    MH_CASE(PRO_F16, EPI_F16)
    MH_CASE(PRO_F16, EPI_F32)
    MH_CASE(PRO_F32, EPI_F16)
    MH_CASE_A8(PRO_LN, EPI_QKV)
    MH_CASE_A8(PRO_LN, EPI_GELU)
    MH_CASE_A8(PRO_F32, EPI_RESID)
    MH_CASE_A8(PRO_LN, EPI_F32)
    MH_CASE_A8(PRO_LATTN, EPI_RESID)
    MH_CASE_A8(PRO_AMERGE, EPI_RESID)
    MH_CASE_A8(PRO_PICK, EPI_QKV)
#undef MH_CASE_A8
#undef MH_LAUNCH
#undef MH_CASE
    return hipErrorInvalidValue;
}

}  // namespace mh
