// attention.hip -- causal attention of query rows over a (paged) KV cache (gfx950).
//
// Replaces LlmModel::attention_core (reference csrc/src/llm.cpp:189-217):
// s_p = (q . k_p) * 0.125, softmax over the row's keys p < n, o = sum_p w_p v_p.
// One kernel serves the single-stream decode (one row), the prefill (row r of a
// prompt attends keys <= start + r) and batched decode (one row per stream,
// each over its own pages).
//
// KV pools are [page][head][page_size][64] (fp16 or fp32): within a page one
// head's keys are contiguous 128-byte (fp16) rows.  The single-stream cache is
// one page of max_ctx positions.
//
// One workgroup per (head, row) with NW wavefronts.  Keys are taken in spans of
// 64; each K load instruction brings 8 whole 128-byte rows (8 lanes per key),
// and the 8 lanes of a key combine their partial dots, so every lane ends with
// one key's score.  Wave w takes spans w, w+NW, ... with an
// online softmax across its spans; the waves are then merged through LDS with a
// log-sum-exp combine -- split-KV inside the workgroup, no cross-workgroup
// traffic.  Every K/V load is unconditional (rows past the live count are
// clamped to a live row and weighted 0), and a span's V values are loaded with
// its K rows, so all of a lane's loads for the span are in flight together.
#include "mh_ll.h"
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

template <int KV, int NW, bool PART, bool CHUNK = false>
__global__ __launch_bounds__(64 * NW) void attn_rows_kernel(AttnArgs a) {
    __shared__ float qs[kHeadDim];
    __shared__ float sc[NW][64];
    __shared__ float4 po[NW][16];
    __shared__ float pm[NW], pl[NW];
    const bool stopped = a.state != nullptr && a.state->stop;  // tested once q is loaded
    // PART: one 64-key span per workgroup (blockIdx.y), one row
    const int h = blockIdx.x, r = (PART || CHUNK) ? 0 : blockIdx.y, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int s = a.row_stream ? a.row_stream[r] : r * a.stream_stride;
    // keys of this row, never past the capacity the caches were built for (a
    // stream parked at capacity keeps pos == capacity)
    const int n = min((a.row_pos ? a.row_pos[r] : a.pos0 + r * a.pos_stride) + 1, a.max_keys);
    if (threadIdx.x < kHeadDim) qs[threadIdx.x] = a.q[(size_t)r * a.q_stride + h * kHeadDim + threadIdx.x];
    __syncthreads();
    if (stopped) return;

    float m = -INFINITY, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    const int pg = lane >> 4, dg = lane & 15;
    // K: load c brings 16 bytes of key RPI*c + rr (dims sub*EPL ..), so one load
    // instruction covers RPI whole rows; the LPR lanes of a key then combine
    // their partial dots, and lane ends with the score of key kl of the span
    constexpr int LPR = KV == KV_F16 ? 8 : 16, EPL = 64 / LPR, RPI = 64 / LPR;
    const int sub = lane & (LPR - 1), rr = lane / LPR, kl = RPI * sub + rr;
    float qsub[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) qsub[e] = qs[sub * EPL + e];
    // PART: exactly one span, [64 * blockIdx.y, min(n, 64 * blockIdx.y + 64));
    // CHUNK: workgroup y takes spans NW*y + w, then every NW*chunks further
    const int span0 = PART ? (int)blockIdx.y : (CHUNK ? NW * (int)blockIdx.y + w : w);
    const int span_step = PART ? 1 : (CHUNK ? NW * (int)gridDim.y : NW);
    const int key_end = PART ? min(n, span0 * 64 + 64) : n;
    if (PART && span0 * 64 >= n) return;  // a span past the live keys: the merge skips it
    for (int span = span0; span * 64 < key_end; span += span_step) {
        const int p0 = span * 64;
        const int cnt = min(64, n - p0);
        const int page = a.page_table ? a.page_table[(size_t)s * a.table_stride + p0 / a.page_size] : s;
        const size_t base = (((size_t)page * a.heads + h) * a.page_size + p0 % a.page_size) * kHeadDim;
        // V values of this lane (dims 4dg..4dg+3 of keys pg + 4t) are loaded with K,
        // before the scores need to be ready
        float4 vv[16];
#pragma unroll
        for (int t = 0; t < 16; ++t)
            vv[t] = load4<KV>(a.v_pool, base + (size_t)min(pg + 4 * t, cnt - 1) * kHeadDim + 4 * dg);
        float pd[LPR];
#pragma unroll
        for (int c = 0; c < LPR; ++c) {
            const size_t ki = base + (size_t)min(RPI * c + rr, cnt - 1) * kHeadDim + sub * EPL;
            float kf[EPL];
            if constexpr (KV == KV_F16) {
                float tmp[8];
                load_row8<KV>(a.k_pool, ki, tmp);
#pragma unroll
                for (int e = 0; e < EPL; ++e) kf[e] = tmp[e];
            } else {
                const float4 v4 = *(const float4 *)((const float *)a.k_pool + ki);
                kf[0] = v4.x; kf[1] = v4.y; kf[2] = v4.z; kf[3] = v4.w;
            }
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) d = fmaf(qsub[e], kf[e], d);
            pd[c] = d;
        }
        float dot = key_reduce<LPR>(pd, sub);  // q . k of key kl
        dot *= 0.125f;  // 1/sqrt(64), applied after the dot as llm.cpp:200 does
        const float smax = wave_max(kl < cnt ? dot : -INFINITY);
        const float m_new = fmaxf(m, smax);
        const float rescale = expf(m - m_new);  // 0 on the first span (m = -inf)
        const float e = kl < cnt ? expf(dot - m_new) : 0.0f;
        l = l * rescale + wave_sum(e);
        m = m_new;
        o.x *= rescale;
        o.y *= rescale;
        o.z *= rescale;
        o.w *= rescale;
        sc[w][kl] = e;
        // sc[w][*] is written and read by different lanes of this one wave
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        // o[d] += sum_p e_p v_p[d]: lane = 16*pg + dg covers dims 4dg..4dg+3 of every 4th key
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const int i = pg + 4 * t;
            const float4 v = vv[t];
            const float ei = sc[w][i];
            o.x = fmaf(ei, v.x, o.x);
            o.y = fmaf(ei, v.y, o.y);
            o.z = fmaf(ei, v.z, o.z);
            o.w = fmaf(ei, v.w, o.w);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    o.x += xshfl<16>(o.x);
    o.y += xshfl<16>(o.y);
    o.z += xshfl<16>(o.z);
    o.w += xshfl<16>(o.w);
    o.x += xshfl<32>(o.x);
    o.y += xshfl<32>(o.y);
    o.z += xshfl<32>(o.z);
    o.w += xshfl<32>(o.w);
    if constexpr (PART) {
        float *pp = a.part + ((size_t)h * gridDim.y + blockIdx.y) * kPartStride;
        if (lane < 16) *(float4 *)(pp + 4 * dg) = o;
        if (lane == 0) {
            pp[64] = m;
            pp[65] = l;
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
    // log-sum-exp merge of the waves that saw keys; lane = output dimension
    const int live = CHUNK ? min(NW, (n + 63) / 64 - NW * (int)blockIdx.y) : min(NW, (n + 63) / 64);
    float M = -INFINITY;
    for (int t = 0; t < live; ++t) M = fmaxf(M, pm[t]);
    float L = 0.0f, O = 0.0f;
    for (int t = 0; t < live; ++t) {
        const float sw = expf(pm[t] - M);
        L = fmaf(pl[t], sw, L);
        O = fmaf(((const float *)&po[t][0])[lane], sw, O);
    }
    if constexpr (CHUNK) {
        // this slice's partial as LL words, then the last slice of the head to
        // arrive collects every partial (each word carries its own flag) and merges
        uint64_t *pp = a.chunk_part + ((size_t)h * gridDim.y + blockIdx.y) * kPartStride;
        ll_put(pp + lane, O, a.chunk_tag);
        if (lane == 0) {
            ll_put(pp + 64, M, a.chunk_tag);
            ll_put(pp + 65, L, a.chunk_tag);
        }
        unsigned prev = 0;
        if (lane == 0) prev = atomicAdd(a.chunk_count + h, 1u);
        prev = __shfl(prev, 0);
        if (prev + 1 != gridDim.y) return;
        const uint64_t *hp = a.chunk_part + (size_t)h * gridDim.y * kPartStride;
        int budget = kPollBudget;
        bool ok = true;
        auto word = [&](size_t i) {  // waits for the word's tag (bounded)
            uint64_t v = ll_load(hp + i);
            while ((uint32_t)(v >> 32) != a.chunk_tag) {
                if (--budget < 0) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
                v = ll_load(hp + i);
            }
            return __uint_as_float((uint32_t)v);
        };
        M = -INFINITY;
        for (unsigned c = 0; c < gridDim.y; ++c) M = fmaxf(M, word(c * kPartStride + 64));
        L = 0.0f;
        O = 0.0f;
        for (unsigned c = 0; c < gridDim.y; ++c) {
            const float sw = expf(word(c * kPartStride + 64) - M);
            L = fmaf(word(c * kPartStride + 65), sw, L);
            O = fmaf(word(c * kPartStride + lane), sw, O);
        }
        if (!ok) O = __int_as_float(0x7fc00000);  // a slice never arrived: NaN, not a stale value
        if (lane == 0) a.chunk_count[h] = 0;       // ready for the next launch on this stream
    }
    const float res = O / L;
    const size_t oi = (size_t)r * a.out_stride + h * kHeadDim + lane;
    if (a.out_f16)
        ((__half *)a.out)[oi] = __float2half_rn(res);
    else
        ((float *)a.out)[oi] = res;
    if (a.q8 != nullptr) {  // W8A8 copy for the proj GEMM: this head's 64 outputs are two blocks
        float d;
        const int q = quant_block32(res, &d);
        a.q8[(size_t)r * kHidden + h * kHeadDim + lane] = (int8_t)q;
        if ((lane & 31) == 0) a.d8[(size_t)r * (kHidden / 32) + 2 * h + (lane >> 5)] = d;
    }
}

template <int KV>
hipError_t launch_kv(const AttnArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    // waves per workgroup from the key capacity the launch is sized for (fixed
    // for a captured graph): one wave per 64 keys up to 4 waves, which then take
    // several spans each (measured faster than 8 or 16 waves at 64 streams x ~540 keys)
    const int spans = (a.max_keys + 63) / 64;
    if (a.part != nullptr) {  // split-KV: one single-wave workgroup per (head, span)
        hipLaunchKernelGGL((attn_rows_kernel<KV, 1, true>), dim3(a.heads, spans), dim3(64), 0, s, a);
        return hipGetLastError();
    }
    if (a.chunks > 0) {  // one row, slices of 4 spans merged by the last slice of each head
        hipLaunchKernelGGL((attn_rows_kernel<KV, 4, false, true>), dim3(a.heads, a.chunks), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const dim3 grid(a.heads, a.rows);
    if (spans <= 1)
        hipLaunchKernelGGL((attn_rows_kernel<KV, 1, false>), grid, dim3(64), 0, s, a);
    else
        hipLaunchKernelGGL((attn_rows_kernel<KV, 4, false>), grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_attn(const AttnArgs &a, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (a.heads <= 0 || a.rows <= 0 || a.max_keys <= 0 || a.page_size <= 0 || (!a.out && !a.part) || !a.q ||
        !a.k_pool || !a.v_pool)
        return hipErrorInvalidValue;
    if (a.part != nullptr && (a.rows != 1 || a.page_table != nullptr)) return hipErrorInvalidValue;
    if (a.q8 != nullptr && (!a.d8 || a.part != nullptr || a.heads != kHeads)) return hipErrorInvalidValue;
    if (a.chunks != 0 && (a.chunks < 0 || a.chunks > kMaxChunks || a.rows != 1 || a.part != nullptr ||
                          a.page_table != nullptr || a.q8 != nullptr || !a.chunk_part || !a.chunk_count ||
                          4 * 64 * (a.chunks - 1) >= a.max_keys))
        return hipErrorInvalidValue;  // every slice holds at least one live span
    return kv == KV_F16 ? launch_kv<KV_F16>(a, s) : launch_kv<KV_F32>(a, s);
}

}  // namespace mh
