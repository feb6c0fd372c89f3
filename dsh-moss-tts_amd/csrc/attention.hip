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
// its K rows, so all of a lane's loads for the span are in flight together; the
// first span is requested before q.
#include <type_traits>

#include "mh_ll.h"
#include "mh_ops.h"

namespace mh {
namespace {

// The raw K and V of one 64-key span as one lane holds them: K load c brings 16
// bytes (dims sub*EPL..) of key RPI*c + rr, V load t the dims 4dg..4dg+3 of key
// pg + 4t.  Rows past the span's live count are clamped to its last live row.
template <int KV>
struct SpanRaw {
    static constexpr int LPR = KV == KV_F16 ? 8 : 16, EPL = 64 / LPR, RPI = 64 / LPR;
    using VT = typename std::conditional<KV == KV_F16, uint2, uint4>::type;
    uint4 k[LPR];
    VT v[16];

    // NT: read the span non-temporally.  The batch engine's paged global caches (fp16:
    // 1.3 GB at 64 streams x ~540 keys) stream through once per frame, and keeping them
    // out of the caches' way measured 50.2k -> 53.4k frames/s (the attention itself 27.9
    // -> 25.8 us per layer).  A single stream's caches stay cache-resident from step to
    // step and load normally (non-temporal loads in the fused global step measured 0.177
    // -> 0.195 ms), as do the small fp32 local caches, re-read at every local position.
    template <bool NT>
    __device__ __forceinline__ void load(const void *k_pool, const void *v_pool, size_t base, int cnt, int sub,
                                         int rr, int pg, int dg) {
        // base and cnt are wave-uniform: a scalar base plus 32-bit lane offsets
        constexpr unsigned esz = KV == KV_F16 ? 2 : 4;
        const char *kb = (const char *)k_pool + base * esz, *vb = (const char *)v_pool + base * esz;
        typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
        typedef unsigned u32xv __attribute__((ext_vector_type(sizeof(VT) / 4)));
#pragma unroll
        for (int c = 0; c < LPR; ++c) {
            const u32x4 *p = (const u32x4 *)(kb + (unsigned)(min(RPI * c + rr, cnt - 1) * kHeadDim + sub * EPL) * esz);
            const u32x4 x = NT ? __builtin_nontemporal_load(p) : *p;
            k[c] = make_uint4(x.x, x.y, x.z, x.w);
        }
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const u32xv *p = (const u32xv *)(vb + (unsigned)(min(pg + 4 * t, cnt - 1) * kHeadDim + 4 * dg) * esz);
            const u32xv x = NT ? __builtin_nontemporal_load(p) : *p;
            __builtin_memcpy(&v[t], &x, sizeof(VT));
        }
    }
    __device__ __forceinline__ float4 vf(int t) const {
        if constexpr (KV == KV_F16) {
            const __half2 *hh = (const __half2 *)&v[t];
            const float2 x = __half22float2(hh[0]), y = __half22float2(hh[1]);
            return make_float4(x.x, x.y, y.x, y.y);
        } else {
            return make_float4(__uint_as_float(v[t].x), __uint_as_float(v[t].y), __uint_as_float(v[t].z),
                               __uint_as_float(v[t].w));
        }
    }
    // this lane's part of q . k for K load c
    __device__ __forceinline__ float kdot(int c, const float (&qsub)[EPL]) const {
        float kf[EPL];
        if constexpr (KV == KV_F16) {
            const __half2 *hh = (const __half2 *)&k[c];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 t = __half22float2(hh[i]);
                kf[2 * i] = t.x;
                kf[2 * i + 1] = t.y;
            }
        } else {
            kf[0] = __uint_as_float(k[c].x);
            kf[1] = __uint_as_float(k[c].y);
            kf[2] = __uint_as_float(k[c].z);
            kf[3] = __uint_as_float(k[c].w);
        }
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) d = fmaf(qsub[e], kf[e], d);
        return d;
    }
};

// NT: the K/V spans are read non-temporally (the batch engine's paged caches)
template <int KV, int NW, bool PART, bool CHUNK = false, bool NT = false>
__global__ __launch_bounds__(64 * NW) void attn_rows_kernel(AttnArgs a) {
    // a span's softmax weights, key k at (k % 4) * 16 + k / 4: the 16 keys pg + 4t a lane's
    // value pass takes are then 16 consecutive floats (four 16-byte LDS reads)
    __shared__ __attribute__((aligned(16))) float sc[NW][64];
    __shared__ float4 po[NW][16];
    __shared__ float pm[NW], pl[NW];
    // PART: one 64-key span per workgroup (blockIdx.y), one row
    // w is wave-uniform; saying so keeps span bases in SGPRs (loads then take a
    // scalar base and a 32-bit lane offset)
    const int h = blockIdx.x, lane = threadIdx.x & 63;
    const int r = (PART || CHUNK) ? 0
                                  : __builtin_amdgcn_readfirstlane(a.row_order ? a.row_order[blockIdx.y] : (int)blockIdx.y);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int s = __builtin_amdgcn_readfirstlane(a.row_stream ? a.row_stream[r] : r * a.stream_stride);
    // keys of this row, never past the capacity the caches were built for (a
    // stream parked at capacity keeps pos == capacity)
    const int n = __builtin_amdgcn_readfirstlane(
        min((a.row_pos ? a.row_pos[r] : a.pos0 + r * a.pos_stride) + 1, a.max_keys));

    using Raw = SpanRaw<KV>;
    constexpr int LPR = Raw::LPR, EPL = Raw::EPL, RPI = Raw::RPI;
    const int pg = lane >> 4, dg = lane & 15;
    const int sub = lane & (LPR - 1), rr = lane / LPR, kl = RPI * sub + rr;
    // PART: exactly one span, [64 * blockIdx.y, min(n, 64 * blockIdx.y + 64));
    // CHUNK: workgroup y takes spans NW*y + w, then every NW*chunks further
    const int span0 = PART ? (int)blockIdx.y : (CHUNK ? NW * (int)blockIdx.y + w : w);
    const int span_step = PART ? 1 : (CHUNK ? NW * (int)gridDim.y : NW);
    const int key_end = PART ? min(n, span0 * 64 + 64) : n;
    if (PART && span0 * 64 >= n) return;  // a span past the live keys: the merge skips it
    auto span_base = [&](int span) -> size_t {
        const int p0 = span * 64;
        const int page = __builtin_amdgcn_readfirstlane(
            a.page_table ? a.page_table[(size_t)s * a.table_stride + p0 / a.page_size] : s);
        return (((size_t)page * a.heads + h) * a.page_size + p0 % a.page_size) * kHeadDim;
    };
    // the launch's LL tag (sliced single-row launches): odd, so never the 0 of a cleared word
    uint32_t tag = 0;
    if constexpr (CHUNK) tag = (ll_gen_load(a.chunk_gen) << 1) | 1u;
    float m = -INFINITY, l = 0.0f;
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
    // q goes straight into registers (no LDS, no barrier), requested right after
    // the first span's K and V so that the two latencies overlap (a wave without
    // a span never needs it)
    float qsub[EPL];
    bool need_q = true;
#pragma unroll 1
    for (int span = span0; span * 64 < key_end; span += span_step) {
        const int cnt = min(64, n - span * 64);
        Raw raw;
        raw.template load<NT>(a.k_pool, a.v_pool, span_base(span), cnt, sub, rr, pg, dg);
        if (need_q) {
            const float4 *qp = (const float4 *)(a.q + (size_t)r * a.q_stride + h * kHeadDim + sub * EPL);
#pragma unroll
            for (int e = 0; e < EPL / 4; ++e) {
                const float4 t = qp[e];
                qsub[4 * e] = t.x;
                qsub[4 * e + 1] = t.y;
                qsub[4 * e + 2] = t.z;
                qsub[4 * e + 3] = t.w;
            }
            need_q = false;
        }
        float pd[LPR];
#pragma unroll
        for (int c = 0; c < LPR; ++c) pd[c] = raw.kdot(c, qsub);
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
        sc[w][(kl & 3) * 16 + (kl >> 2)] = e;
        // sc[w][*] is written and read by different lanes of this one wave
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        float ev[16];
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) *(float4 *)&ev[4 * t4] = *(const float4 *)&sc[w][pg * 16 + 4 * t4];
        // o[d] += sum_p e_p v_p[d]: lane = 16*pg + dg covers dims 4dg..4dg+3 of every 4th key
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float4 v = raw.vf(t);
            const float ei = ev[t];
            o.x = fmaf(ei, v.x, o.x);
            o.y = fmaf(ei, v.y, o.y);
            o.z = fmaf(ei, v.z, o.z);
            o.w = fmaf(ei, v.w, o.w);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    // a stopped stream writes nothing (the flag is the same for every wave of
    // the launch; it is tested here, off the path of the loads)
    if (a.state != nullptr && a.state->stop) return;
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
        // slices 1.. hand their partial on as LL words; slice 0 of the head (the
        // first dispatched) keeps its own in registers and merges the others as
        // their words arrive (each word carries the launch's tag: no counter)
        if (blockIdx.y != 0) {
            uint64_t *pp = a.chunk_part + ((size_t)h * gridDim.y + blockIdx.y) * kPartStride;
            ll_put(pp + lane, O, tag);
            if (lane == 0) {
                ll_put(pp + 64, M, tag);
                ll_put(pp + 65, L, tag);
                ll_gen_arrive(a.chunk_gen, gridDim.x * gridDim.y);
            }
            return;
        }
        // every load of the merge is issued before any is waited on: lane c holds
        // slice c's (m, l) (lane 0 its own); each lane then sums its output
        // dimension over the slices in slice order, 16 slices' words in flight
        // (polling (m, l) alone first measured faster than polling every word)
        const uint64_t *hp = a.chunk_part + (size_t)h * gridDim.y * kPartStride;
        const int nc = (int)gridDim.y;  // <= kMaxChunks = 64
        int budget = kPollBudget;
        bool ok = true;
        float mc = M, lc = L;
        if (lane > 0 && lane < nc) {
            uint64_t wm = ll_load(hp + (size_t)lane * kPartStride + 64);
            uint64_t wl = ll_load(hp + (size_t)lane * kPartStride + 65);
            while ((uint32_t)(wm >> 32) != tag || (uint32_t)(wl >> 32) != tag) {
                if (--budget < 0) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(kPollSleep);
                wm = ll_load(hp + (size_t)lane * kPartStride + 64);
                wl = ll_load(hp + (size_t)lane * kPartStride + 65);
            }
            mc = __uint_as_float((uint32_t)wm);
            lc = __uint_as_float((uint32_t)wl);
        } else if (lane >= nc) {
            mc = -INFINITY;
            lc = 0.0f;
        }
        M = wave_max(mc);
        const float sw = lane < nc ? expf(mc - M) : 0.0f;
        L = 0.0f;
        for (int c = 0; c < nc; ++c) L = fmaf(__shfl(lc, c), __shfl(sw, c), L);
        O *= __shfl(sw, 0);  // slice 0's own
        for (int c0 = 1; c0 < nc; c0 += 16) {
            uint64_t v[16];
            uint32_t pending = 0;
#pragma unroll
            for (int k = 0; k < 16; ++k)  // only slices that exist (uniform test)
                if (c0 + k < nc) {
                    v[k] = ll_load(hp + (size_t)(c0 + k) * kPartStride + lane);
                    pending |= 1u << k;
                }
            while (true) {
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if (((pending >> k) & 1u) && (uint32_t)(v[k] >> 32) == tag) pending &= ~(1u << k);
                if (pending == 0) break;
                if (--budget < 0) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(kPollSleep);
#pragma unroll
                for (int k = 0; k < 16; ++k)
                    if ((pending >> k) & 1u) v[k] = ll_load(hp + (size_t)(c0 + k) * kPartStride + lane);
            }
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (c0 + k < nc) O = fmaf(__uint_as_float((uint32_t)v[k]), __shfl(sw, c0 + k), O);
        }
        // clear every word read (tag 0 is never current), so that no word keeps a
        // tag for the 2^31 launches after which the generation's tags repeat
        for (int c = 1; c < nc; ++c) ll_put((uint64_t *)hp + (size_t)c * kPartStride + lane, 0.0f, 0);
        if (lane > 0 && lane < nc) {
            ll_put((uint64_t *)hp + (size_t)lane * kPartStride + 64, 0.0f, 0);
            ll_put((uint64_t *)hp + (size_t)lane * kPartStride + 65, 0.0f, 0);
        }
        if (lane == 0) ll_gen_arrive(a.chunk_gen, gridDim.x * gridDim.y);
        ok = __all(ok);
        if (!ok) O = __int_as_float(0x7fc00000);  // a slice never arrived: NaN, not a stale value
    }
    const float res = O / L;
    const size_t oi = (size_t)r * a.out_stride + h * kHeadDim + lane;
    if (a.out_hl != nullptr)  // for the next GEMM: hi / lo halves in the matrix-core order
        store_hl(a.out_hl, r, h * kHeadDim + lane, kHidden, res);
    else if (a.out == nullptr)
        ;  // only the W8A8 copy below is read
    else if (a.out_f16)
        ((__half *)a.out)[oi] = __float2half_rn(res);
    else
        ((float *)a.out)[oi] = res;
    if (a.q8 != nullptr) {  // W8A8 copy for the proj GEMM: this head's 64 outputs are two blocks
        float d;
        const int q = quant_block32(res, &d);
        a.q8[q8t_at(r, h * kHeadDim + lane, kHidden)] = (int8_t)q;
        if ((lane & 31) == 0) a.d8[d8t_at(r, 2 * h + (lane >> 5), kHidden)] = d;
    }
}

template <int KV>
hipError_t launch_kv(const AttnArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    // waves per workgroup from the key capacity the launch is sized for (fixed
    // for a captured graph): one wave up to 64 keys, else 2 waves taking every
    // other span (at 64 streams x ~540 keys: 47.9k frames/s against 47.6k with
    // 4 waves; 8 or 16 waves measured slower still)
    const int spans = (a.max_keys + 63) / 64;
    if (a.part != nullptr) {  // split-KV: one single-wave workgroup per (head, span)
        hipLaunchKernelGGL((attn_rows_kernel<KV, 1, true>), dim3(a.heads, spans), dim3(64), 0, s, a);
        return hipGetLastError();
    }
    if (a.chunks > 0) {  // one row, slices of 4 spans merged by the last slice of each head
        if (a.chunk_waves == 2)
            hipLaunchKernelGGL((attn_rows_kernel<KV, 2, false, true>), dim3(a.heads, a.chunks), dim3(128), 0, s, a);
        else
            hipLaunchKernelGGL((attn_rows_kernel<KV, 4, false, true>), dim3(a.heads, a.chunks), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    const dim3 grid(a.heads, a.rows);
    if (a.rows == 1 && a.page_table == nullptr && spans > 2) {
        // one query row (the single-query operator): one workgroup per head, a wave per
        // 64-key span (every K/V load in flight at once), merged in LDS -- no hand-off
        // between workgroups; fp32 caches at most 8 waves (their span needs ~170 VGPRs)
        if (spans <= 4)
            hipLaunchKernelGGL((attn_rows_kernel<KV, 4, false>), grid, dim3(256), 0, s, a);
        else if (KV == KV_F32 || spans <= 8)
            hipLaunchKernelGGL((attn_rows_kernel<KV, 8, false>), grid, dim3(512), 0, s, a);
        else
            hipLaunchKernelGGL((attn_rows_kernel<KV, KV == KV_F16 ? 16 : 8, false>), grid, dim3(KV == KV_F16 ? 1024 : 512), 0,
                               s, a);
        return hipGetLastError();
    }
    if (spans <= 1)
        hipLaunchKernelGGL((attn_rows_kernel<KV, 1, false>), grid, dim3(64), 0, s, a);
    else if (KV == KV_F16 && a.page_table != nullptr)  // the batch engine's paged fp16 caches
        hipLaunchKernelGGL((attn_rows_kernel<KV, 2, false, false, KV == KV_F16>), grid, dim3(128), 0, s, a);
    else
        hipLaunchKernelGGL((attn_rows_kernel<KV, 2, false>), grid, dim3(128), 0, s, a);
    return hipGetLastError();
}

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma_f32x4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Causal attention of 16 consecutive prompt rows x one head on the matrix cores (the
// prefill: row r at position pos0 + r attends keys 0 .. pos0 + r of one cache page,
// llm.cpp:349-392 over attention_core, llm.cpp:189-217).  Each of the 4 waves takes every
// 4th block of 16 keys with an online softmax, fp32 on v_mfma_f32_16x16x4_f32 (K/V widened
// from the cache's fp16 exactly):
//   S^T = K Q^T: A = K[key kb + l%16][16g + t], B = Q[row l%16][16g + t], t = 0..15
//   O^T = V^T P^T per column group j: A = V[key kb + 4g + s][4(l%16) + j], B = P[row][kb + 4g + s]
// so the lane with row l%16 holds S^T for keys kb + 4g + i and O for columns 16g..16g+15
// (g = l/16).  The waves merge through LDS; the output is normalised (and, under W8A8,
// quantised per 32-block as quant_block32 does) and written as the row-per-workgroup kernel
// writes it -- or, in the prefill (proj_part), multiplied by the head's 64 columns of proj
// on the matrix cores (int8 under W8A8, fp16 hi / lo otherwise, the proj GEMM's per-block
// arithmetic) and written as split-K partial h: one launch fewer per layer (the tile's
// kernel time grows 9.7 -> 14.3 us against the 6.1 us proj GEMM it replaces).
template <int KV>
__global__ __launch_bounds__(256) void attn_tile_kernel(const AttnArgs a) {
    __shared__ float red[4][16 * 64 + 32];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, col = lane & 15, grp = lane >> 4;
    const int m0 = blockIdx.x * 16, h = blockIdx.y;
    const int mlast = min(m0 + 15, a.rows - 1);
    const int nkeys = min(a.pos0 + mlast + 1, a.max_keys);  // keys of the tile's last row
    const int nkb = (nkeys + 15) >> 4;
    const int mq = m0 + col, qpos = a.pos0 + mq;
    const bool qvalid = mq < a.rows;
    constexpr unsigned esz = KV == KV_F16 ? 2 : 4;
    const char *kbase = (const char *)a.k_pool + (size_t)h * a.page_size * kHeadDim * esz;
    const char *vbase = (const char *)a.v_pool + (size_t)h * a.page_size * kHeadDim * esz;

    float qv[16];
    {
        const float4 *src = reinterpret_cast<const float4 *>(a.q + (size_t)(qvalid ? mq : 0) * a.q_stride + h * kHeadDim + 16 * grp);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float4 v = qvalid ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            qv[4 * i] = v.x;
            qv[4 * i + 1] = v.y;
            qv[4 * i + 2] = v.z;
            qv[4 * i + 3] = v.w;
        }
    }
    // block b: this lane's 16 K dims of key kb + col, and 4 V dims of keys kb + 4g + s;
    // keys past nkeys read the last key (their scores are masked)
    auto load_block = [&](int b, float (&kv)[16], float4 (&vv)[4]) {
        const int kb = 16 * b;
        const int kk = min(kb + col, nkeys - 1);
        if constexpr (KV == KV_F16) {
            const uint4 *src = reinterpret_cast<const uint4 *>(kbase + ((size_t)kk * kHeadDim + 16 * grp) * esz);
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint4 u = src[i];
                const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float2 f = __half22float2(*reinterpret_cast<const __half2 *>(&w[j]));
                    kv[8 * i + 2 * j] = f.x;
                    kv[8 * i + 2 * j + 1] = f.y;
                }
            }
        } else {
            const float4 *src = reinterpret_cast<const float4 *>(kbase + ((size_t)kk * kHeadDim + 16 * grp) * esz);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 v = src[i];
                kv[4 * i] = v.x;
                kv[4 * i + 1] = v.y;
                kv[4 * i + 2] = v.z;
                kv[4 * i + 3] = v.w;
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int kq = min(kb + 4 * grp + s, nkeys - 1);
            const char *p = vbase + ((size_t)kq * kHeadDim + 4 * col) * esz;
            if constexpr (KV == KV_F16) {
                const uint2 u = *reinterpret_cast<const uint2 *>(p);
                const float2 x = __half22float2(*reinterpret_cast<const __half2 *>(&u.x));
                const float2 y = __half22float2(*reinterpret_cast<const __half2 *>(&u.y));
                vv[s] = make_float4(x.x, x.y, y.x, y.y);
            } else {
                vv[s] = *reinterpret_cast<const float4 *>(p);
            }
        }
    };
    float mrun = -INFINITY, lrun = 0.f;
    floatx4 o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    float kv[16];
    float4 vv[4];
    if (wave < nkb) load_block(wave, kv, vv);
    for (int b = wave; b < nkb; b += 4) {
        const int kb = 16 * b;
        float kn[16];
        float4 vn[4];
        const bool more = b + 4 < nkb;
        if (more) load_block(b + 4, kn, vn);  // the wave's next block in flight
        floatx4 sc0 = {0.f, 0.f, 0.f, 0.f}, sc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            sc0 = mfma_f32x4(kv[i], qv[i], sc0);
            sc1 = mfma_f32x4(kv[i + 1], qv[i + 1], sc1);
        }
        const floatx4 sc = sc0 + sc1;
        float p[4], bmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int kp = kb + 4 * grp + i;
            const bool vis = qvalid && kp <= qpos && kp < nkeys;
            p[i] = vis ? sc[i] * 0.125f : -INFINITY;  // (q . k) / sqrt(64), llm.cpp:200
            bmax = fmaxf(bmax, p[i]);
        }
        bmax = fmaxf(bmax, xshfl<16>(bmax));
        bmax = fmaxf(bmax, xshfl<32>(bmax));
        const float mnew = fmaxf(mrun, bmax);
        const float msafe = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = expf(mrun - msafe);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = expf(p[i] - msafe);
        lrun = lrun * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
        mrun = mnew;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] *= alpha;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            o[0] = mfma_f32x4(vv[s].x, p[s], o[0]);
            o[1] = mfma_f32x4(vv[s].y, p[s], o[1]);
            o[2] = mfma_f32x4(vv[s].z, p[s], o[2]);
            o[3] = mfma_f32x4(vv[s].w, p[s], o[3]);
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
    // proj in the same launch (a.proj_part): wave w takes proj's 16-column subtiles w, w + 4,
    // ..., 12 of the 48; their units for this head's two blocks are requested now, so that they
    // arrive during the merge (the barriers up to the proj MFMAs order LDS only; requested
    // before the key blocks instead, they delay those: 256-row prefill 0.62 -> 0.63 ms)
    const bool fuse = a.proj_part != nullptr;  // uniform
    constexpr int kPS = kHidden / 16 / 4;     // subtiles per wave
    uint2 pq[kPS][2];
    uint16_t pd[kPS][2];
    if (fuse) {
        // B operand of lane c16 + 16 kq: row n = 16 s + c16 of proj, columns 8 kq .. 8 kq + 7 of
        // block 2h + bb, and the row's block scale -- one unit of the matrix-core order, or the
        // row's 32-byte run in its 4-row group's 136-byte block (Q8_0_4X4)
        const int c16 = lane & 15, kq = lane >> 4;
        constexpr int nb = kHidden / 32;
#pragma unroll
        for (int i = 0; i < kPS; ++i)
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const int sub = wave + 4 * i, blk = 2 * h + bb;
                const uint8_t *qp, *dp;
                if (a.proj_tiled) {
                    const uint8_t *unit = a.proj_w + ((size_t)sub * nb + blk) * kTileBytes;
                    qp = unit + 8 * lane;
                    dp = unit + 512 + 2 * c16;
                } else {
                    const int n = 16 * sub + c16;
                    const uint8_t *b4 = a.proj_w + ((size_t)(n >> 2) * nb + blk) * kBlockBytes;
                    qp = b4 + 8 + 32 * (n & 3) + 8 * kq;
                    dp = b4 + 2 * (n & 3);
                }
                pq[i][bb] = *reinterpret_cast<const uint2 *>(qp);
                pd[i][bb] = *reinterpret_cast<const uint16_t *>(dp);
            }
    }
    float *R = red[wave];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) R[(16 * grp + 4 * i + j) * 16 + col] = o[j][i];
    if (grp == 0) {
        R[1024 + col] = mrun;
        R[1040 + col] = lrun;
    }
    lds_barrier();
    // thread t: row q = t / 16, columns 4 (t % 16) .. + 3 of the head
    const int q = t >> 4, d4 = t & 15, m = m0 + q;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, red[w][1024 + q]);
    const float msafe = mx == -INFINITY ? 0.f : mx;
    float l = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float f = expf(red[w][1024 + q] - msafe);
        l += f * red[w][1040 + q];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] += f * red[w][(4 * d4 + e) * 16 + q];
    }
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    float ov[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) ov[e] = acc[e] * inv;
    // W8A8 operand: quant_block32's arithmetic over 8 threads x 4 values (a 32-column block)
    const bool quant = a.q8 != nullptr || (fuse && a.proj_a8);  // uniform
    uint32_t qword = 0;  // the 4 int8 values, column 4 d4 + e in byte e
    float dq = 0.0f;
    if (quant) {
        float amax = fmaxf(fmaxf(fabsf(ov[0]), fabsf(ov[1])), fmaxf(fabsf(ov[2]), fabsf(ov[3])));
        amax = fmaxf(amax, xshfl<1>(amax));
        amax = fmaxf(amax, xshfl<2>(amax));
        amax = fmaxf(amax, xshfl<4>(amax));
        dq = amax / 127.0f;
        const float id = dq > 0.0f ? 1.0f / dq : 0.0f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            int qq = (int)rintf(ov[e] * id);
            qq = qq < -127 ? -127 : (qq > 127 ? 127 : qq);
            qword |= (uint32_t)(qq & 0xff) << (8 * e);
        }
        if (a.q8 != nullptr && m < a.rows) {
            // 4 consecutive columns: one aligned 4-byte run of the matrix-core order
            *reinterpret_cast<uint32_t *>(a.q8 + q8t_at(m, h * kHeadDim + 4 * d4, kHidden)) = qword;
            if ((d4 & 7) == 0) a.d8[d8t_at(m, 2 * h + (d4 >> 3), kHidden)] = dq;
        }
    }
    if (fuse) {
        // proj's A operand for the head's two blocks in the MFMA lane order: lane q + 16 j of
        // block b takes row q, columns 8j .. 8j + 7 of the block (thread (q, d4): block d4 / 8,
        // j = (d4 % 8) / 2, the 4 columns at (d4 % 2) * 4); W8A8: int8 and the rows' block
        // scales, A16: fp16 hi / lo halves (store_hl's split)
        __shared__ uint2 pa8[2][64];
        __shared__ float pda[2][16];
        __shared__ uint4 pah[2][64], pal[2][64];
        const int bb = d4 >> 3, L = q + 16 * ((d4 & 7) >> 1), half = d4 & 1;
        if (a.proj_a8) {
            reinterpret_cast<uint32_t *>(&pa8[bb][L])[half] = qword;
            if ((d4 & 7) == 0) pda[bb][q] = dq;
        } else {
            const auto h01 = __builtin_amdgcn_cvt_pkrtz(ov[0], ov[1]);
            const auto h23 = __builtin_amdgcn_cvt_pkrtz(ov[2], ov[3]);
            const auto l01 = __builtin_amdgcn_cvt_pkrtz(ov[0] - (float)h01[0], ov[1] - (float)h01[1]);
            const auto l23 = __builtin_amdgcn_cvt_pkrtz(ov[2] - (float)h23[0], ov[3] - (float)h23[1]);
            uint2 hw, lw;
            hw.x = __builtin_bit_cast(uint32_t, h01);
            hw.y = __builtin_bit_cast(uint32_t, h23);
            lw.x = __builtin_bit_cast(uint32_t, l01);
            lw.y = __builtin_bit_cast(uint32_t, l23);
            reinterpret_cast<uint2 *>(&pah[bb][L])[half] = hw;
            reinterpret_cast<uint2 *>(&pal[bb][L])[half] = lw;
        }
        lds_barrier();
        // wave w: subtiles w + 4i, both blocks, in block order per output (the GEMM's
        // per-block scale-then-accumulate); lane holds rows 4 kq + r, column c16
        const int kq = lane >> 4, c16 = lane & 15;
        float acc[kPS][4];
#pragma unroll
        for (int i = 0; i < kPS; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][r] = 0.0f;
        if (a.proj_a8) {
            const uint2 a0 = pa8[0][lane], a1 = pa8[1][lane];
            float da[2][4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                da[0][r] = pda[0][4 * kq + r];
                da[1][r] = pda[1][4 * kq + r];
            }
#pragma unroll
            for (int i = 0; i < kPS; ++i)
#pragma unroll
                for (int b2 = 0; b2 < 2; ++b2) {
                    const uint2 av = b2 ? a1 : a0;
                    const long al = (long)(((uint64_t)av.y << 32) | av.x);
                    const long bl = (long)(((uint64_t)pq[i][b2].y << 32) | pq[i][b2].x);
                    const intx4 p = __builtin_amdgcn_mfma_i32_16x16x32_i8(al, bl, intx4{0, 0, 0, 0}, 0, 0, 0);
                    const float dw = h2f(pd[i][b2]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][r] = fmaf((float)p[r], dw * da[b2][r], acc[i][r]);
                }
        } else {
            const half8 h0 = __builtin_bit_cast(half8, pah[0][lane]), l0 = __builtin_bit_cast(half8, pal[0][lane]);
            const half8 h1 = __builtin_bit_cast(half8, pah[1][lane]), l1 = __builtin_bit_cast(half8, pal[1][lane]);
#pragma unroll
            for (int i = 0; i < kPS; ++i)
#pragma unroll
                for (int b2 = 0; b2 < 2; ++b2) {
                    const half8 bw = i8x8_to_h8(pq[i][b2]);
                    floatx4 blk = floatx4{0.f, 0.f, 0.f, 0.f};
                    blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(b2 ? h1 : h0, bw, blk, 0, 0, 0);
                    blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(b2 ? l1 : l0, bw, blk, 0, 0, 0);
                    const float dw = h2f(pd[i][b2]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[i][r] = fmaf(blk[r], dw, acc[i][r]);
                }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int mr = m0 + 4 * kq + r;
            if (mr < a.rows) {
                float *prow = a.proj_part + ((size_t)h * a.rows + mr) * kHidden + c16;
#pragma unroll
                for (int i = 0; i < kPS; ++i) prow[16 * (wave + 4 * i)] = acc[i][r];
            }
        }
    }
    if (m >= a.rows) return;
    if (a.out_hl != nullptr) {  // for the next GEMM: hi / lo halves in the matrix-core order
#pragma unroll
        for (int e = 0; e < 4; ++e) store_hl(a.out_hl, m, h * kHeadDim + 4 * d4 + e, kHidden, ov[e]);
        return;
    }
    if (a.out == nullptr) return;  // (no fp32 rows when only the W8A8 copy is read)
    float *orow = (float *)a.out + (size_t)m * a.out_stride + h * kHeadDim + 4 * d4;
    *reinterpret_cast<float4 *>(orow) = make_float4(ov[0], ov[1], ov[2], ov[3]);
}

}  // namespace

hipError_t launch_attn(const AttnArgs &a, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (a.heads <= 0 || a.rows <= 0 || a.max_keys <= 0 || a.page_size <= 0 ||
        (!a.out && !a.part && !a.out_hl && !a.q8) ||
        !a.q || !a.k_pool || !a.v_pool)
        return hipErrorInvalidValue;
    // a 64-key span is read from one page: paged caches need whole spans per page
    if (a.page_table != nullptr && a.page_size % 64 != 0) return hipErrorInvalidValue;
    if (a.out_hl != nullptr && (a.part != nullptr || a.chunks != 0 || a.heads != kHeads)) return hipErrorInvalidValue;
    if (a.part != nullptr && (a.rows != 1 || a.page_table != nullptr)) return hipErrorInvalidValue;
    if (a.row_order != nullptr && (a.part != nullptr || a.chunks != 0)) return hipErrorInvalidValue;
    if (a.q8 != nullptr && (!a.d8 || a.part != nullptr || a.heads != kHeads)) return hipErrorInvalidValue;
    // every slice holds at least one live span and reaches the end of the kernel (no stop
    // flag), so every workgroup of a sliced launch arrives at the generation counter
    if (a.chunks != 0 && (a.chunks < 0 || a.chunks > kMaxChunks || a.rows != 1 || a.part != nullptr ||
                          a.page_table != nullptr || a.row_pos != nullptr || a.q8 != nullptr ||
                          a.state != nullptr || !a.chunk_part || !a.chunk_gen ||
                          (a.chunk_waves != 2 && a.chunk_waves != 4) ||
                          a.chunk_waves * 64 * (a.chunks - 1) >= a.max_keys))
        return hipErrorInvalidValue;
    return kv == KV_F16 ? launch_kv<KV_F16>(a, s) : launch_kv<KV_F32>(a, s);
}

hipError_t launch_attn_tiles(const AttnArgs &a, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (a.heads != kHeads || a.rows <= 0 || a.max_keys <= 0 || a.page_size < a.max_keys ||
        (!a.out && !a.q8 && !a.out_hl && !a.proj_part) ||
        a.out_f16 ||
        !a.q || !a.k_pool || !a.v_pool || a.part || a.page_table || a.row_pos || a.row_stream || a.chunks ||
        a.pos_stride != 1 || a.pos0 < 0 || a.pos0 + a.rows > a.max_keys || a.q_stride % 4 || a.out_stride % 4 ||
        (a.q8 != nullptr && !a.d8) || (a.proj_part != nullptr && !a.proj_w))
        return hipErrorInvalidValue;
    const dim3 grid((a.rows + 15) / 16, kHeads);
    if (kv == KV_F16)
        hipLaunchKernelGGL(attn_tile_kernel<KV_F16>, grid, dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(attn_tile_kernel<KV_F32>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mh
