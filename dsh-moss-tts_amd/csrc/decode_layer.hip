// decode_layer.hip -- one transformer block of the single-stream decode in one launch (gfx950).
//
// Replaces block_forward (reference csrc/src/llm.cpp:230-246) for one global
// layer at the current position: LN1 -> QKV (bias, RoPE, KV write) ->
// attention over the cache -> proj + residual -> LN2 -> fc_in + gelu_new ->
// fc_out + residual.  Launched as five kernels this chain pays a dependent
// launch (~1.6 us on MI355X) plus a cold re-read of its input at every stage;
// here the stages run inside one launch of kLayerGrid workgroups and hand their
// outputs on through LL words.
//
// LL word: an 8-byte word holding a 32-bit value and a 32-bit tag, written with
// one agent-scope store and read with agent-scope loads (both coherent across
// the XCDs' L2 caches).  The tag is unique to the launch (position, layer), so
// a consumer simply re-reads the words it needs until every tag is current:
// the data is its own flag -- no barrier, counter or fence.  Every wait is
// bounded: a workgroup whose poll budget runs out sets *err and stops, the
// workgroups waiting on it then run out in turn, and the host reports *err.
// The host clears the words before a generate() call, so no stale word from an
// earlier call can carry a current tag.
//
// All kLayerGrid workgroups must be resident at once (a consumer waits for
// producers in other workgroups): the host checks the kernel's occupancy
// before it uses this path (two workgroups per CU on 256 CUs).
//
// Stage layout (workgroup b of 192, one per CU: two workgroups sharing a CU
// would halve each other's issue rate, and every stage is a chain of latencies):
//   Q  b < 144: QKV groups 4b + w (one wave per 4-row group)    -> LL q|k|v
//   A  144 <= b < 144 + 12*Qs (Qs = min(ceil(spans / 4), 4)): unit u = b - 144,
//                 head u / Qs, wave w takes the 64-key span 4*(u % Qs) + w (its
//                 K/V loads issued at the start; past 1024 keys also the spans
//                 every 4*Qs further), merged in the workgroup -> LL partial (o, m, l)
//   P  b < 192: proj group b (4 waves), partials merged first   -> LL x + attn
//   M  b < 192: fc_in groups 4b + w, LN2 first                  -> LL h
//   F  b < 192: fc_out group b (4 waves)                        -> x (memory)
#include <type_traits>

#include "mh_gemv.h"
#include "mh_ll.h"
#include "mh_ops.h"

namespace mh {
namespace {


// Stage timestamps (100 MHz device clock) of the last launch, per workgroup,
// in builds with -DMH_STAGE_TRACE only (a profiling build; the library as
// shipped has none of it).
#ifdef MH_STAGE_TRACE
}  // namespace
__device__ unsigned long long mh_stage_ts[kLayerGrid][16];
namespace {
#define STAGE_TS(k)                                                                              \
    do {                                                                                         \
        if (threadIdx.x == 0) mh_stage_ts[blockIdx.x][k] = __builtin_amdgcn_s_memrealtime();     \
    } while (0)
#else
#define STAGE_TS(k) \
    do {            \
    } while (0)
#endif

// LL regions (words)
constexpr int kMaxUnits = kHeads * kLayerMaxQuarters;
constexpr int kLLQ = 0;                            // q | k | v of the new position (2304)
constexpr int kLLA = kLLQ + 3 * kHidden;           // attention partials, 66 words per unit
constexpr int kLLX = kLLA + kMaxUnits * 66;        // x after the attention sub-block (768)
constexpr int kLLH = kLLX + kHidden;               // fc_in output (3072)
constexpr int kAttnBase = 3 * kHidden / 4 / 4;     // attention workgroups follow the QKV ones (144)
static_assert(kAttnBase + kMaxUnits <= kLayerGrid, "attention workgroups inside the grid");
static_assert(kLLH + kFF == kLayerWords, "LL layout");

// Raw K/V operands of one wave's 64-key span, loaded before the query is known.
template <int KV>
struct SpanRaw {
    using KT = typename std::conditional<KV == KV_F16, uint4, float4>::type;  // 8 halves / 4 floats
    using VT = typename std::conditional<KV == KV_F16, uint2, float4>::type;  // 4 halves / 4 floats
    KT k[KV == KV_F16 ? 8 : 16];
    VT v[16];
};

template <int KV>
__device__ __forceinline__ float4 raw4(const typename SpanRaw<KV>::VT &v) {
    if constexpr (KV == KV_F16) {
        const __half2 *h = (const __half2 *)&v;
        const float2 a = __half22float2(h[0]), b = __half22float2(h[1]);
        return make_float4(a.x, a.y, b.x, b.y);
    } else {
        return v;
    }
}

// KV-precision storage of 4 values that are already KV-precision (exact).
template <int KV>
__device__ __forceinline__ typename SpanRaw<KV>::VT to_raw4(float4 f) {
    if constexpr (KV == KV_F16) {
        const __half2 a = __floats2half2_rn(f.x, f.y), b = __floats2half2_rn(f.z, f.w);
        uint2 r;
        r.x = *(const uint32_t *)&a;
        r.y = *(const uint32_t *)&b;
        return r;
    } else {
        return f;
    }
}

template <int KV>
__device__ __forceinline__ float rawk(const SpanRaw<KV> &r, int i) {  // element i (0..63) of the K row
    if constexpr (KV == KV_F16) {
        const __half *h = (const __half *)&r.k[i >> 3];
        return __half2float(h[i & 7]);
    } else {
        const float *f = (const float *)&r.k[i >> 2];
        return f[i & 3];
    }
}

template <int KV>
__global__ __launch_bounds__(256) void decode_layer_kernel(LayerArgs a) {
#pragma clang fp contract(off)
    __shared__ float act[kFF];                 // GEMV activation
    __shared__ float xm[kHidden];              // x after the attention sub-block (fc_out's residual)
    __shared__ float pbuf[kMaxUnits * 66];     // gathered attention partials
    __shared__ float qkn[3 * kHeadDim];        // q, k, v of the new position for this head
    __shared__ float hw[kHeads][kLayerMaxQuarters + 1];  // per-head merge weights and denominator
    __shared__ float sc[4][64];
    __shared__ float4 po[4][16];
    __shared__ float pm[4], pl[4];
    __shared__ float part[4][4];

    STAGE_TS(0);
    if (a.state->stop) return;  // written only between frames: the same for every workgroup
    const int pos = a.state->pos;
    const uint32_t tag = ((uint32_t)(pos + 1) << 5) | (uint32_t)a.instance;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    const int b = blockIdx.x;
    int budget = kPollBudget;
    uint64_t *LL = a.ll;

    // ---- stage Q: LN1 + QKV, one wave per group
    if (b < kAttnBase) {
        GemvStage<1, 6, kHidden> gs;
        gs.prefetch(a.attn_w, b);
        const int r = gs.row();
        QkvEpi e;
        if (gs.storer()) e.load(a.attn_b, a.rope_cos, a.rope_sin, r, pos);
        float o[3], lw[3], lb[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            xm[t + 256 * i] = a.x[t + 256 * i];
            lw[i] = a.ln1_w[t + 256 * i];
            lb[i] = a.ln1_b[t + 256 * i];
        }
        __syncthreads();
        layernorm_768_lds(xm, lw, lb, o);
#pragma unroll
        for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
        __syncthreads();
        STAGE_TS(1);
        const float yv = gs.dot(act, part);
        const float partner = xshfl<4>(yv);
        if (gs.storer()) {  // bias, RoPE (llm.cpp:234-236), KV write (llm.cpp:224-225)
            float out = e.apply(r, yv, partner);
            const int sec = r / kHidden, within = r - sec * kHidden;
            if (sec > 0) {  // the cache holds KV-precision values: hand on the same
                const size_t idx = ((size_t)(within >> 6) * a.ctx_stride + pos) * kHeadDim + (within & 63);
                void *cache = sec == 1 ? a.k_cache : a.v_cache;
                if constexpr (KV == KV_F16) {
                    const __half hv = __float2half_rn(out);
                    ((__half *)cache)[idx] = hv;
                    out = __half2float(hv);
                } else {
                    ((float *)cache)[idx] = out;
                }
            }
            ll_put(LL + kLLQ + r, out, tag);
        }
        STAGE_TS(2);
    }

    // ---- stage A: attention of head h over 64-key spans, one per wave (more,
    // strided by 4 * Qs, past 1024 keys), online softmax across a wave's spans
    const int n = pos + 1;
    const int spans = (n + 63) >> 6;
    const int Qs = min((spans + 3) >> 2, kLayerMaxQuarters);
    if (b >= kAttnBase && b < kAttnBase + kHeads * Qs) {
        const int unit = b - kAttnBase;
        const int h = unit / Qs, span0 = (unit - h * Qs) * 4 + wave;
        const int pg = lane >> 4, dg = lane & 15;
        const int crow_max = max(pos - 1, 0);
        const size_t hbase = (size_t)h * a.ctx_stride;
        // K/V of a span: this lane's score key and V keys; cache rows are
        // clamped to pos - 1 (or 0), rows written by earlier launches; the key
        // at pos, and the clamped keys past it, take the LL values in run_span
        auto load_span = [&](SpanRaw<KV> &r, int span) {
            const int p0 = span * 64, cnt = max(min(64, n - p0), 1);
            const size_t krow = (hbase + min(p0 + min(lane, cnt - 1), crow_max)) * kHeadDim;
            if constexpr (KV == KV_F16) {
#pragma unroll
                for (int c = 0; c < 8; ++c) r.k[c] = *(const uint4 *)((const __half *)a.k_cache + krow + 8 * c);
            } else {
#pragma unroll
                for (int c = 0; c < 16; ++c) r.k[c] = *(const float4 *)((const float *)a.k_cache + krow + 4 * c);
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const size_t vi = (hbase + min(p0 + min(pg + 4 * q, cnt - 1), crow_max)) * kHeadDim + 4 * dg;
                r.v[q] = *(const typename SpanRaw<KV>::VT *)((const uint8_t *)a.v_cache + vi * (KV == KV_F16 ? 2 : 4));
            }
        };
        SpanRaw<KV> raw;
        load_span(raw, min(span0, spans - 1));  // before q is known
        // q, k, v of head h at pos
        {
            const int seg = t >> 6;
            const bool ok = ll_wait1(LL + kLLQ + seg * kHidden + h * kHeadDim + (t & 63), t < 3 * kHeadDim, tag,
                                     &qkn[min(t, 3 * kHeadDim - 1)], budget);
            if (__syncthreads_or(!ok)) {
                if (t == 0) atomicOr(a.err, 1u);
                return;
            }
        }
        STAGE_TS(3);
        float m = -INFINITY, l = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int span = span0; span < spans; span += 4 * Qs) {
            if (span != span0) load_span(raw, span);
            const int p0 = span * 64, cnt = min(64, n - p0);
            if (p0 + min(lane, cnt - 1) == pos) {  // this lane's score key is the new one
                if constexpr (KV == KV_F16) {
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const typename SpanRaw<KV>::VT lo = to_raw4<KV>(*(const float4 *)&qkn[kHeadDim + 8 * c]);
                        const typename SpanRaw<KV>::VT hi = to_raw4<KV>(*(const float4 *)&qkn[kHeadDim + 8 * c + 4]);
                        raw.k[c] = make_uint4(lo.x, lo.y, hi.x, hi.y);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 16; ++c) raw.k[c] = *(const float4 *)&qkn[kHeadDim + 4 * c];
                }
            }
            if (p0 + cnt - 1 == pos) {  // the span holding the new key
                const typename SpanRaw<KV>::VT nv = to_raw4<KV>(*(const float4 *)&qkn[2 * kHeadDim + 4 * dg]);
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    if (pg + 4 * q >= cnt - 1) raw.v[q] = nv;
            }
            float dot = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c)
#pragma unroll
                for (int e = 0; e < 8; ++e) dot = fmaf(qkn[8 * c + e], rawk<KV>(raw, 8 * c + e), dot);
            dot *= 0.125f;  // 1/sqrt(64), applied after the dot as llm.cpp:200 does
            const float smax = wave_max(lane < cnt ? dot : -INFINITY);
            STAGE_TS(4);
            const float m_new = fmaxf(m, smax);
            const float rescale = expf(m - m_new);  // 0 on the first span (m = -inf)
            const float e = lane < cnt ? expf(dot - m_new) : 0.0f;
            l = l * rescale + wave_sum(e);
            m = m_new;
            o.x *= rescale;
            o.y *= rescale;
            o.z *= rescale;
            o.w *= rescale;
            sc[wave][lane] = e;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const float4 v = raw4<KV>(raw.v[q]);
                const float ei = sc[wave][pg + 4 * q];
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
        if (lane < 16) po[wave][dg] = o;
        if (lane == 0) {
            pm[wave] = m;
            pl[wave] = l;
        }
        __syncthreads();
        if (wave == 0) {  // log-sum-exp merge of the waves that saw keys (a prefix)
            const int nlive = min(4, spans - (unit - h * Qs) * 4);
            float wm[4], wl[4], wo[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {  // every LDS read issued before the first use
                wm[w] = pm[w];
                wl[w] = pl[w];
                wo[w] = ((const float *)&po[w][0])[lane];
            }
            float M = wm[0];
#pragma unroll
            for (int w = 1; w < 4; ++w)
                if (w < nlive) M = fmaxf(M, wm[w]);
            float L = 0.0f, O = 0.0f;
#pragma unroll
            for (int w = 0; w < 4; ++w)
                if (w < nlive) {
                    const float sw = expf(wm[w] - M);
                    L = fmaf(wl[w], sw, L);
                    O = fmaf(wo[w], sw, O);
                }
            uint64_t *dst = LL + kLLA + (size_t)unit * 66;
            ll_put(dst + lane, O, tag);
            if (lane == 0) {
                ll_put(dst + 64, M, tag);
                ll_put(dst + 65, L, tag);
            }
            STAGE_TS(5);
        }
    }

    // ---- stage P: merge the partials, proj + residual (4 waves per group)
    if (b < kHidden / 4) {
        GemvStage<4, 2, kHidden> gs;
        gs.prefetch(a.proj_w, b);
        const int r = gs.row();
        float eb = 0.f, eres = 0.f;
        if (gs.storer()) {
            eb = a.proj_b[r];
            eres = a.x[r];
        }
        const int units = kHeads * Qs;
        const bool ok = ll_gather<(kMaxUnits * 66 + 255) / 256>(LL + kLLA, units * 66, tag, pbuf, budget);
        if (__syncthreads_or(!ok)) {
            if (t == 0) atomicOr(a.err, 1u);
            return;
        }
        STAGE_TS(6);
        // o = sum_q e^(m_q - M) o_q / sum_q e^(m_q - M) l_q: the weights e^(m_q - M)
        // and the denominator once per head (thread h), then every output
        if (t < kHeads) {
            const float *pp = pbuf + (size_t)t * Qs * 66;
            float mq[kLayerMaxQuarters], lq[kLayerMaxQuarters];
#pragma unroll
            for (int q = 0; q < kLayerMaxQuarters; ++q) {
                const int qq = min(q, Qs - 1);
                mq[q] = pp[qq * 66 + 64];
                lq[q] = pp[qq * 66 + 65];
            }
            float M = mq[0];
#pragma unroll
            for (int q = 1; q < kLayerMaxQuarters; ++q)
                if (q < Qs) M = fmaxf(M, mq[q]);
            float L = 0.0f;
#pragma unroll
            for (int q = 0; q < kLayerMaxQuarters; ++q) {
                const float sw = q < Qs ? expf(mq[q] - M) : 0.0f;
                if (q < Qs) L = fmaf(lq[q], sw, L);
                hw[t][q] = sw;
            }
            hw[t][kLayerMaxQuarters] = L;
        }
        __syncthreads();
#pragma unroll
        for (int i3 = 0; i3 < 3; ++i3) {
            const int i = t + 256 * i3, h = i >> 6, d = i & 63;
            const float *pp = pbuf + (size_t)h * Qs * 66;
            float oq[kLayerMaxQuarters];
#pragma unroll
            for (int q = 0; q < kLayerMaxQuarters; ++q) oq[q] = pp[min(q, Qs - 1) * 66 + d];
            float O = 0.0f;
#pragma unroll
            for (int q = 0; q < kLayerMaxQuarters; ++q)
                if (q < Qs) O = fmaf(oq[q], hw[h][q], O);
            act[i] = O / hw[h][kLayerMaxQuarters];
        }
        __syncthreads();
        STAGE_TS(7);
        const float yv = gs.dot(act, part);
        if (gs.storer()) ll_put(LL + kLLX + r, eres + (yv + eb), tag);  // llm.cpp:239
        STAGE_TS(8);
    }

    // ---- stage M: LN2 + fc_in + gelu_new, one wave per group, every workgroup
    {
        GemvStage<1, 6, kHidden> gs;
        gs.prefetch(a.fc_in_w, b);
        const int r = gs.row();
        const float eb = gs.storer() ? a.fc_in_b[r] : 0.0f;
        float lw[3], lb[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            lw[i] = a.ln2_w[t + 256 * i];
            lb[i] = a.ln2_b[t + 256 * i];
        }
        const bool ok = ll_gather<3>(LL + kLLX, kHidden, tag, xm, budget);
        if (__syncthreads_or(!ok)) {
            if (t == 0) atomicOr(a.err, 1u);
            return;
        }
        STAGE_TS(9);
        float o[3];
        layernorm_768_lds(xm, lw, lb, o);
#pragma unroll
        for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
        __syncthreads();
        STAGE_TS(10);
        const float yv = gs.dot(act, part);
        if (gs.storer()) ll_put(LL + kLLH + r, gelu_new(yv + eb), tag);  // llm.cpp:243
        STAGE_TS(11);
        __syncthreads();  // every wave is done with act before stage F gathers into it
    }

    // ---- stage F: fc_out + residual (4 waves per group) -> x
    if (b < kHidden / 4) {
        GemvStage<4, 6, kFF> gs;
        gs.prefetch(a.fc_out_w, b);
        const int r = gs.row();
        const float eb = gs.storer() ? a.fc_out_b[r] : 0.0f;
        const bool ok = ll_gather<kFF / 256>(LL + kLLH, kFF, tag, act, budget);
        if (__syncthreads_or(!ok)) {
            if (t == 0) atomicOr(a.err, 1u);
            return;
        }
        STAGE_TS(12);
        const float yv = gs.dot(act, part);
        if (gs.storer()) a.x[r] = xm[r] + (yv + eb);  // llm.cpp:245
        STAGE_TS(13);
    }
}

}  // namespace

hipError_t decode_layer_fits(int device, bool *fits) {
    *fits = false;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return e;
    int per_cu16 = 0, per_cu32 = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu16, decode_layer_kernel<KV_F16>, 256, 0);
    if (e != hipSuccess) return e;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu32, decode_layer_kernel<KV_F32>, 256, 0);
    if (e != hipSuccess) return e;
    int per_cu_local = 0;
    e = decode_local_occupancy(&per_cu_local);
    if (e != hipSuccess) return e;
    int per_cu = per_cu16 < per_cu32 ? per_cu16 : per_cu32;
    per_cu = per_cu < per_cu_local ? per_cu : per_cu_local;
    *fits = (long)per_cu * prop.multiProcessorCount >= kLayerGrid;
    return hipSuccess;
}

#ifdef MH_STAGE_TRACE
// [kLayerGrid][16] timestamps of the last launch (profiling builds only)
extern "C" int mh_stage_trace_read(unsigned long long *out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(mh_stage_ts), sizeof(mh_stage_ts));
}
#endif

hipError_t launch_decode_layer(const LayerArgs &a, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (!a.attn_w || !a.proj_w || !a.fc_in_w || !a.fc_out_w || !a.x || !a.k_cache || !a.v_cache || !a.state ||
        !a.ll || !a.err || !a.rope_cos || !a.rope_sin)
        return hipErrorInvalidValue;
    // tag bits: instance < 32, position + 1 < 2^27
    if (a.ctx_stride <= 0 || a.ctx_stride >= (1 << 26) || a.instance < 0 || a.instance >= 32)
        return hipErrorInvalidValue;
    if (kv == KV_F16)
        hipLaunchKernelGGL(decode_layer_kernel<KV_F16>, dim3(kLayerGrid), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(decode_layer_kernel<KV_F32>, dim3(kLayerGrid), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mh
