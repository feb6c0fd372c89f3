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
//   A  144 <= b < 144 + 12*Qs: unit u = b - 144 = (head u / Qs, quarter
//                 u % Qs); wave w takes the 64-key spans 4*(u % Qs) + w + 4*Qs*i,
//                 NS per round with all their K/V loads in flight (the first
//                 round's issued at the start); Qs = 1 while the keys fit one
//                 round of 4 waves (768 keys in fp16)        -> LL head output,
//                 more quarters (longer contexts)            -> LL partial (o, m, l)
//   P  b < 192: proj group b (4 waves), partials merged first  -> LL x + attn
//   M  b < 192: fc_in groups 4b + w, LN2 first                  -> LL h
//   F  b < 192: fc_out group b (4 waves)                        -> x (memory)
#include <algorithm>
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
__device__ unsigned long long mh_stage_ts[kLayerGrid][32];
namespace {
// Kept in LDS by thread 0 and written out at the end of the launch: a global
// store inside a stage would make the next barrier wait for it.
#define STAGE_DECL                                         \
    __shared__ unsigned long long stage_ts_lds[32];        \
    if (threadIdx.x == 0)                                  \
        for (int i_ = 0; i_ < 32; ++i_) stage_ts_lds[i_] = i_ == 16 ? __builtin_amdgcn_s_memtime() : 0
#define STAGE_TS(k)                                                               \
    do {                                                                          \
        if (threadIdx.x == 0) stage_ts_lds[k] = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#define STAGE_FLUSH()                                                          \
    do {                                                                       \
        if (threadIdx.x == 0) {                                                \
            stage_ts_lds[17] = __builtin_amdgcn_s_memtime();                   \
            stage_ts_lds[18] = __builtin_amdgcn_s_memrealtime();               \
            for (int i_ = 0; i_ < 32; ++i_) mh_stage_ts[blockIdx.x][i_] = stage_ts_lds[i_]; \
        }                                                                      \
    } while (0)
#else
#define STAGE_DECL \
    do {           \
    } while (0)
#define STAGE_TS(k) \
    do {            \
    } while (0)
#define STAGE_FLUSH() \
    do {              \
    } while (0)
#endif

// LL regions (words)
constexpr int kMaxUnits = kHeads * kLayerMaxQuarters;
constexpr int kLLQ = 0;                            // q | k | v of the new position (2304)
constexpr int kLLA = kLLQ + 3 * kHidden;           // attention partials, 66 words per unit
constexpr int kLLX = kLLA + kMaxUnits * 66;        // x after the attention sub-block (768)
constexpr int kLLH = kLLX + kHidden;               // fc_in output (3072)
constexpr int kLLO = kLLH + kFF;                   // block output, the next block's input (768)
constexpr int kAttnBase = 3 * kHidden / 4 / 4;     // attention workgroups follow the QKV ones (144)
static_assert(kAttnBase + kMaxUnits <= kLayerGrid, "attention workgroups inside the grid");

// 64-key spans a wave holds in registers at once (K and V: 64 VGPRs per span
// in fp16, 128 in fp32), and the attention workgroups per head for n keys:
// one up to 4 * NS spans (768 keys in fp16), at most kLayerMaxQuarters.
template <int KV>
constexpr int kAttnSpansPerWave = KV == KV_F16 ? 3 : 1;
template <int KV>
constexpr int kLanesPerKey = KV == KV_F16 ? 8 : 16;  // 16-byte K loads per 64-dim key
template <int KV>
__device__ __forceinline__ int attn_quarters(int n) {
    constexpr int per = 4 * kAttnSpansPerWave<KV>;
    return min((((n + 63) >> 6) + per - 1) / per, kLayerMaxQuarters);
}
static_assert(kLLO + kHidden == kLayerWords, "LL layout");

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
__device__ __forceinline__ float rawk(const SpanRaw<KV> &r, int c, int e) {  // element e of K load c
    if constexpr (KV == KV_F16) {
        const __half *h = (const __half *)&r.k[c];
        return __half2float(h[e]);
    } else {
        const float *f = (const float *)&r.k[c];
        return f[e];
    }
}

// Stages Q and M (one wave per 4-row group) read their weights from LDS, copied in by
// wave 3 a stage ahead (Q's at the end of the previous block, M's at the end of stage P);
// the gathers before them are waves 0..2's, so none of their polls completes behind a
// copy (at the first, 0.1753 -> 0.1720 ms per global step)
using QStage = LdsGemvStage<6, kHidden>;
constexpr int kDmaWave = 3;

// A8: every GEMV in W8A8 (the activation quantised per 32-block in LDS, quant_act_lds),
// the reference's decode with MOSS_A16 unset (csrc/src/gemv.cpp:23-48,245-274).
template <int KV, bool A8>
__global__ __launch_bounds__(256) void decode_global_kernel(GlobalArgs g) {
#pragma clang fp contract(off)
    __shared__ float act[kFF];                 // GEMV activation
    __shared__ float da[kFF / 32];             // its block scales (A8)
    __shared__ float xin[kHidden];             // block input (x), the last block's output at the end
    __shared__ float xm[kHidden];              // x after the attention sub-block (fc_out's residual)
    __shared__ float pbuf[kMaxUnits * 66];     // gathered attention partials
    __shared__ float qkn[3 * kHeadDim];        // q, k, v of the new position for this head
    __shared__ float hw[kHeads][kLayerMaxQuarters + 1];  // per-head merge weights and denominator
    // a span's softmax weights, key k at (k % 4) * 16 + k / 4: the 16 keys pg + 4q a lane's
    // value pass takes are then 16 consecutive floats (four 16-byte LDS reads)
    __shared__ __attribute__((aligned(16))) float sc[4][kAttnSpansPerWave<KV>][64];
    __shared__ float4 po[4][16];
    __shared__ float pm[4], pl[4];
    __shared__ float part[4][4];
    __shared__ __attribute__((aligned(16))) uint8_t wq_lds[QStage::kBytes];  // stage Q's weights
    __shared__ __attribute__((aligned(16))) uint8_t wm_lds[QStage::kBytes];  // stage M's

    __shared__ int wait_failed;  // set when a wait of this workgroup runs out
    if (threadIdx.x == 0) wait_failed = 0;
    __syncthreads();
    STAGE_DECL;
    STAGE_TS(0);
    if (g.state->stop) return;  // written only between frames: the same for every workgroup
    const int pos = g.state->pos;
    const int t = threadIdx.x;
    const int b = blockIdx.x;
    if (b < kAttnBase && (t >> 6) == kDmaWave) QStage::issue_wave(g.layers[0].attn_w, b, wq_lds);
    int budget = g.poll_budget > 0 ? g.poll_budget : kPollBudget;
    uint64_t *LL = g.ll;

    // embed_row (llm.cpp:114-157): x = wte[row[0]] + sum over channels of
    // aemb[ch][code] (pad 1024 skipped), in channel order; every workgroup
    // builds all of x, which every stage below reads from LDS
    {
        const int nb = kHidden / 32;
        const int w0 = g.row[0];
        int code[kNVq];
#pragma unroll
        for (int ch = 0; ch < kNVq; ++ch) code[ch] = g.row[ch + 1];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            const int c = t + 256 * i;
            float e[kNVq];
#pragma unroll
            for (int ch = 0; ch < kNVq; ++ch) {
                const bool use = !(code[ch] == kAudioPad || code[ch] < 0 || code[ch] >= kCodebook);
                e[ch] = use ? q8x4_elem(g.aemb[ch], nb, code[ch], c) : 0.0f;
            }
            float v = q8x4_elem(g.wte, nb, w0, c);
#pragma unroll
            for (int ch = 0; ch < kNVq; ++ch) {
                const bool use = !(code[ch] == kAudioPad || code[ch] < 0 || code[ch] >= kCodebook);
                if (use) v = v + e[ch];
            }
            xin[c] = v;
        }
        __syncthreads();
    }

    QkvEpi eq;
    int rq = 0;
#pragma unroll 1
    for (int layer = 0; layer < kLayers; ++layer) {
        const LayerArgs a = g.layers[layer];
        const uint32_t tag = ((uint32_t)(pos + 1) << 5) | (uint32_t)layer;
        // W8A8 quantiser capture of this block (tests only; null in the library's own use)
        float *const cap = A8 && g.cap ? g.cap + (size_t)layer * MOSS_HIP_CAP_STEP : nullptr;
        // per-block copies of the indices: nothing derived from them is held across blocks
        // the wave index as a wave-uniform (scalar) value, so that per-span and per-wave
        // conditions below are branches rather than selects executed by every wave
        const int t = tix(), wave = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
        const int b = bix();

        // ---- loads that do not depend on this block's input, issued before
        // waiting for it: the QKV weights (stage Q) and the first round of K/V
        // spans (stage A).  (Requesting stage Q's a block ahead, during stage F,
        // measured 0.178 -> 0.188 ms per step.)
        if (b < kAttnBase) {
            QStage gq;
            gq.setup(b, wq_lds);
            rq = gq.row();
            if (gq.storer()) eq.load(a.attn_b, a.rope_cos, a.rope_sin, rq, pos);
        }
        constexpr int NS = kAttnSpansPerWave<KV>;
        const int n = pos + 1;
        const int spans = (n + 63) >> 6;
        const int Qs = attn_quarters<KV>(n);
        const bool attn_wg = b >= kAttnBase && b < kAttnBase + kHeads * Qs;
        const int unit = b - kAttnBase;
        const int h = unit / Qs, qq = unit - h * Qs;
        const int span0 = qq * 4 + wave, stride = 4 * Qs;
        const int pg = lane >> 4, dg = lane & 15;
        constexpr int EPL = 64 / kLanesPerKey<KV>, RPI = 64 / kLanesPerKey<KV>;  // K dims per lane, keys per load
        const int sub = lane & (kLanesPerKey<KV> - 1), rr = lane / kLanesPerKey<KV>;
        const int kl = RPI * sub + rr;  // the key (within a span) whose score this lane ends with
        const int crow_max = max(pos - 1, 0);
        const size_t hbase = (size_t)h * a.ctx_stride;
        // K of a span: load c brings 16 bytes of key RPI*c + rr (dims sub*EPL ..),
        // so one load covers RPI whole 128/256-byte rows; V: lane (pg, dg) keys
        // pg + 4q, dims 4dg .. 4dg+3.  Cache rows are clamped to pos - 1 (or 0),
        // rows written before this launch; the key at pos, and the clamped keys
        // past it, take this block's k and v (stage Q) below.
        auto load_span = [&](SpanRaw<KV> &r, int span) {
            const int p0 = span * 64, cnt = max(min(64, n - p0), 1);
#pragma unroll
            for (int c = 0; c < kLanesPerKey<KV>; ++c) {
                const int key = min(p0 + min(RPI * c + rr, cnt - 1), crow_max);
                const size_t ki = (hbase + key) * kHeadDim + sub * EPL;
                r.k[c] = *(const typename SpanRaw<KV>::KT *)((const uint8_t *)a.k_cache + ki * (KV == KV_F16 ? 2 : 4));
            }
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const size_t vi = (hbase + min(p0 + min(pg + 4 * q, cnt - 1), crow_max)) * kHeadDim + 4 * dg;
                r.v[q] = *(const typename SpanRaw<KV>::VT *)((const uint8_t *)a.v_cache + vi * (KV == KV_F16 ? 2 : 4));
            }
        };
        SpanRaw<KV> raw[NS];
        if (attn_wg) {
#pragma unroll
            for (int i = 0; i < NS; ++i) load_span(raw[i], min(span0 + stride * i, spans - 1));
        }

        // this block's input: the previous block's output (block 0: the embedding).  The
        // attention workgroups skip it: their gather would wait behind their K/V loads
        // (loads complete in issue order) and so delay their query wait; they need only
        // the residuals of their 4 proj rows, which stage P polls
        if (layer > 0 && !attn_wg) {
            const uint32_t prev = ((uint32_t)(pos + 1) << 5) | (uint32_t)(layer - 1);
            // waves 0..2: wave 3's loads end with the copy of this block's QKV weights
            const bool ok = wave == kDmaWave || ll_gather_by<4, 192>(LL + kLLO, kHidden, prev, xin, budget, t);
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(g.err, 1u);
                return;
            }
        }
        STAGE_TS(14);

        // ---- stage Q: LN1 + QKV, one wave per group
        if (b < kAttnBase) {
            QStage gs;
            gs.setup(b, wq_lds);
            const int r = rq;
            const QkvEpi &e = eq;
            float o[3], lw[3], lb[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                lw[i] = a.ln1_w[t + 256 * i];
                lb[i] = a.ln1_b[t + 256 * i];
            }
            layernorm_768_lds(xin, lw, lb, o);
#pragma unroll
            for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
            __syncthreads();
            if constexpr (A8) {
                float *cp = b == 0 ? cap : nullptr;  // (uniform) quantiser capture, tests only
                if (cp) {
                    cap_copy(cp + MOSS_HIP_CAP_XIN, xin, kHidden);
                    cap_copy(cp + MOSS_HIP_CAP_LN1, act, kHidden);
                    __syncthreads();  // before the quantiser rewrites runs other threads copy
                }
                quant_act_lds_k<kHidden>(act, da);
                __syncthreads();
                if (cp) {
                    cap_copy(cp + MOSS_HIP_CAP_LN1_Q, act, kHidden);
                    cap_copy(cp + MOSS_HIP_CAP_LN1_D, da, kHidden / 32);
                }
            }
            STAGE_TS(1);
            const float yv = gs.template dot<A8>(act, da);
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
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_QKV + r] = out;
            }
            STAGE_TS(2);
        }

        // ---- stage A: attention of head h.  Unit u = (head, quarter) of 12 * Qs;
        // wave w of quarter qq takes the 64-key spans qq*4 + w + 4*Qs*i, NS of them
        // per round with all their K/V loads in flight together; online softmax
        // across the rounds.  Qs == 1 (contexts up to 4 * NS spans) hands on the
        // normalised head output, more quarters hand on partials (o, m, l).
        if (attn_wg) {
            // q, k, v of head h at pos
            {
                const int seg = t >> 6;
                const bool ok = ll_wait1(LL + kLLQ + seg * kHidden + h * kHeadDim + (t & 63), t < 3 * kHeadDim, tag,
                                         &qkn[min(t, 3 * kHeadDim - 1)], budget);
                if (sync_failed(!ok, &wait_failed)) {
                    if (t == 0) atomicOr(g.err, 1u);
                    return;
                }
            }
            STAGE_TS(3);
            float m = -INFINITY, l = 0.0f;
            float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
            for (int c0 = span0; c0 < spans; c0 += NS * stride) {
                if (c0 != span0) {
#pragma unroll
                    for (int i = 0; i < NS; ++i) load_span(raw[i], min(c0 + stride * i, spans - 1));
                }
                float qs[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) qs[e] = qkn[sub * EPL + e];
                STAGE_TS(20);
                float dot[NS];
                int cnt[NS];
                float smax = -INFINITY;
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const int span = c0 + stride * i;
                    const int p0 = span * 64;
                    cnt[i] = span < spans ? min(64, n - p0) : 0;
                    float pd[kLanesPerKey<KV>];
#pragma unroll
                    for (int c = 0; c < kLanesPerKey<KV>; ++c) {
                        float d = 0.0f;
#pragma unroll
                        for (int e = 0; e < EPL; ++e) d = fmaf(qs[e], rawk<KV>(raw[i], c, e), d);
                        pd[c] = d;
                    }
                    float d = key_reduce<kLanesPerKey<KV>>(pd, sub);  // q . k of key kl
                    if (span == spans - 1) {  // the span holding the new key: its k and v from this launch
                        const float snew = wave_sum(qkn[lane] * qkn[kHeadDim + lane]);
                        if (kl == pos - p0) d = snew;
                        const typename SpanRaw<KV>::VT nv = to_raw4<KV>(*(const float4 *)&qkn[2 * kHeadDim + 4 * dg]);
#pragma unroll
                        for (int q = 0; q < 16; ++q)
                            if (pg + 4 * q >= cnt[i] - 1) raw[i].v[q] = nv;
                    }
                    dot[i] = d * 0.125f;  // 1/sqrt(64), applied after the dot as llm.cpp:200 does
                    if (kl < cnt[i]) smax = fmaxf(smax, dot[i]);
                }
                smax = wave_max(smax);
                STAGE_TS(4);
                const float m_new = fmaxf(m, smax);
                const float rescale = expf(m - m_new);  // 0 on the first round (m = -inf)
                float esum = 0.0f;
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const float e = kl < cnt[i] ? expf(dot[i] - m_new) : 0.0f;
                    esum += e;
                    sc[wave][i][(kl & 3) * 16 + (kl >> 2)] = e;
                }
                l = l * rescale + wave_sum(esum);
                STAGE_TS(21);
                m = m_new;
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                float4 os[NS];  // one accumulator per span: independent FMA chains
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    os[i] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (cnt[i] == 0) continue;
                    float ev[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4)
                        *(float4 *)&ev[4 * q4] = *(const float4 *)&sc[wave][i][pg * 16 + 4 * q4];
#pragma unroll
                    for (int q = 0; q < 16; ++q) {
                        const float4 v = raw4<KV>(raw[i].v[q]);
                        const float ei = ev[q];
                        os[i].x = fmaf(ei, v.x, os[i].x);
                        os[i].y = fmaf(ei, v.y, os[i].y);
                        os[i].z = fmaf(ei, v.z, os[i].z);
                        os[i].w = fmaf(ei, v.w, os[i].w);
                    }
                }
                o.x *= rescale;
                o.y *= rescale;
                o.z *= rescale;
                o.w *= rescale;
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    o.x += os[i].x;
                    o.y += os[i].y;
                    o.z += os[i].z;
                    o.w += os[i].w;
                }
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
            }
            STAGE_TS(22);
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
                STAGE_TS(23);
                const int nlive = min(4, spans - qq * 4);
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
                if (Qs == 1) {  // the head's output
                    ll_put(LL + kLLA + h * kHeadDim + lane, O / L, tag);
                } else {
                    uint64_t *dst = LL + kLLA + (size_t)unit * 66;
                    ll_put(dst + lane, O, tag);
                    if (lane == 0) {
                        ll_put(dst + 64, M, tag);
                        ll_put(dst + 65, L, tag);
                    }
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
            const bool own_x = attn_wg && layer > 0;  // no block-input gather: residual words
            uint64_t xw = 0;
            if (gs.storer()) {
                eb = a.proj_b[r];
                if (own_x)
                    xw = ll_load(LL + kLLO + r);
                else
                    eres = xin[r];
            }
            // workgroups without attention work wait ~0.85 us (2,048 clocks) before polling for
            // its output when an attention wave has more than one span (over 1.5 us of work
            // after its query arrives): their polls would share the coherent path with the
            // query hand-off meanwhile (global step 1.5-1.8 us shorter at ctx 512..767)
            if (!attn_wg && spans > 4) __builtin_amdgcn_s_sleep(32);
            if (Qs == 1) {  // the heads' outputs, ready to use
                const bool ok = ll_gather<3>(LL + kLLA, kHidden, tag, act, budget);
                if (sync_failed(!ok, &wait_failed)) {
                    if (t == 0) atomicOr(g.err, 1u);
                    return;
                }
                STAGE_TS(6);
            } else {
                const int units = kHeads * Qs;
                const bool ok = ll_gather<(kMaxUnits * 66 + 255) / 256>(LL + kLLA, units * 66, tag, pbuf, budget);
                if (sync_failed(!ok, &wait_failed)) {
                    if (t == 0) atomicOr(g.err, 1u);
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
            }
            if (own_x && gs.storer()) {  // stored a stage ago: current at the first look, else polled
                const uint32_t prev = ((uint32_t)(pos + 1) << 5) | (uint32_t)(layer - 1);
                bool okx = true;
                while ((uint32_t)(xw >> 32) != prev) {
                    if (--budget < 0) {
                        okx = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(kPollSleep);
                    xw = ll_load(LL + kLLO + r);
                }
                eres = __uint_as_float((uint32_t)xw);
                if (!okx) {  // the launch is reported failed and redone; its outputs are not used
                    atomicOr(g.err, 1u);
                    eres = __int_as_float(0x7fc00000);
                }
            }
            if constexpr (A8) {
                float *cp = b == 0 ? cap : nullptr;
                if (cp) {  // a barrier before the quantiser rewrites runs other threads copy
                    cap_copy(cp + MOSS_HIP_CAP_ATT, act, kHidden);
                    __syncthreads();
                }
                quant_act_lds_k<kHidden>(act, da);
                __syncthreads();
                if (cp) {
                    cap_copy(cp + MOSS_HIP_CAP_ATT_Q, act, kHidden);
                    cap_copy(cp + MOSS_HIP_CAP_ATT_D, da, kHidden / 32);
                }
            }
            STAGE_TS(7);
            const float yv = gs.template dot<A8>(act, part, da);
            // stage M's weights, after this wave's last read of them a block ago (barriers since)
            if (wave == kDmaWave) QStage::issue_wave(a.fc_in_w, b, wm_lds);
            if (gs.storer()) {
                ll_put(LL + kLLX + r, eres + (yv + eb), tag);  // llm.cpp:239
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_XM + r] = eres + (yv + eb);
            }
            STAGE_TS(8);
        }

        // ---- stage M: LN2 + fc_in + gelu_new, one wave per group, every workgroup
        {
            QStage gs;
            gs.setup(b, wm_lds);
            const int r = gs.row();
            const float eb = gs.storer() ? a.fc_in_b[r] : 0.0f;
            float lw[3], lb[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                lw[i] = a.ln2_w[t + 256 * i];
                lb[i] = a.ln2_b[t + 256 * i];
            }
            const bool ok = wave == kDmaWave || ll_gather_by<4, 192>(LL + kLLX, kHidden, tag, xm, budget, t);
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(g.err, 1u);
                return;
            }
            STAGE_TS(9);
            float o[3];
            layernorm_768_lds(xm, lw, lb, o);
#pragma unroll
            for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
            __syncthreads();
            if constexpr (A8) {
                float *cp = b == 0 ? cap : nullptr;
                if (cp) {  // a barrier before the quantiser rewrites runs other threads copy
                    cap_copy(cp + MOSS_HIP_CAP_LN2, act, kHidden);
                    __syncthreads();
                }
                quant_act_lds_k<kHidden>(act, da);
                __syncthreads();
                if (cp) {
                    cap_copy(cp + MOSS_HIP_CAP_LN2_Q, act, kHidden);
                    cap_copy(cp + MOSS_HIP_CAP_LN2_D, da, kHidden / 32);
                }
            }
            STAGE_TS(10);
            const float yv = gs.template dot<A8>(act, da);
            if (gs.storer()) {
                ll_put(LL + kLLH + r, gelu_new(yv + eb), tag);  // llm.cpp:243
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_H + r] = gelu_new(yv + eb);
            }
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
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(g.err, 1u);
                return;
            }
            if constexpr (A8) {
                quant_act_lds_k<kFF>(act, da);
                __syncthreads();
                if (b == 0 && cap) {
                    cap_copy(cap + MOSS_HIP_CAP_H_Q, act, kFF);
                    cap_copy(cap + MOSS_HIP_CAP_H_D, da, kFF / 32);
                }
            }
            STAGE_TS(12);
            const float yv = gs.template dot<A8>(act, part, da);
            if (gs.storer()) {
                ll_put(LL + kLLO + r, xm[r] + (yv + eb), tag);  // llm.cpp:245
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_XOUT + r] = xm[r] + (yv + eb);
            }
            STAGE_TS(13);
            if (layer == kLayers - 2) STAGE_TS(15);
            // the next block's QKV weights, after this wave's last use of stage Q's (barriers
            // since) and behind no gather of its own: the block-input gather is waves 0..2's
            if (wave == kDmaWave && b < kAttnBase && layer + 1 < kLayers)
                QStage::issue_wave(g.layers[layer + 1].attn_w, b, wq_lds);
        }

    }  // layer

    // ln_f (llm.cpp:254) on the last block's output, then the position moves on
    // (every workgroup read it before its first block: their outputs are in)
    if (b == 0) {
        const uint32_t last = ((uint32_t)(pos + 1) << 5) | (uint32_t)(kLayers - 1);
        const bool ok = ll_gather<3>(LL + kLLO, kHidden, last, xin, budget);
        if (sync_failed(!ok, &wait_failed)) {
            if (t == 0) atomicOr(g.err, 1u);
            return;
        }
        float o[3], lw[3], lb[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            lw[i] = g.lnf_w[t + 256 * i];
            lb[i] = g.lnf_b[t + 256 * i];
        }
        layernorm_768_lds(xin, lw, lb, o);
#pragma unroll
        for (int i = 0; i < 3; ++i) g.hidden[t + 256 * i] = o[i];
        if (t == 0) g.state->pos = pos + 1;
    }
    STAGE_FLUSH();
}

}  // namespace

hipError_t decode_layer_fits(int device, bool *fits) {
    *fits = false;
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return e;
    int per_cu16 = 0, per_cu32 = 0;
    for (int v = 0; v < 2; ++v) {  // the W8A16 and the W8A8 builds
        int p16 = 0, p32 = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &p16, v ? decode_global_kernel<KV_F16, true> : decode_global_kernel<KV_F16, false>, 256, 0);
        if (e != hipSuccess) return e;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &p32, v ? decode_global_kernel<KV_F32, true> : decode_global_kernel<KV_F32, false>, 256, 0);
        if (e != hipSuccess) return e;
        per_cu16 = v ? std::min(per_cu16, p16) : p16;
        per_cu32 = v ? std::min(per_cu32, p32) : p32;
    }
    int per_cu_local = 0;
    e = decode_local_occupancy(&per_cu_local);
    if (e != hipSuccess) return e;
    int per_cu = per_cu16 < per_cu32 ? per_cu16 : per_cu32;
    per_cu = per_cu < per_cu_local ? per_cu : per_cu_local;
    *fits = (long)per_cu * prop.multiProcessorCount >= kLayerGrid + 1;  // the local launch adds a gate workgroup
    return hipSuccess;
}

#ifdef MH_STAGE_TRACE
// [kLayerGrid][32] timestamps of the last launch (profiling builds only)
extern "C" int mh_stage_trace_read(unsigned long long *out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(mh_stage_ts), sizeof(mh_stage_ts));
}
#endif

hipError_t launch_decode_global(const GlobalArgs &a, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (!a.layers || !a.wte || !a.row || !a.lnf_w || !a.lnf_b || !a.hidden || !a.state || !a.ll || !a.err)
        return hipErrorInvalidValue;
    for (int ch = 0; ch < kNVq; ++ch)
        if (!a.aemb[ch]) return hipErrorInvalidValue;
    if (kv == KV_F16) {
        if (a.a8)
            hipLaunchKernelGGL((decode_global_kernel<KV_F16, true>), dim3(kLayerGrid), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((decode_global_kernel<KV_F16, false>), dim3(kLayerGrid), dim3(256), 0, s, a);
    } else {
        if (a.a8)
            hipLaunchKernelGGL((decode_global_kernel<KV_F32, true>), dim3(kLayerGrid), dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((decode_global_kernel<KV_F32, false>), dim3(kLayerGrid), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

}  // namespace mh
