// decode_local.hip -- one step of the local transformer of the single-stream decode in one launch (gfx950).
//
// Replaces local_step (reference csrc/src/llm.cpp:259-264: block_forward of the
// one local layer at local position lpos, llm.cpp:230-246) and, for the
// channel steps, the channel's audio head (audio_logits, llm.cpp:686-688:
// logits = aemb[ch] . local_ln_f(x)).  The stages hand their outputs on through
// LL words (mh_ll.h), as in decode_layer.hip:
//   Q  lpos 0 only, b < 144: LN1 + QKV of the block input (the global hidden
//      state), RoPE, k/v into the local cache                  -> LL q|k|v
//   A  b < 12: head h = b: the step's input -- for lpos >= 2 the code of the
//      previous channel, picked here (greedy: penalised argmax of its logits,
//      or the forced code) or written by the sampler -- and the head's q|k|v:
//      from the QKV stage (lpos 0) or from the precomputed row of (lpos,
//      code); k/v into the local cache; the head's attention over keys
//      0..lpos (at most 17)                                    -> LL attn + code
//   P  b < 192: proj + residual (the raw input row is aemb[ch][code]) -> LL x + attn
//   M  b < 192: LN2 + fc_in + gelu_new                          -> LL h
//   F  b < 192: fc_out + residual -> x_out (memory) and, with a head, LL x_out
//   H  b < 64, with a head: local ln_f + the audio head GEMV   -> logits (memory)
// (192 workgroups, one per CU; the GEMV stages take one wave per 4-row group,
// or four for the K slices of proj and fc_out).
//
// Precomputed q|k|v rows.  For lpos >= 1 the block input is an embedding row
// -- wte[slot] at lpos 1, aemb[lpos - 2][code] at lpos >= 2 -- and RoPE uses
// the fixed position lpos, so q|k|v = RoPE_lpos(attn_w . LN1(row) + attn_b) is
// a function of (lpos, code) only.  The host computes every such row once, at
// load, with the one-GEMV kernel of the per-operator path (the same per-row
// arithmetic), so the table holds exactly the values that path computes live.
#include "mh_gemv.h"
#include "mh_ll.h"
#include "mh_ops.h"

namespace mh {
namespace {

// LL regions (words); consecutive launches differ in lpos, so in tag
constexpr int kLQ = 0;                  // q | k | v (lpos 0)
constexpr int kLA = kLQ + 3 * kHidden;  // attention output (768) and the step's input code (1)
constexpr int kLX = kLA + kHidden + 1;  // x after the attention sub-block
constexpr int kLH = kLX + kHidden;      // fc_in output
constexpr int kLO = kLH + kFF;          // block output (head input)
constexpr int kLL = kLO + kHidden;      // head logits, the next step's pick input (1024)
constexpr int kLG = kLL + kCodebook;    // position 0's block output, the end gate's input (768)
static_assert(kLG + kHidden <= kLayerWords, "local LL layout fits the exchange buffer");

// Stage timestamps (100 MHz device clock) of the last launch, per workgroup,
// in builds with -DMH_STAGE_TRACE only.
#ifdef MH_STAGE_TRACE
}  // namespace
__device__ unsigned long long mh_local_ts[kLayerGrid][32];
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
            for (int i_ = 0; i_ < 32; ++i_) mh_local_ts[blockIdx.x][i_] = stage_ts_lds[i_]; \
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

// A8: every GEMV in W8A8 (quant_act_lds), the reference's decode with MOSS_A16 unset.
template <bool A8>
__global__ __launch_bounds__(256) void decode_local_kernel(LocalArgs a) {
#pragma clang fp contract(off)
    __shared__ float act[kFF + 1];
    __shared__ float da[kFF / 32];  // block scales of act (A8)
    __shared__ float xm[kHidden];
    __shared__ float qkv[3 * kHidden];             // q | k | v of this position
    __shared__ float sc[kHeads][kLocalLen + 1];
    __shared__ float part[4][4];
    __shared__ float pbv[4];
    __shared__ int pbi[4];
    __shared__ int used_s;
    __shared__ float lgt[kCodebook];  // the previous step's logits (chained launches)
    __shared__ GateLds gl;

    __shared__ int wait_failed;  // set when a wait of this workgroup runs out
    if (threadIdx.x == 0) wait_failed = 0;
    __syncthreads();
    STAGE_DECL;
    STAGE_TS(0);
    DevState *st = a.state;
    if (st->stop) return;  // written only between frames: the same for every workgroup
    const uint32_t tag_base = (uint32_t)(st->pos + 1) << 5;
    int budget = a.poll_budget > 0 ? a.poll_budget : kPollBudget;
    uint64_t *LL = a.ll;

    // ---- the end gate (llm.cpp:653-679) in a workgroup of its own (the last):
    // ln_f of position 0's block output, the 2-row W8A8 gate, the stop rule.  The
    // channel steps do not wait for it: a frame the gate ends is dropped by the
    // host, and every state it touches is rewritten before it is read again.
    if (a.gate && (int)blockIdx.x == kLayerGrid) {
        const int t = threadIdx.x;
        float lw[3], lb[3];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            lw[i] = a.lnf_w[t + 256 * i];
            lb[i] = a.lnf_b[t + 256 * i];
        }
        const bool ok = ll_gather<3>(LL + kLG, kHidden, tag_base | 12u, xm, budget);
        if (sync_failed(!ok, &wait_failed)) {
            if (t == 0) atomicOr(a.err, 1u);
            return;
        }
        float o[3];
        layernorm_768_lds(xm, lw, lb, o);
#pragma unroll
        for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
        __syncthreads();
        gate_block(act, a.wte, st, gl);
        return;
    }

#pragma unroll 1
    for (int lpos = a.lpos; lpos <= a.lpos_last; ++lpos) {
        const int n = lpos + 1;
        const uint32_t tag = tag_base | (uint32_t)(12 + lpos);
        // per-step copies of the indices: nothing derived from them is held across steps
        const int t = tix();
        const int b = bix();
        const int ch_in = lpos >= 2 ? lpos - 2 : -1;  // channel whose code is this step's input
        const uint8_t *aemb_in = ch_in >= 0 ? a.aemb[ch_in] : nullptr;
        const uint8_t *head_w = a.head && lpos >= 1 ? a.aemb[lpos - 1] : nullptr;
        float *logits_out = lpos >= 1 ? a.logits + (size_t)(lpos - 1) * kCodebook : nullptr;
        const bool live = lpos == 0;  // the block input is the global hidden state: QKV computed here
        const bool picking = !live && ch_in >= 0 && a.pick;
        const bool pick_ll = picking && lpos > a.lpos;  // logits from this launch's previous step
        // W8A8 quantiser capture of this position (tests only; null in the library's own use)
        float *const cap = A8 && a.cap ? a.cap + (size_t)lpos * MOSS_HIP_CAP_STEP : nullptr;

        // ---- stage Q (lpos 0): LN1 + QKV of the block input, one wave per group
        if (live) {
            if (b < 3 * kHidden / 16) {
                GemvStage<1, 6, kHidden> gs;
                gs.prefetch(a.attn_w, b);
                const int r = gs.row();
                QkvEpi e;
                if (gs.storer()) e.load(a.attn_b, a.rope_cos, a.rope_sin, r, lpos);
                float o[3], lw[3], lb[3];
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    xm[t + 256 * i] = a.x_in[t + 256 * i];
                    lw[i] = a.ln1_w[t + 256 * i];
                    lb[i] = a.ln1_b[t + 256 * i];
                }
                __syncthreads();
                layernorm_768_lds(xm, lw, lb, o);
#pragma unroll
                for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
                __syncthreads();
                if constexpr (A8) {
                    float *cp = b == 0 ? cap : nullptr;  // (uniform)
                    if (cp) {
                        cap_copy(cp + MOSS_HIP_CAP_XIN, xm, kHidden);
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
                const float yv = gs.template dot<A8>(act, part, da);
                const float partner = xshfl<4>(yv);
                if (gs.storer()) ll_put(LL + kLQ + r, e.apply(r, yv, partner), tag);  // k, v cached by stage A
                __syncthreads();
            }
        }

        // ---- stage A (b < 12): head h = b of the local attention (llm.cpp:189-217
        // over the local cache, keys 0..lpos) in the reference's order:
        // s_p = (q_h . k_p) * 0.125 summed over d in order; e_p = exp(s_p - max),
        // the in-order sum, w_p = e_p * (1 / sum); o[d] = sum_p w_p v_p[d] in order.
        // Wave 0 computes: lane p < 17 a score, lane d the output dimension d.
        if (b < kHeads) {
            const int h = b, lane = t & 63;
            const bool w0 = t < 64;
            const int kmax = max(lpos - 1, 0);
            // loads complete in issue order: the pick's logits first
            PickIn pin;
            if (picking) {
                if (pick_ll) {  // counts now, values once the previous step's head has stored them
#pragma unroll
                    for (int k = 0; k < kCodebook / 256; ++k)
                        pin.cnt[k] = st->rep_penalty != 1.0f ? a.counts[(size_t)ch_in * kCodebook + t + 256 * k] : 0;
                } else {
                    greedy_pick_load(a.logits + (size_t)ch_in * kCodebook, a.counts + (size_t)ch_in * kCodebook,
                                     st->rep_penalty, pin);
                }
            }
            // the cache rows (keys 0 .. lpos-1, written by earlier launches) before
            // anything else; the key at lpos, and the clamped ones past it, take
            // this step's row below
            float4 kr[kHeadDim / 4];
            float vv[kLocalLen];
            if (w0) {
                const float *krow = a.lk + ((size_t)h * kLocalLen + min(lane, kmax)) * kHeadDim;
#pragma unroll
                for (int c = 0; c < kHeadDim / 4; ++c) kr[c] = *(const float4 *)(krow + 4 * c);
#pragma unroll
                for (int p = 0; p < kLocalLen; ++p) vv[p] = a.lv[((size_t)h * kLocalLen + min(p, kmax)) * kHeadDim + lane];
            }
            // q, k, v of head h at lpos
            if (live) {
                const int seg = min(t >> 6, 2), i = seg * kHidden + h * kHeadDim + (t & 63);
                const bool ok = ll_wait1(LL + kLQ + i, t < 3 * kHeadDim, tag, &qkv[i], budget);
                // this position's k, v into the local cache (llm.cpp:224-225) by the workgroup
                // that reads them at the later positions: same-workgroup ordering, no fence
                if (ok && t < 3 * kHeadDim && seg > 0)
                    (seg == 1 ? a.lk : a.lv)[((size_t)h * kLocalLen + lpos) * kHeadDim + (t & 63)] = qkv[i];
                if (sync_failed(!ok, &wait_failed)) {
                    if (t == 0) atomicOr(a.err, 1u);
                    return;
                }
            } else {
                const float *row = a.qkv_table;  // lpos 1: wte[slot]
                if (ch_in >= 0) {
                    int used;
                    if (picking) {  // greedy pick of channel ch_in (llm.cpp:689-697)
                        if (pick_ll) {
                            // waves 1-3 poll the logits: wave 0's cache-row loads, issued
                            // above, would hold back its polls (loads complete in order)
                            bool ok = true;
                            if (t >= 64)
                                ok = ll_gather_by<(kCodebook + 191) / 192, 192>(LL + kLL, kCodebook, tag - 1, lgt,
                                                                                 budget, t - 64);
                            if (sync_failed(!ok, &wait_failed)) {
                                if (t == 0) atomicOr(a.err, 1u);
                                return;
                            }
#pragma unroll
                            for (int k = 0; k < kCodebook / 256; ++k) pin.vals[k] = lgt[t + 256 * k];
                        }
                        int idx = greedy_pick_reduce(pin, st->rep_penalty, pbv, pbi);
                        if (idx >= kCodebook) idx = 0;
                        used = st->forced_on ? a.forced[st->frame * kNVq + ch_in] : idx;
                        if (b == 0 && t == 0) {
                            st->codes[ch_in] = idx;
                            st->row[ch_in + 1] = used;
                        }
                    } else {  // written by the sampler of channel ch_in
                        if (t == 0) used_s = st->row[ch_in + 1];
                        __syncthreads();
                        used = used_s;
                    }
                    if (b == 0 && t == 0) ll_put(LL + kLA + kHidden, __int_as_float(used), tag);  // for stage P
                    row = a.qkv_table + (1 + (size_t)ch_in * kCodebook + used) * 3 * kHidden;
                }
                STAGE_TS(1);
                if (t < 3 * kHeadDim) {
                    const int seg = t >> 6, i = seg * kHidden + h * kHeadDim + (t & 63);
                    const float v = row[i];
                    qkv[i] = v;
                    if (seg > 0)  // this position's k, v into the local cache (llm.cpp:224-225), for later steps
                        (seg == 1 ? a.lk : a.lv)[((size_t)h * kLocalLen + lpos) * kHeadDim + (t & 63)] = v;
                }
                __syncthreads();
            }
            STAGE_TS(2);
            if constexpr (A8)
                if (cap && t < 3 * kHeadDim) {
                    const int i = (t >> 6) * kHidden + h * kHeadDim + (t & 63);
                    cap[MOSS_HIP_CAP_QKV + i] = qkv[i];
                }
            if (w0) {
                const float *qh = &qkv[h * kHeadDim];
                if (min(lane, n - 1) == lpos)
#pragma unroll
                    for (int c = 0; c < kHeadDim / 4; ++c) kr[c] = *(const float4 *)&qkv[kHidden + h * kHeadDim + 4 * c];
                float dot = 0.0f;
#pragma unroll
                for (int c = 0; c < kHeadDim / 4; ++c) {
                    const float4 qv = *(const float4 *)(qh + 4 * c);
                    dot = dot + qv.x * kr[c].x;
                    dot = dot + qv.y * kr[c].y;
                    dot = dot + qv.z * kr[c].z;
                    dot = dot + qv.w * kr[c].w;
                }
                dot *= 0.125f;
                if (lane < kLocalLen) sc[0][lane] = dot;
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                float sv[kLocalLen];
#pragma unroll
                for (int p = 0; p < kLocalLen; ++p) sv[p] = sc[0][p];
                float mx = -1e30f;
#pragma unroll
                for (int p = 0; p < kLocalLen; ++p)
                    if (p < n) mx = fmaxf(mx, sv[p]);
                const float e = lane < n ? expf(dot - mx) : 0.0f;
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                if (lane < kLocalLen) sc[0][lane] = e;
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int p = 0; p < kLocalLen; ++p) sv[p] = sc[0][p];
                float sum = 0.0f;
#pragma unroll
                for (int p = 0; p < kLocalLen; ++p)
                    if (p < n) sum += sv[p];
                const float wgt = e * (1.0f / sum);  // 0 for keys past n
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                if (lane < kLocalLen) sc[0][lane] = wgt;
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                const float vnew = qkv[2 * kHidden + h * kHeadDim + lane];
                float o = 0.0f;
#pragma unroll
                for (int p = 0; p < kLocalLen; ++p) o = o + sc[0][p] * (min(p, n - 1) == lpos ? vnew : vv[p]);
                ll_put(LL + kLA + h * kHeadDim + lane, o, tag);
            }
            STAGE_TS(3);
            __syncthreads();
        }

        // ---- stage P: proj + residual (4 waves per group)
        if (b < kHidden / 4) {
            GemvStage<4, 2, kHidden> gs;
            gs.prefetch(a.proj_w, b);
            const int r = gs.row();
            const float eb = gs.storer() ? a.proj_b[r] : 0.0f;
            const bool with_code = !live && ch_in >= 0;  // the raw input row is aemb[ch_in][used]
            float eres = 0.0f;
            if (gs.storer() && !with_code) eres = (live ? a.x_in : a.x_slot)[r];
            const bool ok = ll_gather<(kHidden + 1 + 255) / 256>(LL + kLA, kHidden + (with_code ? 1 : 0), tag, act, budget);
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(a.err, 1u);
                return;
            }
            if (gs.storer() && with_code)  // lookup_row (llm.cpp:697)
                eres = q8x4_elem(aemb_in, kHidden / 32, __float_as_int(act[kHidden]), r);
            if constexpr (A8) {  // act[0, 768) only: the code at act[kHidden] stays
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
            const float yv = gs.template dot<A8>(act, part, da);
            if (gs.storer()) {
                ll_put(LL + kLX + r, eres + (yv + eb), tag);  // llm.cpp:239
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_XM + r] = eres + (yv + eb);
            }
            STAGE_TS(4);
            __syncthreads();  // act is reused by stage F
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
            const bool ok = ll_gather<3>(LL + kLX, kHidden, tag, xm, budget);
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(a.err, 1u);
                return;
            }
            STAGE_TS(5);
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
            const float yv = gs.template dot<A8>(act, part, da);
            if (gs.storer()) {
                ll_put(LL + kLH + r, gelu_new(yv + eb), tag);  // llm.cpp:243
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_H + r] = gelu_new(yv + eb);
            }
            STAGE_TS(6);
            __syncthreads();  // every wave is done with act before stage F gathers into it
        }

        // ---- stage F: fc_out + residual (4 waves per group)
        if (b < kHidden / 4) {
            GemvStage<4, 6, kFF> gs;
            gs.prefetch(a.fc_out_w, b);
            const int r = gs.row();
            const float eb = gs.storer() ? a.fc_out_b[r] : 0.0f;
            ll_gather_slice<kFF>(LL + kLH, tag, act, budget, &wait_failed);
            if constexpr (A8) {  // the slice's 24 blocks, quantised by the wave that reads them
                const int w = __builtin_amdgcn_readfirstlane(t >> 6);
                quant_act_lds_k<kFF / 4, 64>(act + (kFF / 4) * w, da + (kFF / 128) * w, t & 63);
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                if (b == 0 && cap) {
                    __syncthreads();
                    cap_copy(cap + MOSS_HIP_CAP_H_Q, act, kFF);
                    cap_copy(cap + MOSS_HIP_CAP_H_D, da, kFF / 32);
                }
            }
            STAGE_TS(7);
            const float yv = gs.template dot<A8>(act, part, da);
            if (*(volatile int *)&wait_failed) {  // read after the dot's barriers
                if (t == 0) atomicOr(a.err, 1u);
                return;
            }
            if (gs.storer()) {
                const float xo = xm[r] + (yv + eb);  // llm.cpp:245
                a.x_out[r] = xo;
                if constexpr (A8)
                    if (cap) cap[MOSS_HIP_CAP_XOUT + r] = xo;
                if (head_w) ll_put(LL + kLO + r, xo, tag);
                if (live && a.gate) ll_put(LL + kLG + r, xo, tag);  // the gate workgroup's input
            }
            STAGE_TS(8);
            __syncthreads();
        }

        // ---- stage H: local ln_f + audio head (4 waves per group)
        if (head_w && b < kCodebook / 16) {
            GemvStage<1, 6, kHidden> gs;
            gs.prefetch(head_w, b);
            float lw[3], lb[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) {
                lw[i] = a.lnf_w[t + 256 * i];
                lb[i] = a.lnf_b[t + 256 * i];
            }
            const bool ok = ll_gather<3>(LL + kLO, kHidden, tag, xm, budget);
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(a.err, 1u);
                return;
            }
            STAGE_TS(9);
            float o[3];
            layernorm_768_lds(xm, lw, lb, o);  // normalize(lx, local_lnf) (llm.cpp:262)
#pragma unroll
            for (int i = 0; i < 3; ++i) act[t + 256 * i] = o[i];
            __syncthreads();
            if constexpr (A8) {
                float *cp = b == 0 ? cap : nullptr;
                if (cp) {  // a barrier before the quantiser rewrites runs other threads copy
                    cap_copy(cp + MOSS_HIP_CAP_LNF, act, kHidden);
                    __syncthreads();
                }
                quant_act_lds_k<kHidden>(act, da);
                __syncthreads();
                if (cp) {
                    cap_copy(cp + MOSS_HIP_CAP_LNF_Q, act, kHidden);
                    cap_copy(cp + MOSS_HIP_CAP_LNF_D, da, kHidden / 32);
                }
            }
            const float yv = gs.template dot<A8>(act, part, da);
            if (gs.storer()) {
                logits_out[gs.row()] = yv;
                if (lpos < a.lpos_last || a.final_pick) ll_put(LL + kLL + gs.row(), yv, tag);  // the next pick
            }
            STAGE_TS(10);
        }

        // ---- after the last position: the greedy pick of its channel, as
        // sample_kernel does for the last channel (workgroup 0)
        if (a.final_pick && lpos == a.lpos_last && b == 0) {
            const int ch = lpos - 1;
            PickIn pin;
#pragma unroll
            for (int k = 0; k < kCodebook / 256; ++k)
                pin.cnt[k] = st->rep_penalty != 1.0f ? a.counts[(size_t)ch * kCodebook + t + 256 * k] : 0;
            const bool ok = ll_gather<kCodebook / 256>(LL + kLL, kCodebook, tag, lgt, budget);
            if (sync_failed(!ok, &wait_failed)) {
                if (t == 0) atomicOr(a.err, 1u);
                return;
            }
#pragma unroll
            for (int k = 0; k < kCodebook / 256; ++k) pin.vals[k] = lgt[t + 256 * k];
            int idx = greedy_pick_reduce(pin, st->rep_penalty, pbv, pbi);
            if (idx >= kCodebook) idx = 0;
            const int used = st->forced_on ? a.forced[st->frame * kNVq + ch] : idx;
            if (t < ch) a.counts[(size_t)t * kCodebook + st->row[t + 1]] += 1;  // the frame's earlier channels
            if (t == 0) {
                st->codes[ch] = idx;
                st->row[ch + 1] = used;
                a.counts[(size_t)ch * kCodebook + used] += 1;
                st->row[0] = kSlotToken;
                st->frame += 1;
            }
        }
    }  // lpos
    STAGE_FLUSH();
}

}  // namespace

#ifdef MH_STAGE_TRACE
// [kLayerGrid][32] timestamps of the last launch (profiling builds only)
extern "C" int mh_local_trace_read(unsigned long long *out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(mh_local_ts), sizeof(mh_local_ts));
}
#endif

hipError_t decode_local_occupancy(int *per_cu) {
    int p16 = 0, p8 = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&p16, decode_local_kernel<false>, 256, 0);
    if (e != hipSuccess) return e;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&p8, decode_local_kernel<true>, 256, 0);
    *per_cu = p16 < p8 ? p16 : p8;
    return e;
}

hipError_t launch_decode_local(const LocalArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (!a.attn_w || !a.proj_w || !a.fc_in_w || !a.fc_out_w || !a.lk || !a.lv || !a.state || !a.ll || !a.err ||
        !a.x_out || a.lpos < 0 || a.lpos_last < a.lpos || a.lpos_last >= kLocalLen)
        return hipErrorInvalidValue;
    if (a.head && (!a.logits || !a.lnf_w || !a.lnf_b)) return hipErrorInvalidValue;
    for (int p = a.lpos < 1 ? 1 : a.lpos; p <= a.lpos_last; ++p)  // aemb rows: inputs (p >= 2) and heads
        if ((p >= 2 && !a.aemb[p - 2]) || (a.head && !a.aemb[p - 1])) return hipErrorInvalidValue;
    if (a.lpos == 0 && (!a.x_in || !a.rope_cos || !a.rope_sin)) return hipErrorInvalidValue;
    if (a.gate && (a.lpos != 0 || !a.wte || !a.lnf_w || !a.lnf_b)) return hipErrorInvalidValue;
    if (a.lpos_last >= 1 && !a.qkv_table) return hipErrorInvalidValue;
    if (a.lpos <= 1 && a.lpos_last >= 1 && !a.x_slot) return hipErrorInvalidValue;
    if (a.lpos_last >= 2 && a.pick && (!a.logits || !a.counts || !a.forced)) return hipErrorInvalidValue;
    // a chained pick reads the previous step's head: every step but the last runs one
    if (a.lpos_last > a.lpos && a.lpos_last >= 2 && a.pick && !a.head) return hipErrorInvalidValue;
    if (a.final_pick && (!a.pick || !a.head || a.lpos_last < 1 || !a.counts || !a.forced)) return hipErrorInvalidValue;
    // one more workgroup for the end gate
    if (a.a8)
        hipLaunchKernelGGL(decode_local_kernel<true>, dim3(kLayerGrid + (a.gate ? 1 : 0)), dim3(256), 0, s, a);
    else
        hipLaunchKernelGGL(decode_local_kernel<false>, dim3(kLayerGrid + (a.gate ? 1 : 0)), dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace mh
