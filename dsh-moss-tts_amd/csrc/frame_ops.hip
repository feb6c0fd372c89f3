// frame_ops.hip -- the small per-step kernels around the GEMVs (gfx950).
#include "mh_ops.h"

namespace mh {
namespace {

// x = deq(wte[row[0]]) + sum over ch of deq(aemb[ch][row[ch+1]]), pads skipped,
// channels added in order (reference csrc/src/llm.cpp:148-157).  Each element is
// an independent serial fp32 sum, so this is bit-identical to the reference.
// One thread per column (12 workgroups of 64); the 17 gathers are issued
// unconditionally (skipped channels read row 0 and are not added) so they are
// all in flight together.
__global__ __launch_bounds__(64) void embed_kernel(EmbedArgs a) {
    const bool stopped = a.state != nullptr && a.state->stop;  // tested before the store
    const int nb = kHidden / 32;
    const int c = blockIdx.x * 64 + threadIdx.x;
    float e[kNVq];
    bool use[kNVq];
#pragma unroll
    for (int ch = 0; ch < kNVq; ++ch) {
        const int code = a.row[ch + 1];
        use[ch] = !(code == kAudioPad || code < 0 || code >= kCodebook);
        e[ch] = q8x4_elem(a.aemb[ch], nb, use[ch] ? code : 0, c);
    }
    float v = q8x4_elem(a.wte, nb, a.row[0], c);
#pragma unroll
    for (int ch = 0; ch < kNVq; ++ch)
        if (use[ch]) v = v + e[ch];
    if (!stopped) a.x[c] = v;
}

__global__ __launch_bounds__(256) void layernorm_kernel(const float *x, const float *w, const float *b, float *out,
                                                        DevState *state, int bump_pos) {
    __shared__ float red[4];
    const bool stopped = state != nullptr && state->stop;  // tested before the stores
    const int t = threadIdx.x;
    float v[3], o[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = x[t + 256 * i];
    layernorm_768(v, w, b, o, red);
    if (stopped) return;
#pragma unroll
    for (int i = 0; i < 3; ++i) out[t + 256 * i] = o[i];
    if (bump_pos && t == 0) state->pos += 1;
}

// Rows outside [0, mat_rows) produce NaN instead of reading outside the matrix.
__global__ __launch_bounds__(256) void dequant_rows_kernel(const uint8_t *w, int mat_rows, int cols, const int *rows,
                                                           float *out) {
    const int r = rows[blockIdx.x];
    const int nb = cols / 32;
    const bool ok = r >= 0 && r < mat_rows;
    for (int c = threadIdx.x; c < cols; c += 256)
        out[(size_t)blockIdx.x * cols + c] = ok ? q8x4_elem(w, nb, r, c) : __int_as_float(0x7fc00000);
}

// ---- sample_token (reference csrc/src/sampler.cpp:9-79) for one 1024-entry
// logit row, by one 256-thread workgroup.  The caller has applied the
// repetition penalty into vals[] (LDS).

struct PickLds {
    float vals[kCodebook];     // penalised (then temperature-scaled) logits
    uint64_t keys[kCodebook];  // sort keys: value descending, index ascending
    float ex[kCodebook];       // exp(v - max) of the candidates, in sorted order
    float bv[4];
    int bi[4];
    int pick;
    int used;
};

// Greedy branch (sampler.cpp:23-28): argmax, the lowest index wins ties, NaN values
// never win; index 0 when the value at index 0 is NaN or every value is NaN (the
// reference's scan compares with its best so far, so it never moves off a NaN at 0).
__device__ int pick_greedy(PickLds &L) {
    const int t = threadIdx.x;
    float best = -INFINITY;
    int besti = kCodebook;
    for (int i = t; i < kCodebook; i += 256) {  // ascending i per thread
        const float v = L.vals[i];
        if (v > best) {
            best = v;
            besti = i;
        }
    }
    wave_argmax(best, besti);
    if ((t & 63) == 0) {
        L.bv[t >> 6] = best;
        L.bi[t >> 6] = besti;
    }
    __syncthreads();
    if (t == 0) {
        float b = L.bv[0];
        int idx = L.bi[0];
        for (int w = 1; w < 4; ++w)
            if (L.bv[w] > b || (L.bv[w] == b && L.bi[w] < idx)) {
                b = L.bv[w];
                idx = L.bi[w];
            }
        L.pick = (idx >= kCodebook || L.vals[0] != L.vals[0]) ? 0 : idx;
    }
    __syncthreads();
    return L.pick;
}

// Order-preserving map of a float to uint32 (larger float -> larger key).
__device__ __forceinline__ uint32_t float_order(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Sampling branch (sampler.cpp:30-78): temperature, top-k by a full sort
// (value descending; equal values by index), softmax over the k candidates,
// top-p cut, one uniform draw walked down the sorted candidates.  The
// sequential sums run in one thread in the reference's order.
__device__ int pick_sampled(PickLds &L, const SampleCfg &c, uint32_t *rng) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    const bool scale = c.temperature > 0.0f && c.temperature != 1.0f;
    const float inv = scale ? 1.0f / c.temperature : 1.0f;
    for (int i = t; i < kCodebook; i += 256) {
        float v = L.vals[i];
        if (scale) v = v * inv;
        L.vals[i] = v;
        L.keys[i] = ((uint64_t)(~float_order(v)) << 32) | (uint32_t)i;
    }
    __syncthreads();
    // bitonic sort, ascending keys
    for (int k = 2; k <= kCodebook; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = t; i < kCodebook; i += 256) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t a = L.keys[i], b = L.keys[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) {
                        L.keys[i] = b;
                        L.keys[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    const int n = c.top_k > 0 ? (c.top_k < kCodebook ? c.top_k : kCodebook) : kCodebook;
    const float maxv = L.vals[(int)(L.keys[0] & 0xffffffffu)];
    for (int i = t; i < n; i += 256) L.ex[i] = expf(L.vals[(int)(L.keys[i] & 0xffffffffu)] - maxv);
    __syncthreads();
    if (t == 0) {
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) sum += L.ex[i];
        int cnt = n;
        if (c.top_p < 1.0f) {
            float cum = 0.0f;
            int keep = 0;
            for (; keep < n; ++keep) {
                cum += L.ex[keep] / sum;
                if (cum >= c.top_p) {
                    ++keep;
                    break;
                }
            }
            cnt = keep > 1 ? keep : 1;
            sum = 0.0f;
            for (int i = 0; i < cnt; ++i) sum += L.ex[i];
        }
        float r = rng_uniform(rng) * sum;
        int pick = (int)(L.keys[cnt - 1] & 0xffffffffu);
        for (int i = 0; i < cnt; ++i) {
            r -= L.ex[i];
            if (r <= 0.0f) {
                pick = (int)(L.keys[i] & 0xffffffffu);
                break;
            }
        }
        L.pick = pick;
    }
    __syncthreads();
    return L.pick;
}

// vals[i] = logits[i] with the repetition penalty applied once per past
// occurrence of i (sampler.cpp:13-21: v<0 ? v*p : v/p, repeated).  Each index
// is penalised independently, so per-index counts reproduce the reference's
// walk over the history exactly.
__device__ void load_penalised(PickLds &L, const float *logits, const int *counts, float p) {
#pragma clang fp contract(off)
    for (int i = threadIdx.x; i < kCodebook; i += 256) {
        float v = logits[i];
        if (p != 1.0f) {
            const int c = counts[i];
            for (int k = 0; k < c; ++k) v = v < 0.0f ? v * p : v / p;
        }
        L.vals[i] = v;
    }
    __syncthreads();
}

// End gate (reference csrc/src/llm.cpp:274-285 + :30-35 + :678):
//  1. h = LayerNorm(x; local lnf)                     (the local step's output)
//  2. W8A8 quantisation of h per 32-block            (csrc/src/quant.cpp:28-43):
//     d = amax/127, id = 1/d, q = clamp(rint(h*id), +-127), scale kept as fp32 d
//  3. rows 7 (end) and 9 (slot) of wte dotted in the AVX2 order of
//     row_dot_q8_4x4 (csrc/src/gemv_avx2.cpp:105-121): 8 lane accumulators, lane j
//     takes the exact int32 sum of bytes 4j..4j+3 of each block, fma'd with
//     (d_w * d_a); then the 8 lanes are summed as _mm256 hsum does.
//  4. stop = frame >= min_frames && end_reached(l_slot, l_end)  (llm.cpp:30-35,678)
// Integer parts are exact and the fp32 operation order is the reference's, so
// the gate values are bit-identical to the reference given the same h.
__global__ __launch_bounds__(256) void gate_kernel(const float *x_raw, const float *lnf_w, const float *lnf_b,
                                                   const uint8_t *wte, DevState *state) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    __shared__ float hbuf[kHidden];
    __shared__ GateLds g;
    const bool stopped = state->stop;  // tested once the input is loaded
    const int t = threadIdx.x;
    float v[3], o[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = x_raw[t + 256 * i];
    if (stopped) return;
    layernorm_768(v, lnf_w, lnf_b, o, red);
#pragma unroll
    for (int i = 0; i < 3; ++i) hbuf[t + 256 * i] = o[i];
    __syncthreads();
    gate_block(hbuf, wte, state, g);
}

// End gate of a frame whose gate is dumped (llm.cpp:653-679): the reference then
// computes the whole text head (text_logits = gemv over wte, the caller's GEMV)
// and takes l_slot, l_end from it, plus the argmax over all 16384 logits (the
// first maximum wins).  The stop rule is end_reached as in gate_kernel.
__global__ __launch_bounds__(256) void gate_text_kernel(const float *logits, DevState *state) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    if (state->stop) return;
    const int t = threadIdx.x;
    float best = -INFINITY;
    int besti = kVocab;
    for (int i = t; i < kVocab; i += 256) {
        const float v = logits[i];
        if (v > best) {
            best = v;
            besti = i;
        }
    }
    wave_argmax(best, besti);
    if ((t & 63) == 0) {
        bv[t >> 6] = best;
        bi[t >> 6] = besti;
    }
    __syncthreads();
    if (t == 0) {
        float b = bv[0];
        int idx = bi[0];
        for (int w = 1; w < 4; ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < idx)) {
                b = bv[w];
                idx = bi[w];
            }
        if (idx >= kVocab || logits[0] != logits[0]) {  // NaN at 0 (or all NaN): the reference's scan keeps index 0
            idx = 0;
            b = logits[0];
        }
        const float l_end = logits[kEndToken], l_slot = logits[kSlotToken];
        state->gate[0] = l_end;
        state->gate[1] = l_slot;
        state->gate_argmax = idx;
        state->gate_argmax_v = b;
        if (state->frame >= state->min_frames && end_reached(l_slot, l_end, state->cfg, state->rng)) state->stop = 1;
    }
}

// One pick of channel ch (reference csrc/src/sampler.cpp:9-79 as called from
// llm.cpp:689-697): repetition penalty over this generate()'s used codes,
// greedy (SampleParams::greedy, top_k == 1 or frame < greedy_frames) or
// sampled with the call's xoshiro stream.  Then the used code (forced under
// teacher forcing) is counted into the history, written into the next
// global-step row, and its aemb row becomes the next local input.
__global__ __launch_bounds__(256) void sample_kernel(SampleArgs a) {
    __shared__ PickLds L;
    DevState *st = a.state;
    const bool stopped = st->stop;  // tested once the logits are loaded
    const int t = threadIdx.x;
    load_penalised(L, a.logits, a.counts + a.ch * kCodebook, st->rep_penalty);
    if (stopped) return;
    const SampleCfg c = st->cfg;
    const bool greedy = c.greedy || st->frame < c.greedy_frames;
    const int idx = greedy ? pick_greedy(L) : pick_sampled(L, c, st->rng);
    if (a.count_all && t < a.ch) a.counts[t * kCodebook + st->row[t + 1]] += 1;  // one channel per thread
    if (t == 0) {
        const int used = st->forced_on ? a.forced[st->frame * kNVq + a.ch] : idx;
        st->codes[a.ch] = idx;
        st->row[a.ch + 1] = used;
        a.counts[a.ch * kCodebook + used] += 1;
        L.used = used;
        if (a.last_channel) {
            st->row[0] = kSlotToken;
            st->frame += 1;
        }
    }
    __syncthreads();
    const int used = L.used;
    const int nb = kHidden / 32;
    for (int c2 = t; c2 < kHidden; c2 += 256) a.next_input[c2] = q8x4_elem(a.aemb, nb, used, c2);
}

template <int KV>
__global__ void kv_import_kernel(const float *src, int n_pos, void *dst, int ctx_stride) {
    const int p = blockIdx.x;
    for (int e = threadIdx.x; e < kHidden; e += blockDim.x) {
        const float v = src[(size_t)p * kHidden + e];
        const size_t idx = ((size_t)(e >> 6) * ctx_stride + p) * kHeadDim + (e & 63);
        if constexpr (KV == KV_F16)
            ((__half *)dst)[idx] = __float2half_rn(v);
        else
            ((float *)dst)[idx] = v;
    }
}

template <int KV>
__global__ void kv_export_kernel(const void *src, int n_pos, int ctx_stride, float *dst) {
    const int p = blockIdx.x;
    for (int e = threadIdx.x; e < kHidden; e += blockDim.x) {
        const size_t idx = ((size_t)(e >> 6) * ctx_stride + p) * kHeadDim + (e & 63);
        float v;
        if constexpr (KV == KV_F16)
            v = __half2float(((const __half *)src)[idx]);
        else
            v = ((const float *)src)[idx];
        dst[(size_t)p * kHidden + e] = v;
    }
}

}  // namespace

hipError_t launch_embed(const EmbedArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(embed_kernel, dim3(kHidden / 64), dim3(64), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_layernorm(const float *x, const float *w, const float *b, float *out, DevState *state,
                            int bump_pos, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(layernorm_kernel, dim3(1), dim3(256), 0, s, x, w, b, out, state, bump_pos);
    return hipGetLastError();
}

hipError_t launch_dequant_rows(const uint8_t *w, int mat_rows, int cols, const int *rows_dev, int n, float *out,
                               hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_rows_kernel, dim3(n), dim3(256), 0, s, w, mat_rows, cols, rows_dev, out);
    return hipGetLastError();
}

hipError_t launch_gate(const float *x_raw, const float *lnf_w, const float *lnf_b, const uint8_t *wte,
                       DevState *state, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(gate_kernel, dim3(1), dim3(256), 0, s, x_raw, lnf_w, lnf_b, wte, state);
    return hipGetLastError();
}

hipError_t launch_gate_text(const float *logits, DevState *state, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(gate_text_kernel, dim3(1), dim3(256), 0, s, logits, state);
    return hipGetLastError();
}

hipError_t launch_sample(const SampleArgs &a, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(sample_kernel, dim3(1), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_kv_import(const float *src, int n_pos, void *dst, int ctx_stride, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n_pos <= 0) return hipSuccess;
    if (n_pos > ctx_stride) return hipErrorInvalidValue;
    if (kv == KV_F16)
        hipLaunchKernelGGL(kv_import_kernel<KV_F16>, dim3(n_pos), dim3(256), 0, s, src, n_pos, dst, ctx_stride);
    else
        hipLaunchKernelGGL(kv_import_kernel<KV_F32>, dim3(n_pos), dim3(256), 0, s, src, n_pos, dst, ctx_stride);
    return hipGetLastError();
}

hipError_t launch_kv_export(const void *src, int n_pos, int ctx_stride, KvType kv, float *dst, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n_pos <= 0) return hipSuccess;
    if (n_pos > ctx_stride) return hipErrorInvalidValue;
    if (kv == KV_F16)
        hipLaunchKernelGGL(kv_export_kernel<KV_F16>, dim3(n_pos), dim3(256), 0, s, src, n_pos, ctx_stride, dst);
    else
        hipLaunchKernelGGL(kv_export_kernel<KV_F32>, dim3(n_pos), dim3(256), 0, s, src, n_pos, ctx_stride, dst);
    return hipGetLastError();
}

}  // namespace mh

// ------------------------------------------------------------------ row-batched kernels
namespace mh {
namespace {

// Row r's 768 values o (thread t holds t, t+256, t+512) to int8 blocks of 32, in the
// matrix-core order of the prefill GEMMs (q8t_at / d8t_at).
__device__ __forceinline__ void quant_row_768(const float (&o)[3], int r, int8_t *q8, float *d8) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int c = t + 256 * i;
        float d;
        const int q = quant_block32(o[i], &d);
        q8[q8t_at(r, c, kHidden)] = (int8_t)q;
        if ((c & 31) == 0) d8[d8t_at(r, c >> 5, kHidden)] = d;
    }
}

__global__ __launch_bounds__(256) void ln_rows_kernel(const float *x, int x_stride, const float *w, const float *b,
                                                      float *out, const unsigned char *mask, int8_t *q8, float *d8,
                                                      uint8_t *out_hl) {
    __shared__ float red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    if (mask != nullptr && !mask[r]) return;
    const float *xr = x + (size_t)r * x_stride;
    float v[3], o[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = xr[t + 256 * i];
    layernorm_768(v, w, b, o, red);
    if (out_hl != nullptr) {  // for the next GEMM: hi / lo halves in the matrix-core order
#pragma unroll
        for (int i = 0; i < 3; ++i) store_hl(out_hl, r, t + 256 * i, kHidden, o[i]);
    } else if (out != nullptr) {  // (null: only the W8A8 copy is read)
#pragma unroll
        for (int i = 0; i < 3; ++i) out[(size_t)r * kHidden + t + 256 * i] = o[i];
    }
    if (q8 != nullptr) quant_row_768(o, r, q8, d8);
}

// One row per workgroup, one 32-block per half-wave at a time.
__global__ __launch_bounds__(256) void quant_rows_kernel(const float *x, int x_stride, int K, int8_t *q8, float *d8) {
    const int r = blockIdx.x;
    for (int c = threadIdx.x; c < K; c += 256) {
        float d;
        const int q = quant_block32(x[(size_t)r * x_stride + c], &d);
        q8[(size_t)r * K + c] = (int8_t)q;
        if ((c & 31) == 0) d8[(size_t)r * (K / 32) + (c >> 5)] = d;
    }
}

// Split-K reduce + residual + LayerNorm of one row per workgroup (launch_resid_ln_rows).
__global__ __launch_bounds__(256) void resid_ln_rows_kernel(const float *part, int ksplit, int rows,
                                                            const float *bias, const float *resid, int resid_stride,
                                                            float *x, const float *ln_w, const float *ln_b,
                                                            float *out, const unsigned char *mask, int8_t *q8,
                                                            float *d8, uint8_t *out_hl) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    const int r = blockIdx.x, t = threadIdx.x;
    // all partials are loaded before the in-order sum (only the ksplit live
    // slices: the test is uniform, and clamped re-reads of the last slice cost
    // a load instruction each)
    float p[3][16], v[3];
#pragma unroll
    for (int z = 0; z < 16; ++z)
        if (z < ksplit)
#pragma unroll
            for (int i = 0; i < 3; ++i) p[i][z] = part[((size_t)z * rows + r) * kHidden + t + 256 * i];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int n = t + 256 * i;
        float acc = p[i][0];
#pragma unroll
        for (int z = 1; z < 16; ++z)
            if (z < ksplit) acc += p[i][z];
        v[i] = resid[(size_t)r * resid_stride + n] + (acc + bias[n]);
    }
    __syncthreads();  // every read of x (through resid) happens before any write of it
#pragma unroll
    for (int i = 0; i < 3; ++i) x[(size_t)r * kHidden + t + 256 * i] = v[i];
    if (ln_w == nullptr || (mask != nullptr && !mask[r])) return;
    float o[3];
    layernorm_768(v, ln_w, ln_b, o, red);
    if (out_hl != nullptr) {  // for the next GEMM: hi / lo halves in the matrix-core order
#pragma unroll
        for (int i = 0; i < 3; ++i) store_hl(out_hl, r, t + 256 * i, kHidden, o[i]);
    } else if (out != nullptr) {  // (null: only the W8A8 copy is read)
#pragma unroll
        for (int i = 0; i < 3; ++i) out[(size_t)r * kHidden + t + 256 * i] = o[i];
    }
    if (q8 != nullptr) quant_row_768(o, r, q8, d8);
}

// grid (12, rows): same per-element serial sum as embed_kernel
__global__ __launch_bounds__(64) void embed_rows_kernel(EmbedArgs a, const int *rows, float *x) {
    const int nb = kHidden / 32;
    const int r = blockIdx.y, c = blockIdx.x * 64 + threadIdx.x;
    const int *row = rows + (size_t)r * (kNVq + 1);
    float e[kNVq];
    bool use[kNVq];
#pragma unroll
    for (int ch = 0; ch < kNVq; ++ch) {
        const int code = row[ch + 1];
        use[ch] = !(code == kAudioPad || code < 0 || code >= kCodebook);
        e[ch] = q8x4_elem(a.aemb[ch], nb, use[ch] ? code : 0, c);
    }
    float v = q8x4_elem(a.wte, nb, row[0], c);
#pragma unroll
    for (int ch = 0; ch < kNVq; ++ch)
        if (use[ch]) v = v + e[ch];
    x[(size_t)r * kHidden + c] = v;
}

// gate_kernel per stream (one workgroup per stream): same arithmetic, per-stream outputs.
__global__ __launch_bounds__(256) void gate_rows_kernel(const float *x_raw, const float *lnf_w, const float *lnf_b,
                                                        const uint8_t *wte, StreamState st) {
#pragma clang fp contract(off)
    __shared__ float red[4];
    __shared__ float hbuf[kHidden];
    __shared__ int8_t qa[kHidden];
    __shared__ float da[kHidden / 32];
    __shared__ float lanes[2][8];
    const int srow = blockIdx.x, t = threadIdx.x;
    if (!st.active[srow]) return;
    const float *xr = x_raw + (size_t)srow * kHidden;
    float v[3], o[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) v[i] = xr[t + 256 * i];
    layernorm_768(v, lnf_w, lnf_b, o, red);
#pragma unroll
    for (int i = 0; i < 3; ++i) hbuf[t + 256 * i] = o[i];
    __syncthreads();
    const int nb = kHidden / 32;
    if (t < nb) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float av = fabsf(hbuf[32 * t + i]);
            amax = amax < av ? av : amax;
        }
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        da[t] = d;
        for (int i = 0; i < 32; ++i) {
            int q = (int)rintf(hbuf[32 * t + i] * id);
            q = q < -127 ? -127 : (q > 127 ? 127 : q);
            qa[32 * t + i] = (int8_t)q;
        }
    }
    __syncthreads();
    if (t < 16) {
        const int which = t >> 3, lane = t & 7;
        const int r = which == 0 ? kEndToken : kSlotToken;
        const uint8_t *grp = wte + (size_t)(r >> 2) * nb * kBlockBytes;
        float acc = 0.0f;
        for (int b = 0; b < nb; ++b) {
            const uint8_t *blk = grp + (size_t)b * kBlockBytes;
            const float dw = h2f(*(const uint16_t *)(blk + 2 * (r & 3)));
            const int8_t *qs = (const int8_t *)(blk + 8 + 32 * (r & 3));
            int32_t p = 0;
#pragma unroll
            for (int u = 0; u < 4; ++u) p += (int32_t)qs[4 * lane + u] * (int32_t)qa[32 * b + 4 * lane + u];
            const float scale = dw * da[b];
            acc = fmaf((float)p, scale, acc);
        }
        lanes[which][lane] = acc;
    }
    __syncthreads();
    if (t == 0) {
        float g[2];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const float *a8 = lanes[w];
            const float s0 = a8[0] + a8[4], s1 = a8[1] + a8[5], s2 = a8[2] + a8[6], s3 = a8[3] + a8[7];
            const float t0 = s0 + s2, t1 = s1 + s3;
            g[w] = t0 + t1;
        }
        st.gate[2 * srow] = g[0];
        st.gate[2 * srow + 1] = g[1];
        if (st.ctrl->frame >= st.ctrl->min_frames && end_reached(g[1], g[0], st.ctrl->cfg, st.rng + 4 * srow))
            st.active[srow] = 0;
    }
}

// One table row (q | k | v, 2304 floats) of stream srow: q into q_out, k and v
// into the local caches at position lpos (page = stream, 17 positions).
__device__ __forceinline__ void local_qkv_row(const LocalQkv &a, const float *row, int srow) {
    for (int i = threadIdx.x; i < 3 * kHidden; i += 256) {
        const float v = row[i];
        if (i < kHidden) {
            a.q_out[(size_t)srow * kHidden + i] = v;
        } else {
            const int j = i - kHidden, sec = j / kHidden, w = j - sec * kHidden;
            float *cache = sec == 0 ? a.lk : a.lv;
            cache[(((size_t)srow * kHeads + (w >> 6)) * kLocalLen + a.lpos) * kHeadDim + (w & 63)] = v;
        }
    }
}

__global__ __launch_bounds__(256) void local_qkv_rows_kernel(LocalQkv a) { local_qkv_row(a, a.rows, blockIdx.x); }

// sample_kernel per stream (one workgroup each, own history and xoshiro
// stream); inactive streams keep their state.  Teacher forcing is not offered
// by the batched engine, so the used code is the pick.
__global__ __launch_bounds__(256) void sample_rows_kernel(const float *logits, int ch, const uint8_t *aemb,
                                                          float *next_in, StreamState st, int last_channel,
                                                          LocalQkv next, int count_prev) {
    __shared__ PickLds L;
    const int srow = blockIdx.x, t = threadIdx.x;
    float *nxt = next_in + (size_t)srow * kHidden;
    const int nb = kHidden / 32;
    // every load that does not depend on the pick is issued first, together: the
    // row's logits and code counts, its active flag, the control block
    const float *lg = logits + (size_t)srow * kCodebook;
    int *cnt = st.counts + ((size_t)srow * kNVq + ch) * kCodebook;
    PickIn in;
#pragma unroll
    for (int k = 0; k < kCodebook / 256; ++k) {
        in.vals[k] = lg[t + 256 * k];
        in.cnt[k] = cnt[t + 256 * k];
    }
    const bool active = st.active[srow] != 0;
    const float pen = st.ctrl->rep_penalty;
    const SampleCfg c = st.ctrl->cfg;
    const bool greedy = c.greedy || st.ctrl->frame < c.greedy_frames;
    int idx = 0;  // inactive: keep the next local input defined (row 0) so later kernels read finite values
    if (active) {
        if (greedy) {  // the single-stream greedy pick, reduced from registers
            if (pen == 1.0f)
#pragma unroll
                for (int k = 0; k < kCodebook / 256; ++k) in.cnt[k] = 0;
            idx = greedy_pick_reduce(in, pen, L.bv, L.bi);
            idx = idx >= kCodebook ? 0 : idx;  // every value NaN: the reference's scan stays at 0
        } else {
            load_penalised(L, lg, cnt, pen);
            idx = pick_sampled(L, c, st.rng + 4 * srow);
        }
        if (t == 0) {
            st.codes[srow * kNVq + ch] = idx;
            st.row[srow * (kNVq + 1) + ch + 1] = idx;
            cnt[idx] += 1;
            if (count_prev)  // the previous channel's pick, counted late by the fused path (below)
                st.counts[((size_t)srow * kNVq + ch - 1) * kCodebook + st.codes[srow * kNVq + ch - 1]] += 1;
            if (last_channel) st.row[srow * (kNVq + 1)] = kSlotToken;
        }
    }
    // the picked code's embedding row and (next local position) q|k|v table row:
    // both requested before either is stored
    float ev[kHidden / 256], qv[3 * kHidden / 256];
#pragma unroll
    for (int j = 0; j < kHidden / 256; ++j) ev[j] = q8x4_elem(aemb, nb, idx, t + 256 * j);
    if (next.rows) {
        const float *row = next.rows + (size_t)idx * 3 * kHidden;
#pragma unroll
        for (int j = 0; j < 3 * kHidden / 256; ++j) qv[j] = row[t + 256 * j];
    }
#pragma unroll
    for (int j = 0; j < kHidden / 256; ++j) nxt[t + 256 * j] = ev[j];
    if (next.rows) {
#pragma unroll
        for (int j = 0; j < 3 * kHidden / 256; ++j) {
            const int i = t + 256 * j;
            if (i < kHidden) {
                next.q_out[(size_t)srow * kHidden + i] = qv[j];
            } else {
                const int jj = i - kHidden, sec = jj / kHidden, w = jj - sec * kHidden;
                float *cache = sec == 0 ? next.lk : next.lv;
                cache[(((size_t)srow * kHeads + (w >> 6)) * kLocalLen + next.lpos) * kHeadDim + (w & 63)] = qv[j];
            }
        }
    }
}

// Greedy frames of the batch engine: the pick of channel c = lpos - 2 (sample_rows_kernel's
// greedy branch, llm.cpp:683-691 per stream) fused with what follows it at local position
// lpos, one workgroup per (head, stream): every head's workgroup makes the same pick from the
// same logits and counts, writes its 64 columns of the next residual input aemb[c][code]
// and its head's q|k|v slice of the load-time table row, and runs its head's attention over
// the stream's local keys 0..lpos (llm.cpp:189-217).  The pick's count is added by the next
// channel's launch (the one reading counts[c + 1]), so no workgroup reads a count another
// one is changing; the last channel's sample kernel adds the last two.
__global__ __launch_bounds__(256) void local_pick_attn_kernel(const PickAttnArgs a) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    __shared__ __attribute__((aligned(16))) float qkv[3][kHeadDim];  // rows read as float4
    __shared__ float es[kLocalLen];
    const int h = blockIdx.x, srow = blockIdx.y, t = threadIdx.x;
    const StreamState &st = a.st;
    const float *lg = a.logits + (size_t)srow * kCodebook;
    const int *cnt = st.counts + ((size_t)srow * kNVq + a.ch) * kCodebook;
    PickIn in;
    float2 pair = make_float2(-INFINITY, 0.0f);
    if (a.pairs != nullptr) {  // the head's partials: 64 per stream, one per lane of each wave
        pair = reinterpret_cast<const float2 *>(a.pairs)[(size_t)srow * (kCodebook / 16) + (t & 63)];
    } else {
#pragma unroll
        for (int k = 0; k < kCodebook / 256; ++k) {
            in.vals[k] = lg[t + 256 * k];
            in.cnt[k] = cnt[t + 256 * k];
        }
    }
    // wave 0: the cached keys 0 .. lpos - 1 of head h do not depend on the pick, so their
    // rows are requested now, behind the logits (loads complete in order): lane k the K
    // row of key k, lane d column d of every V row (rows past lpos - 1 read row lpos - 1)
    const size_t kvrow = ((size_t)srow * kHeads + h) * kLocalLen;
    const int klast = max(a.lpos - 1, 0);
    float4 kr[kHeadDim / 4];
    float vv[kLocalLen];
    if (t < 64) {
        const float4 *krow = (const float4 *)(a.lk + (kvrow + min(t, klast)) * kHeadDim);
#pragma unroll
        for (int c = 0; c < kHeadDim / 4; ++c) kr[c] = krow[c];
#pragma unroll
        for (int k = 0; k < kLocalLen; ++k) vv[k] = a.lv[(kvrow + min(k, klast)) * kHeadDim + t];
    }
    const bool active = st.active[srow] != 0;  // the same for the whole workgroup
    const float pen = st.ctrl->rep_penalty;
    int idx = 0;  // inactive: row 0 keeps the next inputs defined
    if (active) {
        if (a.pairs != nullptr) {  // every wave reduces the 64 pairs itself (lowest index on ties)
            float best = pair.x;
            int besti = __float_as_int(pair.y);
            wave_argmax(best, besti);
            idx = besti;
        } else {
            if (pen == 1.0f)
#pragma unroll
                for (int k = 0; k < kCodebook / 256; ++k) in.cnt[k] = 0;
            idx = greedy_pick_reduce(in, pen, bv, bi);
        }
        idx = idx >= kCodebook ? 0 : idx;  // every value NaN: the reference's scan stays at 0
        if (h == 0 && t == 0) {
            st.codes[srow * kNVq + a.ch] = idx;
            st.row[srow * (kNVq + 1) + a.ch + 1] = idx;
            if (a.ch > 0)
                st.counts[((size_t)srow * kNVq + a.ch - 1) * kCodebook + st.codes[srow * kNVq + a.ch - 1]] += 1;
        }
    }
    if (t < 3 * kHeadDim) {  // this head's q, k, v of the table row (lpos, code)
        const int sec = t >> 6, d = t & 63;
        const float v = a.rows[(size_t)idx * 3 * kHidden + sec * kHidden + h * kHeadDim + d];
        qkv[sec][d] = v;
        if (sec == 1) a.lk[(kvrow + a.lpos) * kHeadDim + d] = v;
        if (sec == 2) a.lv[(kvrow + a.lpos) * kHeadDim + d] = v;
    } else {  // this head's 64 columns of the next residual input
        const int d = t - 3 * kHeadDim;
        a.next_in[(size_t)srow * kHidden + h * kHeadDim + d] = q8x4_elem(a.aemb, kHidden / 32, idx, h * kHeadDim + d);
    }
    __syncthreads();
    if (t >= 64) return;
    // wave 0: lane k scores key k (the new key lpos from LDS), then lane d accumulates column d
    const int nk = a.lpos + 1;
    float sc = -INFINITY;
    if (t < nk) {
        if (t == a.lpos)  // the new key, from the table row
#pragma unroll
            for (int c = 0; c < kHeadDim / 4; ++c) kr[c] = *(const float4 *)&qkv[1][4 * c];
        float d = 0.0f;
#pragma unroll
        for (int c = 0; c < kHeadDim / 4; ++c) {
            d = fmaf(qkv[0][4 * c], kr[c].x, d);
            d = fmaf(qkv[0][4 * c + 1], kr[c].y, d);
            d = fmaf(qkv[0][4 * c + 2], kr[c].z, d);
            d = fmaf(qkv[0][4 * c + 3], kr[c].w, d);
        }
        sc = d * 0.125f;  // 1/sqrt(64), applied after the dot as llm.cpp:200 does
    }
    const float mx = wave_max(sc);
    const float e = t < nk ? expf(sc - mx) : 0.0f;
    const float l = wave_sum(e);
    if (t < kLocalLen) es[t] = e;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    float o = 0.0f;
    const float vnew = qkv[2][t];
#pragma unroll
    for (int k = 0; k < kLocalLen; ++k)
        if (k < nk) o = fmaf(es[k], k == a.lpos ? vnew : vv[k], o);
    const float res = o / l;
    if (a.o_hl != nullptr)  // for the proj GEMM: hi / lo halves in the matrix-core order
        store_hl(a.o_hl, srow, h * kHeadDim + t, kHidden, res);
    else if (a.o != nullptr)
        a.o[(size_t)srow * kHidden + h * kHeadDim + t] = res;
    if (a.o_q8 != nullptr) {  // W8A8 copy for the proj GEMM: this head's 64 outputs are two blocks of 32 lanes
        float d;
        const int q = quant_block32(res, &d);
        a.o_q8[q8t_at(srow, h * kHeadDim + t, kHidden)] = (int8_t)q;
        if ((t & 31) == 0) a.o_d8[d8t_at(srow, 2 * h + (t >> 5), kHidden)] = d;
    }
}

__global__ void advance_rows_kernel(StreamState st, int streams) {
    const int s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s == 0) st.ctrl->frame += 1;
    if (s >= streams || !st.active[s]) return;
    const int p = st.pos[s] + 1;
    st.pos[s] = p;
    if (p >= st.capacity) st.active[s] = 0;
}

template <int KV>
__global__ void kv_import_paged_kernel(const float *src, void *pool, const int *table_row, int page_size) {
    const int p = blockIdx.x;
    const size_t page_base = (size_t)table_row[p / page_size] * kHeads * page_size;
    for (int e = threadIdx.x; e < kHidden; e += blockDim.x) {
        const size_t idx = ((page_base + (size_t)(e >> 6) * page_size) + p % page_size) * kHeadDim + (e & 63);
        const float v = src[(size_t)p * kHidden + e];
        if constexpr (KV == KV_F16)
            ((__half *)pool)[idx] = __float2half_rn(v);
        else
            ((float *)pool)[idx] = v;
    }
}

template <int KV>
__global__ void kv_export_paged_kernel(const void *pool, const int *table_row, int page_size, float *dst) {
    const int p = blockIdx.x;
    const size_t page_base = (size_t)table_row[p / page_size] * kHeads * page_size;
    for (int e = threadIdx.x; e < kHidden; e += blockDim.x) {
        const size_t idx = ((page_base + (size_t)(e >> 6) * page_size) + p % page_size) * kHeadDim + (e & 63);
        float v;
        if constexpr (KV == KV_F16)
            v = __half2float(((const __half *)pool)[idx]);
        else
            v = ((const float *)pool)[idx];
        dst[(size_t)p * kHidden + e] = v;
    }
}

// grid (n_pos, layers, 2): position p of layer l of K (z = 0) or V (z = 1); thread t copies
// element t of the 768 (head t / 64, dim t % 64) and t + 256, t + 512.
template <int SK, int DK>
__global__ __launch_bounds__(256) void kv_admit_kernel(KvAdmit a) {
    const int p = blockIdx.x, l = blockIdx.y, z = blockIdx.z;
    const uint8_t *src = static_cast<const uint8_t *>(z ? a.v_src : a.k_src) +
                         (size_t)l * a.src_layer_elems * (SK == KV_F16 ? 2 : 4);
    uint8_t *pool = static_cast<uint8_t *>(z ? a.v_pool : a.k_pool) + (size_t)l * a.pool_layer_elems * (DK == KV_F16 ? 2 : 4);
    const size_t page_base = (size_t)a.table_row[p / a.page_size] * kHeads * a.page_size;
    for (int e = threadIdx.x; e < kHidden; e += blockDim.x) {
        const int h = e >> 6, d = e & 63;
        const size_t si = ((size_t)h * a.ctx_stride + p) * kHeadDim + d;
        const size_t di = ((page_base + (size_t)h * a.page_size) + p % a.page_size) * kHeadDim + d;
        if constexpr (SK == DK) {
            if constexpr (SK == KV_F16)
                ((__half *)pool)[di] = ((const __half *)src)[si];
            else
                ((float *)pool)[di] = ((const float *)src)[si];
        } else if constexpr (SK == KV_F32) {
            ((__half *)pool)[di] = __float2half_rn(((const float *)src)[si]);
        } else {
            ((float *)pool)[di] = __half2float(((const __half *)src)[si]);
        }
    }
}

}  // namespace

hipError_t launch_kv_admit(const KvAdmit &a, int n_pos, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n_pos <= 0) return hipSuccess;
    if (!a.k_src || !a.v_src || !a.k_pool || !a.v_pool || !a.table_row || a.page_size <= 0 || n_pos > a.ctx_stride)
        return hipErrorInvalidValue;
    const dim3 grid(n_pos, kLayers, 2);
    if (a.src_kv == KV_F16) {
        if (a.pool_kv == KV_F16)
            hipLaunchKernelGGL((kv_admit_kernel<KV_F16, KV_F16>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((kv_admit_kernel<KV_F16, KV_F32>), grid, dim3(256), 0, s, a);
    } else {
        if (a.pool_kv == KV_F16)
            hipLaunchKernelGGL((kv_admit_kernel<KV_F32, KV_F16>), grid, dim3(256), 0, s, a);
        else
            hipLaunchKernelGGL((kv_admit_kernel<KV_F32, KV_F32>), grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_kv_import_paged(const float *src, int n_pos, void *pool, const int *table_row, int page_size,
                                  KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n_pos <= 0) return hipSuccess;
    if (kv == KV_F16)
        hipLaunchKernelGGL(kv_import_paged_kernel<KV_F16>, dim3(n_pos), dim3(256), 0, s, src, pool, table_row, page_size);
    else
        hipLaunchKernelGGL(kv_import_paged_kernel<KV_F32>, dim3(n_pos), dim3(256), 0, s, src, pool, table_row, page_size);
    return hipGetLastError();
}

hipError_t launch_kv_export_paged(const void *pool, const int *table_row, int page_size, int n_pos, KvType kv,
                                  float *dst, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n_pos <= 0) return hipSuccess;
    if (kv == KV_F16)
        hipLaunchKernelGGL(kv_export_paged_kernel<KV_F16>, dim3(n_pos), dim3(256), 0, s, pool, table_row, page_size, dst);
    else
        hipLaunchKernelGGL(kv_export_paged_kernel<KV_F32>, dim3(n_pos), dim3(256), 0, s, pool, table_row, page_size, dst);
    return hipGetLastError();
}

hipError_t launch_ln_rows(const float *x, int x_stride, const float *w, const float *b, float *out, int rows,
                          hipStream_t s, const unsigned char *mask, int8_t *q8, float *d8, uint8_t *out_hl) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (rows <= 0) return hipSuccess;
    if ((q8 && !d8) || (!out && !q8 && !out_hl)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(ln_rows_kernel, dim3(rows), dim3(256), 0, s, x, x_stride, w, b, out, mask, q8, d8, out_hl);
    return hipGetLastError();
}

hipError_t launch_resid_ln_rows(const float *part, int ksplit, int rows, const float *bias, const float *resid,
                                int resid_stride, float *x, const float *ln_w, const float *ln_b, float *out,
                                const unsigned char *mask, hipStream_t s, int8_t *q8, float *d8, uint8_t *out_hl) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (rows <= 0) return hipSuccess;
    if (!part || ksplit <= 0 || ksplit > 16 || !bias || !resid || !x ||
        (ln_w && (!ln_b || (!out && !q8 && !out_hl))) ||
        (q8 && (!d8 || !ln_w)))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(resid_ln_rows_kernel, dim3(rows), dim3(256), 0, s, part, ksplit, rows, bias, resid,
                       resid_stride, x, ln_w, ln_b, out, mask, q8, d8, out_hl);
    return hipGetLastError();
}

hipError_t launch_quant_rows(const float *x, int x_stride, int K, int rows, int8_t *q8, float *d8, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (rows <= 0) return hipSuccess;
    // every lane of a wave takes part in each block's shuffles: K a multiple of 256
    if (!x || !q8 || !d8 || K <= 0 || K % 256 != 0 || x_stride < K) return hipErrorInvalidValue;
    hipLaunchKernelGGL(quant_rows_kernel, dim3(rows), dim3(256), 0, s, x, x_stride, K, q8, d8);
    return hipGetLastError();
}

hipError_t launch_embed_rows(const EmbedArgs &e, const int *rows, int n, float *x, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(embed_rows_kernel, dim3(kHidden / 64, n), dim3(64), 0, s, e, rows, x);
    return hipGetLastError();
}

hipError_t launch_gate_rows(const float *x_raw, const float *lnf_w, const float *lnf_b, const uint8_t *wte,
                            const StreamState &st, int streams, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(gate_rows_kernel, dim3(streams), dim3(256), 0, s, x_raw, lnf_w, lnf_b, wte, st);
    return hipGetLastError();
}

hipError_t launch_sample_rows(const float *logits, int ch, const uint8_t *aemb, float *next_in, const StreamState &st,
                              int streams, int last_channel, const LocalQkv &next, hipStream_t s, int count_prev) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (next.rows && (!next.q_out || !next.lk || !next.lv || next.lpos < 1 || next.lpos >= kLocalLen))
        return hipErrorInvalidValue;
    if (count_prev && ch < 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL(sample_rows_kernel, dim3(streams), dim3(256), 0, s, logits, ch, aemb, next_in, st,
                       last_channel, next, count_prev);
    return hipGetLastError();
}

hipError_t launch_local_pick_attn(const PickAttnArgs &a, int streams, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (!a.logits || !a.aemb || !a.next_in || !a.rows || !a.lk || !a.lv || (!a.o && !a.o_hl && !a.o_q8) ||
        (a.o_q8 && !a.o_d8) || streams <= 0 ||
        a.ch < 0 ||
        a.ch >= kNVq - 1 || a.lpos != a.ch + 2)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(local_pick_attn_kernel, dim3(kHeads, streams), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_local_qkv_rows(const LocalQkv &a, int streams, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (!a.rows || !a.q_out || !a.lk || !a.lv || a.lpos < 1 || a.lpos >= kLocalLen || streams <= 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(local_qkv_rows_kernel, dim3(streams), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_advance_rows(const StreamState &st, int streams, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    hipLaunchKernelGGL(advance_rows_kernel, dim3((streams + 63) / 64), dim3(64), 0, s, st, streams);
    return hipGetLastError();
}

}  // namespace mh
