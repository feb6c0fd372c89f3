// mh_device.h -- device-side helpers shared by the CDNA4 (gfx950) kernels.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mh {

// Model constants of the MOSS-TTS-Nano LLM (reference csrc/include/moss/llm.h:18-29).
constexpr int kHidden = 768;
constexpr int kHeads = 12;
constexpr int kHeadDim = 64;
constexpr int kFF = 3072;
constexpr int kVocab = 16384;
constexpr int kNVq = 16;
constexpr int kCodebook = 1024;
constexpr int kAudioPad = 1024;
constexpr int kSlotToken = 9;
constexpr int kEndToken = 7;
constexpr int kMaxCtx = 768;
constexpr int kLocalLen = 17;
constexpr int kLayers = 12;
constexpr int kRopeHalf = kHeadDim / 2;

// Q8_0_4X4: a 4-row group stores, per 32-column block, 4 fp16 scales (8 B)
// then 4 x 32 int8 (row k at byte 8 + 32k): 136 bytes per block
// (reference csrc/src/quant.cpp:56-65, tools/export_weights.py:160-179).
constexpr int kBlockBytes = 136;
// a weight matrix in the matrix-core order (the GEMMs' copy): one unit per 16 rows and scale
// block, the 512 quants in MFMA lane order then the 16 rows' fp16 scales
constexpr int kTileBytes = 544;

// LDS pointer type of the direct global -> LDS loads (__builtin_amdgcn_global_load_lds)
typedef __attribute__((address_space(3))) void *lds_ptr;

constexpr int kWave = 64;

// Device-resident decode state, read by every kernel of a captured step so the
// same hipGraph can be replayed frame after frame.
// Sampling controls of one generate() call (SampleParams, reference
// csrc/include/moss/sampler.h:8-22).
struct SampleCfg {
    int greedy;          // SampleParams::greedy || top_k == 1 (sampler.cpp:23)
    float temperature;
    int top_k;
    float top_p;
    int end_greedy;
    int greedy_frames;   // frames [0, greedy_frames) pick greedily (llm.cpp:686-687)
};

struct DevState {
    int pos;          // next global position (= LlmModel::pos_)
    int frame;        // frame index inside the current generate() call
    int stop;         // end gate fired in this frame: later kernels of the frame do nothing
    int min_frames;   // SampleParams::min_frames
    int forced_on;    // teacher forcing: the used code comes from `forced`
    float rep_penalty;
    SampleCfg cfg;
    uint32_t rng[4];  // xoshiro128** state of this generate() call, advanced on the device
    int row[17];      // next global-step row: [slot, codes...]
    int codes[16];    // predicted codes of the current frame
    float gate[2];    // (l_end, l_slot) of the current frame
    int gate_argmax;  // gate-dump frames: argmax over the full text head, and its logit
    float gate_argmax_v;
    unsigned ll_err;  // a fused decode-layer launch ran out of its wait budget
};

// xoshiro128** step and uniform draw of the reference's Rng (sampler.h:25-49).
__device__ __forceinline__ uint32_t rng_next(uint32_t *s) {
    const uint32_t x = s[1] * 5u;
    const uint32_t result = ((x << 7) | (x >> 25)) * 9u;
    const uint32_t t = s[1] << 9;
    s[2] ^= s[0];
    s[3] ^= s[1];
    s[1] ^= s[2];
    s[0] ^= s[3];
    s[2] ^= t;
    s[3] = (s[3] << 11) | (s[3] >> 21);
    return result;
}

// 24 random bits as a float in [0, 1): exact in fp32.
__device__ __forceinline__ float rng_uniform(uint32_t *s) { return (float)(rng_next(s) >> 8) * (1.0f / 16777216.0f); }

// end_reached (llm.cpp:30-35): greedy compares the two logits; otherwise one
// uniform draw against the slot probability of a two-way softmax, in double.
__device__ __forceinline__ bool end_reached(float l_slot, float l_end, const SampleCfg &c, uint32_t *rng) {
    if (c.end_greedy) return l_end > l_slot;
    double d = (double)l_end - (double)l_slot;
    d = d < -80.0 ? -80.0 : (d > 80.0 ? 80.0 : d);
    const float p_slot = (float)(1.0 / (1.0 + exp(d)));
    return rng_uniform(rng) >= p_slot;
}

// threadIdx.x / blockIdx.x behind an empty volatile asm.  Inside the block
// loop of a persistent kernel, values derived from them (gather addresses,
// masks, row indices) are then recomputed in each block instead of being
// hoisted out of the loop and held in registers across all blocks.
__device__ __forceinline__ int tix() {
    int v = threadIdx.x;
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ int bix() {
    int v = blockIdx.x;
    asm volatile("" : "+s"(v));
    return v;
}

// Value of lane (lane ^ M) for M = 1, 2, 4, 8, 16, 32, without the LDS
// round trip of ds_bpermute: DPP quad permutes (1, 2), DPP row shifts under
// bank masks (4), a DPP row rotation (8) and the gfx950 permlane swaps (16, 32).
// Same values as __shfl_xor(v, M), so reductions keep their order and results.
template <int M>
__device__ __forceinline__ int xshfl(int v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "xshfl: power of two <= 32");
    if constexpr (M == 1) {
        return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    } else if constexpr (M == 2) {
        return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
    } else if constexpr (M == 4) {
        // banks 0, 2 of each row (lanes 0-3, 8-11) read lane + 4 (row_shl:4),
        // banks 1, 3 (lanes 4-7, 12-15) read lane - 4 (row_shr:4)
        const int t = __builtin_amdgcn_update_dpp(v, v, 0x104, 0xF, 0x5, false);
        return __builtin_amdgcn_update_dpp(t, v, 0x114, 0xF, 0xA, false);
    } else if constexpr (M == 8) {
        return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);  // row_ror:8 within 16 lanes
    } else if constexpr (M == 16) {
        // swap of rows 1 <-> 0 and 3 <-> 2: r.x = rows [0,0,2,2], r.y = rows [1,1,3,3]
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        return (int)(((__lane_id() >> 4) & 1) ? r[0] : r[1]);
    } else {
        // r.x = lanes 0-31 in both halves, r.y = lanes 32-63 in both halves
        const auto r = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        return (int)(__lane_id() >= 32 ? r[0] : r[1]);
    }
}

template <int M>
__device__ __forceinline__ float xshfl(float v) {
    return __int_as_float(xshfl<M>(__float_as_int(v)));
}

// Sum over the L lanes of a key (lanes differing in the low log2(L) bits of
// `sub`) of L partial dots at once: each step keeps half of the values and
// adds the partner's copy of them, so lane sub ends with the total of pd[sub].
template <int L>
__device__ __forceinline__ float key_reduce(float (&pd)[L], int sub) {
    if constexpr (L == 1) {
        return pd[0];
    } else {
        constexpr int H = L / 2;
        const bool upper = (sub & H) != 0;
        float nx[H];
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const float keep = upper ? pd[i + H] : pd[i];
            const float give = upper ? pd[i] : pd[i + H];
            nx[i] = keep + xshfl<H>(give);
        }
        return key_reduce<H>(nx, sub);
    }
}

__device__ __forceinline__ float wave_sum(float v) {
    v += xshfl<32>(v);
    v += xshfl<16>(v);
    v += xshfl<8>(v);
    v += xshfl<4>(v);
    v += xshfl<2>(v);
    v += xshfl<1>(v);
    return v;
}

// Wave-wide (max value, lowest index among ties) reduction; every lane ends
// with the result.
template <int M>
__device__ __forceinline__ void argmax_step(float &best, int &besti) {
    const float ov = xshfl<M>(best);
    const int oi = xshfl<M>(besti);
    if (ov > best || (ov == best && oi < besti)) {
        best = ov;
        besti = oi;
    }
}

__device__ __forceinline__ void wave_argmax(float &best, int &besti) {
    argmax_step<32>(best, besti);
    argmax_step<16>(best, besti);
    argmax_step<8>(best, besti);
    argmax_step<4>(best, besti);
    argmax_step<2>(best, besti);
    argmax_step<1>(best, besti);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, xshfl<32>(v));
    v = fmaxf(v, xshfl<16>(v));
    v = fmaxf(v, xshfl<8>(v));
    v = fmaxf(v, xshfl<4>(v));
    v = fmaxf(v, xshfl<2>(v));
    v = fmaxf(v, xshfl<1>(v));
    return v;
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f2h(float f) { return __half_as_ushort(__float2half_rn(f)); }

// Dequantised element c of row r of a Q8_0_4X4 matrix with nb blocks per row.
__device__ __forceinline__ float q8x4_elem(const uint8_t *w, int nb, int r, int c) {
    const uint8_t *blk = w + ((size_t)(r >> 2) * nb + (c >> 5)) * kBlockBytes;
    const uint16_t d = *(const uint16_t *)(blk + 2 * (r & 3));
    const int8_t q = *(const int8_t *)(blk + 8 + 32 * (r & 3) + (c & 31));
    return h2f(d) * (float)q;  // exact in fp32
}

// Greedy pick over one 1024-entry logit row by a 256-thread workgroup
// (sampler.cpp:13-28 as llm.cpp:689-697 calls it): logits under the
// repetition penalty (applied count times, v < 0 ? v * p : v / p), argmax with
// the lowest index winning ties; kCodebook when every value is NaN (the caller
// maps that to 0, where the reference's scan stays).  bv / bi: 4 LDS slots.
// The loads (issued first, so later loads do not delay them) and the reduction.
// MFMA operand vectors
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef int intx4 __attribute__((ext_vector_type(4)));

// int8 -> fp16, exactly: the half with bits 0x64 : (q ^ 0x80) is 1024 + (q + 128),
// built two at a time with v_perm_b32; subtracting 1152 leaves q.
__device__ __forceinline__ half8 i8x8_to_h8(uint2 q) {
    const uint32_t a = q.x ^ 0x80808080u, b = q.y ^ 0x80808080u;
    const uint32_t w[4] = {__builtin_amdgcn_perm(0x64646464u, a, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, a, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, b, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, b, 0x04030402u)};
    const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    half8 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const half2v v = __builtin_bit_cast(half2v, w[i]) - bias;
        r[2 * i] = v[0];
        r[2 * i + 1] = v[1];
    }
    return r;
}

// Workgroup barrier for LDS traffic only: each wave waits for its own LDS operations, not
// for its global loads in flight (__syncthreads() orders global memory too, so it waits for
// every outstanding load -- a weight prefetch included -- before the barrier).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

struct PickIn {
    float vals[kCodebook / 256];
    int cnt[kCodebook / 256];
};

// v under the repetition penalty applied cnt times (v < 0 ? v * p : v / p)
__device__ __forceinline__ float penalised(float v, int cnt, float pen) {
#pragma clang fp contract(off)
    for (int r = 0; r < cnt; ++r) v = v < 0.0f ? v * pen : v / pen;
    return v;
}

__device__ __forceinline__ void greedy_pick_load(const float *logits, const int *counts, float pen, PickIn &in) {
    const int t = threadIdx.x;
#pragma unroll
    for (int k = 0; k < kCodebook / 256; ++k) {
        in.vals[k] = logits[t + 256 * k];
        in.cnt[k] = pen != 1.0f ? counts[t + 256 * k] : 0;
    }
}

__device__ __forceinline__ int greedy_pick_reduce(const PickIn &in, float pen, float *bv, int *bi) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    const float *vals = in.vals;
    const int *cnt = in.cnt;
    float best = -INFINITY, v0 = 0.0f;
    int besti = kCodebook;
#pragma unroll
    for (int k = 0; k < kCodebook / 256; ++k) {  // ascending index per thread
        const float v = penalised(vals[k], cnt[k], pen);
        if (k == 0) v0 = v;
        if (v > best) {
            best = v;
            besti = t + 256 * k;
        }
    }
    wave_argmax(best, besti);
    if ((t & 63) == 0) {
        bv[t >> 6] = best;
        // thread 0 holds index 0: a NaN there is flagged (sampler.cpp:24-26 never moves off
        // index 0 then, every comparison with it being false)
        bi[t >> 6] = (t == 0 && v0 != v0) ? -1 : besti;
    }
    __syncthreads();
    if (bi[0] < 0) return 0;
    float b = bv[0];
    int idx = bi[0];
    for (int w = 1; w < 4; ++w)
        if (bv[w] > b || (bv[w] == b && bi[w] < idx)) {
            b = bv[w];
            idx = bi[w];
        }
    return idx;
}

__device__ __forceinline__ int greedy_pick_1024(const float *logits, const int *counts, float pen, float *bv, int *bi) {
    PickIn in;
    greedy_pick_load(logits, counts, pen, in);
    return greedy_pick_reduce(in, pen, bv, bi);
}

// Block-wide sum for a 256-thread workgroup (4 waves); `red` needs 4 floats.
__device__ __forceinline__ float block_sum_256(float v, float *red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// LayerNorm over kHidden elements held as 3 values per thread of a 256-thread
// workgroup (reference csrc/src/llm.cpp:159-171: two-pass mean / variance,
// eps 1e-5, (x - mean) * inv * w + b).  Reductions are tree-ordered here.
// The weights of this thread's elements (w[t + 256 i], b[t + 256 i]) come in
// registers, so a caller can load them before its input is ready.
__device__ __forceinline__ void layernorm_768_reg(const float (&x)[3], const float (&w)[3], const float (&b)[3],
                                                  float (&out)[3], float *red) {
#pragma clang fp contract(off)
    float s = (x[0] + x[1]) + x[2];
    const float mean = block_sum_256(s, red) / (float)kHidden;
    float d0 = x[0] - mean, d1 = x[1] - mean, d2 = x[2] - mean;
    float v = (d0 * d0 + d1 * d1) + d2 * d2;
    const float var = block_sum_256(v, red) / (float)kHidden;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        float y = (x[i] - mean) * inv;
        y = y * w[i];
        out[i] = y + b[i];
    }
}

// LayerNorm of 768 values already in LDS: every wave forms both moments itself
// (12 values per lane, then a wave sum), so no workgroup barrier is needed;
// thread t normalises elements t + 256 i.  w, b: this thread's weights.
__device__ __forceinline__ void layernorm_768_lds(const float *x, const float (&w)[3], const float (&b)[3],
                                                  float (&out)[3]) {
#pragma clang fp contract(off)
    const int t = tix(), lane = t & 63;
    float xv[kHidden / 64];
#pragma unroll
    for (int k = 0; k < kHidden / 64; ++k) xv[k] = x[lane + 64 * k];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < kHidden / 64; ++k) s += xv[k];
    const float mean = wave_sum(s) / (float)kHidden;
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < kHidden / 64; ++k) {
        const float d = xv[k] - mean;
        v += d * d;
    }
    const float var = wave_sum(v) / (float)kHidden;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        float y = (x[t + 256 * i] - mean) * inv;
        y = y * w[i];
        out[i] = y + b[i];
    }
}

__device__ __forceinline__ void layernorm_768(const float (&x)[3], const float *w, const float *b, float (&out)[3],
                                              float *red) {
    const int t = threadIdx.x;
    float wv[3], bv[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        wv[i] = w[t + 256 * i];
        bv[i] = b[t + 256 * i];
    }
    layernorm_768_reg(x, wv, bv, out, red);
}

// Activation quantisation of one 32-value block held by 32 consecutive lanes
// (quantize_row_q8_0_scaled, reference csrc/src/quant.cpp:28-54): amax over the
// block, d = amax / 127, id = 1 / d (0 when d == 0), q = clamp(rint(x * id),
// +-127).  The max is order-independent, so this equals the serial scan.
// Returns q; *d_out receives d in every lane of the block.
__device__ __forceinline__ int quant_block32(float x, float *d_out) {
#pragma clang fp contract(off)
    float amax = fabsf(x);
    amax = fmaxf(amax, xshfl<1>(amax));
    amax = fmaxf(amax, xshfl<2>(amax));
    amax = fmaxf(amax, xshfl<4>(amax));
    amax = fmaxf(amax, xshfl<8>(amax));
    amax = fmaxf(amax, xshfl<16>(amax));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int q = (int)rintf(x * id);
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    *d_out = d;
    return q;
}

// W8A8 activations as the prefill writes them for its GEMMs (GemmArgs::a8_tiled), in
// the order the matrix cores take them: an M x K int8 matrix is one 512-byte unit per
// 16 rows and 32-column block, unit (m / 16) * (K / 32) + k / 32, in which row m % 16,
// columns 8j .. 8j + 7 of the block are the 8 bytes at 8 * (m % 16 + 16 j) -- the A
// operand of lane m % 16 + 16 j of a 16x16x32 MFMA -- so a GEMM reads a block of 16
// rows as 4 whole cache lines; the block scales are 16 floats per unit.  Buffers hold
// the row count rounded up to 16.
__device__ __forceinline__ size_t q8t_at(int m, int k, int K) {
    const size_t unit = (size_t)(m >> 4) * (K >> 5) + (k >> 5);
    return unit * 512 + 8 * ((m & 15) + 16 * ((k & 31) >> 3)) + (k & 7);
}
__device__ __forceinline__ size_t d8t_at(int m, int blk, int K) {
    return ((size_t)(m >> 4) * (K >> 5) + blk) * 16 + (m & 15);
}

// fp32 activations as the A16 GEMMs can read them (GemmArgs::a_hl): each value x
// split into fp16 hi = rtz(x) and lo = rtz(x - hi) (hi + lo keeps ~22 bits), in
// the matrix-core order -- one 2048-byte unit per 16 rows and 32-column block
// (unit (m / 16) * (K / 32) + k / 32): the hi halves of lane m % 16 + 16 j's 8
// values (row m % 16, columns 8j .. 8j + 7 of the block) at 16 * lane, the lo
// halves 1024 bytes further.  Rows padded to 16.
__device__ __forceinline__ size_t hlt_at(int m, int k, int K) {  // byte offset of the hi half
    const size_t unit = (size_t)(m >> 4) * (K >> 5) + (k >> 5);
    return unit * 2048 + 16 * ((m & 15) + 16 * ((k & 31) >> 3)) + 2 * (k & 7);
}
__device__ __forceinline__ void store_hl(uint8_t *hl, int m, int k, int K, float x) {
    const size_t o = hlt_at(m, k, K);
    const auto h = __builtin_amdgcn_cvt_pkrtz(x, x);
    const auto l = __builtin_amdgcn_cvt_pkrtz(x - (float)h[0], x - (float)h[0]);
    *reinterpret_cast<_Float16 *>(hl + o) = (_Float16)h[0];
    *reinterpret_cast<_Float16 *>(hl + o + 1024) = (_Float16)l[0];
}

// gelu_new (reference csrc/src/llm.cpp:22-25)
__device__ __forceinline__ float gelu_new(float v) {
#pragma clang fp contract(off)
    const float k = 0.7978845608028654f;
    const float v3 = 0.044715f * v * v * v;
    return 0.5f * v * (1.0f + tanhf(k * (v + v3)));
}

// The 2-row W8A8 end gate on h = ln_f(x) (llm.cpp:272-315, as gate_kernel):
// per-32-block activation quantisation (quant.cpp:28-54), the int32 block dots
// of wte rows 7 (end) and 9 (slot) in the reference's lane order, the stop
// rule.  Called by all 256 threads of a workgroup with h in LDS; thread 0
// writes state->gate and, when the frame ends, state->stop.
struct GateLds {
    int8_t qa[kHidden];
    float da[kHidden / 32];
    float lanes[2][8];
};
__device__ __forceinline__ void gate_block(const float *hbuf, const uint8_t *wte, DevState *state, GateLds &G) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    int8_t *qa = G.qa;
    float *da = G.da;
    float (*lanes)[8] = G.lanes;
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
        state->gate[0] = g[0];
        state->gate[1] = g[1];
        if (state->frame >= state->min_frames && end_reached(g[1], g[0], state->cfg, state->rng)) state->stop = 1;
    }
}

}  // namespace mh
