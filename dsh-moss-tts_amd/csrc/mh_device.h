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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
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
__device__ __forceinline__ void layernorm_768(const float (&x)[3], const float *w, const float *b, float (&out)[3],
                                              float *red) {
#pragma clang fp contract(off)
    const int t = threadIdx.x;
    float s = (x[0] + x[1]) + x[2];
    const float mean = block_sum_256(s, red) / (float)kHidden;
    float d0 = x[0] - mean, d1 = x[1] - mean, d2 = x[2] - mean;
    float v = (d0 * d0 + d1 * d1) + d2 * d2;
    const float var = block_sum_256(v, red) / (float)kHidden;
    const float inv = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        const int c = t + 256 * i;
        float y = (x[i] - mean) * inv;
        y = y * w[c];
        out[i] = y + b[c];
    }
}

// Activation quantisation of one 32-value block held by 32 consecutive lanes
// (quantize_row_q8_0_scaled, reference csrc/src/quant.cpp:28-54): amax over the
// block, d = amax / 127, id = 1 / d (0 when d == 0), q = clamp(rint(x * id),
// +-127).  The max is order-independent, so this equals the serial scan.
// Returns q; *d_out receives d in every lane of the block.
__device__ __forceinline__ int quant_block32(float x, float *d_out) {
#pragma clang fp contract(off)
    float amax = fabsf(x);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int q = (int)rintf(x * id);
    q = q < -127 ? -127 : (q > 127 ? 127 : q);
    *d_out = d;
    return q;
}

// gelu_new (reference csrc/src/llm.cpp:22-25)
__device__ __forceinline__ float gelu_new(float v) {
#pragma clang fp contract(off)
    const float k = 0.7978845608028654f;
    const float v3 = 0.044715f * v * v * v;
    return 0.5f * v * (1.0f + tanhf(k * (v + v3)));
}

}  // namespace mh
