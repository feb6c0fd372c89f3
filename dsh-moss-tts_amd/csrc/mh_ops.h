// mh_ops.h -- host-side launchers of the gfx950 kernels (internal C++ API).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mh_device.h"

namespace mh {

// Activation source of a GEMV (what the kernel stages into LDS as fp32).
enum Prologue : int {
    PRO_F32 = 0,    // x: float[cols]
    PRO_F16 = 1,    // x: half[cols]
    PRO_LN = 2,     // x: float[768], LayerNorm(ln_w, ln_b) applied in the prologue
};

// What happens to each output row.
enum Epilogue : int {
    EPI_F32 = 0,    // y[r] = acc                      (float)
    EPI_F16 = 1,    // y[r] = half(acc)                (half)
    EPI_QKV = 2,    // + bias, RoPE on q/k, q -> q_out, k/v -> KV cache at pos
    EPI_RESID = 3,  // y[r] = xin[r] + (acc + bias[r]), xin = resid_in or y (float)
    EPI_GELU = 4,   // y[r] = gelu_new(acc + bias[r])  (float)
};

enum KvType : int { KV_F16 = 0, KV_F32 = 1 };

struct GemvArgs {
    const uint8_t *w = nullptr;  // Q8_0_4X4 matrix, rows x cols
    int rows = 0, cols = 0;
    // prologue
    const void *x = nullptr;
    const float *ln_w = nullptr, *ln_b = nullptr;
    // epilogue
    void *y = nullptr;
    const float *resid_in = nullptr;  // EPI_RESID reads the residual from here (nullptr: from y)
    const float *bias = nullptr;
    float *q_out = nullptr;
    void *k_cache = nullptr, *v_cache = nullptr;  // [heads][ctx_stride][64]
    int ctx_stride = 0;
    const float *rope_cos = nullptr, *rope_sin = nullptr;  // [pos][32]
    // position (EPI_QKV): *pos_ptr when non-null, else pos_const
    const int *pos_ptr = nullptr;
    int pos_const = 0;
    const DevState *state = nullptr;  // when non-null, the kernel is a no-op once state->stop is set
};

// Launch y = W x with the given prologue/epilogue; kv selects the KV cache type for EPI_QKV.
hipError_t launch_gemv(const GemvArgs &a, Prologue pro, Epilogue epi, KvType kv, hipStream_t s);

struct AttnArgs {
    const float *q = nullptr;                           // [heads*64] fp32 (post-RoPE)
    const void *k_cache = nullptr, *v_cache = nullptr;  // [heads][ctx_stride][64]
    int ctx_stride = 0;
    int heads = kHeads;
    const int *pos_ptr = nullptr;  // keys = *pos_ptr + 1 (or pos_const + 1)
    int pos_const = 0;
    int max_keys = 0;              // capacity the launch shape is sized for (<= attn_max_keys())
    void *out = nullptr;           // [heads*64] normalised output
    int out_f16 = 0;               // out is half (else float)
    const DevState *state = nullptr;
};
// Decode attention, one workgroup per head (split-KV across its waves, LDS merge).
int attn_max_keys();
hipError_t launch_attn_decode(const AttnArgs &a, KvType kv, hipStream_t s);

// ---- frame / step kernels (frame_ops.hip)
struct EmbedArgs {
    const uint8_t *wte = nullptr;
    const uint8_t *aemb[kNVq] = {};
    const int *row = nullptr;  // [17] on device
    float *x = nullptr;        // [768] out
    const DevState *state = nullptr;
};
hipError_t launch_embed(const EmbedArgs &a, hipStream_t s);

// out = LayerNorm(x); when bump_pos, state->pos += 1 afterwards (end of a global step).
hipError_t launch_layernorm(const float *x, const float *w, const float *b, float *out, DevState *state,
                            int bump_pos, hipStream_t s);

// Dequantise `n` rows (device indices) of a mat_rows x cols Q8_0_4X4 matrix into out[n][cols].
hipError_t launch_dequant_rows(const uint8_t *w, int mat_rows, int cols, const int *rows_dev, int n, float *out,
                               hipStream_t s);

// End gate: LN(x; lnf) -> W8A8 dot with wte rows 7 and 9 (reference order) -> state->gate, state->stop.
hipError_t launch_gate(const float *x_raw, const float *lnf_w, const float *lnf_b, const uint8_t *wte,
                       DevState *state, float *gate_log, hipStream_t s);

// Greedy pick for channel ch: repetition penalty from counts, argmax, history update,
// next input = dequant(aemb[ch][used]).
struct SampleArgs {
    const float *logits = nullptr;  // [1024]
    int ch = 0;
    int *counts = nullptr;          // [16][1024] occurrences of each used code in this generate()
    const int *forced = nullptr;    // [frames][16] (used when state->forced_on)
    const uint8_t *aemb = nullptr;  // aemb[ch]
    float *next_input = nullptr;    // [768]
    DevState *state = nullptr;
    int last_channel = 0;           // ch == 15: advance state->frame
};
hipError_t launch_sample_greedy(const SampleArgs &a, hipStream_t s);

// KV import/export between the reference layout [n][768] fp32 of one layer and the
// device layout [heads][ctx_stride][64] (fp16 or fp32).
hipError_t launch_kv_import(const float *src, int n_pos, void *dst, int ctx_stride, KvType kv, hipStream_t s);
hipError_t launch_kv_export(const void *src, int n_pos, int ctx_stride, KvType kv, float *dst, hipStream_t s);

}  // namespace mh
