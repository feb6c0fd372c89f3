// codec.h -- the GPU-resident MOSS audio codec decoder (codes -> 48 kHz stereo PCM).
//
// Device counterpart of moss::AudioDecoder (reference csrc/include/moss/decoder.h:14-83,
// csrc/src/decoder.cpp:26-281, csrc/src/audio_layer.cpp:17-109,
// csrc/src/attn_avx2.cpp:93-204):
//   front   z = sum_i (cb_i[code] W_i^T + b_i), x = z Wq^T + bq          decoder.cpp:224-245
//   stage s (patch 4, 2, 2, 2; 4, 2, 2, 4 layers; window 500, 800, 1200, 1600 positions):
//           y = patch(x) W_in^T; per layer
//             y += ls1 * proj(attn_window(rope(LN1(y) W_qkv^T)))          audio_layer.cpp:48-80
//             y += ls2 * gelu(LN2(y) W_f1^T) W_f2^T                        audio_layer.cpp:82-108
//           x = y W_out^T
//   samples = patch(x, 240) (row-major flattening of the last stage's [rows][240]).
// Activations are fp32 [rows][channels]; the matrices stay as the file stores them (fp16,
// or fp32 where the export kept fp32) and meet fp32 activations in v_mfma_f32_16x16x4_f32,
// i.e. the reference's fp32 products with fp32 accumulation.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/moss_hip.h"

namespace mh {

constexpr int kCodecDModel = 256, kCodecHeads = 4, kCodecHeadDim = 64;
constexpr int kCodecNq = 16, kCodecCb = 1024, kCodecCbDim = 8, kCodecZ = 512;
constexpr int kCodecStages = 4;
constexpr int kCodecFinalPatch = 240;

// Activation source of a codec GEMM (staged into LDS as fp32, 16 rows at a time).
enum CodecPro : int {
    CPRO_ROWS = 0,   // a[m][k], row stride lda
    CPRO_LN = 1,     // LayerNorm(ln_w, ln_b, eps 1e-5) of a[m][0..256)
    CPRO_MERGE = 2,  // attention: merge of the split-KV partials (o, st) into the 256-wide row
};
// What happens to each output element v = sum_k A[m][k] W[n][k].
enum CodecEpi : int {
    CEPI_STORE = 0,  // y[(m*patch + n%patch)*ldy + n/patch] = v (+ bias[n])
    CEPI_GELU = 1,   // y[m*ldy + n] = gelu(v)  (erf form)
    CEPI_RESID = 2,  // y[m*ldy + n] += ls[n] * v
    CEPI_QKV = 3,    // RoPE of q/k at position pos0 + m; q -> q[m], k/v -> ring slot (pos0+m) % ring
};

struct CodecGemmArgs {
    const float *a = nullptr;
    int lda = 0;
    const void *w = nullptr;  // [N][K] row-major, fp16 or fp32
    int w_f32 = 0;
    int M = 0, N = 0, K = 0;
    const float *ln_w = nullptr, *ln_b = nullptr;
    // CPRO_MERGE: o [splits][M][256], st [splits][M][heads] (max, sum)
    const float *o = nullptr;
    const float2 *st = nullptr;
    int splits = 0;
    float *y = nullptr;
    int ldy = 0, patch = 1;
    const float *bias = nullptr, *ls = nullptr;
    // CEPI_QKV
    float *q = nullptr, *kc = nullptr, *vc = nullptr;
    int ring = 0;
    const int *pos0 = nullptr;
    const float *freq = nullptr;  // [32] RoPE frequencies (host-computed as the reference does)
};

struct CodecAttnArgs {
    const float *q = nullptr;                // [M][256], RoPE'd
    const float *kc = nullptr, *vc = nullptr;  // ring [ring][256]
    int ring = 0, window = 0, M = 0, splits = 1;
    const int *pos0 = nullptr;
    float *o = nullptr;   // [splits][M][256] unnormalised partial outputs
    float2 *st = nullptr; // [splits][M][heads] (running max, sum of exponentials)
};

struct CodecFrontArgs {
    const int32_t *codes = nullptr;  // [16][frames]
    int frames = 0;
    const float *cb[kCodecNq], *cw[kCodecNq], *cbias[kCodecNq];  // [1024][8], [512][8], [512]
    float *z = nullptr;  // [frames][512]
};

int codec_gemm_launch(int pro, int epi, const CodecGemmArgs &g, hipStream_t s);
int codec_attn_launch(const CodecAttnArgs &a, hipStream_t s);
int codec_front_launch(const CodecFrontArgs &a, hipStream_t s);
int codec_advance_launch(int *pos0, const int *rows, hipStream_t s);  // pos0[i] += rows[i], i < 4

// One stream's decoder state: per stage the next position and per layer the K/V rings.
struct CodecState {
    int *pos0 = nullptr;  // device [4]
    std::vector<float *> k, v;  // per layer (all stages, in order), [ring_s][256] each
};

class Codec {
public:
    Codec(const void *blob, size_t bytes, const moss_hip_codec_options &opt);
    ~Codec();
    Codec(const Codec &) = delete;
    Codec &operator=(const Codec &) = delete;

    void reset_stream();
    // codes [16][frames] (quantizer-major, as the reference), out [frames * samples_per_frame()]
    void decode_chunk(const int32_t *codes, int frames, float *out);
    void decode(const int32_t *codes, int frames, float *out);
    int samples_per_frame() const { return spf_; }
    double last_ms() const { return last_ms_; }
    const double *stage_ms() const { return stage_ms_; }
    int max_chunk_frames() const { return fmax_; }
    const std::string &info() const { return info_; }

private:
    struct LayerW {
        const void *attn, *proj, *f1, *f2;
        int attn_f32, proj_f32, f1_f32, f2_f32;
        const float *n1w, *n1b, *n2w, *n2b, *ls1, *ls2;
        int ffn;
    };
    struct StageW {
        const void *in, *out;
        int in_f32, out_f32;
        int cin, cout, patch, window, ring, layer0, nlayers;
    };
    void alloc_state(CodecState &st);
    void free_state(CodecState &st);
    void clear_state(CodecState &st);
    // launches of one piece of <= fmax_ frames (codes already in codes_dev_), samples to out_dev_;
    // stage_ev (5 events, [0] recorded by the caller) marks each stage's end
    void enqueue(CodecState &st, int frames, hipEvent_t *stage_ev);
    int splits_for(int stage, int rows) const;
    void check_codes(const int32_t *codes, int frames) const;
    void run_piece(CodecState &st, const int32_t *codes, int frames, float *out, bool graph);

    int device_ = 0;
    int fmax_ = 32, spf_ = 0, ffn_max_ = 0;
    hipStream_t stream_ = nullptr;
    uint8_t *wdev_ = nullptr;  // every tensor of the file, 256-byte aligned
    const float *front_cb_[kCodecNq], *front_w_[kCodecNq], *front_b_[kCodecNq];
    const void *qout_w_ = nullptr;
    int qout_f32_ = 0;
    const float *qout_b_ = nullptr;
    StageW stages_[kCodecStages];
    std::vector<LayerW> layers_;
    float *freq_ = nullptr;  // device [32]
    // activations
    int32_t *codes_dev_ = nullptr;
    float *z_ = nullptr, *xa_ = nullptr, *xb_ = nullptr, *y_ = nullptr, *qb_ = nullptr, *h_ = nullptr;
    float *ao_ = nullptr;
    float2 *ast_ = nullptr;
    float *out_dev_ = nullptr;
    int32_t *codes_host_ = nullptr;  // pinned staging
    float *out_host_ = nullptr;
    size_t out_host_cap_ = 0;
    CodecState stream_state_, whole_state_;
    bool whole_alloc_ = false;
    std::map<int, hipGraphExec_t> graphs_;  // per piece size (frames), stream state
    hipEvent_t ev_[kCodecStages + 1] = {};
    double last_ms_ = 0.0, stage_ms_[kCodecStages] = {0, 0, 0, 0};
    std::string info_;
    int max_splits_ = 1;
    bool eager_ = false;
};

}  // namespace mh
