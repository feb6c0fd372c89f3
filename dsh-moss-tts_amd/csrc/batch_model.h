// batch_model.h -- batched multi-stream decode on one GPU.
//
// Many independent TTS streams (each one LlmModel state in the reference,
// csrc/include/moss/llm.h:39-90, which is single-stream) decoded in lock-step:
// every projection is one W8A16 GEMM over all streams on the matrix cores, the
// global KV cache is paged (per layer a pool of 64-position pages, one block
// table row per stream), attention runs per (head, stream) over that stream's
// pages, and the local transformer, heads, greedy picks and end gate run per
// stream.  Weights are the model's own device copy.  The batch decodes in its model's
// activation mode: W8A16 (fp32 activations), or W8A8 when the model was created with
// decode_a8 (the reference with MOSS_A16 unset) -- then every GEMM input is quantised
// per 32-block by the kernel that produces it and the GEMMs run on the int8 matrix
// cores, the prefill's operand form.
#pragma once

#include <map>
#include <vector>

#include "llm_model.h"

namespace mh {

class Batch {
public:
    static constexpr int kPage = 64;

    Batch(Model &model, int max_streams, int capacity, KvType kv);
    ~Batch();
    Batch(const Batch &) = delete;
    Batch &operator=(const Batch &) = delete;

    int max_streams() const { return S_; }
    int capacity() const { return cap_; }
    int position(int s) const { return pos_[s]; }
    int device() const { return model_.device(); }
    // Loads one stream's state: K/V [12][n_pos][768] fp32 (reference layout) and hidden[768].
    void set_stream(int s, int n_pos, const float *k, const float *v, const float *hidden);
    // The same from a single-stream model's device state (its K/V, hidden, position), on the device.
    void admit(int s, Model &src);
    bool a8() const { return a8_; }
    // Attention capture of the W8A8 batch (tests): every attention of the frames run while on
    // records its fp32 output and int8 operand (graphs are re-captured when this changes).
    void set_capture(bool on);
    size_t capture_read(void *out, size_t bytes);
    void get_hidden(int s, float *out);
    void kv_export(int s, int n_pos, float *k, float *v);
    // One global step for streams [0, n): rows [n][17].
    void global_step(int n, const int32_t *rows);
    // Frames for streams [0, n) (llm.cpp:634-733 per stream, in lock-step); stream s
    // draws from its own xoshiro stream seeded with seeds[s] (0 when seeds is null).
    // out_rows [frames][n][17]; out_frames[s] = frames stream s produced.  Returns elapsed ms.
    double generate(int n, int frames, const moss_hip_sample_params &p, const uint64_t *seeds, int32_t *out_rows,
                    int *out_frames);

private:
    struct Graphs {
        hipGraphExec_t local = nullptr, local_greedy = nullptr, global = nullptr;
    };
    // attn = false: the step's attention output is already in o_ (the fused pick + attention)
    void enqueue_local_step(hipStream_t s, int n, const float *in, int in_stride, int lpos, bool attn = true);
    // W8A8: proj -> LN2 -> fc_in -> fc_out -> ln_f of a local step, after its attention
    void enqueue_local_step_a8(hipStream_t s, int n, const float *in, int in_stride);
    // greedy: channel picks fused with the next position's attention (greedy frames only)
    void enqueue_frame_local(hipStream_t s, int n, bool greedy);
    void enqueue_global(hipStream_t s, int n);
    void enqueue_global_a8(hipStream_t s, int n);
    Graphs &graphs_for(int n);
    StreamState state() const;
    void write_ctrl(int min_frames, float rep, const SampleCfg &cfg);

    Model &model_;
    Model::Weights w_;
    int S_ = 0, cap_ = 0, pages_ = 0;
    KvType kvt_ = KV_F16;
    size_t esize_ = 2;
    hipStream_t stream_ = nullptr;
    hipEvent_t ev_[2] = {};

    void *kpool_ = nullptr, *vpool_ = nullptr;  // [layer][S*pages][heads][64][64]
    size_t layer_pool_elems_ = 0;
    float *lkv_ = nullptr;                      // local K then V: [S][heads][17][64] fp32 each
    int *table_ = nullptr;                      // [S][pages]
    float *rope_ = nullptr;                     // cos [cap+1][32] then sin
    int rope_n_ = 0;
    float *x_ = nullptr, *a_ = nullptr, *q_ = nullptr, *o_ = nullptr, *h_ = nullptr;
    float *hidden_ = nullptr, *lres_ = nullptr, *next_in_ = nullptr, *logits_ = nullptr;
    int *pos_d_ = nullptr, *codes_ = nullptr, *row_ = nullptr, *counts_ = nullptr;
    // the streams longest context first, the order of the paged attention's workgroups
    // (set from pos_ at every generate / global_step call), and its pinned host staging
    int *order_ = nullptr, *order_h_ = nullptr;
    void upload_order(int n);
    float *part_ = nullptr;                     // [16][S][768] split-K partials
    float *xhl_ = nullptr;   // proj's output as hi / lo halves (fc_in's operand), rows padded to 16
    float *xst_ = nullptr;   // its per-16-column LayerNorm statistics [48][S][2]
    float *pairs_ = nullptr; // the audio head's greedy partials [S][64][2]
    // W8A8 (a8_): the current GEMM's int8 operand in the matrix-core order, K = 768 (LN rows,
    // attention outputs) and K = 3072 (fc_in's output), with their block scales; rows padded to 16
    bool a8_ = false;
    int8_t *q8a_ = nullptr, *q8h_ = nullptr;
    float *d8a_ = nullptr, *d8h_ = nullptr;
    // attention capture (tests; set_capture): after every attention of a frame, its fp32
    // output rows and the W8A8 operand quantised from them, [kLayers + kNVq + 1] entries
    bool capture_ = false;
    uint8_t *acap_ = nullptr;
    size_t acap_entry_ = 0;
    void capture_attention(hipStream_t s, int n, int slot);
    BatchCtl *ctrl_ = nullptr;
    uint32_t *rng_ = nullptr;                   // [S][4]
    unsigned char *active_ = nullptr;
    float *gate_ = nullptr;
    int *hist_codes_ = nullptr;                 // [cap+1][S][16] codes per frame
    unsigned char *hist_active_ = nullptr;      // [cap+1][S] active after each frame's gate
    BatchCtl *ctrl_h_ = nullptr;                // pinned host staging for ctrl
    std::vector<int> pos_;
    std::map<int, Graphs> graphs_;
};

}  // namespace mh
