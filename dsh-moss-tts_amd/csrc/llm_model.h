// llm_model.h -- the GPU-resident MOSS-TTS-Nano LLM (host driver).
//
// Device-side counterpart of moss::LlmModel (reference csrc/include/moss/llm.h:39-90):
// owns the uploaded .moss blob, the KV cache, the device decode state and the
// captured hipGraphs of the global step and of a frame's local loop.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <atomic>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/moss_hip.h"
#include "mh_ops.h"

namespace mh {

struct Status : std::runtime_error {
    int code;
    Status(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

void hip_check(hipError_t e, const char *what);

// Fused decode launches redone per operator by every Model of the process.
extern std::atomic<int> fallbacks_total;

// One tensor of a .moss v1 index (reference csrc/src/weights.cpp:27-125).
struct MossEntry {
    uint8_t dtype = 0, ndim = 0;
    uint32_t dims[3] = {0, 0, 0};
    uint64_t off = 0, nbytes = 0;
};
// name -> entry; throws Status(EFORMAT) on a malformed index
std::unordered_map<std::string, MossEntry> parse_moss_index(const uint8_t *blob, size_t bytes);
bool is_vector(const MossEntry &e);

// SampleParams of the C ABI -> the device copy.  Greedy as sample_token decides
// it (sampler.cpp:23: greedy || top_k == 1).
inline SampleCfg sample_cfg(const moss_hip_sample_params &p) {
    SampleCfg c;
    c.greedy = (p.greedy || p.top_k == 1) ? 1 : 0;
    c.temperature = p.temperature;
    c.top_k = p.top_k;
    c.top_p = p.top_p;
    c.end_greedy = p.end_greedy ? 1 : 0;
    c.greedy_frames = p.greedy_frames;
    return c;
}

struct LayerW {
    const float *ln1_w, *ln1_b, *ln2_w, *ln2_b;
    const uint8_t *attn_w;
    const float *attn_b;
    const uint8_t *proj_w;
    const float *proj_b;
    const uint8_t *fc_in_w;
    const float *fc_in_b;
    const uint8_t *fc_out_w;
    const float *fc_out_b;
    // the four matrices again in the matrix-core order (tile_q8x4_mfma) read by
    // the GEMMs of the prefill and the batch engine; null: the GEMMs read the
    // Q8_0_4X4 copy (MOSS_HIP_GEMM_TILED=0)
    const uint8_t *attn_wm, *proj_wm, *fc_in_wm, *fc_out_wm;
};

// K slices of the prefill's fc_out GEMM from 128 rows on
constexpr int kPrefillFcOutSplit = 4;

class Model {
public:
    Model(const void *blob, size_t bytes, const moss_hip_llm_options &opt);
    ~Model();
    Model(const Model &) = delete;
    Model &operator=(const Model &) = delete;

    void reset();
    int position() const { return pos_; }
    int fallbacks() const { return fallbacks_; }
    void get_hidden(float *out);
    void set_hidden(const float *in);
    void prefill(const int32_t *rows, int n, int start);
    void global_step(const int32_t *row17);
    int generate(int max_frames, const moss_hip_sample_params &p, uint64_t seed, const int32_t *forced, int n_forced,
                 int32_t *out_rows, double *timing, float *logits_dump, float *gate_dump, moss_hip_frame_cb cb,
                 void *user);
    void set_cancel_flag(const volatile uint8_t *f) { cancel_ = f; }
    void snapshot_prefix();
    void restore_prefix();
    int prefix_pos() const { return prefix_pos_; }
    int gate_rows() const { return gate_rows_; }
    void kv_export(int n_pos, float *k, float *v);
    void kv_import(int n_pos, const float *k, const float *v, const float *hidden);

    int device() const { return device_; }
    hipStream_t stream() const { return stream_; }
    bool decode_a8() const { return decode_a8_ != 0; }

    // Where the state lives on the device (for a batch stream's admission, Batch::admit).
    struct StateView {
        const void *k, *v;         // layer 0 of K / V: [layer][head][ctx_stride][64]
        size_t layer_elems;        // elements between layers
        int ctx_stride;
        KvType kv;
        const float *hidden;       // [768]
        int pos;
    };
    StateView state_view() const {
        return StateView{kv_layer(0, 0), kv_layer(1, 0), (size_t)kHeads * max_ctx_ * kHeadDim, max_ctx_, kvt_,
                         hidden_, pos_};
    }

    // Quantiser capture (tests; moss_hip_llm_capture): W8A8 quantisers also record their
    // fp32 input, int8 output and scales, and the stage outputs around them.
    void set_capture(bool on);
    // Bytes of the last capture of `what` (MOSS_HIP_CAP_GLOBAL / LOCAL / PREFILL), copied to
    // out when out != nullptr and bytes suffice; 0 when none was taken.
    size_t capture_read(int what, void *out, size_t bytes);

    // Device weights, shared with the batched engine.
    struct Weights {
        const LayerW *global;  // [kLayers]
        const LayerW *local;
        const float *lnf_w, *lnf_b, *llnf_w, *llnf_b;
        const uint8_t *wte;
        const uint8_t *const *aemb;  // [kNVq]
        const uint8_t *const *aemb_m;  // [kNVq] in the matrix-core order (null entries: none)
        const float *slot_in;        // dequantised wte[kSlotToken]
        const float *qkv_table;      // [1 + 15 * 1024][2304] local q|k|v of (lpos >= 1, input code)
    };
    Weights weights() const {
        return Weights{g_, &local_, lnf_w_, lnf_b_, llnf_w_, llnf_b_, wte_, aemb_.data(), aemb_m_.data(), slot_in_,
                       qkv_table_};
    }

private:
    void enqueue_global_step(hipStream_t s, const int *row_dev);
    void enqueue_local_step(hipStream_t s, const float *in, int lpos, int pick_ch);
    void enqueue_frame_local(hipStream_t s, bool text_gate, bool fused);
    void build_graphs();
    void launch_global(hipStream_t s);
    void launch_frame_local(hipStream_t s, bool text_gate, bool fused);
    void write_state_header();
    void *kv_layer(int which, int layer) const;  // which: 0 = K, 1 = V

    int device_ = 0, max_ctx_ = kMaxCtx, use_graphs_ = 1;
    bool prefill_a16_ = false;  // prefill GEMMs on fp32 activations (else W8A8)
    int decode_a8_ = 0;         // decode GEMVs in W8A8 (the reference with MOSS_A16 unset), else W8A16
    bool fused_layers_ = false; // global step as one decode_layer launch per layer, local steps as decode_local
    // Poll rounds a wait of the fused kernels may take (0: kPollBudget, ~0.05 s).  MOSS_HIP_POLL_BUDGET
    // = "N" or "N@K" overrides it (from the K-th fused launch of the model on), so tests can make
    // the waits run out at a chosen launch and exercise the fallback below.
    int poll_budget_ = 0, poll_budget_from_ = 0;
    long fused_launches_ = 0;
    int next_poll_budget() { return fused_launches_++ >= poll_budget_from_ ? poll_budget_ : 0; }
    // A fused launch whose wait ran out (the device did not hold every workgroup at once, e.g.
    // another stream occupied CUs) is redone on the per-operator path from the last good state;
    // the rest of that call stays per operator.  fallbacks_ counts such recoveries.
    int fallbacks_ = 0;
    bool can_fall_back() const { return max_ctx_ <= 64 * 16; }
    float *qkv_table_ = nullptr;   // [1 + 15 * 1024][2304] local q|k|v of (lpos >= 1, input code)
    void build_qkv_table();
    uint64_t *ll_ = nullptr;    // kLayerWords exchange words of the fused layer launches
    LayerArgs *layer_args_ = nullptr;  // [kLayers] per-block arguments of the fused global step (device)
    void clear_exchange();      // before a sequence of fused launches: no stale word carries a current tag
    void check_exchange();      // throws if a fused launch ran out of its wait budget
    KvType kvt_ = KV_F16;
    size_t kv_esize_ = 2;
    hipStream_t stream_ = nullptr;
    // per frame slot (2): local start / end, global start / end (timing), state copied
    enum { kEvLocal0, kEvLocal1, kEvGlobal0, kEvGlobal1, kEvRead, kEvPerSlot };
    hipEvent_t ev_[2 * kEvPerSlot] = {};
    int gate_rows_ = 0;                 // frames whose end gate the last generate evaluated (gate dump rows)

    uint8_t *blob_ = nullptr;
    LayerW g_[kLayers] = {}, local_ = {};
    const float *lnf_w_ = nullptr, *lnf_b_ = nullptr, *llnf_w_ = nullptr, *llnf_b_ = nullptr;
    const uint8_t *wte_ = nullptr;
    std::array<const uint8_t *, kNVq> aemb_{};
    uint8_t *wm_ = nullptr;              // the GEMM matrices in the matrix-core order (LayerW::*_wm, aemb_m_)
    std::array<const uint8_t *, kNVq> aemb_m_{};
    void tile_gemm_weights();

    // device buffers
    void *kv_ = nullptr;                 // [2][layers][heads][max_ctx][64]
    float *lkv_ = nullptr;               // [2][heads][17][64] fp32
    float *rope_ = nullptr;              // cos [n][32] then sin [n][32]
    int rope_n_ = 0;
    float *x_ = nullptr, *q_ = nullptr, *mlp_ = nullptr, *hidden_ = nullptr;
    float *lres_ = nullptr, *next_in_ = nullptr, *slot_in_ = nullptr;
    float *attn_out_ = nullptr;
    float *attn_part_ = nullptr;         // [12][ceil(max_ctx / 64)][kPartStride] split-KV partials
    float *logits_ = nullptr;            // [16][1024]
    int *counts_ = nullptr;              // [16][1024]
    int *forced_ = nullptr;              // [max_ctx][16]
    float *text_logits_ = nullptr;       // [16384] text head of gate-dump frames
    int *rows_dev_ = nullptr;            // prefill rows [n][17]
    int rows_cap_ = 0;
    float *pre_x_ = nullptr, *pre_a_ = nullptr, *pre_q_ = nullptr, *pre_h_ = nullptr;  // prefill rows
    float *pre_part_ = nullptr;          // split-K partials of the prefill proj / fc_out GEMMs
    int8_t *pre_q8_ = nullptr;           // W8A8 prefill: the current GEMM's int8 activations [m][<=768]
    float *pre_d8_ = nullptr;            //   and their block scales [m][<=24]
    int8_t *pre_q8h_ = nullptr;          // W8A8 prefill: fc_in's output quantised by its epilogue [m][3072]
    float *pre_d8h_ = nullptr;           //   and its block scales [m][96]
    DevState *state_ = nullptr;          // device
    DevState *hstate_ = nullptr;         // pinned host mirror
    DevState *hread_ = nullptr;          // [2] pinned per-frame state readback (frames alternate)
    void *snap_ = nullptr;               // prefix snapshot [2][layers][heads][prefix][64]

    hipGraphExec_t g_global_ = nullptr, g_local_ = nullptr, g_local_fused_ = nullptr;

    bool capture_ = false;
    float *cap_dec_ = nullptr;           // [kLayers + kLocalLen][MOSS_HIP_CAP_STEP]: global blocks, local positions
    uint8_t *cap_pre_ = nullptr;         // prefill capture, [kLayers] x cap_layer_bytes(m)
    size_t cap_pre_bytes_ = 0;           // its allocation
    size_t cap_pre_used_ = 0;            // bytes of the last W8A8 prefill captured
    bool cap_taken_[2] = {false, false}; // a global step / local half was captured

    int pos_ = 0, prefix_pos_ = 0;
    const volatile uint8_t *cancel_ = nullptr;
};

}  // namespace mh
