// moss/llm.h -- GPU-backed moss::LlmModel (drop-in for the reference's header).
//
// Same public surface as the reference's csrc/include/moss/llm.h:39-90 (class,
// method names, argument meaning, return conventions, the Row / FrameTiming
// types and the model constants), implemented over the C ABI of libmoss_hip.so
// (include/moss_hip.h) instead of the CPU kernels.  SampleParams comes from the
// reference's own moss/sampler.h, unchanged.  Differences, all documented on the
// member: `threads` is accepted and unused (the GPU replaces the thread pool);
// errors of the device path surface as std::runtime_error (the reference's load()
// can already throw on a missing tensor, weights.cpp:128-138).
#pragma once

#include <array>
#include <atomic>
#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "moss/sampler.h"

struct moss_hip_llm;

namespace moss {

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

// One input row: [text_id, code0..code15]
using Row = std::array<int32_t, kNVq + 1>;

struct FrameTiming {
    double global_ms = 0.0;
    double local_ms = 0.0;
};

class LlmModel {
public:
    // threads: kept for source compatibility; the device is MOSS_HIP_DEVICE (default 0)
    // and the KV cache precision MOSS_HIP_KV ("fp16", default, or "fp32").
    explicit LlmModel(int threads = 1);
    ~LlmModel();
    LlmModel(const LlmModel &) = delete;
    LlmModel &operator=(const LlmModel &) = delete;

    bool load(const std::string &weights_path, std::string *err);
    void reset();
    void prefill(const std::vector<Row> &rows, int start = 0);

    void snapshot_prefix();
    void restore_prefix();
    int prefix_pos() const;

    bool save_prefix(const std::string &path, const std::vector<Row> &rows, std::string *err);
    bool load_prefix(const std::string &path, const std::vector<Row> &rows, std::string *err);
    bool save_state(const std::string &path, const std::vector<Row> &rows, std::string *err);
    bool load_state(const std::string &path, const std::vector<Row> &rows, bool ignore_weights_fp,
                    std::string *err);

    std::vector<Row> generate(int max_frames, const SampleParams &audio_params, uint64_t seed,
                              std::vector<FrameTiming> *timing = nullptr, const std::vector<Row> *forced = nullptr,
                              const std::function<void(int, const Row &)> &on_frame = {});

    void set_logits_dump(const std::string &path) { logits_dump_path_ = path; }
    void set_gate_dump(const std::string &path) { gate_dump_path_ = path; }
    void set_cancel_flag(const std::atomic<bool> *flag);

    // hidden state of the last position, copied from the device on each call
    const float *hidden() const;
    int position() const;
    const std::string &info() const { return info_; }

private:
    bool save_kv(const std::string &path, const char magic[8], bool with_hidden, const std::vector<Row> &rows,
                 std::string *err);
    bool load_kv(const std::string &path, const char magic[8], bool with_hidden, const std::vector<Row> &rows,
                 bool check_weights, std::string *err);
    void require_loaded() const;

    moss_hip_llm *h_ = nullptr;
    uint64_t weights_fp_ = 0;
    mutable std::array<float, kHidden> hidden_{};
    std::string info_;
    std::string logits_dump_path_, gate_dump_path_;
};

}  // namespace moss
