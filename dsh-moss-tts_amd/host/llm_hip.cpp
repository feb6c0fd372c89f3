// llm_hip.cpp -- moss::LlmModel over the libmoss_hip.so C ABI (see moss/llm.h).
#include "moss/llm.h"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>

#include "moss_hip.h"

namespace moss {
namespace {

// FNV-1a 64 fingerprints of the reference (csrc/src/llm.cpp:407-439).
constexpr uint64_t kFnvOffset = 1469598103934665603ull;
constexpr uint64_t kFnvPrime = 1099511628211ull;

uint64_t fnv(uint64_t h, const void *data, size_t n) {
    const uint8_t *p = static_cast<const uint8_t *>(data);
    for (size_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= kFnvPrime;
    }
    return h;
}

uint64_t fingerprint_rows(const std::vector<Row> &rows) {
    uint64_t h = kFnvOffset;
    for (const Row &r : rows) h = fnv(h, r.data(), sizeof(int32_t) * r.size());
    return h;
}

// 40-byte header shared by the prefix and state files (csrc/src/llm.cpp:441-451).
struct FileHeader {
    char magic[8];
    uint32_t version;
    uint32_t layers;
    uint32_t n_pos;
    uint32_t hidden;
    uint64_t rows_fp;
    uint64_t weights_fp;
};
static_assert(sizeof(FileHeader) == 40, "prefix/state header is 40 bytes");

constexpr char kPrefixMagic[8] = {'M', 'O', 'S', 'S', 'P', 'F', 'X', '1'};
constexpr char kStateMagic[8] = {'M', 'O', 'S', 'S', 'S', 'T', '1', '\0'};

[[noreturn]] void device_error(const char *what) {
    throw std::runtime_error(std::string(what) + ": " + moss_hip_last_error());
}

void frame_trampoline(void *user, int frame, const int32_t row[17]) {
    const auto *cb = static_cast<const std::function<void(int, const Row &)> *>(user);
    Row r;
    std::memcpy(r.data(), row, sizeof(int32_t) * 17);
    (*cb)(frame, r);
}

}  // namespace

LlmModel::LlmModel(int threads) { (void)threads; }

LlmModel::~LlmModel() {
    if (!h_) return;
    // MOSS_HIP_REPORT set: one JSON line on stderr with the model's count of fused launches
    // redone on the per-operator path (co-residency lost at run time, e.g. to another stream)
    if (const char *r = std::getenv("MOSS_HIP_REPORT"); r && *r && std::strcmp(r, "0") != 0)
        std::fprintf(stderr, "{\"moss_hip_fallbacks\": %d}\n", moss_hip_llm_fallbacks(h_));
    moss_hip_llm_destroy(h_);
}

void LlmModel::require_loaded() const {
    if (!h_) throw std::runtime_error("LlmModel: load() has not succeeded");
}

bool LlmModel::load(const std::string &path, std::string *err) {
    std::FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) {
        if (err) *err = "cannot open weights file: " + path;
        return false;
    }
    std::fseek(f, 0, SEEK_END);
    const long size = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    std::vector<uint8_t> data(size > 0 ? static_cast<size_t>(size) : 0);
    const size_t got = data.empty() ? 0 : std::fread(data.data(), 1, data.size(), f);
    std::fclose(f);
    if (size <= 16 || got != data.size()) {
        if (err) *err = "weights file too small or unreadable: " + path;
        return false;
    }
    moss_hip_llm_options opt{0, 0, 0, 1, 0, 0, 0};
    if (const char *d = std::getenv("MOSS_HIP_DEVICE")) opt.device = std::atoi(d);
    // the reference's switch (gemv.cpp:23-48), read as it reads it: unset (or any other value) =
    // W8A8 prefill and decode; "decode" = W8A8 prefill, W8A16 decode; "1" / "all" = W8A16 both
    const char *a16 = std::getenv("MOSS_A16");
    const int mode = a16 == nullptr ? 0 : (a16[0] == '1' || std::strcmp(a16, "all") == 0) ? 1
                                          : std::strcmp(a16, "decode") == 0 ? 2 : 0;
    opt.prefill_a16 = mode == 1;
    opt.decode_a8 = mode == 0;
    if (const char *kv = std::getenv("MOSS_HIP_KV")) opt.kv_dtype = std::strcmp(kv, "fp32") == 0 ? 1 : 0;
    moss_hip_llm *h = nullptr;
    if (moss_hip_llm_create(data.data(), data.size(), &opt, &h) != MOSS_HIP_OK) {
        const std::string msg = moss_hip_last_error();
        // a missing tensor throws in the reference (weights.cpp:128-138); keep that behaviour
        if (msg.rfind("missing", 0) == 0) throw std::runtime_error(msg);
        if (err) *err = msg;
        return false;
    }
    if (h_) moss_hip_llm_destroy(h_);
    h_ = h;
    const int64_t sz = size;
    weights_fp_ = fnv(fnv(kFnvOffset, &sz, sizeof(sz)), data.data(), data.size() < 4096 ? data.size() : 4096);
    info_ = "weights=" + path + " bytes=" + std::to_string(data.size()) + " device=" + std::to_string(opt.device);
    return true;
}

void LlmModel::reset() {
    require_loaded();
    if (moss_hip_llm_reset(h_) != MOSS_HIP_OK) device_error("reset");
}

void LlmModel::prefill(const std::vector<Row> &rows, int start) {
    require_loaded();
    static_assert(sizeof(Row) == 17 * sizeof(int32_t), "Row is 17 packed int32");
    if (moss_hip_llm_prefill(h_, rows.empty() ? nullptr : rows[0].data(), static_cast<int>(rows.size()), start) !=
        MOSS_HIP_OK)
        device_error("prefill");
}

void LlmModel::snapshot_prefix() {
    require_loaded();
    if (moss_hip_llm_snapshot_prefix(h_) != MOSS_HIP_OK) device_error("snapshot_prefix");
}

void LlmModel::restore_prefix() {
    require_loaded();
    if (moss_hip_llm_restore_prefix(h_) != MOSS_HIP_OK) device_error("restore_prefix");
}

int LlmModel::prefix_pos() const { return h_ ? moss_hip_llm_prefix_pos(h_) : 0; }
int LlmModel::position() const { return h_ ? moss_hip_llm_position(h_) : 0; }

const float *LlmModel::hidden() const {
    if (h_ && moss_hip_llm_get_hidden(h_, hidden_.data()) != MOSS_HIP_OK) device_error("hidden");
    return hidden_.data();
}

void LlmModel::set_cancel_flag(const std::atomic<bool> *flag) {
    require_loaded();
    static_assert(sizeof(std::atomic<bool>) == 1, "std::atomic<bool> is polled as one byte");
    moss_hip_llm_set_cancel_flag(h_, reinterpret_cast<const volatile uint8_t *>(flag));
}

// .mosskv prefix / state files (csrc/src/llm.cpp:485-632): header, then per layer
// K[n_pos][768] and V[n_pos][768] fp32, then (state only) hidden[768].
bool LlmModel::save_kv(const std::string &path, const char magic[8], bool with_hidden, const std::vector<Row> &rows,
                       std::string *err) {
    require_loaded();
    const int n = position();
    if (n <= 0) {
        if (err) *err = "nothing to save: position is 0";
        return false;
    }
    std::vector<float> k((size_t)12 * n * kHidden), v((size_t)12 * n * kHidden);
    if (moss_hip_llm_kv_export(h_, n, k.data(), v.data()) != MOSS_HIP_OK) device_error("kv_export");
    std::FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) {
        if (err) *err = "cannot write: " + path;
        return false;
    }
    FileHeader h{};
    std::memcpy(h.magic, magic, 8);
    h.version = 1;
    h.layers = 12;
    h.n_pos = static_cast<uint32_t>(n);
    h.hidden = kHidden;
    h.rows_fp = fingerprint_rows(rows);
    h.weights_fp = weights_fp_;
    bool ok = std::fwrite(&h, sizeof(h), 1, f) == 1;
    const size_t per = (size_t)n * kHidden;
    for (int l = 0; l < 12 && ok; ++l) {
        ok = std::fwrite(k.data() + l * per, sizeof(float), per, f) == per &&
             std::fwrite(v.data() + l * per, sizeof(float), per, f) == per;
    }
    if (ok && with_hidden) ok = std::fwrite(hidden(), sizeof(float), kHidden, f) == (size_t)kHidden;
    std::fclose(f);
    if (!ok && err) *err = "short write: " + path;
    return ok;
}

bool LlmModel::load_kv(const std::string &path, const char magic[8], bool with_hidden, const std::vector<Row> &rows,
                       bool check_weights, std::string *err) {
    require_loaded();
    std::FILE *f = std::fopen(path.c_str(), "rb");
    if (!f) {
        if (err) *err = "cannot open: " + path;
        return false;
    }
    FileHeader h{};
    if (std::fread(&h, sizeof(h), 1, f) != 1 || std::memcmp(h.magic, magic, 8) != 0 || h.version != 1 ||
        h.layers != 12 || h.hidden != (uint32_t)kHidden || h.n_pos == 0 || h.n_pos > (uint32_t)kMaxCtx) {
        std::fclose(f);
        if (err) *err = "bad header: " + path;
        return false;
    }
    if (h.rows_fp != fingerprint_rows(rows)) {
        std::fclose(f);
        if (err) *err = "rows fingerprint mismatch: " + path;
        return false;
    }
    if (check_weights && h.weights_fp != weights_fp_) {
        std::fclose(f);
        if (err) *err = "weights fingerprint mismatch: " + path;
        return false;
    }
    const size_t per = (size_t)h.n_pos * kHidden;
    std::vector<float> k(12 * per), v(12 * per), hid(kHidden);
    bool ok = true;
    for (int l = 0; l < 12 && ok; ++l) {
        ok = std::fread(k.data() + l * per, sizeof(float), per, f) == per &&
             std::fread(v.data() + l * per, sizeof(float), per, f) == per;
    }
    if (ok && with_hidden) ok = std::fread(hid.data(), sizeof(float), kHidden, f) == (size_t)kHidden;
    std::fclose(f);
    if (!ok) {
        if (err) *err = "truncated: " + path;
        return false;
    }
    if (moss_hip_llm_kv_import(h_, (int)h.n_pos, k.data(), v.data(), with_hidden ? hid.data() : nullptr) !=
        MOSS_HIP_OK)
        device_error("kv_import");
    snapshot_prefix();  // kept in memory for repeated restores, as the reference does
    return true;
}

bool LlmModel::save_prefix(const std::string &path, const std::vector<Row> &rows, std::string *err) {
    return save_kv(path, kPrefixMagic, false, rows, err);
}
bool LlmModel::load_prefix(const std::string &path, const std::vector<Row> &rows, std::string *err) {
    return load_kv(path, kPrefixMagic, false, rows, true, err);
}
bool LlmModel::save_state(const std::string &path, const std::vector<Row> &rows, std::string *err) {
    return save_kv(path, kStateMagic, true, rows, err);
}
bool LlmModel::load_state(const std::string &path, const std::vector<Row> &rows, bool ignore_weights_fp,
                          std::string *err) {
    return load_kv(path, kStateMagic, true, rows, !ignore_weights_fp, err);
}

std::vector<Row> LlmModel::generate(int max_frames, const SampleParams &p, uint64_t seed,
                                    std::vector<FrameTiming> *timing, const std::vector<Row> *forced,
                                    const std::function<void(int, const Row &)> &on_frame) {
    require_loaded();
    std::vector<Row> frames;
    if (max_frames <= 0) return frames;
    const moss_hip_sample_params sp{p.greedy ? 1 : 0, p.temperature, p.top_k, p.top_p, p.repetition_penalty,
                                    p.end_greedy ? 1 : 0, p.min_frames, p.greedy_frames};
    // frame f runs while position() + f < kMaxCtx (llm.cpp:644), so at most this many
    const int bound = kMaxCtx - position();
    int cap = max_frames < bound ? max_frames : bound;
    if (forced && (int)forced->size() < cap) cap = (int)forced->size();
    if (cap <= 0) return frames;
    std::vector<int32_t> out((size_t)cap * 17);
    std::vector<double> t(timing ? (size_t)cap * 2 : 0);
    std::vector<float> logits(logits_dump_path_.empty() ? 0 : (size_t)cap * kNVq * kCodebook);
    std::vector<float> gate(gate_dump_path_.empty() ? 0 : (size_t)cap * 4);
    int n = 0;
    const int rc = moss_hip_llm_generate(
        h_, max_frames, &sp, seed, forced ? (*forced)[0].data() : nullptr, forced ? (int)forced->size() : 0,
        out.data(), &n, timing ? t.data() : nullptr, logits.empty() ? nullptr : logits.data(),
        gate.empty() ? nullptr : gate.data(), on_frame ? frame_trampoline : nullptr,
        on_frame ? const_cast<std::function<void(int, const Row &)> *>(&on_frame) : nullptr);
    if (rc != MOSS_HIP_OK) device_error("generate");
    frames.resize(n);
    for (int i = 0; i < n; ++i) std::memcpy(frames[i].data(), out.data() + (size_t)i * 17, sizeof(int32_t) * 17);
    if (timing)
        for (int i = 0; i < n; ++i) timing->push_back(FrameTiming{t[2 * i], t[2 * i + 1]});
    if (!logits_dump_path_.empty()) {  // raw fp32 [frames][16][1024], as llm.cpp:714-720
        if (std::FILE *fp = std::fopen(logits_dump_path_.c_str(), "wb")) {
            std::fwrite(logits.data(), sizeof(float), (size_t)n * kNVq * kCodebook, fp);
            std::fclose(fp);
        }
    }
    if (!gate_dump_path_.empty()) {  // the CSV of llm.cpp:721-731
        if (std::FILE *fp = std::fopen(gate_dump_path_.c_str(), "wb")) {
            std::fprintf(fp, "frame,argmax_id,argmax_minus_slot,slot_minus_end\n");
            const int rows = moss_hip_llm_gate_rows(h_);  // the frame the gate stopped has a row too
            for (int i = 0; i < rows; ++i) {
                const float *g = gate.data() + 4 * (size_t)i;  // (l_end, l_slot, argmax_id, argmax_logit)
                std::fprintf(fp, "%d,%d,%.4f,%.4f\n", i, (int)g[2], g[3] - g[1], g[1] - g[0]);
            }
            std::fclose(fp);
        }
    }
    return frames;
}

}  // namespace moss
