// moss_llm_hip -- drives the GPU moss::LlmModel (dsh-moss-tts_amd/host) the way the
// reference's moss_llm CLI drives its CPU LlmModel (csrc/src/main.cpp:44-222):
//   moss_llm_hip --weights x.moss --prompt rows.txt [--frames N] [--min-frames N]
//                [--greedy|--sample] [--seed S] [--end-mode greedy|sample] [--rep P]
//                [--load-state s] [--ignore-state-fp] [--save-state s]
//                [--save-prefix p] [--load-prefix p] [--prefix-rows K]
//                [--force-codes codes.txt] [--dump-logits f] [--dump-gate f]
// Sampling defaults are main.cpp:133-140's (temperature 0.8, top-k 25, top-p 0.95,
// repetition penalty 1.2).
// Prompt rows: 17 integers per line, '#' comments (main.cpp:20-40).  Prints JSON.
// --prefix-rows K follows the engine's voice-prefix flow (engine.cpp:200-242): the
// first K rows are the prefix (loaded from --load-prefix, else prefilled and
// snapshotted), the rest are prefilled at start = K.
#include <chrono>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "moss/llm.h"

using namespace moss;

static bool read_rows(const std::string &path, std::vector<Row> *rows, bool codes_only) {
    std::ifstream in(path);
    if (!in) return false;
    std::string line;
    while (std::getline(in, line)) {
        if (line.empty() || line[0] == '#') continue;
        std::istringstream iss(line);
        Row r{};
        if (codes_only) r[0] = kSlotToken;
        for (int i = codes_only ? 1 : 0; i < kNVq + 1; ++i)
            if (!(iss >> r[i])) return false;
        rows->push_back(r);
    }
    return true;
}

int main(int argc, char **argv) {
    std::string weights, prompt, state_in, state_out, prefix_in, prefix_out, force, logits, gate, end_mode = "greedy";
    uint64_t seed = 0;
    int frames = 8, min_frames = 0, prefix_rows = 0;
    bool greedy = false, ignore_fp = false;
    float rep = 1.2f;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&]() -> std::string { return i + 1 < argc ? argv[++i] : ""; };
        if (a == "--weights") weights = next();
        else if (a == "--prompt") prompt = next();
        else if (a == "--frames") frames = std::stoi(next());
        else if (a == "--min-frames") min_frames = std::stoi(next());
        else if (a == "--greedy") greedy = true;
        else if (a == "--sample") greedy = false;
        else if (a == "--seed") seed = std::stoull(next());
        else if (a == "--end-mode") end_mode = next();
        else if (a == "--dump-gate") gate = next();
        else if (a == "--rep") rep = std::stof(next());
        else if (a == "--load-state") state_in = next();
        else if (a == "--ignore-state-fp") ignore_fp = true;
        else if (a == "--save-state") state_out = next();
        else if (a == "--load-prefix") prefix_in = next();
        else if (a == "--save-prefix") prefix_out = next();
        else if (a == "--force-codes") force = next();
        else if (a == "--dump-logits") logits = next();
        else if (a == "--prefix-rows") prefix_rows = std::stoi(next());
        else {
            std::fprintf(stderr, "unknown argument: %s\n", a.c_str());
            return 1;
        }
    }
    std::vector<Row> rows;
    if (weights.empty() || !read_rows(prompt, &rows, false) || rows.empty()) {
        std::fprintf(stderr, "usage: moss_llm_hip --weights <x.moss> --prompt <rows.txt> [options]\n");
        return 1;
    }
    LlmModel model(4);
    std::string err;
    if (!model.load(weights, &err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return 1;
    }
    if (prefix_rows < 0 || prefix_rows > static_cast<int>(rows.size())) {
        std::fprintf(stderr, "bad --prefix-rows\n");
        return 1;
    }
    const std::vector<Row> prefix(rows.begin(), rows.begin() + (prefix_rows ? prefix_rows : rows.size()));
    const auto t0 = std::chrono::steady_clock::now();
    bool ok = true;
    if (!state_in.empty()) ok = model.load_state(state_in, rows, ignore_fp, &err);
    else if (!prefix_in.empty()) ok = model.load_prefix(prefix_in, prefix, &err);
    else {
        model.prefill(prefix);
        model.snapshot_prefix();
    }
    if (!ok) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return 2;
    }
    if (!prefix_out.empty() && !model.save_prefix(prefix_out, prefix, &err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return 3;
    }
    if (state_in.empty() && prefix_rows) {
        model.restore_prefix();
        model.prefill(std::vector<Row>(rows.begin() + prefix_rows, rows.end()), model.prefix_pos());
    }
    const double prefill_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    if (!state_out.empty() && !model.save_state(state_out, rows, &err)) {
        std::fprintf(stderr, "%s\n", err.c_str());
        return 3;
    }
    std::vector<Row> forced;
    if (!force.empty() && (!read_rows(force, &forced, true) || forced.empty())) {
        std::fprintf(stderr, "bad --force-codes file\n");
        return 1;
    }
    if (!logits.empty()) model.set_logits_dump(logits);
    if (!gate.empty()) model.set_gate_dump(gate);
    SampleParams p;
    p.greedy = greedy;
    p.end_greedy = end_mode != "sample";
    p.min_frames = min_frames;
    p.temperature = 0.8f;
    p.top_k = 25;
    p.top_p = 0.95f;
    p.repetition_penalty = rep;
    std::vector<FrameTiming> timing;
    int callbacks = 0;
    const std::vector<Row> codes =
        model.generate(frames, p, seed, &timing, forced.empty() ? nullptr : &forced, [&](int, const Row &) { ++callbacks; });
    double g = 0, l = 0;
    for (const auto &t : timing) {
        g += t.global_ms;
        l += t.local_ms;
    }
    std::printf("{\"prefill_ms\": %.3f, \"frames\": %zu, \"callbacks\": %d, \"position\": %d, ", prefill_ms,
                codes.size(), callbacks, model.position());
    std::printf("\"global_ms_per_frame\": %.4f, \"local_ms_per_frame\": %.4f, \"hidden0\": %.9g, \"codes\": [",
                timing.empty() ? 0.0 : g / timing.size(), timing.empty() ? 0.0 : l / timing.size(), model.hidden()[0]);
    for (size_t i = 0; i < codes.size(); ++i) {
        std::printf("%s[", i ? ", " : "");
        for (int ch = 0; ch < kNVq; ++ch) std::printf("%s%d", ch ? ", " : "", codes[i][ch + 1]);
        std::printf("]");
    }
    std::printf("]}\n");
    return 0;
}
