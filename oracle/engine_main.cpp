// engine_main.cpp -- drives the reference's TtsEngine (csrc/include/moss/engine.h,
// csrc/src/engine.cpp, compiled unchanged from the reference sources) end to end:
// load -> set_voice -> synthesize (twice: the second from the .mosskv prefix cache
// the first wrote) -> synthesize with a cancel flag raised after the first chunk.
//
// Built twice by oracle/Makefile, from the same source: engine_gpu links the GPU
// drop-in moss::LlmModel (dsh-moss-tts_amd/host/llm_hip.cpp over libmoss_hip.so),
// engine_cpu links the reference's own llm.cpp.  Everything else (tokenizer,
// prompt, codec decoder) is the reference's CPU code in both, so the two outputs
// differ only through the LLM.  Test infrastructure: tests/test_gpu_engine.py
// runs both and compares their codes and PCM.
//
// usage: engine_{gpu,cpu} LLM.moss DECODER.moss TOKENIZER.mossvocab WORKDIR TEXT SEED GREEDY MAX_FRAMES
// writes WORKDIR/run{1,2,3}.pcm (interleaved float32: the codec's output of the LLM's
// codes, frame by frame) and prints one JSON line per run (with its wall time, "ms").
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "moss/engine.h"
#include "moss/profile.h"

namespace {

bool write_file(const std::string &path, const void *data, size_t bytes) {
    std::FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = bytes == 0 || std::fwrite(data, 1, bytes, f) == bytes;
    std::fclose(f);
    return ok;
}

// A voice profile of `frames` frames of seeded codes (a .mossclone needs no encoder).
moss::VoiceProfile synthetic_voice(int frames, uint32_t seed) {
    moss::VoiceProfile p;
    p.name = "synthvoice";
    p.frames = frames;
    p.codes.resize(static_cast<size_t>(frames) * 16);
    uint32_t s = seed * 2654435761u + 1u;
    for (auto &c : p.codes) {
        s = s * 1664525u + 1013904223u;
        c = static_cast<int16_t>((s >> 8) % 1024u);
    }
    return p;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 9) {
        std::fprintf(stderr, "usage: %s LLM DECODER TOKENIZER WORKDIR TEXT SEED GREEDY MAX_FRAMES\n", argv[0]);
        return 2;
    }
    const std::string workdir = argv[4], text = argv[5];
    moss::EngineOptions eo;
    eo.llm_path = argv[1];
    eo.decoder_path = argv[2];
    eo.tokenizer_path = argv[3];
    eo.cache_dir = workdir + "/cache";
    eo.llm_threads = 4;
    eo.decode_threads = 4;
    std::string err;
    moss::TtsEngine engine;
    if (!engine.load(eo, &err)) {
        std::fprintf(stderr, "load: %s\n", err.c_str());
        return 1;
    }
    const std::string voice = workdir + "/synthvoice.mossclone";
    if (!moss::profile_save(voice, synthetic_voice(24, 5), &err) || !engine.set_voice(voice, &err)) {
        std::fprintf(stderr, "voice: %s\n", err.c_str());
        return 1;
    }
    for (int run = 1; run <= 3; ++run) {
        std::vector<float> pcm;
        std::atomic<bool> cancel{false};
        moss::SynthOptions so;
        so.seed = std::strtoull(argv[6], nullptr, 10);
        so.greedy = std::atoi(argv[7]) != 0;
        so.max_frames = std::atoi(argv[8]);
        so.min_frames = so.max_frames;  // the synthetic model's gate would end at random
        so.chunk_frames = 4;
        if (run == 3) so.cancel = &cancel;  // raised once the first chunk's audio is out
        so.on_audio = [&](const float *x, int frames) {
            pcm.insert(pcm.end(), x, x + static_cast<size_t>(frames) * 2);
            if (run == 3) cancel.store(true);
        };
        moss::SynthStats st;
        const auto t0 = std::chrono::steady_clock::now();
        if (!engine.synthesize(text, so, &st, &err)) {
            std::fprintf(stderr, "synthesize: %s\n", err.c_str());
            return 1;
        }
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        const std::string base = workdir + "/run" + std::to_string(run);
        if (!write_file(base + ".pcm", pcm.data(), pcm.size() * sizeof(float))) return 1;
        std::printf("{\"run\": %d, \"chunks\": %d, \"text_tokens\": %d, \"frames\": %d, \"samples\": %zu, "
                    "\"prefix_cache_hit\": %s, \"cancelled\": %s, \"ms\": %.2f}\n",
                    run, st.chunks, st.text_tokens, st.frames, pcm.size() / 2, st.prefix_cache_hit ? "true" : "false",
                    st.cancelled ? "true" : "false", ms);
        std::fflush(stdout);
    }
    return 0;
}
