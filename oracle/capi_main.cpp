// capi_main.cpp -- drives the reference's C API (csrc/include/moss/tts.h, implemented by
// csrc/src/capi.cpp over TtsEngine, both compiled unchanged from the reference sources)
// end to end: moss_version -> moss_create -> moss_set_voice -> moss_text_tokens ->
// moss_set_sampling -> moss_speak (twice, the same text) -> moss_destroy, keeping the
// int16 PCM its callback receives.
//
// Built three times by oracle/Makefile from this one source: tts_cpu over the
// reference's own llm.cpp and decoder.cpp, tts_gpu over the GPU drop-in LlmModel
// (dsh-moss-tts_amd/host/llm_hip.cpp), tts_gpu_codec over both GPU drop-ins
// (LlmModel and AudioDecoder).  Test infrastructure: tests/test_gpu_capi.py runs them
// and compares their PCM.
//
// usage: tts_{cpu,gpu,gpu_codec} LLM DECODER TOKENIZER WORKDIR TEXT SEED GREEDY MAX_FRAMES
// writes WORKDIR/speak{1,2}.pcm (interleaved int16) and prints one JSON line per call.
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "moss/profile.h"  // only to write the synthetic voice profile file
#include "moss/tts.h"

// Fused-launch recoveries of every GPU model of the process (libmoss_hip.so); absent
// from the CPU build, which then reports -1.
extern "C" int moss_hip_fallbacks_total(void) __attribute__((weak));

namespace {

struct Sink {
    std::vector<int16_t> pcm;
    int calls = 0, rate = 0;
};

void on_pcm(void *user, const int16_t *pcm, int frames, int sample_rate) {
    Sink *s = static_cast<Sink *>(user);
    s->pcm.insert(s->pcm.end(), pcm, pcm + static_cast<size_t>(frames) * 2);
    s->rate = sample_rate;
    ++s->calls;
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

bool write_file(const std::string &path, const void *data, size_t bytes) {
    std::FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    const bool ok = bytes == 0 || std::fwrite(data, 1, bytes, f) == bytes;
    std::fclose(f);
    return ok;
}

}  // namespace

int main(int argc, char **argv) {
    if (argc != 9) {
        std::fprintf(stderr, "usage: %s LLM DECODER TOKENIZER WORKDIR TEXT SEED GREEDY MAX_FRAMES\n", argv[0]);
        return 2;
    }
    const std::string workdir = argv[4], text = argv[5];
    const char *a16_before = std::getenv("MOSS_A16");
    const std::string a16_in = a16_before ? a16_before : "(unset)";
    const std::string cache = workdir + "/cache";
    const auto t0 = std::chrono::steady_clock::now();
    moss_engine *e = moss_create(argv[1], argv[2], nullptr, argv[3], nullptr, cache.c_str(), 4, 4);
    if (!e) {
        std::fprintf(stderr, "moss_create failed\n");
        return 1;
    }
    const double create_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    const char *a16_after = std::getenv("MOSS_A16");
    std::string err;
    const std::string voice = workdir + "/synthvoice.mossclone";
    if (!moss::profile_save(voice, synthetic_voice(24, 5), &err)) {
        std::fprintf(stderr, "voice file: %s\n", err.c_str());
        return 1;
    }
    if (moss_set_voice(e, voice.c_str()) != 0) {
        std::fprintf(stderr, "moss_set_voice: %s\n", moss_last_error(e));
        return 1;
    }
    const int tokens = moss_text_tokens(e, text.c_str());
    if (moss_set_sampling(e, 0.8f, 25, 0.95f, 1.2f) != 0) return 1;
    std::printf("{\"version\": \"%s\", \"a16_env_before\": \"%s\", \"a16_env_after\": \"%s\", \"text_tokens\": %d, "
                "\"create_ms\": %.1f}\n",
                moss_version(), a16_in.c_str(), a16_after ? a16_after : "(unset)", tokens, create_ms);
    for (int call = 1; call <= 2; ++call) {
        Sink sink;
        const auto t1 = std::chrono::steady_clock::now();
        const int rc = moss_speak(e, text.c_str(), on_pcm, &sink, std::strtoull(argv[6], nullptr, 10),
                                  std::atoi(argv[7]), std::atoi(argv[8]), 4);
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t1).count();
        if (rc != 0) {
            std::fprintf(stderr, "moss_speak: %s\n", moss_last_error(e));
            return 1;
        }
        if (!write_file(workdir + "/speak" + std::to_string(call) + ".pcm", sink.pcm.data(),
                        sink.pcm.size() * sizeof(int16_t)))
            return 1;
        std::printf("{\"speak\": %d, \"callbacks\": %d, \"sample_rate\": %d, \"samples\": %zu, \"ms\": %.1f, "
                    "\"fallbacks\": %d}\n",
                    call, sink.calls, sink.rate, sink.pcm.size() / 2, ms,
                    moss_hip_fallbacks_total ? moss_hip_fallbacks_total() : -1);
        std::fflush(stdout);
    }
    moss_destroy(e);
    return 0;
}
