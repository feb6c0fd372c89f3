// moss/decoder.h -- GPU-backed moss::AudioDecoder (drop-in for the reference's header).
//
// Same public surface as the reference's csrc/include/moss/decoder.h:14-36 (class name,
// constructor, load / decode / reset_stream / decode_chunk, last_ms / stage_ms / info),
// implemented over the codec calls of libmoss_hip.so (include/moss_hip.h,
// moss_hip_codec_*) instead of the CPU layers.  It lives in its own include root
// (dsh-moss-tts_amd/host/codec) so that a build can take the GPU codec, the GPU LLM
// (dsh-moss-tts_amd/host/moss/llm.h) or both.  Differences, documented on the members:
// `threads` is accepted and unused; device failures throw std::runtime_error.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

struct moss_hip_codec;

namespace moss {

class AudioDecoder {
public:
    // threads: kept for source compatibility; the device is MOSS_HIP_DEVICE (default 0)
    explicit AudioDecoder(int threads = 1);
    ~AudioDecoder();
    AudioDecoder(const AudioDecoder &) = delete;
    AudioDecoder &operator=(const AudioDecoder &) = delete;

    // decoder.cpp:28-70: false + *err on a missing / malformed file or tensor
    bool load(const std::string &path, std::string *err);

    // codes: [nq][frames] (quantizer-major); interleaved stereo samples (L, R, L, R, ...)
    std::vector<float> decode(const int32_t *codes, int frames);

    // ---- streaming ----
    void reset_stream();
    // the next chunk of `frames` frames of the stream; chunks must come in order
    std::vector<float> decode_chunk(const int32_t *codes, int frames);

    double last_ms() const { return last_ms_; }
    const std::vector<double> &stage_ms() const { return stage_ms_; }
    const std::string &info() const { return info_; }

private:
    moss_hip_codec *h_ = nullptr;
    int spf_ = 0;
    double last_ms_ = 0.0;
    std::vector<double> stage_ms_;
    std::string info_;
};

}  // namespace moss
