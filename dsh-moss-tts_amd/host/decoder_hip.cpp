// decoder_hip.cpp -- moss::AudioDecoder (host/codec/moss/decoder.h) over the C ABI of
// libmoss_hip.so.  Mirrors csrc/src/decoder.cpp's public behaviour: load() reports
// failures through *err, decode() sets last_ms and the four stage times, decode_chunk
// continues the stream (reset_stream restarts it; the first call on a fresh decoder
// starts at position 0, as decoder.cpp:212 does).
#include "moss/decoder.h"

#include <cstdlib>
#include <stdexcept>

#include "moss_hip.h"

namespace moss {
namespace {

int device_from_env() {
    const char *d = std::getenv("MOSS_HIP_DEVICE");
    return d ? std::atoi(d) : 0;
}

void check(int rc, const char *what) {
    if (rc != MOSS_HIP_OK) throw std::runtime_error(std::string(what) + ": " + moss_hip_last_error());
}

}  // namespace

AudioDecoder::AudioDecoder(int threads) { (void)threads; }

AudioDecoder::~AudioDecoder() { moss_hip_codec_destroy(h_); }

bool AudioDecoder::load(const std::string &path, std::string *err) {
    moss_hip_codec_destroy(h_);
    h_ = nullptr;
    moss_hip_codec_options o{};
    o.device = device_from_env();
    if (moss_hip_codec_create_from_file(path.c_str(), &o, &h_) != MOSS_HIP_OK) {
        if (err) *err = moss_hip_last_error();
        h_ = nullptr;
        return false;
    }
    spf_ = moss_hip_codec_samples_per_frame(h_);
    info_ = "decoder weights=" + path + " device=" + std::to_string(o.device) + " (gpu)";
    return true;
}

std::vector<float> AudioDecoder::decode(const int32_t *codes, int frames) {
    if (!h_) throw std::runtime_error("AudioDecoder::decode before load");
    std::vector<float> out(static_cast<size_t>(frames > 0 ? frames : 0) * spf_);
    if (frames <= 0) return out;
    check(moss_hip_codec_decode(h_, codes, frames, out.data()), "AudioDecoder::decode");
    last_ms_ = moss_hip_codec_last_ms(h_);
    double st[4];
    check(moss_hip_codec_stage_ms(h_, st), "AudioDecoder::stage_ms");
    stage_ms_.assign(st, st + 4);
    return out;
}

void AudioDecoder::reset_stream() {
    if (!h_) throw std::runtime_error("AudioDecoder::reset_stream before load");
    check(moss_hip_codec_reset_stream(h_), "AudioDecoder::reset_stream");
}

std::vector<float> AudioDecoder::decode_chunk(const int32_t *codes, int frames) {
    if (!h_) throw std::runtime_error("AudioDecoder::decode_chunk before load");
    std::vector<float> out(static_cast<size_t>(frames > 0 ? frames : 0) * spf_);
    if (frames <= 0) return out;
    check(moss_hip_codec_decode_chunk(h_, codes, frames, out.data()), "AudioDecoder::decode_chunk");
    return out;
}

}  // namespace moss
