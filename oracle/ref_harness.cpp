// ref_harness.cpp -- extern "C" wrapper around the reference CPU path.
//
// TEST INFRASTRUCTURE ONLY (checker and CPU baseline).  Compiled by
// oracle/Makefile together with the reference's own LLM-path and audio-decoder
// sources, which
// stay where they are under the reference checkout; the result lands in
// oracle/_ref/libmossref.so.  Nothing in the product links it.
//
// Each wrapper names the reference entry point it forwards to.
#include <chrono>
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "moss/attn.h"
#include "moss/decoder.h"
#include "moss/fp16.h"
#include "moss/gemv.h"
#include "moss/llm.h"
#include "moss/parallel.h"
#include "moss/quant.h"
#include "moss/sampler.h"

using namespace moss;

namespace {
thread_local std::string g_err;

struct RefPool {
    Parallel par;
    GemvPoolScratch pool;
    explicit RefPool(int t, int k) : par(t) { pool.bind(par, k); }
};

Matrix q8x4(const void *data, int rows, int cols) {
    Matrix m;
    m.data = data;
    m.rows = rows;
    m.cols = cols;
    m.dtype = DType::Q8_0_4X4;
    m.scales = nullptr;
    return m;
}

SampleParams to_params(const int32_t *ip, const float *fp) {
    // ip = {greedy, top_k, end_greedy, min_frames, greedy_frames}; fp = {temperature, top_p, rep}
    SampleParams p;
    p.greedy = ip[0] != 0;
    p.top_k = ip[1];
    p.end_greedy = ip[2] != 0;
    p.min_frames = ip[3];
    p.greedy_frames = ip[4];
    p.temperature = fp[0];
    p.top_p = fp[1];
    p.repetition_penalty = fp[2];
    return p;
}

std::vector<Row> to_rows(const int32_t *rows, int n) {
    std::vector<Row> v(static_cast<size_t>(n));
    for (int i = 0; i < n; ++i) std::memcpy(v[i].data(), rows + static_cast<size_t>(i) * 17, sizeof(int32_t) * 17);
    return v;
}
}  // namespace

extern "C" {

const char *ref_last_error() { return g_err.c_str(); }

// MOSS_A16 is read once per process (gemv.cpp:26-35): call before any GEMV.
void ref_set_a16_mode(const char *mode) { setenv("MOSS_A16", mode, 1); }
int ref_act16_enabled() { return act16_enabled() ? 1 : 0; }
void ref_act16_suspend(int on) { act16_suspend(on != 0); }  // gemv.cpp:41

float ref_half_to_float(uint16_t h) { return half_to_float(h); }       // fp16.cpp:7
uint16_t ref_float_to_half(float f) { return float_to_half(f); }       // fp16.cpp:37

// quant.cpp:28 (quantize_row_q8_0_scaled)
void ref_quantize_row(const float *x, int k, int8_t *q, uint16_t *dh, float *d) {
    std::vector<BlockQ8_0> blocks(static_cast<size_t>(k / 32));
    quantize_row_q8_0_scaled(x, blocks.data(), d, k);
    for (int b = 0; b < k / 32; ++b) {
        dh[b] = blocks[b].d;
        std::memcpy(q + b * 32, blocks[b].qs, 32);
    }
}

// quant.cpp:56
void ref_dequant_row_q8x4(const uint8_t *group, int nb, int k, float *out) { dequantize_row_q8_0_4x4(group, nb, k, out); }

// gemv_avx2.cpp:123 / gemv.cpp:51
float ref_row_dot_a16(const uint8_t *group, int nb, int k, const float *act) {
    return row_dot_q8_4x4_actf32(group, nb, k, act);
}
float ref_row_dot_a16_scalar(const uint8_t *group, int nb, int k, const float *act) {
    return row_dot_q8_4x4_actf32_scalar(group, nb, k, act);
}

// gemv_avx2.cpp:105 after quant.cpp:45
float ref_row_dot_w8a8(const uint8_t *group, int nb, int k, const float *x) {
    QuantizedActivation act;
    quantize_activation(x, act, nb * 32);
    return row_dot_q8_4x4(group, nb, k, act);
}

void *ref_pool_create(int threads, int k) { return new RefPool(threads, k); }
void ref_pool_destroy(void *p) { delete static_cast<RefPool *>(p); }

// gemv.cpp:245 (gemv_par over a Q8_0_4X4 Matrix)
void ref_gemv_par(void *p, const void *w, int rows, int cols, const float *x, float *y) {
    gemv_par(q8x4(w, rows, cols), x, y, static_cast<RefPool *>(p)->pool);
}

// gemv_par timed: `reps` calls after `reps / 10` warm-up calls; returns the
// median call time in microseconds (the CPU side of the single-GEMV benchmark)
double ref_gemv_par_median_us(void *p, const void *w, int rows, int cols, const float *x, float *y, int reps) {
    const Matrix m = q8x4(w, rows, cols);
    GemvPoolScratch &pool = static_cast<RefPool *>(p)->pool;
    for (int i = 0; i < reps / 10 + 1; ++i) gemv_par(m, x, y, pool);
    std::vector<double> t(reps > 0 ? reps : 1);
    for (auto &ti : t) {
        const auto t0 = std::chrono::steady_clock::now();
        gemv_par(m, x, y, pool);
        ti = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    }
    std::nth_element(t.begin(), t.begin() + t.size() / 2, t.end());
    return t[t.size() / 2];
}

// gemv.cpp:276 (gemm_par over a Q8_0_4X4 Matrix)
void ref_gemm_par(void *p, const void *w, int rows, int cols, const float *x, int m, float *y) {
    gemm_par(q8x4(w, rows, cols), x, m, y, static_cast<RefPool *>(p)->pool);
}

// attn_avx2.cpp:93 / attn_scalar.cpp
void ref_attention_window(const float *qkv, int t, int q0, int q1, int dim, int heads, const float *cache_k,
                          const float *cache_v, int cache_n, int window, float *out, float *scores, int avx2) {
    if (avx2)
        attention_window_avx2(qkv, t, q0, q1, dim, heads, cache_k, cache_v, cache_n, window, out, scores);
    else
        attention_window_scalar(qkv, t, q0, q1, dim, heads, cache_k, cache_v, cache_n, window, out, scores);
}

// sampler.h:25-49
void ref_rng_stream(uint64_t seed, int n, uint32_t *out) {
    Rng r;
    r.seed(seed);
    for (int i = 0; i < n; ++i) out[i] = r.next();
}

// sampler.cpp:9 with an Rng seeded by `seed` and advanced `skip` draws first
int ref_sample_token(const float *logits, int n, const int32_t *ip, const float *fp, const int *prev, int n_prev,
                     uint64_t seed, int skip) {
    Rng r;
    r.seed(seed);
    for (int i = 0; i < skip; ++i) r.next();
    std::vector<float> scratch;
    return sample_token(logits, n, to_params(ip, fp), prev, n_prev, r, scratch);
}

// ---- LlmModel (llm.h:39-90) ----
void *ref_model_create(int threads) { return new LlmModel(threads); }
void ref_model_destroy(void *m) { delete static_cast<LlmModel *>(m); }

int ref_model_load(void *m, const char *path) {  // llm.cpp:59
    try {
        std::string err;
        if (!static_cast<LlmModel *>(m)->load(path, &err)) {
            g_err = err;
            return 1;
        }
    } catch (const std::exception &e) {
        g_err = e.what();
        return 2;
    }
    return 0;
}

void ref_model_reset(void *m) { static_cast<LlmModel *>(m)->reset(); }
int ref_model_position(void *m) { return static_cast<LlmModel *>(m)->position(); }
void ref_model_hidden(void *m, float *out) {
    std::memcpy(out, static_cast<LlmModel *>(m)->hidden(), sizeof(float) * kHidden);
}

// llm.cpp:327
void ref_model_prefill(void *m, const int32_t *rows, int n, int start) {
    static_cast<LlmModel *>(m)->prefill(to_rows(rows, n), start);
}

// llm.cpp:588 / :560
int ref_model_load_state(void *m, const char *path, const int32_t *rows, int n, int ignore_fp) {
    std::string err;
    if (!static_cast<LlmModel *>(m)->load_state(path, to_rows(rows, n), ignore_fp != 0, &err)) {
        g_err = err;
        return 1;
    }
    return 0;
}
int ref_model_save_state(void *m, const char *path, const int32_t *rows, int n) {
    std::string err;
    if (!static_cast<LlmModel *>(m)->save_state(path, to_rows(rows, n), &err)) {
        g_err = err;
        return 1;
    }
    return 0;
}
int ref_model_save_prefix(void *m, const char *path, const int32_t *rows, int n) {
    std::string err;
    if (!static_cast<LlmModel *>(m)->save_prefix(path, to_rows(rows, n), &err)) {
        g_err = err;
        return 1;
    }
    return 0;
}
int ref_model_load_prefix(void *m, const char *path, const int32_t *rows, int n) {
    std::string err;
    if (!static_cast<LlmModel *>(m)->load_prefix(path, to_rows(rows, n), &err)) {
        g_err = err;
        return 1;
    }
    return 0;
}
void ref_model_snapshot_prefix(void *m) { static_cast<LlmModel *>(m)->snapshot_prefix(); }
void ref_model_restore_prefix(void *m) { static_cast<LlmModel *>(m)->restore_prefix(); }

void ref_model_set_logits_dump(void *m, const char *path) { static_cast<LlmModel *>(m)->set_logits_dump(path); }
void ref_model_set_gate_dump(void *m, const char *path) { static_cast<LlmModel *>(m)->set_gate_dump(path); }

// llm.cpp:634.  out_rows [max_frames][17]; timing [max_frames][2] (global_ms, local_ms) or NULL.
int ref_model_generate(void *m, int max_frames, const int32_t *ip, const float *fp, uint64_t seed,
                       const int32_t *forced, int n_forced, int32_t *out_rows, double *timing) {
    std::vector<Row> forced_rows;
    if (forced) forced_rows = to_rows(forced, n_forced);
    std::vector<FrameTiming> t;
    const std::vector<Row> out = static_cast<LlmModel *>(m)->generate(
        max_frames, to_params(ip, fp), seed, timing ? &t : nullptr, forced ? &forced_rows : nullptr);
    for (size_t i = 0; i < out.size(); ++i) std::memcpy(out_rows + i * 17, out[i].data(), sizeof(int32_t) * 17);
    if (timing) {
        for (size_t i = 0; i < t.size(); ++i) {
            timing[2 * i] = t[i].global_ms;
            timing[2 * i + 1] = t[i].local_ms;
        }
    }
    return static_cast<int>(out.size());
}

// ---- audio codec decoder (decoder.h:15-36) ----
void *ref_dec_create(int threads) { return new AudioDecoder(threads); }
void ref_dec_destroy(void *d) { delete static_cast<AudioDecoder *>(d); }
int ref_dec_load(void *d, const char *path) {  // decoder.cpp:26
    std::string err;
    if (!static_cast<AudioDecoder *>(d)->load(path, &err)) {
        g_err = err;
        return 1;
    }
    return 0;
}
// decoder.cpp:247 (whole utterance).  codes [16][frames]; returns the sample
// count written to out (at most cap), -1 when cap is too small.
int ref_dec_decode(void *d, const int32_t *codes, int frames, float *out, int cap, double *ms) {
    auto *dec = static_cast<AudioDecoder *>(d);
    const std::vector<float> y = dec->decode(codes, frames);
    if (ms) *ms = dec->last_ms();
    if (static_cast<int>(y.size()) > cap) return -1;
    std::memcpy(out, y.data(), sizeof(float) * y.size());
    return static_cast<int>(y.size());
}
void ref_dec_reset_stream(void *d) { static_cast<AudioDecoder *>(d)->reset_stream(); }  // decoder.cpp:100
// decoder.cpp:203 (one streaming chunk, in order after reset_stream)
int ref_dec_decode_chunk(void *d, const int32_t *codes, int frames, float *out, int cap) {
    const std::vector<float> y = static_cast<AudioDecoder *>(d)->decode_chunk(codes, frames);
    if (static_cast<int>(y.size()) > cap) return -1;
    std::memcpy(out, y.data(), sizeof(float) * y.size());
    return static_cast<int>(y.size());
}

}  // extern "C"
