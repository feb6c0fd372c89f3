// capi.hip -- extern "C" entry points of libmoss_hip.so (declared in include/moss_hip.h).
// No exception crosses this boundary: failures become status codes plus a
// thread-local message (moss_hip_last_error).
#include <cstdio>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "batch_model.h"
#include "codec.h"

using mh::Status;

struct moss_hip_llm {
    mh::Model *impl;
};

struct moss_hip_batch {
    mh::Batch *impl;
};

struct moss_hip_codec {
    mh::Codec *impl;
};

namespace {

thread_local std::string g_err;

// Sliced-attention scratch of moss_hip_attn_decode (the generation header and
// the LL-word partials, chunk_scratch_bytes), one block per (device, stream),
// allocated and zeroed on the first sliced call on a stream and grown with the
// head count; kept until the process ends.  Launches on one stream are ordered,
// so they never share the block at once; the kernel's launch generation keeps
// consecutive launches' words apart.  A call that would allocate is refused
// while its stream is being captured into a graph.  A captured launch keeps the
// block of its capture stream: its replays must not overlap other calls on that
// stream.
struct AttnScratch {
    uint8_t *base = nullptr;
    int heads = 0;
};
std::mutex g_scratch_mu;
std::map<std::pair<int, hipStream_t>, AttnScratch> g_scratch;

uint8_t *attn_scratch(hipStream_t s, int heads) {
    int dev = 0;
    mh::hip_check(hipGetDevice(&dev), "hipGetDevice");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    AttnScratch &e = g_scratch[{dev, s}];
    if (e.heads < heads) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        mh::hip_check(hipStreamIsCapturing(s, &cs), "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            throw Status(MOSS_HIP_ESTATE, "moss_hip_attn_decode: the first call on a stream with this head count "
                                          "allocates its scratch and cannot be captured; make one uncaptured call "
                                          "on the stream first");
        if (e.base) {
            mh::hip_check(hipStreamSynchronize(s), "sync");  // launches still using the old block
            (void)hipFree(e.base);
            e = AttnScratch{};
        }
        const size_t bytes = mh::chunk_scratch_bytes(heads);
        mh::hip_check(hipMalloc(&e.base, bytes), "hipMalloc(attention scratch)");
        mh::hip_check(hipMemsetAsync(e.base, 0, bytes, s), "memset(attention scratch)");
        mh::hip_check(hipStreamSynchronize(s), "sync");
        e.heads = heads;
    }
    return e.base;
}

// Scratch of moss_hip_attn_decode_noalloc: the sliced attention's generation
// header and partials for up to kNoAllocHeads heads, in the code object's own
// device memory (each device that loads the library holds a copy until the
// process ends).  Host code uses the address hipGetSymbolAddress returns for the
// current device, never the array's name.  The generation header starts at zero
// (static storage) and the kernel's last workgroup resets the arrival count, so
// no call needs to clear it; the partials need no clearing (their tags are
// never current for a later launch).
constexpr int kNoAllocHeads = 16;
constexpr size_t kNoAllocBytes = mh::chunk_scratch_bytes(kNoAllocHeads);
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
uint8_t *g_noalloc_ptr[kMaxDevices] = {};  // per device: the address of its `scratch`

uint8_t *noalloc_scratch() {
    int dev = 0;
    mh::hip_check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) throw Status(MOSS_HIP_EUNSUPPORTED, "device ordinal beyond 63");
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (g_noalloc_ptr[dev] == nullptr) {
        void *p = nullptr;
        mh::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        g_noalloc_ptr[dev] = static_cast<uint8_t *>(p);
    }
    return g_noalloc_ptr[dev];
}

template <class F>
int guard(F &&f) {
    try {
        f();
        return MOSS_HIP_OK;
    } catch (const Status &s) {
        g_err = s.what();
        return s.code;
    } catch (const std::bad_alloc &) {
        g_err = "host out of memory";
        return MOSS_HIP_EDEVICE;
    } catch (const std::exception &e) {
        g_err = e.what();
        return MOSS_HIP_EDEVICE;
    }
}

mh::Model &model_of(moss_hip_llm *m) {
    if (m == nullptr || m->impl == nullptr) throw Status(MOSS_HIP_EINVAL, "null model handle");
    mh::hip_check(hipSetDevice(m->impl->device()), "hipSetDevice");
    return *m->impl;
}

mh::Batch &batch_of(moss_hip_batch *b) {
    if (b == nullptr || b->impl == nullptr) throw Status(MOSS_HIP_EINVAL, "null batch handle");
    mh::hip_check(hipSetDevice(b->impl->device()), "hipSetDevice");
    return *b->impl;
}

mh::Codec &codec_of(moss_hip_codec *c) {
    if (c == nullptr || c->impl == nullptr) throw Status(MOSS_HIP_EINVAL, "null codec handle");
    return *c->impl;
}

std::vector<uint8_t> read_file(const char *path) {
    if (path == nullptr) throw Status(MOSS_HIP_EINVAL, "null path");
    std::FILE *f = std::fopen(path, "rb");
    if (!f) throw Status(MOSS_HIP_EINVAL, std::string("cannot open weights file: ") + path);
    std::fseek(f, 0, SEEK_END);
    const long size = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    std::vector<uint8_t> data(size > 0 ? (size_t)size : 0);
    const size_t got = data.empty() ? 0 : std::fread(data.data(), 1, data.size(), f);
    std::fclose(f);
    if (size <= 16 || got != data.size()) throw Status(MOSS_HIP_EFORMAT, std::string("short weights file: ") + path);
    return data;
}

moss_hip_llm_options defaults(const moss_hip_llm_options *opt) {
    moss_hip_llm_options o{0, 0, 0, 1, 0, 0, 0};
    if (opt) o = *opt;
    return o;
}

}  // namespace

extern "C" {

const char *moss_hip_last_error(void) { return g_err.c_str(); }
int moss_hip_abi_version(void) { return MOSS_HIP_ABI_VERSION; }

int moss_hip_llm_create(const void *blob, size_t bytes, const moss_hip_llm_options *opt, moss_hip_llm **out) {
    return guard([&] {
        if (out == nullptr || blob == nullptr) throw Status(MOSS_HIP_EINVAL, "null argument");
        *out = nullptr;
        auto *h = new moss_hip_llm{nullptr};
        try {
            h->impl = new mh::Model(blob, bytes, defaults(opt));
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int moss_hip_llm_create_from_file(const char *path, const moss_hip_llm_options *opt, moss_hip_llm **out) {
    return guard([&] {
        if (path == nullptr || out == nullptr) throw Status(MOSS_HIP_EINVAL, "null argument");
        const std::vector<uint8_t> data = read_file(path);
        const int rc = moss_hip_llm_create(data.data(), data.size(), opt, out);
        if (rc != MOSS_HIP_OK) throw Status(rc, g_err);
    });
}

void moss_hip_llm_destroy(moss_hip_llm *m) {
    if (!m) return;
    delete m->impl;
    delete m;
}

int moss_hip_llm_reset(moss_hip_llm *m) {
    return guard([&] { model_of(m).reset(); });
}

int moss_hip_llm_position(const moss_hip_llm *m) { return (m && m->impl) ? m->impl->position() : -1; }
int moss_hip_llm_fallbacks(const moss_hip_llm *m) { return (m && m->impl) ? m->impl->fallbacks() : -1; }

int moss_hip_fallbacks_total(void) { return mh::fallbacks_total.load(std::memory_order_relaxed); }

int moss_hip_llm_get_hidden(moss_hip_llm *m, float *out) {
    return guard([&] {
        if (!out) throw Status(MOSS_HIP_EINVAL, "null output");
        model_of(m).get_hidden(out);
    });
}

int moss_hip_llm_set_hidden(moss_hip_llm *m, const float *in) {
    return guard([&] {
        if (!in) throw Status(MOSS_HIP_EINVAL, "null input");
        model_of(m).set_hidden(in);
    });
}

int moss_hip_llm_prefill(moss_hip_llm *m, const int32_t *rows, int n_rows, int start) {
    return guard([&] {
        if (n_rows < 0 || (n_rows > 0 && !rows)) throw Status(MOSS_HIP_EINVAL, "bad rows");
        model_of(m).prefill(rows, n_rows, start);
    });
}

int moss_hip_llm_global_step(moss_hip_llm *m, const int32_t *row17) {
    return guard([&] {
        if (!row17) throw Status(MOSS_HIP_EINVAL, "null row");
        model_of(m).global_step(row17);
    });
}

int moss_hip_llm_generate(moss_hip_llm *m, int max_frames, const moss_hip_sample_params *p, uint64_t seed,
                          const int32_t *forced, int n_forced, int32_t *out_rows, int *out_frames, double *timing,
                          float *logits_dump, float *gate_dump, moss_hip_frame_cb cb, void *user) {
    return guard([&] {
        if (!p || !out_rows || max_frames < 0) throw Status(MOSS_HIP_EINVAL, "bad arguments");
        const int n = model_of(m).generate(max_frames, *p, seed, forced, n_forced, out_rows, timing, logits_dump,
                                           gate_dump, cb, user);
        if (out_frames) *out_frames = n;
    });
}

int moss_hip_llm_set_cancel_flag(moss_hip_llm *m, const volatile uint8_t *flag) {
    return guard([&] { model_of(m).set_cancel_flag(flag); });
}

int moss_hip_llm_snapshot_prefix(moss_hip_llm *m) {
    return guard([&] { model_of(m).snapshot_prefix(); });
}

int moss_hip_llm_restore_prefix(moss_hip_llm *m) {
    return guard([&] { model_of(m).restore_prefix(); });
}

int moss_hip_llm_prefix_pos(const moss_hip_llm *m) { return (m && m->impl) ? m->impl->prefix_pos() : -1; }

int moss_hip_llm_gate_rows(const moss_hip_llm *m) { return (m && m->impl) ? m->impl->gate_rows() : -1; }

int moss_hip_llm_capture(moss_hip_llm *m, int on) {
    return guard([&] { model_of(m).set_capture(on != 0); });
}

int moss_hip_llm_capture_read(moss_hip_llm *m, int what, void *out, size_t bytes, size_t *needed) {
    return guard([&] {
        if (what < MOSS_HIP_CAP_GLOBAL || what > MOSS_HIP_CAP_PREFILL) throw Status(MOSS_HIP_EINVAL, "bad capture kind");
        const size_t n = model_of(m).capture_read(what, out, bytes);
        if (needed) *needed = n;
        if (n == 0) throw Status(MOSS_HIP_ESTATE, "nothing of that kind was captured");
        if (out && bytes < n) throw Status(MOSS_HIP_EINVAL, "output buffer too small");
    });
}

int moss_hip_llm_kv_export(moss_hip_llm *m, int n_pos, float *k, float *v) {
    return guard([&] {
        if (n_pos > 0 && (!k || !v)) throw Status(MOSS_HIP_EINVAL, "null buffer");
        model_of(m).kv_export(n_pos, k, v);
    });
}

int moss_hip_llm_kv_import(moss_hip_llm *m, int n_pos, const float *k, const float *v, const float *hidden) {
    return guard([&] {
        if (n_pos > 0 && (!k || !v)) throw Status(MOSS_HIP_EINVAL, "null buffer");
        model_of(m).kv_import(n_pos, k, v, hidden);
    });
}

// ------------------------------------------------------------------ batched streams

int moss_hip_batch_create(moss_hip_llm *model, int max_streams, int capacity, int kv_dtype, moss_hip_batch **out) {
    return guard([&] {
        if (out == nullptr) throw Status(MOSS_HIP_EINVAL, "null output");
        *out = nullptr;
        mh::Model &m = model_of(model);
        if (kv_dtype != 0 && kv_dtype != 1) throw Status(MOSS_HIP_EINVAL, "kv_dtype must be 0 (fp16) or 1 (fp32)");
        auto *h = new moss_hip_batch{nullptr};
        try {
            h->impl = new mh::Batch(m, max_streams, capacity, kv_dtype == 1 ? mh::KV_F32 : mh::KV_F16);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

void moss_hip_batch_destroy(moss_hip_batch *b) {
    if (!b) return;
    delete b->impl;
    delete b;
}

int moss_hip_batch_set_stream(moss_hip_batch *b, int stream, int n_pos, const float *k, const float *v,
                              const float *hidden) {
    return guard([&] {
        if (n_pos > 0 && (!k || !v)) throw Status(MOSS_HIP_EINVAL, "null buffer");
        batch_of(b).set_stream(stream, n_pos, k, v, hidden);
    });
}

int moss_hip_batch_capture(moss_hip_batch *b, int on) {
    return guard([&] { batch_of(b).set_capture(on != 0); });
}

int moss_hip_batch_capture_read(moss_hip_batch *b, void *out, size_t bytes, size_t *needed) {
    return guard([&] {
        const size_t n = batch_of(b).capture_read(out, bytes);
        if (needed) *needed = n;
        if (n == 0) throw Status(MOSS_HIP_ESTATE, "no capture taken");
        if (out && bytes < n) throw Status(MOSS_HIP_EINVAL, "output buffer too small");
    });
}

int moss_hip_batch_admit(moss_hip_batch *b, int stream, moss_hip_llm *model) {
    return guard([&] { batch_of(b).admit(stream, model_of(model)); });
}

int moss_hip_batch_get_hidden(moss_hip_batch *b, int stream, float *out) {
    return guard([&] {
        if (!out) throw Status(MOSS_HIP_EINVAL, "null output");
        batch_of(b).get_hidden(stream, out);
    });
}

int moss_hip_batch_position(const moss_hip_batch *b, int stream) {
    if (!b || !b->impl || stream < 0 || stream >= b->impl->max_streams()) return -1;
    return b->impl->position(stream);
}

int moss_hip_batch_kv_export(moss_hip_batch *b, int stream, int n_pos, float *k, float *v) {
    return guard([&] {
        if (n_pos > 0 && (!k || !v)) throw Status(MOSS_HIP_EINVAL, "null buffer");
        batch_of(b).kv_export(stream, n_pos, k, v);
    });
}

int moss_hip_batch_global_step(moss_hip_batch *b, int n_streams, const int32_t *rows) {
    return guard([&] {
        if (!rows) throw Status(MOSS_HIP_EINVAL, "null rows");
        batch_of(b).global_step(n_streams, rows);
    });
}

int moss_hip_batch_generate(moss_hip_batch *b, int n_streams, int frames, const moss_hip_sample_params *p,
                            const uint64_t *seeds, int32_t *out_rows, int *out_frames, double *elapsed_ms) {
    return guard([&] {
        if (!p || !out_rows || frames < 0) throw Status(MOSS_HIP_EINVAL, "bad arguments");
        const double ms = batch_of(b).generate(n_streams, frames, *p, seeds, out_rows, out_frames);
        if (elapsed_ms) *elapsed_ms = ms;
    });
}

// ------------------------------------------------------------------ operators

int moss_hip_gemm_q8x4(const void *w, int rows, int cols, const float *x, int m, float *y, void *stream) {
    return guard([&] {
        if (!w || !x || !y) throw Status(MOSS_HIP_EINVAL, "null pointer");
        if (rows <= 0 || rows % 16 || cols <= 0 || cols % 32 || m <= 0)
            throw Status(MOSS_HIP_EINVAL, "shape must satisfy rows % 16 == 0, cols % 32 == 0, m > 0");
        mh::GemmArgs g;
        g.w = static_cast<const uint8_t *>(w);
        g.N = rows;
        g.K = cols;
        g.a = x;
        g.lda = cols;
        g.M = m;
        g.y = y;
        g.ldy = rows;
        mh::hip_check(mh::launch_gemm(g, mh::EPI_F32, mh::KV_F16, static_cast<hipStream_t>(stream)), "gemm launch");
    });
}


int moss_hip_quantize_rows(const float *x, int m, int cols, int8_t *q, float *d, void *stream) {
    return guard([&] {
        if (!x || !q || !d) throw Status(MOSS_HIP_EINVAL, "null pointer");
        if (m <= 0 || cols <= 0 || cols % 256) throw Status(MOSS_HIP_EINVAL, "shape must satisfy m > 0, cols % 256 == 0");
        mh::hip_check(mh::launch_quant_rows(x, cols, cols, m, q, d, static_cast<hipStream_t>(stream)), "quantize launch");
    });
}

int moss_hip_gemm_q8x4_w8a8(const void *w, int rows, int cols, const int8_t *q, const float *d, int m, float *y,
                            void *stream) {
    return guard([&] {
        if (!w || !q || !d || !y) throw Status(MOSS_HIP_EINVAL, "null pointer");
        if (rows <= 0 || rows % 16 || cols <= 0 || cols % 32 || m <= 0)
            throw Status(MOSS_HIP_EINVAL, "shape must satisfy rows % 16 == 0, cols % 32 == 0, m > 0");
        mh::GemmArgs g;
        g.w = static_cast<const uint8_t *>(w);
        g.N = rows;
        g.K = cols;
        g.a8 = q;
        g.d8 = d;
        g.lda = cols;
        g.M = m;
        g.y = y;
        g.ldy = rows;
        mh::hip_check(mh::launch_gemm(g, mh::EPI_F32, mh::KV_F16, static_cast<hipStream_t>(stream)), "gemm launch");
    });
}

int moss_hip_gemv_q8x4(const void *w, int rows, int cols, const void *x, int x_dtype, void *y, int y_dtype,
                       void *stream) {
    return guard([&] {
        if (!w || !x || !y) throw Status(MOSS_HIP_EINVAL, "null pointer");
        if (rows <= 0 || rows % 4 || cols <= 0 || cols % 128 || cols > 4096)
            throw Status(MOSS_HIP_EINVAL, "shape must satisfy rows % 4 == 0, cols % 128 == 0, cols <= 4096");
        if ((x_dtype != MOSS_HIP_F32 && x_dtype != MOSS_HIP_F16) || (y_dtype != MOSS_HIP_F32 && y_dtype != MOSS_HIP_F16))
            throw Status(MOSS_HIP_EINVAL, "dtype must be MOSS_HIP_F32 or MOSS_HIP_F16");
        mh::GemvArgs a;
        a.w = static_cast<const uint8_t *>(w);
        a.rows = rows;
        a.cols = cols;
        a.x = x;
        a.y = y;
        const auto pro = x_dtype == MOSS_HIP_F16 ? mh::PRO_F16 : mh::PRO_F32;
        const auto epi = y_dtype == MOSS_HIP_F16 ? mh::EPI_F16 : mh::EPI_F32;
        mh::hip_check(mh::launch_gemv(a, pro, epi, mh::KV_F16, static_cast<hipStream_t>(stream)), "gemv launch");
    });
}

int moss_hip_gemv_q8x4_w8a8(const void *w, int rows, int cols, const float *x, float *y, void *stream) {
    return guard([&] {
        if (!w || !x || !y) throw Status(MOSS_HIP_EINVAL, "null pointer");
        if (rows <= 0 || rows % 4 || cols <= 0 || cols % 256 || cols > 4096)
            throw Status(MOSS_HIP_EINVAL, "shape must satisfy rows % 4 == 0, cols % 256 == 0, cols <= 4096");
        mh::GemvArgs a;
        a.w = static_cast<const uint8_t *>(w);
        a.rows = rows;
        a.cols = cols;
        a.x = x;
        a.y = y;
        a.a8 = 1;
        mh::hip_check(mh::launch_gemv(a, mh::PRO_F32, mh::EPI_F32, mh::KV_F16, static_cast<hipStream_t>(stream)),
                      "gemv launch");
    });
}

int moss_hip_dequant_rows_q8x4(const void *w, int mat_rows, int cols, const int32_t *rows_dev, int n, float *out,
                               void *stream) {
    return guard([&] {
        if (!w || !rows_dev || !out || n < 0) throw Status(MOSS_HIP_EINVAL, "bad arguments");
        if (cols <= 0 || cols % 32 || mat_rows <= 0 || mat_rows % 4) throw Status(MOSS_HIP_EINVAL, "bad matrix shape");
        mh::hip_check(mh::launch_dequant_rows(static_cast<const uint8_t *>(w), mat_rows, cols, rows_dev, n, out,
                                              static_cast<hipStream_t>(stream)),
                      "dequant launch");
    });
}

}  // extern "C"

namespace {

// The arguments of both single-query attention entry points; `scratch_of` gives the
// sliced launch's scratch block for `heads` heads.
template <class Scratch>
void attn_decode(const float *q, const void *k_cache, const void *v_cache, int kv_dtype, int heads, int ctx_stride,
                 int n_keys, void *out, int out_dtype, void *stream, Scratch &&scratch_of) {
    if (!q || !k_cache || !v_cache || !out) throw Status(MOSS_HIP_EINVAL, "null pointer");
    if (heads <= 0 || ctx_stride <= 0 || n_keys <= 0 || n_keys > ctx_stride)
        throw Status(MOSS_HIP_EINVAL, "need 0 < n_keys <= ctx_stride");
    if ((kv_dtype != MOSS_HIP_F32 && kv_dtype != MOSS_HIP_F16) || (out_dtype != MOSS_HIP_F32 && out_dtype != MOSS_HIP_F16))
        throw Status(MOSS_HIP_EINVAL, "dtype must be MOSS_HIP_F32 or MOSS_HIP_F16");
    mh::AttnArgs a;  // the cache is one page of ctx_stride positions
    a.q = q;
    a.k_pool = k_cache;
    a.v_pool = v_cache;
    a.page_size = ctx_stride;
    a.heads = heads;
    a.q_stride = heads * mh::kHeadDim;
    a.out_stride = heads * mh::kHeadDim;
    a.pos0 = n_keys - 1;
    a.max_keys = n_keys;
    a.out = out;
    a.out_f16 = out_dtype == MOSS_HIP_F16;
    const auto kv = kv_dtype == MOSS_HIP_F32 ? mh::KV_F32 : mh::KV_F16;
    const int spans = (n_keys + 63) / 64;
    // one workgroup per head (a wave per span) up to kOneWgSpans spans; fp32 caches up to 8
    const int one_wg = kv == mh::KV_F16 ? mh::kOneWgSpans : std::min(mh::kOneWgSpans, 8);
    if (spans > one_wg) {  // slices of slice_waves(spans) spans across workgroups
        uint8_t *sc = scratch_of(static_cast<hipStream_t>(stream), heads);
        a.chunk_waves = mh::slice_waves(spans);
        const int chunks = (spans + a.chunk_waves - 1) / a.chunk_waves;
        a.chunks = chunks < mh::kMaxChunks ? chunks : mh::kMaxChunks;
        a.chunk_gen = reinterpret_cast<uint32_t *>(sc);
        a.chunk_part = reinterpret_cast<uint64_t *>(sc + mh::kChunkHeader);
    }
    mh::hip_check(mh::launch_attn(a, kv, static_cast<hipStream_t>(stream)), "attention launch");
}

}  // namespace

extern "C" {

int moss_hip_attn_decode(const float *q, const void *k_cache, const void *v_cache, int kv_dtype, int heads,
                         int ctx_stride, int n_keys, void *out, int out_dtype, void *stream) {
    return guard([&] {
        attn_decode(q, k_cache, v_cache, kv_dtype, heads, ctx_stride, n_keys, out, out_dtype, stream, attn_scratch);
    });
}

int moss_hip_attn_decode_noalloc(const float *q, const void *k_cache, const void *v_cache, int kv_dtype, int heads,
                                 int ctx_stride, int n_keys, void *out, int out_dtype, void *stream) {
    return guard([&] {
        if (heads > kNoAllocHeads)
            throw Status(MOSS_HIP_EINVAL, "moss_hip_attn_decode_noalloc: at most 16 heads (its scratch is sized for 16)");
        attn_decode(q, k_cache, v_cache, kv_dtype, heads, ctx_stride, n_keys, out, out_dtype, stream,
                    [](hipStream_t, int) { return noalloc_scratch(); });
    });
}

int moss_hip_attn_paged(const float *q, const void *k_pool, const void *v_pool, int kv_dtype, int heads,
                        const int32_t *page_table, int table_stride, int page_size, int rows,
                        const int32_t *row_stream, const int32_t *row_pos, int max_keys, void *out, int out_dtype,
                        void *stream) {
    return guard([&] {
        if (!q || !k_pool || !v_pool || !page_table || !row_pos || !out) throw Status(MOSS_HIP_EINVAL, "null pointer");
        if (heads <= 0 || rows <= 0 || max_keys <= 0 || page_size <= 0 || table_stride <= 0 ||
            (long long)table_stride * page_size < max_keys)
            throw Status(MOSS_HIP_EINVAL, "need heads, rows, max_keys, page_size > 0 and table_stride * page_size >= max_keys");
        if (page_size % 64 != 0)  // the kernel reads 64-key spans, each from one page
            throw Status(MOSS_HIP_EINVAL, "page_size must be a multiple of 64");
        if ((kv_dtype != MOSS_HIP_F32 && kv_dtype != MOSS_HIP_F16) || (out_dtype != MOSS_HIP_F32 && out_dtype != MOSS_HIP_F16))
            throw Status(MOSS_HIP_EINVAL, "dtype must be MOSS_HIP_F32 or MOSS_HIP_F16");
        mh::AttnArgs a;
        a.q = q;
        a.q_stride = heads * mh::kHeadDim;
        a.k_pool = k_pool;
        a.v_pool = v_pool;
        a.page_table = page_table;
        a.table_stride = table_stride;
        a.page_size = page_size;
        a.heads = heads;
        a.row_stream = row_stream;
        a.stream_stride = 1;
        a.row_pos = row_pos;
        a.rows = rows;
        a.max_keys = max_keys;
        a.out = out;
        a.out_stride = heads * mh::kHeadDim;
        a.out_f16 = out_dtype == MOSS_HIP_F16;
        const auto kv = kv_dtype == MOSS_HIP_F32 ? mh::KV_F32 : mh::KV_F16;
        mh::hip_check(mh::launch_attn(a, kv, static_cast<hipStream_t>(stream)), "attention launch");
    });
}

int moss_hip_codec_create(const void *blob, size_t bytes, const moss_hip_codec_options *opt, moss_hip_codec **out) {
    return guard([&] {
        if (out == nullptr || blob == nullptr) throw Status(MOSS_HIP_EINVAL, "null argument");
        *out = nullptr;
        moss_hip_codec_options o{};
        if (opt) o = *opt;
        auto *h = new moss_hip_codec{nullptr};
        try {
            h->impl = new mh::Codec(blob, bytes, o);
        } catch (...) {
            delete h;
            throw;
        }
        *out = h;
    });
}

int moss_hip_codec_create_from_file(const char *path, const moss_hip_codec_options *opt, moss_hip_codec **out) {
    return guard([&] {
        if (out == nullptr) throw Status(MOSS_HIP_EINVAL, "null argument");
        const std::vector<uint8_t> data = read_file(path);
        const int rc = moss_hip_codec_create(data.data(), data.size(), opt, out);
        if (rc != MOSS_HIP_OK) throw Status(rc, g_err);
    });
}

void moss_hip_codec_destroy(moss_hip_codec *c) {
    if (!c) return;
    delete c->impl;
    delete c;
}

int moss_hip_codec_samples_per_frame(const moss_hip_codec *c) { return (c && c->impl) ? c->impl->samples_per_frame() : -1; }

int moss_hip_codec_reset_stream(moss_hip_codec *c) {
    return guard([&] { codec_of(c).reset_stream(); });
}

int moss_hip_codec_decode_chunk(moss_hip_codec *c, const int32_t *codes, int frames, float *out) {
    return guard([&] {
        if (!out) throw Status(MOSS_HIP_EINVAL, "null output");
        codec_of(c).decode_chunk(codes, frames, out);
    });
}

int moss_hip_codec_decode(moss_hip_codec *c, const int32_t *codes, int frames, float *out) {
    return guard([&] {
        if (!out) throw Status(MOSS_HIP_EINVAL, "null output");
        codec_of(c).decode(codes, frames, out);
    });
}

double moss_hip_codec_last_ms(const moss_hip_codec *c) { return (c && c->impl) ? c->impl->last_ms() : -1.0; }

int moss_hip_codec_stage_ms(const moss_hip_codec *c, double out4[4]) {
    return guard([&] {
        if (c == nullptr || c->impl == nullptr || out4 == nullptr) throw Status(MOSS_HIP_EINVAL, "null argument");
        for (int i = 0; i < 4; ++i) out4[i] = c->impl->stage_ms()[i];
    });
}

}  // extern "C"
