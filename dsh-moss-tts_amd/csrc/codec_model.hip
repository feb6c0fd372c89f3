// codec_model.hip -- host driver of the GPU audio codec decoder (see codec.h).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <vector>

#include "codec.h"
#include "llm_model.h"

namespace mh {
namespace {

constexpr int kStageIds[kCodecStages] = {1, 3, 5, 7};       // decoder.cpp:42
constexpr int kPatches[kCodecStages] = {4, 2, 2, 2};        // decoder.cpp:43
constexpr int kLayerCounts[kCodecStages] = {4, 2, 2, 4};    // decoder.cpp:44
constexpr int kContexts[kCodecStages] = {500, 800, 1200, 1600};  // decoder.cpp:21
constexpr int kDtF16 = 0, kDtF32 = 3;  // DType (csrc/include/moss/common.h:26)
constexpr int kMaxPieceFrames = 1024;

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// rows a piece of `frames` frames has at stage s: frames * 4, * 8, * 16, * 32
int stage_rows(int frames, int s) {
    int r = frames;
    for (int i = 0; i <= s; ++i) r *= kPatches[i];
    return r;
}

}  // namespace

Codec::Codec(const void *blob, size_t bytes, const moss_hip_codec_options &opt) {
    device_ = opt.device;
    fmax_ = opt.max_chunk_frames > 0 ? opt.max_chunk_frames : 32;
    if (fmax_ > kMaxPieceFrames) throw Status(MOSS_HIP_EINVAL, "max_chunk_frames > 1024");
    eager_ = opt.eager != 0;
    const uint8_t *b = static_cast<const uint8_t *>(blob);
    auto idx = parse_moss_index(b, bytes);

    // Resolve every tensor AudioDecoder::load asks for (decoder.cpp:28-68) before touching the GPU.
    struct Place {
        uint64_t src, n;
        size_t dst;
    };
    std::vector<Place> places;
    size_t arena = 0;
    auto place = [&](const MossEntry &e, uint64_t n) {
        places.push_back({e.off, n, arena});
        const size_t at = arena;
        arena += align256(n);
        return at;
    };
    auto vec = [&](const std::string &name, uint32_t n) -> size_t {
        auto it = idx.find(name);
        if (it == idx.end() || !is_vector(it->second)) throw Status(MOSS_HIP_EFORMAT, "missing vector: " + name);
        const MossEntry &e = it->second;
        if (e.dims[0] * e.dims[1] != n || e.dtype != kDtF32 || e.nbytes < (uint64_t)n * 4)
            throw Status(MOSS_HIP_EFORMAT, "bad vector: " + name);
        return place(e, (uint64_t)n * 4);
    };
    // a matrix of rows x cols (either may be -1 = taken from the file); fp16 or fp32
    auto mat = [&](const std::string &name, int rows, int cols, int *rows_out, int *cols_out, int *f32) -> size_t {
        auto it = idx.find(name);
        if (it == idx.end() || is_vector(it->second)) throw Status(MOSS_HIP_EFORMAT, "missing matrix: " + name);
        const MossEntry &e = it->second;
        if (e.dtype != kDtF16 && e.dtype != kDtF32)
            throw Status(MOSS_HIP_EUNSUPPORTED, "matrix " + name + " has dtype " + std::to_string(e.dtype) +
                                                    "; only F16 (0) and F32 (3) are supported");
        const int r = (int)e.dims[0], c = (int)e.dims[1];
        if ((rows >= 0 && r != rows) || (cols >= 0 && c != cols)) throw Status(MOSS_HIP_EFORMAT, "bad matrix shape: " + name);
        const uint64_t n = (uint64_t)r * c * (e.dtype == kDtF32 ? 4 : 2);
        if (e.nbytes < n) throw Status(MOSS_HIP_EFORMAT, "matrix truncated: " + name);
        if (rows_out) *rows_out = r;
        if (cols_out) *cols_out = c;
        if (f32) *f32 = e.dtype == kDtF32;
        return place(e, n);
    };

    // quantizer front (decoder.cpp:31-38, 224-245): fp32 codebooks and projections
    size_t o_cb[kCodecNq], o_cw[kCodecNq], o_cbias[kCodecNq];
    for (int i = 0; i < kCodecNq; ++i) {
        const std::string p = "q" + std::to_string(i);
        int f32 = 0;
        o_cb[i] = mat(p + ".cb", kCodecCb, kCodecCbDim, nullptr, nullptr, &f32);
        if (!f32) throw Status(MOSS_HIP_EUNSUPPORTED, p + ".cb must be F32");
        o_cw[i] = mat(p + ".out.w", kCodecZ, kCodecCbDim, nullptr, nullptr, &f32);
        if (!f32) throw Status(MOSS_HIP_EUNSUPPORTED, p + ".out.w must be F32");
        o_cbias[i] = vec(p + ".out.b", kCodecZ);
    }
    int c0 = 0;
    const size_t o_qw = mat("q.out.w", -1, kCodecZ, &c0, nullptr, &qout_f32_);
    const size_t o_qb = vec("q.out.b", (uint32_t)c0);
    if (c0 % 16) throw Status(MOSS_HIP_EUNSUPPORTED, "q.out.w rows must be a multiple of 16");

    struct LayerOff {
        size_t attn, proj, f1, f2, n1w, n1b, n2w, n2b, ls1, ls2;
    };
    std::vector<LayerOff> loff;
    size_t o_in[kCodecStages], o_out[kCodecStages];
    int cin = c0;
    for (int s = 0; s < kCodecStages; ++s) {
        const std::string p = "d" + std::to_string(kStageIds[s]) + ".";
        StageW &S = stages_[s];
        S.patch = kPatches[s];
        if (cin % S.patch) throw Status(MOSS_HIP_EFORMAT, "stage input width does not divide by the patch");
        S.cin = cin / S.patch;
        if (S.cin % 32) throw Status(MOSS_HIP_EUNSUPPORTED, p + "in.w: columns must be a multiple of 32");
        o_in[s] = mat(p + "in.w", kCodecDModel, S.cin, nullptr, nullptr, &S.in_f32);
        o_out[s] = mat(p + "out.w", -1, kCodecDModel, &S.cout, nullptr, &S.out_f32);
        if (S.cout % 16) throw Status(MOSS_HIP_EUNSUPPORTED, p + "out.w: rows must be a multiple of 16");
        S.window = opt.contexts[s] > 0 ? opt.contexts[s] : kContexts[s];
        S.layer0 = (int)layers_.size();
        S.nlayers = kLayerCounts[s];
        S.ring = S.window + stage_rows(fmax_, s);
        for (int n = 0; n < S.nlayers; ++n) {
            const std::string lp = p + "l" + std::to_string(n) + ".";
            LayerW L{};
            LayerOff lo{};
            lo.attn = mat(lp + "attn.w", 3 * kCodecDModel, kCodecDModel, nullptr, nullptr, &L.attn_f32);
            lo.proj = mat(lp + "proj.w", kCodecDModel, kCodecDModel, nullptr, nullptr, &L.proj_f32);
            lo.f1 = mat(lp + "f1.w", -1, kCodecDModel, &L.ffn, nullptr, &L.f1_f32);
            if (L.ffn % 32) throw Status(MOSS_HIP_EUNSUPPORTED, lp + "f1.w: rows must be a multiple of 32");
            lo.f2 = mat(lp + "f2.w", kCodecDModel, L.ffn, nullptr, nullptr, &L.f2_f32);
            lo.n1w = vec(lp + "n1.w", kCodecDModel);
            lo.n1b = vec(lp + "n1.b", kCodecDModel);
            lo.n2w = vec(lp + "n2.w", kCodecDModel);
            lo.n2b = vec(lp + "n2.b", kCodecDModel);
            lo.ls1 = vec(lp + "ls1", kCodecDModel);
            lo.ls2 = vec(lp + "ls2", kCodecDModel);
            ffn_max_ = std::max(ffn_max_, L.ffn);
            layers_.push_back(L);
            loff.push_back(lo);
        }
        cin = S.cout;
    }
    // decode_chunk's final patch_forward(x, 240) (decoder.cpp:218-220) keeps one value per row
    if (cin != kCodecFinalPatch) throw Status(MOSS_HIP_EUNSUPPORTED, "the last stage must have 240 output channels");
    spf_ = stage_rows(1, kCodecStages - 1) * kCodecFinalPatch;

    hip_check(hipSetDevice(device_), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    {
        std::vector<uint8_t> host(arena, 0);
        for (const Place &p : places) std::memcpy(host.data() + p.dst, b + p.src, p.n);
        hip_check(hipMalloc(&wdev_, arena), "hipMalloc(codec weights)");
        hip_check(hipMemcpy(wdev_, host.data(), arena, hipMemcpyHostToDevice), "upload codec weights");
    }
    auto fptr = [&](size_t o) { return reinterpret_cast<const float *>(wdev_ + o); };
    for (int i = 0; i < kCodecNq; ++i) {
        front_cb_[i] = fptr(o_cb[i]);
        front_w_[i] = fptr(o_cw[i]);
        front_b_[i] = fptr(o_cbias[i]);
    }
    qout_w_ = wdev_ + o_qw;
    qout_b_ = fptr(o_qb);
    for (int s = 0; s < kCodecStages; ++s) {
        stages_[s].in = wdev_ + o_in[s];
        stages_[s].out = wdev_ + o_out[s];
    }
    for (size_t i = 0; i < layers_.size(); ++i) {
        LayerW &L = layers_[i];
        const LayerOff &lo = loff[i];
        L.attn = wdev_ + lo.attn;
        L.proj = wdev_ + lo.proj;
        L.f1 = wdev_ + lo.f1;
        L.f2 = wdev_ + lo.f2;
        L.n1w = fptr(lo.n1w);
        L.n1b = fptr(lo.n1b);
        L.n2w = fptr(lo.n2w);
        L.n2b = fptr(lo.n2b);
        L.ls1 = fptr(lo.ls1);
        L.ls2 = fptr(lo.ls2);
    }

    // RoPE frequencies exactly as audio_rope forms them (audio_layer.cpp:34-35), in fp32
    float freq[kCodecHeadDim / 2];
    for (int i = 0; i < kCodecHeadDim / 2; ++i)
        freq[i] = std::exp(-std::log(10000.0f) * 2.0f * static_cast<float>(i) / kCodecHeadDim);
    hip_check(hipMalloc(&freq_, sizeof(freq)), "hipMalloc(freq)");
    hip_check(hipMemcpy(freq_, freq, sizeof(freq), hipMemcpyHostToDevice), "upload freq");

    // activations, sized for pieces of fmax_ frames
    size_t xmax = (size_t)fmax_ * c0;  // q.out output = stage 0 input
    for (int s = 0; s + 1 < kCodecStages; ++s) xmax = std::max(xmax, (size_t)stage_rows(fmax_, s) * stages_[s].cout);
    const size_t rmax = (size_t)stage_rows(fmax_, kCodecStages - 1);
    size_t part_rows = 0;
    for (int f = 1; f <= fmax_; ++f)
        for (int s = 0; s < kCodecStages; ++s) {
            const int r = stage_rows(f, s);
            max_splits_ = std::max(max_splits_, splits_for(s, r));
            part_rows = std::max(part_rows, (size_t)splits_for(s, r) * r);
        }
    auto fmalloc = [&](float **p, size_t n) { hip_check(hipMalloc(p, std::max<size_t>(n, 64) * 4), "hipMalloc(codec act)"); };
    hip_check(hipMalloc(&codes_dev_, sizeof(int32_t) * kCodecNq * fmax_), "hipMalloc(codes)");
    fmalloc(&z_, (size_t)fmax_ * kCodecZ);
    fmalloc(&xa_, xmax);
    fmalloc(&xb_, xmax);
    fmalloc(&y_, rmax * kCodecDModel);
    fmalloc(&qb_, rmax * kCodecDModel);
    fmalloc(&h_, rmax * ffn_max_);
    fmalloc(&ao_, part_rows * kCodecDModel);
    hip_check(hipMalloc(&ast_, sizeof(float2) * part_rows * kCodecHeads), "hipMalloc(attn stats)");
    fmalloc(&out_dev_, (size_t)fmax_ * spf_);
    hip_check(hipHostMalloc(&codes_host_, sizeof(int32_t) * kCodecNq * fmax_), "hipHostMalloc(codes)");
    out_host_cap_ = (size_t)fmax_ * spf_;
    hip_check(hipHostMalloc(&out_host_, sizeof(float) * out_host_cap_), "hipHostMalloc(samples)");
    for (auto &e : ev_) hip_check(hipEventCreate(&e), "hipEventCreate");
    alloc_state(stream_state_);
    clear_state(stream_state_);
    hip_check(hipStreamSynchronize(stream_), "codec init");

    char buf[160];
    std::snprintf(buf, sizeof(buf), "gpu decoder device=%d bytes=%zu ffn=%d windows=%d/%d/%d/%d pieces<=%d frames",
                  device_, arena, ffn_max_, stages_[0].window, stages_[1].window, stages_[2].window, stages_[3].window,
                  fmax_);
    info_ = buf;
}

Codec::~Codec() {
    (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (auto &kv : graphs_) (void)hipGraphExecDestroy(kv.second);
    free_state(stream_state_);
    if (whole_alloc_) free_state(whole_state_);
    for (auto &e : ev_)
        if (e) (void)hipEventDestroy(e);
    void *dev[] = {wdev_, freq_, codes_dev_, z_, xa_, xb_, y_, qb_, h_, ao_, ast_, out_dev_};
    for (void *p : dev)
        if (p) (void)hipFree(p);
    if (codes_host_) (void)hipHostFree(codes_host_);
    if (out_host_) (void)hipHostFree(out_host_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

// Key splits of a stage's attention for a piece of `rows` rows: enough workgroups to
// cover the chip (~512 = row tiles x 4 heads x splits), each split keeping >= 8 key
// blocks of 16 (two per wave) of the steady-state window.  (More splits, ~2048
// workgroups, measured no faster and cost the proj GEMM's merge more.)
int Codec::splits_for(int stage, int rows) const {
    const int tiles = (rows + 15) / 16;
    const int blocks = (stages_[stage].window + 15 + 15) / 16;
    const int want = (512 + tiles * kCodecHeads - 1) / (tiles * kCodecHeads);
    return std::max(1, std::min(want, blocks / 8));
}

void Codec::alloc_state(CodecState &st) {
    hip_check(hipMalloc(&st.pos0, sizeof(int) * kCodecStages), "hipMalloc(codec pos)");
    for (int s = 0; s < kCodecStages; ++s)
        for (int n = 0; n < stages_[s].nlayers; ++n) {
            float *k = nullptr, *v = nullptr;
            const size_t nb = sizeof(float) * stages_[s].ring * kCodecDModel;
            hip_check(hipMalloc(&k, nb), "hipMalloc(codec ring)");
            hip_check(hipMalloc(&v, nb), "hipMalloc(codec ring)");
            // zero once: a ring slot is only read after this stream wrote it, but keep it finite
            hip_check(hipMemsetAsync(k, 0, nb, stream_), "clear ring");
            hip_check(hipMemsetAsync(v, 0, nb, stream_), "clear ring");
            st.k.push_back(k);
            st.v.push_back(v);
        }
}

void Codec::free_state(CodecState &st) {
    if (st.pos0) (void)hipFree(st.pos0);
    for (float *p : st.k) (void)hipFree(p);
    for (float *p : st.v) (void)hipFree(p);
    st.pos0 = nullptr;
    st.k.clear();
    st.v.clear();
}

void Codec::clear_state(CodecState &st) {
    hip_check(hipMemsetAsync(st.pos0, 0, sizeof(int) * kCodecStages, stream_), "reset positions");
}

void Codec::reset_stream() {
    hip_check(hipSetDevice(device_), "hipSetDevice");
    clear_state(stream_state_);
    hip_check(hipStreamSynchronize(stream_), "reset_stream");
}

void Codec::check_codes(const int32_t *codes, int frames) const {
    if (frames <= 0 || !codes) throw Status(MOSS_HIP_EINVAL, "frames must be > 0 and codes non-null");
    for (size_t i = 0; i < (size_t)kCodecNq * frames; ++i)
        if (codes[i] < 0 || codes[i] >= kCodecCb) throw Status(MOSS_HIP_EINVAL, "code out of [0, 1024)");
}

static void ok(int rc, const char *what) {
    if (rc != 0) throw Status(rc, std::string("codec launch failed: ") + what);
}

// The launches of one piece: front, q.out (+ patch 4), four stages, position advance.
void Codec::enqueue(CodecState &st, int frames, hipEvent_t *stage_ev) {
    hipStream_t s = stream_;
    CodecFrontArgs fa;
    fa.codes = codes_dev_;
    fa.frames = frames;
    for (int i = 0; i < kCodecNq; ++i) {
        fa.cb[i] = front_cb_[i];
        fa.cw[i] = front_w_[i];
        fa.cbias[i] = front_b_[i];
    }
    fa.z = z_;
    ok(codec_front_launch(fa, s), "front");
    float *xin = xa_, *xother = xb_;
    {
        CodecGemmArgs g;
        g.a = z_;
        g.lda = kCodecZ;
        g.w = qout_w_;
        g.w_f32 = qout_f32_;
        g.M = frames;
        g.N = stages_[0].cin * stages_[0].patch;
        g.K = kCodecZ;
        g.bias = qout_b_;
        g.y = xin;
        g.patch = stages_[0].patch;
        g.ldy = stages_[0].cin;
        ok(codec_gemm_launch(CPRO_ROWS, CEPI_STORE, g, s), "q.out");
    }
    int rows[kCodecStages];
    for (int si = 0; si < kCodecStages; ++si) {
        const StageW &S = stages_[si];
        const int M = stage_rows(frames, si);
        rows[si] = M;
        const int splits = splits_for(si, M);
        {
            CodecGemmArgs g;
            g.a = xin;
            g.lda = S.cin;
            g.w = S.in;
            g.w_f32 = S.in_f32;
            g.M = M;
            g.N = kCodecDModel;
            g.K = S.cin;
            g.y = y_;
            g.ldy = kCodecDModel;
            ok(codec_gemm_launch(CPRO_ROWS, CEPI_STORE, g, s), "stage in");
        }
        for (int n = 0; n < S.nlayers; ++n) {
            const int li = S.layer0 + n;
            const LayerW &L = layers_[li];
            CodecGemmArgs q;
            q.a = y_;
            q.lda = kCodecDModel;
            q.ln_w = L.n1w;
            q.ln_b = L.n1b;
            q.w = L.attn;
            q.w_f32 = L.attn_f32;
            q.M = M;
            q.N = 3 * kCodecDModel;
            q.K = kCodecDModel;
            q.q = qb_;
            q.kc = st.k[li];
            q.vc = st.v[li];
            q.ring = S.ring;
            q.pos0 = st.pos0 + si;
            q.freq = freq_;
            ok(codec_gemm_launch(CPRO_LN, CEPI_QKV, q, s), "qkv");
            CodecAttnArgs a;
            a.q = qb_;
            a.kc = st.k[li];
            a.vc = st.v[li];
            a.ring = S.ring;
            a.window = S.window;
            a.M = M;
            a.splits = splits;
            a.pos0 = st.pos0 + si;
            a.o = ao_;
            a.st = ast_;
            ok(codec_attn_launch(a, s), "attention");
            CodecGemmArgs p;
            p.o = ao_;
            p.st = ast_;
            p.splits = splits;
            p.w = L.proj;
            p.w_f32 = L.proj_f32;
            p.M = M;
            p.N = kCodecDModel;
            p.K = kCodecDModel;
            p.y = y_;
            p.ldy = kCodecDModel;
            p.ls = L.ls1;
            ok(codec_gemm_launch(CPRO_MERGE, CEPI_RESID, p, s), "proj");
            CodecGemmArgs f;
            f.a = y_;
            f.lda = kCodecDModel;
            f.ln_w = L.n2w;
            f.ln_b = L.n2b;
            f.w = L.f1;
            f.w_f32 = L.f1_f32;
            f.M = M;
            f.N = L.ffn;
            f.K = kCodecDModel;
            f.y = h_;
            f.ldy = L.ffn;
            ok(codec_gemm_launch(CPRO_LN, CEPI_GELU, f, s), "f1");
            CodecGemmArgs f2;
            f2.a = h_;
            f2.lda = L.ffn;
            f2.w = L.f2;
            f2.w_f32 = L.f2_f32;
            f2.M = M;
            f2.N = kCodecDModel;
            f2.K = L.ffn;
            f2.y = y_;
            f2.ldy = kCodecDModel;
            f2.ls = L.ls2;
            ok(codec_gemm_launch(CPRO_ROWS, CEPI_RESID, f2, s), "f2");
        }
        {
            CodecGemmArgs g;
            g.a = y_;
            g.lda = kCodecDModel;
            g.w = S.out;
            g.w_f32 = S.out_f32;
            g.M = M;
            g.N = S.cout;
            g.K = kCodecDModel;
            if (si + 1 < kCodecStages) {
                g.y = xother;
                g.patch = stages_[si + 1].patch;
                g.ldy = stages_[si + 1].cin;
            } else {  // patch 240: the samples, row-major
                g.y = out_dev_;
                g.patch = kCodecFinalPatch;
                g.ldy = 1;
            }
            ok(codec_gemm_launch(CPRO_ROWS, CEPI_STORE, g, s), "stage out");
        }
        std::swap(xin, xother);
        if (stage_ev) hip_check(hipEventRecord(stage_ev[si + 1], s), "hipEventRecord");
    }
    ok(codec_advance_launch(st.pos0, rows, s), "advance");
}

void Codec::run_piece(CodecState &st, const int32_t *codes, int frames, float *out, bool graph) {
    hipStream_t s = stream_;
    hip_check(hipMemcpyAsync(codes_dev_, codes, sizeof(int32_t) * kCodecNq * frames, hipMemcpyHostToDevice, s),
              "upload codes");
    if (graph) {
        auto it = graphs_.find(frames);
        if (it == graphs_.end()) {
            hipGraph_t g = nullptr;
            hipGraphExec_t ge = nullptr;
            hip_check(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal), "begin capture");
            try {
                enqueue(st, frames, nullptr);
            } catch (...) {
                (void)hipStreamEndCapture(s, &g);
                if (g) (void)hipGraphDestroy(g);
                throw;
            }
            hip_check(hipStreamEndCapture(s, &g), "end capture");
            const hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
            (void)hipGraphDestroy(g);
            hip_check(e, "hipGraphInstantiate");
            it = graphs_.emplace(frames, ge).first;
        }
        hip_check(hipGraphLaunch(it->second, s), "hipGraphLaunch");
    } else {
        enqueue(st, frames, nullptr);
    }
    const size_t n = (size_t)frames * spf_;
    hip_check(hipMemcpyAsync(out_host_, out_dev_, n * sizeof(float), hipMemcpyDeviceToHost, s), "download samples");
    hip_check(hipStreamSynchronize(s), "codec piece");
    std::memcpy(out, out_host_, n * sizeof(float));
}

// codes [16][frames] -> the piece [f0, f0 + n) gathered into the pinned staging buffer
static void gather_codes(const int32_t *codes, int frames, int f0, int n, int32_t *dst) {
    for (int i = 0; i < kCodecNq; ++i) std::memcpy(dst + (size_t)i * n, codes + (size_t)i * frames + f0, sizeof(int32_t) * n);
}

void Codec::decode_chunk(const int32_t *codes, int frames, float *out) {
    check_codes(codes, frames);
    hip_check(hipSetDevice(device_), "hipSetDevice");
    for (int f0 = 0; f0 < frames; f0 += fmax_) {
        const int n = std::min(fmax_, frames - f0);
        gather_codes(codes, frames, f0, n, codes_host_);
        run_piece(stream_state_, codes_host_, n, out + (size_t)f0 * spf_, !eager_);
    }
}

void Codec::decode(const int32_t *codes, int frames, float *out) {
    check_codes(codes, frames);
    const auto t0 = std::chrono::steady_clock::now();
    hip_check(hipSetDevice(device_), "hipSetDevice");
    if (!whole_alloc_) {
        alloc_state(whole_state_);
        whole_alloc_ = true;
    }
    clear_state(whole_state_);
    double stage[kCodecStages] = {0, 0, 0, 0};
    for (int f0 = 0; f0 < frames; f0 += fmax_) {
        const int n = std::min(fmax_, frames - f0);
        gather_codes(codes, frames, f0, n, codes_host_);
        hip_check(hipMemcpyAsync(codes_dev_, codes_host_, sizeof(int32_t) * kCodecNq * n, hipMemcpyHostToDevice, stream_),
                  "upload codes");
        hip_check(hipEventRecord(ev_[0], stream_), "hipEventRecord");
        enqueue(whole_state_, n, ev_);
        const size_t ns = (size_t)n * spf_;
        hip_check(hipMemcpyAsync(out_host_, out_dev_, ns * sizeof(float), hipMemcpyDeviceToHost, stream_),
                  "download samples");
        hip_check(hipStreamSynchronize(stream_), "codec decode");
        std::memcpy(out + (size_t)f0 * spf_, out_host_, ns * sizeof(float));
        for (int s = 0; s < kCodecStages; ++s) {
            float ms = 0.f;
            hip_check(hipEventElapsedTime(&ms, ev_[s], ev_[s + 1]), "hipEventElapsedTime");
            stage[s] += ms;
        }
    }
    for (int s = 0; s < kCodecStages; ++s) stage_ms_[s] = stage[s];
    last_ms_ = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace mh
