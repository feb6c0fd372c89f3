// batch_model.hip -- batched multi-stream decode (see batch_model.h).
#include "batch_model.h"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace mh {
namespace {
// at least 4 K slices for fc_out (K = 3072): 6 blocks per wave (64 streams: 49.9k ->
// 50.4k frames/s against 2 slices; 1 slice 47.6k)
constexpr int kBatchFcOutSplit = 4;
// a float buffer holding fp16 hi / lo halves in the matrix-core order (hlt_at)
inline uint8_t *hl(float *p) { return reinterpret_cast<uint8_t *>(p); }
}  // namespace

Batch::Batch(Model &model, int max_streams, int capacity, KvType kv)
    : model_(model), w_(model.weights()), S_(max_streams), cap_(capacity), kvt_(kv) {
    if (S_ <= 0 || S_ > 1024) throw Status(MOSS_HIP_EINVAL, "max_streams must be in [1, 1024]");
    if (cap_ <= kLocalLen || cap_ > 65536) throw Status(MOSS_HIP_EINVAL, "capacity must be in (17, 65536]");
    esize_ = kvt_ == KV_F32 ? 4 : 2;
    pages_ = (cap_ + kPage - 1) / kPage;
    hip_check(hipSetDevice(model.device()), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    for (auto &e : ev_) hip_check(hipEventCreate(&e), "hipEventCreate");

    layer_pool_elems_ = (size_t)S_ * pages_ * kHeads * kPage * kHeadDim;
    const size_t pool_bytes = layer_pool_elems_ * kLayers * esize_;
    hip_check(hipMalloc(&kpool_, pool_bytes), "hipMalloc(k pages)");
    hip_check(hipMalloc(&vpool_, pool_bytes), "hipMalloc(v pages)");
    hip_check(hipMemset(kpool_, 0, pool_bytes), "memset(k pages)");
    hip_check(hipMemset(vpool_, 0, pool_bytes), "memset(v pages)");
    const size_t lkv = (size_t)S_ * kHeads * kLocalLen * kHeadDim;
    hip_check(hipMalloc(&lkv_, 2 * lkv * sizeof(float)), "hipMalloc(local kv)");
    hip_check(hipMemset(lkv_, 0, 2 * lkv * sizeof(float)), "memset(local kv)");

    // Block table: page j of stream s is page j*S + s of the pool, so a stream's
    // pages are spread over the pool and every access goes through the table.
    std::vector<int> table((size_t)S_ * pages_);
    for (int s = 0; s < S_; ++s)
        for (int j = 0; j < pages_; ++j) table[(size_t)s * pages_ + j] = j * S_ + s;
    hip_check(hipMalloc(&table_, table.size() * sizeof(int)), "hipMalloc(table)");
    hip_check(hipMemcpy(table_, table.data(), table.size() * sizeof(int), hipMemcpyHostToDevice), "table h2d");

    // RoPE table for positions [0, cap] (llm.cpp:90-102 formula; a stream parked at
    // capacity still evaluates row `cap`)
    rope_n_ = cap_ + 1;
    std::vector<float> rope(2ull * rope_n_ * kRopeHalf);
    for (int p = 0; p < rope_n_; ++p)
        for (int i = 0; i < kRopeHalf; ++i) {
            const double inv = 1.0 / std::pow(10000.0, static_cast<double>(2 * i) / kHeadDim);
            const double ang = static_cast<double>(p) * inv;
            rope[(size_t)p * kRopeHalf + i] = static_cast<float>(std::cos(ang));
            rope[(size_t)(rope_n_ + p) * kRopeHalf + i] = static_cast<float>(std::sin(ang));
        }
    hip_check(hipMalloc(&rope_, rope.size() * 4), "hipMalloc(rope)");
    hip_check(hipMemcpy(rope_, rope.data(), rope.size() * 4, hipMemcpyHostToDevice), "rope h2d");

    auto fm = [&](float **p, size_t n) {
        hip_check(hipMalloc(p, n * sizeof(float)), "hipMalloc(batch)");
        hip_check(hipMemset(*p, 0, n * sizeof(float)), "memset(batch)");
    };
    // a_, o_ and h_ are read only by GEMMs, as fp16 hi / lo halves in the matrix-core
    // order (hlt_at: 4 bytes a value, rows padded to 16)
    const size_t s16 = (size_t)(S_ + 15) / 16 * 16;
    fm(&x_, (size_t)S_ * kHidden);
    fm(&a_, s16 * kHidden);
    fm(&q_, (size_t)S_ * kHidden);
    fm(&o_, s16 * kHidden);
    fm(&h_, s16 * kFF);
    fm(&hidden_, (size_t)S_ * kHidden);
    fm(&lres_, (size_t)S_ * kHidden);
    fm(&next_in_, (size_t)S_ * kHidden);
    fm(&logits_, (size_t)S_ * kCodebook);
    fm(&gate_, (size_t)S_ * 2);
    auto im = [&](int **p, size_t n) {
        hip_check(hipMalloc(p, n * sizeof(int)), "hipMalloc(batch)");
        hip_check(hipMemset(*p, 0, n * sizeof(int)), "memset(batch)");
    };
    im(&pos_d_, S_);
    im(&order_, S_);
    hip_check(hipHostMalloc(&order_h_, sizeof(int) * S_, hipHostMallocDefault), "hipHostMalloc(order)");
    im(&codes_, (size_t)S_ * kNVq);
    im(&row_, (size_t)S_ * (kNVq + 1));
    im(&counts_, (size_t)S_ * kNVq * kCodebook);
    fm(&part_, (size_t)16 * S_ * kHidden);
    fm(&xhl_, s16 * kHidden);
    fm(&xst_, (size_t)(kHidden / 16) * S_ * 2);
    fm(&pairs_, (size_t)S_ * (kCodebook / 16) * 2);
    a8_ = model.decode_a8();
    if (a8_) {  // zeroed once: the GEMMs read the padding rows and never store them
        hip_check(hipMalloc(&q8a_, s16 * kHidden), "hipMalloc(batch)");
        hip_check(hipMalloc(&q8h_, s16 * kFF), "hipMalloc(batch)");
        hip_check(hipMemset(q8a_, 0, s16 * kHidden), "memset(batch)");
        hip_check(hipMemset(q8h_, 0, s16 * kFF), "memset(batch)");
        fm(&d8a_, s16 * (kHidden / 32));
        fm(&d8h_, s16 * (kFF / 32));
    }
    hip_check(hipMalloc(&ctrl_, sizeof(BatchCtl)), "hipMalloc(ctrl)");
    hip_check(hipMalloc(&rng_, sizeof(uint32_t) * 4 * S_), "hipMalloc(rng)");
    hip_check(hipMemset(rng_, 0, sizeof(uint32_t) * 4 * S_), "memset(rng)");
    im(&hist_codes_, (size_t)(cap_ + 1) * S_ * kNVq);
    hip_check(hipMalloc(&active_, S_), "hipMalloc(active)");
    hip_check(hipMemset(active_, 0, S_), "memset(active)");
    hip_check(hipMalloc(&hist_active_, (size_t)(cap_ + 1) * S_), "hipMalloc(history)");
    hip_check(hipHostMalloc(&ctrl_h_, sizeof(BatchCtl), hipHostMallocDefault), "hipHostMalloc(ctrl)");
    pos_.assign(S_, 0);
}

Batch::~Batch() {
    (void)hipSetDevice(model_.device());
    if (stream_) (void)hipStreamSynchronize(stream_);
    for (auto &kv : graphs_) {
        if (kv.second.local) (void)hipGraphExecDestroy(kv.second.local);
        if (kv.second.local_greedy) (void)hipGraphExecDestroy(kv.second.local_greedy);
        if (kv.second.global) (void)hipGraphExecDestroy(kv.second.global);
    }
    void *bufs[] = {kpool_, vpool_, lkv_, table_, rope_, x_, a_, q_, o_, h_, hidden_, lres_, next_in_, logits_,
                    gate_, pos_d_, codes_, row_, counts_, ctrl_, rng_, hist_codes_, active_, hist_active_, part_,
                    xhl_,  xst_,  pairs_, q8a_, q8h_, d8a_, d8h_, acap_};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    if (ctrl_h_) (void)hipHostFree(ctrl_h_);
    if (order_h_) (void)hipHostFree(order_h_);
    if (order_) (void)hipFree(order_);
    for (auto &e : ev_)
        if (e) (void)hipEventDestroy(e);
    if (stream_) (void)hipStreamDestroy(stream_);
}

StreamState Batch::state() const {
    StreamState st;
    st.pos = pos_d_;
    st.active = active_;
    st.codes = codes_;
    st.row = row_;
    st.gate = gate_;
    st.counts = counts_;
    st.ctrl = ctrl_;
    st.rng = rng_;
    st.capacity = cap_;
    return st;
}

// The paged attention's row order for streams 0..n-1: longest context first (ties by stream),
// measured 24.8 -> 23.3 us per layer for 64 streams at contexts U[64, 1024] (the longest rows
// no longer start last, or two to a CU).  The order only schedules workgroups: every row
// still writes its own output.  Uploaded from pinned memory; every caller synchronises the
// stream before returning, so the staging is free again at the next call.
void Batch::upload_order(int n) {
    for (int s = 0; s < n; ++s) order_h_[s] = s;
    std::stable_sort(order_h_, order_h_ + n, [&](int x, int y) { return pos_[x] > pos_[y]; });
    hip_check(hipMemcpyAsync(order_, order_h_, sizeof(int) * n, hipMemcpyHostToDevice, stream_), "order h2d");
}

void Batch::write_ctrl(int min_frames, float rep, const SampleCfg &cfg) {
    ctrl_h_->frame = 0;
    ctrl_h_->min_frames = min_frames;
    ctrl_h_->rep_penalty = rep;
    ctrl_h_->cfg = cfg;
    hip_check(hipMemcpyAsync(ctrl_, ctrl_h_, sizeof(BatchCtl), hipMemcpyHostToDevice, stream_), "ctrl h2d");
}

void Batch::set_stream(int s, int n_pos, const float *k, const float *v, const float *hidden) {
    if (s < 0 || s >= S_) throw Status(MOSS_HIP_EINVAL, "stream out of range");
    if (n_pos < 0 || n_pos > cap_) throw Status(MOSS_HIP_EINVAL, "n_pos above the batch capacity");
    hip_check(hipSetDevice(model_.device()), "hipSetDevice");
    if (n_pos > 0) {
        float *stage = nullptr;
        const size_t per = (size_t)n_pos * kHidden;
        hip_check(hipMalloc(&stage, per * 4), "hipMalloc(stage)");
        try {
            for (int w = 0; w < 2; ++w)
                for (int l = 0; l < kLayers; ++l) {
                    uint8_t *pool = static_cast<uint8_t *>(w == 0 ? kpool_ : vpool_) + l * layer_pool_elems_ * esize_;
                    hip_check(hipMemcpyAsync(stage, (w == 0 ? k : v) + (size_t)l * per, per * 4, hipMemcpyHostToDevice,
                                             stream_),
                              "kv h2d");
                    hip_check(launch_kv_import_paged(stage, n_pos, pool, table_ + (size_t)s * pages_, kPage, kvt_, stream_),
                              "kv import");
                    hip_check(hipStreamSynchronize(stream_), "sync");
                }
        } catch (...) {
            (void)hipFree(stage);
            throw;
        }
        (void)hipFree(stage);
    }
    if (hidden)
        hip_check(hipMemcpyAsync(hidden_ + (size_t)s * kHidden, hidden, kHidden * 4, hipMemcpyHostToDevice, stream_),
                  "hidden h2d");
    hip_check(hipMemcpyAsync(pos_d_ + s, &n_pos, sizeof(int), hipMemcpyHostToDevice, stream_), "pos h2d");
    hip_check(hipStreamSynchronize(stream_), "sync");
    pos_[s] = n_pos;
}

// Admission of a job prepared on a single-stream model (restore_prefix + prefill, the
// reference's per-job flow, engine.cpp:447-470): its K/V rows go into the stream's pages
// (converted to the batch's precision), its hidden state and position follow, all device to
// device.  The model's last call has returned (calls are serialised), so its state is final
// once its stream is drained.
void Batch::admit(int s, Model &src) {
    if (s < 0 || s >= S_) throw Status(MOSS_HIP_EINVAL, "stream out of range");
    if (src.device() != model_.device()) throw Status(MOSS_HIP_EINVAL, "the model is on another device");
    const Model::StateView v = src.state_view();
    if (v.pos > cap_) throw Status(MOSS_HIP_EINVAL, "the model's position is above the batch capacity");
    hip_check(hipSetDevice(model_.device()), "hipSetDevice");
    hip_check(hipStreamSynchronize(src.stream()), "sync");
    KvAdmit a;
    a.k_src = v.k;
    a.v_src = v.v;
    a.src_layer_elems = v.layer_elems;
    a.ctx_stride = v.ctx_stride;
    a.src_kv = v.kv;
    a.k_pool = kpool_;
    a.v_pool = vpool_;
    a.pool_layer_elems = layer_pool_elems_;
    a.table_row = table_ + (size_t)s * pages_;
    a.page_size = kPage;
    a.pool_kv = kvt_;
    hip_check(launch_kv_admit(a, v.pos, stream_), "kv admit");
    hip_check(hipMemcpyAsync(hidden_ + (size_t)s * kHidden, v.hidden, kHidden * 4, hipMemcpyDeviceToDevice, stream_),
              "hidden d2d");
    hip_check(hipMemcpyAsync(pos_d_ + s, &v.pos, sizeof(int), hipMemcpyHostToDevice, stream_), "pos h2d");
    hip_check(hipStreamSynchronize(stream_), "sync");
    pos_[s] = v.pos;
}

void Batch::get_hidden(int s, float *out) {
    if (s < 0 || s >= S_) throw Status(MOSS_HIP_EINVAL, "stream out of range");
    hip_check(hipMemcpyAsync(out, hidden_ + (size_t)s * kHidden, kHidden * 4, hipMemcpyDeviceToHost, stream_), "d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
}

void Batch::kv_export(int s, int n_pos, float *k, float *v) {
    if (s < 0 || s >= S_ || n_pos < 0 || n_pos > cap_) throw Status(MOSS_HIP_EINVAL, "bad stream / n_pos");
    if (n_pos == 0) return;
    float *stage = nullptr;
    const size_t per = (size_t)n_pos * kHidden;
    hip_check(hipMalloc(&stage, per * 4), "hipMalloc(stage)");
    try {
        for (int w = 0; w < 2; ++w)
            for (int l = 0; l < kLayers; ++l) {
                const uint8_t *pool = static_cast<const uint8_t *>(w == 0 ? kpool_ : vpool_) + l * layer_pool_elems_ * esize_;
                hip_check(launch_kv_export_paged(pool, table_ + (size_t)s * pages_, kPage, n_pos, kvt_, stage, stream_),
                          "kv export");
                hip_check(hipMemcpyAsync((w == 0 ? k : v) + (size_t)l * per, stage, per * 4, hipMemcpyDeviceToHost,
                                         stream_),
                          "kv d2h");
                hip_check(hipStreamSynchronize(stream_), "sync");
            }
    } catch (...) {
        (void)hipFree(stage);
        throw;
    }
    (void)hipFree(stage);
}

// block_forward (llm.cpp:230-246) of the local layer for n streams at local
// position lpos; the residual starts as `in` (row stride in_stride, 0 = one row
// shared by all streams) and ends in lres_, with its local ln_f in a_ (the
// heads' input).  LN1 and LN2 run in the prologue of the GEMM that consumes
// them; proj adds bias and residual in its epilogue (one K slice), fc_out is
// split in K and reduced, in a fixed order, with the residual and ln_f by the
// kernel that follows it.  At lpos >= 1 the block input is an embedding row, so LN1 + QKV
// is a row of the load-time q|k|v table, already written into q_ and the local
// caches by the previous kernel.
void Batch::enqueue_local_step(hipStream_t s, int n, const float *in, int in_stride, int lpos, bool attn) {
    const LayerW &L = *w_.local;
    float *lk = lkv_, *lv = lkv_ + (size_t)S_ * kHeads * kLocalLen * kHeadDim;
    const float *rc = rope_, *rs = rope_ + (size_t)rope_n_ * kRopeHalf;
    if (lpos == 0) {  // `in` is the global hidden state, one row per stream
        GemmArgs q;
        q.w = L.attn_w; q.wm = L.attn_wm; q.N = 3 * kHidden; q.K = kHidden; q.a = in; q.lda = in_stride; q.M = n;
        q.ln_w = L.ln1_w; q.ln_b = L.ln1_b;
        q.bias = L.attn_b; q.q_out = q_; q.k_pool = lk; q.v_pool = lv; q.page_size = kLocalLen;
        q.stream_stride = 1; q.pos0 = lpos; q.pos_stride = 0; q.rope_cos = rc; q.rope_sin = rs;
        if (a8_) {  // LN1 and its int8 copy first, then the int8 GEMM
            hip_check(launch_ln_rows(in, in_stride, L.ln1_w, L.ln1_b, nullptr, n, s, nullptr, q8a_, d8a_),
                      "local ln1");
            q.a = nullptr; q.ln_w = q.ln_b = nullptr; q.lda = kHidden;
            q.a8 = q8a_; q.d8 = d8a_; q.a8_tiled = true;
        }
        hip_check(launch_gemm(q, EPI_QKV, KV_F32, s), "local qkv");
    }
    if (attn) {
        AttnArgs t;
        t.q = q_; t.k_pool = lk; t.v_pool = lv; t.page_size = kLocalLen; t.stream_stride = 1;
        t.pos0 = lpos; t.pos_stride = 0; t.rows = n; t.max_keys = kLocalLen;
        if (a8_) {
            t.out = o_; t.q8 = q8a_; t.d8 = d8a_;
        } else {
            t.out_hl = hl(o_);
        }
        hip_check(launch_attn(t, KV_F32, s), "local attention");
    }
    if (a8_) {
        capture_attention(s, n, kLayers + lpos);
        enqueue_local_step_a8(s, n, in, in_stride);
        return;
    }
    GemmArgs p;
    p.w = L.proj_w; p.wm = L.proj_wm; p.N = kHidden; p.K = kHidden; p.a_hl = hl(o_); p.lda = kHidden; p.M = n;
    p.y = lres_; p.ldy = kHidden; p.bias = L.proj_b; p.resid_in = in; p.resid_stride = in_stride;
    p.y_hl = hl(xhl_); p.y_stats = xst_;  // fc_in's operand and its LN2 statistics
    hip_check(launch_gemm(p, EPI_RESID, KV_F32, s), "local proj");
    GemmArgs f1;
    f1.w = L.fc_in_w; f1.wm = L.fc_in_wm; f1.N = kFF; f1.K = kHidden; f1.a_hl = hl(xhl_); f1.lda = kHidden; f1.M = n;
    f1.ln_w = L.ln2_w; f1.ln_b = L.ln2_b; f1.ln_stats = xst_;
    f1.y_hl = hl(h_); f1.bias = L.fc_in_b;
    hip_check(launch_gemm(f1, EPI_GELU, KV_F32, s), "local fc_in");
    GemmArgs f2;  // x += fc_out + b (lres_: the gate's input at lpos 0), pre-split with its LN
                  // statistics: the audio head applies the local ln_f
    f2.w = L.fc_out_w; f2.wm = L.fc_out_wm; f2.N = kHidden; f2.K = kFF; f2.a_hl = hl(h_); f2.lda = kFF; f2.M = n;
    f2.y = lres_; f2.ldy = kHidden; f2.bias = L.fc_out_b;
    f2.y_hl = hl(a_); f2.y_stats = xst_;
    hip_check(launch_gemm(f2, EPI_RESID, KV_F32, s), "local fc_out");
}

// The W8A8 form of the local step after its attention (q8a_ holds the attention output's int8
// copy): proj as split-K partials, reduced in a fixed order with bias and residual into lres_
// by the kernel that also applies LN2 and quantises it; fc_in with gelu, quantised in its
// epilogue; fc_out as split-K partials, reduced with bias and residual, then the local ln_f
// quantised for the audio head -- the prefill's kernels and operand forms.
void Batch::enqueue_local_step_a8(hipStream_t s, int n, const float *in, int in_stride) {
    const LayerW &L = *w_.local;
    GemmArgs p;
    p.w = L.proj_w; p.wm = L.proj_wm; p.N = kHidden; p.K = kHidden; p.lda = kHidden; p.M = n;
    p.a8 = q8a_; p.d8 = d8a_; p.a8_tiled = true;
    p.part = part_; p.ksplit = gemm_ksplit(n, kHidden, kHidden);
    hip_check(launch_gemm(p, EPI_PART, KV_F32, s), "local proj");
    hip_check(launch_resid_ln_rows(part_, p.ksplit, n, L.proj_b, in, in_stride, lres_, L.ln2_w, L.ln2_b, nullptr,
                                   nullptr, s, q8a_, d8a_),
              "local proj reduce + ln2");
    GemmArgs f1;
    f1.w = L.fc_in_w; f1.wm = L.fc_in_wm; f1.N = kFF; f1.K = kHidden; f1.lda = kHidden; f1.M = n;
    f1.a8 = q8a_; f1.d8 = d8a_; f1.a8_tiled = true;
    f1.bias = L.fc_in_b; f1.q8_out = q8h_; f1.d8_out = d8h_;
    hip_check(launch_gemm(f1, EPI_GELU, KV_F32, s), "local fc_in");
    GemmArgs f2;
    f2.w = L.fc_out_w; f2.wm = L.fc_out_wm; f2.N = kHidden; f2.K = kFF; f2.lda = kFF; f2.M = n;
    f2.a8 = q8h_; f2.d8 = d8h_; f2.a8_tiled = true;
    f2.part = part_; f2.ksplit = std::max(gemm_ksplit(n, kHidden, kFF), kBatchFcOutSplit);
    hip_check(launch_gemm(f2, EPI_PART, KV_F32, s), "local fc_out");
    hip_check(launch_resid_ln_rows(part_, f2.ksplit, n, L.fc_out_b, lres_, kHidden, lres_, w_.llnf_w, w_.llnf_b,
                                   nullptr, nullptr, s, q8a_, d8a_),
              "local fc_out reduce + ln_f");
}

// Attention capture (tests): the fp32 output rows o_ and their int8 copy q8a_ / d8a_ of the
// attention just enqueued go to capture entry `slot` (0..11 global layers, 12..28 local
// positions).  Device-to-device copies, so they are graph nodes like the kernels.
void Batch::capture_attention(hipStream_t s, int n, int slot) {
    if (!capture_ || !a8_) return;
    const size_t s16 = (size_t)(S_ + 15) / 16 * 16;
    uint8_t *e = acap_ + (size_t)slot * acap_entry_;
    hip_check(hipMemcpyAsync(e, o_, sizeof(float) * (size_t)n * kHidden, hipMemcpyDeviceToDevice, s), "capture");
    e += sizeof(float) * (size_t)S_ * kHidden;
    hip_check(hipMemcpyAsync(e, q8a_, s16 * kHidden, hipMemcpyDeviceToDevice, s), "capture");
    e += s16 * kHidden;
    hip_check(hipMemcpyAsync(e, d8a_, sizeof(float) * s16 * (kHidden / 32), hipMemcpyDeviceToDevice, s), "capture");
}

void Batch::set_capture(bool on) {
    if (on == capture_) return;
    if (on && !a8_) throw Status(MOSS_HIP_ESTATE, "attention capture records the W8A8 batch only");
    const size_t s16 = (size_t)(S_ + 15) / 16 * 16;
    acap_entry_ = sizeof(float) * (size_t)S_ * kHidden + s16 * kHidden + sizeof(float) * s16 * (kHidden / 32);
    if (on && !acap_) {
        const size_t bytes = acap_entry_ * (kLayers + kLocalLen);
        hip_check(hipMalloc(&acap_, bytes), "hipMalloc(capture)");
        hip_check(hipMemset(acap_, 0, bytes), "memset(capture)");
    }
    capture_ = on;
    hip_check(hipStreamSynchronize(stream_), "sync");
    for (auto &kv : graphs_) {  // re-captured with (or without) the copies
        if (kv.second.local) (void)hipGraphExecDestroy(kv.second.local);
        if (kv.second.local_greedy) (void)hipGraphExecDestroy(kv.second.local_greedy);
        if (kv.second.global) (void)hipGraphExecDestroy(kv.second.global);
    }
    graphs_.clear();
}

size_t Batch::capture_read(void *out, size_t bytes) {
    if (!acap_) return 0;
    const size_t n = acap_entry_ * (kLayers + kLocalLen);
    if (out == nullptr || bytes < n) return n;
    hip_check(hipMemcpyAsync(out, acap_, n, hipMemcpyDeviceToHost, stream_), "capture d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
    return n;
}

// The local half of a frame for n streams (llm.cpp:648-698).  Greedy frames (the host knows
// which frames are greedy) fuse each channel's pick into the next position's attention:
// 15 launches fewer per frame.
void Batch::enqueue_frame_local(hipStream_t s, int n, bool greedy) {
    const StreamState st = state();
    enqueue_local_step(s, n, hidden_, kHidden, 0);
    hip_check(launch_gate_rows(lres_, w_.llnf_w, w_.llnf_b, w_.wte, st, n, s), "gate");
    // q|k|v of local positions 1..16 come from the load-time table: the row of
    // wte[slot] here, the row of (lpos, picked code) from each channel's sampler
    LocalQkv qkv;
    qkv.q_out = q_;
    qkv.lk = lkv_;
    qkv.lv = lkv_ + (size_t)S_ * kHeads * kLocalLen * kHeadDim;
    qkv.rows = w_.qkv_table;
    qkv.lpos = 1;
    hip_check(launch_local_qkv_rows(qkv, n, s), "local qkv rows");
    for (int ch = 0; ch < kNVq; ++ch) {
        if (ch == 0) {
            enqueue_local_step(s, n, w_.slot_in, 0, 1);
        } else if (greedy) {  // channel ch - 1's pick, lpos ch + 1's q|k|v row and attention, in one launch
            PickAttnArgs pa;
            pa.logits = logits_;
            pa.ch = ch - 1;
            pa.aemb = w_.aemb[ch - 1];
            pa.next_in = next_in_;
            pa.st = st;
            pa.rows = w_.qkv_table + (1 + (size_t)(ch - 1) * kCodebook) * 3 * kHidden;
            pa.lk = qkv.lk;
            pa.lv = qkv.lv;
            pa.lpos = ch + 1;
            if (a8_) {
                pa.o = o_; pa.o_q8 = q8a_; pa.o_d8 = d8a_;
            } else {
                pa.o_hl = hl(o_);
            }
            pa.pairs = pairs_;
            hip_check(launch_local_pick_attn(pa, n, s), "pick + local attention");
            enqueue_local_step(s, n, next_in_, kHidden, ch + 1, false);
        } else {
            enqueue_local_step(s, n, next_in_, kHidden, ch + 1);
        }
        GemmArgs hd;  // the tied audio head on the local ln_f of the step's output
        hd.w = w_.aemb[ch]; hd.wm = w_.aemb_m[ch]; hd.N = kCodebook; hd.K = kHidden; hd.lda = kHidden;
        hd.M = n;
        if (a8_) {  // the local ln_f quantised by the reduce before it
            hd.a8 = q8a_; hd.d8 = d8a_; hd.a8_tiled = true;
        } else {  // the step's output, pre-split by fc_out: the local ln_f applied here
            hd.a_hl = hl(a_);
            hd.ln_w = w_.llnf_w; hd.ln_b = w_.llnf_b; hd.ln_stats = xst_;
        }
        hd.y = logits_; hd.ldy = kCodebook;
        if (greedy && ch + 1 < kNVq) {  // the next launch picks this channel from per-16-code partials
            hd.pick_pairs = pairs_;
            hd.pick_counts = st.counts + (size_t)ch * kCodebook;
            hd.pick_stride = kNVq * kCodebook;
            hd.pick_pen = &st.ctrl->rep_penalty;
        }
        hip_check(launch_gemm(hd, EPI_F32, KV_F32, s), "audio head");
        if (greedy && ch + 1 < kNVq) continue;  // picked by the next position's launch
        LocalQkv next = qkv;  // the input of lpos ch + 2 is channel ch's code
        next.rows = ch + 1 < kNVq ? w_.qkv_table + (1 + (size_t)ch * kCodebook) * 3 * kHidden : nullptr;
        next.lpos = ch + 2;
        hip_check(launch_sample_rows(logits_, ch, w_.aemb[ch], next_in_, st, n, ch == kNVq - 1, next, s,
                                     greedy && ch == kNVq - 1 ? 1 : 0),
                  "sample");
    }
}

// global_step (llm.cpp:248-255) for n streams over the paged cache.
void Batch::enqueue_global(hipStream_t s, int n) {
    const StreamState st = state();
    EmbedArgs e;
    e.wte = w_.wte;
    for (int ch = 0; ch < kNVq; ++ch) e.aemb[ch] = w_.aemb[ch];
    hip_check(launch_embed_rows(e, row_, n, x_, s), "embed");
    hip_check(launch_ln_rows(x_, kHidden, w_.global[0].ln1_w, w_.global[0].ln1_b, nullptr, n, s, nullptr,
                             a8_ ? q8a_ : nullptr, a8_ ? d8a_ : nullptr, a8_ ? nullptr : hl(a_)),
              "ln1");
    if (a8_) {
        enqueue_global_a8(s, n);
        return;
    }
    const float *rc = rope_, *rs = rope_ + (size_t)rope_n_ * kRopeHalf;
    for (int l = 0; l < kLayers; ++l) {
        const LayerW &L = w_.global[l];
        void *kp = static_cast<uint8_t *>(kpool_) + l * layer_pool_elems_ * esize_;
        void *vp = static_cast<uint8_t *>(vpool_) + l * layer_pool_elems_ * esize_;
        GemmArgs q;  // layer 0: on LN1(x) in a_ (hi / lo halves); later layers: on x in a_, LN1 applied
                     // with the statistics the previous fc_out wrote
        q.w = L.attn_w; q.wm = L.attn_wm; q.N = 3 * kHidden; q.K = kHidden; q.a_hl = hl(a_); q.lda = kHidden; q.M = n;
        if (l > 0) {
            q.ln_w = L.ln1_w; q.ln_b = L.ln1_b; q.ln_stats = xst_;
        }
        q.bias = L.attn_b; q.q_out = q_; q.k_pool = kp; q.v_pool = vp;
        q.page_table = table_; q.table_stride = pages_; q.page_size = kPage;
        q.stream_stride = 1; q.row_pos = pos_d_; q.row_active = active_; q.rope_cos = rc; q.rope_sin = rs;
        hip_check(launch_gemm(q, EPI_QKV, kvt_, s), "qkv");
        AttnArgs t;
        t.q = q_; t.k_pool = kp; t.v_pool = vp; t.page_table = table_; t.table_stride = pages_; t.page_size = kPage;
        t.stream_stride = 1; t.row_pos = pos_d_; t.rows = n; t.max_keys = cap_; t.out_hl = hl(o_);
        t.row_order = order_;
        hip_check(launch_attn(t, kvt_, s), "attention");
        GemmArgs p;  // x += proj + b
        p.w = L.proj_w; p.wm = L.proj_wm; p.N = kHidden; p.K = kHidden; p.a_hl = hl(o_); p.lda = kHidden; p.M = n;
        p.y = x_; p.ldy = kHidden; p.bias = L.proj_b;
        p.y_hl = hl(xhl_); p.y_stats = xst_;  // fc_in's operand and its LN2 statistics
        hip_check(launch_gemm(p, EPI_RESID, kvt_, s), "proj");
        GemmArgs f1;  // LN2 of the pre-split rows, statistics from proj
        f1.w = L.fc_in_w; f1.wm = L.fc_in_wm; f1.N = kFF; f1.K = kHidden; f1.a_hl = hl(xhl_); f1.lda = kHidden; f1.M = n;
        f1.ln_w = L.ln2_w; f1.ln_b = L.ln2_b; f1.ln_stats = xst_;
        f1.y_hl = hl(h_); f1.bias = L.fc_in_b;
        hip_check(launch_gemm(f1, EPI_GELU, kvt_, s), "fc_in");
        GemmArgs f2;
        f2.w = L.fc_out_w; f2.wm = L.fc_out_wm; f2.N = kHidden; f2.K = kFF; f2.a_hl = hl(h_); f2.lda = kFF; f2.M = n;
        if (l + 1 < kLayers) {
            // x += fc_out + b in one launch (8 waves split K in the workgroup), written also
            // pre-split with its LN statistics: the next layer's QKV applies LN1
            f2.y = x_; f2.ldy = kHidden; f2.bias = L.fc_out_b;
            f2.y_hl = hl(a_); f2.y_stats = xst_;
            hip_check(launch_gemm(f2, EPI_RESID, kvt_, s), "fc_out");
        } else {
            // split K; the reduce adds bias and residual and writes ln_f into hidden (active
            // streams only)
            f2.part = part_; f2.ksplit = std::max(gemm_ksplit(n, kHidden, kFF), kBatchFcOutSplit);
            hip_check(launch_gemm(f2, EPI_PART, kvt_, s), "fc_out");
            hip_check(launch_resid_ln_rows(part_, f2.ksplit, n, L.fc_out_b, x_, kHidden, x_, w_.lnf_w, w_.lnf_b,
                                           hidden_, active_, s, nullptr, nullptr, nullptr),
                      "fc_out reduce + ln_f");
        }
    }
    hip_check(launch_advance_rows(st, n, s), "advance");
}

// The W8A8 global step after the embedding and LN1 (q8a_ holds LN1's int8 copy): per layer
// the int8 QKV GEMM (bias, RoPE, paged K/V write), paged attention quantising its output, proj
// as split-K partials reduced with bias and residual by the kernel that applies and quantises
// LN2, fc_in with gelu quantised in its epilogue, fc_out as split-K partials reduced with
// bias and residual before the next layer's LN1 (quantised) or ln_f.
void Batch::enqueue_global_a8(hipStream_t s, int n) {
    const StreamState st = state();
    const float *rc = rope_, *rs = rope_ + (size_t)rope_n_ * kRopeHalf;
    for (int l = 0; l < kLayers; ++l) {
        const LayerW &L = w_.global[l];
        void *kp = static_cast<uint8_t *>(kpool_) + l * layer_pool_elems_ * esize_;
        void *vp = static_cast<uint8_t *>(vpool_) + l * layer_pool_elems_ * esize_;
        GemmArgs q;
        q.w = L.attn_w; q.wm = L.attn_wm; q.N = 3 * kHidden; q.K = kHidden; q.lda = kHidden; q.M = n;
        q.a8 = q8a_; q.d8 = d8a_; q.a8_tiled = true;
        q.bias = L.attn_b; q.q_out = q_; q.k_pool = kp; q.v_pool = vp;
        q.page_table = table_; q.table_stride = pages_; q.page_size = kPage;
        q.stream_stride = 1; q.row_pos = pos_d_; q.row_active = active_; q.rope_cos = rc; q.rope_sin = rs;
        hip_check(launch_gemm(q, EPI_QKV, kvt_, s), "qkv");
        AttnArgs t;
        t.q = q_; t.k_pool = kp; t.v_pool = vp; t.page_table = table_; t.table_stride = pages_; t.page_size = kPage;
        t.stream_stride = 1; t.row_pos = pos_d_; t.rows = n; t.max_keys = cap_; t.row_order = order_;
        t.out = o_; t.q8 = q8a_; t.d8 = d8a_;
        hip_check(launch_attn(t, kvt_, s), "attention");
        capture_attention(s, n, l);
        GemmArgs p;
        p.w = L.proj_w; p.wm = L.proj_wm; p.N = kHidden; p.K = kHidden; p.lda = kHidden; p.M = n;
        p.a8 = q8a_; p.d8 = d8a_; p.a8_tiled = true;
        p.part = part_; p.ksplit = gemm_ksplit(n, kHidden, kHidden);
        hip_check(launch_gemm(p, EPI_PART, kvt_, s), "proj");
        hip_check(launch_resid_ln_rows(part_, p.ksplit, n, L.proj_b, x_, kHidden, x_, L.ln2_w, L.ln2_b, nullptr,
                                       nullptr, s, q8a_, d8a_),
                  "proj reduce + ln2");
        GemmArgs f1;
        f1.w = L.fc_in_w; f1.wm = L.fc_in_wm; f1.N = kFF; f1.K = kHidden; f1.lda = kHidden; f1.M = n;
        f1.a8 = q8a_; f1.d8 = d8a_; f1.a8_tiled = true;
        f1.bias = L.fc_in_b; f1.q8_out = q8h_; f1.d8_out = d8h_;
        hip_check(launch_gemm(f1, EPI_GELU, kvt_, s), "fc_in");
        GemmArgs f2;
        f2.w = L.fc_out_w; f2.wm = L.fc_out_wm; f2.N = kHidden; f2.K = kFF; f2.lda = kFF; f2.M = n;
        f2.a8 = q8h_; f2.d8 = d8h_; f2.a8_tiled = true;
        f2.part = part_; f2.ksplit = std::max(gemm_ksplit(n, kHidden, kFF), kBatchFcOutSplit);
        hip_check(launch_gemm(f2, EPI_PART, kvt_, s), "fc_out");
        const bool last = l + 1 == kLayers;
        hip_check(launch_resid_ln_rows(part_, f2.ksplit, n, L.fc_out_b, x_, kHidden, x_,
                                       last ? w_.lnf_w : w_.global[l + 1].ln1_w,
                                       last ? w_.lnf_b : w_.global[l + 1].ln1_b, last ? hidden_ : nullptr,
                                       last ? active_ : nullptr, s, last ? nullptr : q8a_, last ? nullptr : d8a_),
                  "fc_out reduce + ln");
    }
    hip_check(launch_advance_rows(st, n, s), "advance");
}

Batch::Graphs &Batch::graphs_for(int n) {
    auto it = graphs_.find(n);
    if (it != graphs_.end()) return it->second;
    Graphs g;
    hipGraph_t graph = nullptr;
    for (int greedy = 0; greedy < 2; ++greedy) {
        hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
        enqueue_frame_local(stream_, n, greedy != 0);
        hip_check(hipStreamEndCapture(stream_, &graph), "end capture");
        hip_check(hipGraphInstantiate(greedy ? &g.local_greedy : &g.local, graph, nullptr, nullptr, 0), "instantiate");
        (void)hipGraphDestroy(graph);
    }
    hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
    enqueue_global(stream_, n);
    hip_check(hipStreamEndCapture(stream_, &graph), "end capture");
    hip_check(hipGraphInstantiate(&g.global, graph, nullptr, nullptr, 0), "instantiate");
    (void)hipGraphDestroy(graph);
    return graphs_[n] = g;
}

void Batch::global_step(int n, const int32_t *rows) {
    if (n <= 0 || n > S_) throw Status(MOSS_HIP_EINVAL, "n_streams out of range");
    for (int s = 0; s < n; ++s) {
        if (pos_[s] >= cap_) throw Status(MOSS_HIP_ESTATE, "stream " + std::to_string(s) + " is at capacity");
        if (rows[(size_t)s * 17] < 0 || rows[(size_t)s * 17] >= kVocab)
            throw Status(MOSS_HIP_EINVAL, "row " + std::to_string(s) + ": text id out of [0, 16384)");
    }
    hip_check(hipSetDevice(model_.device()), "hipSetDevice");
    Graphs &g = graphs_for(n);
    std::vector<unsigned char> act(n, 1);
    hip_check(hipMemcpyAsync(row_, rows, sizeof(int32_t) * 17 * n, hipMemcpyHostToDevice, stream_), "rows h2d");
    hip_check(hipMemcpyAsync(active_, act.data(), n, hipMemcpyHostToDevice, stream_), "active h2d");
    upload_order(n);
    moss_hip_sample_params gp{};
    gp.greedy = 1;
    gp.end_greedy = 1;
    write_ctrl(0, 1.0f, sample_cfg(gp));
    hip_check(hipGraphLaunch(g.global, stream_), "graph launch");
    hip_check(hipMemcpyAsync(pos_.data(), pos_d_, sizeof(int) * S_, hipMemcpyDeviceToHost, stream_), "pos d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
}

double Batch::generate(int n, int frames, const moss_hip_sample_params &p, const uint64_t *seeds, int32_t *out_rows,
                       int *out_frames) {
    if (n <= 0 || n > S_) throw Status(MOSS_HIP_EINVAL, "n_streams out of range");
    if (frames <= 0) return 0.0;
    if (frames > cap_ + 1) frames = cap_ + 1;
    hip_check(hipSetDevice(model_.device()), "hipSetDevice");
    Graphs &g = graphs_for(n);
    std::vector<unsigned char> act(n);
    for (int s = 0; s < n; ++s) act[s] = pos_[s] < cap_ ? 1 : 0;
    hip_check(hipMemcpyAsync(active_, act.data(), n, hipMemcpyHostToDevice, stream_), "active h2d");
    hip_check(hipMemsetAsync(counts_, 0, sizeof(int) * (size_t)n * kNVq * kCodebook, stream_), "counts clear");
    write_ctrl(p.min_frames, p.repetition_penalty, sample_cfg(p));
    std::vector<uint32_t> rs((size_t)4 * n);
    for (int s = 0; s < n; ++s) rng_seed_host(seeds ? seeds[s] : 0, &rs[(size_t)4 * s]);
    hip_check(hipMemcpyAsync(rng_, rs.data(), rs.size() * sizeof(uint32_t), hipMemcpyHostToDevice, stream_), "rng h2d");
    upload_order(n);
    hip_check(hipStreamSynchronize(stream_), "sync");
    hip_check(hipEventRecord(ev_[0], stream_), "event");
    const SampleCfg cfg = sample_cfg(p);
    for (int f = 0; f < frames; ++f) {
        // the device's rule for a greedy frame (sample_rows_kernel): cfg.greedy || frame < greedy_frames
        const bool greedy = cfg.greedy || f < cfg.greedy_frames;
        hip_check(hipGraphLaunch(greedy ? g.local_greedy : g.local, stream_), "graph launch");
        hip_check(hipMemcpyAsync(hist_active_ + (size_t)f * S_, active_, n, hipMemcpyDeviceToDevice, stream_), "hist");
        hip_check(hipMemcpyAsync(hist_codes_ + (size_t)f * S_ * kNVq, codes_, sizeof(int) * n * kNVq,
                                 hipMemcpyDeviceToDevice, stream_),
                  "hist");
        if (f + 1 < frames) hip_check(hipGraphLaunch(g.global, stream_), "graph launch");
    }
    hip_check(hipEventRecord(ev_[1], stream_), "event");
    std::vector<unsigned char> ha((size_t)frames * S_);
    std::vector<int> hc((size_t)frames * S_ * kNVq);
    hip_check(hipMemcpyAsync(ha.data(), hist_active_, ha.size(), hipMemcpyDeviceToHost, stream_), "hist d2h");
    hip_check(hipMemcpyAsync(hc.data(), hist_codes_, hc.size() * sizeof(int), hipMemcpyDeviceToHost, stream_), "hist d2h");
    hip_check(hipMemcpyAsync(pos_.data(), pos_d_, sizeof(int) * S_, hipMemcpyDeviceToHost, stream_), "pos d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
    float ms = 0.f;
    hip_check(hipEventElapsedTime(&ms, ev_[0], ev_[1]), "elapsed");
    for (int s = 0; s < n; ++s) {
        int nf = 0;
        while (nf < frames && ha[(size_t)nf * S_ + s]) ++nf;
        if (out_frames) out_frames[s] = nf;
        for (int f = 0; f < nf; ++f) {
            int32_t *row = out_rows + ((size_t)f * n + s) * 17;
            row[0] = 0;
            for (int ch = 0; ch < kNVq; ++ch) row[ch + 1] = hc[((size_t)f * S_ + s) * kNVq + ch];
        }
    }
    return ms;
}

}  // namespace mh
