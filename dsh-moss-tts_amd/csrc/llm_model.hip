// llm_model.hip -- host driver of the GPU-resident LLM (see llm_model.h).
#include "llm_model.h"

#include <algorithm>
#include <atomic>

#include <chrono>
#include <cmath>
#include <cstddef>
#include <cstdlib>
#include <cstring>
#include <unordered_map>
#include <vector>

namespace mh {

// fused-launch recoveries of every model of the process (moss_hip_fallbacks_total)
std::atomic<int> fallbacks_total{0};

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess) throw Status(MOSS_HIP_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

// .moss v1 index (reference csrc/src/weights.cpp:27-125): "MOSW", u32 version = 1,
// u32 n; 80-byte entries: name[48], u8 dtype, u8 ndim, u32 dims[3] @52, u64 offset
// @64, u64 nbytes @72.
std::unordered_map<std::string, MossEntry> parse_moss_index(const uint8_t *blob, size_t bytes) {
    if (bytes < 16 || std::memcmp(blob, "MOSW", 4) != 0) throw Status(MOSS_HIP_EFORMAT, "not a .moss file (bad magic)");
    uint32_t version = 0, n = 0;
    std::memcpy(&version, blob + 4, 4);
    std::memcpy(&n, blob + 8, 4);
    if (version != 1) throw Status(MOSS_HIP_EFORMAT, "unsupported .moss version " + std::to_string(version));
    if (16 + (size_t)n * 80 > bytes) throw Status(MOSS_HIP_EFORMAT, ".moss index truncated");
    std::unordered_map<std::string, MossEntry> out;
    for (uint32_t i = 0; i < n; ++i) {
        const uint8_t *e = blob + 16 + (size_t)i * 80;
        char name[49];
        std::memcpy(name, e, 48);
        name[48] = 0;
        MossEntry en;
        en.dtype = e[48];
        en.ndim = e[49];
        std::memcpy(en.dims, e + 52, 12);
        std::memcpy(&en.off, e + 64, 8);
        std::memcpy(&en.nbytes, e + 72, 8);
        if (en.off + en.nbytes > bytes) throw Status(MOSS_HIP_EFORMAT, std::string("tensor out of range: ") + name);
        // the format aligns every tensor to 32 bytes; the kernels copy weight runs by
        // 16-byte DMA, which needs it
        if (en.off % 32) throw Status(MOSS_HIP_EFORMAT, std::string("tensor not 32-byte aligned: ") + name);
        out[name] = en;
    }
    return out;
}

bool is_vector(const MossEntry &e) { return e.ndim == 1 || (e.dims[0] == 1 && e.dims[2] == 1); }

namespace {

constexpr size_t kStateRowOff = offsetof(DevState, row);

}  // namespace

Model::Model(const void *blob, size_t bytes, const moss_hip_llm_options &opt) {
    device_ = opt.device;
    max_ctx_ = opt.max_ctx > 0 ? opt.max_ctx : kMaxCtx;
    if (max_ctx_ > 65536) throw Status(MOSS_HIP_EINVAL, "max_ctx too large");
    kvt_ = opt.kv_dtype == 1 ? KV_F32 : KV_F16;
    kv_esize_ = kvt_ == KV_F32 ? 4 : 2;
    use_graphs_ = opt.use_graphs;
    prefill_a16_ = opt.prefill_a16 != 0;
    decode_a8_ = opt.decode_a8 != 0 ? 1 : 0;
    if (const char *b = std::getenv("MOSS_HIP_POLL_BUDGET")) {
        poll_budget_ = std::max(0, std::atoi(b));
        if (const char *at = std::strchr(b, '@')) poll_budget_from_ = std::max(0, std::atoi(at + 1));
    }
    if (opt.decode_kernels != 0 && opt.decode_kernels != 1) throw Status(MOSS_HIP_EINVAL, "decode_kernels: 0 or 1");
    const uint8_t *b = static_cast<const uint8_t *>(blob);
    auto idx = parse_moss_index(b, bytes);

    // Resolve every tensor LlmModel::load needs (llm.cpp:44-70) before touching the GPU.
    std::unordered_map<std::string, uint64_t> off;
    auto need_vec = [&](const std::string &name, uint32_t n) {
        auto it = idx.find(name);
        if (it == idx.end() || !is_vector(it->second)) throw Status(MOSS_HIP_EFORMAT, "missing vector: " + name);
        if (it->second.dims[0] * it->second.dims[1] != n || it->second.nbytes < (uint64_t)n * 4)
            throw Status(MOSS_HIP_EFORMAT, "bad vector size: " + name);
        off[name] = it->second.off;
    };
    auto need_mat = [&](const std::string &name, uint32_t rows, uint32_t cols) {
        auto it = idx.find(name);
        if (it == idx.end() || is_vector(it->second)) throw Status(MOSS_HIP_EFORMAT, "missing matrix: " + name);
        if (it->second.dtype != 4)
            throw Status(MOSS_HIP_EUNSUPPORTED, "matrix " + name + " has dtype " + std::to_string(it->second.dtype) +
                                                    "; only Q8_0_4X4 (4) is supported");
        if (it->second.dims[0] != rows || it->second.dims[1] != cols ||
            it->second.nbytes < (uint64_t)(rows / 4) * (cols / 32) * kBlockBytes)
            throw Status(MOSS_HIP_EFORMAT, "bad matrix shape: " + name);
        off[name] = it->second.off;
    };
    auto need_layer = [&](const std::string &p) {
        need_vec(p + "ln1.w", kHidden);
        need_vec(p + "ln1.b", kHidden);
        need_vec(p + "ln2.w", kHidden);
        need_vec(p + "ln2.b", kHidden);
        need_mat(p + "attn.w", 3 * kHidden, kHidden);
        need_vec(p + "attn.b", 3 * kHidden);
        need_mat(p + "proj.w", kHidden, kHidden);
        need_vec(p + "proj.b", kHidden);
        need_mat(p + "fc_in.w", kFF, kHidden);
        need_vec(p + "fc_in.b", kFF);
        need_mat(p + "fc_out.w", kHidden, kFF);
        need_vec(p + "fc_out.b", kHidden);
    };
    for (int i = 0; i < kLayers; ++i) need_layer("g" + std::to_string(i) + ".");
    need_layer("local.");
    need_vec("lnf.w", kHidden);
    need_vec("lnf.b", kHidden);
    need_vec("local.lnf.w", kHidden);
    need_vec("local.lnf.b", kHidden);
    need_mat("wte", kVocab, kHidden);
    for (int ch = 0; ch < kNVq; ++ch) need_mat("aemb." + std::to_string(ch), kCodebook, kHidden);

    hip_check(hipSetDevice(device_), "hipSetDevice");
    hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    // per readback slot: four timing events around the two launches (recorded
    // only when the caller asks for timing) and one completion event of the
    // state readback (no timestamp)
    for (int i = 0; i < 2 * kEvPerSlot; ++i)
        hip_check(i % kEvPerSlot == kEvRead ? hipEventCreateWithFlags(&ev_[i], hipEventDisableTiming)
                                            : hipEventCreate(&ev_[i]),
                  "hipEventCreate");
    hip_check(hipMalloc(&blob_, bytes), "hipMalloc(weights)");
    hip_check(hipMemcpy(blob_, blob, bytes, hipMemcpyHostToDevice), "upload weights");

    auto V = [&](const std::string &n) { return reinterpret_cast<const float *>(blob_ + off.at(n)); };
    auto M = [&](const std::string &n) { return static_cast<const uint8_t *>(blob_ + off.at(n)); };
    auto set_layer = [&](LayerW &L, const std::string &p) {
        L.ln1_w = V(p + "ln1.w");
        L.ln1_b = V(p + "ln1.b");
        L.ln2_w = V(p + "ln2.w");
        L.ln2_b = V(p + "ln2.b");
        L.attn_w = M(p + "attn.w");
        L.attn_b = V(p + "attn.b");
        L.proj_w = M(p + "proj.w");
        L.proj_b = V(p + "proj.b");
        L.fc_in_w = M(p + "fc_in.w");
        L.fc_in_b = V(p + "fc_in.b");
        L.fc_out_w = M(p + "fc_out.w");
        L.fc_out_b = V(p + "fc_out.b");
    };
    for (int i = 0; i < kLayers; ++i) set_layer(g_[i], "g" + std::to_string(i) + ".");
    set_layer(local_, "local.");
    lnf_w_ = V("lnf.w");
    lnf_b_ = V("lnf.b");
    llnf_w_ = V("local.lnf.w");
    llnf_b_ = V("local.lnf.b");
    wte_ = M("wte");
    for (int ch = 0; ch < kNVq; ++ch) aemb_[ch] = M("aemb." + std::to_string(ch));

    // KV cache [K|V][layer][head][pos][64]
    const size_t kv_bytes = 2ull * kLayers * kHeads * max_ctx_ * kHeadDim * kv_esize_;
    hip_check(hipMalloc(&kv_, kv_bytes), "hipMalloc(kv)");
    hip_check(hipMemset(kv_, 0, kv_bytes), "memset(kv)");
    hip_check(hipMalloc(&lkv_, 2ull * kHeads * kLocalLen * kHeadDim * 4), "hipMalloc(local kv)");

    // RoPE table: angle = pos * 10000^(-2i/64) in double, stored as float
    // (reference csrc/src/llm.cpp:90-102; identical for every head).
    rope_n_ = max_ctx_ > kLocalLen ? max_ctx_ : kLocalLen;
    std::vector<float> rope(2ull * rope_n_ * kRopeHalf);
    for (int p = 0; p < rope_n_; ++p)
        for (int i = 0; i < kRopeHalf; ++i) {
            const double inv = 1.0 / std::pow(10000.0, static_cast<double>(2 * i) / kHeadDim);
            const double ang = static_cast<double>(p) * inv;
            rope[(size_t)p * kRopeHalf + i] = static_cast<float>(std::cos(ang));
            rope[(size_t)(rope_n_ + p) * kRopeHalf + i] = static_cast<float>(std::sin(ang));
        }
    hip_check(hipMalloc(&rope_, rope.size() * 4), "hipMalloc(rope)");
    hip_check(hipMemcpy(rope_, rope.data(), rope.size() * 4, hipMemcpyHostToDevice), "upload rope");

    auto fmalloc = [&](float **p, size_t n) { hip_check(hipMalloc(p, n * 4), "hipMalloc(act)"); };
    fmalloc(&x_, kHidden);
    fmalloc(&q_, kHidden);
    fmalloc(&mlp_, kFF);
    fmalloc(&hidden_, kHidden);
    fmalloc(&lres_, kHidden);
    fmalloc(&next_in_, kHidden);
    fmalloc(&slot_in_, kHidden);
    fmalloc(&attn_out_, kHidden);
    fmalloc(&attn_part_, (size_t)kHeads * ((max_ctx_ + 63) / 64) * kPartStride);
    fmalloc(&logits_, (size_t)kNVq * kCodebook);
    fmalloc(&text_logits_, kVocab);
    hip_check(hipMalloc(&counts_, sizeof(int) * kNVq * kCodebook), "hipMalloc(counts)");
    if (opt.decode_kernels == 0) {
        bool fits = false;
        hip_check(decode_layer_fits(device_, &fits), "decode layer occupancy");
        fused_layers_ = fits;
    }
    // the per-operator global step merges at most 16 split-KV spans in the proj prologue
    if (!fused_layers_ && max_ctx_ > 64 * 16)
        throw Status(MOSS_HIP_EUNSUPPORTED, "max_ctx > 1024 needs the fused decode kernels (decode_kernels = 0)");
    if (fused_layers_) {
        hip_check(hipMalloc(&ll_, sizeof(uint64_t) * kLayerWords), "hipMalloc(exchange)");
        hip_check(hipMemset(ll_, 0, sizeof(uint64_t) * kLayerWords), "memset(exchange)");
        // tags carry (position + 1) << 5 | block: positions below 2^26, blocks below 32
        if (max_ctx_ >= (1 << 26)) throw Status(MOSS_HIP_EINVAL, "max_ctx too large for the fused decode kernels");
        std::vector<LayerArgs> la(kLayers);
        for (int l = 0; l < kLayers; ++l) {
            const LayerW &L = g_[l];
            LayerArgs &d = la[l];
            d.attn_w = L.attn_w; d.proj_w = L.proj_w; d.fc_in_w = L.fc_in_w; d.fc_out_w = L.fc_out_w;
            d.attn_b = L.attn_b; d.proj_b = L.proj_b; d.fc_in_b = L.fc_in_b; d.fc_out_b = L.fc_out_b;
            d.ln1_w = L.ln1_w; d.ln1_b = L.ln1_b; d.ln2_w = L.ln2_w; d.ln2_b = L.ln2_b;
            d.k_cache = kv_layer(0, l); d.v_cache = kv_layer(1, l); d.ctx_stride = max_ctx_;
            d.rope_cos = rope_; d.rope_sin = rope_ + (size_t)rope_n_ * kRopeHalf;
        }
        hip_check(hipMalloc(&layer_args_, sizeof(LayerArgs) * kLayers), "hipMalloc(layer args)");
        hip_check(hipMemcpy(layer_args_, la.data(), sizeof(LayerArgs) * kLayers, hipMemcpyHostToDevice),
                  "upload layer args");
    }
    hip_check(hipMalloc(&forced_, sizeof(int) * kNVq * (max_ctx_ + 2)), "hipMalloc(forced)");
    hip_check(hipMemset(hidden_, 0, kHidden * 4), "memset(hidden)");
    hip_check(hipMalloc(&state_, sizeof(DevState)), "hipMalloc(state)");
    hip_check(hipHostMalloc(&hstate_, sizeof(DevState), hipHostMallocDefault), "hipHostMalloc(state)");
    hip_check(hipHostMalloc(&hread_, 2 * sizeof(DevState), hipHostMallocDefault), "hipHostMalloc(state readback)");
    std::memset(hstate_, 0, sizeof(DevState));
    hstate_->rep_penalty = 1.0f;
    hip_check(hipMemcpy(state_, hstate_, sizeof(DevState), hipMemcpyHostToDevice), "init state");

    // The first local input of every channel loop is wte[slot] (llm.cpp:682): dequantise once.
    rows_cap_ = 1;
    hip_check(hipMalloc(&rows_dev_, sizeof(int) * 17), "hipMalloc(rows)");
    const int slot = kSlotToken;
    hip_check(hipMemcpy(rows_dev_, &slot, sizeof(int), hipMemcpyHostToDevice), "slot row");
    hip_check(launch_dequant_rows(wte_, kVocab, kHidden, rows_dev_, 1, slot_in_, stream_), "dequant slot row");
    hip_check(hipStreamSynchronize(stream_), "sync");
    build_qkv_table();  // the fused local steps and the batch engine look their q|k|v up
    tile_gemm_weights();
    if (use_graphs_) build_graphs();
}

// The prefill and batch-engine GEMMs read a copy of their matrices in the
// matrix-core order (one 544-byte unit per 16 rows and scale block, quants in
// MFMA lane order): a load of the GEMM then reads whole cache lines.  Same size
// as the Q8_0_4X4 matrices, which the decode GEMVs keep reading.
void Model::tile_gemm_weights() {
    if (const char *t = std::getenv("MOSS_HIP_GEMM_TILED"))
        if (std::strcmp(t, "0") == 0) return;
    const size_t bytes_layer = ((size_t)3 * kHidden * kHidden + (size_t)kHidden * kHidden + 2ull * kFF * kHidden) / 32 * 34;
    const size_t bytes_head = (size_t)kCodebook * kHidden / 32 * 34;
    hip_check(hipMalloc(&wm_, (kLayers + 1) * bytes_layer + kNVq * bytes_head), "hipMalloc(tiled weights)");
    uint8_t *p = wm_;
    auto tile = [&](const uint8_t *w, int n, int k) {
        hip_check(tile_q8x4_mfma(w, n, k, p, stream_), "tile weights");
        const uint8_t *r = p;
        p += (size_t)n * k / 32 * 34;
        return r;
    };
    auto tile_layer = [&](LayerW &L) {
        L.attn_wm = tile(L.attn_w, 3 * kHidden, kHidden);
        L.proj_wm = tile(L.proj_w, kHidden, kHidden);
        L.fc_in_wm = tile(L.fc_in_w, kFF, kHidden);
        L.fc_out_wm = tile(L.fc_out_w, kHidden, kFF);
    };
    for (auto &L : g_) tile_layer(L);
    tile_layer(local_);
    for (int ch = 0; ch < kNVq; ++ch) aemb_m_[ch] = tile(aemb_[ch], kCodebook, kHidden);
    hip_check(hipStreamSynchronize(stream_), "sync");
}

Model::~Model() {
    (void)hipSetDevice(device_);
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (g_global_) (void)hipGraphExecDestroy(g_global_);
    if (g_local_) (void)hipGraphExecDestroy(g_local_);
    if (g_local_fused_) (void)hipGraphExecDestroy(g_local_fused_);
    void *bufs[] = {blob_, wm_, kv_, lkv_, rope_, x_, q_, mlp_, hidden_, lres_, next_in_, slot_in_, attn_out_, attn_part_, pre_x_, pre_a_, pre_q_, pre_h_, pre_part_, pre_q8_, pre_d8_, pre_q8h_, pre_d8h_, logits_, counts_, forced_, text_logits_, rows_dev_, state_, snap_, ll_, qkv_table_, layer_args_, cap_dec_, cap_pre_};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    if (hstate_) (void)hipHostFree(hstate_);
    if (hread_) (void)hipHostFree(hread_);
    for (auto &e : ev_)
        if (e) (void)hipEventDestroy(e);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void *Model::kv_layer(int which, int layer) const {
    const size_t per = (size_t)kHeads * max_ctx_ * kHeadDim * kv_esize_;
    return static_cast<uint8_t *>(kv_) + ((size_t)which * kLayers + layer) * per;
}

// One global step: embed_row -> 12 x block_forward -> ln_f (llm.cpp:248-255).
// With the fused kernels it is one launch (decode_global_kernel).  Per operator,
// block_forward (llm.cpp:230-246) is five kernels: QKV GEMV with LN1 fused in its
// prologue and bias + RoPE + KV write in its epilogue; split-KV attention (one
// workgroup per head and 64-key span, unnormalised partials); proj GEMV merging
// the partials in its prologue, adding bias and residual in its epilogue; fc_in GEMV with LN2 in, bias + gelu out; fc_out GEMV with the
// residual out.  Every position-dependent kernel reads state->pos.
void Model::enqueue_global_step(hipStream_t s, const int *row_dev) {
    const int *pos = &state_->pos;
    if (fused_layers_) {  // embed, 12 blocks and ln_f in one launch
        GlobalArgs g;
        g.layers = layer_args_;
        g.wte = wte_;
        for (int ch = 0; ch < kNVq; ++ch) g.aemb[ch] = aemb_[ch];
        g.row = row_dev;
        g.lnf_w = lnf_w_; g.lnf_b = lnf_b_; g.hidden = hidden_;
        g.state = state_; g.ll = ll_; g.err = &state_->ll_err; g.a8 = decode_a8_;
        g.poll_budget = next_poll_budget();
        if (capture_ && decode_a8_) {
            g.cap = cap_dec_;
            cap_taken_[0] = true;
        }
        hip_check(launch_decode_global(g, kvt_, s), "decode global step");
        return;
    }
    EmbedArgs e;
    e.wte = wte_;
    for (int ch = 0; ch < kNVq; ++ch) e.aemb[ch] = aemb_[ch];
    e.row = row_dev;
    e.x = x_;
    e.state = state_;
    hip_check(launch_embed(e, s), "embed");
    for (int l = 0; l < kLayers; ++l) {
        const LayerW &L = g_[l];
        GemvArgs a;
        a.w = L.attn_w; a.rows = 3 * kHidden; a.cols = kHidden;
        a.x = x_; a.ln_w = L.ln1_w; a.ln_b = L.ln1_b;
        a.bias = L.attn_b; a.q_out = q_;
        a.k_cache = kv_layer(0, l); a.v_cache = kv_layer(1, l); a.ctx_stride = max_ctx_;
        a.rope_cos = rope_; a.rope_sin = rope_ + (size_t)rope_n_ * kRopeHalf;
        a.pos_ptr = pos; a.state = state_; a.a8 = decode_a8_;
        hip_check(launch_gemv(a, PRO_LN, EPI_QKV, kvt_, s), "qkv gemv");

        AttnArgs t;  // the cache is one page of max_ctx positions; split-KV partials per 64 keys
        t.q = q_; t.k_pool = a.k_cache; t.v_pool = a.v_cache; t.page_size = max_ctx_;
        t.row_pos = pos; t.max_keys = max_ctx_; t.part = attn_part_; t.state = state_;
        hip_check(launch_attn(t, kvt_, s), "attention");

        GemvArgs p;  // the partials are merged in the proj prologue
        p.w = L.proj_w; p.rows = kHidden; p.cols = kHidden;
        p.attn_part = attn_part_; p.attn_splits = (max_ctx_ + 63) / 64; p.pos_ptr = pos;
        p.y = x_; p.bias = L.proj_b; p.state = state_; p.a8 = decode_a8_;
        hip_check(launch_gemv(p, PRO_AMERGE, EPI_RESID, kvt_, s), "proj gemv");

        GemvArgs f1;
        f1.w = L.fc_in_w; f1.rows = kFF; f1.cols = kHidden;
        f1.x = x_; f1.ln_w = L.ln2_w; f1.ln_b = L.ln2_b;
        f1.y = mlp_; f1.bias = L.fc_in_b; f1.state = state_; f1.a8 = decode_a8_;
        hip_check(launch_gemv(f1, PRO_LN, EPI_GELU, kvt_, s), "fc_in gemv");

        GemvArgs f2;
        f2.w = L.fc_out_w; f2.rows = kHidden; f2.cols = kFF;
        f2.x = mlp_; f2.y = x_; f2.bias = L.fc_out_b; f2.state = state_; f2.a8 = decode_a8_;
        hip_check(launch_gemv(f2, PRO_F32, EPI_RESID, kvt_, s), "fc_out gemv");
    }
    hip_check(launch_layernorm(x_, lnf_w_, lnf_b_, hidden_, state_, 1, s), "ln_f");
}

// q|k|v rows of the local steps at lpos >= 1, whose block input is an embedding
// row: wte[slot] at lpos 1, aemb[lpos - 2][code] at lpos >= 2.  Each row is
// RoPE_lpos(attn_w . LN1(row) + attn_b), computed by the per-operator QKV GEMV
// (the kernel the per-operator path runs live on the same row), with the
// position folded into the RoPE table pointer and the k / v "cache" pointed at
// the row itself.
void Model::build_qkv_table() {
    const size_t row = 3 * kHidden;
    hip_check(hipMalloc(&qkv_table_, sizeof(float) * row * (1 + (size_t)(kNVq - 1) * kCodebook)),
              "hipMalloc(qkv table)");
    float *emb = nullptr;
    int *ids = nullptr;
    hip_check(hipMalloc(&emb, sizeof(float) * kCodebook * kHidden), "hipMalloc(table input)");
    hip_check(hipMalloc(&ids, sizeof(int) * kCodebook), "hipMalloc(table ids)");
    std::vector<int> iota(kCodebook);
    for (int i = 0; i < kCodebook; ++i) iota[i] = i;
    auto one = [&](const float *x, float *dst, int lpos) {
        GemvArgs a;
        a.w = local_.attn_w; a.rows = 3 * kHidden; a.cols = kHidden;
        a.x = x; a.ln_w = local_.ln1_w; a.ln_b = local_.ln1_b; a.bias = local_.attn_b;
        a.q_out = dst; a.k_cache = dst + kHidden; a.v_cache = dst + 2 * kHidden; a.ctx_stride = 1;
        a.rope_cos = rope_ + (size_t)lpos * kRopeHalf;
        a.rope_sin = rope_ + ((size_t)rope_n_ + lpos) * kRopeHalf;
        a.pos_const = 0;
        a.a8 = decode_a8_;
        hip_check(launch_gemv(a, PRO_LN, EPI_QKV, KV_F32, stream_), "qkv table row");
    };
    try {
        hip_check(hipMemcpyAsync(ids, iota.data(), sizeof(int) * kCodebook, hipMemcpyHostToDevice, stream_), "ids h2d");
        one(slot_in_, qkv_table_, 1);
        for (int ch = 0; ch + 1 < kNVq; ++ch) {  // input channel ch feeds lpos ch + 2
            hip_check(launch_dequant_rows(aemb_[ch], kCodebook, kHidden, ids, kCodebook, emb, stream_), "dequant aemb");
            for (int code = 0; code < kCodebook; ++code)
                one(emb + (size_t)code * kHidden, qkv_table_ + (1 + (size_t)ch * kCodebook + code) * row, ch + 2);
        }
        hip_check(hipStreamSynchronize(stream_), "sync");
    } catch (...) {
        (void)hipFree(emb);
        (void)hipFree(ids);
        throw;
    }
    (void)hipFree(emb);
    (void)hipFree(ids);
}

// local_step (llm.cpp:259-264) without its final ln_f: the residual stream starts
// as `in` (read by the proj epilogue) and lives in lres_; consumers apply the
// local ln_f in their own prologue.
// pick_ch >= 0: the input is the greedy pick of that channel, made in the QKV
// GEMV's prologue (which also stores the picked row in `in` for the residual).
void Model::enqueue_local_step(hipStream_t s, const float *in, int lpos, int pick_ch) {
    const LayerW &L = local_;
    float *lk = lkv_, *lv = lkv_ + (size_t)kHeads * kLocalLen * kHeadDim;
    GemvArgs a;
    a.w = L.attn_w; a.rows = 3 * kHidden; a.cols = kHidden;
    a.x = in; a.ln_w = L.ln1_w; a.ln_b = L.ln1_b;
    a.bias = L.attn_b; a.q_out = q_;
    a.k_cache = lk; a.v_cache = lv; a.ctx_stride = kLocalLen;
    a.rope_cos = rope_; a.rope_sin = rope_ + (size_t)rope_n_ * kRopeHalf;
    a.pos_const = lpos; a.state = state_; a.a8 = decode_a8_;
    if (pick_ch >= 0) {
        a.pick_logits = logits_ + (size_t)pick_ch * kCodebook;
        a.pick_counts = counts_ + (size_t)pick_ch * kCodebook;
        a.pick_aemb = aemb_[pick_ch];
        a.pick_forced = forced_;
        a.pick_ch = pick_ch;
        a.pick_state = state_;
        a.pick_raw = const_cast<float *>(in);
    }
    hip_check(launch_gemv(a, pick_ch >= 0 ? PRO_PICK : PRO_LN, EPI_QKV, KV_F32, s), "local qkv");

    // At most 17 keys: the attention is computed in the proj GEMV's prologue.
    GemvArgs p;
    p.w = L.proj_w; p.rows = kHidden; p.cols = kHidden;
    p.x = q_; p.k_cache = lk; p.v_cache = lv; p.ctx_stride = kLocalLen; p.pos_const = lpos;
    p.y = lres_; p.resid_in = in; p.bias = L.proj_b; p.state = state_; p.a8 = decode_a8_;
    hip_check(launch_gemv(p, PRO_LATTN, EPI_RESID, KV_F32, s), "local proj");

    GemvArgs f1;
    f1.w = L.fc_in_w; f1.rows = kFF; f1.cols = kHidden;
    f1.x = lres_; f1.ln_w = L.ln2_w; f1.ln_b = L.ln2_b;
    f1.y = mlp_; f1.bias = L.fc_in_b; f1.state = state_; f1.a8 = decode_a8_;
    hip_check(launch_gemv(f1, PRO_LN, EPI_GELU, KV_F32, s), "local fc_in");

    GemvArgs f2;
    f2.w = L.fc_out_w; f2.rows = kHidden; f2.cols = kFF;
    f2.x = mlp_; f2.y = lres_; f2.bias = L.fc_out_b; f2.state = state_; f2.a8 = decode_a8_;
    hip_check(launch_gemv(f2, PRO_F32, EPI_RESID, KV_F32, s), "local fc_out");
}

// The local half of a frame (llm.cpp:648-698): local step on hidden, end gate,
// then 16 x (local step, audio head of channel ch, pick + next input).
//
// fused (greedy decoding): the pick of channel ch - 1 runs in the prologue of
// channel ch's QKV GEMV instead of a kernel of its own; only channel 15 keeps
// its sample kernel, which also counts the frame's used codes.
void Model::enqueue_frame_local(hipStream_t s, bool text_gate, bool fused) {
    if (fused_layers_ && !text_gate) {  // one launch when greedy; else per position with a sampler between
        LocalArgs base;
        const LayerW &L = local_;
        base.attn_w = L.attn_w; base.proj_w = L.proj_w; base.fc_in_w = L.fc_in_w; base.fc_out_w = L.fc_out_w;
        base.attn_b = L.attn_b; base.proj_b = L.proj_b; base.fc_in_b = L.fc_in_b; base.fc_out_b = L.fc_out_b;
        base.ln1_w = L.ln1_w; base.ln1_b = L.ln1_b; base.ln2_w = L.ln2_w; base.ln2_b = L.ln2_b;
        base.lnf_w = llnf_w_; base.lnf_b = llnf_b_;
        base.lk = lkv_; base.lv = lkv_ + (size_t)kHeads * kLocalLen * kHeadDim;
        base.rope_cos = rope_; base.rope_sin = rope_ + (size_t)rope_n_ * kRopeHalf;
        base.state = state_; base.ll = ll_; base.err = &state_->ll_err; base.x_out = lres_;
        base.a8 = decode_a8_;
        base.poll_budget = next_poll_budget();
        if (capture_ && decode_a8_) {
            base.cap = cap_dec_ + (size_t)kLayers * MOSS_HIP_CAP_STEP;
            cap_taken_[1] = true;
        }
        for (int ch = 0; ch < kNVq; ++ch) base.aemb[ch] = aemb_[ch];
        base.qkv_table = qkv_table_;
        base.logits = logits_;
        base.counts = counts_;
        base.forced = forced_;
        base.x_in = hidden_;
        base.x_slot = slot_in_;
        if (fused) {  // greedy: the whole local half in one launch (positions 0..16, the gate, channel 15's pick)
            LocalArgs c = base;
            c.lpos = 0;
            c.lpos_last = kNVq;
            c.head = 1;
            c.pick = 1;
            c.gate = 1;
            c.wte = wte_;
            c.final_pick = 1;
            hip_check(launch_decode_local(c, s), "local steps");
            return;
        }
        LocalArgs z = base;  // lpos 0 on the global hidden state, then the end gate
        z.lpos = 0;
        z.lpos_last = 0;
        hip_check(launch_decode_local(z, s), "local step");
        hip_check(launch_gate(lres_, llnf_w_, llnf_b_, wte_, state_, s), "gate");
        LocalArgs c = base;  // the channel steps: input wte[slot] at lpos 1, then aemb[ch - 1][code]
        c.head = 1;
        SampleArgs sa;
        sa.counts = counts_;
        sa.forced = forced_;
        sa.next_input = next_in_;
        sa.state = state_;
        for (int ch = 0; ch < kNVq; ++ch) {
            c.lpos = c.lpos_last = ch + 1;
            hip_check(launch_decode_local(c, s), "local step");
            sa.logits = logits_ + (size_t)ch * kCodebook;
            sa.ch = ch;
            sa.aemb = aemb_[ch];
            sa.last_channel = ch == kNVq - 1;
            sa.count_all = 0;
            hip_check(launch_sample(sa, s), "sample");
        }
        return;
    }
    enqueue_local_step(s, hidden_, 0, -1);
    if (text_gate) {  // gate-dump frames: the whole text head, as llm.cpp:662-667
        GemvArgs t;
        t.w = wte_; t.rows = kVocab; t.cols = kHidden;
        t.x = lres_; t.ln_w = llnf_w_; t.ln_b = llnf_b_;
        t.y = text_logits_; t.state = state_; t.a8 = decode_a8_;
        hip_check(launch_gemv(t, PRO_LN, EPI_F32, KV_F32, s), "text head");
        hip_check(launch_gate_text(text_logits_, state_, s), "gate");
    } else {
        hip_check(launch_gate(lres_, llnf_w_, llnf_b_, wte_, state_, s), "gate");
    }
    for (int ch = 0; ch < kNVq; ++ch) {
        enqueue_local_step(s, ch == 0 ? slot_in_ : next_in_, ch + 1, fused && ch > 0 ? ch - 1 : -1);
        GemvArgs h;
        h.w = aemb_[ch]; h.rows = kCodebook; h.cols = kHidden;
        h.x = lres_; h.ln_w = llnf_w_; h.ln_b = llnf_b_;
        h.y = logits_ + (size_t)ch * kCodebook; h.state = state_; h.a8 = decode_a8_;
        hip_check(launch_gemv(h, PRO_LN, EPI_F32, KV_F32, s), "audio head");
        SampleArgs sa;
        sa.logits = logits_ + (size_t)ch * kCodebook;
        sa.ch = ch;
        sa.counts = counts_;
        sa.forced = forced_;
        sa.aemb = aemb_[ch];
        sa.next_input = next_in_;
        sa.state = state_;
        sa.last_channel = ch == kNVq - 1;
        sa.count_all = fused && ch == kNVq - 1;
        if (!fused || ch == kNVq - 1) hip_check(launch_sample(sa, s), "sample");
    }
}

// Graphs pay off where a step is many dependent kernels: the per-operator path
// (62 kernels per global step, 85-101 per local half) and the sampled local half
// of the fused path (17 local launches with a sampler after each).  The fused
// global step and the fused greedy local half are one kernel each, launched
// directly: a one-node graph measured 14 us per frame slower than the two plain
// launches (0.432 vs 0.418 ms/frame).
void Model::build_graphs() {
    hipGraph_t g = nullptr;
    if (!fused_layers_) {
        hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
        enqueue_global_step(stream_,
                            reinterpret_cast<const int *>(reinterpret_cast<uint8_t *>(state_) + kStateRowOff));
        hip_check(hipStreamEndCapture(stream_, &g), "end capture");
        hip_check(hipGraphInstantiate(&g_global_, g, nullptr, nullptr, 0), "instantiate global");
        (void)hipGraphDestroy(g);
    }
    for (int fused = 0; fused < 2; ++fused) {
        if (fused_layers_ && fused) continue;
        hip_check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "begin capture");
        enqueue_frame_local(stream_, false, fused != 0);
        hip_check(hipStreamEndCapture(stream_, &g), "end capture");
        hip_check(hipGraphInstantiate(fused ? &g_local_fused_ : &g_local_, g, nullptr, nullptr, 0),
                  "instantiate local");
        (void)hipGraphDestroy(g);
    }
}

void Model::launch_global(hipStream_t s) {
    if (g_global_)
        hip_check(hipGraphLaunch(g_global_, s), "graph launch");
    else
        enqueue_global_step(s, reinterpret_cast<const int *>(reinterpret_cast<uint8_t *>(state_) + kStateRowOff));
}

void Model::launch_frame_local(hipStream_t s, bool text_gate, bool fused) {
    hipGraphExec_t g = fused ? g_local_fused_ : g_local_;
    if (g && !text_gate)
        hip_check(hipGraphLaunch(g, s), "graph launch");
    else
        enqueue_frame_local(s, text_gate, fused);
}

// Pushes the scalar header (pos .. rep_penalty) of the host mirror to the device.
void Model::clear_exchange() {
    if (!fused_layers_) return;
    hip_check(hipMemsetAsync(ll_, 0, sizeof(uint64_t) * kLayerWords, stream_), "exchange clear");
    hip_check(hipMemsetAsync(&state_->ll_err, 0, sizeof(unsigned), stream_), "exchange error clear");
    hstate_->ll_err = 0;
}

void Model::check_exchange() {
    if (hstate_->ll_err != 0)
        throw Status(MOSS_HIP_EDEVICE, "decode layer: a stage waited past its budget for another workgroup "
                                       "(the device did not hold all workgroups of the launch at once)");
}

void Model::write_state_header() {
    hstate_->pos = pos_;
    hip_check(hipMemcpyAsync(state_, hstate_, offsetof(DevState, row), hipMemcpyHostToDevice, stream_), "state h2d");
}

void Model::reset() { pos_ = 0; }

// Per layer of a prefill capture of m rows: fp32 rows (xin, ln1, att, xm, ln2: 768 wide; h:
// 3072; xout: 768), then the int8 operands (ln1, att, ln2: M16 x 768; h: M16 x 3072) and their
// block scales (M16 x 24 x 3, M16 x 96), as moss_hip.h lays them out.
static size_t cap_layer_bytes(size_t m) {
    const size_t m16 = (m + 15) / 16 * 16;
    return 4 * m * (6 * kHidden + kFF) + m16 * (3 * kHidden + kFF) + 4 * m16 * (3 * (kHidden / 32) + kFF / 32);
}

void Model::set_capture(bool on) {
    if (on && !cap_dec_) {
        const size_t n = (size_t)(kLayers + kLocalLen) * MOSS_HIP_CAP_STEP;
        hip_check(hipMalloc(&cap_dec_, sizeof(float) * n), "hipMalloc(capture)");
        hip_check(hipMemsetAsync(cap_dec_, 0, sizeof(float) * n, stream_), "capture clear");
        hip_check(hipStreamSynchronize(stream_), "sync");
    }
    capture_ = on;
}

size_t Model::capture_read(int what, void *out, size_t bytes) {
    const void *src = nullptr;
    size_t n = 0;
    if (what == MOSS_HIP_CAP_GLOBAL && cap_taken_[0]) {
        src = cap_dec_;
        n = sizeof(float) * kLayers * MOSS_HIP_CAP_STEP;
    } else if (what == MOSS_HIP_CAP_LOCAL && cap_taken_[1]) {
        src = cap_dec_ + (size_t)kLayers * MOSS_HIP_CAP_STEP;
        n = sizeof(float) * kLocalLen * MOSS_HIP_CAP_STEP;
    } else if (what == MOSS_HIP_CAP_PREFILL && cap_pre_used_ > 0) {
        src = cap_pre_;
        n = cap_pre_used_;
    }
    if (n == 0 || out == nullptr || bytes < n) return n;
    hip_check(hipMemcpyAsync(out, src, n, hipMemcpyDeviceToHost, stream_), "capture d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
    return n;
}

void Model::get_hidden(float *out) {
    hip_check(hipMemcpyAsync(out, hidden_, kHidden * 4, hipMemcpyDeviceToHost, stream_), "hidden d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
}

void Model::set_hidden(const float *in) {
    hip_check(hipMemcpyAsync(hidden_, in, kHidden * 4, hipMemcpyHostToDevice, stream_), "hidden h2d");
    hip_check(hipStreamSynchronize(stream_), "sync");
}

// Token ids index wte directly (lookup_row, llm.cpp:149): reject what would read
// outside the table.  Codes outside [0, 1024) are skipped as pads (llm.cpp:153).
static void check_rows(const int32_t *rows, int n) {
    for (int i = 0; i < n; ++i)
        if (rows[(size_t)i * 17] < 0 || rows[(size_t)i * 17] >= kVocab)
            throw Status(MOSS_HIP_EINVAL, "row " + std::to_string(i) + ": text id out of [0, 16384)");
}

void Model::global_step(const int32_t *row) {
    if (pos_ >= max_ctx_) throw Status(MOSS_HIP_ESTATE, "KV cache full (position == max_ctx)");
    check_rows(row, 1);
    hstate_->stop = 0;
    write_state_header();
    hip_check(hipMemcpyAsync(reinterpret_cast<uint8_t *>(state_) + kStateRowOff, row, 17 * sizeof(int32_t),
                             hipMemcpyHostToDevice, stream_),
              "row h2d");
    clear_exchange();
    launch_global(stream_);
    hip_check(hipMemcpyAsync(&hstate_->ll_err, &state_->ll_err, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
              "state d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
    if (hstate_->ll_err != 0 && fused_layers_ && can_fall_back()) {
        // the step is a function of the row, the position and the cache below it: redo it
        // per operator (it rewrites the K/V row at pos and the hidden state)
        ++fallbacks_;
        fallbacks_total.fetch_add(1, std::memory_order_relaxed);
        hstate_->ll_err = 0;
        write_state_header();
        hip_check(hipMemcpyAsync(reinterpret_cast<uint8_t *>(state_) + kStateRowOff, row, 17 * sizeof(int32_t),
                                 hipMemcpyHostToDevice, stream_),
                  "row h2d");
        hip_check(hipMemsetAsync(&state_->ll_err, 0, sizeof(unsigned), stream_), "exchange error clear");
        fused_layers_ = false;
        try {
            launch_global(stream_);
        } catch (...) {
            fused_layers_ = true;
            throw;
        }
        fused_layers_ = true;
        hip_check(hipStreamSynchronize(stream_), "sync");
    }
    check_exchange();
    ++pos_;
}

// LlmModel::prefill (llm.cpp:327-401), batched over the m rows like the
// reference: embed all rows, then per layer LN1 -> QKV GEMM (bias, RoPE and the
// K/V of positions [start, start+m) written in its epilogue) -> causal
// attention of row i over keys <= start+i -> proj GEMM + residual -> LN2 ->
// fc_in GEMM + gelu -> fc_out GEMM + residual; hidden = ln_f of the last row.
// The GEMMs run on the matrix cores: W8A8 by default (int8 activations per
// 32-block, i8 MFMA, fp32 block-scale FMA -- the reference's prefill), or
// W8A16 on fp32 activations (the reference with MOSS_A16=1) when prefill_a16.
void Model::prefill(const int32_t *rows, int n, int start) {
    start = start < 0 ? 0 : (start > max_ctx_ ? max_ctx_ : start);
    const int m = n < max_ctx_ - start ? n : max_ctx_ - start;
    if (m <= 0) return;
    check_rows(rows, m);
    if (m > rows_cap_) {
        void *bufs[] = {rows_dev_, pre_x_, pre_a_, pre_q_, pre_h_, pre_part_, pre_q8_, pre_d8_, pre_q8h_, pre_d8h_};
        for (void *p : bufs)
            if (p) hip_check(hipFree(p), "free prefill buffers");
        rows_dev_ = nullptr;
        pre_x_ = pre_a_ = pre_q_ = pre_h_ = pre_part_ = pre_d8_ = pre_d8h_ = nullptr;
        pre_q8_ = pre_q8h_ = nullptr;
        rows_cap_ = 0;
        hip_check(hipMalloc(&rows_dev_, sizeof(int) * 17 * (size_t)m), "hipMalloc(rows)");
        // pre_a_, pre_h_: GEMM inputs, as fp16 hi / lo halves in the matrix-core
        // order under A16 (hlt_at: 4 bytes a value, rows padded to 16)
        const size_t mp = (size_t)(m + 15) / 16 * 16;
        hip_check(hipMalloc(&pre_x_, sizeof(float) * kHidden * (size_t)m), "hipMalloc(prefill)");
        hip_check(hipMalloc(&pre_a_, sizeof(float) * kHidden * mp), "hipMalloc(prefill)");
        hip_check(hipMalloc(&pre_q_, sizeof(float) * kHidden * (size_t)m), "hipMalloc(prefill)");
        hip_check(hipMalloc(&pre_h_, sizeof(float) * kFF * mp), "hipMalloc(prefill)");
        hip_check(hipMemsetAsync(pre_a_, 0, sizeof(float) * kHidden * mp, stream_), "memset(prefill)");
        hip_check(hipMemsetAsync(pre_h_, 0, sizeof(float) * kFF * mp, stream_), "memset(prefill)");
        // split-K partials: proj's (one per head when the attention applies proj) and fc_out's
        const int kz = std::max(std::max(gemm_ksplit(m, kHidden, kHidden), gemm_ksplit(m, kHidden, kFF)),
                                std::max(kPrefillFcOutSplit, kHeads));
        hip_check(hipMalloc(&pre_part_, sizeof(float) * kHidden * (size_t)m * kz), "hipMalloc(prefill)");
        // W8A8 operands in the matrix-core order: rows padded to 16 (the padding rows are
        // read by the GEMMs and never stored; zeroed once)
        const size_t m16 = (size_t)(m + 15) / 16 * 16;
        hip_check(hipMalloc(&pre_q8_, (size_t)kHidden * m16), "hipMalloc(prefill)");
        hip_check(hipMalloc(&pre_d8_, sizeof(float) * (kHidden / 32) * m16), "hipMalloc(prefill)");
        hip_check(hipMalloc(&pre_q8h_, (size_t)kFF * m16), "hipMalloc(prefill)");
        hip_check(hipMalloc(&pre_d8h_, sizeof(float) * (kFF / 32) * m16), "hipMalloc(prefill)");
        hip_check(hipMemsetAsync(pre_q8_, 0, (size_t)kHidden * m16, stream_), "memset(prefill)");
        hip_check(hipMemsetAsync(pre_d8_, 0, sizeof(float) * (kHidden / 32) * m16, stream_), "memset(prefill)");
        hip_check(hipMemsetAsync(pre_q8h_, 0, (size_t)kFF * m16, stream_), "memset(prefill)");
        hip_check(hipMemsetAsync(pre_d8h_, 0, sizeof(float) * (kFF / 32) * m16, stream_), "memset(prefill)");
        rows_cap_ = m;
    }
    hip_check(hipMemcpyAsync(rows_dev_, rows, sizeof(int) * 17 * (size_t)m, hipMemcpyHostToDevice, stream_), "rows h2d");
    hstate_->stop = 0;
    pos_ = start;
    write_state_header();
    hipStream_t s = stream_;
    EmbedArgs e;
    e.wte = wte_;
    for (int ch = 0; ch < kNVq; ++ch) e.aemb[ch] = aemb_[ch];
    hip_check(launch_embed_rows(e, rows_dev_, m, pre_x_, s), "prefill embed");
    // W8A8 (the reference's prefill, llm.cpp:319-328): every GEMM input is also
    // quantised per 32-block by the kernel that produces it
    const bool a8 = !prefill_a16_;
    // quantiser capture (tests): the producers also write their fp32 rows into the
    // capture, and each int8 operand and the residual stream are copied there before
    // the next kernel overwrites them
    const bool cap = capture_ && a8;
    const size_t m16 = (size_t)(m + 15) / 16 * 16, cap_lb = cap_layer_bytes(m);
    if (cap && cap_pre_bytes_ < cap_lb * kLayers) {
        if (cap_pre_) hip_check(hipFree(cap_pre_), "free capture");
        cap_pre_ = nullptr;
        cap_pre_bytes_ = 0;
        hip_check(hipMalloc(&cap_pre_, cap_lb * kLayers), "hipMalloc(prefill capture)");
        cap_pre_bytes_ = cap_lb * kLayers;
    }
    cap_pre_used_ = 0;
    auto cap_f = [&](int l, int sec) -> float * {  // 0 xin, 1 ln1, 2 att, 3 xm, 4 ln2, 5 h, 6 xout
        if (!cap || l >= kLayers) return nullptr;
        const size_t off = sec <= 5 ? (size_t)sec * m * kHidden : (size_t)5 * m * kHidden + (size_t)m * kFF;
        return reinterpret_cast<float *>(cap_pre_ + (size_t)l * cap_lb) + off;
    };
    const size_t cap_q0 = 4 * (size_t)m * (6 * kHidden + kFF);
    const size_t cap_d0 = cap_q0 + m16 * (3 * kHidden + kFF);
    auto cap_copy_q = [&](int l, int sec, const int8_t *q, const float *d) {  // 0 ln1, 1 att, 2 ln2, 3 h
        if (!cap || l >= kLayers) return;
        uint8_t *base = cap_pre_ + (size_t)l * cap_lb;
        const size_t K = sec == 3 ? kFF : kHidden;
        hip_check(hipMemcpyAsync(base + cap_q0 + m16 * kHidden * sec, q, m16 * K, hipMemcpyDeviceToDevice, s),
                  "capture q8");
        hip_check(hipMemcpyAsync(base + cap_d0 + 4 * m16 * (kHidden / 32) * sec, d, 4 * m16 * (K / 32),
                                 hipMemcpyDeviceToDevice, s),
                  "capture d8");
    };
    auto cap_copy_x = [&](int l, int sec) {
        if (!cap || l >= kLayers) return;
        hip_check(hipMemcpyAsync(cap_f(l, sec), pre_x_, sizeof(float) * m * kHidden, hipMemcpyDeviceToDevice, s),
                  "capture x");
    };
    cap_copy_x(0, 0);
    int8_t *q8 = a8 ? pre_q8_ : nullptr;
    float *d8 = a8 ? pre_d8_ : nullptr;
    auto operand = [&](GemmArgs &g) {
        if (a8) {  // written in the matrix-core order by the kernel before
            g.a8 = pre_q8_;
            g.d8 = pre_d8_;
            g.a8_tiled = true;
        }
    };
    // the GEMMs read their inputs in the matrix-core order, written so by the kernel
    // before: int8 + block scales under W8A8, fp16 hi / lo halves under A16
    uint8_t *a_hl = a8 ? nullptr : reinterpret_cast<uint8_t *>(pre_a_);
    uint8_t *h_hl = a8 ? nullptr : reinterpret_cast<uint8_t *>(pre_h_);
    hip_check(launch_ln_rows(pre_x_, kHidden, g_[0].ln1_w, g_[0].ln1_b, cap_f(0, 1), m, s, nullptr, q8, d8, a_hl),
              "prefill ln1");
    cap_copy_q(0, 0, pre_q8_, pre_d8_);
    const float *rc = rope_, *rs = rope_ + (size_t)rope_n_ * kRopeHalf;
    for (int l = 0; l < kLayers; ++l) {
        const LayerW &L = g_[l];
        GemmArgs q;
        q.w = L.attn_w; q.wm = L.attn_wm; q.N = 3 * kHidden; q.K = kHidden; q.a_hl = a_hl; q.lda = kHidden; q.M = m;
        q.bias = L.attn_b; q.q_out = pre_q_;
        q.k_pool = kv_layer(0, l); q.v_pool = kv_layer(1, l); q.page_size = max_ctx_;
        q.pos0 = start; q.rope_cos = rc; q.rope_sin = rs;
        operand(q);
        hip_check(launch_gemm(q, EPI_QKV, kvt_, s), "prefill qkv");
        AttnArgs t;
        t.q = pre_q_; t.k_pool = q.k_pool; t.v_pool = q.v_pool; t.page_size = max_ctx_;
        t.pos0 = start; t.rows = m; t.max_keys = start + m;
        t.out = cap_f(l, 2);
        // the attention applies proj itself: each head's tile writes split-K partial h (12
        // partials, reduced in head order with the bias and the residual below)
        t.proj_w = L.proj_wm ? L.proj_wm : L.proj_w; t.proj_tiled = L.proj_wm ? 1 : 0;
        t.proj_part = pre_part_; t.proj_a8 = a8 ? 1 : 0;
        if (cap) {  // the int8 operand, for the capture only
            t.q8 = q8; t.d8 = d8;
        }
        hip_check(launch_attn_tiles(t, kvt_, s), "prefill attention");
        cap_copy_q(l, 1, pre_q8_, pre_d8_);
        hip_check(launch_resid_ln_rows(pre_part_, kHeads, m, L.proj_b, pre_x_, kHidden, pre_x_, L.ln2_w, L.ln2_b,
                                       cap_f(l, 4), nullptr, s, q8, d8, a_hl),
                  "prefill attention + proj reduce + ln2");
        cap_copy_x(l, 3);
        cap_copy_q(l, 2, pre_q8_, pre_d8_);
        GemmArgs f1;
        f1.w = L.fc_in_w; f1.wm = L.fc_in_wm; f1.N = kFF; f1.K = kHidden; f1.a_hl = a_hl; f1.lda = kHidden; f1.M = m;
        f1.y_hl = h_hl; f1.bias = L.fc_in_b;
        operand(f1);
        if (a8) {  // fc_out's int8 operand, quantised in fc_in's epilogue
            f1.q8_out = pre_q8h_;
            f1.d8_out = pre_d8h_;
            f1.y = cap_f(l, 5);
            f1.ldy = kFF;
        }
        hip_check(launch_gemm(f1, EPI_GELU, kvt_, s), "prefill fc_in");
        cap_copy_q(l, 3, pre_q8h_, pre_d8h_);
        GemmArgs f2;
        f2.w = L.fc_out_w; f2.wm = L.fc_out_wm; f2.N = kHidden; f2.K = kFF; f2.a_hl = h_hl; f2.lda = kFF; f2.M = m;
        f2.part = pre_part_; f2.ksplit = gemm_ksplit(m, kHidden, kFF);
        // many rows: 4 slices of K = 3072 (6 blocks per wave instead of 24) measured faster
        // (256 rows: W8A8 0.668 -> 0.647 ms, A16 0.722 -> 0.696 ms)
        if (m >= 128) f2.ksplit = kPrefillFcOutSplit;
        if (a8) {
            f2.a8 = pre_q8h_;
            f2.d8 = pre_d8h_;
            f2.a8_tiled = true;
        }
        hip_check(launch_gemm(f2, EPI_PART, kvt_, s), "prefill fc_out");
        const bool last = l + 1 == kLayers;  // LN1 of the next layer rides on the reduce
        hip_check(launch_resid_ln_rows(pre_part_, f2.ksplit, m, L.fc_out_b, pre_x_, kHidden, pre_x_,
                                       last ? nullptr : g_[l + 1].ln1_w, last ? nullptr : g_[l + 1].ln1_b,
                                       cap_f(l + 1, 1), nullptr, s, last ? nullptr : q8, last ? nullptr : d8,
                                       last ? nullptr : a_hl),
                  "prefill fc_out reduce");
        cap_copy_x(l, 6);
        cap_copy_x(l + 1, 0);
        cap_copy_q(l + 1, 0, pre_q8_, pre_d8_);
    }
    hip_check(launch_layernorm(pre_x_ + (size_t)(m - 1) * kHidden, lnf_w_, lnf_b_, hidden_, nullptr, 0, s), "ln_f");
    if (cap) cap_pre_used_ = cap_lb * kLayers;
    pos_ = start + m;
    write_state_header();
    hip_check(hipStreamSynchronize(s), "sync");
}

int Model::generate(int max_frames, const moss_hip_sample_params &p, uint64_t seed, const int32_t *forced,
                    int n_forced, int32_t *out_rows, double *timing, float *logits_dump, float *gate_dump,
                    moss_hip_frame_cb cb, void *user) {
    if (forced && n_forced < max_frames) max_frames = n_forced;
    if (max_frames <= 0) return 0;
    const int cap = max_ctx_ + 1;  // frames beyond this cannot happen: pos reaches max_ctx first
    const int nf = max_frames < cap ? max_frames : cap;
    if (forced) {
        std::vector<int> codes((size_t)nf * kNVq);
        for (int f = 0; f < nf; ++f)
            for (int ch = 0; ch < kNVq; ++ch) {
                const int c = forced[(size_t)f * 17 + ch + 1];
                if (c < 0 || c >= kCodebook) throw Status(MOSS_HIP_EINVAL, "forced code out of range");
                codes[(size_t)f * kNVq + ch] = c;
            }
        hip_check(hipMemcpyAsync(forced_, codes.data(), codes.size() * sizeof(int), hipMemcpyHostToDevice, stream_),
                  "forced h2d");
    }
    hip_check(hipMemsetAsync(counts_, 0, sizeof(int) * kNVq * kCodebook, stream_), "counts clear");
    gate_rows_ = 0;
    hstate_->frame = 0;
    hstate_->stop = 0;
    hstate_->min_frames = p.min_frames;
    hstate_->forced_on = forced ? 1 : 0;
    hstate_->rep_penalty = p.repetition_penalty;
    hstate_->cfg = sample_cfg(p);
    rng_seed_host(seed, hstate_->rng);  // Rng rng; rng.seed(seed) (llm.cpp:638-639)
    write_state_header();
    clear_exchange();
    DevState start_state;  // the device state before L(0): where a recovery at frame 0 restarts
    hip_check(hipMemcpyAsync(&start_state, state_, sizeof(DevState), hipMemcpyDeviceToHost, stream_), "state d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");
    // a recovery switches this call to the per-operator path; the next call tries the fused one again
    struct FusedRestore {
        bool &flag;
        bool saved;
        ~FusedRestore() { flag = saved; }
    } fused_restore{fused_layers_, fused_layers_};

    // Frame f is two launches: its local half L(f), followed by the copy of the
    // decode state (codes, stop flag) into readback slot f & 1 and an event, then
    // its global step G(f) on the frame's codes.  The host waits for frame f's
    // state, runs on_frame(f), and only then enqueues L(f + 1) and G(f + 1) --
    // while G(f) still runs on the device, so the GPU does not wait for the host.
    // As in the reference's loop (llm.cpp:643-713), G(f) runs whatever on_frame(f)
    // does, and a cancel flag raised there stops the loop before frame f + 1.
    // A G(f) enqueued behind an L(f) that the end gate stopped is a no-op on the
    // device (every kernel tests state->stop first); the host does not count it.
    bool global_enq[2] = {false, false};
    int pos_next = pos_;  // position once every enqueued global step has run
    auto enqueue = [&](int f) {
        const int slot = f & 1;
        hipEvent_t *ev = ev_ + kEvPerSlot * slot;
        if (timing) hip_check(hipEventRecord(ev[kEvLocal0], stream_), "event");
        launch_frame_local(stream_, gate_dump != nullptr, hstate_->cfg.greedy != 0);
        if (timing) hip_check(hipEventRecord(ev[kEvLocal1], stream_), "event");
        if (logits_dump)
            hip_check(hipMemcpyAsync(logits_dump + (size_t)f * kNVq * kCodebook, logits_,
                                     sizeof(float) * kNVq * kCodebook, hipMemcpyDeviceToHost, stream_),
                      "logits d2h");
        hip_check(hipMemcpyAsync(hread_ + slot, state_, sizeof(DevState), hipMemcpyDeviceToHost, stream_),
                  "state d2h");
        hip_check(hipEventRecord(ev[kEvRead], stream_), "event");
        global_enq[slot] = f + 1 < max_frames && pos_next < max_ctx_;
        if (global_enq[slot]) {
            if (timing) hip_check(hipEventRecord(ev[kEvGlobal0], stream_), "event");
            launch_global(stream_);
            if (timing) hip_check(hipEventRecord(ev[kEvGlobal1], stream_), "event");
            ++pos_next;
        }
    };
    // FrameTiming of a frame whose global step has finished (llm.h:34-37)
    auto frame_timing = [&](int f) {
        const int slot = f & 1;
        const hipEvent_t *ev = ev_ + kEvPerSlot * slot;
        float lm = 0.f, gm = 0.f;
        hip_check(hipEventElapsedTime(&lm, ev[kEvLocal0], ev[kEvLocal1]), "elapsed");
        if (global_enq[slot]) hip_check(hipEventElapsedTime(&gm, ev[kEvGlobal0], ev[kEvGlobal1]), "elapsed");
        timing[2 * f] = gm;
        timing[2 * f + 1] = lm;
    };
    auto cancelled = [&] { return cancel_ != nullptr && __atomic_load_n(cancel_, __ATOMIC_RELAXED); };
    // Frame f's readback reports a fused launch whose wait ran out: L(f), or G(f - 1) whose hidden
    // state L(f) started from.  Frames 0 .. f - 1 are good.  Put the device back to the state
    // after L(f - 1) (read back then; the start of the call for f = 0) with the repetition counts
    // of frames 0 .. f - 1 (from their rows), redo G(f - 1) and enqueue frame f again -- all per
    // operator, which needs no co-resident workgroups.  G(f), enqueued behind the failed L(f), is
    // superseded: it wrote only the K/V row and hidden state that the new G(f) rewrites.
    auto recover = [&](int f) {
        hip_check(hipStreamSynchronize(stream_), "sync");
        ++fallbacks_;
        fallbacks_total.fetch_add(1, std::memory_order_relaxed);
        fused_layers_ = false;
        DevState st = f == 0 ? start_state : hread_[(f - 1) & 1];
        st.ll_err = 0;
        hip_check(hipMemcpyAsync(state_, &st, sizeof(DevState), hipMemcpyHostToDevice, stream_), "state h2d");
        std::vector<int> cnt((size_t)kNVq * kCodebook, 0);
        for (int g = 0; g < f; ++g)
            for (int ch = 0; ch < kNVq; ++ch) {
                const int used = forced ? forced[(size_t)g * 17 + ch + 1] : out_rows[(size_t)g * 17 + ch + 1];
                ++cnt[(size_t)ch * kCodebook + used];
            }
        hip_check(hipMemcpyAsync(counts_, cnt.data(), cnt.size() * sizeof(int), hipMemcpyHostToDevice, stream_),
                  "counts h2d");
        if (f > 0 && global_enq[(f - 1) & 1]) launch_global(stream_);
        if (global_enq[f & 1]) --pos_next;
        enqueue(f);
        hip_check(hipEventSynchronize(ev_[kEvPerSlot * (f & 1) + kEvRead]), "sync");
    };

    int frames = 0;
    if (pos_ < max_ctx_ && !cancelled()) {
        enqueue(0);
        for (int f = 0;; ++f) {
            const int slot = f & 1;
            hip_check(hipEventSynchronize(ev_[kEvPerSlot * slot + kEvRead]), "sync");
            if (hread_[slot].ll_err != 0) {  // the local half's or the previous global step's
                hstate_->ll_err = hread_[slot].ll_err;
                if (!fused_layers_ || !can_fall_back()) check_exchange();  // throws
                recover(f);
            }
            const DevState &hs = hread_[slot];
            hstate_->ll_err = hs.ll_err;
            check_exchange();
            if (timing && f > 0) frame_timing(f - 1);  // G(f - 1) ran before L(f)
            if (gate_dump) {
                float *gd = gate_dump + 4 * (size_t)f;
                gd[0] = hs.gate[0];
                gd[1] = hs.gate[1];
                gd[2] = (float)hs.gate_argmax;
                gd[3] = hs.gate_argmax_v;
                gate_rows_ = f + 1;
            }
            if (hs.stop) break;
            int32_t *row = out_rows + (size_t)f * 17;
            row[0] = 0;
            for (int ch = 0; ch < kNVq; ++ch) row[ch + 1] = hs.codes[ch];
            if (global_enq[slot]) ++pos_;
            frames = f + 1;
            if (cb) cb(user, f, row);
            if (!global_enq[slot] || pos_next >= max_ctx_ || cancelled()) break;  // last frame, full KV, cancel
            enqueue(f + 1);
        }
    }
    hip_check(hipMemcpyAsync(&hstate_->ll_err, &state_->ll_err, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
              "state d2h");
    hip_check(hipStreamSynchronize(stream_), "sync");  // the last global step has drained
    if (hstate_->ll_err != 0 && frames > 0 && global_enq[(frames - 1) & 1] && fused_layers_ && can_fall_back()) {
        // the last frame's global step ran out: redo it per operator from the state after its local half
        ++fallbacks_;
        fallbacks_total.fetch_add(1, std::memory_order_relaxed);
        fused_layers_ = false;
        DevState st = hread_[(frames - 1) & 1];
        st.ll_err = 0;
        hip_check(hipMemcpyAsync(state_, &st, sizeof(DevState), hipMemcpyHostToDevice, stream_), "state h2d");
        launch_global(stream_);
        hip_check(hipMemcpyAsync(&hstate_->ll_err, &state_->ll_err, sizeof(unsigned), hipMemcpyDeviceToHost, stream_),
                  "state d2h");
        hip_check(hipStreamSynchronize(stream_), "sync");
    }
    check_exchange();
    if (timing && frames > 0) frame_timing(frames - 1);
    return frames;
}

void Model::snapshot_prefix() {
    prefix_pos_ = pos_;
    if (snap_) {
        hip_check(hipFree(snap_), "free snapshot");
        snap_ = nullptr;
    }
    if (prefix_pos_ <= 0) return;
    const size_t width = (size_t)prefix_pos_ * kHeadDim * kv_esize_;
    hip_check(hipMalloc(&snap_, 2ull * kLayers * kHeads * width), "hipMalloc(snapshot)");
    for (int w = 0; w < 2; ++w)
        for (int l = 0; l < kLayers; ++l) {
            uint8_t *dst = static_cast<uint8_t *>(snap_) + ((size_t)w * kLayers + l) * kHeads * width;
            hip_check(hipMemcpy2DAsync(dst, width, kv_layer(w, l), (size_t)max_ctx_ * kHeadDim * kv_esize_, width,
                                       kHeads, hipMemcpyDeviceToDevice, stream_),
                      "snapshot copy");
        }
    hip_check(hipStreamSynchronize(stream_), "sync");
}

void Model::restore_prefix() {
    if (prefix_pos_ <= 0 || !snap_) {
        pos_ = 0;
        return;
    }
    const size_t width = (size_t)prefix_pos_ * kHeadDim * kv_esize_;
    for (int w = 0; w < 2; ++w)
        for (int l = 0; l < kLayers; ++l) {
            const uint8_t *src = static_cast<const uint8_t *>(snap_) + ((size_t)w * kLayers + l) * kHeads * width;
            hip_check(hipMemcpy2DAsync(kv_layer(w, l), (size_t)max_ctx_ * kHeadDim * kv_esize_, src, width, width,
                                       kHeads, hipMemcpyDeviceToDevice, stream_),
                      "restore copy");
        }
    hip_check(hipStreamSynchronize(stream_), "sync");
    pos_ = prefix_pos_;
}

void Model::kv_export(int n_pos, float *k, float *v) {
    if (n_pos < 0 || n_pos > max_ctx_) throw Status(MOSS_HIP_EINVAL, "n_pos out of range");
    if (n_pos == 0) return;
    float *stage = nullptr;
    const size_t per = (size_t)n_pos * kHidden;
    hip_check(hipMalloc(&stage, per * 4), "hipMalloc(stage)");
    try {
        for (int w = 0; w < 2; ++w)
            for (int l = 0; l < kLayers; ++l) {
                hip_check(launch_kv_export(kv_layer(w, l), n_pos, max_ctx_, kvt_, stage, stream_), "kv export");
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

void Model::kv_import(int n_pos, const float *k, const float *v, const float *hidden) {
    if (n_pos < 0 || n_pos > max_ctx_) throw Status(MOSS_HIP_EINVAL, "n_pos out of range");
    float *stage = nullptr;
    const size_t per = (size_t)n_pos * kHidden;
    if (n_pos > 0) {
        hip_check(hipMalloc(&stage, per * 4), "hipMalloc(stage)");
        try {
            for (int w = 0; w < 2; ++w)
                for (int l = 0; l < kLayers; ++l) {
                    hip_check(hipMemcpyAsync(stage, (w == 0 ? k : v) + (size_t)l * per, per * 4, hipMemcpyHostToDevice,
                                             stream_),
                              "kv h2d");
                    hip_check(launch_kv_import(stage, n_pos, kv_layer(w, l), max_ctx_, kvt_, stream_), "kv import");
                    hip_check(hipStreamSynchronize(stream_), "sync");
                }
        } catch (...) {
            (void)hipFree(stage);
            throw;
        }
        (void)hipFree(stage);
    }
    if (hidden) set_hidden(hidden);
    pos_ = n_pos;
}

}  // namespace mh
