// mh_ops.h -- host-side launchers of the gfx950 kernels (internal C++ API).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mh_device.h"

namespace mh {

// Activation source of a GEMV (what the kernel stages into LDS as fp32).
enum Prologue : int {
    PRO_F32 = 0,    // x: float[cols]
    PRO_F16 = 1,    // x: half[cols]
    PRO_LN = 2,     // x: float[768], LayerNorm(ln_w, ln_b) applied in the prologue
    PRO_LATTN = 3,  // x: q float[768]; the prologue computes the local attention of q over
                    // k_cache/v_cache (fp32 [12][ctx_stride][64], keys 0..pos_const)
    PRO_AMERGE = 4, // the prologue merges split-KV attention partials attn_part
                    // ([12][attn_splits][kPartStride]: o[64], m, l) over keys 0..*pos_ptr
    PRO_PICK = 5,   // greedy pick of channel pick_ch from pick_logits (repetition penalty from
                    // pick_counts), the used code (forced under teacher forcing) selects row
                    // `used` of pick_aemb, then LayerNorm(ln_w, ln_b); workgroup 0 records the
                    // pick in pick_state (codes, row)
};

// What happens to each output row.
enum Epilogue : int {
    EPI_F32 = 0,    // y[r] = acc                      (float)
    EPI_F16 = 1,    // y[r] = half(acc)                (half)
    EPI_QKV = 2,    // + bias, RoPE on q/k, q -> q_out, k/v -> KV cache at pos
    EPI_RESID = 3,  // y[r] = xin[r] + (acc + bias[r]), xin = resid_in or y (float)
    EPI_GELU = 4,   // y[r] = gelu_new(acc + bias[r])  (float)
    EPI_PART = 5,   // GEMM only: split-K partial sums, part[z][m][n] for K slice z (no bias)
};

enum KvType : int { KV_F16 = 0, KV_F32 = 1 };

struct GemvArgs {
    const uint8_t *w = nullptr;  // Q8_0_4X4 matrix, rows x cols
    int rows = 0, cols = 0;
    // prologue
    const void *x = nullptr;
    const float *ln_w = nullptr, *ln_b = nullptr;
    // epilogue
    void *y = nullptr;
    const float *resid_in = nullptr;  // EPI_RESID reads the residual from here (nullptr: from y)
    const float *bias = nullptr;
    float *q_out = nullptr;
    void *k_cache = nullptr, *v_cache = nullptr;  // [heads][ctx_stride][64]
    int ctx_stride = 0;
    const float *rope_cos = nullptr, *rope_sin = nullptr;  // [pos][32]
    // position (EPI_QKV, PRO_LATTN, PRO_AMERGE): *pos_ptr when non-null, else pos_const
    const int *pos_ptr = nullptr;
    int pos_const = 0;
    const float *attn_part = nullptr;  // PRO_AMERGE partials
    int attn_splits = 0;
    const float *pick_logits = nullptr;  // PRO_PICK: [1024] logits of channel pick_ch
    const int *pick_counts = nullptr;    // [1024] used-code counts of that channel
    const uint8_t *pick_aemb = nullptr;  // aemb[pick_ch]
    const int *pick_forced = nullptr;    // [frames][16] teacher-forcing codes
    int pick_ch = 0;
    DevState *pick_state = nullptr;
    float *pick_raw = nullptr;  // workgroup 0 stores the picked aemb row (the step's residual input)
    const DevState *state = nullptr;  // when non-null, the kernel is a no-op once state->stop is set
    int a8 = 0;  // W8A8: the staged activation quantised per 32-block (decode prologues only)
};

// Launch y = W x with the given prologue/epilogue; kv selects the KV cache type for EPI_QKV.
hipError_t launch_gemv(const GemvArgs &a, Prologue pro, Epilogue epi, KvType kv, hipStream_t s);

// Attention over one query row per (head, row) workgroup.  Keys of row r live in
// stream s = row_stream[r] (0 when null); key p of stream s is at page
// page_table[s * table_stride + p / page_size], slot p % page_size, in
// pools laid out [page][head][page_size][64].  A null page_table means one
// contiguous page per stream (page = stream index).  page_size must be a
// multiple of 64 or exceed every key count.
struct AttnArgs {
    const float *q = nullptr;  // row r: q + r * q_stride, [heads*64] fp32 (post-RoPE)
    int q_stride = kHidden;
    const void *k_pool = nullptr, *v_pool = nullptr;
    const int *page_table = nullptr;
    int table_stride = 0, page_size = 0;
    int heads = kHeads;
    const int *row_stream = nullptr;  // stream of row r (r * stream_stride when null)
    int stream_stride = 0;
    const int *row_pos = nullptr;  // keys of row r = row_pos[r] + 1 (pos0 + r * pos_stride + 1 when null)
    int pos0 = 0, pos_stride = 1;
    int rows = 1;
    // workgroups (blockIdx.y) take the rows in this order when set (the batch engine passes its
    // streams longest context first, so the longest rows start first and share no CU round
    // with each other); row y when null.  Rows of one launch, not split-KV or sliced launches.
    const int *row_order = nullptr;
    int max_keys = 0;              // key capacity: sizes the launch and caps every row's key count
    void *out = nullptr;           // row r: out + r * out_stride
    int out_stride = kHidden;
    int out_f16 = 0;               // out is half (else float)
    // split-KV output (single row only): workgroup (h, s) writes the unnormalised partial of
    // keys [64 s, 64 s + 64) to part[(h * splits + s) * kPartStride]: o[64], running max m,
    // sum l; splits = ceil(max_keys / 64).  A consumer merges them (PRO_AMERGE).
    float *part = nullptr;
    // optional W8A8 copy of the (normalised) output rows: int8 + block scales in the
    // matrix-core order (q8t_at / d8t_at, rows padded to 16)
    int8_t *q8 = nullptr;
    float *d8 = nullptr;
    // the output as hi / lo halves in the matrix-core order (hlt_at, rows padded to 16)
    // for the next GEMM's a_hl, instead of out (no split-KV or sliced launches)
    uint8_t *out_hl = nullptr;
    const DevState *state = nullptr;
    // prefill tiles (launch_attn_tiles): proj applied to the tile's output in the same launch.
    // proj_w is the proj matrix (768 x 768), in the matrix-core order (544-byte units) when
    // proj_tiled, else Q8_0_4X4; head h's 64 columns of it times the head's output give
    // split-K partial h, written to proj_part[(h * rows + m) * 768 + n] -- the reduce that
    // follows sums the 12 partials in head order.  Under W8A8 (proj_a8) the operand is the
    // output quantised per 32-block (the int8 copy q8 / d8 holds), else its fp16 hi / lo halves.
    const uint8_t *proj_w = nullptr;
    int proj_tiled = 0;
    float *proj_part = nullptr;
    int proj_a8 = 0;
    // single row, long context: the keys are cut into `chunks` slices of 64 * chunk_waves
    // keys (one workgroup of chunk_waves waves each, one 64-key span per wave, more spans
    // per wave past kMaxChunks); slices 1.. write their partial
    // (o[64], m, l) as LL words to chunk_part[(h * chunks + c) * kPartStride], and slice 0 of
    // each head waits for them, merges all in slice order and writes the output.  The words
    // carry a tag made from the launch generation chunk_gen[0], which every workgroup reads at
    // its start; chunk_gen[1] counts the workgroups that are done, and the last of a launch
    // resets it and bumps the generation -- so consecutive launches on a scratch block (graph
    // replays included) never share a tag, and a partial left by a launch whose merge gave up
    // is never read as current.  Both words start at zero.
    int chunks = 0;
    int chunk_waves = 4;  // 2 or 4
    uint64_t *chunk_part = nullptr;
    uint32_t *chunk_gen = nullptr;
};
// Bytes of a sliced-attention scratch block for `heads` heads: a 256-byte header (the
// generation and arrival words) followed by the partials [heads][kMaxChunks][kPartStride].
constexpr size_t kChunkHeader = 256;
constexpr int kPartStride = 68;
constexpr int kMaxChunks = 64;
constexpr size_t chunk_scratch_bytes(int heads) {
    return kChunkHeader + sizeof(uint64_t) * (size_t)heads * kMaxChunks * kPartStride;
}
#ifndef MH_ONE_WG_SPANS
#define MH_ONE_WG_SPANS 8
#endif
// single-row attention: the keys stay in one workgroup up to kOneWgSpans 64-key spans;
// past that, slices of slice_waves(spans) waves (one span each), about 8 slices per head
constexpr int kOneWgSpans = MH_ONE_WG_SPANS;
constexpr int slice_waves(int spans) { return spans <= 16 ? 2 : 4; }
hipError_t launch_attn(const AttnArgs &a, KvType kv, hipStream_t s);
// The prefill's form on the matrix cores: 16 rows x one head per workgroup, rows r at
// positions pos0 + r of one cache page (no page table, per-row positions or split output).
hipError_t launch_attn_tiles(const AttnArgs &a, KvType kv, hipStream_t s);

// W8A16 GEMM on the matrix cores: Y[M][N] = A[M][K] W[N][K]^T with an epilogue.
struct GemmArgs {
    const uint8_t *w = nullptr;  // Q8_0_4X4, N x K
    const uint8_t *wm = nullptr; // the same weights in the matrix-core order (tile_q8x4_mfma), read instead of w when set
    int N = 0, K = 0;
    const float *a = nullptr;    // fp32 activations [M][lda]
    int lda = 0, M = 0;
    float *y = nullptr;          // EPI_F32 / EPI_RESID / EPI_GELU output [M][ldy]
    int ldy = 0;
    const float *resid_in = nullptr;  // EPI_RESID: y = resid_in[m*resid_stride + n] + (acc + bias) (y itself when null)
    int resid_stride = 0;
    const float *bias = nullptr;
    // EPI_QKV: q -> q_out[M][768]; k, v -> pages (same addressing as AttnArgs)
    float *q_out = nullptr;
    void *k_pool = nullptr, *v_pool = nullptr;
    const int *page_table = nullptr;
    int table_stride = 0, page_size = 0;
    const int *row_stream = nullptr;  // stream of row m (m * stream_stride when null)
    int stream_stride = 0;
    const int *row_pos = nullptr;     // position of row m (pos0 + m * pos_stride when null)
    int pos0 = 0, pos_stride = 1;
    const unsigned char *row_active = nullptr;  // rows with row_active[m] == 0 write no K/V
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    // EPI_PART: K is cut into ksplit slices of whole blocks (grid z); slice z writes
    // part + z * M * N (row-major [M][N]).  ksplit <= 0 picks a split from the shape.
    float *part = nullptr;
    int ksplit = 0;
    // W8A8 (reference gemv_avx2.cpp:105-121 per block): when a8 is non-null the activations are
    // int8 a8[M][lda] with fp32 block scales d8[M][lda / 32], and `a` is unused;
    // a8_tiled: a8 / d8 are in the matrix-core order instead (q8t_at / d8t_at with K = lda)
    const int8_t *a8 = nullptr;
    const float *d8 = nullptr;
    bool a8_tiled = false;
    // fp32 activations already split into fp16 hi / lo halves in the matrix-core order
    // (hlt_at with K = lda, rows padded to 16): read instead of `a` when set
    const uint8_t *a_hl = nullptr;
    // EPI_GELU: the output as hi / lo halves in that order (for the next GEMM's a_hl)
    // instead of fp32 rows in y; EPI_RESID: in addition to y
    uint8_t *y_hl = nullptr;
    // EPI_RESID, N = 768: for every stored row m and 16-column group j, the group's mean and
    // sum of squared deviations at y_stats[2 * (j * M + m)] -- the next LayerNorm's row
    // statistics, combined in a fixed order by the GEMM that reads them (ln_stats)
    float *y_stats = nullptr;
    // with a_hl and ln_w (EPI_GELU, EPI_QKV, EPI_F32; K = 768): LN of the pre-split rows, the
    // rows' statistics combined from ln_stats (a producer's y_stats) instead of formed from the rows
    const float *ln_stats = nullptr;
    // LayerNorm prologue: the GEMM multiplies LN(a_row) = (a - mean) * inv * ln_w + ln_b
    // (llm.cpp:159-171) when ln_w is non-null -- over fp32 rows `a` (K <= 1024, no K
    // split), or over pre-split rows a_hl with the statistics from ln_stats
    const float *ln_w = nullptr, *ln_b = nullptr;
    // EPI_GELU with q8_out (16*NT >= 32 columns per tile; y may then be null: no fp32 rows): the stored rows are also quantised
    // per 32-block (quantize_activation, quant.cpp:45) into q8_out / d8_out in the matrix-core
    // order (q8t_at / d8t_at with K = N, rows padded to 16)
    int8_t *q8_out = nullptr;
    float *d8_out = nullptr;
    // EPI_F32 with pick_pairs (N % 16 == 0): for every stored row m and 16-column group j,
    // the greedy pick's partial -- the group's largest value under the repetition penalty
    // (applied pick_counts[m * pick_stride + n] times, v < 0 ? v * p : v / p, p = *pick_pen)
    // and its column, the lowest on ties (-inf and N when none can win) -- as the float
    // pair pick_pairs[2 * (m * N / 16 + j)] (the column's int bits second)
    float *pick_pairs = nullptr;
    const int *pick_counts = nullptr;
    int pick_stride = 0;
    const float *pick_pen = nullptr;
};
hipError_t launch_gemm(const GemmArgs &g, Epilogue epi, KvType kv, hipStream_t s);
// Copy of a Q8_0_4X4 N x K matrix in the matrix-core order the GEMM reads through
// GemmArgs::wm (same size: N/16 * K/32 units of 544 bytes).
hipError_t tile_q8x4_mfma(const uint8_t *w, int N, int K, uint8_t *out, hipStream_t s);
// The K split launch_gemm uses for an EPI_PART GEMM of this shape (1..16).
int gemm_ksplit(int M, int N, int K);

// Deterministic split-K reduce + residual (+ LayerNorm), one workgroup per row:
//   x[m][n]   = resid[m * resid_stride + n] + ((sum_z part[z][m][n]) + bias[n])   (z in order)
//   out[m][:] = LayerNorm(x[m][:]; ln_w, ln_b) when ln_w is non-null; rows with mask[m] == 0 keep
//   their out row.  resid may alias x (in-place residual stream).  N == 768.
hipError_t launch_resid_ln_rows(const float *part, int ksplit, int rows, const float *bias, const float *resid,
                                int resid_stride, float *x, const float *ln_w, const float *ln_b, float *out,
                                const unsigned char *mask, hipStream_t s, int8_t *q8 = nullptr, float *d8 = nullptr,
                                uint8_t *out_hl = nullptr);
// (q8 / d8 of launch_resid_ln_rows and launch_ln_rows: the W8A8 copy of out in the
// matrix-core order, q8t_at / d8t_at, rows padded to 16; out_hl: out as hi / lo halves in
// that order (hlt_at) instead of fp32 rows; out may be null when q8 or out_hl is set)

// W8A8 activation quantisation of rows (quant.cpp:28-54): q8[r][K] int8 and d8[r][K/32]
// fp32 block scales from x[r * x_stride + k].  K % 256 == 0.
hipError_t launch_quant_rows(const float *x, int x_stride, int K, int rows, int8_t *q8, float *d8, hipStream_t s);

// ---- frame / step kernels (frame_ops.hip)
struct EmbedArgs {
    const uint8_t *wte = nullptr;
    const uint8_t *aemb[kNVq] = {};
    const int *row = nullptr;  // [17] on device
    float *x = nullptr;        // [768] out
    const DevState *state = nullptr;
};
hipError_t launch_embed(const EmbedArgs &a, hipStream_t s);

// out = LayerNorm(x); when bump_pos, state->pos += 1 afterwards (end of a global step).
hipError_t launch_layernorm(const float *x, const float *w, const float *b, float *out, DevState *state,
                            int bump_pos, hipStream_t s);

// Dequantise `n` rows (device indices) of a mat_rows x cols Q8_0_4X4 matrix into out[n][cols].
hipError_t launch_dequant_rows(const uint8_t *w, int mat_rows, int cols, const int *rows_dev, int n, float *out,
                               hipStream_t s);

// End gate: LN(x; lnf) -> W8A8 dot with wte rows 7 and 9 (reference order) -> state->gate, state->stop.
hipError_t launch_gate(const float *x_raw, const float *lnf_w, const float *lnf_b, const uint8_t *wte,
                       DevState *state, hipStream_t s);
// End gate from the full text-head logits[16384] (gate-dump frames): gate, argmax, stop.
hipError_t launch_gate_text(const float *logits, DevState *state, hipStream_t s);

// Pick for channel ch: repetition penalty from counts, greedy or sampled choice,
// history update, next input = dequant(aemb[ch][used]).
struct SampleArgs {
    const float *logits = nullptr;  // [1024]
    int ch = 0;
    int *counts = nullptr;          // [16][1024] occurrences of each used code in this generate()
    const int *forced = nullptr;    // [frames][16] (used when state->forced_on)
    const uint8_t *aemb = nullptr;  // aemb[ch]
    float *next_input = nullptr;    // [768]
    DevState *state = nullptr;
    int last_channel = 0;           // ch == 15: advance state->frame
    int count_all = 0;              // also count the used codes of channels 0..14 (state->row), whose
                                    // picks ran in GEMV prologues that deferred their counting
};
hipError_t launch_sample(const SampleArgs &a, hipStream_t s);

// Rng::seed of the reference (csrc/include/moss/sampler.h:28-35), on the host.
inline void rng_seed_host(uint64_t v, uint32_t s[4]) {
    s[0] = (uint32_t)v;
    s[1] = (uint32_t)(v >> 32) ^ 0x9E3779B9u;
    s[2] = 0x243F6A88u;
    s[3] = 0xB7E15162u;
    for (int i = 0; i < 8; ++i) {
        const uint32_t t = s[1] << 9;
        s[2] ^= s[0];
        s[3] ^= s[1];
        s[1] ^= s[2];
        s[0] ^= s[3];
        s[2] ^= t;
        s[3] = (s[3] << 11) | (s[3] >> 21);
    }
}

// ---- row-batched kernels (prefill rows or one row per stream)
// out[r] = LayerNorm(x[r * x_stride]) for r < rows (x_stride 0 broadcasts one row);
// rows with mask[r] == 0 are left untouched when mask is non-null.
hipError_t launch_ln_rows(const float *x, int x_stride, const float *w, const float *b, float *out, int rows,
                          hipStream_t s, const unsigned char *mask = nullptr, int8_t *q8 = nullptr,
                          float *d8 = nullptr, uint8_t *out_hl = nullptr);
// x[r] = embedding of rows[r][17] (llm.cpp:148-157)
hipError_t launch_embed_rows(const EmbedArgs &e, const int *rows, int n, float *x, hipStream_t s);

// Controls of one batched generate() call, shared by all streams; device-side
// so the captured graphs stay valid from call to call.
struct BatchCtl {
    int frame;          // frame index of the current generate call
    int min_frames;     // SampleParams::min_frames
    float rep_penalty;  // SampleParams::repetition_penalty
    SampleCfg cfg;
};

// Per-stream decode state of the batched engine (device arrays of `streams` entries).
struct StreamState {
    int *pos = nullptr;            // next global position
    unsigned char *active = nullptr;  // 1 while the stream decodes (cleared by the gate / capacity)
    int *codes = nullptr;          // [S][16] predicted codes of the frame
    int *row = nullptr;            // [S][17] next global-step row
    float *gate = nullptr;         // [S][2] (l_end, l_slot)
    int *counts = nullptr;         // [S][16][1024] used-code occurrences (repetition penalty)
    uint32_t *rng = nullptr;       // [S][4] xoshiro128** state per stream
    BatchCtl *ctrl = nullptr;
    int capacity = 0;              // KV positions per stream
};
// End gate per stream (gate_kernel on each row); inactive streams are left alone.
hipError_t launch_gate_rows(const float *x_raw, const float *lnf_w, const float *lnf_b, const uint8_t *wte,
                            const StreamState &st, int streams, hipStream_t s);
// Pick per stream for channel ch over logits[S][1024] (greedy or sampled, as the
// single-stream sample kernel); next_in[S][768] = aemb[ch][used].
// q|k|v of the next local position taken from the load-time table (rows of
// (position, input code)): q into q_out[S][768], k and v into the local caches
// [S][12][17][64] at lpos.  The sampler writes them for the code it picks.
struct LocalQkv {
    const float *rows = nullptr;  // table rows of this position's input channel: [1024][2304] (or one row)
    float *q_out = nullptr;
    float *lk = nullptr, *lv = nullptr;
    int lpos = 0;
};
hipError_t launch_sample_rows(const float *logits, int ch, const uint8_t *aemb, float *next_in, const StreamState &st,
                              int streams, int last_channel, const LocalQkv &next, hipStream_t s, int count_prev = 0);
// Greedy frames: channel ch's pick fused with local position lpos = ch + 2's table row and
// attention, one workgroup per (head, stream); the pick's count is added by the next launch.
struct PickAttnArgs {
    const float *logits = nullptr;  // [S][1024] logits of channel ch
    int ch = 0;
    const uint8_t *aemb = nullptr;  // aemb[ch]: the next residual input's row
    float *next_in = nullptr;       // [S][768]
    StreamState st;
    const float *rows = nullptr;    // q|k|v table rows of channel ch's inputs at lpos: [1024][2304]
    float *lk = nullptr, *lv = nullptr;  // local KV [S][heads][17][64] (fp32)
    int lpos = 0;
    float *o = nullptr;             // [S][768] attention output
    uint8_t *o_hl = nullptr;        // or the output as hi / lo halves (hlt_at, rows padded to 16)
    int8_t *o_q8 = nullptr;         // and / or its W8A8 copy in the matrix-core order (q8t_at / d8t_at)
    float *o_d8 = nullptr;
    // greedy: the head GEMM's per-16-code partials of channel ch ([S][64] pairs,
    // GemmArgs::pick_pairs) instead of the logits and counts
    const float *pairs = nullptr;
};
hipError_t launch_local_pick_attn(const PickAttnArgs &a, int streams, hipStream_t s);
// The same copy of one shared row (lpos 1: wte[slot]) for every stream.
hipError_t launch_local_qkv_rows(const LocalQkv &a, int streams, hipStream_t s);
// pos[s] += 1 for active streams; streams reaching capacity become inactive.
hipError_t launch_advance_rows(const StreamState &st, int streams, hipStream_t s);

// KV import/export between the reference layout [n][768] fp32 of one layer and the
// device layout [heads][ctx_stride][64] (fp16 or fp32).
hipError_t launch_kv_import(const float *src, int n_pos, void *dst, int ctx_stride, KvType kv, hipStream_t s);
// Same into pages: position p -> page table_row[p / page_size], slot p % page_size of [page][head][page_size][64].
hipError_t launch_kv_import_paged(const float *src, int n_pos, void *pool, const int *table_row, int page_size,
                                  KvType kv, hipStream_t s);
hipError_t launch_kv_export_paged(const void *pool, const int *table_row, int page_size, int n_pos, KvType kv,
                                  float *dst, hipStream_t s);
hipError_t launch_kv_export(const void *src, int n_pos, int ctx_stride, KvType kv, float *dst, hipStream_t s);
// Device to device, every layer's K and V: positions [0, n_pos) of a contiguous cache
// ([layer][head][ctx_stride][64], layer l of K at k_src + l * src_layer_elems) into the pages
// of one stream (layer l of K at k_pool + l * pool_layer_elems), converted from src_kv to
// pool_kv (fp32 -> fp16 rounds to nearest even, as launch_kv_import_paged does).
struct KvAdmit {
    const void *k_src = nullptr, *v_src = nullptr;
    size_t src_layer_elems = 0;
    int ctx_stride = 0;
    KvType src_kv = KV_F16;
    void *k_pool = nullptr, *v_pool = nullptr;
    size_t pool_layer_elems = 0;
    const int *table_row = nullptr;
    int page_size = 0;
    KvType pool_kv = KV_F16;
};
hipError_t launch_kv_admit(const KvAdmit &a, int n_pos, hipStream_t s);

// ---- one transformer block of the single-stream decode in one launch (decode_layer.hip)
constexpr int kLayerGrid = 192;          // workgroups, one per CU; all resident at once
constexpr int kLayerMaxQuarters = 4;     // attention workgroups per head (4 spans of 64 keys each)
constexpr int kLayerWords = 3 * kHidden + kHeads * kLayerMaxQuarters * 66 + kHidden + kFF + kHidden;  // LL words
struct LayerArgs {
    const uint8_t *attn_w = nullptr, *proj_w = nullptr, *fc_in_w = nullptr, *fc_out_w = nullptr;
    const float *attn_b = nullptr, *proj_b = nullptr, *fc_in_b = nullptr, *fc_out_b = nullptr;
    const float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
    void *k_cache = nullptr, *v_cache = nullptr;  // this layer's [head][ctx_stride][64]
    int ctx_stride = 0;
    const float *rope_cos = nullptr, *rope_sin = nullptr;
};
// Whether kLayerGrid workgroups of every fused decode kernel fit the device at once.
hipError_t decode_layer_fits(int device, bool *fits);
// The whole global step in one launch: embedding of the row, kLayers blocks, ln_f.
struct GlobalArgs {
    const LayerArgs *layers = nullptr;  // kLayers entries in device memory
    const uint8_t *wte = nullptr;
    const uint8_t *aemb[kNVq] = {};
    const int *row = nullptr;           // [17] on device
    const float *lnf_w = nullptr, *lnf_b = nullptr;
    float *hidden = nullptr;            // [768] out: ln_f of the last block's output
    DevState *state = nullptr;          // pos (read, then bumped by workgroup 0), stop
    uint64_t *ll = nullptr;             // kLayerWords exchange words
    unsigned *err = nullptr;            // set when a wait runs out
    int a8 = 0;                         // W8A8 GEMVs (activations quantised per 32-block), else W8A16
    int poll_budget = 0;                // poll rounds a wait may take before it gives up (kPollBudget)
    float *cap = nullptr;               // W8A8 only: quantiser capture [kLayers][MOSS_HIP_CAP_STEP] (tests)
};
hipError_t launch_decode_global(const GlobalArgs &a, KvType kv, hipStream_t s);

// ---- one local-transformer step (+ the channel's audio head) in one launch (decode_local.hip)
struct LocalArgs {
    const uint8_t *attn_w = nullptr, *proj_w = nullptr, *fc_in_w = nullptr, *fc_out_w = nullptr;
    const float *attn_b = nullptr, *proj_b = nullptr, *fc_in_b = nullptr, *fc_out_b = nullptr;
    const float *ln1_w = nullptr, *ln1_b = nullptr, *ln2_w = nullptr, *ln2_b = nullptr;
    const float *lnf_w = nullptr, *lnf_b = nullptr;  // local ln_f (head input)
    float *lk = nullptr, *lv = nullptr;              // local cache [12][17][64] fp32
    const float *rope_cos = nullptr, *rope_sin = nullptr;
    DevState *state = nullptr;
    uint64_t *ll = nullptr;
    unsigned *err = nullptr;
    int lpos = 0;                      // first local position of the launch
    int lpos_last = 0;                 // last one (positions 1..16 may run as one chain)
    const float *x_in = nullptr;       // lpos 0: block input (the global hidden state; QKV computed here)
    const float *x_slot = nullptr;     // lpos 1: the raw input row (dequantised wte[slot])
    const float *qkv_table = nullptr;  // [1 + 15 * 1024][2304]: row 0 for lpos 1, then (lpos, code) rows
    const uint8_t *aemb[kNVq] = {};    // audio embeddings / tied heads
    int pick = 0;                      // 1: greedy pick of the previous channel here; 0: the sampler wrote state->row
    int head = 0;                      // 1: position lpos >= 1 also runs the audio head of channel lpos - 1
    float *logits = nullptr;           // [16][1024] head outputs (channel ch at ch * 1024)
    int *counts = nullptr;             // [16][1024] repetition counts (the final pick adds the frame's codes)
    const int *forced = nullptr;
    float *x_out = nullptr;            // block output (768)
    int gate = 0;                      // 1: after position 0, the W8A8 end gate (wte rows 7, 9); a stop ends the launch
    const uint8_t *wte = nullptr;
    int final_pick = 0;                // 1: after the last position, the greedy pick of its channel, the
                                       // frame's code counts, row[0] = slot and frame + 1 (sample_kernel's work)
    int a8 = 0;                        // W8A8 GEMVs (activations quantised per 32-block), else W8A16
    int poll_budget = 0;               // poll rounds a wait may take before it gives up (kPollBudget)
    float *cap = nullptr;              // W8A8 only: quantiser capture [kLocalLen][MOSS_HIP_CAP_STEP] (tests)
};
hipError_t decode_local_occupancy(int *per_cu);
hipError_t launch_decode_local(const LocalArgs &a, hipStream_t s);

}  // namespace mh
