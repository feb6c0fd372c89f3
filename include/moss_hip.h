/*
 * moss_hip.h -- C ABI of libmoss_hip.so, the MI355X (gfx950) backend of the
 * MOSS-TTS-Nano LLM decode path.
 *
 * Two layers, both plain C (no C++ types, no exceptions cross this boundary):
 *
 *  1. Model layer (moss_hip_llm_*): the GPU replacement of moss::LlmModel
 *     (reference csrc/include/moss/llm.h:39-90).  Host pointers in, host
 *     pointers out; the library owns the weights, the KV cache and the decode
 *     state on the device.  A C++ class with LlmModel's public surface sits on
 *     top of these calls (dsh-moss-tts_amd/host/moss/llm.h, host/llm_hip.cpp).
 *  2. Operator layer (moss_hip_gemv_q8x4, moss_hip_attn_decode, ...): the hot
 *     kernels on caller-owned device memory, for tests and benchmarks.  Every
 *     pointer argument is a device pointer; `stream` is a hipStream_t (NULL =
 *     the default stream).
 *
 * Conventions (mirroring csrc/include/moss/tts.h:10-41): every int-returning
 * call returns MOSS_HIP_OK (0) on success, non-zero on failure; the reason is
 * available from moss_hip_last_error() on the calling thread.  A model handle
 * is not thread-safe; calls on it must be serialised (the reference engine
 * calls prefill on its caller thread and generate on a producer thread, never
 * concurrently, csrc/src/engine.cpp:460-470).  Every model call makes the
 * model's device current and uses the model's own stream.
 */
#ifndef MOSS_HIP_H
#define MOSS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOSS_HIP_ABI_VERSION 8

enum {
    MOSS_HIP_OK = 0,
    MOSS_HIP_EINVAL = 1,       /* bad argument */
    MOSS_HIP_EDEVICE = 2,      /* HIP runtime failure */
    MOSS_HIP_EFORMAT = 3,      /* malformed .moss / missing tensor */
    MOSS_HIP_EUNSUPPORTED = 4, /* valid request this build does not implement */
    MOSS_HIP_ESTATE = 5        /* call not valid in the model's current state */
};

/* Last error message of this thread (cf. moss_last_error, csrc/include/moss/tts.h:40). */
const char *moss_hip_last_error(void);
int moss_hip_abi_version(void);

/* ------------------------------------------------------------------ model layer */

typedef struct moss_hip_llm moss_hip_llm;

typedef struct {
    int device;     /* HIP device ordinal */
    int max_ctx;    /* KV capacity in positions; 0 = 768 (kMaxCtx, csrc/include/moss/llm.h:28) */
    int kv_dtype;   /* 0 = fp16 KV cache (default), 1 = fp32 KV cache (the reference's own precision) */
    int use_graphs; /* 1 = replay the global step and the frame as hipGraphs (default), 0 = direct launches */
    int prefill_a16; /* prefill activations: 0 = W8A8, int8 per 32-block (the reference's prefill unless
                        MOSS_A16 is 1/all, csrc/src/gemv.cpp:23-48, llm.cpp:319-328); 1 = W8A16 fp32 */
    int decode_kernels; /* single-stream decode: 0 = fused kernels (default, when the device holds every
                           workgroup of a launch at once): the whole global step is one launch, and the
                           local half of a greedy frame (17 local steps, 16 audio heads, the end gate)
                           another; 1 = one launch per operator (GEMV / attention / head), replayed as
                           hipGraphs.  Both follow the reference's arithmetic per value; they differ in
                           fp32 summation order only. */
    int decode_a8;  /* decode activations (csrc/src/gemv.cpp:23-48, 229-274): 0 = W8A16, fp32 activations
                       (the reference with MOSS_A16=decode/1/all, the release setting); 1 = W8A8, each decode
                       GEMV's input quantised per 32-block (quantize_activation, quant.cpp:45) and the
                       int8 row dot of row_dot_q8_4x4 (gemv_avx2.cpp:105-121) -- the reference's default,
                       MOSS_A16 unset.  The end gate is W8A8 in both (llm.cpp:274-315). */
} moss_hip_llm_options;

/* SampleParams (csrc/include/moss/sampler.h:8-22), field for field. */
typedef struct {
    int greedy;
    float temperature;
    int top_k;
    float top_p;
    float repetition_penalty;
    int end_greedy;
    int min_frames;
    int greedy_frames;
} moss_hip_sample_params;

/* on_frame callback of LlmModel::generate (llm.h:74-77): frame index and its row. */
typedef void (*moss_hip_frame_cb)(void *user, int frame, const int32_t row[17]);

/* LlmModel::LlmModel + LlmModel::load (llm.h:41-43, csrc/src/llm.cpp:59-110): parses a
 * .moss v1 blob (csrc/src/weights.cpp:27-125), uploads it once to HBM, allocates the
 * KV cache and the decode state.  opt may be NULL (defaults).  Only Q8_0_4X4 matrices
 * are accepted (the release format, scripts/model_lock.json). */
int moss_hip_llm_create(const void *moss_blob, size_t bytes, const moss_hip_llm_options *opt,
                        moss_hip_llm **out);
int moss_hip_llm_create_from_file(const char *path, const moss_hip_llm_options *opt, moss_hip_llm **out);
void moss_hip_llm_destroy(moss_hip_llm *m);

int moss_hip_llm_reset(moss_hip_llm *m);              /* LlmModel::reset, llm.h:46 */
int moss_hip_llm_position(const moss_hip_llm *m);     /* LlmModel::position, llm.h:89 */
int moss_hip_llm_get_hidden(moss_hip_llm *m, float *out768); /* LlmModel::hidden, llm.h:88 */
int moss_hip_llm_set_hidden(moss_hip_llm *m, const float *in768);

/* LlmModel::prefill (llm.h:50, llm.cpp:327-401): rows [n_rows][17], from `start`.
 * W8A8 (activations quantised per 32-block, as the reference's default prefill) unless
 * opt->prefill_a16 (W8A16, the reference with MOSS_A16=1/all). */
int moss_hip_llm_prefill(moss_hip_llm *m, const int32_t *rows, int n_rows, int start);

/* LlmModel::global_step (llm.cpp:248-255): embed row -> 12 layers -> ln_f -> hidden; pos += 1. */
int moss_hip_llm_global_step(moss_hip_llm *m, const int32_t *row17);

/* LlmModel::generate (llm.h:74-77, llm.cpp:634-733).
 *   forced   [n_forced][17] teacher-forcing rows or NULL; max_frames is clamped to n_forced.
 *   out_rows [max_frames][17] receives the predicted rows; *out_frames their count.
 *   timing   [max_frames][2] (global_ms, local_ms) or NULL (FrameTiming, llm.h:34-37).
 *   logits_dump [max_frames][16][1024] or NULL (set_logits_dump, llm.h:80).
 *   gate_dump   [max_frames][4] (l_end, l_slot, argmax_id, argmax_logit) or NULL (set_gate_dump,
 *               llm.h:83).  As in the reference (llm.cpp:653-679), a dumped frame computes the whole
 *               16384-row text head and takes the gate logits from it instead of the 2-row W8A8 gate.
 *   cb/user: on_frame.  Every SampleParams mode runs on the device (sampler.cpp:9-79,
 *   llm.cpp:30-35): greedy, temperature / top-k / top-p sampling and the sampled end gate,
 *   drawing from xoshiro128** seeded with `seed` in the reference's order. */
int moss_hip_llm_generate(moss_hip_llm *m, int max_frames, const moss_hip_sample_params *p, uint64_t seed,
                          const int32_t *forced, int n_forced, int32_t *out_rows, int *out_frames, double *timing,
                          float *logits_dump, float *gate_dump, moss_hip_frame_cb cb, void *user);

/* Rows of gate_dump the last moss_hip_llm_generate filled: one per frame whose end gate was
 * evaluated -- the frames it returned, plus the frame the gate stopped (the rows the reference
 * writes to its gate CSV, llm.cpp:653-679,721-731); 0 when it was called without gate_dump. */
int moss_hip_llm_gate_rows(const moss_hip_llm *m);

/* Fused decode launches this model has redone on the per-operator path.  The fused kernels
 * (decode_kernels = 0) need every workgroup of a launch resident at once; when one of their
 * bounded waits runs out (another stream or process held CUs), the step is redone per
 * operator from the last good state and the rest of that call stays per operator, so results
 * do not change beyond fp32 summation order.  No counterpart in the reference (its decode
 * has no such path); for monitoring. */
int moss_hip_llm_fallbacks(const moss_hip_llm *m);
/* The same count summed over every model of the process, destroyed ones included: what a
 * caller that reaches the models only through the engine ABI (csrc/include/moss/tts.h) can
 * read. */
int moss_hip_fallbacks_total(void);

/* LlmModel::set_cancel_flag (llm.h:86): a byte polled (relaxed) before each frame, as
 * llm.cpp:645 does; a flag raised in the on_frame callback of frame k ends generate after
 * frame k's global step, with k + 1 frames.  NULL clears it.  std::atomic<bool> is one byte
 * with bool's representation on the supported ABIs. */
int moss_hip_llm_set_cancel_flag(moss_hip_llm *m, const volatile uint8_t *flag);

/* Prefix KV (llm.h:52-57, llm.cpp:455-483): device-to-device snapshot / restore. */
int moss_hip_llm_snapshot_prefix(moss_hip_llm *m);
int moss_hip_llm_restore_prefix(moss_hip_llm *m);
int moss_hip_llm_prefix_pos(const moss_hip_llm *m);

/* KV in the reference layout [12][n_pos][768] fp32 (llm.cpp:72-75), for the host
 * side of save_prefix / save_state (llm.cpp:485-586).  Export converts fp16 -> fp32. */
int moss_hip_llm_kv_export(moss_hip_llm *m, int n_pos, float *k, float *v);
/* Import for load_prefix / load_state (llm.cpp:512-632): sets pos = n_pos and, when
 * hidden768 != NULL, the hidden state.  fp32 values are rounded to fp16 for an fp16 cache. */
int moss_hip_llm_kv_import(moss_hip_llm *m, int n_pos, const float *k, const float *v, const float *hidden768);

/* ---- Quantiser capture (test instrumentation).  No counterpart in the reference, whose
 * activation quantiser is a plain function a test can call directly (quantize_row_q8_0_scaled,
 * csrc/src/quant.cpp:28-54).  Here the W8A8 quantisers run inside other kernels -- the prefill's
 * LayerNorm rows, attention epilogue and fc_in epilogue, and the in-LDS quantiser of every GEMV
 * stage of the fused decode kernels -- so with capture on each of them also records the fp32
 * vector it quantised, the int8 values and fp32 block scales it produced, and the stage outputs
 * around it, for a test to check every quantiser bit for bit and every W8A8 stage on its own
 * int8 inputs.  Capture costs memory (~130 MB for a 256-row prefill) and time: tests only.
 * Only W8A8 paths record: the prefill without prefill_a16, the fused decode with decode_a8. */
int moss_hip_llm_capture(moss_hip_llm *m, int on);

enum {
    MOSS_HIP_CAP_GLOBAL = 0,  /* the last fused global step: [12 blocks][MOSS_HIP_CAP_STEP] float */
    MOSS_HIP_CAP_LOCAL = 1,   /* the last fused greedy local half: [17 positions][MOSS_HIP_CAP_STEP] float */
    MOSS_HIP_CAP_PREFILL = 2  /* the last W8A8 prefill of m rows (M16 = m rounded up to 16), per layer:
                                 float xin[m][768], ln1[m][768], att[m][768], xm[m][768], ln2[m][768],
                                 h[m][3072], xout[m][768]; int8 ln1_q[M16 * 768], att_q[M16 * 768],
                                 ln2_q[M16 * 768], h_q[M16 * 3072]; float ln1_d[M16 * 24], att_d[M16 * 24],
                                 ln2_d[M16 * 24], h_d[M16 * 96] -- the int8 operands and scales exactly as
                                 the GEMMs read them, in the matrix-core order (row m, column k of a K-wide
                                 operand at byte ((m / 16) * (K / 32) + k / 32) * 512 + 8 * (m % 16 + 16 *
                                 ((k % 32) / 8)) + k % 8; block b's scale at float ((m / 16) * (K / 32) +
                                 b) * 16 + m % 16) */
};
/* Offsets (floats) within one decode step of a capture.  Int8 values are stored as floats. */
enum {
    MOSS_HIP_CAP_XIN = 0,       /* block input x (768) */
    MOSS_HIP_CAP_LN1 = 768,     /* LN1(x): QKV's fp32 input (768), its int8 values, its 24 scales */
    MOSS_HIP_CAP_LN1_Q = 1536,
    MOSS_HIP_CAP_LN1_D = 2304,
    MOSS_HIP_CAP_QKV = 2328,    /* q | k | v after bias and RoPE; k, v as the cache holds them (2304) */
    MOSS_HIP_CAP_ATT = 4632,    /* attention output: proj's fp32 input, int8, scales */
    MOSS_HIP_CAP_ATT_Q = 5400,
    MOSS_HIP_CAP_ATT_D = 6168,
    MOSS_HIP_CAP_XM = 6192,     /* x after the attention sub-block (768) */
    MOSS_HIP_CAP_LN2 = 6960,    /* LN2(xm): fc_in's fp32 input, int8, scales */
    MOSS_HIP_CAP_LN2_Q = 7728,
    MOSS_HIP_CAP_LN2_D = 8496,
    MOSS_HIP_CAP_H = 8520,      /* gelu(fc_in): fc_out's fp32 input (3072), int8 (3072), scales (96) */
    MOSS_HIP_CAP_H_Q = 11592,
    MOSS_HIP_CAP_H_D = 14664,
    MOSS_HIP_CAP_XOUT = 14760,  /* block output (768) */
    MOSS_HIP_CAP_LNF = 15528,   /* local positions >= 1: local ln_f(xout), the audio head's fp32 input, */
    MOSS_HIP_CAP_LNF_Q = 16296, /*   int8, scales */
    MOSS_HIP_CAP_LNF_D = 17064,
    MOSS_HIP_CAP_STEP = 17088
};
/* Copies the last capture of `what` into out (bytes >= its size); *needed (may be NULL) receives
 * the size.  out == NULL only reports the size.  ESTATE when nothing of that kind was captured. */
int moss_hip_llm_capture_read(moss_hip_llm *m, int what, void *out, size_t bytes, size_t *needed);

/* ------------------------------------------------------------------ batched streams */

/* Many independent TTS streams decoded in lock-step on one GPU.  No counterpart in the
 * reference, which runs one LlmModel per stream (csrc/include/moss/llm.h:39-90, one
 * generate() per job, csrc/src/runtime.cpp:336); each stream here has exactly that
 * per-stream state and semantics (global KV, hidden, position, history, end gate).
 * The global KV cache is paged (64-position pages behind a block table).  A batch
 * shares `model`'s device weights and must be destroyed before it.  It decodes in the
 * model's activation mode (options.decode_a8): W8A16, or W8A8 -- every GEMM input
 * quantised per 32-block by its producer (quantize_row_q8_0_scaled, quant.cpp:28-54), int8
 * block dots scaled by d_w * d_a (row_dot_q8_4x4, gemv_avx2.cpp:105-121). */
typedef struct moss_hip_batch moss_hip_batch;

/* max_streams <= 1024; capacity = KV positions per stream (> 17); kv_dtype as in the options. */
int moss_hip_batch_create(moss_hip_llm *model, int max_streams, int capacity, int kv_dtype, moss_hip_batch **out);
void moss_hip_batch_destroy(moss_hip_batch *b);
/* One stream's state, as load_state (csrc/src/llm.cpp:588-632): K/V [12][n_pos][768] fp32 and hidden[768]. */
int moss_hip_batch_set_stream(moss_hip_batch *b, int stream, int n_pos, const float *k, const float *v,
                              const float *hidden768);
/* The same from a single-stream model, device to device: K/V of positions [0, position) into the
 * stream's pages (converted to the batch's KV precision: fp32 -> fp16 rounds to nearest even),
 * the hidden state and the position.  This admits a job prepared by the reference's per-job
 * flow on a moss_hip_llm (restore_prefix -> prefill, csrc/src/engine.cpp:447-470,
 * csrc/src/llm.cpp:327-401,455-483) into the lock-step batch without a host round trip
 * (~72 KB per position in fp32).  `model` must be on the batch's device and hold the batch's
 * weights (normally the batch's own model); it is left unchanged. */
int moss_hip_batch_admit(moss_hip_batch *b, int stream, moss_hip_llm *model);
int moss_hip_batch_get_hidden(moss_hip_batch *b, int stream, float *out768);
int moss_hip_batch_position(const moss_hip_batch *b, int stream);
int moss_hip_batch_kv_export(moss_hip_batch *b, int stream, int n_pos, float *k, float *v);
/* global_step (csrc/src/llm.cpp:248-255) of streams [0, n_streams): rows [n_streams][17]. */
int moss_hip_batch_global_step(moss_hip_batch *b, int n_streams, const int32_t *rows);
/* generate (csrc/src/llm.cpp:634-733) for streams [0, n_streams), frames in lock-step: out_rows
 * [frames][n_streams][17]; out_frames[s] = frames stream s produced (its end gate / capacity);
 * *elapsed_ms = device time of the whole run.  Stream s samples like its own LlmModel::generate
 * with seed seeds[s] (seeds NULL = 0 for every stream). */
int moss_hip_batch_generate(moss_hip_batch *b, int n_streams, int frames, const moss_hip_sample_params *p,
                            const uint64_t *seeds, int32_t *out_rows, int *out_frames, double *elapsed_ms);
/* Attention capture of a W8A8 batch (test instrumentation, as moss_hip_llm_capture): while on,
 * every attention of the frames run records its fp32 output rows and the int8 operand and block
 * scales quantised from them for proj (ESTATE on a W8A16 batch).  moss_hip_batch_capture_read
 * copies the last frame's records: 29 entries (12 global layers, then local positions 0..16),
 * each float out[max_streams][768], int8 q[S16 * 768], float d[S16 * 24] with S16 = max_streams
 * rounded up to 16, q and d in the matrix-core order of MOSS_HIP_CAP_PREFILL. */
int moss_hip_batch_capture(moss_hip_batch *b, int on);
int moss_hip_batch_capture_read(moss_hip_batch *b, void *out, size_t bytes, size_t *needed);

/* ------------------------------------------------------------------ operator layer */

enum { MOSS_HIP_F32 = 0, MOSS_HIP_F16 = 1 };

/* y[rows] = W[rows][cols] x over Q8_0_4X4 weights -- gemv_par (csrc/include/moss/gemv.h:48,
 * csrc/src/gemv.cpp:245-274) with MOSS_A16 on (row kernel csrc/src/gemv_avx2.cpp:123-150).
 * x_dtype / y_dtype: MOSS_HIP_F32 or MOSS_HIP_F16.  rows % 4 == 0, cols % 128 == 0, cols <= 4096. */
int moss_hip_gemv_q8x4(const void *w, int rows, int cols, const void *x, int x_dtype, void *y, int y_dtype,
                       void *stream);

/* y[rows] = W[rows][cols] x in W8A8 -- gemv_par with MOSS_A16 unset (csrc/src/gemv.cpp:229-274): x
 * quantised once per 32-block (quantize_activation, csrc/src/quant.cpp:45-54), each row the int8 row
 * dot of row_dot_q8_4x4 (csrc/src/gemv_avx2.cpp:105-121).  x, y fp32; rows % 4 == 0,
 * cols % 256 == 0, cols <= 4096. */
int moss_hip_gemv_q8x4_w8a8(const void *w, int rows, int cols, const float *x, float *y, void *stream);

/* Y[m][rows] = X[m][cols] W^T on the matrix cores -- gemm_par (csrc/include/moss/gemv.h:54,
 * csrc/src/gemv.cpp:276-309) in its A16 mode.  x, y fp32; rows % 16 == 0, cols % 32 == 0. */
int moss_hip_gemm_q8x4(const void *w, int rows, int cols, const float *x, int m, float *y, void *stream);

/* W8A8 activation quantisation -- quantize_row_q8_0_scaled (csrc/src/quant.cpp:28-54) per row:
 * q[m][cols] int8 and d[m][cols/32] fp32 block scales of x[m][cols].  cols % 256 == 0. */
int moss_hip_quantize_rows(const float *x, int m, int cols, int8_t *q, float *d, void *stream);

/* W8A8 GEMM -- gemm_par without MOSS_A16 (csrc/src/gemv.cpp:281-309; row kernel
 * row_dot_q8_4x4, csrc/src/gemv_avx2.cpp:105-121): Y[m][rows] from int8 activations q[m][cols]
 * with block scales d[m][cols/32] (as moss_hip_quantize_rows writes them).  rows % 16 == 0. */
int moss_hip_gemm_q8x4_w8a8(const void *w, int rows, int cols, const int8_t *q, const float *d, int m, float *y,
                            void *stream);

/* Dequantise rows of a mat_rows x cols Q8_0_4X4 matrix to fp32 -- LlmModel::lookup_row
 * (llm.cpp:114-146) / dequantize_row_q8_0_4x4 (csrc/src/quant.cpp:56-65).  rows_dev: n device
 * int32 indices; an index outside [0, mat_rows) yields a row of NaN. */
int moss_hip_dequant_rows_q8x4(const void *w, int mat_rows, int cols, const int32_t *rows_dev, int n, float *out,
                               void *stream);

/* Single-query attention over one layer's cache -- LlmModel::attention_core (llm.cpp:189-217).
 * q [heads*64] fp32 (post-RoPE); k_cache/v_cache [heads][ctx_stride][64] of kv_dtype; the
 * first n_keys positions are attended.  out [heads*64] of out_dtype.  Up to 512 keys one
 * workgroup per head attends them (a wave per 64 keys, merged in LDS); past 512 the keys are
 * cut into slices of 128 keys (up to 1,024 keys) or 256 (at most 64 slices per head)
 * attended by separate workgroups and merged by
 * the first slice of each head (log-sum-exp, slice order); the partials live in a scratch block
 * the library allocates once per (device, stream) on the first call on that stream (which must
 * not be under graph capture), so calls on one stream are ordered and calls on different
 * streams do not share it. */
int moss_hip_attn_decode(const float *q, const void *k_cache, const void *v_cache, int kv_dtype, int heads,
                         int ctx_stride, int n_keys, void *out, int out_dtype, void *stream);

/* Single-query attention of a batch of streams over paged K/V: the 64-stream engine's global
 * attention (csrc/batch_model.hip) on caller-owned pages.  Per row it is attention_core
 * (reference csrc/src/llm.cpp:189-217: scores q . k * 0.125, softmax, weighted sum of v); the
 * batch over streams and the paging have no reference counterpart (the reference decodes one
 * stream).  Pools are [page][heads][page_size][64] (kv_dtype MOSS_HIP_F16 or MOSS_HIP_F32;
 * page_size a multiple of 64, else MOSS_HIP_EINVAL: keys are read in 64-key spans); row
 * r is the query of stream row_stream[r] (r when row_stream is NULL) at position row_pos[r]
 * and attends that stream's keys 0 .. row_pos[r], whose j-th page of page_size positions is
 * page_table[stream * table_stride + j].  q: [rows][heads * 64] fp32 (RoPE applied); out:
 * [rows][heads * 64] (out_dtype).  max_keys bounds every row's key count (row_pos[r] + 1 is
 * clamped to it) and sizes the launch.  page_table, row_stream and row_pos are device arrays.
 * No scratch, no allocation: one workgroup per (head, row). */
int moss_hip_attn_paged(const float *q, const void *k_pool, const void *v_pool, int kv_dtype, int heads,
                        const int32_t *page_table, int table_stride, int page_size, int rows,
                        const int32_t *row_stream, const int32_t *row_pos, int max_keys, void *out, int out_dtype,
                        void *stream);

/* moss_hip_attn_decode without any allocation.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under hipGraph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, kernel and results; heads <= 16
 * (EINVAL beyond).  Its scratch (557,312 bytes: the sliced launch's generation header and
 * partials for 16 heads) is a static array in the library's device code, one per GPU, held
 * until the process ends; the first call on a device looks its address up
 * (hipGetSymbolAddress), nothing is allocated or cleared per call.  Every call on one GPU
 * shares that scratch, so calls that overlap on one GPU (other streams, concurrent graph
 * replays) race: serialise them. */
int moss_hip_attn_decode_noalloc(const float *q, const void *k_cache, const void *v_cache, int kv_dtype, int heads,
                                 int ctx_stride, int n_keys, void *out, int out_dtype, void *stream);

/* ---- Audio codec decoder (codes -> 48 kHz stereo PCM) --------------------------------
 * The GPU replacement of moss::AudioDecoder (reference csrc/include/moss/decoder.h:14-83,
 * csrc/src/decoder.cpp:26-281): the MOSS-Audio-Tokenizer-Nano decoder of a decoder .moss
 * (decoder_f16.moss: fp16 matrices, fp32 vectors and codebooks).  A host-side
 * moss::AudioDecoder with the reference's public surface sits on top
 * (dsh-moss-tts_amd/host/moss/decoder.h, host/decoder_hip.cpp).  Codes are
 * quantizer-major [16][frames] int32 in [0, 1024); output is frames * 7680 interleaved
 * stereo float samples (L, R, L, R, ...).  Same threading rule as the model handle. */
typedef struct moss_hip_codec moss_hip_codec;

typedef struct {
    int device;           /* HIP device ordinal */
    int max_chunk_frames; /* a chunk is run in pieces of at most this many frames; 0 = 32.  Sizes the
                             activation buffers and the K/V rings (window + 32 * this positions at the last
                             stage).  Results do not depend on it beyond fp32 rounding. */
    int contexts[4];      /* per-stage attention windows in positions; 0 = the reference's 500, 800, 1200, 1600
                             (decoder.cpp:21; other values are for tests of the window) */
    int eager;            /* 0 = decode_chunk replays a hipGraph per piece size (default); 1 = direct launches */
} moss_hip_codec_options;

/* AudioDecoder::AudioDecoder + load (decoder.h:19-21, decoder.cpp:26-70): parses the file,
 * checks every tensor the reference loads, uploads them, allocates the stream state.
 * opt may be NULL (defaults).  Matrices must be F16 (dtype 0) or F32 (dtype 3), their
 * column counts multiples of 32 and row counts multiples of 16. */
int moss_hip_codec_create(const void *blob, size_t bytes, const moss_hip_codec_options *opt, moss_hip_codec **out);
int moss_hip_codec_create_from_file(const char *path, const moss_hip_codec_options *opt, moss_hip_codec **out);
void moss_hip_codec_destroy(moss_hip_codec *c);
int moss_hip_codec_samples_per_frame(const moss_hip_codec *c); /* 7680 for the release decoder */
/* AudioDecoder::reset_stream (decoder.cpp:105-115): positions back to 0, rings emptied. */
int moss_hip_codec_reset_stream(moss_hip_codec *c);
/* AudioDecoder::decode_chunk (decoder.cpp:203-221): the next `frames` frames of the stream
 * (every layer attends to its cached keys of earlier chunks within its window); out receives
 * frames * samples_per_frame floats.  Codes outside [0, 1024) -> EINVAL, nothing run. */
int moss_hip_codec_decode_chunk(moss_hip_codec *c, const int32_t *codes, int frames, float *out);
/* AudioDecoder::decode (decoder.cpp:247-281): a whole utterance from position 0, on a state
 * of its own (the stream is untouched); sets last_ms and the four stage times. */
int moss_hip_codec_decode(moss_hip_codec *c, const int32_t *codes, int frames, float *out);
double moss_hip_codec_last_ms(const moss_hip_codec *c);             /* decoder.h:31 */
int moss_hip_codec_stage_ms(const moss_hip_codec *c, double out4[4]); /* decoder.h:32 */

#ifdef __cplusplus
}
#endif
#endif /* MOSS_HIP_H */
