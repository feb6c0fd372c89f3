/*
 * moss_oracle.h -- CPU oracle for the MOSS-TTS-Nano LLM decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * algorithm, used as the checker for the HIP path.  Only tests/, the smoke()
 * entry of __graft_entry__.py and the cpu_baseline leg of bench.py may load it.
 * The product library never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  Arithmetic follows the reference source
 * operator by operator (fp32, no contraction: this file is compiled with
 * -ffp-contract=off), using fmaf() exactly where the reference uses
 * _mm256_fmadd_ps, so that results are bit-identical to the reference compiled
 * with -ffp-contract=off.
 *
 * Parity pins (tests/test_oracle_*.py):
 *   - fp16 conversion: exhaustive over all 65536 halves vs numpy float16, and
 *     every fp32 bit pattern class vs numpy rounding (RNE).
 *   - 4x4 dequant / activation quantisation: golden vectors written by the
 *     compiled reference + closed forms.
 *   - W8A16 / W8A8 row dots: golden vectors (bit-exact) + fp64 brute force.
 *   - LayerNorm / RoPE / attention / gelu: through the full-model golden
 *     vectors (hidden state and logits after global/local steps, bit-exact)
 *     plus closed-form invariants (ctx=1 attention returns v, RoPE at pos 0
 *     is the identity, LN output has zero mean / unit variance).
 *   - sampler: greedy argmax/penalty closed forms; xoshiro128** stream vs the
 *     golden vector.
 */
#ifndef MOSS_ORACLE_H
#define MOSS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    MO_HIDDEN = 768, MO_HEADS = 12, MO_HEAD_DIM = 64, MO_FF = 3072, MO_VOCAB = 16384,
    MO_NVQ = 16, MO_CODEBOOK = 1024, MO_AUDIO_PAD = 1024, MO_SLOT = 9, MO_END = 7,
    MO_MAX_CTX = 768, MO_LOCAL_LEN = 17, MO_LAYERS = 12
};

/* ---- fp16 (reference csrc/src/fp16.cpp:7-66) ---- */
float mo_half_to_float(uint16_t h);
uint16_t mo_float_to_half(float f);
/* round-to-nearest-even variant (hardware fp16 store; emulates an fp16 KV cache) */
uint16_t mo_float_to_half_rne(float f);

/* ---- quantisation (reference csrc/src/quant.cpp:28-65) ---- */
void mo_dequant_row_q8x4(const uint8_t *group, int nb, int k, float *out);
/* quantize_row_q8_0_scaled: q[k] int8, dh[nb] fp16 bits, d[nb] fp32 scales */
void mo_quantize_row_q8(const float *x, int k, int8_t *q, uint16_t *dh, float *d);

/* ---- row dots over the 4x4 layout (reference csrc/src/gemv_avx2.cpp:105-150) ---- */
float mo_row_dot_a16(const uint8_t *group, int nb, int k, const float *act);
float mo_row_dot_a16_scalar(const uint8_t *group, int nb, int k, const float *act);
float mo_row_dot_w8a8(const uint8_t *group, int nb, int k, const int8_t *qa, const float *da);
/* y[rows] = W x, W in Q8_0_4X4 (reference csrc/src/gemv.cpp:192-208 + :245-274) */
void mo_gemv_a16(const uint8_t *w, int rows, int cols, const float *x, float *y);
/* Y[m][rows] = X[m][cols] W^T, W8A8 (quantised activations) or A16 (reference gemv.cpp:276-309) */
void mo_gemm(const uint8_t *w, int rows, int cols, const float *x, int m, float *y, int a16);
/* W8A8 gemm on given int8 activations q[m][cols] and block scales d[m][cols/32] */
void mo_gemm_w8a8_q(const uint8_t *w, int rows, int cols, const int8_t *q, const float *d, int m, float *y);

/* ---- elementwise pieces (reference csrc/src/llm.cpp) ---- */
float mo_gelu_new(float v);                                                    /* llm.cpp:22-25 */
void mo_layernorm(const float *x, const float *w, const float *b, float *out); /* llm.cpp:159-171 */
void mo_rope_tables(int max_pos, float *cos_t, float *sin_t);                  /* llm.cpp:90-102 */
void mo_rope_apply(float *vec, int pos, const float *cos_t, const float *sin_t); /* llm.cpp:173-187 */
/* llm.cpp:189-217; k/v rows have stride `stride` floats, heads*64 = row width used */
void mo_attention_core(const float *k_cache, const float *v_cache, int stride, int n_pos, const float *q,
                       float *out, float *scores);

/* ---- sampler (reference csrc/src/sampler.cpp:9-79, csrc/include/moss/sampler.h:8-50) ---- */
typedef struct {
    int greedy;
    float temperature;
    int top_k;
    float top_p;
    float repetition_penalty;
    int end_greedy;
    int min_frames;
    int greedy_frames;
} mo_sample_params;
typedef struct { uint32_t s[4]; } mo_rng;
void mo_rng_seed(mo_rng *r, uint64_t v);
uint32_t mo_rng_next(mo_rng *r);
float mo_rng_uniform(mo_rng *r);
/* scratch must hold n floats + n ints (n*8 bytes) */
int mo_sample_token(const float *logits, int n, const mo_sample_params *p, const int *prev, int n_prev,
                    mo_rng *rng, void *scratch);

/* ---- .moss v1 blob + model (reference csrc/src/weights.cpp:27-125, csrc/src/llm.cpp) ---- */
typedef struct mo_model mo_model;
/* blob must outlive the model; returns NULL and fills err (if non-NULL, 256 bytes) on failure */
mo_model *mo_model_create(const uint8_t *blob, size_t bytes, int max_ctx, char *err);
void mo_model_destroy(mo_model *m);
/* kv_f16 != 0: global K/V are rounded to fp16 when written (emulates an fp16 KV cache;
 * the 17-position local cache stays fp32) */
void mo_model_set_kv_f16(mo_model *m, int on);
/* on != 0: decode GEMVs (global and local blocks, audio and text heads) in W8A8, the
 * reference with MOSS_A16 unset (gemv.cpp:23-48,229-274); 0 (default): W8A16 */
void mo_model_set_decode_a8(mo_model *m, int on);
void mo_model_reset(mo_model *m);
int mo_model_position(const mo_model *m);
const float *mo_model_hidden(const mo_model *m);
void mo_model_set_hidden(mo_model *m, const float *h);
/* import [12][n_pos][768] K and V (reference layout), sets pos = n_pos */
int mo_model_kv_import(mo_model *m, int n_pos, const float *k, const float *v);
int mo_model_kv_export(const mo_model *m, int n_pos, float *k, float *v);
void mo_model_embed_row(const mo_model *m, const int32_t *row17, float *out);       /* llm.cpp:148-157 */
void mo_model_global_step(mo_model *m, const int32_t *row17);                        /* llm.cpp:248-255 */
void mo_model_local_reset(mo_model *m);                                              /* llm.cpp:257 */
void mo_model_local_step(mo_model *m, const float *in, float *out);                  /* llm.cpp:259-264 */
void mo_model_audio_logits(mo_model *m, int ch, const float *hidden, float *logits); /* llm.cpp:268-270 */
void mo_model_assistant_logits(mo_model *m, const float *hidden, float *pair);       /* llm.cpp:274-315 */
void mo_model_text_logits(mo_model *m, const float *hidden, float *logits);          /* llm.cpp:266 */
/* llm.cpp:327-401; a16 = 0 for the reference default (W8A8 prefill) */
void mo_model_prefill(mo_model *m, const int32_t *rows17, int n_rows, int start, int a16);
/* llm.cpp:634-733.  forced: [n_forced][17] or NULL.  out_rows: [max_frames][17].
 * logits_dump (optional): [max_frames][16][1024].  gate_out (optional): the reference's gate-dump
 * mode (llm.cpp:653-679): [max_frames][4] = (l_end, l_slot, argmax_id, argmax_logit) from the
 * full text head, which then also decides the end gate.
 * returns number of frames produced. */
int mo_model_generate(mo_model *m, int max_frames, const mo_sample_params *p, uint64_t seed,
                      const int32_t *forced, int n_forced, int32_t *out_rows, float *logits_dump,
                      float *gate_out);

#ifdef __cplusplus
}
#endif
#endif
