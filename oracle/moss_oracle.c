/*
 * moss_oracle.c -- CPU oracle (test infrastructure only; see moss_oracle.h).
 *
 * Plain-C restatement of the reference LLM decode path.  Compiled with
 * -ffp-contract=off: every '*', '+' and '-' below rounds on its own, exactly
 * as the reference source reads when its compiler does not contract; fmaf()
 * appears only where the reference calls _mm256_fmadd_ps.
 */
#include "moss_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

/* reference csrc/src/fp16.cpp:7-35 */
float mo_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t mant = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: renormalise */
            e = 127 - 15 + 1;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                --e;
            }
            mant &= 0x3FFu;
            bits = sign | (e << 23) | (mant << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((e - 15 + 127) << 23) | (mant << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

/* reference csrc/src/fp16.cpp:37-66 (round-half-up on the dropped bit in the
 * normal range, as the reference writes it) */
uint16_t mo_float_to_half(float f) {
    uint32_t bits;
    memcpy(&bits, &f, 4);
    uint32_t sign = (bits >> 16) & 0x8000u;
    int32_t e = (int32_t)((bits >> 23) & 0xFF) - 127 + 15;
    uint32_t mant = bits & 0x7FFFFFu;
    if (((bits >> 23) & 0xFF) == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? 0x200u : 0));
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        mant |= 0x800000u;
        int shift = 14 - e;
        uint32_t hm = mant >> shift;
        if ((mant >> (shift - 1)) & 1u) ++hm;
        return (uint16_t)(sign | hm);
    }
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    uint32_t hm = mant >> 13;
    if (mant & 0x1000u) ++hm;
    if (hm == 0x400u) {
        hm = 0;
        ++e;
        if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | hm);
}

/* IEEE round-to-nearest-even float -> half (what a hardware fp16 store does;
 * used only to emulate an fp16 KV cache -- the reference keeps KV in fp32) */
uint16_t mo_float_to_half_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                     /* below 2^-14: subnormal half */
        float a;
        memcpy(&a, &ax, 4);
        /* a * 2^24 is exact; nearbyintf rounds half-even in the default mode */
        float r = nearbyintf(a * 16777216.0f);
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t mant = ax & 0x7FFFFFu;
    uint32_t hm = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) ++hm; /* carries into the exponent correctly */
    return (uint16_t)(sign | hm);
}

/* ------------------------------------------------------------ quantisation */

static uint16_t rd16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

/* reference csrc/src/quant.cpp:56-65: block b of a 4-row group is 136 bytes:
 * 4 fp16 scales (row k at +2k) then 4 x 32 int8 (row k at +8+32k). */
void mo_dequant_row_q8x4(const uint8_t *group, int nb, int k, float *out) {
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = group + (size_t)b * 136;
        float d = mo_half_to_float(rd16(blk + 2 * k));
        const int8_t *qs = (const int8_t *)(blk + 8 + (size_t)k * 32);
        for (int i = 0; i < 32; ++i) out[b * 32 + i] = d * (float)qs[i];
    }
}

/* reference csrc/src/quant.cpp:28-43 (quantize_row_q8_0_scaled) */
void mo_quantize_row_q8(const float *x, int k, int8_t *q, uint16_t *dh, float *dscale) {
    int nb = k / 32;
    for (int b = 0; b < nb; ++b) {
        const float *src = x + b * 32;
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float a = fabsf(src[i]);
            amax = amax < a ? a : amax; /* std::max(amax, a) returns amax unless amax < a */
        }
        float d = amax / 127.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        if (dh) dh[b] = mo_float_to_half(d);
        if (dscale) dscale[b] = d;
        for (int i = 0; i < 32; ++i) {
            long v = lrintf(src[i] * id);
            int qi = (int)v;
            if (qi < -127) qi = -127;
            if (qi > 127) qi = 127;
            q[b * 32 + i] = (int8_t)qi;
        }
    }
}

/* ------------------------------------------------------------- row dots */

/* _mm_add_ps(lo,hi) -> movehl add -> add_ss (reference gemv_avx2.cpp:24-31) */
static float hsum8(const float a[8]) {
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    float t0 = s0 + s2, t1 = s1 + s3;
    return t0 + t1;
}

/* W8A16 row dot, AVX2 order (reference csrc/src/gemv_avx2.cpp:123-150):
 * per block, 8 lane partials: mul for cols [0,8), fma for [8,16), [16,24),
 * [24,32); hsum; then sum += hsum * d (two roundings). */
float mo_row_dot_a16(const uint8_t *group, int nb, int k, const float *act) {
    float sum = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = group + (size_t)b * 136;
        float dw = mo_half_to_float(rd16(blk + 2 * k));
        const int8_t *qs = (const int8_t *)(blk + 8 + (size_t)k * 32);
        const float *a = act + (size_t)b * 32;
        float acc[8];
        for (int i = 0; i < 8; ++i) acc[i] = (float)qs[i] * a[i];
        for (int i = 0; i < 8; ++i) acc[i] = fmaf((float)qs[8 + i], a[8 + i], acc[i]);
        for (int i = 0; i < 8; ++i) acc[i] = fmaf((float)qs[16 + i], a[16 + i], acc[i]);
        for (int i = 0; i < 8; ++i) acc[i] = fmaf((float)qs[24 + i], a[24 + i], acc[i]);
        float h = hsum8(acc);
        float t = h * dw;
        sum = sum + t;
    }
    return sum;
}

/* W8A16 row dot, scalar fallback order (reference csrc/src/gemv.cpp:51-63) */
float mo_row_dot_a16_scalar(const uint8_t *group, int nb, int k, const float *act) {
    float sum = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = group + (size_t)b * 136;
        const int8_t *qs = (const int8_t *)(blk + 8 + (size_t)k * 32);
        float dot = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float p = (float)qs[i] * act[b * 32 + i];
            dot = dot + p;
        }
        float t = dot * mo_half_to_float(rd16(blk + 2 * k));
        sum = sum + t;
    }
    return sum;
}

/* W8A8 row dot, AVX2 order (reference csrc/src/gemv_avx2.cpp:105-121):
 * lane j (0..7) of the 256-bit accumulator gets the exact int32 sum of the
 * products of bytes 4j..4j+3 (maddubs+madd with |q| <= 127 cannot saturate),
 * converted to float and fma'd with (d_w * d_a) rounded once; hsum at the end. */
float mo_row_dot_w8a8(const uint8_t *group, int nb, int k, const int8_t *qa, const float *da) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = group + (size_t)b * 136;
        float dw = mo_half_to_float(rd16(blk + 2 * k));
        const int8_t *qs = (const int8_t *)(blk + 8 + (size_t)k * 32);
        const int8_t *as = qa + (size_t)b * 32;
        float scale = dw * da[b];
        for (int j = 0; j < 8; ++j) {
            int32_t p = 0;
            for (int t = 0; t < 4; ++t) p += (int32_t)qs[4 * j + t] * (int32_t)as[4 * j + t];
            acc[j] = fmaf((float)p, scale, acc[j]);
        }
    }
    return hsum8(acc);
}

void mo_gemv_a16(const uint8_t *w, int rows, int cols, const float *x, float *y) {
    int nb = cols / 32;
#pragma omp parallel for schedule(static) if (rows >= 512)
    for (int r = 0; r < rows; ++r) y[r] = mo_row_dot_a16(w + (size_t)(r / 4) * nb * 136, nb, r % 4, x);
}

/* reference csrc/src/gemv.cpp:281-309 (4x4 branch of gemm_par) */
void mo_gemm(const uint8_t *w, int rows, int cols, const float *x, int m, float *y, int a16) {
    int nb = cols / 32;
    int8_t *q = NULL;
    float *d = NULL;
    if (!a16) {
        q = (int8_t *)malloc((size_t)m * cols);
        d = (float *)malloc((size_t)m * nb * sizeof(float));
        for (int i = 0; i < m; ++i) mo_quantize_row_q8(x + (size_t)i * cols, cols, q + (size_t)i * cols, NULL, d + (size_t)i * nb);
    }
#pragma omp parallel for schedule(static) if ((size_t)rows * m >= 4096)
    for (int g = 0; g < rows / 4; ++g) {
        const uint8_t *grp = w + (size_t)g * nb * 136;
        for (int i = 0; i < m; ++i) {
            for (int k = 0; k < 4; ++k) {
                float v = a16 ? mo_row_dot_a16(grp, nb, k, x + (size_t)i * cols)
                              : mo_row_dot_w8a8(grp, nb, k, q + (size_t)i * cols, d + (size_t)i * nb);
                y[(size_t)i * rows + g * 4 + k] = v;
            }
        }
    }
    free(q);
    free(d);
}

/* The W8A8 product of gemm_par (reference csrc/src/gemv.cpp:281-309) on activations
 * quantised elsewhere: row r of Y for activation row i is row_dot_q8_4x4's block sum
 * (gemv_avx2.cpp:105-121) of q[i] with block scales d[i].  Lets a test evaluate a GPU
 * stage on the GPU's own int8 operand. */
void mo_gemm_w8a8_q(const uint8_t *w, int rows, int cols, const int8_t *q, const float *d, int m, float *y) {
    int nb = cols / 32;
#pragma omp parallel for schedule(static) if ((size_t)rows * m >= 4096)
    for (int g = 0; g < rows / 4; ++g) {
        const uint8_t *grp = w + (size_t)g * nb * 136;
        for (int i = 0; i < m; ++i)
            for (int k = 0; k < 4; ++k)
                y[(size_t)i * rows + g * 4 + k] =
                    mo_row_dot_w8a8(grp, nb, k, q + (size_t)i * cols, d + (size_t)i * nb);
    }
}

/* ------------------------------------------------------------- elementwise */

/* reference csrc/src/llm.cpp:22-25 */
float mo_gelu_new(float v) {
    const float k = 0.7978845608028654f;
    float v3 = 0.044715f * v * v * v;
    float inner = k * (v + v3);
    return 0.5f * v * (1.0f + tanhf(inner));
}

/* reference csrc/src/llm.cpp:159-171 */
void mo_layernorm(const float *x, const float *w, const float *b, float *out) {
    float mean = 0.0f;
    for (int i = 0; i < MO_HIDDEN; ++i) mean += x[i];
    mean /= (float)MO_HIDDEN;
    float var = 0.0f;
    for (int i = 0; i < MO_HIDDEN; ++i) {
        float d = x[i] - mean;
        float dd = d * d;
        var += dd;
    }
    var /= (float)MO_HIDDEN;
    float inv = 1.0f / sqrtf(var + 1e-5f);
    for (int i = 0; i < MO_HIDDEN; ++i) {
        float t = (x[i] - mean) * inv;
        t = t * w[i];
        out[i] = t + b[i];
    }
}

/* reference csrc/src/llm.cpp:90-102: angle computed in double, stored as float,
 * table [pos][12*32] (identical for every head) */
void mo_rope_tables(int max_pos, float *cos_t, float *sin_t) {
    const int half = MO_HEAD_DIM / 2;
    for (int pos = 0; pos < max_pos; ++pos) {
        for (int h = 0; h < MO_HEADS; ++h) {
            for (int i = 0; i < half; ++i) {
                double inv = 1.0 / pow(10000.0, (double)(2 * i) / MO_HEAD_DIM);
                double angle = (double)pos * inv;
                cos_t[(size_t)pos * (MO_HIDDEN / 2) + h * half + i] = (float)cos(angle);
                sin_t[(size_t)pos * (MO_HIDDEN / 2) + h * half + i] = (float)sin(angle);
            }
        }
    }
}

/* reference csrc/src/llm.cpp:173-187: interleaved pairs (2i, 2i+1) */
void mo_rope_apply(float *vec, int pos, const float *cos_t, const float *sin_t) {
    const float *c = cos_t + (size_t)pos * (MO_HIDDEN / 2);
    const float *s = sin_t + (size_t)pos * (MO_HIDDEN / 2);
    for (int h = 0; h < MO_HEADS; ++h) {
        float *base = vec + h * MO_HEAD_DIM;
        for (int i = 0; i < MO_HEAD_DIM / 2; ++i) {
            float c0 = c[h * (MO_HEAD_DIM / 2) + i];
            float s0 = s[h * (MO_HEAD_DIM / 2) + i];
            float x0 = base[2 * i], x1 = base[2 * i + 1];
            float a = x0 * c0, bb = x1 * s0;
            float cc = x1 * c0, dd = x0 * s0;
            base[2 * i] = a - bb;
            base[2 * i + 1] = cc + dd;
        }
    }
}

/* reference csrc/src/llm.cpp:189-217 */
void mo_attention_core(const float *k_cache, const float *v_cache, int stride, int n_pos, const float *q,
                       float *out, float *scores) {
    const float scale = 1.0f / sqrtf((float)MO_HEAD_DIM);
    for (int h = 0; h < MO_HEADS; ++h) {
        const float *qh = q + h * MO_HEAD_DIM;
        float *oh = out + h * MO_HEAD_DIM;
        float max_score = -1e30f;
        for (int p = 0; p < n_pos; ++p) {
            const float *kh = k_cache + (size_t)p * stride + h * MO_HEAD_DIM;
            float dot = 0.0f;
            for (int d = 0; d < MO_HEAD_DIM; ++d) {
                float t = qh[d] * kh[d];
                dot = dot + t;
            }
            dot = dot * scale;
            scores[p] = dot;
            max_score = max_score < dot ? dot : max_score; /* std::max(max_score, dot) */
        }
        float sum = 0.0f;
        for (int p = 0; p < n_pos; ++p) {
            scores[p] = expf(scores[p] - max_score);
            sum += scores[p];
        }
        float inv_sum = 1.0f / sum;
        for (int d = 0; d < MO_HEAD_DIM; ++d) oh[d] = 0.0f;
        for (int p = 0; p < n_pos; ++p) {
            float wgt = scores[p] * inv_sum;
            const float *vh = v_cache + (size_t)p * stride + h * MO_HEAD_DIM;
            for (int d = 0; d < MO_HEAD_DIM; ++d) {
                float t = wgt * vh[d];
                oh[d] = oh[d] + t;
            }
        }
    }
}

/* ----------------------------------------------------------------- sampler */

/* reference csrc/include/moss/sampler.h:25-49 (xoshiro128**) */
static uint32_t rotl32(uint32_t x, int k) { return (x << k) | (x >> (32 - k)); }
uint32_t mo_rng_next(mo_rng *r) {
    uint32_t result = rotl32(r->s[1] * 5u, 7) * 9u;
    uint32_t t = r->s[1] << 9;
    r->s[2] ^= r->s[0];
    r->s[3] ^= r->s[1];
    r->s[1] ^= r->s[2];
    r->s[0] ^= r->s[3];
    r->s[2] ^= t;
    r->s[3] = rotl32(r->s[3], 11);
    return result;
}
void mo_rng_seed(mo_rng *r, uint64_t v) {
    r->s[0] = (uint32_t)v;
    r->s[1] = (uint32_t)(v >> 32) ^ 0x9E3779B9u;
    r->s[2] = 0x243F6A88u;
    r->s[3] = 0xB7E15162u;
    for (int i = 0; i < 8; ++i) mo_rng_next(r);
}
float mo_rng_uniform(mo_rng *r) { return (float)(mo_rng_next(r) >> 8) * (1.0f / 16777216.0f); }

static const float *g_sort_vals;
/* descending by value; equal values by ascending index (the reference's
 * std::partial_sort leaves ties unordered; seeded float logits have none) */
static int cmp_desc(const void *a, const void *b) {
    int ia = *(const int *)a, ib = *(const int *)b;
    float va = g_sort_vals[ia], vb = g_sort_vals[ib];
    if (va > vb) return -1;
    if (va < vb) return 1;
    return ia < ib ? -1 : (ia > ib);
}

/* reference csrc/src/sampler.cpp:9-79 */
int mo_sample_token(const float *logits, int n, const mo_sample_params *p, const int *prev, int n_prev,
                    mo_rng *rng, void *scratch_mem) {
    float *sc = (float *)scratch_mem;
    int *idx = (int *)(sc + n);
    memcpy(sc, logits, sizeof(float) * (size_t)n);
    if (p->repetition_penalty != 1.0f && prev != NULL && n_prev > 0) {
        for (int i = 0; i < n_prev; ++i) {
            int t = prev[i];
            if (t < 0 || t >= n) continue;
            float v = sc[t];
            sc[t] = v < 0.0f ? v * p->repetition_penalty : v / p->repetition_penalty;
        }
    }
    if (p->greedy || p->top_k == 1) {
        int best = 0;
        for (int i = 1; i < n; ++i)
            if (sc[i] > sc[best]) best = i;
        return best;
    }
    if (p->temperature > 0.0f && p->temperature != 1.0f) {
        float inv = 1.0f / p->temperature;
        for (int i = 0; i < n; ++i) sc[i] *= inv;
    }
    int k = p->top_k > 0 ? (p->top_k < n ? p->top_k : n) : n;
    for (int i = 0; i < n; ++i) idx[i] = i;
    g_sort_vals = sc;
    qsort(idx, (size_t)n, sizeof(int), cmp_desc);
    int cnt = k;
    float maxv = sc[idx[0]];
    float sum = 0.0f;
    for (int j = 0; j < cnt; ++j) {
        int i = idx[j];
        sc[i] = expf(sc[i] - maxv);
        sum += sc[i];
    }
    if (p->top_p < 1.0f) {
        float cum = 0.0f;
        int keep = 0;
        for (; keep < cnt; ++keep) {
            cum += sc[idx[keep]] / sum;
            if (cum >= p->top_p) {
                ++keep;
                break;
            }
        }
        cnt = keep > 1 ? keep : 1;
        sum = 0.0f;
        for (int j = 0; j < cnt; ++j) sum += sc[idx[j]];
    }
    float r = mo_rng_uniform(rng) * sum;
    for (int j = 0; j < cnt; ++j) {
        r -= sc[idx[j]];
        if (r <= 0.0f) return idx[j];
    }
    return idx[cnt - 1];
}

/* ------------------------------------------------------------------ model */

typedef struct {
    const uint8_t *data;
    int rows, cols;
} mo_mat;
typedef struct {
    const float *data;
    int n;
} mo_vec;
typedef struct {
    mo_vec ln1_w, ln1_b, ln2_w, ln2_b;
    mo_mat attn_w;
    mo_vec attn_b;
    mo_mat proj_w;
    mo_vec proj_b;
    mo_mat fc_in_w;
    mo_vec fc_in_b;
    mo_mat fc_out_w;
    mo_vec fc_out_b;
} mo_layer;

struct mo_model {
    const uint8_t *blob;
    size_t bytes;
    mo_layer g[MO_LAYERS], local;
    mo_vec lnf_w, lnf_b, llnf_w, llnf_b;
    mo_mat wte, aemb[MO_NVQ];
    int max_ctx, kv_f16;
    int decode_a8;                   /* decode GEMVs in W8A8 (MOSS_A16 unset), else W8A16 */
    float *gk, *gv;                  /* [12][max_ctx][768] */
    float *lk, *lv;                  /* [17][768] */
    float *cos_t, *sin_t;            /* [max_ctx][384] */
    int pos, lpos;
    float hidden[MO_HIDDEN];
    /* per-step scratch */
    float x[MO_HIDDEN], ln[MO_HIDDEN], qkv[3 * MO_HIDDEN], att[MO_HIDDEN], mlp[MO_FF], res[MO_HIDDEN];
    float lx[MO_HIDDEN], lqkv[3 * MO_HIDDEN], latt[MO_HIDDEN], lmlp[MO_FF];
    float *scores;
};

/* reference csrc/src/weights.cpp:27-125: "MOSW", u32 version=1, u32 n; 80-byte
 * entries (name[48], u8 dtype, u8 ndim, dims u32[3] @52, offset u64 @64,
 * nbytes u64 @72).  ndim==1 or dims (1,n,1) is an fp32 vector. */
typedef struct {
    char name[49];
    uint8_t dtype, ndim;
    uint32_t dims[3];
    uint64_t off, nbytes;
} mo_entry;

static int find_entry(const uint8_t *blob, size_t bytes, const char *name, mo_entry *e) {
    uint32_t n;
    memcpy(&n, blob + 8, 4);
    for (uint32_t i = 0; i < n; ++i) {
        size_t base = 16 + (size_t)i * 80;
        if (base + 80 > bytes) return 0;
        char nm[49];
        memcpy(nm, blob + base, 48);
        nm[48] = 0;
        if (strcmp(nm, name) != 0) continue;
        memcpy(e->name, nm, 49);
        e->dtype = blob[base + 48];
        e->ndim = blob[base + 49];
        memcpy(e->dims, blob + base + 52, 12);
        memcpy(&e->off, blob + base + 64, 8);
        memcpy(&e->nbytes, blob + base + 72, 8);
        if (e->off + e->nbytes > bytes) return 0;
        return 1;
    }
    return 0;
}

static int get_vec(mo_model *m, const char *name, mo_vec *v, char *err) {
    mo_entry e;
    if (!find_entry(m->blob, m->bytes, name, &e) || !(e.ndim == 1 || (e.dims[0] == 1 && e.dims[2] == 1))) {
        if (err) snprintf(err, 256, "missing vector: %s", name);
        return 0;
    }
    v->data = (const float *)(m->blob + e.off);
    v->n = (int)(e.dims[0] * e.dims[1]);
    return 1;
}

static int get_mat(mo_model *m, const char *name, mo_mat *mt, char *err) {
    mo_entry e;
    if (!find_entry(m->blob, m->bytes, name, &e) || e.ndim == 1 || (e.dims[0] == 1 && e.dims[2] == 1) ||
        e.dtype != 4) {
        if (err) snprintf(err, 256, "missing Q8_0_4X4 matrix: %s", name);
        return 0;
    }
    mt->data = m->blob + e.off;
    mt->rows = (int)e.dims[0];
    mt->cols = (int)e.dims[1];
    return 1;
}

static int load_layer(mo_model *m, mo_layer *L, const char *p, char *err) {
    char nm[64];
#define V(field, suffix) snprintf(nm, sizeof nm, "%s" suffix, p); if (!get_vec(m, nm, &L->field, err)) return 0;
#define M(field, suffix) snprintf(nm, sizeof nm, "%s" suffix, p); if (!get_mat(m, nm, &L->field, err)) return 0;
    V(ln1_w, "ln1.w") V(ln1_b, "ln1.b") V(ln2_w, "ln2.w") V(ln2_b, "ln2.b")
    M(attn_w, "attn.w") V(attn_b, "attn.b") M(proj_w, "proj.w") V(proj_b, "proj.b")
    M(fc_in_w, "fc_in.w") V(fc_in_b, "fc_in.b") M(fc_out_w, "fc_out.w") V(fc_out_b, "fc_out.b")
#undef V
#undef M
    return 1;
}

mo_model *mo_model_create(const uint8_t *blob, size_t bytes, int max_ctx, char *err) {
    if (bytes < 16 || memcmp(blob, "MOSW", 4) != 0) {
        if (err) snprintf(err, 256, "not a .moss v1 blob");
        return NULL;
    }
    uint32_t ver;
    memcpy(&ver, blob + 4, 4);
    if (ver != 1) {
        if (err) snprintf(err, 256, "unsupported .moss version %u", ver);
        return NULL;
    }
    mo_model *m = (mo_model *)calloc(1, sizeof(mo_model));
    m->blob = blob;
    m->bytes = bytes;
    m->max_ctx = max_ctx > 0 ? max_ctx : MO_MAX_CTX;
    char nm[64];
    int ok = 1;
    for (int i = 0; i < MO_LAYERS && ok; ++i) {
        snprintf(nm, sizeof nm, "g%d.", i);
        ok = load_layer(m, &m->g[i], nm, err);
    }
    ok = ok && load_layer(m, &m->local, "local.", err);
    ok = ok && get_vec(m, "lnf.w", &m->lnf_w, err) && get_vec(m, "lnf.b", &m->lnf_b, err);
    ok = ok && get_vec(m, "local.lnf.w", &m->llnf_w, err) && get_vec(m, "local.lnf.b", &m->llnf_b, err);
    ok = ok && get_mat(m, "wte", &m->wte, err);
    for (int ch = 0; ch < MO_NVQ && ok; ++ch) {
        snprintf(nm, sizeof nm, "aemb.%d", ch);
        ok = get_mat(m, nm, &m->aemb[ch], err);
    }
    if (!ok) {
        free(m);
        return NULL;
    }
    size_t kv = (size_t)MO_LAYERS * m->max_ctx * MO_HIDDEN;
    m->gk = (float *)calloc(kv, sizeof(float));
    m->gv = (float *)calloc(kv, sizeof(float));
    m->lk = (float *)calloc((size_t)MO_LOCAL_LEN * MO_HIDDEN, sizeof(float));
    m->lv = (float *)calloc((size_t)MO_LOCAL_LEN * MO_HIDDEN, sizeof(float));
    m->cos_t = (float *)malloc((size_t)m->max_ctx * (MO_HIDDEN / 2) * sizeof(float));
    m->sin_t = (float *)malloc((size_t)m->max_ctx * (MO_HIDDEN / 2) * sizeof(float));
    m->scores = (float *)malloc((size_t)m->max_ctx * sizeof(float));
    mo_rope_tables(m->max_ctx, m->cos_t, m->sin_t);
    return m;
}

void mo_model_destroy(mo_model *m) {
    if (!m) return;
    free(m->gk);
    free(m->gv);
    free(m->lk);
    free(m->lv);
    free(m->cos_t);
    free(m->sin_t);
    free(m->scores);
    free(m);
}

void mo_model_set_kv_f16(mo_model *m, int on) { m->kv_f16 = on; }
void mo_model_set_decode_a8(mo_model *m, int on) { m->decode_a8 = on; }

/* gemv_par in decode (reference csrc/src/gemv.cpp:229-274): W8A16 rows
 * (row_dot_q8_4x4_actf32) when act16_enabled(), else the activation quantised
 * once per 32-block (quantize_activation, quant.cpp:45-54) and W8A8 rows
 * (row_dot_q8_4x4, gemv_avx2.cpp:105-121) -- the reference's default mode. */
static void decode_gemv(const mo_model *m, const uint8_t *w, int rows, int cols, const float *x, float *y) {
    if (!m->decode_a8) {
        mo_gemv_a16(w, rows, cols, x, y);
        return;
    }
    int nb = cols / 32;
    int8_t *q = (int8_t *)malloc((size_t)cols);
    float *d = (float *)malloc(sizeof(float) * (size_t)nb);
    mo_quantize_row_q8(x, cols, q, NULL, d);
#pragma omp parallel for schedule(static) if (rows >= 512)
    for (int r = 0; r < rows; ++r) y[r] = mo_row_dot_w8a8(w + (size_t)(r / 4) * nb * 136, nb, r % 4, q, d);
    free(q);
    free(d);
}
void mo_model_reset(mo_model *m) { m->pos = 0; }
int mo_model_position(const mo_model *m) { return m->pos; }
const float *mo_model_hidden(const mo_model *m) { return m->hidden; }
void mo_model_set_hidden(mo_model *m, const float *h) { memcpy(m->hidden, h, sizeof m->hidden); }

int mo_model_kv_import(mo_model *m, int n_pos, const float *k, const float *v) {
    if (n_pos < 0 || n_pos > m->max_ctx) return -1;
    for (int l = 0; l < MO_LAYERS; ++l) {
        memcpy(m->gk + (size_t)l * m->max_ctx * MO_HIDDEN, k + (size_t)l * n_pos * MO_HIDDEN,
               sizeof(float) * (size_t)n_pos * MO_HIDDEN);
        memcpy(m->gv + (size_t)l * m->max_ctx * MO_HIDDEN, v + (size_t)l * n_pos * MO_HIDDEN,
               sizeof(float) * (size_t)n_pos * MO_HIDDEN);
    }
    m->pos = n_pos;
    return 0;
}

int mo_model_kv_export(const mo_model *m, int n_pos, float *k, float *v) {
    if (n_pos < 0 || n_pos > m->max_ctx) return -1;
    for (int l = 0; l < MO_LAYERS; ++l) {
        memcpy(k + (size_t)l * n_pos * MO_HIDDEN, m->gk + (size_t)l * m->max_ctx * MO_HIDDEN,
               sizeof(float) * (size_t)n_pos * MO_HIDDEN);
        memcpy(v + (size_t)l * n_pos * MO_HIDDEN, m->gv + (size_t)l * m->max_ctx * MO_HIDDEN,
               sizeof(float) * (size_t)n_pos * MO_HIDDEN);
    }
    return 0;
}

static void lookup_row(const mo_mat *mt, int row, float *out) {
    int nb = mt->cols / 32;
    mo_dequant_row_q8x4(mt->data + (size_t)(row / 4) * nb * 136, nb, row % 4, out);
}

/* reference csrc/src/llm.cpp:148-157 */
void mo_model_embed_row(const mo_model *m, const int32_t *row, float *out) {
    lookup_row(&m->wte, row[0], out);
    float tmp[MO_HIDDEN];
    for (int ch = 0; ch < MO_NVQ; ++ch) {
        int code = row[ch + 1];
        if (code == MO_AUDIO_PAD || code < 0 || code >= MO_CODEBOOK) continue;
        lookup_row(&m->aemb[ch], code, tmp);
        for (int i = 0; i < MO_HIDDEN; ++i) out[i] += tmp[i];
    }
}

static float kv_round(const mo_model *m, float v) {
    return m->kv_f16 ? mo_half_to_float(mo_float_to_half_rne(v)) : v;
}

/* reference csrc/src/llm.cpp:219-246 (attention + block_forward) */
static void block_forward(mo_model *m, const mo_layer *L, int local, int layer, int pos, float *x, float *qkv,
                          float *att, float *mlp) {
    mo_layernorm(x, L->ln1_w.data, L->ln1_b.data, m->ln);
    decode_gemv(m, L->attn_w.data, 3 * MO_HIDDEN, MO_HIDDEN, m->ln, qkv);
    for (int i = 0; i < 3 * MO_HIDDEN; ++i) qkv[i] += L->attn_b.data[i];
    mo_rope_apply(qkv, pos, m->cos_t, m->sin_t);
    mo_rope_apply(qkv + MO_HIDDEN, pos, m->cos_t, m->sin_t);
    float *kc = local ? m->lk : m->gk + (size_t)layer * m->max_ctx * MO_HIDDEN;
    float *vc = local ? m->lv : m->gv + (size_t)layer * m->max_ctx * MO_HIDDEN;
    for (int i = 0; i < MO_HIDDEN; ++i) {
        kc[(size_t)pos * MO_HIDDEN + i] = local ? qkv[MO_HIDDEN + i] : kv_round(m, qkv[MO_HIDDEN + i]);
        vc[(size_t)pos * MO_HIDDEN + i] = local ? qkv[2 * MO_HIDDEN + i] : kv_round(m, qkv[2 * MO_HIDDEN + i]);
    }
    mo_attention_core(kc, vc, MO_HIDDEN, pos + 1, qkv, att, m->scores);
    decode_gemv(m, L->proj_w.data, MO_HIDDEN, MO_HIDDEN, att, m->res);
    for (int i = 0; i < MO_HIDDEN; ++i) x[i] += m->res[i] + L->proj_b.data[i];
    mo_layernorm(x, L->ln2_w.data, L->ln2_b.data, m->ln);
    decode_gemv(m, L->fc_in_w.data, MO_FF, MO_HIDDEN, m->ln, mlp);
    for (int i = 0; i < MO_FF; ++i) mlp[i] = mo_gelu_new(mlp[i] + L->fc_in_b.data[i]);
    decode_gemv(m, L->fc_out_w.data, MO_HIDDEN, MO_FF, mlp, m->res);
    for (int i = 0; i < MO_HIDDEN; ++i) x[i] += m->res[i] + L->fc_out_b.data[i];
}

/* reference csrc/src/llm.cpp:248-255 */
void mo_model_global_step(mo_model *m, const int32_t *row) {
    mo_model_embed_row(m, row, m->x);
    for (int i = 0; i < MO_LAYERS; ++i) block_forward(m, &m->g[i], 0, i, m->pos, m->x, m->qkv, m->att, m->mlp);
    mo_layernorm(m->x, m->lnf_w.data, m->lnf_b.data, m->hidden);
    ++m->pos;
}

void mo_model_local_reset(mo_model *m) { m->lpos = 0; }

/* reference csrc/src/llm.cpp:259-264 */
void mo_model_local_step(mo_model *m, const float *in, float *out) {
    memcpy(m->lx, in, sizeof m->lx);
    block_forward(m, &m->local, 1, 0, m->lpos, m->lx, m->lqkv, m->latt, m->lmlp);
    mo_layernorm(m->lx, m->llnf_w.data, m->llnf_b.data, out);
    ++m->lpos;
}

/* reference csrc/src/llm.cpp:268-270 */
void mo_model_audio_logits(mo_model *m, int ch, const float *hidden, float *logits) {
    decode_gemv(m, m->aemb[ch].data, MO_CODEBOOK, MO_HIDDEN, hidden, logits);
}

/* reference csrc/src/llm.cpp:266 (text_logits: gemv_par over wte) */
void mo_model_text_logits(mo_model *m, const float *hidden, float *logits) {
    decode_gemv(m, m->wte.data, MO_VOCAB, MO_HIDDEN, hidden, logits);
}

/* reference csrc/src/llm.cpp:274-315 (Q8_0_4X4 branch: W8A8 AVX2 row dot on
 * rows 7 (end) and 9 (slot) of wte) */
void mo_model_assistant_logits(mo_model *m, const float *hidden, float *pair) {
    int8_t q[MO_HIDDEN];
    float d[MO_HIDDEN / 32];
    mo_quantize_row_q8(hidden, MO_HIDDEN, q, NULL, d);
    const int rows[2] = {MO_END, MO_SLOT};
    int nb = MO_HIDDEN / 32;
    for (int i = 0; i < 2; ++i) {
        int r = rows[i];
        pair[i] = mo_row_dot_w8a8(m->wte.data + (size_t)(r / 4) * nb * 136, nb, r % 4, q, d);
    }
}

/* reference csrc/src/llm.cpp:327-401 */
void mo_model_prefill(mo_model *m, const int32_t *rows, int n_rows, int start, int a16) {
    if (start < 0) start = 0;
    if (start > m->max_ctx) start = m->max_ctx;
    int mrows = n_rows < m->max_ctx - start ? n_rows : m->max_ctx - start;
    if (mrows <= 0) return;
    size_t H = MO_HIDDEN;
    float *bx = (float *)malloc(sizeof(float) * mrows * H);
    float *bln = (float *)malloc(sizeof(float) * mrows * H);
    float *bqkv = (float *)malloc(sizeof(float) * mrows * 3 * H);
    float *batt = (float *)malloc(sizeof(float) * mrows * H);
    float *bmlp = (float *)malloc(sizeof(float) * mrows * MO_FF);
    float *bres = (float *)malloc(sizeof(float) * mrows * H);
    for (int i = 0; i < mrows; ++i) mo_model_embed_row(m, rows + (size_t)i * 17, bx + i * H);
    for (int layer = 0; layer < MO_LAYERS; ++layer) {
        const mo_layer *L = &m->g[layer];
        float *kc = m->gk + (size_t)layer * m->max_ctx * H;
        float *vc = m->gv + (size_t)layer * m->max_ctx * H;
        for (int i = 0; i < mrows; ++i) mo_layernorm(bx + i * H, L->ln1_w.data, L->ln1_b.data, bln + i * H);
        mo_gemm(L->attn_w.data, 3 * MO_HIDDEN, MO_HIDDEN, bln, mrows, bqkv, a16);
        for (int i = 0; i < mrows; ++i) {
            float *qkv = bqkv + (size_t)i * 3 * H;
            int p = start + i;
            for (int k = 0; k < 3 * MO_HIDDEN; ++k) qkv[k] += L->attn_b.data[k];
            mo_rope_apply(qkv, p, m->cos_t, m->sin_t);
            mo_rope_apply(qkv + H, p, m->cos_t, m->sin_t);
            for (size_t k = 0; k < H; ++k) {
                kc[(size_t)p * H + k] = kv_round(m, qkv[H + k]);
                vc[(size_t)p * H + k] = kv_round(m, qkv[2 * H + k]);
            }
        }
        for (int i = 0; i < mrows; ++i)
            mo_attention_core(kc, vc, MO_HIDDEN, start + i + 1, bqkv + (size_t)i * 3 * H, batt + i * H, m->scores);
        mo_gemm(L->proj_w.data, MO_HIDDEN, MO_HIDDEN, batt, mrows, bres, a16);
        for (int i = 0; i < mrows; ++i)
            for (size_t k = 0; k < H; ++k) bx[i * H + k] += bres[i * H + k] + L->proj_b.data[k];
        for (int i = 0; i < mrows; ++i) mo_layernorm(bx + i * H, L->ln2_w.data, L->ln2_b.data, bln + i * H);
        mo_gemm(L->fc_in_w.data, MO_FF, MO_HIDDEN, bln, mrows, bmlp, a16);
        for (int i = 0; i < mrows; ++i)
            for (int k = 0; k < MO_FF; ++k)
                bmlp[(size_t)i * MO_FF + k] = mo_gelu_new(bmlp[(size_t)i * MO_FF + k] + L->fc_in_b.data[k]);
        mo_gemm(L->fc_out_w.data, MO_HIDDEN, MO_FF, bmlp, mrows, bres, a16);
        for (int i = 0; i < mrows; ++i)
            for (size_t k = 0; k < H; ++k) bx[i * H + k] += bres[i * H + k] + L->fc_out_b.data[k];
    }
    mo_layernorm(bx + (size_t)(mrows - 1) * H, m->lnf_w.data, m->lnf_b.data, m->hidden);
    m->pos = start + mrows;
    free(bx);
    free(bln);
    free(bqkv);
    free(batt);
    free(bmlp);
    free(bres);
}

/* reference csrc/src/llm.cpp:30-35 */
static int end_reached(float l_slot, float l_end, const mo_sample_params *p, mo_rng *rng) {
    if (p->end_greedy) return l_end > l_slot;
    double d = (double)l_end - (double)l_slot;
    if (d < -80.0) d = -80.0;
    if (d > 80.0) d = 80.0;
    float p_slot = (float)(1.0 / (1.0 + exp(d)));
    return mo_rng_uniform(rng) >= p_slot;
}

/* reference csrc/src/llm.cpp:634-713 */
int mo_model_generate(mo_model *m, int max_frames, const mo_sample_params *p, uint64_t seed,
                      const int32_t *forced, int n_forced, int32_t *out_rows, float *logits_dump,
                      float *gate_out) {
    mo_rng rng;
    mo_rng_seed(&rng, seed);
    int *hist = (int *)malloc(sizeof(int) * (size_t)MO_NVQ * (max_frames > 0 ? max_frames : 1));
    int hist_n = 0;
    void *scratch = malloc((size_t)MO_CODEBOOK * 8);
    float *text = gate_out ? (float *)malloc(sizeof(float) * MO_VOCAB) : NULL;
    float logits[MO_CODEBOOK];
    float lx[MO_HIDDEN], input[MO_HIDDEN];
    int frames = 0;
    if (forced && n_forced < max_frames) max_frames = n_forced;
    for (int f = 0; f < max_frames; ++f) {
        if (m->pos >= m->max_ctx) break;
        mo_model_local_reset(m);
        mo_model_local_step(m, m->hidden, lx);
        float l_end, l_slot;
        if (gate_out) {
            /* gate-dump path (llm.cpp:653-679): the whole text head, its argmax
             * (first maximum wins) and the gate logits taken from it */
            mo_model_text_logits(m, lx, text);
            int am = 0;
            float av = text[0];
            for (int v = 1; v < MO_VOCAB; ++v)
                if (text[v] > av) {
                    av = text[v];
                    am = v;
                }
            l_slot = text[MO_SLOT];
            l_end = text[MO_END];
            gate_out[4 * f] = l_end;
            gate_out[4 * f + 1] = l_slot;
            gate_out[4 * f + 2] = (float)am;
            gate_out[4 * f + 3] = av;
        } else {
            float pair[2];
            mo_model_assistant_logits(m, lx, pair);
            l_end = pair[0];
            l_slot = pair[1];
        }
        if (f >= p->min_frames && end_reached(l_slot, l_end, p, &rng)) break;
        int32_t frame[17];
        memset(frame, 0, sizeof frame);
        lookup_row(&m->wte, MO_SLOT, input);
        mo_sample_params fp = *p;
        if (f < p->greedy_frames) fp.greedy = 1;
        for (int ch = 0; ch < MO_NVQ; ++ch) {
            mo_model_local_step(m, input, lx);
            mo_model_audio_logits(m, ch, lx, logits);
            if (logits_dump) memcpy(logits_dump + ((size_t)f * MO_NVQ + ch) * MO_CODEBOOK, logits, sizeof logits);
            /* history of channel ch = hist[ch*max_frames .. +hist_n) */
            int pred = mo_sample_token(logits, MO_CODEBOOK, &fp, hist + (size_t)ch * max_frames, hist_n, &rng,
                                       scratch);
            int used = forced ? forced[(size_t)f * 17 + ch + 1] : pred;
            frame[ch + 1] = pred;
            hist[(size_t)ch * max_frames + hist_n] = used;
            lookup_row(&m->aemb[ch], used, input);
        }
        ++hist_n;
        memcpy(out_rows + (size_t)f * 17, frame, sizeof frame);
        frames = f + 1;
        if (f + 1 < max_frames && m->pos < m->max_ctx) {
            int32_t next[17];
            next[0] = MO_SLOT;
            for (int ch = 0; ch < MO_NVQ; ++ch) next[ch + 1] = forced ? forced[(size_t)f * 17 + ch + 1] : frame[ch + 1];
            mo_model_global_step(m, next);
        }
    }
    free(hist);
    free(scratch);
    free(text);
    return frames;
}
