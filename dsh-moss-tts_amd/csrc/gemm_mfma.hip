// gemm_mfma.hip -- W8A16 GEMM over the native Q8_0_4X4 layout on CDNA4 matrix cores.
//
// Replaces gemm_par (reference csrc/include/moss/gemv.h:54, csrc/src/gemv.cpp:276-309)
// in its A16 mode -- Y[m][n] = sum_b fp32(d[n,b]) * sum_i q[n,b,i] * x[m][32b+i] --
// for M >= 16 rows: prefill (M = prompt rows) and batched multi-stream decode
// (M = streams).
//
// v_mfma_f32_16x16x32_f16: one instruction covers one 32-column scale block.
// Lane l holds A[row l%16][k 8(l/16)..+7], B[k 8(l/16)..+7][col l%16] and gets
// D[row 4(l/16)+i][col l%16].  B is the weight row n = col: 8 consecutive int8
// of one row of the 4x4 block (one 8-byte load), exact in fp16.  A is the fp32
// activation split as x = hi + lo (hi = fp16(x) toward zero, lo = fp16(x - hi)): two
// MFMAs (hi, lo) give the block dot to ~2^-22 relative, then the fp32 block
// scale d[n,b] (the same for all 4 values a lane holds) is applied with an FMA
// into the fp32 accumulator -- the reference's per-block scale-then-accumulate
// order.
//
// Workgroup tile: 16 rows x 16*NT columns; grid (N / (16 NT), ceil(M / 16),
// K slices).  The 4 waves split the slice's blocks and sum in LDS; each wave
// streams its A rows and B columns KB blocks at a time, two chunks in flight.
#include "mh_ops.h"

namespace mh {
#ifdef MH_GEMM_TRACE
// Start and end time (100 MHz device clock) of every workgroup of the last
// launch, in builds with -DMH_GEMM_TRACE only (a profiling build).
__device__ unsigned long long mh_gemm_ts[8192][2];
#define GT_START const unsigned long long gt0_ = __builtin_amdgcn_s_memrealtime();
#define GT_END                                                                           \
    if (threadIdx.x == 0) {                                                              \
        const int id_ = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z); \
        if (id_ < 8192) {                                                                \
            mh_gemm_ts[id_][0] = gt0_;                                                   \
            mh_gemm_ts[id_][1] = __builtin_amdgcn_s_memrealtime();                       \
        }                                                                                \
    }
#else
#define GT_START
#define GT_END
#endif
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

#ifndef MH_GEMM_KB
#define MH_GEMM_KB 3
#endif
// scale blocks per load chunk: 3 divides every per-wave block count of the model's
// GEMMs (K = 768: 6 per wave, or 3 per wave in two K slices; K = 3072: 24 or 12)
constexpr int KB = MH_GEMM_KB;


// x = hi + lo: hi rounds toward zero (v_cvt_pkrtz, two values per
// instruction), so x - hi is exact in fp32; lo keeps the next ~10 bits.
__device__ __forceinline__ void split_hi_lo(const float (&x)[8], half8 &hi, half8 &lo) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto h = __builtin_amdgcn_cvt_pkrtz(x[2 * i], x[2 * i + 1]);
        const auto l = __builtin_amdgcn_cvt_pkrtz(x[2 * i] - (float)h[0], x[2 * i + 1] - (float)h[1]);
        hi[2 * i] = (_Float16)h[0];
        hi[2 * i + 1] = (_Float16)h[1];
        lo[2 * i] = (_Float16)l[0];
        lo[2 * i + 1] = (_Float16)l[1];
    }
}

// What the epilogue needs of a lane's row, computed once: a lane stores one row
// of every column subtile of its tile.  A tile (16, 32 or 64 columns) lies inside
// one section (q, k or v) and one head of the QKV output.
struct EpiRow {
    float *out = nullptr;        // the row's output at column 0 (q_out's row under QKV)
    const float *res = nullptr;  // EPI_RESID: the row's residual input
    const float *rc = nullptr, *rs = nullptr;  // EPI_QKV: RoPE factors at the row's position
    void *pool = nullptr;        // EPI_QKV, k or v section: the row's K/V slot (d = 0) in its page
    int sec = 0;                 // EPI_QKV: 0 q, 1 k, 2 v
    uint8_t *hl = nullptr;       // EPI_GELU with y_hl: the output as hi/lo halves (hlt_at), row m, width N
    int m = 0, N = 0;
};

template <int EPI, int KV>
__device__ __forceinline__ EpiRow epi_row(const GemmArgs &g, int m, int n_base) {
    EpiRow r;
    const int mm = min(m, g.M - 1);  // rows past M store nothing; their lookups stay in bounds
    if constexpr (EPI == EPI_PART) {
        r.out = g.part + ((size_t)blockIdx.z * g.M + mm) * g.N;
    } else if constexpr (EPI == EPI_F32 || EPI == EPI_GELU) {
        r.out = g.y ? g.y + (size_t)mm * g.ldy : nullptr;
        if constexpr (EPI == EPI_GELU) {
            r.hl = g.y_hl;
            r.m = mm;
            r.N = g.N;
        }
    } else if constexpr (EPI == EPI_RESID) {
        r.out = g.y + (size_t)mm * g.ldy;
        r.res = g.resid_in ? g.resid_in + (size_t)mm * g.resid_stride : r.out;
        r.hl = g.y_hl;
        r.m = mm;
        r.N = g.N;
    } else {  // EPI_QKV
        r.sec = n_base / kHidden;
        const int h = (n_base - r.sec * kHidden) >> 6;
        const int s = g.row_stream ? g.row_stream[mm] : mm * g.stream_stride;
        const int pos = g.row_pos ? g.row_pos[mm] : g.pos0 + mm * g.pos_stride;
        r.rc = g.rope_cos + (size_t)pos * kRopeHalf;
        r.rs = g.rope_sin + (size_t)pos * kRopeHalf;
        if (r.sec == 0) {
            r.out = g.q_out + (size_t)mm * kHidden;
        } else if (g.row_active == nullptr || g.row_active[mm]) {
            const int page = g.page_table ? g.page_table[(size_t)s * g.table_stride + pos / g.page_size] : s;
            const size_t slot = (((size_t)page * kHeads + h) * g.page_size + pos % g.page_size) * kHeadDim;
            void *pool = r.sec == 1 ? g.k_pool : g.v_pool;
            r.pool = KV == KV_F16 ? (void *)((__half *)pool + slot) : (void *)((float *)pool + slot);
        }
    }
    return r;
}

// The epilogue's operands of a lane's NT values (column n_base + 16t + l16 of its row):
// loaded when the workgroup starts, so they are in registers when the sums are.
template <int NT>
struct EpiOps {
    float b[NT], bp[NT], c[NT], sn[NT], res[NT];  // bias, partner column's bias, RoPE, residual
};

template <int EPI, int NT>
__device__ __forceinline__ void epi_load(const GemmArgs &g, const EpiRow &r, int n_base, int l16, EpiOps<NT> &o) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int n = n_base + 16 * t + l16;
        if constexpr (EPI == EPI_RESID || EPI == EPI_GELU || EPI == EPI_QKV) o.b[t] = g.bias[n];
        if constexpr (EPI == EPI_RESID) o.res[t] = r.res[n];
        if constexpr (EPI == EPI_QKV) {
            // loaded for the v section too, where RoPE does not apply (the addresses are valid
            // there as well): conditionally filled, the arrays were kept in private memory
            const int d = n & 63;
            o.bp[t] = g.bias[n ^ 1];
            o.c[t] = r.rc[d >> 1];
            o.sn[t] = r.rs[d >> 1];
        }
    }
}

template <int EPI, int KV, int NT>
__device__ __forceinline__ void gemm_finish(const EpiRow &r, const EpiOps<NT> &o, int t, int n, float v,
                                            float partner) {
#pragma clang fp contract(off)
    if constexpr (EPI == EPI_PART || EPI == EPI_F32) {
        r.out[n] = v;
    } else if constexpr (EPI == EPI_RESID) {
        const float y = o.res[t] + (v + o.b[t]);
        r.out[n] = y;
        if (r.hl != nullptr) store_hl(r.hl, r.m, n, r.N, y);  // uniform
    } else if constexpr (EPI == EPI_GELU) {
        const float hv = gelu_new(v + o.b[t]);
        if (r.hl != nullptr)  // uniform: the next GEMM reads the hi/lo halves
            store_hl(r.hl, r.m, n, r.N, hv);
        else
            r.out[n] = hv;
    } else {  // EPI_QKV: bias, RoPE at the row's position, q -> q_out, k/v -> KV pages
        const float val = v + o.b[t];
        const int d = n & 63;
        float out = val;
        if (r.sec < 2) {
            const float pv = partner + o.bp[t];
            const float p0 = val * o.c[t], p1 = pv * o.sn[t];
            out = (d & 1) == 0 ? p0 - p1 : p0 + p1;
        }
        if (r.sec == 0) {
            r.out[n] = out;
        } else if (r.pool != nullptr) {
            if constexpr (KV == KV_F16)
                ((__half *)r.pool)[d] = __float2half_rn(out);
            else
                ((float *)r.pool)[d] = out;
        }
    }
}


// Operands through buffer resources: the lane's byte offset at the wave's first
// block is one VGPR per operand; the block within a chunk is the instruction's
// immediate offset and the chunk base and column subtile an SGPR offset, so a
// load costs no address arithmetic.  A load past a resource's last byte returns
// 0 instead of faulting, so every load is unconditional (blocks past the wave's
// last one, or rows past M, are read and never used).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 raw buffer word 3 (32-bit data format)

__device__ __forceinline__ rsrc_t make_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, kRsrcWord3);
}

// Weights in the matrix-core order (tile_q8x4_mfma): for each 16-row subtile s
// of W and scale block b, one 544-byte unit at (s * K/32 + b) * 544 holding the
// 512 quants in MFMA lane order -- lane l = c + 16 kq takes the 8 bytes at 8 l
// (row 16 s + c, columns 32 b + 8 kq .. + 7) as its B operand -- then the 16
// rows' fp16 scales.  A column-subtile load is 4 whole 128-byte lines; in the
// Q8_0_4X4 order it gathers 4 groups' 128-byte runs that start 8 bytes into
// 136-byte blocks (8 lines), plus 4 more lines for the scales.

template <bool A8>
struct Src {
    rsrc_t a, ad, w;  // activations (fp32, or int8 under W8A8), their block scales, weights
    int va, vad;      // lane offsets of the activations and their scale at the wave's first block
    int vw, vs;       // lane offsets of its weight run and its column's scale (column subtile 0)
    int wt;           // bytes from one 16-column subtile to the next (4 groups)
};

// One chunk of KB scale blocks: this lane's 8 activations per block (fp32, or
// int8 + the block scale of the lane's row under W8A8) and its 8 weights +
// scale per block and column subtile.
template <int NT, bool A8, bool AT>
struct Chunk {
    float xa[(A8 || AT) ? 1 : KB][8];
    half8 xh[(!A8 && AT) ? KB : 1], xl[(!A8 && AT) ? KB : 1];  // fp32 activations pre-split (a_hl)
    uint64_t xq[A8 ? KB : 1];
    float xd[A8 ? KB : 1];
    uint2 qb[KB][NT];
    uint32_t db[KB][NT];
};

// weights: default caching -- every row tile of the launch reads them again (a
// non-temporal hint measured slower end to end: 0.83 vs 0.78 ms per 256-row prefill)
constexpr int kCpolW = 0;

// AT: activations in the matrix-core order -- W8A8: q8t_at / d8t_at, a block of the
// wave's 16 rows is one 512-byte unit and 16 scales; fp32: hlt_at, the block's hi and
// lo fp16 halves are two 1024-byte runs, loaded as the MFMA's A operands
template <int NT, bool A8, bool AT>
__device__ __forceinline__ void load_chunk_a(Chunk<NT, A8, AT> &c, int b0, const Src<A8> &s) {
    constexpr int QB = AT ? 512 : 32, DB = AT ? 64 : 4;  // bytes from one block to the next
#pragma unroll
    for (int j = 0; j < KB; ++j) {
        if constexpr (A8) {
            const auto q = __builtin_amdgcn_raw_buffer_load_b64(s.a, s.va + QB * j, QB * b0, 0);
            c.xq[j] = ((uint64_t)q[1] << 32) | q[0];
            c.xd[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s.ad, s.vad + DB * j, DB * b0, 0));
        } else if constexpr (AT) {
            c.xh[j] = __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(s.a, s.va + 2048 * j, 2048 * b0, 0));
            c.xl[j] =
                __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(s.a, s.va + 2048 * j + 1024, 2048 * b0, 0));
        } else {
            // the whole vector is reinterpreted: a bit cast of one element of the
            // builtin's vector type reads element 0
            const floatx4 x0 =
                __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(s.a, s.va + 128 * j, 128 * b0, 0));
            const floatx4 x1 = __builtin_bit_cast(
                floatx4, __builtin_amdgcn_raw_buffer_load_b128(s.a, s.va + 128 * j + 16, 128 * b0, 0));
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                c.xa[j][i] = x0[i];
                c.xa[j][4 + i] = x1[i];
            }
        }
    }
}

// TL: weights in the matrix-core order (one 544-byte unit per subtile and block)
// instead of Q8_0_4X4 (4 groups of 136-byte blocks per subtile)
template <int NT, bool A8, bool AT, bool TL>
__device__ __forceinline__ void load_chunk_b(Chunk<NT, A8, AT> &c, int b0, const Src<A8> &s) {
    constexpr int UB = TL ? kTileBytes : kBlockBytes;  // bytes from one block to the next
#pragma unroll
    for (int j = 0; j < KB; ++j) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int so = t * s.wt + UB * b0;
            const auto q = __builtin_amdgcn_raw_buffer_load_b64(s.w, s.vw + UB * j, so, kCpolW);
            c.qb[j][t] = make_uint2(q[0], q[1]);
            c.db[j][t] = __builtin_amdgcn_raw_buffer_load_b16(s.w, s.vs + UB * j, so, 0);
        }
    }
}

template <int NT, bool A8, bool TL, bool AT>
__device__ __forceinline__ void load_chunk(Chunk<NT, A8, AT> &c, int b0, const Src<A8> &s) {
    load_chunk_a<NT, A8, AT>(c, b0, s);
    load_chunk_b<NT, A8, AT, TL>(c, b0, s);
}


template <int NT, bool A8, bool AT>
__device__ __forceinline__ void mfma_chunk(const Chunk<NT, A8, AT> &c, int b0, int nb, int kq, floatx4 (&acc)[NT]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < KB; ++j) {
        const bool live = b0 + j < nb;  // uniform
        if (!live) break;               // blocks past the wave's last one (loaded, clamped) are skipped
        if constexpr (A8) {
            // W8A8 (gemv_avx2.cpp:105-121): the exact int32 block dot, times
            // scale = d_w * d_a (fp32), accumulated with an FMA.  D row 4kq + i
            // takes d_a from the lane that loaded that A row.
            float da[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) da[i] = __shfl(c.xd[j], 4 * kq + i);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const long bq = (long)(((uint64_t)c.qb[j][t].y << 32) | c.qb[j][t].x);
                const intx4 p = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)c.xq[j], bq, intx4{0, 0, 0, 0}, 0, 0, 0);
                const float dw = h2f((uint16_t)c.db[j][t]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float scale = dw * da[i];
                    acc[t][i] = fmaf((float)p[i], scale, acc[t][i]);
                }
            }
        } else {
            half8 hi, lo;
            if constexpr (AT) {
                hi = c.xh[j];
                lo = c.xl[j];
            } else {
                split_hi_lo(c.xa[j], hi, lo);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const half8 bw = i8x8_to_h8(c.qb[j][t]);
                floatx4 blk = floatx4{0.f, 0.f, 0.f, 0.f};
                blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, bw, blk, 0, 0, 0);
                blk = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, bw, blk, 0, 0, 0);
                const float d = h2f((uint16_t)c.db[j][t]);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(blk[i], d, acc[t][i]);
            }
        }
    }
}

// The 4 waves of a 16 x 16*NT tile take the 4
// quarters of the K slice (grid z) and meet in LDS, summed in wave order
// (w0 + w1) + w2) + w3, and each wave finishes NT of the 4*NT (subtile, row)
// pairs.  A workgroup reads 16 activation rows instead of 64: the panel is
// what limits a GEMM with M <= 64, read by every column tile.
//
// LN: the activation rows are LayerNormed on the way in.  From fp32 rows (AT =
// false): the wave's whole K quarter (at most 8 blocks: K <= 1024) is loaded first,
// the row sums of the 4 waves meet in LDS (two passes: mean, then the squared
// deviations), and the values are normalised in registers with ln_w / ln_b staged
// in LDS.  From pre-split rows (AT = true, K = 768): the statistics come from the
// producer (ln_rows_from_stats) and the chunks stream as in the plain loop.
// LayerNorm row statistics of a workgroup's 16 rows (K = 768) from a producer's
// per-16-column (mean, M2) pairs (GemmArgs::ln_stats), combined in a fixed order (Chan
// et al.'s pairwise update; every merge is symmetric in its two sides, so all lanes
// agree); ln_w / ln_b are staged in lw2 / lb2.  Returns (mean, 1 / sqrt(var + eps)) of
// row m_base + l16 after one barrier.
__device__ __forceinline__ float2 ln_rows_from_stats(const GemmArgs &g, int m_base, int l16, float *lw2, float *lb2,
                                                     float2 *rstat) {
#pragma clang fp contract(off)
    const int tr = threadIdx.x >> 4, sub = threadIdx.x & 15;
    const int sr = min(m_base + tr, g.M - 1);
    const float2 *ps = reinterpret_cast<const float2 *>(g.ln_stats);
    float2 p[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) p[i] = ps[(size_t)(3 * sub + i) * g.M + sr];
    float lw[3], lb[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        lw[i] = g.ln_w[threadIdx.x + 256 * i];
        lb[i] = g.ln_b[threadIdx.x + 256 * i];
    }
    // groups 3 sub .. 3 sub + 2 (16 columns each), then the 16 lanes of the row
    float mean = p[0].x, m2 = p[0].y;
    {
        const float d = p[1].x - mean;
        mean = (mean + p[1].x) * 0.5f;
        m2 = (m2 + p[1].y) + d * d * 8.0f;  // 16 x 16 / 32
    }
    {
        const float d = p[2].x - mean;
        mean = mean + d * (1.0f / 3.0f);              // counts 32 and 16
        m2 = (m2 + p[2].y) + d * d * (32.0f / 3.0f);  // 32 x 16 / 48
    }
    float cnt = 48.0f;
#pragma unroll
    for (int k = 1; k < 16; k <<= 1) {
        const float om = __shfl_xor(mean, k), om2 = __shfl_xor(m2, k);
        const float d = om - mean;
        mean = (mean + om) * 0.5f;
        m2 = (m2 + om2) + d * d * (cnt * 0.5f);
        cnt *= 2.0f;
    }
#pragma unroll
    for (int i = 0; i < 3; ++i) {
        lw2[threadIdx.x + 256 * i] = lw[i];
        lb2[threadIdx.x + 256 * i] = lb[i];
    }
    if (sub == 0) rstat[tr] = make_float2(mean, 1.0f / sqrtf(m2 / (float)kHidden + 1e-5f));
    __syncthreads();
    return rstat[l16];
}

// WV: waves per workgroup, 4, or 8 for a long K with the residual epilogue (fc_out, K = 3072:
// 12 blocks per wave, so the sum needs no second kernel); waves 4..7 only contribute partials.
template <int EPI, int KV, int NT, bool A8, bool LN, bool TL, bool AT, int WV = 4>
__global__ __launch_bounds__(64 * WV) void gemm_wk_kernel(GemmArgs g) {
#pragma clang fp contract(off)
    static_assert(WV == 4 || (WV == 8 && EPI == EPI_RESID && !LN), "8 waves: the residual epilogue only");
    GT_START
    __shared__ floatx4 red[WV][NT][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int l16 = lane & 15, kq = lane >> 4;  // kq: which 8-column quarter of the block
    const int m_base = blockIdx.y * 16;
    const int n_base = blockIdx.x * 16 * NT;
    const int nb_all = g.K >> 5;
    // K slice z: blocks [z * nb_all / Z, (z + 1) * nb_all / Z); wave w its w-th quarter
    const int z0 = (int)((blockIdx.z * (unsigned)nb_all) / gridDim.z);
    const int nbz = (int)(((blockIdx.z + 1) * (unsigned)nb_all) / gridDim.z) - z0;
    const int kb0 = z0 + (wave * nbz) / WV;
    const int nb = z0 + ((wave + 1) * nbz) / WV - kb0;  // 0 when the slice has fewer than WV blocks
    const int arow = min(m_base + l16, g.M - 1);      // rows past M read row M-1, never stored
    const int krow = l16 & 3;
    // the epilogue: wave w finishes row 4kq + w of every column subtile; its operands
    // are requested first (loads complete in order, so these never delay the operands')
    const int erow = m_base + 4 * kq + (wave & 3);
    const EpiRow er = epi_row<EPI, KV>(g, erow, n_base);
    EpiOps<NT> eo;
    epi_load<EPI, NT>(g, er, n_base, l16, eo);
    Src<A8> src;
    {
        const uint32_t a_elems = (uint32_t)((g.M - 1) * g.lda + g.K);
        if constexpr (!A8 && AT) {  // hi/lo fp16 units of 2048 bytes (hlt_at), K = lda; rows padded to 16
            const uint32_t units = (uint32_t)((g.M + 15) / 16) * (uint32_t)(g.lda / 32);
            src.a = make_rsrc(g.a_hl, units * 2048u);
            src.va = (int)(((m_base / 16) * (g.lda / 32) + kb0) * 2048) + 16 * lane;
        } else if constexpr (A8 && AT) {  // K = lda; rows padded to 16
            const uint32_t units = (uint32_t)((g.M + 15) / 16) * (uint32_t)(g.lda / 32);
            const int unit = (m_base / 16) * (g.lda / 32) + kb0;  // this row tile's first block
            src.a = make_rsrc(g.a8, units * 512u);
            src.ad = make_rsrc(g.d8, units * 64u);
            src.va = unit * 512 + 8 * lane;
            src.vad = unit * 64 + 4 * l16;
        } else if constexpr (A8) {
            src.a = make_rsrc(g.a8, a_elems);
            src.ad = make_rsrc(g.d8, 4u * (uint32_t)((g.M - 1) * (g.lda / 32) + nb_all));
            src.va = arow * g.lda + 8 * kq + 32 * kb0;
            src.vad = 4 * (arow * (g.lda / 32) + kb0);
        } else {
            src.a = make_rsrc(g.a, 4u * a_elems);
            src.va = 4 * (arow * g.lda + 8 * kq + 32 * kb0);
        }
        src.w = make_rsrc(TL ? g.wm : g.w, (uint32_t)(g.N / 16) * (uint32_t)nb_all * kTileBytes);
        if constexpr (TL) {
            const int unit = ((n_base >> 4) * nb_all + kb0) * kTileBytes;  // column subtile 0, first block
            src.vw = unit + 8 * lane;
            src.vs = unit + 512 + 2 * l16;
        } else {
            const int grp = (n_base >> 2) + (l16 >> 2);  // this lane's group in column subtile 0
            src.vw = (grp * nb_all + kb0) * kBlockBytes + 8 + 32 * krow + 8 * kq;
            src.vs = (grp * nb_all + kb0) * kBlockBytes + 2 * krow;
        }
        src.wt = nb_all * kTileBytes;  // 16 rows of W: 4 groups of 136-byte blocks, or one tile per block
    }

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    if constexpr (LN) {
        static_assert(!A8, "the LayerNorm prologue takes fp32 activation rows");
    }
    if constexpr (LN && AT) {
        // LayerNorm of pre-split rows, the rows' statistics from the producer (their own
        // two-pass form, read from fp32 rows, measured 9.1 us against 7.9 us here): the
        // chunks stream as in the plain loop, each joined, normalised and split again in
        // registers before its MFMAs.  (The fp32 rows with the producer's statistics
        // measured slower than either.)
        __shared__ float lnw2[kHidden], lnb2[kHidden];
        __shared__ float2 rstat[16];
        Chunk<NT, A8, AT> ca, cb;
        if (nb > 0) load_chunk<NT, A8, TL, AT>(ca, 0, src);
        const float2 st = ln_rows_from_stats(g, m_base, l16, lnw2, lnb2, rstat);
        const float mean = st.x, inv = st.y;
        auto ln_apply = [&](Chunk<NT, A8, AT> &c, int b0) {  // columns 32 blk + 8 kq + i
#pragma unroll
            for (int j = 0; j < KB; ++j)
                if (b0 + j < nb) {
                    const int col = 32 * (kb0 + b0 + j) + 8 * kq;
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        float y = ((float)c.xh[j][i] + (float)c.xl[j][i] - mean) * inv;
                        y = y * lnw2[col + i];
                        x[i] = y + lnb2[col + i];
                    }
                    split_hi_lo(x, c.xh[j], c.xl[j]);
                }
        };
        for (int b0 = 0; b0 < nb; b0 += 2 * KB) {
            load_chunk<NT, A8, TL, AT>(cb, b0 + KB, src);
            ln_apply(ca, b0);
            mfma_chunk<NT, A8, AT>(ca, b0, nb, kq, acc);
            if (b0 + KB >= nb) break;
            if (b0 + 2 * KB < nb) load_chunk<NT, A8, TL, AT>(ca, b0 + 2 * KB, src);
            ln_apply(cb, b0 + KB);
            mfma_chunk<NT, A8, AT>(cb, b0 + KB, nb, kq, acc);
        }
    } else if constexpr (LN && !AT) {
        __shared__ float lnw[4 * 2 * KB * 32], lnb[4 * 2 * KB * 32];
        __shared__ float lsum[4][16], lsq[4][16];
        // loads in completion order: the activations, ln_w / ln_b (into registers),
        // then the weights, which stay in flight while the statistics are formed;
        // ln_w / ln_b go to LDS only after every load is issued (an LDS store of a
        // loaded value waits for that load, and loads complete in order)
        constexpr int LNR = (4 * 2 * KB * 32 + 255) / 256;
        Chunk<NT, A8, AT> ca, cb;
        load_chunk_a<NT, A8, AT>(ca, 0, src);
        load_chunk_a<NT, A8, AT>(cb, KB, src);
        float lw[LNR], lb[LNR];
#pragma unroll
        for (int i = 0; i < LNR; ++i) {
            const int c = min((int)threadIdx.x + 256 * i, g.K - 1);
            lw[i] = g.ln_w[c];
            lb[i] = g.ln_b[c];
        }
        load_chunk_b<NT, A8, AT, TL>(ca, 0, src);
        load_chunk_b<NT, A8, AT, TL>(cb, KB, src);
#pragma unroll
        for (int i = 0; i < LNR; ++i) {
            const int c = (int)threadIdx.x + 256 * i;
            if (c < g.K) {
                lnw[c] = lw[i];
                lnb[c] = lb[i];
            }
        }
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < KB; ++j)
            if (j < nb)
#pragma unroll
                for (int i = 0; i < 8; ++i) s += ca.xa[j][i];
#pragma unroll
        for (int j = 0; j < KB; ++j)
            if (KB + j < nb)
#pragma unroll
                for (int i = 0; i < 8; ++i) s += cb.xa[j][i];
        s += xshfl<16>(s);
        s += xshfl<32>(s);
        if (lane < 16) lsum[wave][lane] = s;
        __syncthreads();
        const float mean = (((lsum[0][l16] + lsum[1][l16]) + lsum[2][l16]) + lsum[3][l16]) / (float)g.K;
        float v = 0.0f;
#pragma unroll
        for (int j = 0; j < KB; ++j)
            if (j < nb)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float d = ca.xa[j][i] - mean;
                    v += d * d;
                }
#pragma unroll
        for (int j = 0; j < KB; ++j)
            if (KB + j < nb)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const float d = cb.xa[j][i] - mean;
                    v += d * d;
                }
        v += xshfl<16>(v);
        v += xshfl<32>(v);
        if (lane < 16) lsq[wave][lane] = v;
        __syncthreads();
        const float var = (((lsq[0][l16] + lsq[1][l16]) + lsq[2][l16]) + lsq[3][l16]) / (float)g.K;
        const float inv = 1.0f / sqrtf(var + 1e-5f);
        auto norm = [&](float (&x)[8], int blk) {  // columns 32 blk + 8 kq + i
            const int c = 32 * blk + 8 * kq;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float y = (x[i] - mean) * inv;
                y = y * lnw[c + i];
                x[i] = y + lnb[c + i];
            }
        };
#pragma unroll
        for (int j = 0; j < KB; ++j) {
            if (j < nb) norm(ca.xa[j], kb0 + j);
            if (KB + j < nb) norm(cb.xa[j], kb0 + KB + j);
        }
        mfma_chunk<NT, A8, AT>(ca, 0, nb, kq, acc);
        if (KB < nb) mfma_chunk<NT, A8, AT>(cb, KB, nb, kq, acc);
    } else if (nb > 0) {
        Chunk<NT, A8, AT> ca, cb;
        load_chunk<NT, A8, TL, AT>(ca, 0, src);
        for (int b0 = 0; b0 < nb; b0 += 2 * KB) {
            load_chunk<NT, A8, TL, AT>(cb, b0 + KB, src);
            mfma_chunk<NT, A8, AT>(ca, b0, nb, kq, acc);
            if (b0 + KB >= nb) break;
            if (b0 + 2 * KB < nb)  // (uniform) a chunk past the wave's blocks is not requested
                load_chunk<NT, A8, TL, AT>(ca, b0 + 2 * KB, src);
            mfma_chunk<NT, A8, AT>(cb, b0 + KB, nb, kq, acc);
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) red[wave][t][lane] = acc[t];
    __syncthreads();
    // lane holds rows m_base + 4kq + i, column n_base + 16t + l16
    if constexpr (EPI == EPI_GELU && NT >= 2) {
        if (g.q8_out != nullptr) {  // uniform
            // wave w finishes row 4kq + w of every subtile: a 32-block is subtiles (2b, 2b + 1)
            // across the 16 lanes of a kq group, so its amax is a 16-lane reduction
            const int i = wave, m = erow;
            float h[NT];
            const float *redf = (const float *)&red[0][0][lane] + i;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float v = redf[4 * (t * 64)];
                v += redf[4 * ((NT + t) * 64)];
                v += redf[4 * ((2 * NT + t) * 64)];
                v += redf[4 * ((3 * NT + t) * 64)];
                const int n = n_base + 16 * t + l16;
                h[t] = gelu_new(v + eo.b[t]);
                if (m < g.M && g.y != nullptr) g.y[(size_t)m * g.ldy + n] = h[t];
            }
#pragma unroll
            for (int b = 0; b < NT / 2; ++b) {
                // quant_block32's arithmetic (quantize_activation, quant.cpp:45-55)
                float amax = fmaxf(fabsf(h[2 * b]), fabsf(h[2 * b + 1]));
                amax = fmaxf(amax, xshfl<1>(amax));
                amax = fmaxf(amax, xshfl<2>(amax));
                amax = fmaxf(amax, xshfl<4>(amax));
                amax = fmaxf(amax, xshfl<8>(amax));
                const float d = amax / 127.0f;
                const float id = d > 0.0f ? 1.0f / d : 0.0f;
                int q0 = (int)rintf(h[2 * b] * id), q1 = (int)rintf(h[2 * b + 1] * id);
                q0 = q0 < -127 ? -127 : (q0 > 127 ? 127 : q0);
                q1 = q1 < -127 ? -127 : (q1 > 127 ? 127 : q1);
                if (m < g.M) {  // in the matrix-core order (q8t_at / d8t_at)
                    const int k0 = n_base + 32 * b;
                    g.q8_out[q8t_at(m, k0 + l16, g.N)] = (int8_t)q0;
                    g.q8_out[q8t_at(m, k0 + 16 + l16, g.N)] = (int8_t)q1;
                    if (l16 == 0) g.d8_out[d8t_at(m, k0 >> 5, g.N)] = d;
                }
            }
            GT_END
            return;
        }
    }
    if (WV > 4 && wave >= 4) return;  // (uniform) their partials are in LDS
    // component w of each lane's partials: one 4-byte LDS read each, at an offset
    // uniform in the wave; the waves' partials summed in wave order
    const int i = wave, m = erow;
    const float *redf = (const float *)&red[0][0][lane] + i;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        float v = redf[4 * (t * 64)];
#pragma unroll
        for (int w = 1; w < WV; ++w) v += redf[4 * ((w * NT + t) * 64)];
        const int n = n_base + 16 * t + l16;
        const float partner = xshfl<1>(v);  // column n ^ 1, same row
        if (m < g.M) gemm_finish<EPI, KV, NT>(er, eo, t, n, v, partner);
        if constexpr (EPI == EPI_F32) {
            if (g.pick_pairs != nullptr) {  // uniform: the 16 lanes of a row hold 16 consecutive columns
                float best = -INFINITY;
                int besti = g.N;
                if (m < g.M) {
                    const float pen = *g.pick_pen;
                    const int cnt = pen != 1.0f ? g.pick_counts[(size_t)m * g.pick_stride + n] : 0;
                    const float pv = penalised(v, cnt, pen);
                    if (pv > best) {  // greedy_pick_reduce's comparisons
                        best = pv;
                        besti = n;
                    }
                }
                argmax_step<1>(best, besti);
                argmax_step<2>(best, besti);
                argmax_step<4>(best, besti);
                argmax_step<8>(best, besti);
                // a NaN at column 0 wins outright (the reference's scan never leaves index 0,
                // sampler.cpp:24-26): the pair (+inf, 0) beats every other pair, ties go to
                // the lowest index
                int nan0 = (m < g.M && n == 0 && !(v == v)) ? 1 : 0;
                nan0 |= xshfl<1>(nan0);
                nan0 |= xshfl<2>(nan0);
                nan0 |= xshfl<4>(nan0);
                nan0 |= xshfl<8>(nan0);
                if (nan0) {
                    best = INFINITY;
                    besti = 0;
                }
                if (l16 == 0 && m < g.M)
                    reinterpret_cast<float2 *>(g.pick_pairs)[(size_t)m * (g.N >> 4) + (n >> 4)] =
                        make_float2(best, __int_as_float(besti));
            }
        }
        if constexpr (EPI == EPI_RESID) {
            if (g.y_stats != nullptr) {  // uniform: (mean, M2) of the row's 16 columns of subtile t
#pragma clang fp contract(off)
                const float y = eo.res[t] + (v + eo.b[t]);  // the value stored
                float sm = y;
                sm += xshfl<1>(sm);
                sm += xshfl<2>(sm);
                sm += xshfl<4>(sm);
                sm += xshfl<8>(sm);
                const float mean = sm * 0.0625f;
                const float d = y - mean;
                float q = d * d;
                q += xshfl<1>(q);
                q += xshfl<2>(q);
                q += xshfl<4>(q);
                q += xshfl<8>(q);
                if (l16 == 0 && m < g.M)
                    reinterpret_cast<float2 *>(g.y_stats)[(size_t)((n_base >> 4) + t) * g.M + m] = make_float2(mean, q);
            }
        }
    }
    GT_END
}

template <int EPI, int KV, bool A8, bool LN, bool TL, bool AT>
hipError_t launch_nt(const GemmArgs &g, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    const int mt = (g.M + 15) / 16;
    if constexpr (EPI == EPI_RESID && !LN) {
        // a long K (fc_out, K = 3072) in one workgroup of 8 waves, 16 columns a tile: each wave
        // takes 12 blocks (4 chunks of 3) and the residual epilogue completes the rows (no
        // split-K reduce) (32-column tiles, half the workgroups: 64 streams 56.4k -> 54.4k
        // frames/s; 16 waves of 6 blocks: 56.66k -> 56.59k)
        if (g.K >= 2048) {
            hipLaunchKernelGGL((gemm_wk_kernel<EPI, KV, 1, A8, LN, TL, AT, 8>), dim3(g.N / 16, mt, 1), dim3(512), 0, s,
                               g);
            return hipGetLastError();
        }
    }
    const int kz = EPI == EPI_PART ? (g.ksplit > 0 ? g.ksplit : gemm_ksplit(g.M, g.N, g.K)) : 1;
    // the widest column tile that still gives ~192 workgroups (a quantising epilogue needs
    // whole 32-blocks in a tile: at least 32 columns)
    if (g.N % 64 == 0 && (g.N / 64) * mt * kz >= 192) {
        hipLaunchKernelGGL((gemm_wk_kernel<EPI, KV, 4, A8, LN, TL, AT>), dim3(g.N / 64, mt, kz), dim3(256), 0, s, g);
    } else if (g.N % 32 == 0 && ((g.N / 32) * mt * kz >= 192 || g.q8_out != nullptr)) {
        hipLaunchKernelGGL((gemm_wk_kernel<EPI, KV, 2, A8, LN, TL, AT>), dim3(g.N / 32, mt, kz), dim3(256), 0, s, g);
    } else {
        hipLaunchKernelGGL((gemm_wk_kernel<EPI, KV, 1, A8, LN, TL, AT>), dim3(g.N / 16, mt, kz), dim3(256), 0, s, g);
    }
    return hipGetLastError();
}

template <int EPI, int KV, bool TL>
hipError_t launch_l(const GemmArgs &g, hipStream_t s) {
    if (g.a8 != nullptr)
        return g.a8_tiled ? launch_nt<EPI, KV, true, false, TL, true>(g, s)
                          : launch_nt<EPI, KV, true, false, TL, false>(g, s);
    if constexpr (EPI == EPI_GELU || EPI == EPI_QKV || EPI == EPI_F32) {
        if (g.a_hl != nullptr && g.ln_w != nullptr) return launch_nt<EPI, KV, false, true, TL, true>(g, s);
    }
    if (g.a_hl != nullptr) return launch_nt<EPI, KV, false, false, TL, true>(g, s);
    if constexpr (EPI != EPI_PART) {
        if (g.ln_w != nullptr) return launch_nt<EPI, KV, false, true, TL, false>(g, s);
    }
    return launch_nt<EPI, KV, false, false, TL, false>(g, s);
}

template <int EPI, int KV>
hipError_t launch_a(const GemmArgs &g, hipStream_t s) {
    return g.wm != nullptr ? launch_l<EPI, KV, true>(g, s) : launch_l<EPI, KV, false>(g, s);
}

__global__ __launch_bounds__(64) void tile_q8x4_mfma_kernel(const uint8_t *w, int nb_all, uint8_t *out) {
    const int sub = blockIdx.x, b = blockIdx.y, l = threadIdx.x;
    const int c = l & 15, kq = l >> 4, n = 16 * sub + c;
    const uint8_t *blk = w + ((size_t)(n >> 2) * nb_all + b) * kBlockBytes;
    uint8_t *unit = out + ((size_t)sub * nb_all + b) * kTileBytes;
    *(uint64_t *)(unit + 8 * l) = *(const uint64_t *)(blk + 8 + 32 * (n & 3) + 8 * kq);
    if (kq == 0) *(uint16_t *)(unit + 512 + 2 * c) = *(const uint16_t *)(blk + 2 * (n & 3));
}
}  // namespace

// Split K so that a GEMM with few output tiles still spreads over the CUs:
// about 256 workgroups of 16 x 16 tiles, at least 12 blocks (3 per wave) per
// slice, at most 16 slices (targets of 512-1024 workgroups, or 6 blocks per
// slice, measured slower at 64 streams).  Slices are balanced: sizes differ by at most one block.
int gemm_ksplit(int M, int N, int K) {
    const int tiles = ((M + 15) / 16) * (N / 16);
    const int nb = K / 32;
    int z = (256 + tiles - 1) / tiles;
    z = z > nb / 12 ? nb / 12 : z;
    z = z > 16 ? 16 : z;
    return z < 1 ? 1 : z;
}

hipError_t tile_q8x4_mfma(const uint8_t *w, int N, int K, uint8_t *out, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (!w || !out || N <= 0 || K <= 0 || N % 16 || K % 32) return hipErrorInvalidValue;
    hipLaunchKernelGGL(tile_q8x4_mfma_kernel, dim3(N / 16, K / 32), dim3(64), 0, s, w, K / 32, out);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs &g, Epilogue epi, KvType kv, hipStream_t s) {
    (void)hipGetLastError();  // report only this launch's error, not a stale one
    if (g.M <= 0 || g.N <= 0 || g.N % 16 || g.K % 32 || g.K <= 0 || g.lda < g.K || g.lda % 4) return hipErrorInvalidValue;
    if (epi == EPI_QKV && (g.N != 3 * kHidden || g.page_size <= 0)) return hipErrorInvalidValue;
    if (epi == EPI_PART) {  // every K slice must hold at least one block
        const int nb = g.K / 32, z = g.ksplit;
        if (!g.part || z > 16 || z > nb) return hipErrorInvalidValue;
    }
    if (g.a8 != nullptr && (!g.d8 || g.lda % 32)) return hipErrorInvalidValue;
    if (g.a8_tiled && (g.a8 == nullptr || g.lda != g.K)) return hipErrorInvalidValue;
    if (g.a_hl != nullptr && (g.a8 != nullptr || g.lda != g.K)) return hipErrorInvalidValue;
    // LN of pre-split rows: statistics from a producer's y_stats, K = 768 (fc_in, QKV, the heads)
    if (g.a_hl != nullptr && g.ln_w != nullptr &&
        (!g.ln_stats || !g.ln_b || (epi != EPI_GELU && epi != EPI_QKV && epi != EPI_F32) || g.K != kHidden))
        return hipErrorInvalidValue;
    if (g.ln_stats != nullptr && (g.a_hl == nullptr || g.ln_w == nullptr)) return hipErrorInvalidValue;
    if (g.y_hl != nullptr && ((epi != EPI_GELU && epi != EPI_RESID) || g.q8_out != nullptr || g.N % 32))
        return hipErrorInvalidValue;
    if (g.y_stats != nullptr && (epi != EPI_RESID || g.N != kHidden)) return hipErrorInvalidValue;
    if (g.pick_pairs != nullptr && (epi != EPI_F32 || g.N % 16 || !g.pick_counts || !g.pick_pen))
        return hipErrorInvalidValue;
    if (g.q8_out != nullptr && (epi != EPI_GELU || !g.d8_out || g.N % 32 || (g.y && g.ldy < g.N)))
        return hipErrorInvalidValue;
    if (g.q8_out == nullptr && g.y_hl == nullptr && epi != EPI_PART && epi != EPI_QKV && !g.y)
        return hipErrorInvalidValue;
    // LayerNorm prologue: fp32 rows of at most 4 waves x 2 chunks of blocks, whole K in the workgroup
    if (g.ln_w != nullptr && g.a_hl == nullptr &&
        (!g.ln_b || g.a8 != nullptr || epi == EPI_PART || g.K > 4 * 2 * KB * 32 || g.K < 4 * 32))
        return hipErrorInvalidValue;
    switch (epi) {
        case EPI_PART: return launch_a<EPI_PART, KV_F16>(g, s);
        case EPI_F32: return launch_a<EPI_F32, KV_F16>(g, s);
        case EPI_RESID: return launch_a<EPI_RESID, KV_F16>(g, s);
        case EPI_GELU: return launch_a<EPI_GELU, KV_F16>(g, s);
        case EPI_QKV: return kv == KV_F32 ? launch_a<EPI_QKV, KV_F32>(g, s) : launch_a<EPI_QKV, KV_F16>(g, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace mh
#ifdef MH_GEMM_TRACE
extern "C" int mh_gemm_trace_read(unsigned long long *out) {
    return (int)hipMemcpyFromSymbol(out, HIP_SYMBOL(mh::mh_gemm_ts), sizeof(mh::mh_gemm_ts));
}
#endif
