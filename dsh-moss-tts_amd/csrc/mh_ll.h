// mh_ll.h -- LL words: the exchange between workgroups of one launch used by
// the fused decode kernels (gfx950).
//
// An LL word is 8 bytes: a 32-bit value and a 32-bit tag, written with one
// agent-scope store and read with agent-scope loads (both coherent across the
// XCDs' L2 caches).  The tag is unique to the launch, so a consumer re-reads
// the words it needs until every tag is current: the data is its own flag --
// no barrier, counter or fence.  Every wait is bounded by a poll budget.
#pragma once
#include "mh_device.h"
#include "mh_gemv.h"

namespace mh {

// poll rounds per thread and launch: each round waits one load round trip
// (~0.5-1 us) plus the sleep, so a wait gives up after ~0.05 s
constexpr int kPollBudget = 1 << 16;
// s_sleep between poll rounds (units of 64 clocks): 1 measured 0.7 % faster per
// batch-1 frame than 2, 4 1.2 % slower; 0 was within noise of 1
constexpr int kPollSleep = 1;

__device__ __forceinline__ void ll_put(uint64_t *w, float v, uint32_t tag) {
    __hip_atomic_store(w, ((uint64_t)tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t ll_load(const uint64_t *w) {
    return __hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch generation of a sliced attention scratch block (gen[0]: generation,
// gen[1]: workgroups of the current launch that are done).
__device__ __forceinline__ uint32_t ll_gen_load(const uint32_t *gen) {
    return __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Called once per workgroup after its last use of the launch's tag: the last of
// `total` workgroups resets the count and starts the next generation.  Every
// workgroup has read the generation before it arrives, so no workgroup of this
// launch can see the new value; the next launch on the stream sees it.
__device__ __forceinline__ void ll_gen_arrive(uint32_t *gen, uint32_t total) {
    const uint32_t done = __hip_atomic_fetch_add(gen + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done + 1 == total) {
        __hip_atomic_store(gen + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Waits until words [0, n) of src carry `tag` and copies their values to dst
// (LDS).  Thread t takes words t, t + 256, ... (at most MAXK); all of its loads
// are in flight together.  Returns false when the thread's budget runs out.
// ll_gather by NT threads: thread tt (0 <= tt < NT) takes words tt, tt + NT, ...
template <int MAXK, int NT>
__device__ __forceinline__ bool ll_gather_by(const uint64_t *src, int n, uint32_t tag, float *dst, int &budget,
                                             int tt) {
    uint64_t w[MAXK];
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        w[k] = ll_load(src + min(tt + NT * k, n - 1));
        if (tt + NT * k < n) pending |= 1u << k;
    }
    while (true) {
#pragma unroll
        for (int k = 0; k < MAXK; ++k)
            if (((pending >> k) & 1u) && (uint32_t)(w[k] >> 32) == tag) {
                dst[tt + NT * k] = __uint_as_float((uint32_t)w[k]);
                pending &= ~(1u << k);
            }
        if (pending == 0) return true;
        if (--budget < 0) return false;
        __builtin_amdgcn_s_sleep(kPollSleep);
#pragma unroll
        for (int k = 0; k < MAXK; ++k) w[k] = ll_load(src + min(tt + NT * k, n - 1));
    }
}

template <int MAXK>
__device__ __forceinline__ bool ll_gather(const uint64_t *src, int n, uint32_t tag, float *dst, int &budget) {
    const int t = tix();
    uint64_t w[MAXK];
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
        w[k] = ll_load(src + min(t + 256 * k, n - 1));
        if (t + 256 * k < n) pending |= 1u << k;
    }
    while (true) {
#pragma unroll
        for (int k = 0; k < MAXK; ++k)
            if (((pending >> k) & 1u) && (uint32_t)(w[k] >> 32) == tag) {
                dst[t + 256 * k] = __uint_as_float((uint32_t)w[k]);
                pending &= ~(1u << k);
            }
        if (pending == 0) return true;
        if (--budget < 0) return false;
        __builtin_amdgcn_s_sleep(kPollSleep);
#pragma unroll
        for (int k = 0; k < MAXK; ++k) w[k] = ll_load(src + min(t + 256 * k, n - 1));
    }
}

// Workgroup barrier that also tells every thread whether any thread failed its
// wait: one barrier and one LDS read (__syncthreads_or costs three barriers and
// a dispatch-packet load).  *flag is an LDS word the launch sets to 0, behind a
// barrier, before any wait, and that is only ever set to 1 afterwards (a failed
// wait ends the launch).
__device__ __forceinline__ bool sync_failed(bool failed, volatile int *flag) {
    if (failed) *flag = 1;
    __syncthreads();
    return *flag != 0;
}

// The gather before a row dot split in K over the 4 waves of a workgroup (GemvStage<4, NB, N>):
// wave w reads only K slice w, [w N / 4, (w + 1) N / 4), of the activation, so it gathers that
// slice itself and starts its dot when the slice is in, with no workgroup barrier in between.
// A failed wait sets *flag, which the caller tests after the dot's barriers.
template <int N>
__device__ __forceinline__ void ll_gather_slice(const uint64_t *src, uint32_t tag, float *dst, int &budget,
                                                volatile int *flag) {
    constexpr int S = N / 4;
    static_assert(S % 64 == 0 && S / 64 <= 32, "a whole number of words per lane, at most 32");
    const int w = __builtin_amdgcn_readfirstlane(tix() >> 6), lane = tix() & 63;
    if (!ll_gather_by<S / 64, 64>(src + S * w, S, tag, dst + S * w, budget, lane)) *flag = 1;
    // the slice's LDS writes before any lane of this wave reads them
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

// One word per thread (threads with active == false return true at once).
__device__ __forceinline__ bool ll_wait1(const uint64_t *src, bool active, uint32_t tag, float *dst, int &budget) {
    if (!active) return true;
    while (true) {
        const uint64_t w = ll_load(src);
        if ((uint32_t)(w >> 32) == tag) {
            *dst = __uint_as_float((uint32_t)w);
            return true;
        }
        if (--budget < 0) return false;
        __builtin_amdgcn_s_sleep(kPollSleep);
    }
}

// A GEMV stage of a fused launch: workgroup b takes the 4-row groups
// b * (4 / SPLIT) + w / SPLIT (SPLIT waves per group, each a K slice of one
// batch of NB blocks per lane), the split of the one-GEMV kernels, so every
// row is summed in the same order.  prefetch() issues the weight loads before
// the activation is ready; dot() returns the row sum (valid in every lane of
// the row, lanes 16*bl + 4*kk + j) once act[] is complete; all waves call it.
template <int SPLIT, int NB, int K>
struct GemvStage {
    static constexpr int nb = K / 32, per = nb / SPLIT;
    static_assert(per <= 4 * NB && nb % SPLIT == 0, "one batch per wave");
    uint2 qv[NB];
    uint16_t dh[NB];
    int g, ks, b0;

    __device__ __forceinline__ void prefetch(const uint8_t *w, int b) {
        const int wave = tix() >> 6, lane = tix() & 63;
        g = b * (4 / SPLIT) + wave / SPLIT;
        ks = wave % SPLIT;
        b0 = ks * per;
        load_batch<NB>(w + (size_t)g * nb * kBlockBytes, b0 + (lane >> 4), b0 + per, lane & 15, (lane & 15) >> 2, qv,
                       dh);
    }
    // row of this lane's result (valid in the storer lanes: ks == 0, lane < 16, j == 0)
    __device__ __forceinline__ int row() const { return 4 * g + ((tix() & 15) >> 2); }
    __device__ __forceinline__ bool storer() const {
        const int lane = tix() & 63;
        return ks == 0 && lane < 16 && (lane & 3) == 0;
    }
    // A8: act / da as quant_act_lds leaves them (W8A8 row dots)
    template <bool A8 = false>
    __device__ __forceinline__ float dot(const float *act, float (*part)[4], const float *da = nullptr) const {
        const int wave = tix() >> 6, lane = tix() & 63, kk = (lane & 15) >> 2, j = lane & 3;
        float acc = dot_batch<NB, A8>(act, b0 + (lane >> 4), b0 + per, j, qv, dh, 0.0f, da);
        acc = row_lane_sum(acc);
        if constexpr (SPLIT == 1) {
            return acc;
        } else {
            if (lane < 16 && j == 0) part[wave][kk] = acc;
            __syncthreads();
            const int g0 = (wave / SPLIT) * SPLIT;
            float yv = part[g0][kk];
#pragma unroll
            for (int s2 = 1; s2 < SPLIT; ++s2) yv += part[g0 + s2][kk];
            __syncthreads();
            return yv;
        }
    }
};

}  // namespace mh
