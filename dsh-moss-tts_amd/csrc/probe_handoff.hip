// probe_handoff.hip -- what it costs to hand bulk data from every workgroup to another
// workgroup, inside one launch or across a launch boundary (gfx950, 256 workgroups of
// 256 threads).  A measurement for bench.py --mode handoff, built as libmoss_probe.so
// beside the library; nothing of the decode path uses it.
//
// Every round each workgroup b writes `words` 32-bit values and then reads the `words`
// values workgroup (b + 37) % 256 wrote in that round (on another XCD: workgroup i runs on
// XCD i % 8), checking each.  Forms:
//   MODE_FENCE_ALL   one persistent launch; plain stores, __threadfence() in every thread,
//                    an arrival counter, a spin on it, __threadfence(), plain loads
//   MODE_FENCE_ONE   the same with the two fences in one thread per workgroup
//   MODE_LL          one persistent launch; the values travel as LL words (value + round
//                    tag, agent-scope relaxed 8-byte stores and loads), every load of a
//                    thread in flight at once, re-polled until its tag is current
//   MODE_LAUNCH      one launch per round, replayed from a captured graph: the kernel
//                    boundary is the hand-off (plain stores and loads)
// Persistent forms need every workgroup resident: the probe checks the occupancy first.
// Every wait is bounded and a failed check or wait sets an error word; nothing hangs.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kG = 256, kT = 256, kMaxPer = 64;  // workgroups, threads, words per thread
constexpr int kMaxWords = kT * kMaxPer;           // 64 KB of values per workgroup

enum { MODE_FENCE_ALL = 0, MODE_FENCE_ONE = 1, MODE_LL = 2, MODE_LAUNCH = 3 };

__device__ __forceinline__ uint32_t pattern(int r, int b, int i) { return (uint32_t)(r * 100003 + b * 7 + i); }

// Thread t's words t, t + 256, ... of workgroup src's round-r values: every load issued
// before the first is checked.
__device__ __forceinline__ uint32_t read_check(const uint32_t *sp, int per, int r, int src, int t, int *err) {
    uint32_t v[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
        if (k < per) v[k] = sp[t + kT * k];
    uint32_t sum = 0;
    bool bad = false;
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
        if (k < per) {
            bad |= v[k] != pattern(r, src, t + kT * k);
            sum += v[k];
        }
    if (bad) atomicOr(err, 8);
    return sum;
}

__global__ __launch_bounds__(kT) void fence_rounds(int one, int rounds, int words, uint32_t *cnt, uint32_t *buf,
                                                   int *err) {
    const int b = blockIdx.x, t = threadIdx.x, src = (b + 37) % kG;
    uint32_t sum = 0;
    for (int r = 0; r < rounds; ++r) {
        uint32_t *dst = buf + ((size_t)(r & 1) * kG + b) * words;
        for (int i = t; i < words; i += kT) dst[i] = pattern(r, b, i);
        if (!one) __threadfence();
        __syncthreads();
        if (t == 0) {
            if (one) __threadfence();
            __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int budget = 1 << 22;
            while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (uint32_t)(kG * (r + 1))) {
                if (--budget < 0) {
                    atomicOr(err, 4);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (one) __threadfence();
        }
        __syncthreads();
        if (!one) __threadfence();
        sum += read_check(buf + ((size_t)(r & 1) * kG + src) * words, words / kT, r, src, t, err);
        __syncthreads();  // the buffer read here is rewritten two rounds on
    }
    if (sum == 0x5a5a5a5au) atomicOr(err, 16);  // keeps the loads
}

// One buffer per round (tags never repeat in a buffer, so no workgroup can overwrite words
// its reader has not seen).
__global__ __launch_bounds__(kT) void ll_rounds(int rounds, int words, uint64_t *ll, int *err) {
    const int b = blockIdx.x, t = threadIdx.x, src = (b + 37) % kG;
    const int per = words / kT;
    uint32_t sum = 0;
    for (int r = 0; r < rounds; ++r) {
        const uint32_t tag = (uint32_t)r + 1u;
        uint64_t *dst = ll + ((size_t)r * kG + b) * words;
        for (int i = t; i < words; i += kT)
            __hip_atomic_store(dst + i, ((uint64_t)tag << 32) | pattern(r, b, i), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t *sp = ll + ((size_t)r * kG + src) * words;
        uint64_t w[kMaxPer];
        uint64_t pending = 0;
#pragma unroll
        for (int k = 0; k < kMaxPer; ++k)
            if (k < per) {
                w[k] = __hip_atomic_load(sp + t + kT * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                pending |= 1ull << k;
            }
        int budget = 1 << 20;
        while (true) {
#pragma unroll
            for (int k = 0; k < kMaxPer; ++k)
                if (((pending >> k) & 1ull) && (uint32_t)(w[k] >> 32) == tag) {
                    pending &= ~(1ull << k);
                    if ((uint32_t)w[k] != pattern(r, src, t + kT * k)) atomicOr(err, 2);
                    sum += (uint32_t)w[k];
                }
            if (!pending) break;
            if (--budget < 0) {
                atomicOr(err, 1);
                return;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int k = 0; k < kMaxPer; ++k)
                if ((pending >> k) & 1ull) w[k] = __hip_atomic_load(sp + t + kT * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
    }
    if (sum == 0x5a5a5a5au) atomicOr(err, 16);
}

// Round r of the launch-per-round form: read (and check) round r - 1's values of the
// source workgroup from `in`, write round r's to `out`.
__global__ __launch_bounds__(kT) void launch_round(int r, int words, const uint32_t *in, uint32_t *out, int *err) {
    const int b = blockIdx.x, t = threadIdx.x, src = (b + 37) % kG;
    uint32_t sum = 0;
    if (r > 0) sum = read_check(in + (size_t)src * words, words / kT, r - 1, src, t, err);
    uint32_t *dst = out + (size_t)b * words;
    for (int i = t; i < words; i += kT) dst[i] = pattern(r, b, i);
    if (sum == 0x5a5a5a5au) atomicOr(err, 16);
}

template <typename F>
int resident(F kernel) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, kT, 0) != hipSuccess) return 0;
    return cus * per;
}

}  // namespace

// Returns 0 and the average time of one round in *us (device time from HIP events around
// the timed launches), a negative HIP error, or a positive error word (a failed value
// check: 2 or 8, or a wait that ran out: 1 or 4).  words % 256 == 0, 256 <= words <= 16384.
extern "C" int moss_probe_handoff(int mode, int rounds, int words, double *us) {
    if (mode < 0 || mode > MODE_LAUNCH || rounds < 2 || rounds > 400 || words < kT || words > kMaxWords ||
        words % kT || !us)
        return -(int)hipErrorInvalidValue;
    if (mode == MODE_LL && rounds > 64) return -(int)hipErrorInvalidValue;  // one buffer per round
    if ((mode == MODE_LL && resident(ll_rounds) < kG) ||
        ((mode == MODE_FENCE_ALL || mode == MODE_FENCE_ONE) && resident(fence_rounds) < kG))
        return -(int)hipErrorCooperativeLaunchTooLarge;
    uint32_t *cnt = nullptr, *buf = nullptr;
    uint64_t *ll = nullptr;
    int *err = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int rc = 0;
    auto ck = [&](hipError_t e) {
        if (e != hipSuccess && rc == 0) rc = -(int)e;
        return rc == 0;
    };
    const size_t llw = mode == MODE_LL ? (size_t)rounds * kG * words : 0;
    if (ck(hipStreamCreateWithFlags(&s, hipStreamNonBlocking)) && ck(hipEventCreate(&e0)) && ck(hipEventCreate(&e1)) &&
        ck(hipMalloc(&cnt, 4)) && ck(hipMalloc(&err, 4)) && ck(hipMalloc(&buf, (size_t)2 * kG * words * 4)) &&
        (llw == 0 || (ck(hipMalloc(&ll, llw * 8)) && ck(hipMemsetAsync(ll, 0, llw * 8, s)))) &&
        ck(hipMemsetAsync(cnt, 0, 4, s)) && ck(hipMemsetAsync(err, 0, 4, s))) {
        float ms = 0.f;
        if (mode == MODE_LAUNCH) {
            // rounds launches ping-ponging between the two halves of buf, captured once
            if (ck(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal))) {
                for (int r = 0; r < rounds; ++r) {
                    uint32_t *in = buf + (size_t)((r + 1) & 1) * kG * words, *out = buf + (size_t)(r & 1) * kG * words;
                    hipLaunchKernelGGL(launch_round, dim3(kG), dim3(kT), 0, s, r, words, in, out, err);
                }
                ck(hipStreamEndCapture(s, &graph));
            }
            if (rc == 0 && ck(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0)) && ck(hipGraphLaunch(exec, s)) &&
                ck(hipEventRecord(e0, s)) && ck(hipGraphLaunch(exec, s)) && ck(hipEventRecord(e1, s)))
                ck(hipEventSynchronize(e1));
        } else if (ck(hipEventRecord(e0, s))) {
            if (mode == MODE_LL)
                hipLaunchKernelGGL(ll_rounds, dim3(kG), dim3(kT), 0, s, rounds, words, ll, err);
            else
                hipLaunchKernelGGL(fence_rounds, dim3(kG), dim3(kT), 0, s, mode == MODE_FENCE_ONE ? 1 : 0, rounds,
                                   words, cnt, buf, err);
            if (ck(hipGetLastError()) && ck(hipEventRecord(e1, s))) ck(hipEventSynchronize(e1));
        }
        if (rc == 0 && ck(hipEventElapsedTime(&ms, e0, e1))) {
            int herr = 0;
            if (ck(hipMemcpy(&herr, err, 4, hipMemcpyDeviceToHost))) rc = herr;
            *us = ms * 1000.0 / rounds;
        }
    }
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (s) (void)hipStreamSynchronize(s);
    (void)hipFree(cnt);
    (void)hipFree(err);
    (void)hipFree(buf);
    (void)hipFree(ll);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    return rc;
}
