// Phase-cost microbenchmarks: what one dependent phase of a batch-1 token
// costs on this GPU, under the two ways a chain of phases can run.
//
//   kernel-per-phase: a captured graph of dependent launches, each reading
//     the previous launch's small output (and, with weights, streaming its
//     own slice of a weight buffer);
//   persistent: one cooperative kernel whose workgroups meet at a software
//     grid barrier between phases (per-workgroup flags, relaxed system-scope
//     atomics; exchanged data written and read at system scope, since the
//     XCDs' L2 caches are not coherent with each other), streaming weights
//     after the barrier, or issuing the next phase's weight loads before the
//     wait so the barrier hides them.
//
// Every spin is bounded (and an abort flag stops the other workgroups), so
// every wave exits even if a barrier never completes.  Profiling support
// (chk_phase_bench, kernels.h); no reference counterpart.
#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "cherenkov/kernels.h"
#include "kernels_internal.h"

namespace chk {
namespace {

constexpr uint32_t PB_WG = 256;
constexpr uint32_t PB_SPIN_LIMIT = 1u << 22;
constexpr int PB_WORDS = 16;  // uint4 weight loads per thread and phase in flight

__device__ __forceinline__ uint32_t ld_sys(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float ldf_sys(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void stf_sys(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__global__ void __launch_bounds__(PB_WG) k_pb_empty(float* x) {
    if (threadIdx.x == PB_WG) x[0] = 1.0f;  // never taken
}

// One dependent phase: read 64 values of the previous phase's output,
// stream `words` uint4 per thread of weights, write 64 values.
__global__ void __launch_bounds__(PB_WG) k_pb_stream(const float* __restrict__ in, float* __restrict__ out,
                                                      const uint4* __restrict__ w, uint32_t words) {
    const uint32_t t = threadIdx.x, lane = t & 63;
    float acc = in[(blockIdx.x * 7 + lane) & 1023];
    const uint4* p = w + (size_t)blockIdx.x * PB_WG * words + t;
    uint32_t x = 0;
    // every load of a round issued before any is used
    for (uint32_t i0 = 0; i0 < words; i0 += PB_WORDS) {
        uint4 v[PB_WORDS];
#pragma unroll
        for (int i = 0; i < PB_WORDS; ++i)
            if (i0 + i < words) v[i] = p[(size_t)(i0 + i) * PB_WG];
#pragma unroll
        for (int i = 0; i < PB_WORDS; ++i)
            if (i0 + i < words) x ^= v[i].x + v[i].y + v[i].z + v[i].w;
    }
    acc += (float)(x & 1);
    if (t < 64) out[(blockIdx.x * 64 + t) & 1023] = acc;
}

struct PbArgs {
    uint32_t* flags;     // [nwg] arrival flags, 64 B apart
    uint32_t* abort_flag;
    uint32_t* err;
    float* data;         // [2][nwg][64] exchanged values
    const uint4* w;      // weights: [nrot][nwg][words][256], phase p reads slice p % nrot
    uint32_t phases, words, nrot;
    int prefetch;        // issue the next phase's weight loads before the wait
};

// Persistent chain: per phase, publish 64 values, wait until every
// workgroup has published (flags polled by wave 0), read two other
// workgroups' values, stream this phase's weight slice.
__global__ void __launch_bounds__(PB_WG) k_pb_persistent(PbArgs a) {
    const uint32_t nwg = gridDim.x, wg = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    __shared__ uint32_t s_abort;
    if (t == 0) s_abort = 0;
    __syncthreads();
    uint32_t bad = 0, x = 0;
    uint4 wr[PB_WORDS];
    const uint32_t words = a.words, w0 = words < PB_WORDS ? words : PB_WORDS;
    // the first round of phase p: words 0 .. w0 of this workgroup's slice
    auto issue = [&](uint32_t p) {
        const uint4* src = a.w + ((size_t)(p % a.nrot) * nwg + wg) * PB_WG * words + t;
#pragma unroll
        for (int i = 0; i < PB_WORDS; ++i)
            if ((uint32_t)i < w0) wr[i] = src[(size_t)i * PB_WG];
    };
    auto consume = [&]() {
#pragma unroll
        for (int i = 0; i < PB_WORDS; ++i)
            if ((uint32_t)i < w0) x ^= wr[i].x + wr[i].y + wr[i].z + wr[i].w;
    };
    // the rest of phase p's slice, round by round
    auto rest = [&](uint32_t p) {
        const uint4* src = a.w + ((size_t)(p % a.nrot) * nwg + wg) * PB_WG * words + t;
        for (uint32_t r0 = PB_WORDS; r0 < words; r0 += PB_WORDS) {
            uint4 v[PB_WORDS];
#pragma unroll
            for (int i = 0; i < PB_WORDS; ++i) v[i] = src[(size_t)min(r0 + i, words - 1) * PB_WG];
#pragma unroll
            for (int i = 0; i < PB_WORDS; ++i)
                if (r0 + i < words) x ^= v[i].x + v[i].y + v[i].z + v[i].w;
        }
    };
    if (a.prefetch) issue(0);
    for (uint32_t p = 0; p < a.phases; ++p) {
        float* buf = a.data + (size_t)(p & 1) * nwg * 64;
        if (wave == 0) {
            stf_sys(buf + wg * 64 + lane, (float)(p * 7 + wg));
            __builtin_amdgcn_s_waitcnt(0);
            if (lane == 0) st_sys(a.flags + wg * 16, p + 1);
            uint32_t spins = 0;
            while (true) {
                bool ok = true;
                for (uint32_t k = lane; k < nwg; k += 64) ok &= ld_sys(a.flags + k * 16) >= p + 1;
                if (__all(ok)) break;
                if (++spins > PB_SPIN_LIMIT || ld_sys(a.abort_flag)) {
                    if (lane == 0) st_sys(a.abort_flag, 1);
                    s_abort = 1;
                    break;
                }
            }
        }
        __syncthreads();
        if (s_abort) break;
        if (wave == 1) {
            const uint32_t o1 = (wg + 1) % nwg, o2 = (wg + 97) % nwg;
            const float v1 = ldf_sys(buf + o1 * 64 + lane), v2 = ldf_sys(buf + o2 * 64 + lane);
            bad += (v1 != (float)(p * 7 + o1)) + (v2 != (float)(p * 7 + o2));
        }
        // the first round (issued before the wait under prefetch), then the
        // rest of the slice
        if (!a.prefetch) issue(p);
        consume();
        rest(p);
        if (a.prefetch && p + 1 < a.phases) issue(p + 1);
    }
    if (wave == 1 && bad) atomicAdd(a.err, bad);
    if (x == 0x9e3779b9u) a.err[1] = x;  // keeps the loads live
}

// XCD-local barrier: the workgroups of one XCD (dealt round-robin by
// linear id, so workgroup g runs on XCD g % 8, checked against the
// hardware's XCC_ID) meet at a counter in that XCD's L2: agent-scope
// read-modify-writes without the system-coherence bit are performed in the
// local L2, which every CU of the XCD shares, so neither the counter nor
// the exchanged values go to memory.  The counter only grows (arrival k of
// a phase waits for the next multiple of the XCD's workgroup count), so no
// reset is needed between launches.
struct PbXArgs {
    uint32_t* bar;  // [8] counters, 64 B apart
    uint32_t* abort_flag;
    uint32_t* err;  // [0] wrong values read, [1] workgroups not on XCD g % 8
    float* data;    // [8][2][per][64]
    uint32_t phases;
};

__global__ void __launch_bounds__(PB_WG) k_pb_xcd(PbXArgs a) {
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const uint32_t xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // hwreg(HW_REG_XCC_ID, 0, 4)
    const uint32_t per = gridDim.x >> 3, rank = blockIdx.x >> 3, x = blockIdx.x & 7;
    __shared__ uint32_t s_abort;
    if (t == 0) {
        s_abort = 0;
        if (xcc != x) atomicAdd(a.err + 1, 1u);
    }
    __syncthreads();
    uint32_t bad = 0;
    uint32_t* bar = a.bar + x * 16;
    for (uint32_t p = 0; p < a.phases; ++p) {
        float* buf = a.data + ((size_t)(x * 2 + (p & 1)) * per) * 64;
        if (wave == 0) buf[rank * 64 + lane] = (float)(p * 7 + rank);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (t == 0) {
            const uint32_t old = __hip_atomic_fetch_add(bar, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t target = (old / per + 1) * per;
            uint32_t spins = 0;
            while ((int32_t)(__hip_atomic_fetch_add(bar, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) - target) < 0) {
                if (++spins > PB_SPIN_LIMIT || ld_sys(a.abort_flag)) {
                    st_sys(a.abort_flag, 1);
                    s_abort = 1;
                    break;
                }
            }
        }
        __syncthreads();
        if (s_abort) break;
        if (wave == 1) {
            // other workgroups' values, read at device scope (past this CU's L1)
            const uint32_t o1 = (rank + 1) % per, o2 = (rank + per / 2) % per;
            const float v1 = __hip_atomic_load(buf + o1 * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float v2 = __hip_atomic_load(buf + o2 * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            bad += (v1 != (float)(p * 7 + o1)) + (v2 != (float)(p * 7 + o2));
        }
    }
    if (wave == 1 && bad) atomicAdd(a.err, bad);
}

// Float atomics without a return value: workgroup g adds 1 to `per_wg`
// addresses starting at (g * stride) % n_addr.
__global__ void __launch_bounds__(PB_WG) k_pb_atomics(float* acc, uint32_t n_addr, uint32_t per_wg, uint32_t stride) {
    const uint32_t base = blockIdx.x * stride;
    for (uint32_t i = threadIdx.x; i < per_wg; i += PB_WG) atomicAdd(acc + (base + i) % n_addr, 1.0f);
}

struct Dev {
    std::vector<void*> ptrs;
    template <class T>
    T* alloc(size_t bytes) {
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) throw std::runtime_error("hipMalloc failed");
        ptrs.push_back(p);
        return (T*)p;
    }
    ~Dev() {
        for (void* p : ptrs) (void)hipFree(p);
    }
};

void ck(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

}  // namespace
}  // namespace chk

using namespace chk;

extern "C" int chk_phase_bench(int mode, uint32_t wgs, uint32_t phases, uint64_t bytes_per_phase,
                               double* us_per_phase, uint32_t* errors) {
    try {
        if (wgs < 1 || wgs > 1024) throw std::runtime_error("1..=1024 workgroups");
        if (mode != 5 && (phases < 8 || phases > 20000)) throw std::runtime_error("8..=20000 phases");
        if (mode == 5 && (phases < 1 || phases > (1u << 24))) throw std::runtime_error("1..=2^24 addresses");
        uint32_t words = (uint32_t)std::max<uint64_t>(1, bytes_per_phase / ((uint64_t)wgs * PB_WG * 16));
        // weights rotate over enough slices (>= 512 MB) that they come from
        // HBM, not from the memory-side cache
        const uint64_t slice = (uint64_t)wgs * PB_WG * words * 16;
        const uint32_t nrot = mode == 5 ? 1u : (uint32_t)std::min<uint64_t>(
            std::max<uint64_t>(2, (512ull << 20) / slice + 1), std::max<uint32_t>(phases, 2));
        Dev d;
        hipStream_t st;
        ck(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "stream");
        hipEvent_t e0, e1;
        ck(hipEventCreate(&e0), "event");
        ck(hipEventCreate(&e1), "event");
        float* vec = d.alloc<float>(2 * 1024 * sizeof(float));
        const size_t wbytes = (size_t)nrot * slice;
        uint4* w = d.alloc<uint4>(wbytes);
        ck(hipMemsetAsync(w, 1, wbytes, st), "memset");
        ck(hipMemsetAsync(vec, 0, 2 * 1024 * sizeof(float), st), "memset");
        float ms = 0.0f;
        *errors = 0;
        if (mode == 0 || mode == 1) {
            // graph of `phases` dependent launches (mode 1 streams weights)
            hipGraph_t g;
            hipGraphExec_t ge;
            ck(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "capture");
            for (uint32_t p = 0; p < phases; ++p) {
                if (mode == 0) k_pb_empty<<<wgs, PB_WG, 0, st>>>(vec);
                else k_pb_stream<<<wgs, PB_WG, 0, st>>>(vec + (p & 1) * 1024, vec + ((p + 1) & 1) * 1024,
                                                        w + (size_t)(p % nrot) * wgs * PB_WG * words, words);
            }
            ck(hipStreamEndCapture(st, &g), "capture end");
            ck(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0), "instantiate");
            ck(hipGraphLaunch(ge, st), "launch");
            ck(hipEventRecord(e0, st), "record");
            ck(hipGraphLaunch(ge, st), "launch");
            ck(hipEventRecord(e1, st), "record");
            ck(hipEventSynchronize(e1), "sync");
            ck(hipEventElapsedTime(&ms, e0, e1), "elapsed");
            (void)hipGraphExecDestroy(ge);
            (void)hipGraphDestroy(g);
        } else if (mode == 2 || mode == 3 || mode == 4) {
            // persistent: 2 = barrier only, 3 = weights after the barrier,
            // 4 = the next phase's weights issued before the wait
            PbArgs a{};
            a.flags = d.alloc<uint32_t>((size_t)wgs * 64);  // one flag per 64 bytes
            a.abort_flag = d.alloc<uint32_t>(256);
            a.err = d.alloc<uint32_t>(256);
            a.data = d.alloc<float>((size_t)2 * wgs * 64 * 4);
            a.w = w;
            a.words = mode == 2 ? 0 : words;
            a.nrot = nrot;
            a.prefetch = mode == 4;
            float t[3];
            const uint32_t ph[3] = {phases / 4, phases / 4, phases};
            for (int k = 0; k < 3; ++k) {  // the first run only warms the launch path
                a.phases = ph[k];
                ck(hipMemsetAsync(a.flags, 0, (size_t)wgs * 64, st), "memset");
                ck(hipMemsetAsync(a.abort_flag, 0, 256, st), "memset");
                ck(hipMemsetAsync(a.err, 0, 256, st), "memset");
                ck(hipStreamSynchronize(st), "sync");
                void* args[] = {&a};
                ck(hipEventRecord(e0, st), "record");
                ck(hipLaunchCooperativeKernel((const void*)k_pb_persistent, dim3(wgs), dim3(PB_WG), args, 0, st),
                   "cooperative launch");
                ck(hipEventRecord(e1, st), "record");
                ck(hipEventSynchronize(e1), "sync");
                ck(hipEventElapsedTime(&t[k], e0, e1), "elapsed");
                uint32_t h[2];
                ck(hipMemcpy(h, a.err, 4, hipMemcpyDeviceToHost), "copy");
                ck(hipMemcpy(h + 1, a.abort_flag, 4, hipMemcpyDeviceToHost), "copy");
                *errors += h[0] + (h[1] ? 1000000u : 0u);
            }
            // slope between the two timed runs removes the launch's fixed cost
            ms = (t[2] - t[1]) * (float)phases / (float)(ph[2] - ph[1]);
        } else if (mode == 6) {
            // XCD-local barrier (wgs a multiple of 8)
            if (wgs % 8) throw std::runtime_error("the XCD-local barrier takes a multiple of 8 workgroups");
            PbXArgs a{};
            a.bar = d.alloc<uint32_t>(8 * 16 * 4);
            a.abort_flag = d.alloc<uint32_t>(256);
            a.err = d.alloc<uint32_t>(256);
            a.data = d.alloc<float>((size_t)2 * wgs * 64 * 4);
            float t[3];
            const uint32_t ph[3] = {phases / 4, phases / 4, phases};
            for (int k = 0; k < 3; ++k) {
                a.phases = ph[k];
                // each run starts its counters at 0: a run that aborted at the
                // spin limit leaves them off a multiple of the XCD's workgroups
                ck(hipMemsetAsync(a.bar, 0, 8 * 16 * 4, st), "memset");
                ck(hipMemsetAsync(a.abort_flag, 0, 256, st), "memset");
                ck(hipMemsetAsync(a.err, 0, 256, st), "memset");
                ck(hipStreamSynchronize(st), "sync");
                void* args[] = {&a};
                ck(hipEventRecord(e0, st), "record");
                ck(hipLaunchCooperativeKernel((const void*)k_pb_xcd, dim3(wgs), dim3(PB_WG), args, 0, st),
                   "cooperative launch");
                ck(hipEventRecord(e1, st), "record");
                ck(hipEventSynchronize(e1), "sync");
                ck(hipEventElapsedTime(&t[k], e0, e1), "elapsed");
                uint32_t h[3];
                ck(hipMemcpy(h, a.err, 8, hipMemcpyDeviceToHost), "copy");
                ck(hipMemcpy(h + 2, a.abort_flag, 4, hipMemcpyDeviceToHost), "copy");
                *errors += h[0] + h[1] * 1000u + (h[2] ? 1000000u : 0u);
            }
            ms = (t[2] - t[1]) * (float)phases / (float)(ph[2] - ph[1]);
        } else if (mode == 5) {
            // float atomics: wgs workgroups x bytes_per_phase/4 adds each over
            // a window of `phases` addresses (phases = contention spread)
            const uint32_t per_wg = (uint32_t)std::max<uint64_t>(1, bytes_per_phase / 4);
            float* acc = d.alloc<float>((size_t)phases * 4 + 256);
            ck(hipMemsetAsync(acc, 0, (size_t)phases * 4, st), "memset");
            k_pb_atomics<<<wgs, PB_WG, 0, st>>>(acc, phases, per_wg, per_wg);
            ck(hipEventRecord(e0, st), "record");
            for (int r = 0; r < 10; ++r) k_pb_atomics<<<wgs, PB_WG, 0, st>>>(acc, phases, per_wg, per_wg);
            ck(hipEventRecord(e1, st), "record");
            ck(hipEventSynchronize(e1), "sync");
            ck(hipEventElapsedTime(&ms, e0, e1), "elapsed");
            *us_per_phase = ms * 1e3 / 10.0;  // per launch of wgs * per_wg atomics
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
            (void)hipStreamDestroy(st);
            return 0;
        } else {
            throw std::runtime_error("mode must be 0..6");
        }
        *us_per_phase = ms * 1e3 / phases;
        ck(hipGetLastError(), "kernel");
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        (void)hipStreamDestroy(st);
        return 0;
    } catch (const std::exception& ex) {
        g_err = ex.what();
        return -1;
    }
}
