// zh_probe.hip -- measurement probes behind the decode step's launch structure
// (no counterpart in the reference; they time the hardware, not the model).
//
// ziggy_hip_probe_chain: a byte plan (the bytes each launch of a decode step
// streams, in order) streamed three ways: as one kernel over all the bytes,
// as one streaming kernel per entry captured in a HIP graph (the step's
// launch boundaries with no data dependency inside the kernels), and as the
// same number of empty kernels in a graph (the boundaries alone).
//
// ziggy_hip_probe_sync: what a dependency between workgroups costs inside
// one launch: a one-way hand-off between two workgroups (relaxed device-scope
// stores and loads; release/acquire), and a barrier of every workgroup of a
// CU-sized grid (per-workgroup arrival words polled by one wavefront; an
// arrival counter).
//
// ziggy_hip_probe_row_load: what a matvec's input row costs to bring into
// its lanes, per workgroup, right after the launch that wrote it: every lane
// loading its own 256-byte slot (the 16-byte loads of a wavefront 256 bytes
// apart), coalesced 16-byte loads of the same byte count, and the row loaded
// once per workgroup, coalesced, through LDS, every lane then reading its
// slot there; each for the row alone and with a second row of the same size
// beside it (the RMSNorm weights).
//
// Every wait is bounded (a spin limit far above any real wait); on expiry the
// result carries the flag and the timings are not valid.  The grids of the
// waiting kernels are at most one workgroup per CU, so all are resident.
#include <algorithm>
#include <vector>

#include "zh_internal.h"

using namespace zh;

namespace {

constexpr long kProbeSpin = 1L << 20;

// Streams n16 16-byte words of buf (128-byte aligned) with 16-byte loads, 8
// to 16 in flight per thread.  The shares are whole
// 128-byte lines, as equal as the line count allows (the last workgroup also
// takes the words past the last whole line), so every wavefront's 1 KiB load
// covers whole lines, as the decode kernels' row-aligned streams do.  One
// value per workgroup keeps the loads live.
__global__ void __launch_bounds__(256) probe_stream(const uint4 *buf, uint64_t n16, float *sink) {
    const uint64_t lines = n16 >> 3, q = lines / gridDim.x, r = lines % gridDim.x, b = blockIdx.x;
    uint64_t per = 8 * (q + (b < r ? 1 : 0));
    if (b == gridDim.x - 1) per += n16 & 7;
    const uint4 *p = buf + 8 * (b * q + (b < r ? b : r));
    if (per == 0) return;
    // every component feeds the value (a load whose other words go unused is
    // narrowed by the compiler to the words used).  Two register sets of
    // eight loads alternate: one set is issued before the other is consumed,
    // and neither is copied (a copy of a register still being loaded waits
    // for the load).  Loads are clamped to the share's last word: those past
    // the end re-read a line already fetched.
    const uint64_t last = per - 1;
    uint32_t acc = 0;
    uint4 va[8], vb[8];
    auto issue = [&](uint4 (&v)[8], uint64_t i) {
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = p[min(i + 256 * k, last)];
    };
    auto consume = [&](uint4 (&v)[8], uint64_t i) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            // opaque here, so the fold stays after the other set's issue
            asm volatile("" : "+v"(v[k].x), "+v"(v[k].y), "+v"(v[k].z), "+v"(v[k].w));
            const uint32_t f = v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
            acc ^= i + 256 * k < per ? f : 0u;
        }
    };
    uint64_t i = threadIdx.x;
    issue(va, i);
    for (; i < per; i += 16 * 256) {
        issue(vb, i + 8 * 256);
        __builtin_amdgcn_sched_barrier(0);
        consume(va, i);
        __builtin_amdgcn_sched_barrier(0);
        issue(va, i + 16 * 256);
        __builtin_amdgcn_sched_barrier(0);
        consume(vb, i + 8 * 256);
        __builtin_amdgcn_sched_barrier(0);
    }
    if (acc == 0x12345678u) sink[blockIdx.x] = (float)acc;
}

__global__ void probe_empty(float *sink) {
    if (threadIdx.x == 1u << 20) sink[0] = 0.f;
}

__device__ __forceinline__ unsigned ld_relaxed(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned ld_acquire(const unsigned *p) {
    return __hip_atomic_load(p, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
}

// Ping-pong between workgroup 0 and the last workgroup (another XCD), n round trips.
template <bool ACQREL>
__global__ void probe_pingpong(unsigned *a, unsigned *b, int n, unsigned long long *t, int *err) {
    const int last = gridDim.x - 1;
    if (threadIdx.x || (blockIdx.x != 0 && blockIdx.x != last)) return;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 1; i <= n; i++) {
        unsigned *mine = blockIdx.x == 0 ? a : b, *theirs = blockIdx.x == 0 ? b : a;
        if (blockIdx.x == 0) {
            if (ACQREL) __hip_atomic_store(mine, (unsigned)i, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            else __hip_atomic_store(mine, (unsigned)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        long s = 0;
        while ((ACQREL ? ld_acquire(theirs) : ld_relaxed(theirs)) != (unsigned)i)
            if (++s > kProbeSpin) {
                *err = 1;
                return;
            }
        if (blockIdx.x == last) {
            if (ACQREL) __hip_atomic_store(mine, (unsigned)i, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            else __hip_atomic_store(mine, (unsigned)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (blockIdx.x == 0) t[0] = __builtin_amdgcn_s_memrealtime() - t0;
}

// n barriers of the whole grid.  FLAGS: every workgroup stores its count to
// its own word (64 bytes apart), one wavefront polls all of them.  Else: one
// arrival counter, added to by every workgroup, polled by one thread.
template <bool FLAGS>
__global__ void __launch_bounds__(256) probe_barrier(unsigned *words, int n, unsigned long long *t, int *err) {
    const int G = gridDim.x, tid = threadIdx.x;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 1; i <= n; i++) {
        if (FLAGS) {
            if (tid == 0)
                __hip_atomic_store(words + blockIdx.x * 16, (unsigned)i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (tid < 64) {
                long s = 0;
                for (;;) {
                    bool ok = true;
                    for (int w = tid; w < G; w += 64) ok = ok && ld_relaxed(words + w * 16) >= (unsigned)i;
                    if (__all(ok)) break;
                    if (++s > kProbeSpin) {
                        if (tid == 0) *err = 2;
                        break;
                    }
                }
            }
        } else if (tid == 0) {
            __hip_atomic_fetch_add(words, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            long s = 0;
            while (ld_relaxed(words) < (unsigned)(i * G))
                if (++s > kProbeSpin) {
                    *err = 3;
                    break;
                }
        }
        __syncthreads();
    }
    if (blockIdx.x == 0 && tid == 0) t[0] = __builtin_amdgcn_s_memrealtime() - t0;
}

int cu_count(int dev) {
    int cus = 0;
    hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    return cus > 0 ? cus : 1;
}

constexpr int kRowProbeValues = 4096;

__global__ void __launch_bounds__(256) probe_row_write(float *row, float v) {
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < kRowProbeValues; i += gridDim.x * blockDim.x)
        row[i] = v + (float)i;
}

// NIN rows (x, then w) of kRowProbeValues floats.  MODE 0: lane l loads
// float4s 16l .. 16l + 15 of each row; 1: float4s 64j + l (coalesced, the
// same bytes per wavefront); 2: the workgroup loads each row once,
// coalesced, into LDS (one float4 of padding per 16) and lane l reads float4s
// 16l .. 16l + 15 there.  t[2b], t[2b + 1]: workgroup b's clock before its
// first load and after every lane holds its values.
template <int NIN, int MODE>
__global__ void __launch_bounds__(256, 2) probe_row_load(const float *x, const float *w, unsigned long long *t,
                                                         float *sink) {
    __shared__ float4 xs[MODE == 2 ? NIN * 1088 : 1];
    const int lane = threadIdx.x & 63, tid = threadIdx.x;
    const float4 *x4 = reinterpret_cast<const float4 *>(x), *w4 = reinterpret_cast<const float4 *>(w);
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    float4 r[NIN][16];
    if constexpr (MODE == 0 || MODE == 1) {
#pragma unroll
        for (int j = 0; j < 16; j++) {
            const int q = MODE == 0 ? lane * 16 + j : j * 64 + lane;
            r[0][j] = x4[q];
            if constexpr (NIN == 2) r[1][j] = w4[q];
        }
    } else {
        float4 g[NIN][4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            g[0][j] = x4[j * 256 + tid];
            if constexpr (NIN == 2) g[1][j] = w4[j * 256 + tid];
        }
#pragma unroll
        for (int i = 0; i < NIN; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int q = j * 256 + tid;
                xs[i * 1088 + q + (q >> 4)] = g[i][j];
            }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NIN; i++)
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int q = lane * 16 + j;
                r[i][j] = xs[i * 1088 + q + (q >> 4)];
            }
    }
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < NIN; i++)
#pragma unroll
        for (int j = 0; j < 16; j++) a += (r[i][j].x + r[i][j].y) + (r[i][j].z + r[i][j].w);
    __syncthreads();
    const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
    if (tid == 0) t[2 * blockIdx.x] = t0, t[2 * blockIdx.x + 1] = t1;
    if (a == -1.f) sink[0] = a;  // keeps the loads live
}

}  // namespace

extern "C" {

int ziggy_hip_probe_chain(ZiggyHipContext *ctx, const uint64_t *bytes, uint32_t n, uint32_t reps,
                          ZiggyHipChainProbe *out, char *err, size_t err_len) {
    if (!ctx || !bytes || !n || !out || n > 100000) {
        set_err(err, err_len, "invalid probe_chain arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    hipSetDevice(ctx->device);
    const int G = cu_count(ctx->device);
    // every entry streams its bytes in whole 16-byte words, from a 256-byte
    // aligned offset of one buffer
    std::vector<uint64_t> off(n), len(n);
    uint64_t total = 0, streamed = 0;
    for (uint32_t i = 0; i < n; i++) {
        len[i] = bytes[i] & ~15ull;
        off[i] = total;
        total += (len[i] + 255) & ~255ull;
        streamed += len[i];
    }
    if (!streamed) {
        set_err(err, err_len, "probe_chain: the plan streams nothing");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    hipStream_t st = ctx->stream;
    uint8_t *buf = nullptr;
    float *sink = nullptr;
    hipGraph_t g1 = nullptr, g2 = nullptr;
    hipGraphExec_t x1 = nullptr, x2 = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipMalloc(&buf, total);
    if (e == hipSuccess) e = hipMalloc(&sink, 4 * (size_t)G);
    if (e == hipSuccess) e = hipMemsetAsync(buf, 1, total, st);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    auto chain = [&](bool empty) {
        for (uint32_t i = 0; i < n; i++) {
            if (empty) hipLaunchKernelGGL(probe_empty, dim3(G), dim3(256), 0, st, sink);
            else hipLaunchKernelGGL(probe_stream, dim3(G), dim3(256), 0, st, (const uint4 *)(buf + off[i]), len[i] / 16, sink);
        }
        return hipGetLastError();
    };
    for (int k = 0; k < 2 && e == hipSuccess; k++) {
        e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
        hipError_t ec = e == hipSuccess ? chain(k == 1) : e;
        hipGraph_t gg = nullptr;
        hipError_t ee = hipStreamEndCapture(st, &gg);
        e = ec != hipSuccess ? ec : ee;
        if (e == hipSuccess) e = hipGraphInstantiate(k ? &x2 : &x1, gg, nullptr, nullptr, 0);
        (k ? g2 : g1) = gg;
    }
    double best[3] = {1e30, 1e30, 1e30};
    for (uint32_t r = 0; r < reps + 1 && e == hipSuccess; r++) {
        for (int k = 0; k < 3 && e == hipSuccess; k++) {
            e = hipEventRecord(e0, st);
            if (e == hipSuccess) {
                if (k == 0) {
                    hipLaunchKernelGGL(probe_stream, dim3(G), dim3(256), 0, st, (const uint4 *)buf, streamed / 16, sink);
                    e = hipGetLastError();
                } else {
                    e = hipGraphLaunch(k == 1 ? x1 : x2, st);
                }
            }
            if (e == hipSuccess) e = hipEventRecord(e1, st);
            if (e == hipSuccess) e = hipEventSynchronize(e1);
            float ms = 0.f;
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
            if (e == hipSuccess && r > 0 && ms < best[k]) best[k] = ms;  // the first round warms up
        }
    }
    if (x1) hipGraphExecDestroy(x1);
    if (x2) hipGraphExecDestroy(x2);
    if (g1) hipGraphDestroy(g1);
    if (g2) hipGraphDestroy(g2);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    hipStreamSynchronize(st);
    if (buf) hipFree(buf);
    if (sink) hipFree(sink);
    if (e != hipSuccess) return hip_fail(e, "probe_chain", err, err_len);
    out->bytes = streamed;
    out->kernels = n;
    out->workgroups = (uint32_t)G;
    out->one_kernel_ms = best[0];
    out->chain_ms = best[1];
    out->empty_chain_ms = best[2];
    return ZIGGY_HIP_OK;
}

int ziggy_hip_probe_sync(ZiggyHipContext *ctx, uint32_t rounds, ZiggyHipSyncProbe *out, char *err, size_t err_len) {
    if (!ctx || !out || rounds == 0 || rounds > 100000) {
        set_err(err, err_len, "invalid probe_sync arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    hipSetDevice(ctx->device);
    const int G = cu_count(ctx->device);
    hipStream_t st = ctx->stream;
    unsigned *words = nullptr;
    unsigned long long *t = nullptr;
    int *flag = nullptr;
    const size_t nwords = (size_t)G * 16 + 64;
    hipError_t e = hipMalloc(&words, nwords * 4);
    if (e == hipSuccess) e = hipMalloc(&t, 64);
    if (e == hipSuccess) e = hipMalloc(&flag, 4);
    if (e == hipSuccess) e = hipMemsetAsync(flag, 0, 4, st);
    const int n = (int)rounds;
    double res[4] = {0, 0, 0, 0};
    for (int k = 0; k < 4 && e == hipSuccess; k++) {
        e = hipMemsetAsync(words, 0, nwords * 4, st);
        if (e != hipSuccess) break;
        unsigned *a = words + (size_t)G * 16, *b = a + 32;
        switch (k) {
        case 0: hipLaunchKernelGGL(probe_pingpong<false>, dim3(G), dim3(64), 0, st, a, b, n, t, flag); break;
        case 1: hipLaunchKernelGGL(probe_pingpong<true>, dim3(G), dim3(64), 0, st, a, b, n, t, flag); break;
        case 2: hipLaunchKernelGGL(probe_barrier<true>, dim3(G), dim3(256), 0, st, words, n, t, flag); break;
        default: hipLaunchKernelGGL(probe_barrier<false>, dim3(G), dim3(256), 0, st, words, n, t, flag); break;
        }
        e = hipGetLastError();
        unsigned long long ticks = 0;
        if (e == hipSuccess) e = hipMemcpyAsync(&ticks, t, 8, hipMemcpyDeviceToHost, st);
        if (e == hipSuccess) e = hipStreamSynchronize(st);
        // s_memrealtime counts at 100 MHz; a ping-pong round trip is two hand-offs
        res[k] = (double)ticks * 0.01 / n / (k < 2 ? 2.0 : 1.0);
    }
    int f = 0;
    if (e == hipSuccess) e = hipMemcpyAsync(&f, flag, 4, hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (words) hipFree(words);
    if (t) hipFree(t);
    if (flag) hipFree(flag);
    if (e != hipSuccess) return hip_fail(e, "probe_sync", err, err_len);
    out->workgroups = (uint32_t)G;
    out->timed_out = f;
    out->handoff_relaxed_us = res[0];
    out->handoff_acqrel_us = res[1];
    out->barrier_flags_us = res[2];
    out->barrier_counter_us = res[3];
    return ZIGGY_HIP_OK;
}

int ziggy_hip_probe_row_load(ZiggyHipContext *ctx, uint32_t reps, ZiggyHipRowLoadProbe *out, char *err,
                             size_t err_len) {
    if (!ctx || !out || reps == 0 || reps > 10000) {
        set_err(err, err_len, "invalid probe_row_load arguments");
        return ZIGGY_HIP_INVALID_ARGUMENT;
    }
    hipSetDevice(ctx->device);
    const int G = 2 * cu_count(ctx->device);  // two workgroups per CU, as the decode matvecs
    hipStream_t st = ctx->stream;
    float *rows = nullptr, *sink = nullptr;
    unsigned long long *t = nullptr;
    hipError_t e = hipMalloc(&rows, 2 * kRowProbeValues * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&sink, 64);
    if (e == hipSuccess) e = hipMalloc(&t, (size_t)G * 16);
    if (e == hipSuccess) e = hipMemsetAsync(rows, 0, 2 * kRowProbeValues * sizeof(float), st);
    std::vector<unsigned long long> h((size_t)G * 2);
    double res[6] = {0, 0, 0, 0, 0, 0};
    for (int k = 0; k < 6 && e == hipSuccess; k++) {
        std::vector<double> per_rep;
        for (uint32_t r = 0; r <= reps && e == hipSuccess; r++) {  // rep 0 warms up
            hipLaunchKernelGGL(probe_row_write, dim3(16), dim3(256), 0, st, rows, (float)r);
            const float *x = rows, *w = rows + kRowProbeValues;
            switch (k) {
            case 0: hipLaunchKernelGGL((probe_row_load<1, 0>), dim3(G), dim3(256), 0, st, x, w, t, sink); break;
            case 1: hipLaunchKernelGGL((probe_row_load<1, 1>), dim3(G), dim3(256), 0, st, x, w, t, sink); break;
            case 2: hipLaunchKernelGGL((probe_row_load<1, 2>), dim3(G), dim3(256), 0, st, x, w, t, sink); break;
            case 3: hipLaunchKernelGGL((probe_row_load<2, 0>), dim3(G), dim3(256), 0, st, x, w, t, sink); break;
            case 4: hipLaunchKernelGGL((probe_row_load<2, 1>), dim3(G), dim3(256), 0, st, x, w, t, sink); break;
            default: hipLaunchKernelGGL((probe_row_load<2, 2>), dim3(G), dim3(256), 0, st, x, w, t, sink); break;
            }
            e = hipGetLastError();
            if (e == hipSuccess) e = hipMemcpyAsync(h.data(), t, (size_t)G * 16, hipMemcpyDeviceToHost, st);
            if (e == hipSuccess) e = hipStreamSynchronize(st);
            if (e != hipSuccess || r == 0) continue;
            std::vector<double> d(G);
            for (int b = 0; b < G; b++) d[b] = (double)(h[2 * b + 1] - h[2 * b]) * 0.01;  // 100 MHz clock
            std::nth_element(d.begin(), d.begin() + G / 2, d.end());
            per_rep.push_back(d[G / 2]);
        }
        if (e != hipSuccess) break;
        std::nth_element(per_rep.begin(), per_rep.begin() + per_rep.size() / 2, per_rep.end());
        res[k] = per_rep[per_rep.size() / 2];
    }
    if (rows) hipFree(rows);
    if (sink) hipFree(sink);
    if (t) hipFree(t);
    if (e != hipSuccess) return hip_fail(e, "probe_row_load", err, err_len);
    out->workgroups = (uint32_t)G;
    out->values = kRowProbeValues;
    for (int i = 0; i < 2; i++) {
        out->slot_us[i] = res[3 * i];
        out->coalesced_us[i] = res[3 * i + 1];
        out->lds_us[i] = res[3 * i + 2];
    }
    return ZIGGY_HIP_OK;
}

}  // extern "C"
