// Measurement kernels for bench.py, built as their own library (libflint_probe.so, not part
// of the attention library or its C ABI): what this GPU itself reaches for the three limits the
// attention kernels are judged against, measured in the same run as the kernels.
//   * streaming read: a plain read of a large buffer, 16-byte non-temporal loads, one contiguous
//     range per workgroup (the decode kernel's access pattern without its maths);
//   * f16 MFMA rate: v_mfma_f32_32x32x16_f16 (the prefill kernel's instruction) in 4 or 8
//     independent accumulator chains per wave, two waves per SIMD;
//   * launch cost: an empty kernel, and a tiny kernel that reads what the previous launch wrote
//     (the dependency a split merge has on the kernel before it).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int STREAM_THREADS = 512;
constexpr uint32_t NEVER = 0x9e3779b9u;

// Workgroup g folds the 16-byte units [g * n16, (g + 1) * n16) of src into one word. Two sets of
// D 16-byte loads per thread are in flight; each set is refilled with the chunk two further on as
// soon as it is folded (the decode kernel's two register sets). Loads past the range read its
// last unit again. The store depends on every load and is practically never taken, so the loads
// stay live.
template <int D>
__global__ __launch_bounds__(STREAM_THREADS) void stream_read_kernel(const u32x4 *__restrict__ src, uint32_t n16,
                                                                     uint32_t *sink) {
    constexpr uint32_t CHUNK = (uint32_t)D * STREAM_THREADS;
    const u32x4 *p = src + (uint64_t)blockIdx.x * n16;  // scalar base; 32-bit unit offsets per thread
    const uint32_t last = n16 - 1, n_chunks = (n16 + CHUNK - 1) / CHUNK;
    const uint32_t t = threadIdx.x;
    u32x4 a[D], b[D];
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < D; j++) a[j] = __builtin_nontemporal_load(p + min(t + j * STREAM_THREADS, last));
#pragma unroll
    for (int j = 0; j < D; j++) b[j] = __builtin_nontemporal_load(p + min(CHUNK + t + j * STREAM_THREADS, last));
    for (uint32_t c = 0; c < n_chunks; c += 2) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < D; j++) acc ^= a[j].x ^ a[j].y ^ a[j].z ^ a[j].w;
        if (c + 2 < n_chunks) {
#pragma unroll
            for (int j = 0; j < D; j++)
                a[j] = __builtin_nontemporal_load(p + min((c + 2) * CHUNK + t + j * STREAM_THREADS, last));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < D; j++) acc ^= b[j].x ^ b[j].y ^ b[j].z ^ b[j].w;
        if (c + 3 < n_chunks) {
#pragma unroll
            for (int j = 0; j < D; j++)
                b[j] = __builtin_nontemporal_load(p + min((c + 3) * CHUNK + t + j * STREAM_THREADS, last));
        }
    }
    if (acc == NEVER) sink[blockIdx.x] = acc;
}

// Each wave runs `iters` steps of NC independent 32x32x16 f16 MFMAs (NC x 32768 FLOPs).
template <int NC>
__global__ __launch_bounds__(512) void mfma_rate_kernel(int iters, float *sink) {
    const float t = (float)threadIdx.x * 1e-3f;
    f16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        a[j] = (_Float16)(t + 0.01f * j);
        b[j] = (_Float16)(t - 0.01f * j);
    }
    f32x16 c[NC];
#pragma unroll
    for (int k = 0; k < NC; k++) c[k] = f32x16{};
    for (int i = 0; i < iters; i++) {
#pragma unroll
        for (int k = 0; k < NC; k++) c[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[k], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NC; k++)
#pragma unroll
        for (int j = 0; j < 16; j++) s += c[k][j];
    if (s == 1234.5f) sink[blockIdx.x] = s;
}

__global__ void empty_kernel() {}

// 64 workgroups of 64 threads: out[i] = in[i] + 1 over 4096 floats
__global__ __launch_bounds__(64) void chain_kernel(const float *in, float *out) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    out[i] = in[i] + 1.f;
}

}  // namespace

extern "C" {

// Reads `bytes` of `buf` over `n_wg` workgroups (equal contiguous ranges). bytes must be a
// multiple of 16 * n_wg and buf 16-byte aligned; `sink` holds n_wg words. Returns 0, or -1 for
// bad arguments, or the HIP error code.
// `depth` (4, 8 or 12) is the number of 16-byte loads in each of a thread's two sets. A workgroup's
// range is at most 2^32 - 1 units.
int32_t flint_probe_stream_read(const void *buf, uint64_t bytes, int32_t n_wg, int32_t depth, void *sink,
                                void *stream) {
    if (!buf || !sink || n_wg < 1 || n_wg > 65535 || ((uintptr_t)buf & 15) || bytes % (16ull * n_wg) ||
        bytes / 16 / n_wg == 0 || bytes / 16 / n_wg > 0xffffffffull)
        return -1;
    const dim3 grid(n_wg), block(STREAM_THREADS);
    const u32x4 *src = (const u32x4 *)buf;
    const uint32_t n16 = (uint32_t)(bytes / 16 / n_wg);
    if (depth == 4)
        hipLaunchKernelGGL(stream_read_kernel<4>, grid, block, 0, (hipStream_t)stream, src, n16, (uint32_t *)sink);
    else if (depth == 8)
        hipLaunchKernelGGL(stream_read_kernel<8>, grid, block, 0, (hipStream_t)stream, src, n16, (uint32_t *)sink);
    else if (depth == 12)
        hipLaunchKernelGGL(stream_read_kernel<12>, grid, block, 0, (hipStream_t)stream, src, n16, (uint32_t *)sink);
    else
        return -1;
    return (int32_t)hipGetLastError();
}

// n_wg workgroups of 8 waves, each wave `iters` x `chains` (4 or 8) independent MFMAs:
// n_wg * 8 * iters * chains * 32768 FLOPs. `sink` holds n_wg floats.
int32_t flint_probe_mfma(int32_t n_wg, int32_t iters, int32_t chains, void *sink, void *stream) {
    if (!sink || n_wg < 1 || n_wg > 65535 || iters < 1) return -1;
    if (chains == 4)
        hipLaunchKernelGGL(mfma_rate_kernel<4>, dim3(n_wg), dim3(512), 0, (hipStream_t)stream, iters, (float *)sink);
    else if (chains == 8)
        hipLaunchKernelGGL(mfma_rate_kernel<8>, dim3(n_wg), dim3(512), 0, (hipStream_t)stream, iters, (float *)sink);
    else
        return -1;
    return (int32_t)hipGetLastError();
}

int32_t flint_probe_empty(void *stream) {
    hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream);
    return (int32_t)hipGetLastError();
}

// out[i] = in[i] + 1 for i < 4096 (in and out hold 4096 floats)
int32_t flint_probe_chain(const float *in, float *out, void *stream) {
    if (!in || !out) return -1;
    hipLaunchKernelGGL(chain_kernel, dim3(64), dim3(64), 0, (hipStream_t)stream, in, out);
    return (int32_t)hipGetLastError();
}

}  // extern "C"
