// Peak probes: what this device's HBM and matrix cores sustain, measured with
// HIP events, so roofline fractions can be given against the measured peaks
// as well as the datasheet's. No counterpart in the reference.
//
// - copy: 16-byte nontemporal loads and stores, four in flight per thread,
//   32 workgroups per CU, over two buffers of `bytes` each (traffic 2 x bytes
//   per pass);
// - read: the same loads with an XOR reduction, 16 workgroups per CU, one
//   word written per thread (traffic bytes per pass);
// - mfma: v_mfma_f32_32x32x16_f16 on register operands (32,768 FLOP each), two
//   independent accumulators per wavefront, two wavefronts per SIMD; and the
//   same for v_mfma_f32_16x16x32_f16 (16,384 FLOP each, four wavefronts per
//   SIMD), the instruction the fused value net issues.
// Shapes chosen by a sweep on MI355X (workgroups per CU 4..64, 4..16 loads in
// flight, plain and nontemporal accesses; 1..8 accumulators, 1..4 wavefronts
// per SIMD): the fastest of each.
#include <hip/hip_runtime.h>

#include <string>

#include "../../include/wc_wave.h"

namespace wc {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int PROBE_BLOCK = 256;
constexpr int UNROLL = 4;

__global__ __launch_bounds__(PROBE_BLOCK) void k_probe_copy(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                           size_t n) {
    const size_t stride = size_t(gridDim.x) * PROBE_BLOCK;
    size_t i = size_t(blockIdx.x) * PROBE_BLOCK + threadIdx.x;
    for (; i + (UNROLL - 1) * stride < n; i += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; u++) __builtin_nontemporal_store(v[u], dst + i + u * stride);
    }
    for (; i < n; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(PROBE_BLOCK) void k_probe_read(const u32x4* __restrict__ src, uint32_t* __restrict__ out,
                                                           size_t n) {
    const size_t stride = size_t(gridDim.x) * PROBE_BLOCK;
    size_t i = size_t(blockIdx.x) * PROBE_BLOCK + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (UNROLL - 1) * stride < n; i += UNROLL * stride) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; u++) v[u] = __builtin_nontemporal_load(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; u++) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < n; i += stride) acc ^= src[i][0] ^ src[i][1] ^ src[i][2] ^ src[i][3];
    out[size_t(blockIdx.x) * PROBE_BLOCK + threadIdx.x] = acc;
}

__device__ inline void probe_operands(half8* a, half8* b) {
    const uint32_t lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        (*a)[k] = (_Float16)(1e-3f * (float)((lane + k) & 7));
        (*b)[k] = (_Float16)(1e-3f * (float)((lane * 3 + k) & 7));
    }
}

__global__ __launch_bounds__(PROBE_BLOCK) void k_probe_mfma32(float* __restrict__ out, uint32_t iters) {
    half8 a, b;
    probe_operands(&a, &b);
    float16v c0, c1;
#pragma unroll
    for (int j = 0; j < 16; j++) c0[j] = c1[j] = 0.0f;
    for (uint32_t it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; j++) s += c0[j] + c1[j];
    out[size_t(blockIdx.x) * PROBE_BLOCK + threadIdx.x] = s;
}

__global__ __launch_bounds__(PROBE_BLOCK) void k_probe_mfma16(float* __restrict__ out, uint32_t iters) {
    half8 a, b;
    probe_operands(&a, &b);
    float4v c0 = {0, 0, 0, 0}, c1 = c0;
    for (uint32_t it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c1, 0, 0, 0);
    }
    const float4v s = c0 + c1;
    out[size_t(blockIdx.x) * PROBE_BLOCK + threadIdx.x] = s[0] + s[1] + s[2] + s[3];
}

struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    Events() {
        hipEventCreate(&a);
        hipEventCreate(&b);
    }
    ~Events() {
        hipEventDestroy(a);
        hipEventDestroy(b);
    }
};

}  // namespace
int fail(int code, const std::string& msg);  // capi_host.cpp: sets wc_last_error

}  // namespace wc

using namespace wc;

extern "C" int wc_peak_probe(int device, size_t bytes, double* copy_gbs, double* read_gbs, double* mfma_tflops,
                             double* mfma16_tflops) {
    if (!copy_gbs || !read_gbs || !mfma_tflops || !mfma16_tflops || bytes < (1u << 20))
        return fail(WC_ERR_INVALID, "wc_peak_probe: null output or fewer than 1 MiB");
    if (hipSetDevice(device) != hipSuccess) return fail(WC_ERR_DEVICE, "wc_peak_probe: hipSetDevice failed");
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess)
        return fail(WC_ERR_DEVICE, "wc_peak_probe: hipGetDeviceProperties failed");
    const int cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
    const size_t n = bytes / sizeof(u32x4);
    const int copy_grid = cus * 32, read_grid = cus * 16;
    void *src = nullptr, *dst = nullptr, *out = nullptr;
    int rc = WC_OK;
    hipStream_t s = nullptr;
    // out holds one word per thread of the largest probe grid (read: 16 workgroups per CU)
    if (hipMalloc(&src, n * sizeof(u32x4)) != hipSuccess || hipMalloc(&dst, n * sizeof(u32x4)) != hipSuccess ||
        hipMalloc(&out, size_t(read_grid) * PROBE_BLOCK * 4) != hipSuccess || hipStreamCreate(&s) != hipSuccess) {
        rc = fail(WC_ERR_DEVICE, "wc_peak_probe: could not allocate the probe buffers");
    } else {
        Events ev;
        float ms = 0.0f;
        const int reps = 5;
        auto timed = [&](auto launch, int warm, int n_reps) {
            for (int w = 0; w < warm; w++) launch();
            hipEventRecord(ev.a, s);
            for (int r = 0; r < n_reps; r++) launch();
            hipEventRecord(ev.b, s);
            hipEventSynchronize(ev.b);
            hipEventElapsedTime(&ms, ev.a, ev.b);
            return double(ms) * 1e-3 / n_reps;
        };
        // contents do not matter to the copy or the read; fill them once so the
        // pages are resident
        hipMemsetAsync(src, 1, n * sizeof(u32x4), s);
        hipMemsetAsync(dst, 0, n * sizeof(u32x4), s);
        double t = timed([&] {
            hipLaunchKernelGGL(k_probe_copy, dim3(copy_grid), dim3(PROBE_BLOCK), 0, s, (const u32x4*)src, (u32x4*)dst,
                               n);
        }, 5, reps);
        *copy_gbs = 2.0 * double(n * sizeof(u32x4)) / t / 1e9;
        t = timed([&] {
            hipLaunchKernelGGL(k_probe_read, dim3(read_grid), dim3(PROBE_BLOCK), 0, s, (const u32x4*)src,
                               (uint32_t*)out, n);
        }, 5, reps);
        *read_gbs = double(n * sizeof(u32x4)) / t / 1e9;
        // 32x32x16: two wavefronts per SIMD (two 256-thread workgroups per CU);
        // 16x16x32: four (four workgroups per CU). Two accumulators each.
        const uint32_t iters = 8192;
        t = timed([&] {
            hipLaunchKernelGGL(k_probe_mfma32, dim3(cus * 2), dim3(PROBE_BLOCK), 0, s, (float*)out, iters);
        }, 100, 3);  // about 50 ms of warm-up launches: the clocks settle under a sustained MFMA load
        *mfma_tflops = double(cus) * 2 * (PROBE_BLOCK / 64) * iters * 2.0 * 32768.0 / t / 1e12;
        t = timed([&] {
            hipLaunchKernelGGL(k_probe_mfma16, dim3(cus * 4), dim3(PROBE_BLOCK), 0, s, (float*)out, iters);
        }, 2, 3);
        *mfma16_tflops = double(cus) * 4 * (PROBE_BLOCK / 64) * iters * 2.0 * 16384.0 / t / 1e12;
        if (hipGetLastError() != hipSuccess) rc = fail(WC_ERR_DEVICE, "wc_peak_probe: a probe kernel failed");
    }
    if (s) hipStreamDestroy(s);
    hipFree(src);
    hipFree(dst);
    hipFree(out);
    return rc;
}
