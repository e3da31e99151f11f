// Measured HBM bandwidth: a read stream and a copy over a device buffer far
// larger than the 256 MB memory-side cache, timed with HIP events.  The
// roofline of the decode prices its algorithmic bytes against both the
// published peak and this measured one.
#include <hip/hip_runtime.h>

#include "internal.h"

namespace {

constexpr uint32_t HBM_THREADS = 256, HBM_UNROLL = 8, HBM_BLOCKS_PER_CU = 64;
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Every 16-byte word of p[0..n16) read once with non-temporal loads, eight in
// flight per thread, 64 workgroups per CU (the fastest of the launch shapes
// and policies measured on MI355X: 6.9 TB/s over 4 GiB, against 5.4-6.2 TB/s
// with cached loads or fewer loads in flight); the xor of the words decides a
// store that practically never happens, so the loads cannot be dropped.
__global__ void __launch_bounds__(HBM_THREADS) hbm_read_kernel(const u32x4v *__restrict__ p, size_t n16,
                                                                unsigned *out) {
    const size_t stride = (size_t)gridDim.x * HBM_THREADS;
    size_t i = (size_t)blockIdx.x * HBM_THREADS + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (HBM_UNROLL - 1) * stride < n16; i += HBM_UNROLL * stride) {
        u32x4v v[HBM_UNROLL];
#pragma unroll
        for (uint32_t k = 0; k < HBM_UNROLL; k++) v[k] = __builtin_nontemporal_load(p + i + k * stride);
#pragma unroll
        for (uint32_t k = 0; k < HBM_UNROLL; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += stride) {
        const u32x4v v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) out[blockIdx.x & 255u] = acc;
}

__global__ void __launch_bounds__(HBM_THREADS) hbm_copy_kernel(const u32x4v *__restrict__ src, u32x4v *__restrict__ dst,
                                                                size_t n16) {
    const size_t stride = (size_t)gridDim.x * HBM_THREADS;
    size_t i = (size_t)blockIdx.x * HBM_THREADS + threadIdx.x;
    for (; i + (HBM_UNROLL - 1) * stride < n16; i += HBM_UNROLL * stride) {
        u32x4v v[HBM_UNROLL];
#pragma unroll
        for (uint32_t k = 0; k < HBM_UNROLL; k++) v[k] = __builtin_nontemporal_load(src + i + k * stride);
#pragma unroll
        for (uint32_t k = 0; k < HBM_UNROLL; k++) __builtin_nontemporal_store(v[k], dst + i + k * stride);
    }
    for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

using namespace sinter;

extern "C" int sinter_hbm_peak(uint64_t bytes, uint32_t reps, double *read_gbs, double *copy_gbs) {
    if (!read_gbs || !copy_gbs || reps == 0 || bytes < (64ull << 20))
        return set_error(SINTER_ERR_ARG, "hbm_peak: bytes >= 64 MiB, reps >= 1, outputs non-null");
    bytes &= ~((16ull << 20) - 1);   // whole 16 MiB units
    int dev = 0, cus = 0;
    if (!hip_ok(hipGetDevice(&dev), "hbm_peak: device") ||
        !hip_ok(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hbm_peak: CUs"))
        return SINTER_ERR_HIP;
    unsigned char *buf = nullptr;
    unsigned *out = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    int rc = SINTER_OK;
    if (!hip_ok(hipMalloc(&buf, bytes), "hbm_peak: alloc") || !hip_ok(hipMalloc(&out, 1024), "hbm_peak: alloc") ||
        !hip_ok(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hbm_peak: stream") ||
        !hip_ok(hipEventCreate(&e0), "hbm_peak: event") || !hip_ok(hipEventCreate(&e1), "hbm_peak: event")) {
        rc = SINTER_ERR_HIP;
    }
    if (rc == SINTER_OK) {
        const size_t n16 = bytes / 16, half16 = n16 / 2;
        const uint32_t grid = (uint32_t)cus * HBM_BLOCKS_PER_CU;
        const u32x4v *src = reinterpret_cast<const u32x4v *>(buf);
        u32x4v *dst = reinterpret_cast<u32x4v *>(buf + bytes / 2);
        float ms_r = 0.0f, ms_c = 0.0f;
        bool ok = hip_ok(hipMemsetAsync(buf, 0x5a, bytes, s), "hbm_peak: fill");
        // one untimed pass of each, then reps timed passes
        hipLaunchKernelGGL(hbm_read_kernel, dim3(grid), dim3(HBM_THREADS), 0, s, src, n16, out);
        hipLaunchKernelGGL(hbm_copy_kernel, dim3(grid), dim3(HBM_THREADS), 0, s, src, dst, half16);
        ok = ok && hip_ok(hipEventRecord(e0, s), "hbm_peak: event");
        for (uint32_t r = 0; r < reps; r++)
            hipLaunchKernelGGL(hbm_read_kernel, dim3(grid), dim3(HBM_THREADS), 0, s, src, n16, out);
        ok = ok && hip_ok(hipEventRecord(e1, s), "hbm_peak: event") && hip_ok(hipEventSynchronize(e1), "hbm_peak: read") &&
             hip_ok(hipEventElapsedTime(&ms_r, e0, e1), "hbm_peak: time");
        ok = ok && hip_ok(hipEventRecord(e0, s), "hbm_peak: event");
        for (uint32_t r = 0; r < reps; r++)
            hipLaunchKernelGGL(hbm_copy_kernel, dim3(grid), dim3(HBM_THREADS), 0, s, src, dst, half16);
        ok = ok && hip_ok(hipEventRecord(e1, s), "hbm_peak: event") && hip_ok(hipEventSynchronize(e1), "hbm_peak: copy") &&
             hip_ok(hipEventElapsedTime(&ms_c, e0, e1), "hbm_peak: time");
        ok = ok && hip_ok(hipGetLastError(), "hbm_peak: launch");
        if (!ok || ms_r <= 0.0f || ms_c <= 0.0f) {
            rc = SINTER_ERR_HIP;
        } else {
            *read_gbs = (double)bytes * reps / (ms_r * 1e-3) / 1e9;
            *copy_gbs = (double)bytes * reps / (ms_c * 1e-3) / 1e9;   // half read + half written
        }
    }
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    if (out) (void)hipFree(out);
    if (buf) (void)hipFree(buf);
    return rc;
}
