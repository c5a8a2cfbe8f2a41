// Test support for the co-tenant gate (kda/mi350x/benchmark/eval_kda_mi350x.py:883-976): a kernel that holds whole
// CUs for a bounded time.  Each 64-thread workgroup allocates the LDS it is given (all of a CU's 160 KiB: one per CU),
// marks itself started and sleeps until `ticks` of the constant-rate wall clock have passed, then exits: every wave
// reaches the exit by itself.  The started marks are plain vector stores, one dword per lane of the workgroup's slot.
#include <hip/hip_runtime.h>

namespace {
__global__ void __launch_bounds__(64) hog_kernel(unsigned long long ticks, int* started) {
    extern __shared__ int lds[];
    lds[threadIdx.x] = 1;
    started[(size_t)blockIdx.x * 64 + threadIdx.x] = 1;
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < ticks) __builtin_amdgcn_s_sleep(8);
    if (lds[threadIdx.x] == 2) started[(size_t)blockIdx.x * 64 + threadIdx.x] = 2;  // keeps the LDS allocation live
}
}  // namespace

// blocks workgroups with lds_bytes of LDS each for `seconds` on `stream`; `started` holds blocks * 64 ints.  Returns
// 0 or the HIP error code.
extern "C" int kda355_test_hog(int blocks, int lds_bytes, double seconds, int* started, void* stream) {
    if (blocks < 1 || lds_bytes < 256 || lds_bytes > 160 * 1024 || seconds <= 0.0 || seconds > 10.0 || !started)
        return (int)hipErrorInvalidValue;
    int rate_khz = 0;
    hipError_t e = hipDeviceGetAttribute(&rate_khz, hipDeviceAttributeWallClockRate, 0);
    if (e != hipSuccess) return (int)e;
    e = hipFuncSetAttribute(reinterpret_cast<const void*>(hog_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            lds_bytes);
    if (e != hipSuccess) return (int)e;
    const unsigned long long ticks = (unsigned long long)(seconds * (double)rate_khz * 1000.0);
    hipLaunchKernelGGL(hog_kernel, dim3(blocks), dim3(64), lds_bytes, reinterpret_cast<hipStream_t>(stream), ticks,
                       started);
    return (int)hipGetLastError();
}
