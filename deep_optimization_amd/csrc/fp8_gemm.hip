// FP8 e4m3 scaled GEMM launcher (kernels and tiling in fp8_gemm.h).
//
// Configuration: 256 x 256 workgroup tiles (128 x 128 per wave), GROUP_M = 4 tile rows per
// L2 group, even MFMA / memory interleave; the persistent kernels with one workgroup per CU
// (16x16x128 MFMAs from K = 8192, 32x32x64 below; the non-persistent kernel for an odd number of
// K slabs); measured on MI355X at 8192^3 and 4096x11008x4096.
#include <atomic>

#include "fp8_gemm.h"

namespace dopt {

using Fp8GemmDefault = Fp8GemmCfg<256, 256, 4, 0>;

namespace {
// compute units of the current device, queried once per device
int device_cu_count() {
    constexpr int MAX_DEV = 64;
    static std::atomic<int> cached[MAX_DEV];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return 256;
    int n = cached[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}
}  // namespace

int launch_fp8_gemm_nt(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, float out_scale, uint16_t* C, int64_t ldc, hipStream_t s) {
    return fp8_gemm_persistent_launch<Fp8GemmDefault>(A, B, M, N, K, lda, ldb, out_scale, C, ldc,
                                                      device_cu_count(), s);
}

}  // namespace dopt
