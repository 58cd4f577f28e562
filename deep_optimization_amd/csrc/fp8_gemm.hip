// FP8 e4m3 scaled GEMM launcher (kernel and tiling in fp8_gemm.h).
//
// Configuration: 256 x 256 workgroup tiles (128 x 128 per wave), GROUP_M = 4 tile rows per
// L2 group, even MFMA / memory interleave; measured on MI355X at 8192^3 and 4096x11008x4096.
#include "fp8_gemm.h"

namespace dopt {

using Fp8GemmDefault = Fp8GemmCfg<256, 256, 4, 0>;

int launch_fp8_gemm_nt(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K, int64_t lda,
                       int64_t ldb, float out_scale, uint16_t* C, int64_t ldc, hipStream_t s) {
    return fp8_gemm_launch<Fp8GemmDefault>(A, B, M, N, K, lda, ldb, out_scale, C, ldc, s);
}

}  // namespace dopt
