// Weight-gradient GEMM dW = dy^T x_hat (+ db = column sums of dy) from a Linear layer's saved
// activation, x_hat given in bf16 or as the quantizer's packed codes (decoded in the kernel).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dopt {

enum { DW_B_BF16 = 0, DW_B_PACKED = 1 };

struct DwArgs {
    const uint16_t* dy;       // bf16 [K][ldd], M columns used
    int64_t ldd;
    const uint16_t* xh;       // bf16 [K][ldx] (DW_B_BF16)
    int64_t ldx;
    const uint32_t* packed;   // codes of the flat [K * N] activation, groups of 2^lg (DW_B_PACKED)
    const uint16_t* scale;    // bf16 per group
    const uint16_t* minv;
    int lg;
    int bits;
    int64_t M, N, K;
    int64_t kt_per_split;     // set by the launcher
    int splits;               // splits with work (set by the launcher)
    float* partial;           // workspace: [splits][M][N] fp32, then [splits][M] for db
    float* db_partial;        // set by the launcher
};

int dw_splits(int64_t M, int64_t N, int64_t K);
int64_t dw_workspace_floats(int64_t M, int64_t N, int64_t K);
int launch_dw_gemm(DwArgs a, int mode, bool with_db, float* out32, uint16_t* out16, float* db, hipStream_t st);

}  // namespace dopt
