// BatchNorm normalize + quant-pack (forward) and dequant + reduce / input-gradient (backward).
//
// Channel c of an [N, C, HW] activation is one flat sequence of M = N * HW elements, element
// e = n * HW + s at offset n * stride_n + c * stride_c + s (spatial stride 1). Every element
// tensor of one call (x, y, x_hat, dy, dx) shares that geometry. Per channel, groups are runs of
// `group` consecutive elements, and the packed codes, the 1-bit ReLU mask and the bf16 scale/min
// are flat per-channel arrays:
//   packed       [C, M * bits / 32]   little-endian bitstream of the codes ([C, M * bits / 32 / A]
//                                     with avg_alam: one code per run of A elements)
//   relu_packed  [C, M / 32]          bit e of channel c = mask of element e
//   scale, minv  [C, M / group]       bf16
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dopt {

enum { BN_NORM = 0, BN_QUANT = 1, BN_RELU_QUANT = 2, BN_RELU6_QUANT = 3 };

// Elements one workgroup of the stats / backward-reduce kernels sums into one partial; a
// multiple of every group size, so a chunk holds whole groups.
constexpr int64_t BN_CHUNK = 8192;

struct BnGeom {
    int64_t N, C, HW, stride_n, stride_c;
};

struct BnFwdArgs {
    BnGeom g;
    const void* x;
    const float* sum;        // per-channel sum and sum of squares (sync == 0)
    const float* sumsq;
    const float* mean_in;    // per-channel mean and inverse std (sync == 1)
    const float* invstd_in;
    const float* w;
    const float* b;
    float eps;
    int sync;
    uint16_t* y;             // bf16
    uint16_t* xhat;          // bf16, BN_NORM only
    uint32_t* packed;
    uint32_t* relu_packed;
    uint16_t* scale;
    uint16_t* minv;
    float* mean_out;         // written when sync == 0
    float* var_out;
    float* run_mean;         // when set (sync == 0): run = run * run_keep + run_mom * batch statistic
    float* run_var;
    float run_keep, run_mom;
    const float* partial;    // when set (sync == 0): the statistics kernel's [2, C, nchunks] partials,
    int64_t nchunks;         // summed here instead of reading sum / sumsq
    int alam_lg;             // BN_QUANT with avg_alam: log2 of the run length A (0: off)
};

struct BnBwdArgs {
    BnGeom g;
    const uint16_t* xhat;    // bf16 x_hat tensor (BN_NORM)
    const uint32_t* packed;  // codes (other modes)
    const uint32_t* relu_packed;
    const uint16_t* scale;
    const uint16_t* minv;
    const void* dy;
    float* partial;          // [2, C, nchunks] workspace of the reduce
    float* dw;               // reduce outputs: sum(dy * x_hat), sum(dy)
    float* db;
    const float* dw_in;      // dx inputs; when NULL the dx kernel sums the reduce kernel's partials
    const float* db_in;      // itself and writes dw / db (no separate finalize launch)
    int64_t nchunks;
    const float* w;
    const float* var;        // variance, or the inverse std when var_is_invstd
    float eps;
    int var_is_invstd;
    uint16_t* dx;            // bf16
    int alam;                // BN_QUANT with avg_alam (the reduce adds the reference's noise, also at A = 1)
    int alam_lg;             // log2 of avg_alam's run length A
};

// vw: elements per vector access (8, 4, 2 or 1); it divides HW, stride_n and stride_c, and every
// element pointer is aligned to vw elements (bn_width in the C ABI picks it)
int64_t bn_nchunks(int64_t M);
// finalize = false: only the workgroup partials (for a consumer that sums them itself)
int launch_bn_reduce(const void* x, int dt, const BnGeom& g, float* partial, float* sum, float* sumsq, int vw,
                     hipStream_t s, bool finalize = true);
int launch_bn_fwd(const BnFwdArgs& a, int dt, int mode, int group, int bits, int vw, hipStream_t s);
int launch_bn_bwd_reduce(const BnBwdArgs& a, int dyt, int mode, int group, int bits, int vw, hipStream_t s,
                         bool finalize = true);
int launch_bn_bwd_dx(const BnBwdArgs& a, int dyt, int mode, int group, int bits, int vw, hipStream_t s);

}  // namespace dopt
