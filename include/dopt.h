/*
 * dopt.h - C ABI of the MI355X (gfx950) activation-compression library `libdopt.so`.
 *
 * The library replaces the device side of Deep_Optimization's activation compression:
 *   - the Triton kernels and their `act_lib::*` ops in
 *     Activation_Compression/act_triton_kernel.py:23-433, and
 *   - the pybind surface of the CUDA extension in
 *     Activation_Compression/cpp_extension/bind.cpp:44-63.
 * Each entry point below cites the reference interface it replaces.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers (HBM). The library never allocates, frees or synchronises;
 *     the caller owns every buffer.
 *   - `stream` is a hipStream_t passed as void*; NULL means the legacy default stream.
 *     Work is enqueued asynchronously on that stream.
 *   - Return value: DOPT_OK (0) or a negative DOPT_E* code. dopt_last_error() returns a
 *     thread-local, human-readable message for the last failure on the calling thread.
 *   - Packed codes form a little-endian bitstream per group: with b bits per code, element e of
 *     a group occupies bits [e*b, e*b+b) of the group's block of group_size*b/32 uint32 words
 *     (the word layout of act_triton_kernel.py:110-111 and :159-160).
 *   - Groups are numbered r = 0..n_groups-1 in the order of the reference's [N, G, g] tensor.
 */
#ifndef DOPT_H
#define DOPT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DOPT_ABI_VERSION 1

/* element types */
#define DOPT_F32 0
#define DOPT_F16 1
#define DOPT_BF16 2

/* rounding modes */
/* rounding modes; fma() is one correctly rounded multiply-add, matching the FMA contraction the
 * reference's compilers apply to `a * b + c` (Triton enable_fp_fusion, nvcc --fmad=true) */
#define DOPT_ROUND_NEAREST 0 /* q = trunc(fma(x-min, inv, 0.5-1e-6)), act_triton_kernel.py:114,:155-157 */
#define DOPT_ROUND_STOCH_NOISE 1 /* q = rint(fma(x-min, inv, u) - 0.5), quant_common.h:150-151; u from a tensor */
#define DOPT_ROUND_STOCH_PHILOX 2 /* same, u = (byte + 0.5)/256, one byte of Philox4x32-10 output per element:
                                   * element i (group order) uses byte i%16 of the call with counter
                                   * {i/16 (64 bit), offset (64 bit)} and key seed */

/* pre-transform flags (act_triton_kernel.py:55-58) */
#define DOPT_FLAG_CLAMP 1 /* x = clamp(x, -alpha, alpha) */
#define DOPT_FLAG_SQUASH 2 /* x = tanh(x / 0.5) * 0.5 (always on in the reference Triton path) */

/* status codes */
#define DOPT_OK 0
#define DOPT_EBITS -1 /* bits not in {1,2,4,8}: the reference raises ValueError (act_triton_kernel.py:329-330) */
#define DOPT_EINVAL -2 /* bad size, shape, dtype, layout, alignment or null pointer */
#define DOPT_EUNSUPPORTED -3 /* a valid request this build does not implement */
#define DOPT_EHIP -4 /* a HIP runtime error (launch failure, no device, ...) */

/* Version of this ABI; bump on any signature change. */
int dopt_abi_version(void);

/* Message describing the last failure on the calling thread ("" if none). */
const char* dopt_last_error(void);

/*
 * Per-group min/max quantize + bit-pack.
 * Replaces act_lib::quant_pack_triton (act_triton_kernel.py:336-368, kernel :23-171) and the
 * cpp_extension pack1..pack8 entry points (cpp_extension/bind.cpp:48-52,
 * cpp_extension/src/quant_pack_dispatch.cpp:17-115).
 *
 *   x           input activations, dtype x_dtype (F32/F16/BF16), 16-byte aligned.
 *               tile_nchw == NULL: contiguous [n_groups, group_size] (flat layout,
 *               tensor_act_reshape_utils.py:46).
 *               tile_nchw != NULL: a contiguous [N, C, H, W] tensor read through the s x s spatial
 *               tile gather of tensor_act_reshape_utils.py:100-128 (s*s == group_size, H % s == 0,
 *               W % s == 0, n_groups == N*C*(H/s)*(W/s)); the permuted copy is never materialised.
 *   group_size  power of two in [64, 1024]
 *   bits        1, 2, 4 or 8
 *   rounding    DOPT_ROUND_*; noise (fp32 [n_groups, group_size] in group order, values in [0,1))
 *               is read only for DOPT_ROUND_STOCH_NOISE; seed/offset only for DOPT_ROUND_STOCH_PHILOX.
 *   flags       DOPT_FLAG_* bit set; clamp_alpha used with DOPT_FLAG_CLAMP. The pre-transform
 *               (the reference's, act_triton_kernel.py:55-58) combines with every rounding mode.
 *   packed      out: uint32 [n_groups, group_size*bits/32], 16-byte aligned.
 *   scale, minv out: [n_groups] of meta_dtype (F32 or BF16): step = (max-min)/(2^b-1) (1.0 when
 *               max == min) and the group minimum (act_triton_kernel.py:60-68).
 */
int dopt_quant_pack(const void* x, int x_dtype, int64_t n_groups, int group_size, int bits,
                    const int64_t* tile_nchw, int rounding, const float* noise, uint64_t seed,
                    uint64_t offset, int flags, float clamp_alpha, uint32_t* packed, void* scale,
                    void* minv, int meta_dtype, void* stream);

/*
 * Unpack + dequantize: y = fma(float(q), scale, min), rounded once to y_dtype (F32 or BF16).
 * Replaces act_lib::dequant_unpack_triton (act_triton_kernel.py:372-395, kernel :174-241) and
 * the cpp_extension unpack1..unpack8 entry points (cpp_extension/bind.cpp:54-58,
 * cpp_extension/src/dequant_unpack_dispatch.cpp:12-41).
 *   tile_nchw == NULL: y is [n_groups, group_size]; otherwise y is the [N, C, H, W] tensor and
 *   the inverse tile scatter of tensor_act_reshape_utils.py:131-154 is fused in.
 */
int dopt_dequant_unpack(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype,
                        int64_t n_groups, int group_size, int bits, const int64_t* tile_nchw,
                        void* y, int y_dtype, void* stream);

/*
 * The reference quantizer's avg_alam mode (act_triton_kernel.py:336-395: quant_pack_triton and
 * dequant_unpack_triton with avg_alam=True; kernels :116-118 and :212-219).
 *
 * dopt_alam_quant_pack: as dopt_quant_pack with nearest rounding and bf16 scale/min, flat layout,
 * except that each run of alam_bits consecutive nearest-code arguments fma(x - min, 1/step,
 * 0.5 - 1e-6) is averaged (summed left to right) before truncation: group_size / alam_bits codes
 * per group in packed [n_groups, group_size*bits/32/alam_bits] uint32. alam_bits is a power of two
 * dividing group_size*bits/32 (the reference's reshape needs it); x any alignment of its dtype.
 *
 * dopt_alam_dequant_unpack: y bf16 [n_groups, group_size]; element e of group r is
 * bf16(fma(code[e / alam_bits] + randn(seed + r, e) - 0.5, scale[r], min[r])) with Triton's randn
 * (Philox4x32-10, counter (e, 0, 0, 0), key seed + r; Box-Muller); the reference passes seed 42.
 */
int dopt_alam_quant_pack(const void* x, int x_dtype, int64_t n_groups, int group_size, int bits, int alam_bits,
                         int flags, float clamp_alpha, uint32_t* packed, uint16_t* scale, uint16_t* minv,
                         void* stream);
int dopt_alam_dequant_unpack(const uint32_t* packed, const uint16_t* scale, const uint16_t* minv, int64_t n_groups,
                             int group_size, int bits, int alam_bits, uint64_t seed, uint16_t* y, void* stream);

/*
 * Code-only pack: int8 codes [n_groups, group_size] -> uint32 words [n_groups, group_size*bits/32],
 * word = sum_j int32(code[j]) << (j*bits) with 32-bit wrap-around (identical to OR for codes in
 * [0, 2^bits)). Replaces act_lib::pack_triton (act_triton_kernel.py:398-417, kernel :246-281).
 */
int dopt_pack_codes(const int8_t* codes, int64_t n_groups, int group_size, int bits,
                    uint32_t* packed, void* stream);

/*
 * Code-only unpack: words -> int8 codes, code = (word >> (j*bits)) & (2^bits-1).
 * Replaces act_lib::unpack_triton (act_triton_kernel.py:419-433, kernel :284-322).
 */
int dopt_unpack_codes(const uint32_t* packed, int64_t n_groups, int group_size, int bits,
                      int8_t* codes, void* stream);

/*
 * FP8 (OCP e4m3) scaled GEMM, NT layout: C[m][n] = out_scale * sum_k A[m][k] * B[n][k],
 * fp32 accumulation, C rounded once to bf16. A is [M, K] (row stride lda bytes), B is [N, K]
 * (row stride ldb bytes), C is [M, N] bf16 (row stride ldc elements). out_scale is
 * 1/(sA*sB) for per-tensor quantisation scales sX = 448/amax(X).
 * The reference's counterpart is the scale-less Triton GEMM Triton_Linear
 * (Activation_Compression/triton_kernel/linear.py:43-95, fp32 accumulate :81-86, cast :91), which
 * has no callers; the contraction it stands for is the weight/input-gradient GEMM of
 * _DOLinear.backward (Activation_Compression/modules/ops.py:508-512).
 * Any M, N >= 0 (edge tiles masked, like linear.py's masked loads and stores :80-81, :93-95);
 * K % 16 == 0 (DOPT_EUNSUPPORTED otherwise; K == 0 gives C = 0); A, B 16-byte aligned; lda, ldb
 * multiples of 16, >= K and < 2^23; ldc >= N (16-byte stores when C is 16-byte aligned and
 * ldc % 8 == 0, element stores otherwise).
 */
int dopt_fp8_gemm_nt(const uint8_t* A, const uint8_t* B, int64_t M, int64_t N, int64_t K,
                     int64_t lda, int64_t ldb, float out_scale, void* C, int64_t ldc, void* stream);

/*
 * Layout conversion for dopt_fp8_gemm_nt: dst[r * ld_dst + c] = src[r * stride_r + c * stride_c]
 * (byte matrices, element strides in bytes). The reference's Triton_Linear
 * (Activation_Compression/triton_kernel/linear.py:43-95) takes A [M, K] and B [K, N] with arbitrary
 * strides (:52-55); operands that are not K-contiguous with 16-byte aligned rows are packed with
 * this first (rows = M or N, cols = K). stride_r == 1 (B in its row-major [K, N] layout) runs a
 * tiled transpose, anything else a byte gather.
 */
int dopt_fp8_pack_kmajor(const uint8_t* src, int64_t rows, int64_t cols, int64_t stride_r, int64_t stride_c,
                         uint8_t* dst, int64_t ld_dst, void* stream);

/* ---------------------------------------------------------------- fused activation layers
 * The compressed ReLU / GELU / SiLU layers of Activation_Compression/modules/activations/ save the
 * layer's mask (ReLU) or its quantized derivative (GELU, SiLU) in the forward pass and apply it to
 * the incoming gradient in the backward pass. */
#define DOPT_ACT_RELU 0
#define DOPT_ACT_RELU6 1 /* mask = 0 < x < 6 */
#define DOPT_ACT_GELU 2  /* tanh form: x (1 + tanh(a (x + b x^3))) / 2, a = sqrt(2/pi), b = 0.044715 */
#define DOPT_ACT_SILU 3  /* x sigmoid(x) */

/*
 * y = relu(x) (x where the mask holds, else 0; fp32 inputs come out rounded to bf16 as in the
 * reference) and the mask packed as `bits`-bit codes (0 or 1) in the quantizer's bitstream.
 * x, y: n elements of x_dtype (F32 or BF16); packed: n*bits/32 uint32; n % 64 == 0.
 * Replaces act_lib::relu_fwd_fused_pack (modules/activations/kernel_registration.py:42-72,
 * kernel modules/activations/kernel_implementation.py:34-90).
 */
int dopt_relu_pack(const void* x, int x_dtype, int64_t n, int relu6, int bits, void* y, uint32_t* packed,
                   void* stream);

/*
 * dx = bf16(dy * mask), mask = lowest bit of each `bits`-bit code. dy: n elements of dy_dtype
 * (F32, F16 or BF16); dx: n bf16; n % 64 == 0.
 * Replaces act_lib::relu_bwd_fused_unpack (kernel_registration.py:74-94, kernel_implementation.py:93-143).
 */
int dopt_relu_unpack(const uint32_t* packed, const void* dy, int dy_dtype, int64_t n, int bits, void* dx,
                     void* stream);

/*
 * Unfused activation forward over n elements (any n): RELU/RELU6 -> y in x's type and an int8
 * mask in aux; GELU/SILU -> bf16 y and the bf16 derivative in aux.
 * Replaces act_lib::relu_triton, silu_triton, gelu_triton (kernel_registration.py:22-39,
 * :132-146, :245-259).
 */
int dopt_act_forward(const void* x, int x_dtype, int64_t n, int act, void* y, void* aux, void* stream);

/*
 * PACT clamp over n elements (any n): y = bf16(clamp(x, -alpha, alpha)) (fmaxf then fminf: a NaN
 * x gives -alpha) and the int8 mask |x| <= alpha. x F32, F16 or BF16, 16-byte aligned like y;
 * mask 8-byte aligned; alpha > 0 (else DOPT_EINVAL: at 0 the output's zero signs would depend
 * on how min and max order -0 and +0).
 * Replaces act_lib::group_pact_clamp_fwd (AC/modules/ops.py:587-603, kernel :545-561).
 */
int dopt_pact_clamp_forward(const void* x, int x_dtype, int64_t n, float alpha, void* y, int8_t* mask,
                            void* stream);

/*
 * Its gradient: dx = bf16(mask[e] != 0 ? dy[e] : 0) over n elements; dy F32, F16 or BF16.
 * Replaces act_lib::group_pact_clamp_bwd (AC/modules/ops.py:606-622, kernel :563-584).
 */
int dopt_pact_clamp_backward(const int8_t* mask, const void* dy, int dy_dtype, int64_t n, void* dx, void* stream);

/*
 * Fused GELU / SiLU forward: y = act(x) written as bf16, and per group the derivative
 * d = tanh(clamp(act'(x), -3, 3) / 0.5) * 0.5 quantized like dopt_quant_pack with nearest rounding,
 * the range floored at 1e-4 (kernel_implementation.py:225-243, :496-535). Layout arguments as in
 * dopt_quant_pack (tile_nchw != NULL: x and y are [N, C, H, W] read/written through the tile map).
 * x_dtype F32 or BF16; act DOPT_ACT_GELU or DOPT_ACT_SILU.
 * Replaces act_lib::gelu_fwd_fused_quan_pack (kernel_registration.py:261-292) and
 * act_lib::silu_fwd_quan_pack (:148-198).
 */
int dopt_act_quant_pack(const void* x, int x_dtype, int act, int64_t n_groups, int group_size, int bits,
                        const int64_t* tile_nchw, void* y, uint32_t* packed, void* scale, void* minv, int meta_dtype,
                        void* stream);

/*
 * Fused GELU / SiLU backward: dx = bf16(dy * fma(float(q), scale, min)) with dy (F32 or BF16) in
 * the output's layout. Replaces act_lib::gelu_bwd_fused_dequan_unpack (kernel_registration.py:295-319)
 * and act_lib::silu_bwd_fused_dequan_unpack (:202-237).
 */
int dopt_act_dequant_mul(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype, int64_t n_groups,
                         int group_size, int bits, const int64_t* tile_nchw, const void* dy, int dy_dtype, void* dx,
                         void* stream);

/*
 * dopt_act_dequant_mul with the SiLU backward's avg_alam noise at alam_bits = 1: dx = bf16(dy *
 * fma(float(q) + (u - 0.5), scale, min)), u = Triton's tl.rand(seed + r, e) for element e of group
 * r (Philox4x32-10 first word, counter (e, 0, 0, 0), key the low and high words of seed + r, as a
 * uniform in [0, 1)); the reference passes seed 42. Replaces act_lib::silu_bwd_fused_dequan_unpack
 * with avg_alam=True, alam_bits=1 (kernel_registration.py:201-237, kernel_implementation.py:376-400).
 */
int dopt_act_dequant_mul_alam(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype,
                              int64_t n_groups, int group_size, int bits, const int64_t* tile_nchw, const void* dy,
                              int dy_dtype, uint64_t seed, void* dx, void* stream);

/* ---------------------------------------------------------------- BatchNorm
 * An activation [N, C, HW] with element strides (stride_n, stride_c, 1): channel c is the flat
 * sequence e = n*HW + s of M = N*HW elements. Every element tensor of a call (x, y, x_hat, dy,
 * dx) has that geometry; all of them 16-byte aligned. Per channel, groups are runs of group_size
 * consecutive elements, and
 *   packed       uint32 [C, M*bits/32]   the little-endian code bitstream of the channel
 *   relu_packed  uint32 [C, M/32]        bit e = ReLU mask of element e
 *   scale, minv  bf16   [C, M/group_size]
 * Sums are two-stage (per-workgroup partials in `workspace`, then per channel in a fixed order):
 * deterministic, no atomics, nothing to zero. `workspace` holds dopt_bn_workspace_floats() floats.
 *
 * Modes: */
#define DOPT_BN_NORM 0        /* y, x_hat (bf16), kernel_implementation.py:38-91 */
#define DOPT_BN_QUANT 1       /* y, codes of 2 tanh(clamp(x_hat, -3, 3)/2), kernel_implementation.py:94-201 */
#define DOPT_BN_RELU_QUANT 2  /* relu(y), mask, codes of x_hat, bn_act_fusion.py:8-118 */
#define DOPT_BN_RELU6_QUANT 3 /* min(max(y, 0), 6), mask 0 < y < 6, codes of x_hat */

/* Floats of workspace the BatchNorm reductions need for this shape. */
int64_t dopt_bn_workspace_floats(int64_t N, int64_t C, int64_t HW);

/* sum[c], sumsq[c] over the channel (fp32). Replaces act_lib::bn_fwd_reduce
 * (AC/modules/normalization/kernel_registration.py:13-39, kernel_implementation.py:12-35). */
int dopt_bn_reduce(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c,
                   float* workspace, float* sum, float* sumsq, void* stream);

/* Normalize (+ ReLU) (+ quant-pack). sync = 0: mean = sum/M, var = max(fma(-mean, mean, sumsq/M), 0),
 * invstd = 1/sqrt(var + eps), mean_out/var_out written; sync = 1: mean_in and invstd_in are used
 * (SyncBatchNorm). x_hat = (x - mean)*invstd, y = fma(x_hat, weight, bias) -> bf16.
 * DOPT_BN_QUANT codes: t = 2 tanh(clamp(x_hat, -3, 3)/2), q = trunc(fma(t - min, 1/scale, 0.5-1e-6));
 * ReLU modes: q = trunc((x_hat - min)/scale + (0.5-1e-6)); scale = (max-min)/QMAX or 1.
 * M % group_size == 0 for the quant modes. Replaces act_lib::bn_fwd_norm (kernel_registration.py:42-80),
 * act_lib::bn_fwd_norm_quant_pack_fused (:83-150) and act_lib::bn_relu_fwd_norm_fused_quant_pack
 * (AC/triton_kernel/norm_act_fusion/kernel_registration.py:19-74). */
int dopt_bn_norm_quant(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                       int64_t stride_c, const float* sum, const float* sumsq, const float* mean_in,
                       const float* invstd_in, int sync, const float* weight, const float* bias, float eps, int mode,
                       int group_size, int bits, void* y, void* x_hat, uint32_t* packed, uint32_t* relu_packed,
                       void* scale, void* minv, float* mean_out, float* var_out, void* stream);

/* dopt_bn_norm_quant in DOPT_BN_QUANT mode with avg_alam: every run of A = alam_bits consecutive
 * elements of a channel becomes one code, trunc((qf[0] + ... + qf[A-1]) / A) clamped to
 * [0, QMAX] (NaN -> 0), qf = fma(t - min, 1/scale, 0.5-1e-6) as above, summed left to right.
 * alam_bits is a power of two dividing group_size*bits/32; packed is [C, M*bits/32/A], the
 * channel's M/A codes as one bitstream; scale / min per group as without avg_alam. Replaces
 * act_lib::bn_fwd_norm_quant_pack_fused with avg_alam=True (kernel_registration.py:83-150,
 * kernel_implementation.py:194-237). */
int dopt_bn_norm_quant_alam(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                            int64_t stride_c, const float* sum, const float* sumsq, const float* mean_in,
                            const float* invstd_in, int sync, const float* weight, const float* bias, float eps,
                            int group_size, int bits, int alam_bits, void* y, uint32_t* packed, void* scale,
                            void* minv, float* mean_out, float* var_out, void* stream);

/* The training forward of the compressed BatchNorm layer in one call: the statistics kernel's
 * workgroup partials (into workspace, dopt_bn_workspace_floats() floats), then the normalize (+ ReLU)
 * + quant-pack kernel of dopt_bn_norm_quant (sync = 0), which sums the partials itself in the
 * finalize order (bit-identical to dopt_bn_reduce's sums), writes mean_out / var_out and updates
 * running_mean / running_var (when not NULL) with run = fma(momentum, stat, run * (1 - momentum)),
 * stat the batch mean and biased variance. Replaces the act_lib::bn_fwd_reduce +
 * act_lib::bn_fwd_norm_quant_pack_fused (or bn_relu_fwd_norm_fused_quant_pack) pair and the
 * running-statistics update of _DOBatchNorm.forward (AC/modules/normalization/normalization_ops.py:45-57). */
int dopt_bn_train_forward(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                          int64_t stride_c, float* workspace, const float* weight, const float* bias, float eps,
                          int mode, int group_size, int bits, void* y, void* x_hat, uint32_t* packed,
                          uint32_t* relu_packed, void* scale, void* minv, float* mean_out, float* var_out,
                          float* running_mean, float* running_var, float momentum, void* stream);

/* No counterpart in the reference. dopt_bn_train_forward for callers that cannot allocate device
 * memory (code under HIP graph capture that may not call hipMalloc, tight serving loops, harnesses
 * that forbid allocation): the same arguments without `workspace`, the same outputs bit for bit.
 * The statistics kernel's partials go to a static per-device scratch array of
 * DOPT_BN_SCRATCH_FLOATS floats (4 MiB, held on each GPU the library runs on until the process
 * ends); a shape with dopt_bn_workspace_floats(N, C, HW) > DOPT_BN_SCRATCH_FLOATS returns
 * DOPT_EINVAL. No allocation of any kind. Every call on one GPU shares that GPU's scratch, so calls
 * that overlap on one GPU (e.g. on two streams at once) race; calls ordered on one stream do not. */
#define DOPT_BN_SCRATCH_FLOATS (1 << 20)
int dopt_bn_train_forward_noalloc(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t stride_n,
                                  int64_t stride_c, const float* weight, const float* bias, float eps, int mode,
                                  int group_size, int bits, void* y, void* x_hat, uint32_t* packed,
                                  uint32_t* relu_packed, void* scale, void* minv, float* mean_out, float* var_out,
                                  float* running_mean, float* running_var, float momentum, void* stream);

/* The backward of that layer in one call (quantized modes): the reduce kernel's partials into
 * workspace, then the dx kernel, which sums them (bit-identical to dopt_bn_bwd_reduce's dweight /
 * dbias), writes dweight / dbias and dx. Replaces the act_lib::bn_bwd_reduce_dequant_unpack_fused +
 * bn_bwd_dx_dequant_unpack_fused (or the bn_relu_* pair) of the reference's layers
 * (normalization_ops.py:95-157, AC/fusion/fused_ops.py:60-86). */
int dopt_bn_train_backward(int mode, const uint32_t* packed, const uint32_t* relu_packed, const void* scale,
                           const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C, int64_t HW,
                           int64_t stride_n, int64_t stride_c, int group_size, int bits, float* workspace,
                           const float* weight, const float* var, float eps, float* dweight, float* dbias, void* dx,
                           void* stream);

/* dweight[c] = sum(dy*m * x_hat'), dbias[c] = sum(dy*m), with x_hat' = fma(q, scale, min) (or the bf16
 * x_hat for DOPT_BN_NORM) and m the ReLU mask (ReLU modes) or 1. Replaces act_lib::bn_bwd_reduce
 * (kernel_registration.py:153-178), act_lib::bn_bwd_reduce_dequant_unpack_fused (:211-240) and
 * act_lib::bn_relu_bwd_reduce_fused_dequant_unpack (norm_act_fusion/kernel_registration.py:77-119). */
int dopt_bn_bwd_reduce(int mode, const void* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                       const void* scale, const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C,
                       int64_t HW, int64_t stride_n, int64_t stride_c, int group_size, int bits, float* workspace,
                       float* dweight, float* dbias, void* stream);

/* dopt_bn_bwd_reduce of dopt_bn_norm_quant_alam's codes: element e of a channel carries code e/A
 * plus the reference's noise, x_hat' = fma(q + (u - 0.5), scale, min) with u = Triton's
 * tl.rand(42 + e / (2 group_size), e mod group_size) (Philox4x32-10 first word, counter
 * (offset, 0, 0, 0), key the seed's low and high words, as a uniform in [0, 1)); the noise is
 * added at alam_bits = 1 too, whose codes are dopt_bn_norm_quant's. Replaces
 * act_lib::bn_bwd_reduce_dequant_unpack_fused with avg_alam=True (kernel_registration.py:211-240,
 * kernel_implementation.py:374-391). */
int dopt_bn_bwd_reduce_alam(const uint32_t* packed, const void* scale, const void* minv, const void* dy, int dy_dtype,
                            int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c, int group_size,
                            int bits, int alam_bits, float* workspace, float* dweight, float* dbias, void* stream);

/* dx = (fma(-x_hat', dweight/M, dy*m - dbias/M) * weight) * invstd -> bf16, invstd = var_is_invstd ? var :
 * 1/sqrt(var + eps). Replaces act_lib::bn_bwd_dx (kernel_registration.py:181-208),
 * act_lib::bn_bwd_dx_dequant_unpack_fused (:243-276) and act_lib::bn_relu_bwd_dx_fused_dequant_unpack
 * (norm_act_fusion/kernel_registration.py:122-166). */
int dopt_bn_bwd_dx(int mode, const void* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                   const void* scale, const void* minv, const void* dy, int dy_dtype, int64_t N, int64_t C, int64_t HW,
                   int64_t stride_n, int64_t stride_c, int group_size, int bits, const float* dweight,
                   const float* dbias, const float* weight, const float* var, float eps, int var_is_invstd, void* dx,
                   void* stream);

/* dopt_bn_bwd_dx of dopt_bn_norm_quant_alam's codes: x_hat' = fma(q, scale, min) with q = code e/A
 * (no noise). Replaces act_lib::bn_bwd_dx_dequant_unpack_fused with avg_alam=True
 * (kernel_registration.py:243-276, kernel_implementation.py:455-462). */
int dopt_bn_bwd_dx_alam(const uint32_t* packed, const void* scale, const void* minv, const void* dy, int dy_dtype,
                        int64_t N, int64_t C, int64_t HW, int64_t stride_n, int64_t stride_c, int group_size,
                        int bits, int alam_bits, const float* dweight, const float* dbias, const float* weight,
                        const float* var, float eps, int var_is_invstd, void* dx, void* stream);

/* ---------------------------------------------------------------- Linear weight gradient
 * dW[m][n] = sum_k dy[k][m] * x_hat[k][n] (bf16 MFMA, fp32 accumulation) and, when db is not NULL,
 * db[m] = sum_k dy[k][m]: the weight and bias gradients of a Linear layer with K tokens, M out and
 * N in features. dy: bf16 [K, ldd] (M columns used). x_hat either bf16 [K, ldx] (x_hat != NULL) or
 * the quantizer's packed codes of the flat [K*N] activation (packed, scale, minv bf16 per group of
 * group_size consecutive elements, b bits), decoded in the kernel to bf16(fma(q, scale, min)), the
 * value dequant_unpack writes. Outputs fp32 dw_f32 and/or bf16 dw_bf16 [M, N] row-major, fp32 db.
 * The K range is split across workgroups; the fp32 partials go through `workspace`
 * (dopt_dw_gemm_workspace_floats(M, N, K) floats) and are summed in a fixed order (deterministic).
 * Requires M % 256 == 0, N % 256 == 0, ldd % 8 == 0, ldx % 8 == 0, 16-byte aligned dy / x_hat.
 * Replaces, for the compressed Linear layer, the dequantize + `dy_flatten.T.mm(input_flatten)` of
 * AC/modules/ops.py:508-512 (the reference's Triton fused attempt lives only in test2.ipynb). */
int64_t dopt_dw_gemm_workspace_floats(int64_t M, int64_t N, int64_t K);
int dopt_dw_gemm(const void* dy, int64_t ldd, const void* x_hat, int64_t ldx, const uint32_t* packed,
                 const void* scale, const void* minv, int group_size, int bits, int64_t M, int64_t N, int64_t K,
                 float* workspace, float* dw_f32, void* dw_bf16, float* db, void* stream);

/*
 * HIP graph tools for capturing a whole training step (forward, backward, optimizer step) as
 * Activation_Compression/cuda_graph_utils.py:82-120 (`Graph.capture_cuda_graph_qdrop`) does.
 * `graph` is a captured, not yet instantiated hipGraph_t passed as void* (torch:
 * `torch.cuda.CUDAGraph(keep_graph=True).raw_cuda_graph()` after capture).
 *
 * dopt_graph_node_counts: counts[t] = number of nodes of hipGraphNodeType t (child graphs' nodes
 * included) for t < n_counts; other types are not counted.
 *
 * dopt_graph_replace_memsets: replaces every memset node (the record of a hipMemsetAsync made
 * during capture, by this library's caller or by any library it calls) with a kernel node that
 * writes the same bytes, with the same dependencies and dependents; *n_replaced = number
 * replaced. Call it before the graph is instantiated. (Memset nodes in replayed graphs are
 * avoided on this platform; this library's own entry points issue none.)
 */
int dopt_graph_node_counts(void* graph, int64_t* counts, int n_counts);
int dopt_graph_replace_memsets(void* graph, int64_t* n_replaced);

#ifdef __cplusplus
}
#endif

#endif /* DOPT_H */
