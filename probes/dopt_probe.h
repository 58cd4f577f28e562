/*
 * Measurement probes of this repository's benchmark (bench.py) and tests: libdopt_probe.so.
 *
 * They are no part of the product library (libdopt.so, include/dopt.h) and have no counterpart in
 * the reference. Each returns 0 or a negative status (-2 bad argument, -4 HIP error, the codes of
 * dopt.h) and leaves a message for dopt_probe_last_error(); each launches asynchronously on
 * `stream` (a hipStream_t passed as void*; NULL = the default stream) and never allocates or
 * synchronises.
 */
#ifndef DOPT_PROBE_H
#define DOPT_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

const char* dopt_probe_last_error(void);

/*
 * The memory system's ceiling for the quant-pack kernel's byte mix, measured with the same reads
 * and writes and no arithmetic. n_units units of 8 elements; per unit it reads 16 bytes of x and, when noise != NULL, 32 bytes of noise, and for
 * bits > 0 writes `bits` bytes to codes plus, every 32 units (a 256-element group), 8 bytes to
 * meta. bits = 0 reads only (codes must still point to one writable byte). The bytes written are
 * meaningless. Sizes: x 16*n_units, noise 32*n_units, codes bits*n_units, meta 8*ceil(n_units/32).
 */
int dopt_stream_probe(const void* x, const void* noise, void* codes, void* meta, int64_t n_units, int bits,
                      void* stream);

/*
 * The issue cost of one VALU instruction kind on this GPU, for the cost model of the instruction-bound kernels. Launches n_blocks workgroups of
 * 256 lanes (4 waves); every lane runs 8 independent chains of 512 steps of kind 0 = v_fma_f32,
 * 1 = v_exp_f32, 2 = v_rcp_f32, 3 = v_mad_u64_u32 + v_xor_b32 and writes one float to
 * out[n_blocks * 256] (meaningless values). Time per wave-instruction per SIMD = launch time *
 * (SIMDs) / (n_blocks * 4 * 8 * 512). Kinds 4 and 5 instead stream v_mfma_f32_32x32x16_bf16 in
 * the weight-gradient GEMM's inner-loop shape (a 4 x 4 grid of accumulators per wave, one wave per
 * SIMD, 64 steps of 16 MFMAs, nothing else), with pseudo-random (4) or constant (5) operands:
 * n_blocks * 4 * 64 * 16 * 32768 flops per launch. Kinds 6 and 7 do the same with the FP8 GEMM's
 * v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3, unit scales; 131072 flops each), random (6) or
 * constant (7) operands. Kind 8 checks the quant-pack kernels' fast exact-division helpers (step =
 * range / QMAX for QMAX = 3, 15, 255 and inv = 1 / step) against the IEEE fp32 division for every
 * non-negative fp32 bit pattern, strided over the grid: out[t] = thread t's count of differing
 * results (0 expected). n_blocks in [1, 65536].
 */
int dopt_valu_probe(int kind, float* out, int64_t n_blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DOPT_PROBE_H */
