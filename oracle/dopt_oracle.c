/*
 * dopt_oracle.c - CPU restatement of Deep_Optimization's activation-compression quantizer.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP library: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. It is never linked into,
 * or called by, the product path (deep_optimization_amd/).
 *
 * Every entry point mirrors the C ABI in include/dopt.h (same argument meaning, no stream) and
 * cites the reference lines it restates. Paths are relative to the reference repository;
 * AC/ = Activation_Compression/.
 *
 * Arithmetic contract (built with -ffp-contract=off, no -ffast-math, round-to-nearest-even):
 *   every fp32 operation below is rounded separately, in the order written, except the three
 *   multiply-adds written as fmaf(): the reference's kernels are compiled with FMA contraction on
 *   (Triton's enable_fp_fusion default for AC/act_triton_kernel.py:114 `(x - xmin) * inv_scale +
 *   (0.5 - 1e-6)` and :223 `q * scale + xmin`; nvcc's default --fmad=true for
 *   AC/cpp_extension/include/quant_common.h:150 `(x - minv) * scale + noise - 0.5f`), so each of
 *   those is one correctly rounded fused multiply-add (C99 fmaf).
 *   Division (step = rng/QMAX, inv = 1/step) is IEEE correctly rounded; the reference's Triton
 *   division on NVIDIA hardware is not pinned at bit level (no golden data exists for it).
 *
 * Parity status of each function (how it is pinned; the tests in tests/test_oracle.py do it):
 *   grouping (flat / tile gather)  pinned: brute-force index maps + torch view/permute restatement
 *   min/max/step/inv               pinned: closed forms and known-answer groups
 *   nearest codes                  pinned: known-answer groups, |deq-x| <= step/2 bound, numpy
 *                                  restatement, exact rational fma on boundary cases
 *   stochastic codes (noise)       pinned: closed form with a given noise tensor, |deq-x| < step
 *   bit packing                    pinned: numpy.packbits(bitorder='little') special case
 *   dequant                        pinned: closed form
 *   Philox4x32-10                  pinned: published known-answer vectors (Salmon et al., SC'11)
 *   squash (tanh(2x)/2)            parity unpinned at bit level: the reference uses libdevice tanh
 *                                  on an NVIDIA GPU; this oracle uses the C library's tanhf.
 *   ReLU mask pack / unpack        pinned: known answers, numpy.packbits, closed form dy * mask
 *   GELU / SiLU value, derivative  parity unpinned at bit level (Triton exp, libdevice tanh);
 *                                  pinned to tolerance against torch's float64 gelu / silu and
 *                                  their autograd derivatives
 *   fused activation quant-pack    pinned: equals the quantizer above applied to the squashed
 *                                  derivative with the range floored at 1e-4
 *   fused activation backward      pinned: closed form bf16(dy * dequant)
 *   BatchNorm statistics           pinned: float64 sums; the normalization against torch's float64
 *                                  batch_norm (mean, biased variance, eps, affine)
 *   BatchNorm codes / mask / pack  pinned: known-answer ramps through the sync path (mean 0,
 *                                  invstd 1 makes x_hat = x), the pinned quantizer applied to the
 *                                  quantized values (squashed mode), bounds |x_hat' - t| <= scale/2
 *   BatchNorm squash (2 tanh(x/2)) parity unpinned at bit level (libdevice tanh in the reference)
 *   BatchNorm backward             pinned: against torch's float64 batch_norm autograd on x_hat
 *   ALAM averaging (quantize)      pinned: closed form (mean of the runs' nearest-code arguments),
 *                                  A = 1 equals oracle_quant_pack, A = 2 brute force in float64;
 *                                  summation order for A >= 4 is a stated choice
 *   ALAM noise (Triton randn)      Philox part pinned by the known-answer vectors; Box-Muller
 *                                  pinned against float64 from the same uniforms; moments of
 *                                  the noise checked; the fp32 log/cos are the C library's
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define O_F32 0
#define O_F16 1
#define O_BF16 2

#define O_NEAREST 0
#define O_STOCH_NOISE 1
#define O_STOCH_PHILOX 2

#define O_FLAG_CLAMP 1
#define O_FLAG_SQUASH 2

#define O_OK 0
#define O_EBITS -1
#define O_EINVAL -2

/* ---------------------------------------------------------------- scalar conversions */

static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* round-to-nearest-even fp32 -> bf16 (the rule of c10::BFloat16); NaN -> quiet NaN */
static uint16_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static float f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (ex == 0) {
        float v = (float)man * (1.0f / 16777216.0f); /* man * 2^-24, exact */
        return u2f(f2u(v) | sign);
    }
    if (ex == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((ex + 112u) << 23) | (man << 13));
}

static float load_elem(const void* x, int dtype, int64_t i) {
    if (dtype == O_F32) return ((const float*)x)[i];
    if (dtype == O_BF16) return bf16_to_f32(((const uint16_t*)x)[i]);
    return f16_to_f32(((const uint16_t*)x)[i]);
}

/* ---------------------------------------------------------------- Philox4x32-10
 * Counter-based generator of Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
 * 1, 2, 3", SC'11: round (c0,c1,c2,c3) -> (hi(M1*c2)^c1^k0, lo(M1*c2), hi(M0*c0)^c3^k1, lo(M0*c0))
 * with M0 = 0xD2511F53, M1 = 0xCD9E8D57; the key is bumped by the Weyl constants
 * (0x9E3779B9, 0xBB67AE85) between rounds. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

/* Noise for element `idx` (group-order linear index r*g + e) in Philox mode: the 16-element block
 * idx>>4 is the counter {blk_lo, blk_hi, offset_lo, offset_hi}, the seed is the key; element k of
 * the block takes byte k&3 of word k>>2, and u = (b + 0.5) * 2^-8 (exact in fp32). */
static float philox_u(int64_t idx, uint64_t seed, uint64_t offset) {
    uint64_t blk = (uint64_t)idx >> 4;
    uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)(blk >> 32), (uint32_t)offset,
                       (uint32_t)(offset >> 32)};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t w[4];
    oracle_philox4x32_10(ctr, key, w);
    int k = (int)(idx & 15);
    uint32_t b = (w[k >> 2] >> ((k & 3) * 8)) & 0xffu;
    return (float)b * (1.0f / 256.0f) + (1.0f / 512.0f);
}

/* Philox noise values for n consecutive group-order indices starting at idx0 (test helper). */
void oracle_philox_noise(int64_t idx0, int64_t n, uint64_t seed, uint64_t offset, float* u) {
    for (int64_t i = 0; i < n; ++i) u[i] = philox_u(idx0 + i, seed, offset);
}

/* ---------------------------------------------------------------- group layout
 * Element e of group r, as a linear index into x.
 * Flat: r*g + e (tensor_act_reshape_utils.py:46 `X.reshape(N, -1, Group_Size)`).
 * Tiles (tensor_act_reshape_utils.py:115-125): x viewed (N, C, H/s, s, W/s, s), permuted
 * (0,1,2,4,3,5), reshaped (N, C*(H/s)*(W/s), s*s): group r = ((n*C + c)*(H/s) + th)*(W/s) + tw
 * holds x[n, c, th*s + e/s, tw*s + e%s]. */
static int64_t elem_index(int64_t r, int e, int g, const int64_t* t, int s) {
    if (!t) return r * g + e;
    int64_t W = t[3], nW = W / s;
    int64_t band = r / nW, tw = r % nW;
    return band * s * W + tw * s + (int64_t)(e / s) * W + (e % s);
}

static int check_common(int64_t n_groups, int g, int bits, const int64_t* t, int* s_out) {
    if (bits != 1 && bits != 2 && bits != 4 && bits != 8) return O_EBITS;
    if (n_groups < 0 || g < 64 || g > 1024 || (g & (g - 1))) return O_EINVAL;
    *s_out = 0;
    if (t) {
        int s = (int)lrint(sqrt((double)g));
        if (s * s != g) return O_EINVAL;
        if (t[0] < 0 || t[1] < 0 || t[2] <= 0 || t[3] <= 0) return O_EINVAL;
        if (t[2] % s || t[3] % s) return O_EINVAL;
        if (t[0] * t[1] * (t[2] / s) * (t[3] / s) != n_groups) return O_EINVAL;
        *s_out = s;
    }
    return O_OK;
}

/* ---------------------------------------------------------------- quant-pack
 * AC/act_triton_kernel.py:53-171 per group (one Triton program per group):
 *   x = f32(x); [clamp(x, -a, a)] (:55-56); [x = tanh(x/0.5)*0.5] (:58)
 *   mn = min(x), mx = max(x) (:60-61); rng = mx - mn; step = rng > 0 ? rng/QMAX : 1 (:63-65)
 *   inv = 1/step (:71)
 *   nearest: q = clamp(trunc(fma(x-mn, inv, f32(0.5-1e-6))), 0, QMAX) (:114, :155-157)
 *   stochastic (the dormant CUDA form, AC/cpp_extension/include/quant_common.h:148-156, with the
 *   Triton step convention): q = clamp(rint_even(fma(x-mn, inv, u) - 0.5), 0, QMAX)
 *   word[w] = OR_j q[w*VPW + j] << (j*b) (:110-111, :159-160)
 *   scale = step, min = mn (:67-68; stored in meta_dtype).
 * Two definitions this restatement makes explicit (the reference leaves them to the hardware):
 *   - the stored minimum is canonicalised with mn + 0.0f, so -0.0 is stored as +0.0;
 *   - the code of a NaN is 0 (the clamp is applied in the float domain before truncation, which
 *     equals trunc-then-clamp for every non-NaN value). */
int oracle_quant_pack(const void* x, int x_dtype, int64_t n_groups, int g, int bits,
                      const int64_t* tile_nchw, int rounding, const float* noise, uint64_t seed,
                      uint64_t offset, int flags, float clamp_alpha, uint32_t* packed, void* scale,
                      void* minv, int meta_dtype) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, tile_nchw, &s);
    if (rc) return rc;
    if (x_dtype != O_F32 && x_dtype != O_F16 && x_dtype != O_BF16) return O_EINVAL;
    if (meta_dtype != O_F32 && meta_dtype != O_BF16) return O_EINVAL;
    if (rounding < 0 || rounding > 2) return O_EINVAL;
    if (rounding == O_STOCH_NOISE && !noise) return O_EINVAL;
    const int QMAX = (1 << bits) - 1;
    const int VPW = 32 / bits, NW = g / VPW;
    const float qmaxf = (float)QMAX;
    const float half_m = (float)(0.5 - 1e-6); /* 0x3EFFFFDE */

#pragma omp parallel
    {
        float* xs = (float*)malloc(sizeof(float) * g);
        int* q = (int*)malloc(sizeof(int) * g);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n_groups; ++r) {
            for (int e = 0; e < g; ++e) {
                float v = load_elem(x, x_dtype, elem_index(r, e, g, tile_nchw, s));
                if (flags & O_FLAG_CLAMP) v = fminf(fmaxf(v, -clamp_alpha), clamp_alpha);
                if (flags & O_FLAG_SQUASH) v = tanhf(v / 0.5f) * 0.5f;
                xs[e] = v;
            }
            float mn = xs[0], mx = xs[0];
            for (int e = 1; e < g; ++e) {
                mn = fminf(mn, xs[e]);
                mx = fmaxf(mx, xs[e]);
            }
            mn = mn + 0.0f;
            float rng = mx - mn;
            float step = (rng > 0.0f) ? rng / qmaxf : 1.0f;
            float inv = 1.0f / step;
            for (int e = 0; e < g; ++e) {
                float t = xs[e] - mn;
                float qf;
                if (rounding == O_NEAREST) {
                    qf = fmaf(t, inv, half_m);
                } else {
                    float u = (rounding == O_STOCH_NOISE) ? noise[r * g + e]
                                                          : philox_u(r * g + e, seed, offset);
                    qf = fmaf(t, inv, u);
                    qf = qf - 0.5f;
                }
                if (qf != qf) qf = 0.0f;
                qf = fminf(fmaxf(qf, 0.0f), qmaxf);
                q[e] = (rounding == O_NEAREST) ? (int)qf : (int)rintf(qf);
            }
            for (int w = 0; w < NW; ++w) {
                uint32_t word = 0;
                for (int j = 0; j < VPW; ++j) word |= (uint32_t)q[w * VPW + j] << (j * bits);
                packed[r * NW + w] = word;
            }
            if (meta_dtype == O_F32) {
                ((float*)scale)[r] = step;
                ((float*)minv)[r] = mn;
            } else {
                ((uint16_t*)scale)[r] = f32_to_bf16(step);
                ((uint16_t*)minv)[r] = f32_to_bf16(mn);
            }
        }
        free(xs);
        free(q);
    }
    return O_OK;
}

/* ---------------------------------------------------------------- dequant-unpack
 * AC/act_triton_kernel.py:199-241: q = (word >> (j*b)) & QMAX (:206-210);
 * y = fma(f32(q), scale, min) (:223, scale/min widened to fp32 :201-204), one rounding to y_dtype
 * (:241). With tiles the inverse layout of tensor_act_reshape_utils.py:131-154 is applied. */
int oracle_dequant_unpack(const uint32_t* packed, const void* scale, const void* minv,
                          int meta_dtype, int64_t n_groups, int g, int bits,
                          const int64_t* tile_nchw, void* y, int y_dtype) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, tile_nchw, &s);
    if (rc) return rc;
    if (meta_dtype != O_F32 && meta_dtype != O_BF16) return O_EINVAL;
    if (y_dtype != O_F32 && y_dtype != O_BF16) return O_EINVAL;
    const uint32_t QMAX = (1u << bits) - 1u;
    const int VPW = 32 / bits, NW = g / VPW;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_groups; ++r) {
        float sc, mn;
        if (meta_dtype == O_F32) {
            sc = ((const float*)scale)[r];
            mn = ((const float*)minv)[r];
        } else {
            sc = bf16_to_f32(((const uint16_t*)scale)[r]);
            mn = bf16_to_f32(((const uint16_t*)minv)[r]);
        }
        for (int e = 0; e < g; ++e) {
            uint32_t word = packed[r * NW + e / VPW];
            uint32_t qv = (word >> ((e % VPW) * bits)) & QMAX;
            float v = fmaf((float)qv, sc, mn);
            int64_t o = elem_index(r, e, g, tile_nchw, s);
            if (y_dtype == O_F32)
                ((float*)y)[o] = v;
            else
                ((uint16_t*)y)[o] = f32_to_bf16(v);
        }
    }
    return O_OK;
}

/* ---------------------------------------------------------------- ALAM averaging
 * The reference quantizer's avg_alam mode (AC/act_triton_kernel.py:336-368 host side, :116-118 and
 * :212-219 in the kernels; seed 42 in both operators, :339 and :374).
 *
 * Quantize: the non-ALAM pre-transform, min/max, step (rng/QMAX, 1 for rng = 0) and
 * qf[e] = fma(t[e], inv, 0.5 - 1e-6) (:55-114), then every run of A = alam_bits consecutive qf is
 * averaged: qa[c] = (qf[cA] + qf[cA+1] + ... + qf[cA+A-1]) / A (:116-118, a reshape to
 * (g/A, A) and tl.sum over the runs). The sum is taken left to right: Triton reduces the elements
 * a thread holds in index order, and a run of A <= 8 consecutive values of a 1-D block sits in
 * one thread; that order is this restatement's choice where A >= 4 (parity of the summation
 * order unpinned at bit level). code = clamp(trunc(qa), 0, QMAX) (:156-158; NaN -> 0 as in
 * oracle_quant_pack), g/A codes packed into NW/A words (:160-171). Scale and min are bf16.
 * Requires A a power of two dividing NW = g * bits / 32 (the reference's reshape).
 *
 * Dequantize (:199-241): code c = e / A repeated A times (:212-214), plus Gaussian noise
 * n = randn(seed + r, e) - 0.5 (:216-218), y = bf16(fma(code + n, scale, min)) (:223, :241).
 * randn is Triton's (triton/language/random.py, restated): Philox4x32-10 with counter
 * (e, 0, 0, 0) and key (lo32(seed + r), hi32(seed + r)); the first two output words w0, w1 map to
 * uniforms u = f32(w < 0 ? ~w : w) * 0x2fffffff (w as int32; the fp32 constant 4.6566127342e-10);
 * u1 = max(1e-7, u1), r = sqrt(-2 log u1), n = r cos(6.283185307179586 u2) (Box-Muller, first
 * output). log, cos and sqrt are the C library's fp32 functions here and libdevice's in the
 * reference: parity of the noise is to a few fp32 ulps, not bits. */
static float triton_uniform(uint32_t w) {
    int32_t i = (int32_t)w;
    if (i < 0) i = ~i;
    return (float)i * u2f(0x2fffffffu);
}

float oracle_triton_randn(uint64_t seed, uint32_t offset) {
    const uint32_t ctr[4] = {offset, 0u, 0u, 0u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t w[4];
    oracle_philox4x32_10(ctr, key, w);
    float u1 = triton_uniform(w[0]), u2 = triton_uniform(w[1]);
    u1 = fmaxf(1.0e-7f, u1);
    const float th = 6.283185307179586f * u2;
    const float r = sqrtf(-2.0f * logf(u1));
    return r * cosf(th);
}

/* Triton's tl.rand(seed, offset) for a 32-bit offset (triton/language/random.py, restated): the
 * first word of Philox4x32-10 with counter (offset, 0, 0, 0) and key (lo32, hi32 of seed), mapped
 * to [0, 1) as above. */
float oracle_triton_rand(uint64_t seed, uint32_t offset) {
    const uint32_t ctr[4] = {offset, 0u, 0u, 0u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t w[4];
    oracle_philox4x32_10(ctr, key, w);
    return triton_uniform(w[0]);
}

static int alam_check(int64_t n_groups, int g, int bits, int alam_bits) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, NULL, &s);
    if (rc) return rc;
    const int NW = g / (32 / bits);
    if (alam_bits < 1 || (alam_bits & (alam_bits - 1)) || NW % alam_bits) return O_EINVAL;
    return O_OK;
}

int oracle_alam_quant_pack(const void* x, int x_dtype, int64_t n_groups, int g, int bits, int alam_bits,
                           int flags, float clamp_alpha, uint32_t* packed, uint16_t* scale, uint16_t* minv) {
    int rc = alam_check(n_groups, g, bits, alam_bits);
    if (rc) return rc;
    if (x_dtype != O_F32 && x_dtype != O_F16 && x_dtype != O_BF16) return O_EINVAL;
    const int A = alam_bits, QMAX = (1 << bits) - 1, VPW = 32 / bits, ANW = g / VPW / A;
    const float qmaxf = (float)QMAX, half_m = (float)(0.5 - 1e-6);
#pragma omp parallel
    {
        float* xs = (float*)malloc(sizeof(float) * g);
        int* q = (int*)malloc(sizeof(int) * (g / A));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n_groups; ++r) {
            for (int e = 0; e < g; ++e) {
                float v = load_elem(x, x_dtype, r * g + e);
                if (flags & O_FLAG_CLAMP) v = fminf(fmaxf(v, -clamp_alpha), clamp_alpha);
                if (flags & O_FLAG_SQUASH) v = tanhf(v / 0.5f) * 0.5f;
                xs[e] = v;
            }
            float mn = xs[0], mx = xs[0];
            for (int e = 1; e < g; ++e) {
                mn = fminf(mn, xs[e]);
                mx = fmaxf(mx, xs[e]);
            }
            mn = mn + 0.0f;
            const float rng = mx - mn;
            const float step = (rng > 0.0f) ? rng / qmaxf : 1.0f;
            const float inv = 1.0f / step;
            for (int c = 0; c < g / A; ++c) {
                float sum = fmaf(xs[c * A] - mn, inv, half_m);
                for (int k = 1; k < A; ++k) sum = sum + fmaf(xs[c * A + k] - mn, inv, half_m);
                float qa = sum / (float)A;
                if (qa != qa) qa = 0.0f;
                qa = fminf(fmaxf(qa, 0.0f), qmaxf);
                q[c] = (int)qa;
            }
            for (int w = 0; w < ANW; ++w) {
                uint32_t word = 0;
                for (int j = 0; j < VPW; ++j) word |= (uint32_t)q[w * VPW + j] << (j * bits);
                packed[r * ANW + w] = word;
            }
            scale[r] = f32_to_bf16(step);
            minv[r] = f32_to_bf16(mn);
        }
        free(xs);
        free(q);
    }
    return O_OK;
}

int oracle_alam_dequant_unpack(const uint32_t* packed, const uint16_t* scale, const uint16_t* minv,
                               int64_t n_groups, int g, int bits, int alam_bits, uint64_t seed, uint16_t* y) {
    int rc = alam_check(n_groups, g, bits, alam_bits);
    if (rc) return rc;
    const int A = alam_bits, VPW = 32 / bits, ANW = g / VPW / A;
    const uint32_t QMAX = (1u << bits) - 1u;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_groups; ++r) {
        const float sc = bf16_to_f32(scale[r]), mn = bf16_to_f32(minv[r]);
        for (int e = 0; e < g; ++e) {
            const int c = e / A;
            const uint32_t qv = (packed[r * ANW + c / VPW] >> ((c % VPW) * bits)) & QMAX;
            const float n = oracle_triton_randn(seed + (uint64_t)r, (uint32_t)e);
            const float qf = (float)qv + (n - 0.5f);
            y[r * g + e] = f32_to_bf16(fmaf(qf, sc, mn));
        }
    }
    return O_OK;
}

/* ---------------------------------------------------------------- code-only pack / unpack
 * AC/act_triton_kernel.py:266-271: words = sum_j int32(int8 code[j]) << (j*b), int32 wrap-around.
 * AC/act_triton_kernel.py:304-322: code = (word >> (j*b)) & QMAX, stored as int8. */
int oracle_pack_codes(const int8_t* codes, int64_t n_groups, int g, int bits, uint32_t* packed) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, NULL, &s);
    if (rc) return rc;
    const int VPW = 32 / bits;
    const int64_t nw = n_groups * (g / VPW);
    for (int64_t w = 0; w < nw; ++w) {
        uint32_t acc = 0;
        for (int j = 0; j < VPW; ++j)
            acc += (uint32_t)(int32_t)codes[w * VPW + j] << (j * bits);
        packed[w] = acc;
    }
    return O_OK;
}

int oracle_unpack_codes(const uint32_t* packed, int64_t n_groups, int g, int bits, int8_t* codes) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, NULL, &s);
    if (rc) return rc;
    const int VPW = 32 / bits;
    const uint32_t QMAX = (1u << bits) - 1u;
    const int64_t nw = n_groups * (g / VPW);
    for (int64_t w = 0; w < nw; ++w)
        for (int j = 0; j < VPW; ++j)
            codes[w * VPW + j] = (int8_t)((packed[w] >> (j * bits)) & QMAX);
    return O_OK;
}

/* ---------------------------------------------------------------- fused activation layers
 * AC/modules/activations/kernel_implementation.py. Transcendentals use the C library's tanhf /
 * expf in fp32 (the reference uses Triton's exp and libdevice tanh): "parity unpinned" at bit
 * level for the GELU / SiLU values and derivatives; everything downstream of them (min/max,
 * codes, packing, the backward multiply) follows the quantizer's exact arithmetic. */
#define O_ACT_RELU 0
#define O_ACT_RELU6 1
#define O_ACT_GELU 2
#define O_ACT_SILU 3

static void store_elem(void* y, int dtype, int64_t i, float v) {
    if (dtype == O_F32)
        ((float*)y)[i] = v;
    else
        ((uint16_t*)y)[i] = f32_to_bf16(v);
}

/* GELU, tanh form (:496-519): u = a (x + b x^3), t = tanh(u), y = 0.5 x (1 + t),
 * dy/dx = 0.5 (1 + t) + 0.5 x (1 - t^2) a (1 + 3 b x^2) */
static void gelu_and_grad(float x, float* y, float* d) {
    const float a = 0.7978845608028654f, b = 0.044715f, b3 = 0.134145f;
    float x2 = x * x;
    float x3 = x * x2;
    float u = a * (x + b * x3);
    float t = tanhf(u);
    *y = 0.5f * x * (1.0f + t);
    float dt = 1.0f - t * t;
    float du = a * (1.0f + b3 * x2);
    *d = 0.5f * (1.0f + t) + 0.5f * x * dt * du;
}

/* SiLU (:225-229): s = 1 / (1 + exp(-x)), y = x s, dy/dx = s + x s (1 - s) */
static void silu_and_grad(float x, float* y, float* d) {
    float s = 1.0f / (1.0f + expf(-x));
    *y = x * s;
    *d = s + x * s * (1.0f - s);
}

/* relu_variance_fwd_fused_pack_kernel (:34-90): mask = x > 0 (relu6: 0 < x < 6),
 * y = mask ? bf16(x) : 0 stored in x's type, mask codes (0/1) packed b bits each. */
int oracle_relu_pack(const void* x, int x_dtype, int64_t n, int relu6, int bits, void* y, uint32_t* packed) {
    if (bits != 1 && bits != 2 && bits != 4 && bits != 8) return O_EBITS;
    if (x_dtype != O_F32 && x_dtype != O_BF16) return O_EINVAL;
    if (n < 0 || n % 64) return O_EINVAL;
    const int VPW = 32 / bits;
    for (int64_t w = 0; w < n / VPW; ++w) packed[w] = 0;
    for (int64_t i = 0; i < n; ++i) {
        float v = load_elem(x, x_dtype, i);
        int m = relu6 ? (v > 0.0f && v < 6.0f) : (v > 0.0f);
        float o = m ? bf16_to_f32(f32_to_bf16(v)) : 0.0f;
        store_elem(y, x_dtype, i, o);
        packed[i / VPW] |= (uint32_t)m << ((i % VPW) * bits);
    }
    return O_OK;
}

/* relu_bwd_fused_unpack_kernel (:93-143): dx = bf16(dy * float(code & 1)) */
int oracle_relu_unpack(const uint32_t* packed, const void* dy, int dy_dtype, int64_t n, int bits, uint16_t* dx) {
    if (bits != 1 && bits != 2 && bits != 4 && bits != 8) return O_EBITS;
    if (n < 0 || n % 64) return O_EINVAL;
    const int VPW = 32 / bits;
    for (int64_t i = 0; i < n; ++i) {
        uint32_t m = (packed[i / VPW] >> ((i % VPW) * bits)) & 1u;
        float g = load_elem(dy, dy_dtype, i);
        dx[i] = f32_to_bf16(g * (float)m);
    }
    return O_OK;
}

/* the unfused helpers relu_variance_kernel (:9-31), silu_triton (:154-175), gelu_triton (:437-466) */
int oracle_act_forward(const void* x, int x_dtype, int64_t n, int act, void* y, void* aux) {
    if (n < 0 || act < 0 || act > 3) return O_EINVAL;
    for (int64_t i = 0; i < n; ++i) {
        float v = load_elem(x, x_dtype, i);
        if (act == O_ACT_RELU || act == O_ACT_RELU6) {
            int m = act == O_ACT_RELU6 ? (v > 0.0f && v < 6.0f) : (v > 0.0f);
            if (x_dtype == O_F32)
                ((float*)y)[i] = m ? v : 0.0f;
            else
                ((uint16_t*)y)[i] = m ? ((const uint16_t*)x)[i] : 0;
            ((int8_t*)aux)[i] = (int8_t)m;
        } else {
            float yv, dv;
            if (act == O_ACT_GELU)
                gelu_and_grad(v, &yv, &dv);
            else
                silu_and_grad(v, &yv, &dv);
            ((uint16_t*)y)[i] = f32_to_bf16(yv);
            ((uint16_t*)aux)[i] = f32_to_bf16(dv);
        }
    }
    return O_OK;
}

/* The PACT clamp of AC/modules/ops.py: clamp_fused_fwd_triton (:545-561) stores
 * bf16(clamp(x, -alpha, alpha)) and the int8 mask |x| <= alpha; clamp_fused_bwd_triton (:563-584)
 * stores bf16(mask != 0 ? dy : 0). The clamp is fmaxf then fminf (a NaN x gives -alpha). */
int oracle_pact_clamp_fwd(const void* x, int x_dtype, int64_t n, float alpha, uint16_t* y, int8_t* mask) {
    if (n < 0 || !(alpha > 0.0f)) return O_EINVAL;
    for (int64_t i = 0; i < n; ++i) {
        const float v = load_elem(x, x_dtype, i);
        y[i] = f32_to_bf16(fminf(fmaxf(v, -alpha), alpha));
        mask[i] = (int8_t)(fabsf(v) <= alpha);
    }
    return O_OK;
}

int oracle_pact_clamp_bwd(const int8_t* mask, const void* dy, int dy_dtype, int64_t n, uint16_t* dx) {
    if (n < 0) return O_EINVAL;
    for (int64_t i = 0; i < n; ++i) dx[i] = f32_to_bf16(mask[i] != 0 ? load_elem(dy, dy_dtype, i) : 0.0f);
    return O_OK;
}

/* gelu_fwd_fused_quan_pack_triton (:468-535) / silu_fwd_fused_quan_pack_triton (:180-243):
 * y = act(x) as bf16; d = tanh(clamp(act'(x), -3, 3) / 0.5) * 0.5; per group mn, mx,
 * rng = max(mx - mn, 1e-4), step = rng / QMAX, inv = 1 / step,
 * q = clamp(trunc(fma(d - mn, inv, 0.5 - 1e-6)), 0, QMAX), packed as the quantizer does. */
int oracle_act_quant_pack(const void* x, int x_dtype, int act, int64_t n_groups, int g, int bits,
                          const int64_t* tile_nchw, uint16_t* y, uint32_t* packed, void* scale, void* minv,
                          int meta_dtype) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, tile_nchw, &s);
    if (rc) return rc;
    if (x_dtype != O_F32 && x_dtype != O_BF16) return O_EINVAL;
    if (act != O_ACT_GELU && act != O_ACT_SILU) return O_EINVAL;
    if (meta_dtype != O_F32 && meta_dtype != O_BF16) return O_EINVAL;
    const int QMAX = (1 << bits) - 1;
    const int VPW = 32 / bits, NW = g / VPW;
    const float qmaxf = (float)QMAX;
    const float half_m = (float)(0.5 - 1e-6);
#pragma omp parallel
    {
        float* ds = (float*)malloc(sizeof(float) * g);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < n_groups; ++r) {
            for (int e = 0; e < g; ++e) {
                int64_t idx = elem_index(r, e, g, tile_nchw, s);
                float v = load_elem(x, x_dtype, idx), yv, dv;
                if (act == O_ACT_GELU)
                    gelu_and_grad(v, &yv, &dv);
                else
                    silu_and_grad(v, &yv, &dv);
                y[idx] = f32_to_bf16(yv);
                dv = fminf(fmaxf(dv, -3.0f), 3.0f);
                ds[e] = tanhf(dv / 0.5f) * 0.5f;
            }
            float mn = ds[0], mx = ds[0];
            for (int e = 1; e < g; ++e) {
                mn = fminf(mn, ds[e]);
                mx = fmaxf(mx, ds[e]);
            }
            mn = mn + 0.0f;
            float rng = fmaxf(mx - mn, 1e-4f);
            float step = rng / qmaxf;
            float inv = 1.0f / step;
            for (int w = 0; w < NW; ++w) {
                uint32_t word = 0;
                for (int j = 0; j < VPW; ++j) {
                    float qf = fmaf(ds[w * VPW + j] - mn, inv, half_m);
                    if (qf != qf) qf = 0.0f;
                    qf = fminf(fmaxf(qf, 0.0f), qmaxf);
                    word |= (uint32_t)(int)qf << (j * bits);
                }
                packed[r * NW + w] = word;
            }
            if (meta_dtype == O_F32) {
                ((float*)scale)[r] = step;
                ((float*)minv)[r] = mn;
            } else {
                ((uint16_t*)scale)[r] = f32_to_bf16(step);
                ((uint16_t*)minv)[r] = f32_to_bf16(mn);
            }
        }
        free(ds);
    }
    return O_OK;
}

/* gelu_bwd / silu_bwd_fused_dequan_unpack (:360-395): dx = bf16(dy * fma(float(q), scale, min));
 * with noise (the SiLU backward's avg_alam at alam_bits = 1, :376-400) the code carries
 * tl.rand(seed + r, e) - 0.5: fma(float(q) + (u - 0.5), scale, min) */
static int act_dequant_mul_impl(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype,
                                int64_t n_groups, int g, int bits, const int64_t* tile_nchw, const void* dy,
                                int dy_dtype, int noise, uint64_t seed, uint16_t* dx) {
    int s = 0;
    int rc = check_common(n_groups, g, bits, tile_nchw, &s);
    if (rc) return rc;
    const uint32_t QMAX = (1u << bits) - 1u;
    const int VPW = 32 / bits, NW = g / VPW;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n_groups; ++r) {
        float sc, mn;
        if (meta_dtype == O_F32) {
            sc = ((const float*)scale)[r];
            mn = ((const float*)minv)[r];
        } else {
            sc = bf16_to_f32(((const uint16_t*)scale)[r]);
            mn = bf16_to_f32(((const uint16_t*)minv)[r]);
        }
        for (int e = 0; e < g; ++e) {
            uint32_t qv = (packed[r * NW + e / VPW] >> ((e % VPW) * bits)) & QMAX;
            int64_t o = elem_index(r, e, g, tile_nchw, s);
            float qf = (float)qv;
            if (noise) qf = qf + (oracle_triton_rand(seed + (uint64_t)r, (uint32_t)e) - 0.5f);
            float act = fmaf(qf, sc, mn);
            dx[o] = f32_to_bf16(load_elem(dy, dy_dtype, o) * act);
        }
    }
    return O_OK;
}

int oracle_act_dequant_mul(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype,
                           int64_t n_groups, int g, int bits, const int64_t* tile_nchw, const void* dy,
                           int dy_dtype, uint16_t* dx) {
    return act_dequant_mul_impl(packed, scale, minv, meta_dtype, n_groups, g, bits, tile_nchw, dy, dy_dtype, 0, 0,
                                dx);
}

int oracle_act_dequant_mul_alam(const uint32_t* packed, const void* scale, const void* minv, int meta_dtype,
                                int64_t n_groups, int g, int bits, const int64_t* tile_nchw, const void* dy,
                                int dy_dtype, uint64_t seed, uint16_t* dx) {
    return act_dequant_mul_impl(packed, scale, minv, meta_dtype, n_groups, g, bits, tile_nchw, dy, dy_dtype, 1,
                                seed, dx);
}

/* ---------------------------------------------------------------- BatchNorm
 * AC/modules/normalization/kernel_implementation.py (DOBatchNorm2d's kernels) and
 * AC/triton_kernel/norm_act_fusion/bn_act_fusion.py (BatchNorm + ReLU). Channel c is the flat
 * sequence e = n*HW + s (offset n*stride_n + c*stride_c + s); groups are runs of g consecutive
 * elements of a channel; packed [C, M*bits/32], relu_packed [C, M/32], scale/min bf16 [C, M/g].
 * The statistics here are double-precision sums (the GPU's fp32 sums differ only in rounding
 * order; the tests compare them with a tolerance and feed the GPU's sums back in), everything
 * downstream of them is the kernels' fp32 operation sequence. */
#define O_BN_NORM 0
#define O_BN_QUANT 1
#define O_BN_RELU_QUANT 2
#define O_BN_RELU6_QUANT 3

/* avg_alam's run length: a power of two dividing the group's g * bits / 32 code words
 * (kernel_registration.py:124-128) */
static int bn_alam_check(int g, int bits, int alam_bits) {
    const int nw = g * bits / 32;
    return alam_bits < 1 || (alam_bits & (alam_bits - 1)) || nw < 1 || nw % alam_bits;
}

static int64_t bn_off(int64_t HW, int64_t sn, int64_t sc, int64_t c, int64_t e) {
    int64_t n = e / HW;
    return n * sn + c * sc + (e - n * HW);
}

/* sum and sum of squares per channel (kernel_implementation.py:12-35), in double */
int oracle_bn_reduce(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t sn, int64_t sc,
                     double* sum, double* sumsq) {
    if (N < 0 || C < 0 || HW < 0) return O_EINVAL;
    const int64_t M = N * HW;
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < C; ++c) {
        double a = 0.0, b = 0.0;
        for (int64_t e = 0; e < M; ++e) {
            double v = load_elem(x, x_dtype, bn_off(HW, sn, sc, c, e));
            a += v;
            b += v * v;
        }
        sum[c] = a;
        sumsq[c] = b;
    }
    return O_OK;
}

/* Normalize (+ ReLU) (+ quant-pack), one fp32 rounding per operation:
 *   mean = sum/M; var = max(fma(-mean, mean, sumsq/M), 0); invstd = 1/sqrtf(var + eps)
 *     (kernel_implementation.py:66-71, :138-143; bn_act_fusion.py:55-60), or mean_in / invstd_in (sync)
 *   x_hat = (x - mean)*invstd; y = fma(x_hat, w, b) (:76-77, :150-151)
 *   BN_NORM: y, x_hat -> bf16 (:78-79)
 *   BN_QUANT: t = tanhf(clamp(x_hat, -3, 3)*0.5)/0.5 (:155-156); per group min/max,
 *     scale = rng > 0 ? rng/QMAX : 1, inv = 1/scale, q = trunc(fma(t - min, inv, 0.5-1e-6)),
 *     clamped to [0, QMAX] (:157-177)
 *   BN_RELU*: m = y > 0 (relu6: 0 < y < 6); y = m ? y : 0 (relu6: min(max(y, 0), 6)); codes of
 *     t = x_hat with q = trunc((t - min)/scale + (0.5-1e-6)) (bn_act_fusion.py:63-101)
 *   t_out (optional, fp32 [C, M]): the values the codes quantize
 *   alam_bits > 0 (BN_QUANT only, the avg_alam mode, :194-237): one code per run of A = alam_bits
 *     elements, trunc of the run's qf summed left to right and divided by A (the summation order is
 *     this restatement's choice, as in oracle_alam_quant_pack); packed [C, M*bits/32/A] */
int oracle_bn_norm_quant(const void* x, int x_dtype, int64_t N, int64_t C, int64_t HW, int64_t sn, int64_t sc,
                         const float* sum, const float* sumsq, const float* mean_in, const float* invstd_in,
                         int sync, const float* w, const float* b, float eps, int mode, int g, int bits,
                         uint16_t* y, uint16_t* x_hat, uint32_t* packed, uint32_t* relu_packed, uint16_t* scale,
                         uint16_t* minv, float* mean_out, float* var_out, float* t_out, int alam_bits) {
    if (N < 0 || C < 0 || HW < 0 || mode < 0 || mode > 3) return O_EINVAL;
    const int64_t M = N * HW;
    if (mode != O_BN_NORM) {
        if (bits != 1 && bits != 2 && bits != 4 && bits != 8) return O_EBITS;
        if (g < 32 || g > 512 || (g & (g - 1)) || M % g) return O_EINVAL;
    }
    if (alam_bits && (mode != O_BN_QUANT || bn_alam_check(g, bits, alam_bits))) return O_EINVAL;
    const int A = alam_bits > 0 ? alam_bits : 1;
    const int QMAX = (1 << bits) - 1;
    const float qmaxf = (float)QMAX;
    const float half_m = (float)(0.5 - 1e-6);
    const int64_t TW = M * bits / 32 / A, NG = mode == O_BN_NORM ? 0 : M / g;
#pragma omp parallel
    {
        float* t = (float*)malloc(sizeof(float) * (g > 0 ? g : 1));
#pragma omp for schedule(static)
        for (int64_t c = 0; c < C; ++c) {
            float mean, inv;
            if (sync) {
                mean = mean_in[c];
                inv = invstd_in[c];
            } else {
                const float Mf = (float)M;
                mean = sum[c] / Mf;
                float var = fmaf(-mean, mean, sumsq[c] / Mf);
                var = fmaxf(var, 0.0f);
                inv = 1.0f / sqrtf(var + eps);
                mean_out[c] = mean;
                var_out[c] = var;
            }
            const float wc = w[c], bc = b[c];
            if (mode == O_BN_NORM) {
                for (int64_t e = 0; e < M; ++e) {
                    const int64_t o = bn_off(HW, sn, sc, c, e);
                    float xh = (load_elem(x, x_dtype, o) - mean) * inv;
                    y[o] = f32_to_bf16(fmaf(xh, wc, bc));
                    x_hat[o] = f32_to_bf16(xh);
                }
                continue;
            }
            if (mode != O_BN_QUANT)
                for (int64_t k = 0; k < M / 32; ++k) relu_packed[c * (M / 32) + k] = 0;
            for (int64_t r = 0; r < NG; ++r) {
                float mn = INFINITY, mx = -INFINITY;
                for (int e = 0; e < g; ++e) {
                    const int64_t ee = r * g + e;
                    const int64_t o = bn_off(HW, sn, sc, c, ee);
                    float xh = (load_elem(x, x_dtype, o) - mean) * inv;
                    float yv = fmaf(xh, wc, bc);
                    if (mode == O_BN_QUANT) {
                        float cl = fminf(fmaxf(xh, -3.0f), 3.0f);
                        t[e] = tanhf(cl * 0.5f) / 0.5f;
                    } else {
                        int m = mode == O_BN_RELU6_QUANT ? (yv > 0.0f && yv < 6.0f) : (yv > 0.0f);
                        relu_packed[c * (M / 32) + ee / 32] |= (uint32_t)m << (ee % 32);
                        yv = mode == O_BN_RELU6_QUANT ? fminf(fmaxf(yv, 0.0f), 6.0f) : (m ? yv : 0.0f);
                        t[e] = xh;
                    }
                    y[o] = f32_to_bf16(yv);
                    if (t_out) t_out[c * M + ee] = t[e];
                    mn = fminf(mn, t[e]);
                    mx = fmaxf(mx, t[e]);
                }
                float rng = mx - mn;
                float step = rng > 0.0f ? rng / qmaxf : 1.0f;
                float invs = 1.0f / step;
                uint32_t* words = packed + c * TW + r * (g * bits / 32 / A);
                for (int k = 0; k < g * bits / 32 / A; ++k) words[k] = 0;
                /* one code per run of A elements (A = 1 without avg_alam): the run's qf summed left
                 * to right, divided by A (kernel_implementation.py:194-199) */
                for (int k = 0; k < g / A; ++k) {
                    float qf = 0.0f;
                    for (int j = 0; j < A; ++j) {
                        const int e = k * A + j;
                        const float v = mode == O_BN_QUANT ? fmaf(t[e] - mn, invs, half_m)
                                                           : (t[e] - mn) / step + half_m;
                        qf = j ? qf + v : v;
                    }
                    if (A > 1) qf = qf / (float)A;
                    if (qf != qf) qf = 0.0f;
                    qf = fminf(fmaxf(qf, 0.0f), qmaxf);
                    int q = (int)qf;
                    words[(k * bits) / 32] |= (uint32_t)q << ((k * bits) % 32);
                }
                scale[c * NG + r] = f32_to_bf16(step);
                minv[c * NG + r] = f32_to_bf16(mn);
            }
        }
        free(t);
    }
    return O_OK;
}

/* x_hat' and dy*m of element e of channel c for the backward (kernel_implementation.py:392-403,
 * :463-470; bn_act_fusion.py:160-172, :247-255): x_hat' = fma(q, scale, min) or the bf16 x_hat */
static void bn_bwd_elem(int mode, const uint16_t* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                        const uint16_t* scale, const uint16_t* minv, const void* dy, int dy_dtype, int64_t M,
                        int64_t HW, int64_t sn, int64_t sc, int g, int bits, int A, int noise, int64_t c, int64_t e,
                        float* xh, float* dyv) {
    const int64_t o = bn_off(HW, sn, sc, c, e);
    float d = load_elem(dy, dy_dtype, o);
    if (mode == O_BN_NORM) {
        *xh = bf16_to_f32(x_hat[o]);
    } else {
        /* code e / A (each code repeated A times with avg_alam, :374-377, :455-458), plus
         * tl.rand(42 + b, e mod g) - 0.5 in the avg_alam reduce, b = e / (2 g) the reference's
         * two-group block index (:379-381) */
        const int64_t bit = (e / A) * bits;
        uint32_t q = (packed[c * (M * bits / 32 / A) + bit / 32] >> (bit % 32)) & ((1u << bits) - 1u);
        const int64_t gi = c * (M / g) + e / g;
        float qf = (float)q;
        if (noise) qf = qf + (oracle_triton_rand(42u + (uint64_t)(e / (2 * g)), (uint32_t)(e % g)) - 0.5f);
        *xh = fmaf(qf, bf16_to_f32(scale[gi]), bf16_to_f32(minv[gi]));
        if (mode != O_BN_QUANT) {
            uint32_t m = (relu_packed[c * (M / 32) + e / 32] >> (e % 32)) & 1u;
            d = d * (float)m;
        }
    }
    *dyv = d;
}

/* dweight = sum(dy*m * x_hat'), dbias = sum(dy*m) per channel, in double */
int oracle_bn_bwd_reduce(int mode, const uint16_t* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                         const uint16_t* scale, const uint16_t* minv, const void* dy, int dy_dtype, int64_t N,
                         int64_t C, int64_t HW, int64_t sn, int64_t sc, int g, int bits, double* dw, double* db,
                         int alam_bits) {
    if (N < 0 || C < 0 || HW < 0 || mode < 0 || mode > 3) return O_EINVAL;
    if (alam_bits && (mode != O_BN_QUANT || bn_alam_check(g, bits, alam_bits))) return O_EINVAL;
    const int A = alam_bits > 0 ? alam_bits : 1;
    const int64_t M = N * HW;
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < C; ++c) {
        double a = 0.0, s = 0.0;
        for (int64_t e = 0; e < M; ++e) {
            float xh, d;
            bn_bwd_elem(mode, x_hat, packed, relu_packed, scale, minv, dy, dy_dtype, M, HW, sn, sc, g, bits, A,
                        alam_bits > 0, c, e, &xh, &d);
            a += (double)d * (double)xh;
            s += d;
        }
        dw[c] = a;
        db[c] = s;
    }
    return O_OK;
}

/* dx = ((fma(-x_hat', dw/M, dy*m - db/M)) * w) * invstd -> bf16, invstd = var_is_invstd ? var :
 * 1/sqrtf(var + eps) (kernel_implementation.py:252-255, :471-481; bn_act_fusion.py:256-278) */
int oracle_bn_bwd_dx(int mode, const uint16_t* x_hat, const uint32_t* packed, const uint32_t* relu_packed,
                     const uint16_t* scale, const uint16_t* minv, const void* dy, int dy_dtype, int64_t N, int64_t C,
                     int64_t HW, int64_t sn, int64_t sc, int g, int bits, const float* dw, const float* db,
                     const float* w, const float* var, float eps, int var_is_invstd, uint16_t* dx, int alam_bits) {
    if (N < 0 || C < 0 || HW < 0 || mode < 0 || mode > 3) return O_EINVAL;
    if (alam_bits && (mode != O_BN_QUANT || bn_alam_check(g, bits, alam_bits))) return O_EINVAL;
    const int A = alam_bits > 0 ? alam_bits : 1;
    const int64_t M = N * HW;
    const float Mf = (float)M;
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < C; ++c) {
        const float dwm = dw[c] / Mf, dbm = db[c] / Mf, wc = w[c];
        const float inv = var_is_invstd ? var[c] : 1.0f / sqrtf(var[c] + eps);
        for (int64_t e = 0; e < M; ++e) {
            float xh, d;
            bn_bwd_elem(mode, x_hat, packed, relu_packed, scale, minv, dy, dy_dtype, M, HW, sn, sc, g, bits, A, 0,
                        c, e, &xh, &d);
            dx[bn_off(HW, sn, sc, c, e)] = f32_to_bf16((fmaf(-xh, dwm, d - dbm) * wc) * inv);
        }
    }
    return O_OK;
}

/* ---------------------------------------------------------------- helpers for tests / bench */
int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void oracle_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }
