// Device-side helpers shared by the gfx950 activation-compression kernels.
//
// Wave model: CDNA4 wavefronts are 64 lanes. A group of `group_size` values is spread over LPG
// consecutive lanes (LPG a power of two, aligned), so every cross-lane reduction stays inside an
// aligned LPG-lane block and is done with DPP lane permutes folded into the min/max (no LDS
// round trip) up to 16 lanes, and with v_permlane16/32_swap beyond that.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dopt {

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };
enum { RN_NEAREST = 0, RN_NOISE = 1, RN_PHILOX = 2 };
enum { FL_CLAMP = 1, FL_SQUASH = 2 };

template <int DT>
struct DType {
    static constexpr int bytes = DT == DT_F32 ? 4 : 2;
    static constexpr int per16 = 16 / bytes;  // elements in one 16-byte chunk
};

// ------------------------------------------------------------------ grids past 2^32 work-items
// A dispatch's grid size is a 32-bit count of work-items per dimension, so a 1-D grid holds at
// most 2^32 - 1 work-items. Launchers whose block count grows with the input take linear_grid():
// a 1-D grid while it fits, else rows of GRID_ROW blocks, block b at x = b % GRID_ROW and
// y = b / GRID_ROW. Kernels recover b with linear_block() (every row of a multi-row grid is
// GRID_ROW wide); the blocks past the last one, in the final row, take the kernels' own
// past-the-end path (loads clamped or skipped, no stores).
constexpr uint32_t GRID_ROW = 1u << 16;

inline dim3 linear_grid(uint64_t blocks, uint32_t threads) {
    if (blocks * threads <= 0xFFFFFFFFull) return dim3((uint32_t)blocks);
    return dim3(GRID_ROW, (uint32_t)((blocks + GRID_ROW - 1) / GRID_ROW));
}

__device__ __forceinline__ uint64_t linear_block() { return (uint64_t)blockIdx.y * GRID_ROW + blockIdx.x; }

// ------------------------------------------------------------------ lane permutes (DPP)
// DPP controls: quad_perm [1,0,3,2] = 0xB1 (lane ^ 1), quad_perm [2,3,0,1] = 0x4E (lane ^ 2),
// row_half_mirror = 0x141 (lane i <-> 7-i within 8), row_mirror = 0x140 (i <-> 15-i within 16),
// row_shl:4 = 0x104 (lane i reads lane i+4 within its row of 16).
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}

// Raw v_min/v_max (and 3-operand forms): no NaN canonicalisation of the operands, which fminf /
// fmaxf would add in IEEE mode. Equal to fminf / fmaxf for operands that are numbers or quiet NaNs
// (every arithmetic result and every bit copy of one), the only operands these kernels pass.
// Inline asm is outside the compiler's hazard tracking: an operand must not be the direct result
// of a transcendental (v_exp/v_rcp/v_sqrt...), which a following VALU may read only after one
// wait state; callers with such operands use fminf / fmaxf.
__device__ __forceinline__ float vmin3(float a, float b, float c) {
    float d;
    asm("v_min3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    float d;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
    return d;
}
__device__ __forceinline__ float vmin(float a, float b) {
    float d;
    asm("v_min_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}
__device__ __forceinline__ float vmax(float a, float b) {
    float d;
    asm("v_max_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b));
    return d;
}

// min / max of v and its DPP-permuted copy (CTRL one of 0xB1, 0x4E, 0x141, 0x140 above) in one
// VALU instruction: v_min_f32_dpp / v_max_f32_dpp, the permute applied to src0. The leading
// s_nop 4 gives the wait states a DPP instruction requires after a VALU write of its VGPR operand
// (two) or of EXEC (five), which the compiler does not insert before inline asm; the nop idles
// only this wave, not the SIMD's VALU. Raw v_min / v_max semantics as for vmin / vmax.
#define DOPT_DPP_ASM(OP, CTRLTXT) \
    asm("s_nop 4\n\t" OP " %0, %1, %1 " CTRLTXT " row_mask:0xf bank_mask:0xf" : "=v"(d) : "v"(v))
template <int CTRL>
__device__ __forceinline__ float vmin_dpp(float v) {
    float d;
    if constexpr (CTRL == 0xB1) DOPT_DPP_ASM("v_min_f32_dpp", "quad_perm:[1,0,3,2]");
    else if constexpr (CTRL == 0x4E) DOPT_DPP_ASM("v_min_f32_dpp", "quad_perm:[2,3,0,1]");
    else if constexpr (CTRL == 0x141) DOPT_DPP_ASM("v_min_f32_dpp", "row_half_mirror");
    else {
        static_assert(CTRL == 0x140, "vmin_dpp: quad_perm 0xB1 / 0x4E, row_half_mirror or row_mirror");
        DOPT_DPP_ASM("v_min_f32_dpp", "row_mirror");
    }
    return d;
}
template <int CTRL>
__device__ __forceinline__ float vmax_dpp(float v) {
    float d;
    if constexpr (CTRL == 0xB1) DOPT_DPP_ASM("v_max_f32_dpp", "quad_perm:[1,0,3,2]");
    else if constexpr (CTRL == 0x4E) DOPT_DPP_ASM("v_max_f32_dpp", "quad_perm:[2,3,0,1]");
    else if constexpr (CTRL == 0x141) DOPT_DPP_ASM("v_max_f32_dpp", "row_half_mirror");
    else {
        static_assert(CTRL == 0x140, "vmax_dpp: quad_perm 0xB1 / 0x4E, row_half_mirror or row_mirror");
        DOPT_DPP_ASM("v_max_f32_dpp", "row_mirror");
    }
    return d;
}
#undef DOPT_DPP_ASM

// min/max with lane l ^ D (D = 16 or 32) on every lane: v_permlane16_swap / v_permlane32_swap
// of a register with itself leaves the pair {x[l & ~D], x[l | D]}, in that order on both lanes of
// the pair (measured on MI355X), one VALU op per exchange instead of an LDS permute; both lanes
// then compute the same min/max of the same ordered operands
template <int D>
__device__ __forceinline__ void swap_minmax(float& mn, float& mx) {
    static_assert(D == 16 || D == 32, "row swaps exchange 16 or 32 lanes");
    const uint32_t a = __float_as_uint(mn), b = __float_as_uint(mx);
    if constexpr (D == 16) {
        const auto sa = __builtin_amdgcn_permlane16_swap(a, a, false, false);
        const auto sb = __builtin_amdgcn_permlane16_swap(b, b, false, false);
        mn = vmin(__uint_as_float(sa[0]), __uint_as_float(sa[1]));
        mx = vmax(__uint_as_float(sb[0]), __uint_as_float(sb[1]));
    } else {
        const auto sa = __builtin_amdgcn_permlane32_swap(a, a, false, false);
        const auto sb = __builtin_amdgcn_permlane32_swap(b, b, false, false);
        mn = vmin(__uint_as_float(sa[0]), __uint_as_float(sa[1]));
        mx = vmax(__uint_as_float(sb[0]), __uint_as_float(sb[1]));
    }
}

// ------------------------------------------------------------------ 16-byte global access
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte load / store, optionally non-temporal (streamed data touched once: the nt bit keeps
// it from displacing reusable lines).
template <bool NT>
__device__ __forceinline__ uint4 ld16(const void* p) {
    u32x4_t v;
    if constexpr (NT)
        v = __builtin_nontemporal_load((const u32x4_t*)p);
    else
        v = *(const u32x4_t*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <bool NT>
__device__ __forceinline__ void st16(void* p, const uint4& d) {
    const u32x4_t v = {d.x, d.y, d.z, d.w};
    if constexpr (NT)
        __builtin_nontemporal_store(v, (u32x4_t*)p);
    else
        *(u32x4_t*)p = v;
}

// ------------------------------------------------------------------ element conversions
template <int DT>
__device__ __forceinline__ void widen16(const uint4& r, float* f) {
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
    if constexpr (DT == DT_F32) {
#pragma unroll
        for (int k = 0; k < 4; ++k) f[k] = __uint_as_float(w[k]);
    } else if constexpr (DT == DT_BF16) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f[2 * k] = __uint_as_float(w[k] << 16);
            f[2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            f[2 * k] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] & 0xffffu));
            f[2 * k + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[k] >> 16));
        }
    }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round-to-nearest-even fp32 pair -> packed bf16 pair (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    f32x2_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ uint16_t to_bf16(float v) { return (uint16_t)(pack_bf16x2(v, 0.0f) & 0xffffu); }

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// ------------------------------------------------------------------ activation math
// Fast fp32 transcendentals for the fused kernels (v_exp_f32 / v_rcp_f32 based; the reference's
// own are Triton's exp and libdevice tanh, so these are tolerance-level anyway).
//
// The quantizer's squash tanh(x / 0.5) * 0.5 = tanh(2x) / 2, within about 2 fp32 ulps of the
// exact value everywhere (the reference evaluates it with libdevice tanh):
//   |x| < 0.45:  x + x^3 Q(x^2), Q of degree 5: a weighted minimax fit of (tanh(2x)/2 - x)/x^3
//                over x^2 in [0, 0.2025] whose relative error is 1.6e-8; evaluated in fp32 the
//                branch is within 1.01 ulp, and tiny values keep their relative accuracy (exact
//                0 at 0, -0 at -0);
//   |x| >= 0.45: 1/2 - 1/(e^{4|x|} + 1) with the sign of x (v_exp_f32, v_rcp_f32). The result is
//                >= 0.358 there and the subtracted term <= 0.142, so nothing cancels: within 1.3
//                ulps with a correctly rounded exp, 1.7 with one ulp of exp error. +-inf gives
//                +-1/2 and NaN stays NaN.
// (a float64 emulation of both branches over 7 million arguments gave a 1.80 ulp maximum.)
__device__ __forceinline__ float squash_half_tanh2(float x) {
    const float a = fabsf(x);
    const float e = __builtin_amdgcn_exp2f(5.7707801635558535f * a);  // e^{4|x|} = 2^{4|x|/ln 2}
    const float r = __builtin_copysignf(0.5f - __builtin_amdgcn_rcpf(e + 1.0f), x);
    const float t = x * x;
    float q = __builtin_fmaf(t, 5.341052532196045f, -7.024715423583984f);
    q = __builtin_fmaf(q, t, 5.351459980010986f);
    q = __builtin_fmaf(q, t, -3.438175678253174f);
    q = __builtin_fmaf(q, t, 2.13285756111145f);
    q = __builtin_fmaf(q, t, -1.3333284854888916f);
    const float p = __builtin_fmaf(x * t, q, x);
    return a < 0.45f ? p : r;
}
__device__ __forceinline__ float fast_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}
// GELU (tanh form) value and derivative of act_triton kernels
// (AC/modules/activations/kernel_implementation.py:496-519): u = a (x + b x^3), t = tanh(u),
// y = x (1 + t) / 2, dy/dx = (1 + t)/2 + x (1 - t^2) a (1 + 3 b x^2) / 2. Evaluated through
// s = (1 + t)/2 = sigmoid(2u) and 1 - t^2 = 4 s (1 - s), the same function without the
// cancellation of 1 + t for x below about -4 (where an fp32 tanh is already -1):
// u = x (a + a b x^2), s = 1 / (1 + 2^(-2 log2(e) u)), dy/dx = s + x s (1 - s) (2a + 6ab x^2).
// The factor -2 log2(e) is folded into the polynomial's coefficients and x s (1 - s) = y - y s is
// one fma.
__device__ __forceinline__ void gelu_and_grad(float x, float& y, float& d) {
    const float a = 0.7978845608028654f, ab = 0.7978845608028654f * 0.044715f;
    const float k = -2.8853900817779268f;  // -2 log2(e)
    const float x2 = x * x;
    const float ku = x * __builtin_fmaf(k * ab, x2, k * a);
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(ku));
    y = x * s;
    const float c = __builtin_fmaf(6.0f * ab, x2, 2.0f * a);
    d = __builtin_fmaf(__builtin_fmaf(-y, s, y), c, s);
}
// SiLU value and derivative (kernel_implementation.py:225-229): s = sigmoid(x), y = x s,
// dy/dx = s + x s (1 - s)
__device__ __forceinline__ void silu_and_grad(float x, float& y, float& d) {
    const float s = fast_sigmoid(x);
    y = x * s;
    d = __builtin_fmaf(y, 1.0f - s, s);
}
// 2 tanh(x / 2) of BatchNorm's squash, as 4 sigmoid(x) - 2 (two transcendentals, two other
// instructions; absolute error ~2e-7)
__device__ __forceinline__ float two_tanh_half_fast(float x) {
    const float r = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
    return __builtin_fmaf(4.0f, r, -2.0f);
}
// tanh(2d) / 2 of a clamped activation derivative is sigmoid(4d) - 1/2 (absolute error ~1e-7);
// this returns sigmoid(4d), the caller subtracts 1/2 where it can do so once per group
__device__ __forceinline__ float sigmoid4_fast(float d) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-5.7707801635558535f * d));
}

// ------------------------------------------------------------------ exact division, fewer instructions
__device__ __forceinline__ bool wave_any(bool p) { return __builtin_amdgcn_ballot_w64(p) != 0; }

// step = rng / qmax for rng > 0 (finite or +inf) and qmax = 2^bits - 1, rounded as the IEEE fp32
// division rounds it: q0 = rng * c with c = RN(1/qmax), r = fma(-q0, qmax, rng) (exact),
// q1 = fma(r, c, q0). Checked on gfx950 against the correctly rounded division for every
// non-negative fp32 rng and qmax = 1, 3, 15, 255 (compile-time and run-time divisors): equal for
// all but rng = +inf, where r is NaN and q0 = +inf is the quotient. Five VALU instructions against
// about eleven for the division sequence. qmax = 1 gives c = 1, r = 0 and q1 = rng.
__device__ __forceinline__ float div_by_qmax_rt(float rng, float qmax, float c) {
    const float q0 = rng * c;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, qmax, rng), c, q0);
    return rng == __builtin_inff() ? q0 : q1;
}
template <int QMAX>
__device__ __forceinline__ float div_by_qmax(float rng) {
    if constexpr (QMAX == 1) return rng;
    else return div_by_qmax_rt(rng, (float)QMAX, 1.0f / (float)QMAX);
}

// 1 / x for x > 0, rounded as the IEEE fp32 division rounds it: v_rcp_f32 and one fma Newton step,
// y = fma(fma(-x, y0, 1), y0, y0), which on gfx950 equals the correctly rounded reciprocal for
// every normal x in [2^-126, 2^126) (checked for each of them). A wave holding any x outside that
// range (subnormal, huge, +inf) takes the division for all its lanes.
__device__ __forceinline__ float exact_rcp(float x) {
    if (!wave_any(!(x >= 0x1p-126f && x < 0x1p126f))) {
        const float y0 = __builtin_amdgcn_rcpf(x);
        return __builtin_fmaf(__builtin_fmaf(-x, y0, 1.0f), y0, y0);
    }
    return 1.0f / x;
}

// ------------------------------------------------------------------ Philox4x32-10
// Salmon et al., SC'11: multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
// 0x9E3779B9 / 0xBB67AE85, key bumped between rounds. Each round is two 32x32->64 multiplies
// (v_mad_u64_u32) and two 3-input XORs (v_bitop3_b32 with truth table 0x96 = a ^ b ^ c).
__device__ __forceinline__ uint32_t xor3(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0x96);
}

__device__ __forceinline__ uint4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                               uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = xor3((uint32_t)(p1 >> 32), c1, k0);
        const uint32_t n2 = xor3((uint32_t)(p0 >> 32), c3, k1);
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
    }
    return make_uint4(c0, c1, c2, c3);
}

// Byte k (0..3) of a Philox output word -> u = (b + 0.5) / 256 in (0, 1). The fma is exact
// (b * 2^-8 + 2^-9 has at most 9 significant bits), so it equals the separately rounded form.
__device__ __forceinline__ float philox_byte_to_u(uint32_t w, int k) {
    const float b = (float)((w >> (8 * k)) & 0xffu);  // v_cvt_f32_ubyte<k>
    return __builtin_fmaf(b, 1.0f / 256.0f, 1.0f / 512.0f);
}

// Triton's uint_to_uniform_float (triton/language/random.py) of a Philox output word: the word as
// int32, folded to non-negative (~i for i < 0), times fp32(4.6566127342e-10) = 0x2fffffff.
__device__ __forceinline__ float triton_uniform(uint32_t w) {
    int32_t i = (int32_t)w;
    if (i < 0) i = ~i;
    return (float)i * __uint_as_float(0x2fffffffu);
}

// Triton's tl.rand(seed, offset) for a 32-bit offset: the first word of Philox4x32-10 with counter
// (offset, 0, 0, 0) and key (lo32, hi32 of seed), as a uniform in [0, 1).
__device__ __forceinline__ float triton_rand(uint64_t seed, uint32_t offset) {
    return triton_uniform(philox4x32_10(offset, 0u, 0u, 0u, (uint32_t)seed, (uint32_t)(seed >> 32)).x);
}

}  // namespace dopt
