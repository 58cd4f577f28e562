// The reference quantizer's avg_alam mode on gfx950 (Activation_Compression/act_triton_kernel.py:
// 336-395 host side; :116-118 quantize, :212-219 dequantize; seed 42 in both operators).
//
// Quantize, one wave per group: the reference pre-transform ([clamp], tanh squash), min/max,
// step = rng/QMAX (1 for an empty range), the nearest-code argument qf = fma(x - min, 1/step,
// 0.5 - 1e-6) of every element, then the mean of every run of A = alam_bits consecutive qf
// (summed left to right, as a thread of the reference's Triton kernel holds such a run), truncated
// and clamped to [0, QMAX]: g/A codes in NW/A words, bf16 scale and min.
//
// Dequantize, one lane per element: code c = e / A, plus Triton's randn(seed + group, e) - 0.5,
// y = bf16(fma(code + noise, scale, min)). randn is Philox4x32-10 with counter (e, 0, 0, 0) and key
// (lo32, hi32 of seed + group); its first two words become uniforms (int32 folded to
// non-negative, times fp32(4.6566127342e-10)) and Box-Muller's first output
// sqrt(-2 log max(u1, 1e-7)) cos(2 pi u2).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dequant_unpack.h"
#include "dopt_device.h"

namespace dopt {
namespace {

constexpr int ALAM_WAVES = 4;  // groups per workgroup, one wave each
constexpr int ALAM_GMAX = 1024;

template <int DT>
__device__ __forceinline__ float load_one(const void* x, int64_t i) {
    if constexpr (DT == DT_F32) return ((const float*)x)[i];
    else if constexpr (DT == DT_BF16) return bf16_bits_to_f32(((const uint16_t*)x)[i]);
    else return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)x)[i]);
}

__device__ __forceinline__ float wave_min(float v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v = fminf(v, __shfl_xor(v, d, 64));
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}

struct AlamArgs {
    const void* x;
    uint32_t* packed;
    uint16_t* scale;
    uint16_t* minv;
    int64_t n_groups;
    int g, bits, alam, flags;
    float clamp_alpha;
};

template <int DT>
__global__ __launch_bounds__(64 * ALAM_WAVES) void alam_quant_pack_kernel(AlamArgs a) {
    __shared__ float qs[ALAM_WAVES][ALAM_GMAX];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // a wave past the last group redoes the last one and stores nothing, so every wave reaches
    // the barrier (n_groups >= 1: the launcher skips empty calls)
    const int64_t r0 = (int64_t)linear_block() * ALAM_WAVES + wave;
    const bool active = r0 < a.n_groups;
    const int64_t r = active ? r0 : a.n_groups - 1;
    const int g = a.g, per = g / 64;
    const float qmaxf = (float)((1 << a.bits) - 1);
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    // element e = lane + 64 j: consecutive lanes read consecutive elements
    float v[ALAM_GMAX / 64];
#pragma unroll
    for (int j = 0; j < ALAM_GMAX / 64; ++j) {
        if (j >= per) break;
        float t = load_one<DT>(a.x, r * g + lane + 64 * j);
        if (a.flags & 1) t = fminf(fmaxf(t, -a.clamp_alpha), a.clamp_alpha);  // FL_CLAMP, NaN -> -alpha
        if (a.flags & 2) t = squash_half_tanh2(t);                             // FL_SQUASH
        v[j] = t;
        mn = fminf(mn, t);
        mx = fmaxf(mx, t);
    }
    mn = wave_min(mn) + 0.0f;
    mx = wave_max(mx);
    const float rng = mx - mn;
    const float step = rng > 0.0f ? rng / qmaxf : 1.0f;
    const float inv = 1.0f / step;
    const float half_m = 0.49999899f;  // fp32(0.5 - 1e-6)
#pragma unroll
    for (int j = 0; j < ALAM_GMAX / 64; ++j) {
        if (j >= per) break;
        qs[wave][lane + 64 * j] = __builtin_fmaf(v[j] - mn, inv, half_m);
    }
    __syncthreads();
    // word w holds codes w*VPW .. w*VPW + VPW-1, code c the mean of qf[cA .. cA + A-1]
    const int A = a.alam, bits = a.bits, vpw = 32 / bits;
    const int nw = g / vpw / A;
    const float inv_a = 1.0f / (float)A;  // A is a power of two: the division is this product
    for (int w = lane; w < nw; w += 64) {
        uint32_t word = 0;
        for (int j = 0; j < vpw; ++j) {
            const int c = w * vpw + j;
            float s = qs[wave][c * A];
            for (int k = 1; k < A; ++k) s = s + qs[wave][c * A + k];
            float q = s * inv_a;
            q = __builtin_amdgcn_fmed3f(q, 0.0f, qmaxf);  // NaN -> 0 (med3 of NaN, 0, QMAX is 0)
            word |= (uint32_t)q << (j * bits);
        }
        if (active) a.packed[r * nw + w] = word;
    }
    if (active && lane == 0) {
        a.scale[r] = to_bf16(step);
        a.minv[r] = to_bf16(mn);
    }
}

struct AlamDqArgs {
    const uint32_t* packed;
    const uint16_t* scale;
    const uint16_t* minv;
    uint16_t* y;
    int64_t total;  // n_groups * g
    int g, bits, alam;
    uint64_t seed;
};

__global__ __launch_bounds__(256) void alam_dequant_kernel(AlamDqArgs a) {
    const int64_t i = (int64_t)linear_block() * 256 + threadIdx.x;
    if (i >= a.total) return;
    const int64_t r = i / a.g;
    const int e = (int)(i - r * a.g);
    const int vpw = 32 / a.bits, c = e / a.alam, nw = a.g / vpw / a.alam;
    const uint32_t q = (a.packed[r * nw + c / vpw] >> ((c % vpw) * a.bits)) & ((1u << a.bits) - 1u);
    const uint64_t key = a.seed + (uint64_t)r;
    const uint4 w = philox4x32_10((uint32_t)e, 0u, 0u, 0u, (uint32_t)key, (uint32_t)(key >> 32));
    const float u1 = fmaxf(1.0e-7f, triton_uniform(w.x)), u2 = triton_uniform(w.y);
    const float th = 6.283185307179586f * u2;
    const float n = sqrtf(-2.0f * logf(u1)) * cosf(th);
    const float qf = (float)q + (n - 0.5f);
    a.y[i] = to_bf16(__builtin_fmaf(qf, bf16_bits_to_f32(a.scale[r]), bf16_bits_to_f32(a.minv[r])));
}

// The SiLU backward with avg_alam at alam_bits = 1 (activations/kernel_implementation.py:376-400,
// kernel_registration.py:201-237): the plain codes plus Triton's tl.rand(seed + group, e) - 0.5,
// dx = bf16(dy * fma(code + noise, scale, min)); one lane per element, the group's element e at
// the flat or spatial-tile position of the plain operators. The mode has no other user, so the
// kernel is plain: Philox per element costs ~60 instructions.
struct AlamDyArgs {
    DequantArgs d;
    int g, bits, dy_f32;
    uint64_t seed;
    int64_t total;
};

__device__ __forceinline__ uint64_t alam_elem_index(const DequantArgs& a, uint32_t r, uint32_t e, int g) {
    if (!a.tiled) return (uint64_t)r * (uint32_t)g + e;
    const uint32_t band = r / a.tiles_w;
    const uint32_t tw = r - band * a.tiles_w;
    const uint32_t smask = (1u << a.log2s) - 1u;
    return (((uint64_t)band * a.row) << a.log2s) + ((uint64_t)tw << a.log2s) + (uint64_t)(e >> a.log2s) * a.row +
           (e & smask);
}

__global__ __launch_bounds__(256) void alam_act_dequant_mul_kernel(AlamDyArgs a) {
    const int64_t i = (int64_t)linear_block() * 256 + threadIdx.x;
    if (i >= a.total) return;
    const uint32_t r = (uint32_t)(i / a.g), e = (uint32_t)(i - (int64_t)r * a.g);
    const int vpw = 32 / a.bits, nw = a.g / vpw;
    const uint32_t q =
        (a.d.packed[(int64_t)r * nw + e / vpw] >> ((e % vpw) * a.bits)) & ((1u << a.bits) - 1u);
    float sc, mn;
    if (a.d.meta_bf16) {
        sc = bf16_bits_to_f32(((const uint16_t*)a.d.scale)[r]);
        mn = bf16_bits_to_f32(((const uint16_t*)a.d.minv)[r]);
    } else {
        sc = ((const float*)a.d.scale)[r];
        mn = ((const float*)a.d.minv)[r];
    }
    const float act = __builtin_fmaf((float)q + (triton_rand(a.seed + r, e) - 0.5f), sc, mn);
    const uint64_t o = alam_elem_index(a.d, r, e, a.g);
    const float dy = a.dy_f32 ? ((const float*)a.d.dy)[o] : bf16_bits_to_f32(((const uint16_t*)a.d.dy)[o]);
    ((uint16_t*)a.d.y)[o] = to_bf16(dy * act);
}

}  // namespace

int launch_alam_act_dequant_mul(const DequantArgs& d, int g, int bits, int dy_f32, uint64_t seed, hipStream_t s) {
    const AlamDyArgs a{d, g, bits, dy_f32, seed, (int64_t)d.n_groups * g};
    hipLaunchKernelGGL(alam_act_dequant_mul_kernel, linear_grid((uint64_t)(a.total + 255) / 256, 256), dim3(256), 0, s, a);
    return 0;
}

int launch_alam_quant_pack(const void* x, int dt, int64_t n_groups, int g, int bits, int alam, int flags,
                           float clamp_alpha, uint32_t* packed, uint16_t* scale, uint16_t* minv, hipStream_t s) {
    const AlamArgs a{x, packed, scale, minv, n_groups, g, bits, alam, flags, clamp_alpha};
    const dim3 grid = linear_grid((uint64_t)(n_groups + ALAM_WAVES - 1) / ALAM_WAVES, 64 * ALAM_WAVES);
    if (dt == DT_F32) hipLaunchKernelGGL(alam_quant_pack_kernel<DT_F32>, grid, dim3(64 * ALAM_WAVES), 0, s, a);
    else if (dt == DT_F16) hipLaunchKernelGGL(alam_quant_pack_kernel<DT_F16>, grid, dim3(64 * ALAM_WAVES), 0, s, a);
    else hipLaunchKernelGGL(alam_quant_pack_kernel<DT_BF16>, grid, dim3(64 * ALAM_WAVES), 0, s, a);
    return 0;
}

int launch_alam_dequant(const uint32_t* packed, const uint16_t* scale, const uint16_t* minv, int64_t n_groups,
                        int g, int bits, int alam, uint64_t seed, uint16_t* y, hipStream_t s) {
    const AlamDqArgs a{packed, scale, minv, y, n_groups * g, g, bits, alam, seed};
    const dim3 grid = linear_grid((uint64_t)(a.total + 255) / 256, 256);
    hipLaunchKernelGGL(alam_dequant_kernel, grid, dim3(256), 0, s, a);
    return 0;
}

}  // namespace dopt
