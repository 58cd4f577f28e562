// Fused activation kernels of the compressed activation layers (AC/modules/activations/):
//
//   relu_pack_kernel      y = relu(x) (or relu6's band), and the mask (x > 0, or 0 < x < 6) packed
//                         as BITS-bit codes in the little-endian bitstream of the quantizer
//                         (kernel_implementation.py:34-90)
//   relu_unpack_kernel    dx = bf16(dy * mask) from that bitstream (kernel_implementation.py:93-143)
//   act_forward_kernel    the unfused helpers: relu/relu6 -> (y, int8 mask); gelu/silu -> (bf16 y,
//                         bf16 derivative) (kernel_implementation.py:9-31, :154-175, :437-466)
//   pact_clamp_*_kernel   the PACT clamp of AC/modules/ops.py:545-585 and its masked gradient
//
// All are flat elementwise passes over n elements: lane l of a wave owns 8 consecutive
// elements (one 16-byte vector of bf16, two of fp32) per pass, the wave's lanes consecutive
// chunks, so the mask bits of consecutive lanes are consecutive in the bitstream; pieces narrower
// than a dword are merged across lanes with DPP and written by the first lane of each dword.
#include "dopt_device.h"

namespace dopt {

enum { ACT_RELU = 0, ACT_RELU6 = 1, ACT_GELU = 2, ACT_SILU = 3 };

namespace {

constexpr int CE = 8;  // elements per lane chunk

template <int DT>
__device__ __forceinline__ void load8(const void* base, uint64_t e0, float* v) {
    const char* p = (const char*)base + e0 * DType<DT>::bytes;
    if constexpr (DT == DT_F32) {
        widen16<DT>(ld16<false>(p), v);
        widen16<DT>(ld16<false>(p + 16), v + 4);
    } else {
        widen16<DT>(ld16<false>(p), v);
    }
}

// stores 8 floats in the element type DT (bf16 rounding RNE; f32 verbatim). The outputs of these
// kernels are written once and read by another kernel later, so they are streamed (non-temporal):
// measured on bf16 [256,256,56,56] at 1 bit, the ReLU forward 138 -> 133 us, its backward 139 -> 132.5 us
template <int DT>
__device__ __forceinline__ void store8(void* base, uint64_t e0, const float* v) {
    char* p = (char*)base + e0 * DType<DT>::bytes;
    if constexpr (DT == DT_F32) {
        st16<true>(p, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                 __float_as_uint(v[3])));
        st16<true>(p + 16, make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]),
                                      __float_as_uint(v[7])));
    } else if constexpr (DT == DT_BF16) {
        st16<true>(p, make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                                 pack_bf16x2(v[6], v[7])));
    } else {
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * k]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v[2 * k + 1]) << 16);
        st16<true>(p, make_uint4(w[0], w[1], w[2], w[3]));
    }
}

// y = x where the mask holds, else +0, in x's own type: the input bits pass through unchanged
template <int DT>
__device__ __forceinline__ void store8_masked(void* base, uint64_t e0, const void* xbase, uint32_t mbits) {
    const char* src = (const char*)xbase + e0 * DType<DT>::bytes;
    char* dst = (char*)base + e0 * DType<DT>::bytes;
    if constexpr (DT == DT_F32) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint4 r = ld16<false>(src + 16 * h);
            const uint32_t m = mbits >> (4 * h);
            r.x = (m & 1u) ? r.x : 0u;
            r.y = (m & 2u) ? r.y : 0u;
            r.z = (m & 4u) ? r.z : 0u;
            r.w = (m & 8u) ? r.w : 0u;
            st16<true>(dst + 16 * h, r);
        }
    } else {
        uint4 r = ld16<false>(src);
        uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = (mbits >> (2 * k)) & 1u, hi = (mbits >> (2 * k + 1)) & 1u;
            w[k] &= (lo ? 0x0000ffffu : 0u) | (hi ? 0xffff0000u : 0u);
        }
        st16<true>(dst, make_uint4(w[0], w[1], w[2], w[3]));
    }
}

template <int DT, int BITS, bool RELU6>
__global__ __launch_bounds__(256) void relu_pack_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                        uint32_t* __restrict__ packed, uint64_t n) {
    constexpr int UBITS = CE * BITS;  // code bits per chunk
    const int lane = threadIdx.x & 63;
    const uint64_t c = (linear_block() * 4 + (threadIdx.x >> 6)) * 64 + lane;  // chunk index
    const uint64_t e0 = c * CE;
    const bool ok = e0 < n;
    uint32_t mbits = 0;  // one bit per element
    if (ok) {
        float v[CE];
        load8<DT>(x, e0, v);
#pragma unroll
        for (int k = 0; k < CE; ++k) {
            const bool m = RELU6 ? (v[k] > 0.0f && v[k] < 6.0f) : (v[k] > 0.0f);
            mbits |= (uint32_t)m << k;
        }
        if constexpr (DT == DT_BF16) {
            store8_masked<DT>(y, e0, x, mbits);
        } else {
            // the reference stores x.to(bfloat16) into y of x's type (kernel_implementation.py:90):
            // fp32 inputs come out rounded to bf16
            float o[CE];
#pragma unroll
            for (int k = 0; k < CE; ++k) o[k] = ((mbits >> k) & 1u) ? bf16_bits_to_f32(to_bf16(v[k])) : 0.0f;
            store8<DT>(y, e0, o);
        }
    }
    // spread the mask bits to BITS-bit codes (value 0 or 1 per code)
    uint32_t d[UBITS >= 32 ? UBITS / 32 : 1];
#pragma unroll
    for (int j = 0; j < (UBITS >= 32 ? UBITS / 32 : 1); ++j) {
        constexpr int PER = UBITS >= 32 ? 32 / BITS : CE;
        uint32_t acc = 0;
#pragma unroll
        for (int k = 0; k < PER; ++k) acc |= ((mbits >> (j * PER + k)) & 1u) << (k * BITS);
        d[j] = acc;
    }
    const uint64_t n_words = n * BITS / 32;
    if constexpr (UBITS >= 32) {
        constexpr int ND = UBITS / 32;
        if (ok) {
            if constexpr (ND == 1) packed[c] = d[0];
            else *(uint2*)(packed + 2 * c) = make_uint2(d[0], d[1]);
        }
    } else {
        uint32_t m = d[0];
        m |= dpp_u32<0xB1>(m) << UBITS;
        if constexpr (UBITS * 2 < 32) m |= dpp_u32<0x4E>(m) << (2 * UBITS);
        constexpr int LPD = 32 / UBITS;
        const uint64_t w = c / LPD;
        if ((lane % LPD) == 0 && w < n_words) packed[w] = m;
    }
}

template <int DYT, int BITS>
__global__ __launch_bounds__(256) void relu_unpack_kernel(const uint32_t* __restrict__ packed, const void* __restrict__ dy,
                                                          void* __restrict__ dx, uint64_t n) {
    constexpr int UBITS = CE * BITS;
    const uint64_t c = (linear_block() * 4 + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    const uint64_t e0 = c * CE;
    if (e0 >= n) return;
    uint32_t cw[UBITS > 32 ? 2 : 1];
    if constexpr (UBITS > 32) {
        const uint2 d = *(const uint2*)(packed + 2 * c);
        cw[0] = d.x;
        cw[1] = d.y;
    } else {
        const uint32_t d = packed[(c * UBITS) / 32];
        cw[0] = d >> ((c * UBITS) % 32);
    }
    float g[CE], o[CE];
    load8<DYT>(dy, e0, g);
#pragma unroll
    for (int k = 0; k < CE; ++k) {
        const uint32_t m = (cw[(k * BITS) / 32] >> ((k * BITS) % 32)) & 1u;
        o[k] = g[k] * (float)m;  // dy * mask in fp32, as the reference (kernel_implementation.py:132-134)
    }
    store8<DT_BF16>(dx, e0, o);
}

// unfused helpers: relu/relu6 -> y (x's type) + int8 mask; gelu/silu -> bf16 y + bf16 derivative
template <int DT>
__device__ __forceinline__ float load1(const void* base, uint64_t e) {
    if constexpr (DT == DT_F32) return ((const float*)base)[e];
    else if constexpr (DT == DT_BF16) return bf16_bits_to_f32(((const uint16_t*)base)[e]);
    else return (float)__builtin_bit_cast(_Float16, ((const uint16_t*)base)[e]);
}

template <int DT, int ACT>
__global__ __launch_bounds__(256) void act_forward_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                          void* __restrict__ aux, uint64_t n) {
    const uint64_t c = (linear_block() * 4 + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    const uint64_t e0 = c * CE;
    if (e0 >= n) return;
    if (e0 + CE > n) {
        // ragged tail: one element at a time
        for (uint64_t e = e0; e < n; ++e) {
            const float v = load1<DT>(x, e);
            if constexpr (ACT == ACT_RELU || ACT == ACT_RELU6) {
                const bool m = ACT == ACT_RELU6 ? (v > 0.0f && v < 6.0f) : (v > 0.0f);
                if constexpr (DT == DT_F32)
                    ((float*)y)[e] = m ? v : 0.0f;
                else
                    ((uint16_t*)y)[e] = m ? ((const uint16_t*)x)[e] : (uint16_t)0;
                ((int8_t*)aux)[e] = (int8_t)m;
            } else {
                float yv, dv;
                if constexpr (ACT == ACT_GELU)
                    gelu_and_grad(v, yv, dv);
                else
                    silu_and_grad(v, yv, dv);
                ((uint16_t*)y)[e] = to_bf16(yv);
                ((uint16_t*)aux)[e] = to_bf16(dv);
            }
        }
        return;
    }
    float v[CE];
    load8<DT>(x, e0, v);
    if constexpr (ACT == ACT_RELU || ACT == ACT_RELU6) {
        uint32_t mbits = 0;
        uint64_t bytes = 0;
#pragma unroll
        for (int k = 0; k < CE; ++k) {
            const bool m = ACT == ACT_RELU6 ? (v[k] > 0.0f && v[k] < 6.0f) : (v[k] > 0.0f);
            mbits |= (uint32_t)m << k;
            bytes |= (uint64_t)m << (8 * k);
        }
        store8_masked<DT>(y, e0, x, mbits);
        *(uint64_t*)((char*)aux + e0) = bytes;
    } else {
        float yv[CE], dv[CE];
#pragma unroll
        for (int k = 0; k < CE; ++k) {
            if constexpr (ACT == ACT_GELU)
                gelu_and_grad(v[k], yv[k], dv[k]);
            else
                silu_and_grad(v[k], yv[k], dv[k]);
        }
        store8<DT_BF16>(y, e0, yv);
        store8<DT_BF16>(aux, e0, dv);
    }
}

// PACT clamp (AC/modules/ops.py:545-585): y = bf16(clamp(x, -alpha, alpha)) and the int8 mask
// |x| <= alpha; backward dx = bf16(mask != 0 ? dy : 0). The clamp is fmaxf then fminf, so a NaN x
// gives -alpha (and mask 0).
template <int DT>
__global__ __launch_bounds__(256) void pact_clamp_fwd_kernel(const void* __restrict__ x, float alpha,
                                                             void* __restrict__ y, int8_t* __restrict__ mask,
                                                             uint64_t n) {
    const uint64_t c = (linear_block() * 4 + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    const uint64_t e0 = c * CE;
    if (e0 >= n) return;
    if (e0 + CE > n) {  // ragged tail: one element at a time
        for (uint64_t e = e0; e < n; ++e) {
            const float v = load1<DT>(x, e);
            ((uint16_t*)y)[e] = to_bf16(fminf(fmaxf(v, -alpha), alpha));
            mask[e] = (int8_t)(fabsf(v) <= alpha);
        }
        return;
    }
    float v[CE], o[CE];
    load8<DT>(x, e0, v);
    uint64_t bytes = 0;
#pragma unroll
    for (int k = 0; k < CE; ++k) {
        o[k] = fminf(fmaxf(v[k], -alpha), alpha);
        bytes |= (uint64_t)(fabsf(v[k]) <= alpha) << (8 * k);
    }
    store8<DT_BF16>(y, e0, o);
    *(uint64_t*)(mask + e0) = bytes;
}

template <int DYT>
__global__ __launch_bounds__(256) void pact_clamp_bwd_kernel(const int8_t* __restrict__ mask, const void* __restrict__ dy,
                                                             void* __restrict__ dx, uint64_t n) {
    const uint64_t c = (linear_block() * 4 + (threadIdx.x >> 6)) * 64 + (threadIdx.x & 63);
    const uint64_t e0 = c * CE;
    if (e0 >= n) return;
    if (e0 + CE > n) {
        for (uint64_t e = e0; e < n; ++e) ((uint16_t*)dx)[e] = to_bf16(mask[e] != 0 ? load1<DYT>(dy, e) : 0.0f);
        return;
    }
    float g[CE], o[CE];
    load8<DYT>(dy, e0, g);
    const uint64_t mb = *(const uint64_t*)(mask + e0);
#pragma unroll
    for (int k = 0; k < CE; ++k) o[k] = ((mb >> (8 * k)) & 0xffu) != 0 ? g[k] : 0.0f;
    store8<DT_BF16>(dx, e0, o);
}

template <class K, class... Args>
int launch_flat(K kernel, uint64_t n, hipStream_t s, Args... args) {
    const uint64_t chunks = (n + CE - 1) / CE;
    const uint64_t blocks = (chunks + 255) / 256;
    if (blocks == 0) return 0;
    hipLaunchKernelGGL(kernel, linear_grid(blocks, 256), dim3(256), 0, s, args..., n);
    return 0;
}

template <int DT, int BITS>
int relu_pack_bits(const void* x, void* y, uint32_t* packed, uint64_t n, bool relu6, hipStream_t s) {
    return relu6 ? launch_flat(relu_pack_kernel<DT, BITS, true>, n, s, x, y, packed)
                 : launch_flat(relu_pack_kernel<DT, BITS, false>, n, s, x, y, packed);
}

template <int DT>
int relu_pack_dt(const void* x, void* y, uint32_t* packed, uint64_t n, int bits, bool relu6, hipStream_t s) {
    switch (bits) {
        case 1: return relu_pack_bits<DT, 1>(x, y, packed, n, relu6, s);
        case 2: return relu_pack_bits<DT, 2>(x, y, packed, n, relu6, s);
        case 4: return relu_pack_bits<DT, 4>(x, y, packed, n, relu6, s);
        case 8: return relu_pack_bits<DT, 8>(x, y, packed, n, relu6, s);
    }
    return -1;
}

template <int DYT>
int relu_unpack_dt(const uint32_t* packed, const void* dy, void* dx, uint64_t n, int bits, hipStream_t s) {
    switch (bits) {
        case 1: return launch_flat(relu_unpack_kernel<DYT, 1>, n, s, packed, dy, dx);
        case 2: return launch_flat(relu_unpack_kernel<DYT, 2>, n, s, packed, dy, dx);
        case 4: return launch_flat(relu_unpack_kernel<DYT, 4>, n, s, packed, dy, dx);
        case 8: return launch_flat(relu_unpack_kernel<DYT, 8>, n, s, packed, dy, dx);
    }
    return -1;
}

template <int DT>
int act_forward_dt(const void* x, void* y, void* aux, uint64_t n, int act, hipStream_t s) {
    switch (act) {
        case ACT_RELU: return launch_flat(act_forward_kernel<DT, ACT_RELU>, n, s, x, y, aux);
        case ACT_RELU6: return launch_flat(act_forward_kernel<DT, ACT_RELU6>, n, s, x, y, aux);
        case ACT_GELU: return launch_flat(act_forward_kernel<DT, ACT_GELU>, n, s, x, y, aux);
        case ACT_SILU: return launch_flat(act_forward_kernel<DT, ACT_SILU>, n, s, x, y, aux);
    }
    return -1;
}

}  // namespace

int launch_relu_pack(const void* x, int dt, void* y, uint32_t* packed, uint64_t n, int bits, bool relu6, hipStream_t s) {
    switch (dt) {
        case DT_F32: return relu_pack_dt<DT_F32>(x, y, packed, n, bits, relu6, s);
        case DT_BF16: return relu_pack_dt<DT_BF16>(x, y, packed, n, bits, relu6, s);
    }
    return -1;
}

int launch_relu_unpack(const uint32_t* packed, const void* dy, int dyt, void* dx, uint64_t n, int bits, hipStream_t s) {
    switch (dyt) {
        case DT_F32: return relu_unpack_dt<DT_F32>(packed, dy, dx, n, bits, s);
        case DT_F16: return relu_unpack_dt<DT_F16>(packed, dy, dx, n, bits, s);
        case DT_BF16: return relu_unpack_dt<DT_BF16>(packed, dy, dx, n, bits, s);
    }
    return -1;
}

int launch_act_forward(const void* x, int dt, void* y, void* aux, uint64_t n, int act, hipStream_t s) {
    switch (dt) {
        case DT_F32: return act_forward_dt<DT_F32>(x, y, aux, n, act, s);
        case DT_F16: return act_forward_dt<DT_F16>(x, y, aux, n, act, s);
        case DT_BF16: return act_forward_dt<DT_BF16>(x, y, aux, n, act, s);
    }
    return -1;
}

int launch_pact_clamp_fwd(const void* x, int dt, float alpha, void* y, int8_t* mask, uint64_t n, hipStream_t s) {
    switch (dt) {
        case DT_F32: return launch_flat(pact_clamp_fwd_kernel<DT_F32>, n, s, x, alpha, y, mask);
        case DT_F16: return launch_flat(pact_clamp_fwd_kernel<DT_F16>, n, s, x, alpha, y, mask);
        case DT_BF16: return launch_flat(pact_clamp_fwd_kernel<DT_BF16>, n, s, x, alpha, y, mask);
    }
    return -1;
}

int launch_pact_clamp_bwd(const int8_t* mask, const void* dy, int dyt, void* dx, uint64_t n, hipStream_t s) {
    switch (dyt) {
        case DT_F32: return launch_flat(pact_clamp_bwd_kernel<DT_F32>, n, s, mask, dy, dx);
        case DT_F16: return launch_flat(pact_clamp_bwd_kernel<DT_F16>, n, s, mask, dy, dx);
        case DT_BF16: return launch_flat(pact_clamp_bwd_kernel<DT_BF16>, n, s, mask, dy, dx);
    }
    return -1;
}

}  // namespace dopt
