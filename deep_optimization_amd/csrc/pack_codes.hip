// Code-only pack / unpack (the pack_only path used for 1-bit masks).
// pack:   word = sum_j int32(int8 code[j]) << (j*BITS), 32-bit wrap-around
//         (Activation_Compression/act_triton_kernel.py:266-271);
// unpack: code = (word >> (j*BITS)) & (2^BITS - 1) as int8 (act_triton_kernel.py:304-322).
// One lane per 32-bit word; its VPW = 32/BITS codes are one 4/8/16/32-byte vector access.
#include "dopt_device.h"

namespace dopt {

template <int BITS>
__global__ __launch_bounds__(256) void pack_codes_kernel(const int8_t* __restrict__ codes, uint32_t* __restrict__ out,
                                                         uint64_t n_words) {
    constexpr int VPW = 32 / BITS;
    const uint64_t w = linear_block() * 256 + threadIdx.x;
    if (w >= n_words) return;
    uint32_t b[8];
    const int8_t* src = codes + w * VPW;
    if constexpr (VPW == 32) {
        const uint4 u0 = ((const uint4*)src)[0], u1 = ((const uint4*)src)[1];
        b[0] = u0.x; b[1] = u0.y; b[2] = u0.z; b[3] = u0.w;
        b[4] = u1.x; b[5] = u1.y; b[6] = u1.z; b[7] = u1.w;
    } else if constexpr (VPW == 16) {
        const uint4 u0 = *(const uint4*)src;
        b[0] = u0.x; b[1] = u0.y; b[2] = u0.z; b[3] = u0.w;
    } else if constexpr (VPW == 8) {
        const uint2 u0 = *(const uint2*)src;
        b[0] = u0.x; b[1] = u0.y;
    } else {
        b[0] = *(const uint32_t*)src;
    }
    uint32_t acc = 0;
#pragma unroll
    for (int j = 0; j < VPW; ++j) {
        const int32_t code = (int32_t)(int8_t)((b[j >> 2] >> ((j & 3) * 8)) & 0xffu);
        acc += (uint32_t)code << (j * BITS);
    }
    out[w] = acc;
}

template <int BITS>
__global__ __launch_bounds__(256) void unpack_codes_kernel(const uint32_t* __restrict__ packed, int8_t* __restrict__ codes,
                                                           uint64_t n_words) {
    constexpr int VPW = 32 / BITS;
    constexpr uint32_t QMAX = (1u << BITS) - 1u;
    const uint64_t w = linear_block() * 256 + threadIdx.x;
    if (w >= n_words) return;
    const uint32_t word = packed[w];
    uint32_t b[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < VPW; ++j) b[j >> 2] |= ((word >> (j * BITS)) & QMAX) << ((j & 3) * 8);
    int8_t* dst = codes + w * VPW;
    if constexpr (VPW == 32) {
        ((uint4*)dst)[0] = make_uint4(b[0], b[1], b[2], b[3]);
        ((uint4*)dst)[1] = make_uint4(b[4], b[5], b[6], b[7]);
    } else if constexpr (VPW == 16) {
        *(uint4*)dst = make_uint4(b[0], b[1], b[2], b[3]);
    } else if constexpr (VPW == 8) {
        *(uint2*)dst = make_uint2(b[0], b[1]);
    } else {
        *(uint32_t*)dst = b[0];
    }
}

int launch_pack_codes(const int8_t* codes, uint32_t* out, uint64_t n_words, int bits, hipStream_t s) {
    const uint64_t blocks = (n_words + 255) / 256;
    if (blocks == 0) return 0;
    switch (bits) {
        case 1: hipLaunchKernelGGL(pack_codes_kernel<1>, linear_grid(blocks, 256), dim3(256), 0, s, codes, out, n_words); return 0;
        case 2: hipLaunchKernelGGL(pack_codes_kernel<2>, linear_grid(blocks, 256), dim3(256), 0, s, codes, out, n_words); return 0;
        case 4: hipLaunchKernelGGL(pack_codes_kernel<4>, linear_grid(blocks, 256), dim3(256), 0, s, codes, out, n_words); return 0;
        case 8: hipLaunchKernelGGL(pack_codes_kernel<8>, linear_grid(blocks, 256), dim3(256), 0, s, codes, out, n_words); return 0;
    }
    return -1;
}

int launch_unpack_codes(const uint32_t* packed, int8_t* codes, uint64_t n_words, int bits, hipStream_t s) {
    const uint64_t blocks = (n_words + 255) / 256;
    if (blocks == 0) return 0;
    switch (bits) {
        case 1: hipLaunchKernelGGL(unpack_codes_kernel<1>, linear_grid(blocks, 256), dim3(256), 0, s, packed, codes, n_words); return 0;
        case 2: hipLaunchKernelGGL(unpack_codes_kernel<2>, linear_grid(blocks, 256), dim3(256), 0, s, packed, codes, n_words); return 0;
        case 4: hipLaunchKernelGGL(unpack_codes_kernel<4>, linear_grid(blocks, 256), dim3(256), 0, s, packed, codes, n_words); return 0;
        case 8: hipLaunchKernelGGL(unpack_codes_kernel<8>, linear_grid(blocks, 256), dim3(256), 0, s, packed, codes, n_words); return 0;
    }
    return -1;
}

}  // namespace dopt
