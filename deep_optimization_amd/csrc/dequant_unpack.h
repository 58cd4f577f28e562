// gfx950 unpack-dequant kernel: y = float(q) * scale + min, one rounding to the output type.
// Semantics follow Activation_Compression/act_triton_kernel.py:199-241; with the tile layout the
// inverse scatter of tensor_act_reshape_utils.py:131-154 is fused into the stores.
//
// Work decomposition mirrors quant_pack.h: LPG lanes per group, each lane CPL 16-byte output
// chunks c = i*LPG + li (whole-cache-line stores per instruction), P passes per iteration.
// Per-group scale/min of the wave's GPW groups are staged once in LDS (one coalesced load per
// array) and read back by the LPG lanes of each group; codes are read as the dword (or dword
// pair) holding the chunk's E*BITS bits.
#pragma once

#include "dopt_device.h"

namespace dopt {

struct DequantArgs {
    const uint32_t* packed;
    const void* scale;
    const void* minv;
    void* y;
    uint32_t n_groups;
    uint32_t tiled;
    uint32_t tiles_w;
    uint32_t log2s;
    uint64_t row;
    uint32_t meta_bf16;
};

template <int YT, int BITS, int G>
struct DequantCfg {
    static constexpr int E = DType<YT>::per16;
    static constexpr int CPG = G / E;
    static constexpr int CPL = CPG >= 32 ? 4 : (CPG >= 16 ? 2 : 1);
    static constexpr int LPG = CPG / CPL;
    static constexpr int GPP = 64 / LPG;
    static constexpr int P = 8 / CPL;
    static constexpr int GPW = P * GPP;
    static constexpr int W = G * BITS / 32;
    static constexpr int PW = E * BITS;
    static constexpr int WAVES = 4;
    static_assert(LPG >= 4 && LPG <= 64, "group must span 4..64 lanes");
    static_assert(GPW <= 64, "one lane per staged group");
};

template <int G>
__device__ __forceinline__ uint64_t dq_elem_index(const DequantArgs& a, uint32_t r, uint32_t e0) {
    if (!a.tiled) return (uint64_t)r * G + e0;
    const uint32_t band = r / a.tiles_w;
    const uint32_t tw = r - band * a.tiles_w;
    const uint32_t smask = (1u << a.log2s) - 1u;
    return (((uint64_t)band * a.row) << a.log2s) + ((uint64_t)tw << a.log2s) +
           (uint64_t)(e0 >> a.log2s) * a.row + (e0 & smask);
}

template <int YT, int BITS, int G>
__global__ __launch_bounds__(256) void dequant_unpack_kernel(DequantArgs a) {
    using C = DequantCfg<YT, BITS, G>;
    constexpr int E = C::E, CPL = C::CPL, LPG = C::LPG, GPP = C::GPP, P = C::P, W = C::W;
    constexpr int PW = C::PW;
    constexpr uint32_t QMAX = (1u << BITS) - 1u;

    __shared__ float s_scale[C::WAVES][C::GPW];
    __shared__ float s_min[C::WAVES][C::GPW];

    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int slot = lane / LPG;
    const int li = lane % LPG;
    const uint32_t g0 = (blockIdx.x * C::WAVES + wv) * (uint32_t)C::GPW;

    // ---- stage the wave's per-group scale/min (one coalesced load per array)
    if (lane < C::GPW) {
        const uint32_t r = g0 + lane;
        float sc = 0.0f, mn = 0.0f;
        if (r < a.n_groups) {
            if (a.meta_bf16) {
                sc = bf16_bits_to_f32(((const uint16_t*)a.scale)[r]);
                mn = bf16_bits_to_f32(((const uint16_t*)a.minv)[r]);
            } else {
                sc = ((const float*)a.scale)[r];
                mn = ((const float*)a.minv)[r];
            }
        }
        s_scale[wv][lane] = sc;
        s_min[wv][lane] = mn;
    }

    // ---- code loads: the dword(s) holding each chunk's E*BITS bits
    uint32_t cw[P][CPL][PW > 32 ? 2 : 1];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        const bool ok = r < a.n_groups;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t c = (uint32_t)(i * LPG + li);
            const uint32_t* src = a.packed + (uint64_t)r * W;
            if constexpr (PW > 32) {
                uint2 d = make_uint2(0u, 0u);
                if (ok) d = *(const uint2*)(src + 2 * c);
                cw[p][i][0] = d.x;
                cw[p][i][1] = d.y;
            } else {
                uint32_t d = 0u;
                if (ok) d = src[(c * PW) / 32];
                cw[p][i][0] = d >> ((c * PW) % 32);
            }
        }
    }
    __syncthreads();

    char* yb = (char*)a.y;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        const bool ok = r < a.n_groups;
        const float sc = s_scale[wv][p * GPP + slot];
        const float mn = s_min[wv][p * GPP + slot];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t c = (uint32_t)(i * LPG + li);
            float out[E];
#pragma unroll
            for (int k = 0; k < E; ++k) {
                uint32_t q;
                if constexpr (PW > 32)
                    q = (cw[p][i][(k * BITS) / 32] >> ((k * BITS) % 32)) & QMAX;
                else
                    q = (cw[p][i][0] >> (k * BITS)) & QMAX;
                float t = (float)q * sc;
                out[k] = t + mn;
            }
            uint4 v;
            if constexpr (YT == DT_F32) {
                v = make_uint4(__float_as_uint(out[0]), __float_as_uint(out[1]), __float_as_uint(out[2]),
                               __float_as_uint(out[3]));
            } else {
                v = make_uint4(pack_bf16x2(out[0], out[1]), pack_bf16x2(out[2], out[3]),
                               pack_bf16x2(out[4], out[5]), pack_bf16x2(out[6], out[7]));
            }
            if (ok) *(uint4*)(yb + dq_elem_index<G>(a, r, c * E) * DType<YT>::bytes) = v;
        }
    }
}

template <int YT>
int launch_dequant_unpack_dt(const DequantArgs& a, int bits, int g, hipStream_t s);

}  // namespace dopt
