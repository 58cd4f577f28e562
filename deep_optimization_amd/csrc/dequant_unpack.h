// gfx950 unpack-dequant kernel: y = fma(float(q), scale, min), one rounding to the output type.
// Semantics follow Activation_Compression/act_triton_kernel.py:199-241 (`q * scale + xmin`,
// compiled by Triton with FMA contraction); with the tile layout the inverse scatter of
// tensor_act_reshape_utils.py:131-154 is fused into the stores.
//
// Work decomposition mirrors quant_pack.h: a lane owns units of UE output elements (UB bytes,
// written as UB/16 consecutive 16-byte stores), a group's CPG units are spread over LPG lanes
// (unit c = i*LPG + li), and a wave handles GPW = P*64/LPG groups. Each lane loads its groups'
// scale and minimum itself (the LPG lanes of a group share one request) and a unit's UE*BITS
// code bits as the one dword (or 2/4-dword vector) that holds them; nothing is staged in LDS and
// no wave waits for another. (Staging them in LDS behind a workgroup barrier cost 12 us of the
// 81 us the kernel took on the 2-bit, g = 256 bf16 [256,256,56,56] case when its inputs came
// cold from HBM right after quant-pack.)
#pragma once

#include "dopt_device.h"

namespace dopt {

// DYT (template parameter of dequant_unpack_kernel): DY_NONE writes the dequantized values; DT_BF16
// / DT_F32 multiply them by an incoming gradient dy of that type (same layout as the output) and
// write dx = dy * dequant(q), the backward of the fused GELU / SiLU layers
// (AC/modules/activations/kernel_implementation.py:392-395, :620-640).
enum { DY_NONE = -1 };

struct DequantArgs {
    const void* dy;
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

template <int YT, int BITS, int G, int UB, int LPG_, int P, bool NT>
struct DequantCfg {
    static constexpr int BYTES = DType<YT>::bytes;
    static constexpr int UE = UB / BYTES;
    static constexpr int STORES = UB / 16;
    static constexpr int CPG = G / UE;
    static constexpr int LPG = LPG_ ? LPG_ : (CPG < 64 ? CPG : 64);  // lanes per group
    static constexpr int CPL = CPG / LPG;
    static constexpr int GPP = 64 / LPG;
    static constexpr int GPW = P * GPP;
    static constexpr int W = G * BITS / 32;
    static constexpr int UBITS = UE * BITS;
    static constexpr int CW = UBITS >= 32 ? UBITS / 32 : 1;  // code dwords read per unit
    static constexpr int WAVES = 4;
    static_assert(UB % 16 == 0 && UE * BYTES == UB, "unit must be whole 16-byte stores");
    static_assert(CPG * UE == G && LPG * CPL == CPG, "group must split evenly over lanes");
    static_assert(UBITS <= 128, "a unit reads at most one 16-byte code vector");
};

// the layout is a template parameter, as in quant_pack.h's group_elem_index
template <int G, bool TILED>
__device__ __forceinline__ uint64_t dq_elem_index(const DequantArgs& a, uint32_t r, uint32_t e0) {
    if constexpr (!TILED) return (uint64_t)r * G + e0;
    const uint32_t band = r / a.tiles_w;
    const uint32_t tw = r - band * a.tiles_w;
    const uint32_t smask = (1u << a.log2s) - 1u;
    return (((uint64_t)band * a.row) << a.log2s) + ((uint64_t)tw << a.log2s) +
           (uint64_t)(e0 >> a.log2s) * a.row + (e0 & smask);
}

template <int YT, int BITS, int G, int UB, int LPG_, int P, bool NT, int DYT, bool TILED>
__global__ __launch_bounds__(256) void dequant_unpack_kernel(DequantArgs a) {
    using C = DequantCfg<YT, BITS, G, UB, LPG_, P, NT>;
    constexpr int UE = C::UE, STORES = C::STORES, CPL = C::CPL, LPG = C::LPG, GPP = C::GPP, W = C::W;
    constexpr int UBITS = C::UBITS, CW = C::CW;
    constexpr uint32_t QMAX = (1u << BITS) - 1u;
    constexpr int E16 = DType<YT>::per16;

    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int slot = lane / LPG;
    const int li = lane % LPG;
    const uint32_t g0 = (uint32_t)((linear_block() * C::WAVES + wv) * C::GPW);  // < 2^32 as in quant_pack

    // ---- each lane loads its groups' scale and min itself (the LPG lanes of a group read the
    // same address, one request); no staging, so the waves of a workgroup never wait for each other
    float scs[P], mns[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        scs[p] = mns[p] = 0.0f;
        if (r < a.n_groups) {
            if (a.meta_bf16) {
                scs[p] = bf16_bits_to_f32(((const uint16_t*)a.scale)[r]);
                mns[p] = bf16_bits_to_f32(((const uint16_t*)a.minv)[r]);
            } else {
                scs[p] = ((const float*)a.scale)[r];
                mns[p] = ((const float*)a.minv)[r];
            }
        }
    }

    // ---- code loads: the dword(s) holding each unit's UE*BITS bits
    uint32_t cw[P][CPL][CW];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        const bool ok = r < a.n_groups;
        const uint32_t* src = a.packed + (uint64_t)r * W;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t c = (uint32_t)(i * LPG + li);
            if constexpr (CW == 4) {
                uint4 d = make_uint4(0u, 0u, 0u, 0u);
                if (ok) d = *(const uint4*)(src + 4 * c);
                cw[p][i][0] = d.x;
                cw[p][i][1] = d.y;
                cw[p][i][2] = d.z;
                cw[p][i][3] = d.w;
            } else if constexpr (CW == 2) {
                uint2 d = make_uint2(0u, 0u);
                if (ok) d = *(const uint2*)(src + 2 * c);
                cw[p][i][0] = d.x;
                cw[p][i][1] = d.y;
            } else {
                uint32_t d = 0u;
                if (ok) d = src[(c * UBITS) / 32];
                cw[p][i][0] = UBITS >= 32 ? d : d >> ((c * UBITS) % 32);
            }
        }
    }
    char* yb = (char*)a.y;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint32_t r = g0 + p * GPP + slot;
        const bool ok = r < a.n_groups;
        const float sc = scs[p];
        const float mn = mns[p];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const uint32_t c = (uint32_t)(i * LPG + li);
            float out[UE];
#pragma unroll
            for (int k = 0; k < UE; ++k) {
                const uint32_t q = (cw[p][i][(k * BITS) / 32] >> ((k * BITS) % 32)) & QMAX;
                out[k] = __builtin_fmaf((float)q, sc, mn);
            }
            if constexpr (DYT != DY_NONE) {
                constexpr int DB = DType<DYT>::bytes;
                constexpr int DE = DType<DYT>::per16;
                float g[UE];
                if (ok) {
#pragma unroll
                    for (int l = 0; l < UE / DE; ++l)
                        widen16<DYT>(ld16<false>((const char*)a.dy + dq_elem_index<G, TILED>(a, r, c * UE + l * DE) * DB),
                                     &g[l * DE]);
                } else {
#pragma unroll
                    for (int k = 0; k < UE; ++k) g[k] = 0.0f;
                }
#pragma unroll
                for (int k = 0; k < UE; ++k) out[k] = g[k] * out[k];
            }
#pragma unroll
            for (int l = 0; l < STORES; ++l) {
                const float* o = &out[l * E16];
                uint4 v;
                if constexpr (YT == DT_F32) {
                    v = make_uint4(__float_as_uint(o[0]), __float_as_uint(o[1]), __float_as_uint(o[2]),
                                   __float_as_uint(o[3]));
                } else {
                    v = make_uint4(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]),
                                   pack_bf16x2(o[6], o[7]));
                }
                if (ok) st16<NT>(yb + dq_elem_index<G, TILED>(a, r, c * UE + l * E16) * C::BYTES, v);
            }
        }
    }
}

template <int YT>
int launch_dequant_unpack_dt(const DequantArgs& a, int bits, int g, int dyt, hipStream_t s);

}  // namespace dopt
