// Compile-time dispatch of quant_pack_kernel over (bits, group size, rounding, pre-transform) for
// one element type, with the launch shape of each configuration. Included by
// quant_pack_<dtype>.hip, each of which instantiates launch_quant_pack_dt<DT>.
//
// Launch shapes (measured on MI355X, bf16 [256, 256, 56, 56], g = 256, 2-bit): one pass per wave
// (P = 1: a modest 32-64 bytes of loads in flight per lane across many short waves streams
// best), two units per lane (one for a noise tensor and for Philox), units of 16 bytes (32 for
// Philox rounding, so that one Philox4x32-10 call covers a lane's 16 contiguous bf16 elements),
// cached loads (non-temporal loads measured slower here).
#pragma once

#include "quant_pack.h"

namespace dopt {

template <int DT, int BITS, int G, int RN, int PRE>
struct QuantPackShape {
    static constexpr int BYTES = DType<DT>::bytes;
    // unit bytes: Philox units hold NOISE_EPC elements where that is at most 64 bytes
    static constexpr int UB = RN == RN_PHILOX ? (NOISE_EPC * BYTES <= 64 ? NOISE_EPC * BYTES : 64) : 16;
    static constexpr int UE = UB / BYTES;
    static constexpr int CPG = G / UE;
    static constexpr int UBITS = UE * BITS;
    static constexpr int LPD = UBITS >= 32 ? 1 : 32 / UBITS;  // lanes merged per code dword
    // noise tensor and Philox: one unit per lane (Philox: 16 elements, one generator call; measured
    // 3% faster than two units per lane on bf16 [256,256,56,56], g = 256, 2-bit); otherwise two. The fused activations run
    // GELU with two passes per wave, SiLU with one: measured on the ViT MLP activation (bf16
    // [256,197,3072], g = 128) over 1-16 units per lane and 1-4 passes, two units per lane gave
    // the fastest kernels at 1-8 bits (four units, 108 VGPRs for GELU, ran 4-10% slower)
    static constexpr int L0 = RN == RN_NOISE || RN == RN_PHILOX ? CPG : CPG / 2;
    static constexpr int L1 = L0 < LPD ? LPD : L0;
    static constexpr int L2 = L1 < 2 ? 2 : L1;
    static constexpr int LPG = L2 > 64 ? 64 : L2;
    static constexpr int P = PRE == PRE_GELU ? 2 : 1;
};

template <int DT, int BITS, int G, int RN, int PRE>
static int qp_launch(const QuantPackArgs& a, hipStream_t s) {
    using S = QuantPackShape<DT, BITS, G, RN, PRE>;
    using C = QuantPackCfg<DT, BITS, G, RN, S::UB, S::LPG, S::P>;
    const uint64_t waves = ((uint64_t)a.n_groups + C::GPW - 1) / C::GPW;
    const uint64_t blocks = (waves + C::WAVES - 1) / C::WAVES;
    if (blocks == 0) return 0;
    if (!a.tiled) {
        hipLaunchKernelGGL((quant_pack_kernel<DT, BITS, G, RN, S::UB, S::LPG, S::P, PRE, false, false>),
                           linear_grid(blocks, 64 * C::WAVES), dim3(64 * C::WAVES), 0, s, a);
        return 0;
    }
    if constexpr (G == 64 || G == 256 || G == 1024) {  // the square group sizes
        hipLaunchKernelGGL((quant_pack_kernel<DT, BITS, G, RN, S::UB, S::LPG, S::P, PRE, false, true>),
                           linear_grid(blocks, 64 * C::WAVES), dim3(64 * C::WAVES), 0, s, a);
        return 0;
    }
    return -1;
}

template <int DT, int BITS, int G>
static int qp_rn(const QuantPackArgs& a, int rn, int pre, hipStream_t s) {
    if (pre == PRE_REF) {  // the reference quantizer's clamp / squash, with any rounding
        switch (rn) {
            case RN_NEAREST: return qp_launch<DT, BITS, G, RN_NEAREST, PRE_REF>(a, s);
            case RN_NOISE: return qp_launch<DT, BITS, G, RN_NOISE, PRE_REF>(a, s);
            case RN_PHILOX: return qp_launch<DT, BITS, G, RN_PHILOX, PRE_REF>(a, s);
        }
        return -1;
    }
    if (pre != PRE_NONE) {  // the fused activations round to nearest
        if (rn != RN_NEAREST) return -1;
        switch (pre) {
            case PRE_GELU:
                if constexpr (DT == DT_F16) return -1;
                else return qp_launch<DT, BITS, G, RN_NEAREST, PRE_GELU>(a, s);
            case PRE_SILU:
                if constexpr (DT == DT_F16) return -1;
                else return qp_launch<DT, BITS, G, RN_NEAREST, PRE_SILU>(a, s);
        }
        return -1;
    }
    switch (rn) {
        case RN_NEAREST: return qp_launch<DT, BITS, G, RN_NEAREST, PRE_NONE>(a, s);
        case RN_NOISE: return qp_launch<DT, BITS, G, RN_NOISE, PRE_NONE>(a, s);
        case RN_PHILOX: return qp_launch<DT, BITS, G, RN_PHILOX, PRE_NONE>(a, s);
    }
    return -1;
}

template <int DT, int BITS>
static int qp_g(const QuantPackArgs& a, int g, int rn, int pre, hipStream_t s) {
    switch (g) {
        case 64: return qp_rn<DT, BITS, 64>(a, rn, pre, s);
        case 128: return qp_rn<DT, BITS, 128>(a, rn, pre, s);
        case 256: return qp_rn<DT, BITS, 256>(a, rn, pre, s);
        case 512: return qp_rn<DT, BITS, 512>(a, rn, pre, s);
        case 1024: return qp_rn<DT, BITS, 1024>(a, rn, pre, s);
    }
    return -1;
}

template <int DT>
int launch_quant_pack_dt(const QuantPackArgs& a, int bits, int g, int rn, int pre, hipStream_t s) {
    switch (bits) {
        case 1: return qp_g<DT, 1>(a, g, rn, pre, s);
        case 2: return qp_g<DT, 2>(a, g, rn, pre, s);
        case 4: return qp_g<DT, 4>(a, g, rn, pre, s);
        case 8: return qp_g<DT, 8>(a, g, rn, pre, s);
    }
    return -1;
}

}  // namespace dopt
