// Instantiates and dispatches the unpack-dequant kernels (see dequant_unpack.h).
//
// Launch shape (measured on MI355X, bf16 [256, 256, 56, 56], g = 256, 2-bit): 16-byte units,
// at most 16 lanes per group, about four 16-byte stores per lane, and non-temporal stores: the
// dequantized activation is written once and consumed later by another kernel, and the nt
// stores lifted the kernel from 67% to 88% of HBM peak.
#include "dequant_unpack.h"

namespace dopt {

template <int YT, int G>
struct DequantShape {
    static constexpr int UB = 16;
    static constexpr int CPG = G / (UB / DType<YT>::bytes);
    static constexpr int LPG = CPG < 16 ? CPG : 16;
    static constexpr int CPL = CPG / LPG;
    static constexpr int P = CPL >= 4 ? 1 : 4 / CPL;
};

template <int YT, int BITS, int G, int DYT>
static int dq_launch(const DequantArgs& a, hipStream_t s) {
    using S = DequantShape<YT, G>;
    using C = DequantCfg<YT, BITS, G, S::UB, S::LPG, S::P, true>;  // shape of every DYT variant
    const uint64_t waves = ((uint64_t)a.n_groups + C::GPW - 1) / C::GPW;
    const uint64_t blocks = (waves + C::WAVES - 1) / C::WAVES;
    if (blocks == 0) return 0;
    if (!a.tiled) {
        hipLaunchKernelGGL((dequant_unpack_kernel<YT, BITS, G, S::UB, S::LPG, S::P, true, DYT, false>),
                           linear_grid(blocks, 64 * C::WAVES), dim3(64 * C::WAVES), 0, s, a);
        return 0;
    }
    if constexpr (G == 64 || G == 256 || G == 1024) {  // the square group sizes
        hipLaunchKernelGGL((dequant_unpack_kernel<YT, BITS, G, S::UB, S::LPG, S::P, true, DYT, true>),
                           linear_grid(blocks, 64 * C::WAVES), dim3(64 * C::WAVES), 0, s, a);
        return 0;
    }
    return -1;
}

template <int YT, int BITS, int G>
static int dq_dy(const DequantArgs& a, int dyt, hipStream_t s) {
    if (dyt == DY_NONE) return dq_launch<YT, BITS, G, DY_NONE>(a, s);
    if constexpr (YT == DT_BF16) {  // the fused activation backward writes bf16 dx
        if (dyt == DT_BF16) return dq_launch<YT, BITS, G, DT_BF16>(a, s);
        if (dyt == DT_F32) return dq_launch<YT, BITS, G, DT_F32>(a, s);
    }
    return -1;
}

template <int YT, int BITS>
static int dq_g(const DequantArgs& a, int g, int dyt, hipStream_t s) {
    switch (g) {
        case 64: return dq_dy<YT, BITS, 64>(a, dyt, s);
        case 128: return dq_dy<YT, BITS, 128>(a, dyt, s);
        case 256: return dq_dy<YT, BITS, 256>(a, dyt, s);
        case 512: return dq_dy<YT, BITS, 512>(a, dyt, s);
        case 1024: return dq_dy<YT, BITS, 1024>(a, dyt, s);
    }
    return -1;
}

template <int YT>
int launch_dequant_unpack_dt(const DequantArgs& a, int bits, int g, int dyt, hipStream_t s) {
    switch (bits) {
        case 1: return dq_g<YT, 1>(a, g, dyt, s);
        case 2: return dq_g<YT, 2>(a, g, dyt, s);
        case 4: return dq_g<YT, 4>(a, g, dyt, s);
        case 8: return dq_g<YT, 8>(a, g, dyt, s);
    }
    return -1;
}

template int launch_dequant_unpack_dt<DT_F32>(const DequantArgs&, int, int, int, hipStream_t);
template int launch_dequant_unpack_dt<DT_BF16>(const DequantArgs&, int, int, int, hipStream_t);

}  // namespace dopt
