// Compile-time dispatch of quant_pack_kernel over (bits, group size, rounding) for one element
// type. Included by quant_pack_<dtype>.hip, each of which instantiates launch_quant_pack_dt<DT>.
#pragma once

#include "quant_pack.h"

namespace dopt {

template <int DT, int BITS, int G, int RN>
static int qp_launch(const QuantPackArgs& a, hipStream_t s) {
    using C = QuantPackCfg<DT, BITS, G, RN>;
    const uint64_t waves = ((uint64_t)a.n_groups + C::GPW - 1) / C::GPW;
    const uint64_t blocks = (waves + C::WAVES - 1) / C::WAVES;
    if (blocks == 0) return 0;
    hipLaunchKernelGGL((quant_pack_kernel<DT, BITS, G, RN>), dim3((uint32_t)blocks), dim3(64 * C::WAVES), 0, s,
                       a);
    return 0;
}

template <int DT, int BITS, int G>
static int qp_rn(const QuantPackArgs& a, int rn, hipStream_t s) {
    switch (rn) {
        case RN_NEAREST: return qp_launch<DT, BITS, G, RN_NEAREST>(a, s);
        case RN_NOISE: return qp_launch<DT, BITS, G, RN_NOISE>(a, s);
        case RN_PHILOX: return qp_launch<DT, BITS, G, RN_PHILOX>(a, s);
    }
    return -1;
}

template <int DT, int BITS>
static int qp_g(const QuantPackArgs& a, int g, int rn, hipStream_t s) {
    switch (g) {
        case 64: return qp_rn<DT, BITS, 64>(a, rn, s);
        case 128: return qp_rn<DT, BITS, 128>(a, rn, s);
        case 256: return qp_rn<DT, BITS, 256>(a, rn, s);
        case 512: return qp_rn<DT, BITS, 512>(a, rn, s);
        case 1024: return qp_rn<DT, BITS, 1024>(a, rn, s);
    }
    return -1;
}

template <int DT>
int launch_quant_pack_dt(const QuantPackArgs& a, int bits, int g, int rn, hipStream_t s) {
    switch (bits) {
        case 1: return qp_g<DT, 1>(a, g, rn, s);
        case 2: return qp_g<DT, 2>(a, g, rn, s);
        case 4: return qp_g<DT, 4>(a, g, rn, s);
        case 8: return qp_g<DT, 8>(a, g, rn, s);
    }
    return -1;
}

}  // namespace dopt
