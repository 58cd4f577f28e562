// Instantiates and dispatches the unpack-dequant kernels (see dequant_unpack.h).
#include "dequant_unpack.h"

namespace dopt {

template <int YT, int BITS, int G>
static int dq_launch(const DequantArgs& a, hipStream_t s) {
    using C = DequantCfg<YT, BITS, G>;
    const uint64_t waves = ((uint64_t)a.n_groups + C::GPW - 1) / C::GPW;
    const uint64_t blocks = (waves + C::WAVES - 1) / C::WAVES;
    if (blocks == 0) return 0;
    hipLaunchKernelGGL((dequant_unpack_kernel<YT, BITS, G>), dim3((uint32_t)blocks), dim3(64 * C::WAVES), 0, s, a);
    return 0;
}

template <int YT, int BITS>
static int dq_g(const DequantArgs& a, int g, hipStream_t s) {
    switch (g) {
        case 64: return dq_launch<YT, BITS, 64>(a, s);
        case 128: return dq_launch<YT, BITS, 128>(a, s);
        case 256: return dq_launch<YT, BITS, 256>(a, s);
        case 512: return dq_launch<YT, BITS, 512>(a, s);
        case 1024: return dq_launch<YT, BITS, 1024>(a, s);
    }
    return -1;
}

template <int YT>
int launch_dequant_unpack_dt(const DequantArgs& a, int bits, int g, hipStream_t s) {
    switch (bits) {
        case 1: return dq_g<YT, 1>(a, g, s);
        case 2: return dq_g<YT, 2>(a, g, s);
        case 4: return dq_g<YT, 4>(a, g, s);
        case 8: return dq_g<YT, 8>(a, g, s);
    }
    return -1;
}

template int launch_dequant_unpack_dt<DT_F32>(const DequantArgs&, int, int, hipStream_t);
template int launch_dequant_unpack_dt<DT_BF16>(const DequantArgs&, int, int, hipStream_t);

}  // namespace dopt
