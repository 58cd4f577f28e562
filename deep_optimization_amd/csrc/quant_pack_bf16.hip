// Instantiates the quant-pack kernels for one input element type (see quant_pack.h).
#include "quant_pack_launch.h"

namespace dopt {
template int launch_quant_pack_dt<DT_BF16>(const QuantPackArgs&, int, int, int, int, hipStream_t);
}  // namespace dopt
