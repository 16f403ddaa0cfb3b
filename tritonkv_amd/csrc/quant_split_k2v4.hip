// quant_split_lds_kernel (and read-probe) instantiations for 2-bit K and 4-bit V codes.
#include "quant_split.h"

namespace tkv {

template void launch_quant<128, 2, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 2, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 2, 4, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 2, 4, 128>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 2, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 2, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 2, 4, 64>(const SplitParams&, dim3, int, hipStream_t);

template void launch_read_probe<128, 2, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 2, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 2, 4, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 2, 4, 128>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 2, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 2, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 2, 4, 64>(const SplitParams&, dim3, int, hipStream_t);

}  // namespace tkv
