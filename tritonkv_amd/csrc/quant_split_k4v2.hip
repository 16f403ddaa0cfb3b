// quant_split_lds_kernel (and read-probe) instantiations for 4-bit K and 2-bit V codes.
#include "quant_split.h"

namespace tkv {

template void launch_quant<128, 4, 2, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 4, 2, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 4, 2, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 4, 2, 128>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 4, 2, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 4, 2, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 4, 2, 64>(const SplitParams&, dim3, int, hipStream_t);

template void launch_read_probe<128, 4, 2, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 4, 2, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 4, 2, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 4, 2, 128>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 4, 2, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 4, 2, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 4, 2, 64>(const SplitParams&, dim3, int, hipStream_t);

}  // namespace tkv
