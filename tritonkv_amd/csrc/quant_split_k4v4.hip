// quant_split_lds_kernel (and read-probe) instantiations for 4-bit K and 4-bit V codes:
// the launch dispatcher and the kernels with 16 head columns.  The 4- and 8-column
// kernels are instantiated in quant_split_k4v4_h4.hip and quant_split_k4v4_h8.hip.
#include "quant_split.h"

namespace tkv {

extern template void launch_quant_hs<128, 4, 4, 16, 4>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<128, 4, 4, 32, 4>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<128, 4, 4, 64, 4>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<64, 4, 4, 16, 4>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<64, 4, 4, 32, 4>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<128, 4, 4, 16, 8>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<128, 4, 4, 32, 8>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<128, 4, 4, 64, 8>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<64, 4, 4, 16, 8>(const SplitParams&, dim3, int, hipStream_t);
extern template void launch_quant_hs<64, 4, 4, 32, 8>(const SplitParams&, dim3, int, hipStream_t);

template void launch_quant<128, 4, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 4, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 4, 4, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<128, 4, 4, 128>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 4, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 4, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant<64, 4, 4, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 4, 4, 16, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 4, 4, 32, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 4, 4, 64, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 4, 4, 128, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 4, 4, 16, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 4, 4, 32, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 4, 4, 64, 16>(const SplitParams&, dim3, int, hipStream_t);

template void launch_read_probe<128, 4, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 4, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 4, 4, 64>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<128, 4, 4, 128>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 4, 4, 16>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 4, 4, 32>(const SplitParams&, dim3, int, hipStream_t);
template void launch_read_probe<64, 4, 4, 64>(const SplitParams&, dim3, int, hipStream_t);

}  // namespace tkv
