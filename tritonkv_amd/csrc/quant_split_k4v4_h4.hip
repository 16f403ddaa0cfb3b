// quant_split_lds_kernel instantiations for 4-bit K and 4-bit V codes with
// 4 head columns (GQA groups of at most 4 query heads).
#include "quant_split.h"

namespace tkv {

template void launch_quant_hs<128, 4, 4, 16, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 4, 4, 32, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 4, 4, 64, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 4, 4, 16, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 4, 4, 32, 4>(const SplitParams&, dim3, int, hipStream_t);

}  // namespace tkv
