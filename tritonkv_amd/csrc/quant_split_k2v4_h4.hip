// quant_split_lds_kernel instantiations for 2-bit K and 4-bit V codes with
// 4 head columns (GQA groups of at most 4 query heads).
#include "quant_split.h"

namespace tkv {

template void launch_quant_hs<128, 2, 4, 16, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 2, 4, 32, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 2, 4, 64, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 2, 4, 16, 4>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 2, 4, 32, 4>(const SplitParams&, dim3, int, hipStream_t);

}  // namespace tkv
