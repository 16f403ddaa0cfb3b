// quant_split_lds_kernel instantiations for 2-bit K and 2-bit V codes with
// 8 head columns (GQA groups of at most 8 query heads).
#include "quant_split.h"

namespace tkv {

template void launch_quant_hs<128, 2, 2, 16, 8>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 2, 2, 32, 8>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<128, 2, 2, 64, 8>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 2, 2, 16, 8>(const SplitParams&, dim3, int, hipStream_t);
template void launch_quant_hs<64, 2, 2, 32, 8>(const SplitParams&, dim3, int, hipStream_t);

}  // namespace tkv
