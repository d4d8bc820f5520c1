// fp16 instances of the bottleneck-pair kernel.
#include "conv_pair_inst.h"

namespace aexrt {
namespace pair {
template hipError_t pair_launch_family<false>(const PairParams&, int, int, int, hipStream_t);
template int pair_resident_blocks<false>(int, int, int);
}  // namespace pair
}  // namespace aexrt
