// int8 halo-tile 3x3 conv instances, epilogue variant 0.
#include "conv_halo.h"

namespace aexrt {
namespace halo {
AEXRT_HALO_INSTANCE(true, 0)
}  // namespace halo
}  // namespace aexrt
