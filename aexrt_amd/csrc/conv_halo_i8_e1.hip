// int8 halo-tile 3x3 conv instances, epilogue variant 1.
#include "conv_halo.h"

namespace aexrt {
namespace halo {
AEXRT_HALO_INSTANCE(true, 1)
}  // namespace halo
}  // namespace aexrt
