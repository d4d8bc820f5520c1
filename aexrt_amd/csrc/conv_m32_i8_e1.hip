// int8 32x32-MFMA 3x3 conv instances, epilogue variant 1.
#include "conv_m32.h"

namespace aexrt {
namespace m32 {
AEXRT_M32_INSTANCE(true, 1)
}  // namespace m32
}  // namespace aexrt
