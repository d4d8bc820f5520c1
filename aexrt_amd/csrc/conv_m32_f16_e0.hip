// fp16 32x32-MFMA 3x3 conv instances, epilogue variant 0.
#include "conv_m32.h"

namespace aexrt {
namespace m32 {
AEXRT_M32_INSTANCE(false, 0)
}  // namespace m32
}  // namespace aexrt
