// Streaming 1x1 int8 conv kernel instances: epilogue SiLU to fp16.
#include "conv_s1x1.h"

namespace aexrt {
namespace s1x1 {

AEXRT_S1X1_INSTANCE(1)

}  // namespace s1x1
}  // namespace aexrt
