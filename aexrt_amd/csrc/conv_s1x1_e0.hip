// Streaming 1x1 int8 conv kernel instances: epilogue with run-time flags (fp32 output, no SiLU, int32 accumulators).
#include "conv_s1x1.h"

namespace aexrt {
namespace s1x1 {

AEXRT_S1X1_INSTANCE(0)

}  // namespace s1x1
}  // namespace aexrt
