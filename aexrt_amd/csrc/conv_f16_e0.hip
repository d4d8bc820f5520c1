// Implicit-GEMM conv kernel instances: fp16, weights staged once per block, any epilogue flags.
#include "conv_igemm.h"

namespace aexrt {
namespace igemm {

AEXRT_IGEMM_INSTANCE(false, false, 0)

}  // namespace igemm
}  // namespace aexrt
