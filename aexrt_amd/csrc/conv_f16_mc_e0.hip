// Implicit-GEMM conv kernel instances: fp16, weights staged chunk by chunk, any epilogue flags.
#include "conv_igemm.h"

namespace aexrt {
namespace igemm {

AEXRT_IGEMM_INSTANCE(false, true, 0)

}  // namespace igemm
}  // namespace aexrt
