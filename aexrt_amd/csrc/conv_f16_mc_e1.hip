// Implicit-GEMM conv kernel instances: fp16, weights staged chunk by chunk, SiLU to fp16.
#include "conv_igemm.h"

namespace aexrt {
namespace igemm {

AEXRT_IGEMM_INSTANCE(false, true, 1)

}  // namespace igemm
}  // namespace aexrt
