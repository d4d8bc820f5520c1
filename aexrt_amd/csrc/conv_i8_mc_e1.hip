// Implicit-GEMM conv kernel instances: int8, weights staged chunk by chunk, SiLU to fp16.
#include "conv_igemm.h"

namespace aexrt {
namespace igemm {

AEXRT_IGEMM_INSTANCE(true, true, 1)

}  // namespace igemm
}  // namespace aexrt
