// Implicit-GEMM conv kernel instances: int8, weights staged once per block, SiLU to fp16.
#include "conv_igemm.h"

namespace aexrt {
namespace igemm {

AEXRT_IGEMM_INSTANCE(true, false, 1)

}  // namespace igemm
}  // namespace aexrt
