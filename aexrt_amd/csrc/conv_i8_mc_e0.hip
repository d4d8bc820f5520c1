// Implicit-GEMM conv kernel instances: int8, weights staged chunk by chunk, any epilogue flags.
#include "conv_igemm.h"

namespace aexrt {
namespace igemm {

AEXRT_IGEMM_INSTANCE(true, true, 0)

}  // namespace igemm
}  // namespace aexrt
