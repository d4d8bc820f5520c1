// Halo-tile 3x3 conv instances reading the fp32 NCHW network input (fp16
// MFMA, SiLU, fp16 NHWC output): the network's first conv without a
// separate layout-conversion pass.
#include "conv_halo.h"

namespace aexrt {
namespace halo {

hipError_t halo_launch_nchw(const HaloParams& h, int jn, int pw, int np, hipStream_t stream) {
#define AEXRT_HALO_NCHW_CASE(J, P, N) \
    if (jn == J && pw == P && np == N) return halo_launch_cfg<false, J, P, N, igemm::kEpiSilu, true>(h, stream);
    AEXRT_HALO_NCHW_CASE(1, 2, 4) AEXRT_HALO_NCHW_CASE(1, 4, 4) AEXRT_HALO_NCHW_CASE(2, 2, 4)
    AEXRT_HALO_NCHW_CASE(2, 4, 4) AEXRT_HALO_NCHW_CASE(4, 2, 4) AEXRT_HALO_NCHW_CASE(4, 4, 4)
    AEXRT_HALO_NCHW_CASE(1, 2, 8) AEXRT_HALO_NCHW_CASE(1, 4, 8) AEXRT_HALO_NCHW_CASE(2, 2, 8)
    AEXRT_HALO_NCHW_CASE(2, 4, 8) AEXRT_HALO_NCHW_CASE(4, 2, 8) AEXRT_HALO_NCHW_CASE(4, 4, 8)
#undef AEXRT_HALO_NCHW_CASE
    return hipErrorInvalidValue;
}

}  // namespace halo
}  // namespace aexrt
