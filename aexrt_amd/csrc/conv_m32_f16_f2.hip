// fp16 32x32-MFMA 3x3 SiLU conv instances with a fused 1x1 conv in the
// epilogue: block tiles that cover every output channel (nq 2 or 3).
#include "conv_m32.h"

namespace aexrt {
namespace m32 {

hipError_t m32_launch_f2(const M32Params& h, int mq, int nq, int np, int nw, int ng, hipStream_t stream) {
    // 8 waves in two groups of 4
#define AEXRT_M32_F2_CASE2G(M, N, P) \
    if (ng == 2 && nw == 8 && mq == M && nq == N && np == P) return m32_launch_cfg<false, M, N, P, 1, 8, true, 2>(h, stream);
    AEXRT_M32_F2_CASE2G(1, 2, 4) AEXRT_M32_F2_CASE2G(1, 3, 4) AEXRT_M32_F2_CASE2G(1, 2, 8) AEXRT_M32_F2_CASE2G(1, 3, 8)
#undef AEXRT_M32_F2_CASE2G
    if (ng != 1) return hipErrorInvalidValue;
#define AEXRT_M32_F2_CASE(M, N, P, W) \
    if (mq == M && nq == N && np == P && nw == W) return m32_launch_cfg<false, M, N, P, 1, W, true>(h, stream);
    AEXRT_M32_F2_CASE(1, 2, 4, 4) AEXRT_M32_F2_CASE(2, 2, 4, 4) AEXRT_M32_F2_CASE(1, 3, 4, 4)
    AEXRT_M32_F2_CASE(2, 3, 4, 4) AEXRT_M32_F2_CASE(1, 2, 8, 4) AEXRT_M32_F2_CASE(2, 2, 8, 4)
    AEXRT_M32_F2_CASE(1, 3, 8, 4) AEXRT_M32_F2_CASE(1, 2, 4, 8) AEXRT_M32_F2_CASE(2, 2, 4, 8)
    AEXRT_M32_F2_CASE(1, 3, 4, 8) AEXRT_M32_F2_CASE(1, 2, 8, 8)
#undef AEXRT_M32_F2_CASE
    return hipErrorInvalidValue;
}

}  // namespace m32
}  // namespace aexrt
