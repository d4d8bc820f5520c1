// Kernel instances of the bottleneck-pair kernel for one arithmetic (int8 or
// fp16), included by conv_pair_i8.hip / conv_pair_f16.hip.
#pragma once
#include "conv_pair.h"

namespace aexrt {
namespace pair {

template <bool INT8, int NQ, int MQ>
int pair_resident_cfg(int lds) {
    int per_cu = 0, cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, conv_pair_kernel<INT8, NQ, MQ>, kNT, (size_t)lds) !=
            hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu < 1 || cus < 1)
        return 0;
    return per_cu * cus;
}

#define AEXRT_PAIR_CASES(X) X(1, 1) X(1, 2) X(1, 4) X(2, 1) X(2, 2) X(4, 1)

// Blocks of the (nq, mq) instance the GPU holds at once with lds bytes of
// dynamic LDS (0 when unknown: no launch then).
template <bool INT8>
int pair_resident_blocks(int nq, int mq, int lds) {
#define AEXRT_PAIR_RES(Q, M) \
    if (nq == Q && mq == M) return pair_resident_cfg<INT8, Q, M>(lds);
    AEXRT_PAIR_CASES(AEXRT_PAIR_RES)
#undef AEXRT_PAIR_RES
    return 0;
}

template <bool INT8>
hipError_t pair_launch_family(const PairParams& h, int nq, int mq, int lds, hipStream_t s) {
#define AEXRT_PAIR_LAUNCH(Q, M)                                                                                   \
    if (nq == Q && mq == M) {                                                                                     \
        hipLaunchKernelGGL((conv_pair_kernel<INT8, Q, M>), dim3((unsigned)h.ntile), dim3(kNT), (size_t)lds, s, h); \
        return hipGetLastError();                                                                                 \
    }
    AEXRT_PAIR_CASES(AEXRT_PAIR_LAUNCH)
#undef AEXRT_PAIR_LAUNCH
    return hipErrorInvalidValue;
}

}  // namespace pair
}  // namespace aexrt
