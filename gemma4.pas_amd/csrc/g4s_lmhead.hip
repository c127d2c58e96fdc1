/*
 * g4s_lmhead.hip -- Q4_0 LM head, bit-exact with CpuMatVecQ4.
 */
#include "g4s_lmhead.h"

namespace g4s {

hipError_t lmhead_q4_0_launch(const uint8_t*, int32_t, int32_t, const float*, int32_t, float*,
                              int64_t, hipStream_t)
{
    return hipErrorNotSupported;
}

}  // namespace g4s
