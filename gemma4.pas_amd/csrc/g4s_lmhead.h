/*
 * g4s_lmhead.h -- Q4_0 LM head (g4s_lmhead.hip).
 */
#ifndef G4S_LMHEAD_H
#define G4S_LMHEAD_H

#include "g4s_device.h"

namespace g4s {

hipError_t lmhead_q4_0_launch(const uint8_t* w, int32_t rows, int32_t cols, const float* h,
                              int32_t batch, float* logits, int64_t stride, hipStream_t s);

}  // namespace g4s

#endif
