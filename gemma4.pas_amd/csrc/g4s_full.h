/*
 * g4s_full.h -- launch interface of the full-vocabulary path (g4s_full.hip).
 */
#ifndef G4S_FULL_H
#define G4S_FULL_H

#include "g4s_device.h"

namespace g4s {

struct FullWorkspace {
    void* base = nullptr;
    size_t bytes = 0;
};

struct FullArgs {
    const void* logits;
    int64_t row_stride;
    int32_t vocab;
    int32_t batch;
    const g4s_params* params;
    const double* u;
    g4s_params p0;
    double u0;
    float softcap;
    FullWorkspace ws;
    int32_t* ids;
    g4s_outputs out;
};

hipError_t full_alloc(FullWorkspace& ws, int32_t vocab, int32_t max_batch);
void full_free(FullWorkspace& ws);
hipError_t full_init(FullWorkspace& ws, hipStream_t s);
hipError_t full_launch(const FullArgs& a, int dtype, hipStream_t s);

}  // namespace g4s

#endif
