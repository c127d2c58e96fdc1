/*
 * g4s_full.hip -- the full-vocabulary sampling path (TopK <= 0 or TopK >= V).
 */
#include "g4s_full.h"

namespace g4s {

hipError_t full_alloc(FullWorkspace& ws, int32_t, int32_t)
{
    ws.base = nullptr;
    ws.bytes = 0;
    return hipSuccess;
}
void full_free(FullWorkspace& ws)
{
    if (ws.base) (void)hipFree(ws.base);
    ws.base = nullptr;
}
hipError_t full_init(FullWorkspace&, hipStream_t) { return hipSuccess; }
hipError_t full_launch(const FullArgs&, int, hipStream_t) { return hipErrorNotSupported; }

}  // namespace g4s
