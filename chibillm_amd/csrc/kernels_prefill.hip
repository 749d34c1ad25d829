// Chunked-prefill causal attention over paged KV (MFMA tiles): placeholder
// until the MFMA kernel lands; rows take the decode kernels meanwhile.
#include "ckv_internal.h"

namespace ckv {

bool prefill_supported(const pool_view&, uint32_t)
{
    return false;
}

hipError_t launch_prefill(hipStream_t, const pool_view&, const meta_view&, uint32_t, const void*,
                          uint32_t, float, void*)
{
    return hipErrorInvalidValue;
}

} // namespace ckv
