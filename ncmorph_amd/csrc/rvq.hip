// Multiscale RVQ encode (placeholder until the MFMA distance path lands).
#include "common.h"
#include "rvq.h"

namespace ncm {

int rvq_encode(ncm_ctx_t*, const float*, int64_t, int64_t, int64_t, int64_t, const int32_t*,
               const uint16_t*, const float*, int64_t, int32_t*, float*, float*, const int32_t*,
               int64_t*) {
    return NCM_E_SHAPE;
}

}  // namespace ncm
