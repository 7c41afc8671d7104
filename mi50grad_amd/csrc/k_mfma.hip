// Multi-query (chunked prefill / tree verify) attention with MFMA tiles.
#include "k_common.h"
#include "kva_internal.h"

namespace kva {

hipError_t launch_multi_query(const MultiQueryArgs &, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace kva
