// mfma_causal.hip -- matrix-core (MFMA) causal forward for gfx950.
#include "race_internal.h"

namespace race {

bool mfma_causal_supported(int S, int d) {
    (void)S;
    (void)d;
    return false;
}

hipError_t launch_causal_mfma(const void*, const void*, const void*, void*, float*, float*,
                              const Problem&, hipStream_t, Marks*) {
    return hipErrorInvalidValue;
}

}  // namespace race
