// hashed_causal_bf16.hip -- the bf16 instantiation of the hashed causal
// kernels (hashed_kernels.h); launch_hashed_causal (hashed_causal.hip)
// dispatches here for bf16 rows.
#include "hashed_kernels.h"

namespace race {

hipError_t launch_hashed_causal_bf16(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks) {
    return hashed::dispatch_hashed<bf16_t>(a, p, stream, marks);
}

}  // namespace race
