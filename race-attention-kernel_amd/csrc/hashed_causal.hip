// hashed_causal.hip -- the causal op with the hashing inside (kernels in
// hashed_kernels.h): the entry from race_api.hip and the fp32 instantiation.
// The bf16 one is in hashed_causal_bf16.hip (a file each keeps compile times
// short).
#include "hashed_kernels.h"

namespace race {

bool hashed_causal_supported(int L, int K, int d) {
    if (L < 1 || K < 2 || K > 8 || L * K > 64) return false;
    const int S = L << K;
    return mfma_causal_supported(S, d);
}

hipError_t launch_hashed_causal(const HashedArgs& a, const Problem& p, hipStream_t stream, Marks* marks) {
    if (!hashed_causal_supported(a.L, a.K, p.d) || p.S != (a.L << a.K)) return hipErrorInvalidValue;
    if (p.dtype == RACE_BF16) return launch_hashed_causal_bf16(a, p, stream, marks);
    return hashed::dispatch_hashed<float>(a, p, stream, marks);
}

}  // namespace race
