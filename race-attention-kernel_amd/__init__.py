"""MI355X-native per-bucket RACE attention: race_fused_fwd(probsQ, probsK, V, causal).

The op and its backward (causal and non-causal) run hand-written gfx950 HIP kernels behind
the C ABI of include/race_mi355x.h (librace_mi355x.so), reached from PyTorch
through the _race_torch binding.  There is no CPU fallback.
"""
from . import causal_v2
from .batched_ace import BatchedACE
from .inputs import CONFIGS, Config, config_inputs, make_inputs
from .ops import (HashedRaceFunction, HashProbsFunction, RaceFusedFunction, hashed_supported,
                  race_causal_backward, race_fused_fwd, race_fused_fwd_carry, race_fused_fwd_hashed,
                  race_fused_fwd_with_state, race_hash_probs, race_noncausal_backward,
                  select_tile_tokens)

__all__ = [
    "BatchedACE", "CONFIGS", "Config", "RaceFusedFunction", "config_inputs", "make_inputs",
    "race_fused_fwd", "race_fused_fwd_carry", "race_fused_fwd_with_state", "race_noncausal_backward",
    "race_causal_backward", "race_fused_fwd_hashed", "hashed_supported", "HashedRaceFunction",
    "HashProbsFunction", "race_hash_probs", "select_tile_tokens", "causal_v2",
]
