"""Causal RACE attention with the hashing inside (paper Algorithm 1 made causal).

The drop-in for the reference's causal v2 extension
(src/causal_v2/kernels/torch_binding.cpp:1-25, :249-273): the same functions,
argument meanings and errors, running the gfx950 kernels of alg1.hip behind
the C ABI (race_alg1_fwd):

    forward(q, k, v, W, beta, tile_tokens=0, tensor_cores=False) -> o
    forward_debug(q, k, v, W, beta, tile_tokens=0, tensor_cores=False)
        -> (o, prefix_A, prefix_B, final_A, final_B, tile_tokens)
    forward_carry(q, k, v, W, beta, state_A, state_B, tile_tokens=0, tensor_cores=False)
        -> (o, final_A, final_B)      (no counterpart in the reference binding)
    sub_chunk_tokens(head_dim, num_planes, tensor_cores=False) -> C
    select_tile_tokens(batch_heads, seq_len, head_dim, num_planes, num_tables,
                       tensor_cores=False) -> T_blk
    output_pass_smem_bytes(head_dim, num_planes, num_tables, tensor_cores=False) -> bytes
    fits_on_device(head_dim, num_planes, num_tables, tensor_cores=False) -> bool
    precise_carry() -> bool

Math (src/causal_v2/kernels/race_causal_fwd.h:6-10): with Phi(x) the L
tables' corner probabilities softmax_r(beta <tanh(W_l x), c_r>) and A_i, B_i
the inclusive sums of Phi(k_j) and Phi(k_j) (x) v_j over j <= i,
o_i = (Phi(q_i) . B_i) / (Phi(q_i) . A_i).

q, k, v: [B, H, T, d] bf16 GPU tensors, contiguous, 16-byte aligned, one
shape; W: [L, P, d] fp32 on the same device; beta: a one-element floating
tensor on any device (copied to the GPU as fp32; the kernels read it there).
d in {64, 128}, P in 1..5, L in 1..4.  Invalid inputs raise RuntimeError.

tensor_cores=False runs the fp32-accurate rounding (features as bf16 hi/lo
in every matrix-core product), True the reference v2b's rounding points
(features rounded to bf16 once; the carried state and the masked Gram matrix
hi/lo).  Both run on the MI355X matrix cores.
"""
from __future__ import annotations

import torch

from . import _lib


def forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, W: torch.Tensor, beta: torch.Tensor,
            tile_tokens: int = 0, tensor_cores: bool = False) -> torch.Tensor:
    """o [B, H, T, d] bf16."""
    return _lib.ext().alg1_forward(q, k, v, W, beta, int(tile_tokens), bool(tensor_cores))


def forward_debug(q, k, v, W, beta, tile_tokens: int = 0, tensor_cores: bool = False):
    """(o, prefix_A [B, H, tiles, L, R], prefix_B [B, H, tiles, L, R, d],
    final_A [B, H, L, R], final_B [B, H, L, R, d], tile_tokens): the exclusive
    prefix state at every tile start and the state after all T tokens (fp32)."""
    return _lib.ext().alg1_forward_debug(q, k, v, W, beta, int(tile_tokens), bool(tensor_cores))


def forward_carry(q, k, v, W, beta, state_A, state_B, tile_tokens: int = 0, tensor_cores: bool = False):
    """(o, final_A, final_B): the forward of these tokens continued from a carried
    state, (state_A [B, H, L, R], state_B [B, H, L, R, d]) fp32 as forward_debug
    returns final_A, final_B for the earlier tokens.  Every output sees the sums
    over the earlier tokens plus those of this call up to itself, so splitting a
    sequence anywhere gives the unsplit outputs; the returned state continues
    the next call.  The reference hands its final state off for incremental
    generation (race_causal_fwd.h:20-21) without a function that takes it back;
    this is that function."""
    return _lib.ext().alg1_forward_carry(q, k, v, W, beta, state_A, state_B, int(tile_tokens),
                                         bool(tensor_cores))


def sub_chunk_tokens(head_dim: int, num_planes: int, tensor_cores: bool = False) -> int:
    return _lib.ext().alg1_sub_chunk_tokens(int(head_dim), int(num_planes), bool(tensor_cores))


def select_tile_tokens(batch_heads: int, seq_len: int, head_dim: int, num_planes: int,
                       num_tables: int, tensor_cores: bool = False) -> int:
    return _lib.ext().alg1_select_tile_tokens(int(batch_heads), int(seq_len), int(head_dim),
                                              int(num_planes), int(num_tables), bool(tensor_cores))


def output_pass_smem_bytes(head_dim: int, num_planes: int, num_tables: int,
                           tensor_cores: bool = False) -> int:
    """Dynamic LDS of the output pass in bytes."""
    return _lib.ext().alg1_output_lds_bytes(int(head_dim), int(num_planes), int(num_tables),
                                            bool(tensor_cores))


def fits_on_device(head_dim: int, num_planes: int, num_tables: int, tensor_cores: bool = False) -> bool:
    return _lib.ext().alg1_fits_on_device(int(head_dim), int(num_planes), int(num_tables),
                                          bool(tensor_cores))


def precise_carry() -> bool:
    """The carried state enters every product as bf16 hi/lo in both variants."""
    return True
