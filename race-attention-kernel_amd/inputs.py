"""Seeded synthetic inputs of the benchmark configurations cfg1 .. cfg5.

probsQ and probsK are each a softmax over R of logits ~ N(0, 1) * 4
(temperature 0.25), V ~ N(0, 1), the upstream gradient ~ N(0, 1); generated
in fp32 from one torch.Generator, then rounded to the run's dtype.  On the
CPU generator the values are identical on every machine, which is what lets
the CPU oracle see exactly the GPU's inputs.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

LOGIT_SCALE = 4.0


@dataclass(frozen=True)
class Config:
    name: str
    N: int
    T: int
    L: int
    R: int
    d: int
    dtype: torch.dtype
    causal: bool

    @property
    def S(self) -> int:
        return self.L * self.R


# The benchmark configurations, in order: cfg1 the reference's CPU path,
# cfg2 the headline causal fp32 sweep (T = 512 .. 65536), cfg3 long-context
# bf16, cfg4 non-causal forward + backward, cfg5 large buckets (S = 256).
CONFIGS = {
    "cfg1_cpu_causal_fp32": Config("cfg1_cpu_causal_fp32", 8, 4096, 4, 16, 64, torch.float32, True),
    "cfg2_causal_fp32": Config("cfg2_causal_fp32", 8, 65536, 4, 16, 64, torch.float32, True),
    "cfg3_causal_bf16": Config("cfg3_causal_bf16", 8, 1 << 20, 4, 16, 64, torch.bfloat16, True),
    "cfg4_noncausal_fp32": Config("cfg4_noncausal_fp32", 384, 1024, 4, 16, 64, torch.float32, False),
    "cfg5_causal_bf16_S256": Config("cfg5_causal_bf16_S256", 128, 16384, 8, 32, 128, torch.bfloat16, True),
}
CFG2_T_SWEEP = [1 << p for p in range(9, 17)]          # 512 .. 65536
CFG3_T = [1 << 17, 1 << 18, 1 << 20]


def make_inputs(N: int, T: int, L: int, R: int, d: int, *, seed: int = 0,
                dtype: torch.dtype = torch.float32, device="cpu", gen_device="cpu",
                grad_out: bool = False):
    """(probsQ [N,T,L,R], probsK [N,T,L,R], V [N,T,d][, dOut [N,T,d]]) in ``dtype`` on ``device``.

    gen_device="cpu" gives machine-independent values; "cuda" is faster for
    benchmark-sized inputs.
    """
    g = torch.Generator(device=gen_device).manual_seed(seed)

    def probs():
        logits = torch.randn((N, T, L, R), generator=g, device=gen_device, dtype=torch.float32)
        return torch.softmax(logits * LOGIT_SCALE, dim=-1)

    q = probs()
    k = probs()
    v = torch.randn((N, T, d), generator=g, device=gen_device, dtype=torch.float32)
    out = [q, k, v]
    if grad_out:
        out.append(torch.randn((N, T, d), generator=g, device=gen_device, dtype=torch.float32))
    return tuple(x.to(device=device, dtype=dtype).contiguous() for x in out)


def config_inputs(cfg: Config, T: int | None = None, *, seed: int = 0, device="cpu",
                  gen_device="cpu", grad_out: bool = False, N: int | None = None):
    return make_inputs(N or cfg.N, T or cfg.T, cfg.L, cfg.R, cfg.d, seed=seed, dtype=cfg.dtype,
                       device=device, gen_device=gen_device, grad_out=grad_out)
