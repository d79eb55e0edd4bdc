"""Writes tests/golden/race_golden.npz: known-answer vectors from exact arithmetic.

Each case holds float32 inputs and float64 expected outputs computed with
Python's fractions.Fraction -- no floating-point rounding anywhere -- straight
from the definition of the reference's hot span (src/race_baseline.py:45-51):

    causal:     A_t = sum_{j<=t} k_j, B_t = sum_{j<=t} k_j v_j^T,
                out_t[c] = sum_s q_t[s] * B_t[s][c] / (A_t[s] + eps)
    non-causal: the same with sums over all T (analysis/hot-path.md:157-162)

with eps the double nearest 1e-6.  Gradients of the non-causal and causal
cases are computed by forward-mode differentiation with exact dual numbers
(one pass per input element), so they do not share a derivation with the
closed-form VJPs the oracle and the kernels use.

Run: python tests/golden/make_golden.py  (seconds; deterministic)
"""
from __future__ import annotations

import pathlib
from fractions import Fraction

import numpy as np

EPS = Fraction(1e-6)
OUT = pathlib.Path(__file__).resolve().parent / "race_golden.npz"


class Dual:
    """a + b*epsilon with epsilon^2 = 0, over exact rationals."""

    __slots__ = ("a", "b")

    def __init__(self, a, b=Fraction(0)):
        self.a, self.b = a, b

    @staticmethod
    def lift(x):
        return x if isinstance(x, Dual) else Dual(x)

    def __add__(self, o):
        o = Dual.lift(o)
        return Dual(self.a + o.a, self.b + o.b)

    __radd__ = __add__

    def __mul__(self, o):
        o = Dual.lift(o)
        return Dual(self.a * o.a, self.a * o.b + self.b * o.a)

    __rmul__ = __mul__

    def __truediv__(self, o):
        o = Dual.lift(o)
        return Dual(self.a / o.a, (self.b * o.a - self.a * o.b) / (o.a * o.a))


def zero_like(x):
    return Dual(Fraction(0)) if isinstance(x, Dual) else Fraction(0)


def exact_forward(q, k, v, causal):
    """q, k: [T][S], v: [T][d] nested lists of Fraction or Dual. Returns [T][d]."""
    T, S, d = len(q), len(q[0]), len(v[0])
    out = []
    if causal:
        A = [zero_like(q[0][0]) for _ in range(S)]
        B = [[zero_like(q[0][0]) for _ in range(d)] for _ in range(S)]
        for t in range(T):
            for s in range(S):
                A[s] = A[s] + k[t][s]
                for c in range(d):
                    B[s][c] = B[s][c] + k[t][s] * v[t][c]
            row = []
            for c in range(d):
                acc = zero_like(q[0][0])
                for s in range(S):
                    acc = acc + q[t][s] * B[s][c] / (A[s] + EPS)
                row.append(acc)
            out.append(row)
        return out
    A = [sum((k[t][s] for t in range(T)), zero_like(q[0][0])) for s in range(S)]
    B = [[sum((k[t][s] * v[t][c] for t in range(T)), zero_like(q[0][0])) for c in range(d)]
         for s in range(S)]
    for t in range(T):
        out.append([sum((q[t][s] * B[s][c] / (A[s] + EPS) for s in range(S)), zero_like(q[0][0]))
                    for c in range(d)])
    return out


def to_frac(a):
    return [[Fraction(float(x)) for x in row] for row in a]


def probs(rng, T, L, R):
    logits = rng.standard_normal((T, L, R)).astype(np.float32) * np.float32(4.0)
    e = np.exp(logits - logits.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32).reshape(T, L * R)


def case(rng, N, T, L, R, d):
    q = np.stack([probs(rng, T, L, R) for _ in range(N)])
    k = np.stack([probs(rng, T, L, R) for _ in range(N)])
    v = rng.standard_normal((N, T, d)).astype(np.float32)
    return q, k, v


def forward_case(q, k, v, causal):
    out = np.array([[[float(x) for x in row] for row in
                     exact_forward(to_frac(q[n]), to_frac(k[n]), to_frac(v[n]), causal)]
                    for n in range(q.shape[0])])
    return out


def exact_grads(q, k, v, g, causal):
    """Exact d/d(inputs) of sum(g * out) for one stream, by forward-mode duals."""
    T, S = q.shape
    d = v.shape[1]
    qf, kf, vf, gf = to_frac(q), to_frac(k), to_frac(v), to_frac(g)

    def lifted(arr, seed):
        return [[Dual(x, Fraction(1) if (i, j) == seed else Fraction(0)) for j, x in enumerate(row)]
                for i, row in enumerate(arr)]

    def loss(qq, kk, vv):
        o = exact_forward(qq, kk, vv, causal)
        acc = Dual(Fraction(0))
        for t in range(T):
            for c in range(d):
                acc = acc + o[t][c] * gf[t][c]
        return acc.b

    none = (-1, -1)
    dq = np.array([[float(loss(lifted(qf, (t, s)), lifted(kf, none), lifted(vf, none)))
                    for s in range(S)] for t in range(T)])
    dk = np.array([[float(loss(lifted(qf, none), lifted(kf, (t, s)), lifted(vf, none)))
                    for s in range(S)] for t in range(T)])
    dv = np.array([[float(loss(lifted(qf, none), lifted(kf, none), lifted(vf, (t, c))))
                    for c in range(d)] for t in range(T)])
    return dq, dk, dv


def main():
    rng = np.random.default_rng(20261201)
    data = {}
    # Causal and non-causal forward cases: (name, N, T, L, R, d).
    for name, N, T, L, R, d in [("small", 2, 9, 2, 4, 3), ("one_token", 2, 1, 4, 4, 5),
                                ("wide", 1, 12, 4, 16, 8), ("s1", 1, 7, 1, 1, 2)]:
        q, k, v = case(rng, N, T, L, R, d)
        data[f"{name}_q"], data[f"{name}_k"], data[f"{name}_v"] = q, k, v
        data[f"{name}_causal"] = forward_case(q, k, v, True)
        data[f"{name}_noncausal"] = forward_case(q, k, v, False)
    # A case where probsK hits eps exactly: k = fp32(1e-6) in one bucket at t=0.
    q, k, v = case(rng, 1, 5, 1, 4, 2)
    k[0, 0, :] = np.float32(1e-6)
    k[0, 0, 0] = np.float32(1.0) - np.float32(3e-6)
    data["eps_q"], data["eps_k"], data["eps_v"] = q, k, v
    data["eps_causal"] = forward_case(q, k, v, True)
    data["eps_noncausal"] = forward_case(q, k, v, False)
    # Non-causal gradients, one stream.
    q, k, v = case(rng, 1, 6, 2, 2, 3)
    g = rng.standard_normal((1, 6, 3)).astype(np.float32)
    dq, dk, dv = exact_grads(q[0], k[0], v[0], g[0], causal=False)
    data.update(grad_q=q, grad_k=k, grad_v=v, grad_g=g, grad_dq=dq[None], grad_dk=dk[None],
                grad_dv=dv[None], grad_out=forward_case(q, k, v, False))
    # Causal gradients, one stream each (appended last so the cases above keep
    # their random draws).
    for name, T, L, R, d in [("cgrad", 7, 2, 2, 3), ("cgrad_wide", 5, 2, 4, 2)]:
        q, k, v = case(rng, 1, T, L, R, d)
        g = rng.standard_normal((1, T, d)).astype(np.float32)
        dq, dk, dv = exact_grads(q[0], k[0], v[0], g[0], causal=True)
        data.update({f"{name}_q": q, f"{name}_k": k, f"{name}_v": v, f"{name}_g": g,
                     f"{name}_dq": dq[None], f"{name}_dk": dk[None], f"{name}_dv": dv[None]})
    np.savez(OUT, **data)
    print(f"wrote {OUT} ({len(data)} arrays)")


if __name__ == "__main__":
    main()
