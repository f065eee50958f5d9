"""CPU generator of adversarial router logits for the LOWP routing mode
(softmax in bf16, top-k on the bf16 probabilities: fused_moe.py:92-96,
qwen3_moe/__init__.py:473-475).

In that mode the routing indices depend on the exact bf16 bits of every
probability.  Each row built here puts the top-k boundary where those bits
are fragile:

* the k-th and (k+1)-th experts sit one or two logit ulps apart, the
  (k+1)-th with the LOWER index, so a probability rounded up makes a tie that
  the lower index wins;
* three low "trim" experts are set (on the bf16 grid) so that the softmax
  denominator puts one of the two boundary probabilities within about 1e-9
  relative of a bf16 rounding midpoint, i.e. inside the rounding error of
  any fp32 evaluation of exp(l - m) / s.

Whether such a probability rounds up or down is decided by the exact fp32
arithmetic, so GPU routing can equal the oracle's on these rows only if the
two compute the same bits.  Everything here is float64 numpy on the host.
"""
from __future__ import annotations

import numpy as np

import ftm_oracle as O


def _bf16(v: float) -> float:
    return float(O.round_bf16(np.float32([v]))[0])


def _bf16_ulp(v: float) -> float:
    b = int(O.f32_to_bf16_bits(np.float32([abs(v)]))[0])
    return float(O.bf16_bits_to_f32(np.uint16([b + 1]))[0]) - float(O.bf16_bits_to_f32(np.uint16([b]))[0])


def near_midpoint_row(E: int, k: int, rng: np.random.RandomState, target_kth: bool) -> np.ndarray:
    """One row of bf16 logits [E] (as fp32); target_kth: tune the k-th
    probability onto a midpoint, else the (k+1)-th."""
    perm = rng.permutation(E)
    top = perm[: k + 1]
    b_i, a_i = sorted(top[k - 1:k + 1].tolist())  # a: k-th (higher index), b: (k+1)-th (lower index)
    sure, rest = top[: k - 1], perm[k + 1:]
    trims, low = rest[:3], rest[3:]
    l = np.empty(E)
    a = _bf16(rng.uniform(0.26, 0.49))
    l[a_i] = a
    l[b_i] = _bf16(a - _bf16_ulp(a) * rng.randint(1, 3))
    l[sure] = [_bf16(a + rng.uniform(0.05, 1.0)) for _ in sure]
    l[low] = [_bf16(v) for v in rng.randn(len(low)) * 0.5 - 4.0]
    l[trims] = [_bf16(-2.5), _bf16(-8.0), _bf16(-14.0)]
    tgt = a_i if target_kth else b_i
    m = l.max()
    for _ in range(3):
        e = np.exp(l - m)
        p = e[tgt] / e.sum()
        base, u = _bf16(p), _bf16_ulp(p)
        mid = base + u / 2 if p >= base else base - u / 2
        want_s = e[tgt] / mid
        for tr in trims:  # coarse to fine: each trim's bf16 step is ~1e3 x finer than the last
            d = want_s - np.exp(l - m).sum()
            cur = np.exp(l[tr] - m)
            if cur + d > 0:
                l[tr] = _bf16(np.log(cur + d) + m)
    return l.astype(np.float32)


def adversarial_logits(T: int, E: int, k: int, seed: int) -> np.ndarray:
    """[T, E] bf16-exact fp32 logits: even rows tune the k-th probability onto
    a bf16 midpoint, odd rows the (k+1)-th."""
    rng = np.random.RandomState(seed)
    return np.stack([near_midpoint_row(E, k, rng, t % 2 == 0) for t in range(T)])


def midpoint_distance_ulps(p: np.ndarray) -> np.ndarray:
    """Distance of float64 probabilities to the nearest bf16 rounding midpoint,
    in fp32 ulps of the probability."""
    p = np.asarray(p, np.float64)
    bits = O.f32_to_bf16_bits(p.astype(np.float32)).astype(np.int64)
    b = O.bf16_bits_to_f32(bits.astype(np.uint16)).astype(np.float64)
    up = O.bf16_bits_to_f32((bits + 1).astype(np.uint16)).astype(np.float64)
    dn = O.bf16_bits_to_f32((bits - 1).astype(np.uint16)).astype(np.float64)
    d = np.minimum(np.abs(p - (b + up) / 2), np.abs(p - (b + dn) / 2))
    return d / (np.abs(p) * 2.0 ** -23)


def boundary_stats(L: np.ndarray, k: int) -> dict:
    """How adversarial a logits batch is: rows whose k-th or (k+1)-th exact
    probability lies within one fp32 ulp of a bf16 midpoint, and rows whose
    bf16 probabilities tie across the top-k boundary."""
    m = L.max(1, keepdims=True)
    e = np.exp((L - m).astype(np.float64))
    p = e / e.sum(1, keepdims=True)
    order = np.argsort(-p, 1, kind="stable")
    pk = np.take_along_axis(p, order[:, k - 1:k + 1], 1)
    srt = np.sort(O.round_bf16(p.astype(np.float32)), 1)[:, ::-1]
    return {"near_midpoint": int((midpoint_distance_ulps(pk).min(1) < 1.0).sum()),
            "boundary_ties": int((srt[:, k - 1] == srt[:, k]).sum())}
