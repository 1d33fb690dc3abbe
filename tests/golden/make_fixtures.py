"""Write the known-answer fixtures used by the oracle and GPU tests.

The inputs are the reference tests' explicit fixtures; the expected values
come from the closed forms those tests assert, evaluated here in float64
with plain numpy (no reference code is imported or run):

* extreme_logits.json -- tests/ops/test_address_numerics.py:83-102: logits of
  magnitude ~1000 (U=2, P=3, T=2). Expected top-K weights are
  exp(s - r * logsumexp(selected s)) with s the Kronecker sum of the per-digit
  log-softmax (digit 0 least significant), for K in {1, 4, 9} and
  r in {0, 0.5, 1}. Stored as a dense (T, A) weight map per case so that the
  order of tied entries does not matter.
* inactive.json -- tests/ops/test_address_numerics.py:58-71: every digit -inf
  at t=0, digit 0 all -inf at t=1, active at t=2; inactive addresses must
  get weight 0 (and finite values everywhere).
* product_distribution.json -- tests/ops/test_address_numerics.py:20-56:
  seeded logits (B=2, H=2, U=2, P=3, T=5); expected weights in probability
  space q(c) = p_0[d_0] p_1[d_1] restricted to the top-K and scaled by
  (sum q)^-r, with CAPE positions 3t + b on head 0.

Run: python tests/golden/make_fixtures.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def log_softmax(x, axis):
    m = np.max(x, axis=axis, keepdims=True)
    return (x - m) - np.log(np.sum(np.exp(x - m), axis=axis, keepdims=True))


def topk_sets(scores, k):
    """Indices of the top-k scores, ties by index ascending (stable)."""
    order = np.argsort(-scores, kind="stable")
    return order[:k]


def extreme_logits():
    src = np.array([
        [[1000.0, -1000.0], [999.0, -999.0], [-1000.0, 1000.0]],
        [[1000.0, -1000.0], [998.0, -998.0], [-1000.0, 1000.0]],
    ])  # (U, P, T)
    U, P, T = src.shape
    A = P ** U
    lp = log_softmax(src, axis=1)  # (U, P, T)
    cases = []
    for k in (1, 4, 9):
        for r in (0.0, 0.5, 1.0):
            dense = np.zeros((T, A))
            for t in range(T):
                s = np.array([lp[0, c % P, t] + lp[1, c // P, t] for c in range(A)])
                sel = topk_sets(s, k)
                m = s[sel].max()
                lse = m + np.log(np.sum(np.exp(s[sel] - m)))
                dense[t, sel] = np.exp(s[sel] - r * lse)
            cases.append({"top_k": k, "re_norm": r, "dense": dense.tolist()})
    return {"shape": [1, 1, U, P, T], "addr": src.reshape(-1).tolist(), "A": A, "cases": cases}


def inactive():
    rng = np.random.default_rng(1234)
    src = rng.standard_normal((2, 2, 2, 3, 3))
    src[..., 0] = -np.inf
    src[:, :, 0, :, 1] = -np.inf
    return {"shape": list(src.shape), "addr": [x if np.isfinite(x) else "-inf" for x in src.reshape(-1).tolist()],
            "A": 9, "inactive_t": [0, 1]}


def product_distribution():
    rng = np.random.default_rng(5678)
    B, H, U, P, T = 2, 2, 2, 3, 5
    A = P ** U
    src = rng.standard_normal((B, H, U, P, T))
    positions = (np.arange(T)[None, :] * 3 + np.arange(B)[:, None])  # (B, T)
    probs = np.exp(log_softmax(src, axis=3))
    cases = []
    for k in (1, 4, A):
        for r in (0.0, 0.5, 1.0):
            dense = np.zeros((B, H, T, A))  # indexed by OUTPUT slot (after CAPE)
            for b in range(B):
                for h in range(H):
                    for t in range(T):
                        q = np.array([probs[b, h, 0, c % P, t] * probs[b, h, 1, c // P, t] for c in range(A)])
                        sel = topk_sets(q, k)
                        w = q[sel] / np.sum(q[sel]) ** r
                        shift = positions[b, t] if h < 1 else 0
                        dense[b, h, t, (sel - shift) % A] = w
            cases.append({"top_k": k, "re_norm": r, "dense": dense.reshape(-1).tolist()})
    return {"shape": [B, H, U, P, T], "addr": src.reshape(-1).tolist(), "positions": positions.tolist(),
            "embed_num": 1, "A": A, "cases": cases}


def main():
    for name, fn in (("extreme_logits.json", extreme_logits), ("inactive.json", inactive),
                     ("product_distribution.json", product_distribution)):
        with open(os.path.join(HERE, name), "w") as fh:
            json.dump(fn(), fh)
        print("wrote", name)


if __name__ == "__main__":
    main()
