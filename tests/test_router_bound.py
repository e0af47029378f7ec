"""The two-phase router's candidate rule (CPU).

k_route_mfma (kappa_amd/csrc/route.hip) computes every logit on the matrix cores,
L~ = L + eps with |eps| <= delta_e = c * ||x|| * ||r_e|| (+1e-30), takes tau = the
K-th largest of lo = L~ - delta, keeps the candidates {e : hi_e = L~_e + delta_e >= tau},
recomputes their canonical logits L and ranks them (value descending, ties to the
lower expert index, as lax.top_k, kappa/qwen3/ffn_moe.py:51). The claim: whatever
eps within the bound, the first K of that ranking are the top K of L. This restates
the rule in float32 numpy and checks it against a stable sort with planted exact
ties and near ties at the K-th place and eps pushed to the edge of the bound in the
worst direction; a rule with half the bound (a plausible mistake) fails the same
cases.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def key(v: np.ndarray) -> np.ndarray:
    """The kernel's order-preserving float key (-0.0 keyed as +0.0)."""
    v = np.where(v == 0, F32(0), v).astype(F32)
    u = v.view(np.uint32)
    return np.where(u >> 31, ~u, u | np.uint32(0x80000000)).astype(np.uint32)


def select(L: np.ndarray, L_approx: np.ndarray, delta: np.ndarray, K: int) -> np.ndarray:
    """The kernel's two phases for one token: candidates from the bound, then the
    rank among the candidates' exact logits."""
    lo = (L_approx - delta).astype(F32)
    hi = (L_approx + delta).astype(F32)
    thr = np.sort(key(lo))[::-1][K - 1]
    cand = np.nonzero(key(hi) >= thr)[0]
    assert len(cand) >= K
    # value descending, ties to the lower index (np.lexsort: last key is primary)
    order = np.lexsort((cand, -L[cand].astype(np.float64)))
    return cand[order[:K]]


def reference_topk(L: np.ndarray, K: int) -> np.ndarray:
    return np.lexsort((np.arange(len(L)), -L.astype(np.float64)))[:K]


def planted_token(rng, E: int, K: int, kind: str):
    """Exact logits with a tie or near tie across the K-th place."""
    L = (rng.standard_normal(E) * 0.9).astype(F32)
    order = np.argsort(-L)
    kth, nxt = order[K - 1], order[K]
    if kind == "tie":
        L[nxt] = L[kth]
    elif kind == "near":
        L[nxt] = np.nextafter(L[kth], F32(-np.inf))
    elif kind == "near_up":  # the lower-ranked one just above
        L[nxt] = np.nextafter(L[kth], F32(np.inf))
    elif kind == "band":  # several experts within a few ulps of the K-th
        for j in range(K - 3, K + 3):
            L[order[j]] = L[kth] + F32(1e-7) * (j - K)
    return L


def adversarial(L: np.ndarray, delta: np.ndarray, K: int, scale: float) -> np.ndarray:
    """eps at scale * delta: the true top K pushed down, the rest pushed up."""
    top = np.zeros(len(L), bool)
    top[reference_topk(L, K)] = True
    eps = np.where(top, -delta, delta) * scale
    return (L.astype(np.float64) + eps).astype(F32)


def _delta(rng, E, D):
    c = F32(np.ldexp(4.0 * D + 512.0, -24))
    nx = F32(np.sqrt(D))
    rn = (np.abs(rng.standard_normal(E)) * 0.02 * np.sqrt(D)).astype(F32) + F32(0.5)
    return (c * nx * rn + F32(1e-30)).astype(F32)


def test_candidates_hold_the_top_k_at_the_edge_of_the_bound():
    rng = np.random.default_rng(0)
    E, K, D = 128, 8, 2048
    n = 0
    for kind in ("tie", "near", "near_up", "band", "none"):
        for _ in range(200):
            L = planted_token(rng, E, K, kind)
            delta = _delta(rng, E, D)
            want = reference_topk(L, K)
            for scale in (0.999, -0.999, 0.0, 0.5):
                got = select(L, adversarial(L, delta, K, scale), delta, K)
                np.testing.assert_array_equal(got, want)
                n += 1
            # random eps inside the bound
            eps = (rng.uniform(-0.999, 0.999, E) * delta).astype(F32)
            np.testing.assert_array_equal(select(L, (L + eps).astype(F32), delta, K), want)
    assert n == 4000


def test_all_equal_logits_select_the_first_k():
    E, K = 128, 8
    L = np.zeros(E, F32)
    delta = np.full(E, F32(1e-3))
    for scale in (0.999, -0.999):
        np.testing.assert_array_equal(select(L, adversarial(L, delta, K, scale), delta, K), np.arange(K))


def test_half_the_bound_misses():
    """The candidate rule with delta / 2 (a plausible mistake, e.g. a dropped factor
    of two for the canonical order's own rounding): eps at the true bound then loses
    an expert of the top K on planted near ties."""
    rng = np.random.default_rng(1)
    E, K, D = 128, 8, 2048
    misses = 0
    for _ in range(200):
        L = planted_token(rng, E, K, "near")
        delta = _delta(rng, E, D)
        got = select(L, adversarial(L, delta, K, 0.999), delta / 2, K)
        misses += not np.array_equal(got, reference_topk(L, K))
    assert misses > 100
