"""CPU checks of the block-symmetric feature basis of the segment-state chunked path
(trainium-linear-attention_amd/csrc/la_general.hpp): groups (i, J) of 16 features a'_i a'_j, j in
block J, over the dims padded to DP = 16 ceil(d/16) plus the augmented index DP, with weights
1/2 (diagonal block), 1 (above it, and the augmented row).  The weighted feature products must
give p(s) = 1 + s + s^2/2 for every pair of vectors; this restates the table in Python (the
kernels' copy is device code) and checks the identity, the group count and the order."""

import numpy as np
import pytest


def groups(DP):
    """(i, J, weight) in the kernels' i-major order."""
    DB = DP // 16
    g = []
    for i in range(DP):
        for J in range(i // 16, DB):
            g.append((i, J, 0.5 if J == i // 16 else 1.0))
    for J in range(DB + 1):
        g.append((DP, J, 1.0))
    return g


def group_ij(DP, g):
    """The closed form the kernels use to find group g (la_general.hpp group_ij)."""
    DB = DP // 16
    NQ = 8 * DB * (DB + 1)
    if g < NQ:
        start = 0
        for I in range(DB):
            c = DB - I
            if g < start + 16 * c:
                off = g - start
                return 16 * I + off // c, I + off % c
            start += 16 * c
    r = g - NQ
    return DP, (r if r < DB else DB)


def features(x, DP, G):
    xp = np.zeros(DP + 32)
    xp[:x.shape[0]] = x
    xp[DP] = 1.0
    i = np.array([gi for gi, J, _ in G for _ in range(16)])
    j = np.array([16 * J + jj for _, J, _ in G for jj in range(16)])
    w = np.array([wt for _, _, wt in G for _ in range(16)])
    return xp[i] * xp[j], w


@pytest.mark.parametrize("d", [1, 2, 5, 15, 16, 17, 31, 32, 33, 48, 63, 64])
def test_weighted_features_give_p(d):
    rng = np.random.default_rng(d)
    DP = 16 * ((d + 15) // 16)
    G = groups(DP)
    DB = DP // 16
    assert len(G) == 8 * DB * (DB + 1) + DB + 1
    assert all(group_ij(DP, g) == G[g][:2] for g in range(len(G)))
    for _ in range(5):
        a = rng.standard_normal(d) * 0.7
        b = rng.standard_normal(d) * 1.3
        fa, w = features(a, DP, G)
        fb, _ = features(b, DP, G)
        s = a @ b
        assert abs((w * fa) @ fb - (1 + s + s * s / 2)) < 1e-12 * (1 + s * s)


def test_feature_count_against_the_minimal_basis():
    """2640 features at d = 64 against the 2145 of the reference's symmetric map (23 % more MFMA
    work for 16-aligned groups), 288 against 153 at d = 16."""
    for d, want, minimal in ((64, 2640, 2145), (16, 288, 153)):
        assert 16 * len(groups(d)) == want
        assert 1 + d + d * (d + 1) // 2 == minimal


def test_planted_weight_mistake_fails():
    """A weight of 1 on the diagonal blocks (the symmetry factor applied twice) breaks the
    identity: the check above is not vacuous."""
    d, DP = 16, 16
    G = [(i, J, 1.0) for i, J, _ in groups(DP)]
    a, b = np.linspace(-1, 1, d), np.linspace(0.5, -0.3, d)
    fa, w = features(a, DP, G)
    fb, _ = features(b, DP, G)
    s = a @ b
    assert abs((w * fa) @ fb - (1 + s + s * s / 2)) > 1e-3
