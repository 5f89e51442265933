"""The identify oracle (pyoracle.registry_topk) pinned without a reference
function to run: the reference has no identify (README.md:15 promises it), so
its scoring is pinned to the reference's verify rule (src/model.cpp:65-78,
distance = 1 - sum(ea*eb) in double), to an exact brute force (math.fsum of
the exact f64 products), to the closed form that an L2-normalised embedding is
its own best match with score 1, and to the tie rule (lower row first)."""
import math

import numpy as np

import pyoracle as O


def _unit(rng, n, d):
    x = rng.standard_normal((n, d)).astype(np.float32)
    return (x / np.linalg.norm(x, axis=1, keepdims=True)).astype(np.float32)


def test_registry_scores_are_one_minus_verify_distance_and_exact():
    rng = np.random.default_rng(3)
    q, reg = _unit(rng, 4, 256), _unit(rng, 50, 256)
    idx, score = O.registry_topk(q, reg, 50)
    for b in range(4):
        for j in range(50):
            n = idx[b, j]
            exact = math.fsum(float(a) * float(c) for a, c in zip(q[b], reg[n]))
            assert abs(score[b, j] - exact) <= 1e-15
            assert abs((1.0 - score[b, j]) - O.verify_distance(q[b], reg[n])) <= 1e-15
        # a full ranking: scores non-increasing and every row present once
        assert np.all(np.diff(score[b]) <= 0) and sorted(idx[b].tolist()) == list(range(50))


def test_registry_self_match_and_ties():
    rng = np.random.default_rng(5)
    reg = _unit(rng, 40, 192)
    reg[30] = reg[7]          # duplicate row: the tie goes to the lower index
    q = reg[[7, 12, 39]]
    idx, score = O.registry_topk(q, reg, 3)
    assert idx[0, 0] == 7 and idx[0, 1] == 30 and score[0, 0] == score[0, 1]
    assert idx[1, 0] == 12 and idx[2, 0] == 39
    assert np.all(np.abs(score[:, 0] - 1.0) < 1e-6)
