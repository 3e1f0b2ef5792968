"""Pins the sampling oracle (oracle/sampling.py, qwen3-1.7b/kernels.py:1286-1370) on the CPU:
Philox4x32-10 against the published Random123 known-answer vectors, the uniform map's closed
forms, greedy sampling as the first maximal index, and Gumbel-max frequencies against
softmax(logits / tau)."""

import numpy as np
import pytest

from oracle import sampling as osm

# Random123 kat_vectors (philox4x32, rounds, counter[4], key[2] -> output[4])
KAT = [
    (10, [0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    (10, [0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    (10, [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
    (7, [0, 0, 0, 0], [0, 0], [0x5F6FB709, 0x0D893F64, 0x4F121F81, 0x4F730A48]),
]


@pytest.mark.parametrize("rounds,ctr,key,out", KAT)
def test_philox_known_answers(rounds, ctr, key, out):
    got = osm.philox4x32(*([np.uint64(c)] for c in ctr), *key, rounds=rounds)
    assert [int(w[0]) for w in got] == out


def test_philox_vectorized_matches_scalar():
    ctr = np.arange(1000, 1010, dtype=np.uint64)
    z = np.zeros_like(ctr)
    vec = osm.philox4x32(ctr, z, z, z, 7, 9)
    for i, c in enumerate(ctr):
        one = osm.philox4x32([c], [0], [0], [0], 7, 9)
        assert [int(w[i]) for w in vec] == [int(w[0]) for w in one]


def test_uniform_map_closed_forms():
    u = osm.uniform_from_u32(np.array([0, 1, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF], np.uint64))
    scale = np.float32(4.6566127342e-10)
    assert u[0] == 0.0 and u[4] == 0.0  # 0 and -1 (-(-1) - 1 = 0)
    assert u[1] == scale
    assert u[2] == u[3] < 1.0  # INT_MAX and INT_MIN (-INT_MIN - 1 = INT_MAX) map below 1
    assert u[2] == np.float32(np.float32(2 ** 31 - 1) * scale)


def test_rand_is_uniform():
    u = osm.rand(1234, np.arange(200_000, dtype=np.int64))
    assert u.min() >= 0.0 and u.max() < 1.0
    hist = np.histogram(u, bins=20, range=(0, 1))[0]
    assert np.abs(hist - 10_000).max() < 600  # ~6 sigma
    # the key is the seed: other seeds give other streams, the same seed the same one
    assert not np.array_equal(u[:100], osm.rand(1235, np.arange(100)))
    assert np.array_equal(u[:100], osm.rand(1234, np.arange(100)))


def test_greedy_is_first_argmax():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((6, 5000)).astype(np.float32)
    x[1, [17, 4000]] = 9.0  # tie: the first index wins
    x[2, :] = -np.inf
    x[2, 3333] = -1e30
    x[3, :] = 0.0  # all equal: index 0
    tok, nxt = osm.sample(x, 0.0, 41)
    assert nxt == 42
    assert tok.shape == (6, 1) and tok.dtype == np.int64
    assert tok[1, 0] == 17 and tok[2, 0] == 3333 and tok[3, 0] == 0
    assert np.array_equal(tok[:, 0], np.argmax(x, axis=1))


def test_gumbel_frequencies_follow_softmax():
    # P(token = v) = softmax(logits / tau)[v]
    logits = np.array([0.0, 1.0, 2.0, -1.0, 0.5], np.float32)
    tau = 0.7
    rows = 4000
    counts = np.zeros(5)
    for seed in range(5):
        tok, _ = osm.sample(np.tile(logits, (rows, 1)), tau, seed)
        counts += np.bincount(tok[:, 0], minlength=5)
    n = counts.sum()
    p = np.exp(logits / tau) / np.exp(logits / tau).sum()
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < 25.0  # 4 degrees of freedom: p < 1e-4 under the null
