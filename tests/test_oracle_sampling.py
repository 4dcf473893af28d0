"""Pins of the oracle's sampling restatement (oracle/stark_oracle.c,
so_unified_sampling after unified_sampling.rs:14-117 and gumbel.rs):

* Philox4x32-10 against the published known-answer vectors of the algorithm
  (Salmon et al., SC'11; the Random123 distribution's kat_vectors);
* unit_interval against the reference's own test (gumbel_test.rs:8-13);
* revidx gives every logit of a row its own (counter, word) pair;
* greedy sampling against numpy's first-maximum argmax, the bitmask, the
  non-finite and all-masked rows; the filters against brute force on small
  rows (sorted-order semantics written from the definitions); Gumbel sampling
  without filters against argmax(x + noise) with the noise in float64.
"""
import numpy as np
import pytest

F32, BF16 = 0, 30


@pytest.mark.parametrize("ctr,key,want", [
    ([0, 0, 0, 0], [0, 0], [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]),
    ([0xffffffff] * 4, [0xffffffff] * 2, [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]),
    ([0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344], [0xa4093822, 0x299f31d0],
     [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]),
])
def test_philox_known_answers(oracle, ctr, key, want):
    assert oracle.philox4x32_10(ctr, key).tolist() == want


def test_unit_interval(oracle):
    u = oracle.lib().so_unit_interval
    assert u(0xFFFFFFFF) == np.float32(1.0 - 2.0 ** -24)
    assert u(0) == np.float32(2.0 ** -24) and u(255) == np.float32(2.0 ** -24)


@pytest.mark.parametrize("vocab", [1, 1000, 4096, 4097, 151936])
def test_revidx_distinct(vocab):
    i = np.arange(vocab, dtype=np.int64)
    t, blk = i % 1024, i // 1024
    offset = ((vocab + 4095) // 4096) * t + blk // 4
    pairs = offset * 4 + blk % 4
    assert np.unique(pairs).size == vocab


def _rows(rng, batch, vocab):
    mean = rng.uniform(-100, 100)
    sd = rng.uniform(24, 64)
    return rng.normal(mean, sd, (batch, vocab)).astype(np.float32)


def test_greedy(oracle):
    rng = np.random.default_rng(1)
    x = _rows(rng, 4, 3000)
    x[1, 100] = x[1, 200] = x[1].max() + 1  # tie: the lower index wins
    got = oracle.unified_sampling(x.ravel(), 4, 3000)
    assert got.tolist() == [int(np.argmax(r)) for r in x]
    bad = x.copy()
    bad[2, 7] = np.nan
    bad[3, 9] = np.inf
    got = oracle.unified_sampling(bad.ravel(), 4, 3000)
    assert got[2] == 0xFFFFFFFF and got[3] == 0xFFFFFFFF
    words = (3000 + 31) // 32
    mask = rng.integers(0, 2 ** 32, (4, words), dtype=np.uint64).astype(np.uint32)
    mask[3] = 0  # everything masked: nothing finite left
    got = oracle.unified_sampling(x.ravel(), 4, 3000, bitmask=mask)
    for b in range(3):
        allowed = np.array([(mask[b, i // 32] >> (i % 32)) & 1 for i in range(3000)], bool)
        assert got[b] == int(np.argmax(np.where(allowed, x[b], -np.inf)))
    assert got[3] == 0xFFFFFFFF


def _brute(oracle, x, seed, temperature=None, top_k=None, top_p=None, min_p=None):
    v = x.astype(np.float32).copy()
    if temperature is not None:
        r = np.float32(1.0) / np.float32(temperature)
        if np.any(np.isfinite(v) & ~np.isfinite(v * r)):
            v = v - v.max()
        v = (v * r).astype(np.float32)
    order = sorted(range(v.size), key=lambda i: (-v[i], i))
    mx = v[order[0]]
    norm = np.float32(0)
    for i in order:
        norm = np.float32(norm + np.exp(np.float32(v[i] - mx), dtype=np.float32))
    kept = np.full(v.size, -np.inf, np.float32)
    mass = np.float32(0)
    for rank, i in enumerate(order):
        if (top_k is not None and rank >= top_k) or (top_p is not None and mass >= np.float32(top_p)) or \
                (min_p is not None and v[i] < mx + np.log(np.float32(min_p), dtype=np.float32)):
            break
        kept[i] = v[i]
        mass = np.float32(mass + np.float32(np.exp(np.float32(v[i] - mx), dtype=np.float32) / norm))
    g = np.array([oracle.gumbel(seed, i, v.size) for i in range(v.size)], np.float32)
    s = kept + g
    return int(np.argmax(s)) if np.isfinite(s.max()) else 0xFFFFFFFF


@pytest.mark.parametrize("opts", [dict(), dict(top_k=5), dict(top_p=0.5), dict(min_p=0.3),
                                  dict(temperature=2.0, top_k=20, top_p=0.9),
                                  dict(temperature=0.5, min_p=0.01), dict(top_k=1)])
def test_stochastic_against_brute_force(oracle, opts):
    rng = np.random.default_rng(len(str(opts)))
    vocab, batch = 257, 6
    x = rng.normal(0, 3, (batch, vocab)).astype(np.float32)
    seeds = rng.integers(0, 2 ** 63, batch, dtype=np.uint64)
    got = oracle.unified_sampling(x.ravel(), batch, vocab, seeds=seeds, **opts)
    for b in range(batch):
        assert got[b] == _brute(oracle, x[b], int(seeds[b]), **opts), (opts, b)
    if opts.get("top_k") == 1:
        assert got.tolist() == [int(np.argmax(r)) for r in x]
