"""GPU UnifiedSampling (stark_qmm_unified_sampling) against the oracle's
restatement of unified_sampling.rs:14-117 on the reference's own test
distribution (sampling_test.rs:86-160: per case N(mean in [-100, 100], sd in
[24, 64]) logits, batch 1..7, vocab 1..123456, random bitmasks, temperature
0.05..4, top_k 1..vocab, top_p 0.01..1, min_p 0..1), token for token, as the
reference compares its GPU backend with its CPU one. Greedy rows are exact
by construction; Gumbel rows share the Philox noise bit for bit and differ only
in the device's logf (a last-bit difference can flip only a near-exact tie of
two noisy logits) and in the top-p mass summation order (only where a prefix
mass lands within about 1e-6 of p)."""
import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu
F32, BF16 = H.F32, H.BF16


def _case(oracle, rng, batch, vocab, dt, bitmask):
    mean, sd = rng.uniform(-100, 100), rng.uniform(24, 64)
    x = H.store(oracle, rng.normal(mean, sd, batch * vocab).astype(np.float32), dt)
    words = (vocab + 31) // 32
    mask = rng.integers(0, 2 ** 32, batch * words, dtype=np.uint64).astype(np.uint32) if bitmask else None
    seeds = rng.integers(0, 2 ** 63, batch, dtype=np.uint64)
    return x, mask, seeds


def _run(qmm, x, dt, vocab, batch, method, seeds, mask):
    out = qmm.unified_sampling(H.to_dev(x), dt, vocab, batch, method,
                               seeds=None if seeds is None else torch.from_numpy(seeds.view(np.int64)).cuda(),
                               bitmask=None if mask is None else H.to_dev(mask))
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("vocab,batch", [(1, 3), (63, 7), (4097, 2), (123456, 3), (151936, 1)])
@pytest.mark.parametrize("bitmask", [False, True])
def test_greedy(qmm, oracle, dt, vocab, batch, bitmask):
    rng = np.random.default_rng(vocab + batch + dt + bitmask)
    x, mask, _ = _case(oracle, rng, batch, vocab, dt, bitmask)
    want = oracle.unified_sampling(x, batch, vocab, t_dt=dt, bitmask=mask)
    got = _run(qmm, x, dt, vocab, batch, qmm.SamplingMethod(), None, mask)
    assert np.array_equal(got, want)


OPTIONS = [dict(), dict(temperature=0.7), dict(top_k=1), dict(top_k=40), dict(top_p=0.9), dict(top_p=0.05),
           dict(min_p=0.05), dict(min_p=1.0), dict(temperature=4.0, top_p=0.95),
           dict(temperature=0.05, top_k=64, top_p=0.5, min_p=0.1), dict(temperature=1.5, top_k=5000, min_p=0.0),
           dict(top_p=1.0)]


@pytest.mark.parametrize("opts", OPTIONS, ids=[str(o) for o in OPTIONS])
@pytest.mark.parametrize("dt", [F32, BF16])
def test_stochastic(qmm, oracle, opts, dt):
    rng = np.random.default_rng(len(str(opts)) * 7 + dt)
    for vocab, batch, bitmask in ((1000, 7, False), (123456, 2, True), (151936, 2, False)):
        if opts.get("top_k", 0) > vocab:
            continue
        x, mask, seeds = _case(oracle, rng, batch, vocab, dt, bitmask)
        want = oracle.unified_sampling(x, batch, vocab, t_dt=dt, seeds=seeds, bitmask=mask, **opts)
        got = _run(qmm, x, dt, vocab, batch, qmm.SamplingMethod(stochastic=True, **opts), seeds, mask)
        assert np.array_equal(got, want), (vocab, got, want)


def test_flat_logits_top_p_and_ties(qmm, oracle):
    """Many equal logits (top-p and top-k cut inside a run of ties, which the
    index order decides) and a flat row where most of the vocabulary is kept."""
    rng = np.random.default_rng(5)
    vocab, batch = 5000, 4
    x = np.round(rng.normal(0, 2, (batch, vocab))).astype(np.float32)
    seeds = rng.integers(0, 2 ** 63, batch, dtype=np.uint64)
    for opts in (dict(top_k=700), dict(top_p=0.3), dict(top_p=0.99, temperature=3.0), dict(min_p=0.2)):
        want = oracle.unified_sampling(x.ravel(), batch, vocab, seeds=seeds, **opts)
        got = _run(qmm, x.ravel(), F32, vocab, batch, qmm.SamplingMethod(stochastic=True, **opts), seeds, None)
        assert np.array_equal(got, want), opts


def test_non_finite_and_validation(qmm, oracle):
    x = np.zeros(2 * 64, np.float32)
    x[5] = np.nan
    x[64 + 3] = -np.inf
    got = _run(qmm, x, F32, 64, 2, qmm.SamplingMethod(), None, None)
    assert got.tolist() == [0xFFFFFFFF, 0xFFFFFFFF]
    d = H.to_dev(np.zeros(64, np.float32))
    for m in (qmm.SamplingMethod(stochastic=True, temperature=0.0), qmm.SamplingMethod(stochastic=True, top_k=65),
              qmm.SamplingMethod(stochastic=True, top_k=0), qmm.SamplingMethod(stochastic=True, top_p=1.1),
              qmm.SamplingMethod(stochastic=True, min_p=-0.5), qmm.SamplingMethod(temperature=float("inf"))):
        with pytest.raises(qmm.MatmulError):
            qmm.unified_sampling(d, F32, 64, 1, m, seeds=torch.zeros(1, dtype=torch.int64, device="cuda"))
    with pytest.raises(qmm.MatmulError):
        qmm.unified_sampling(d, F32, 0, 1)


def _ref_masses(x):
    """The reference's running top-p masses (unified_sampling.rs:85-97) in f32:
    mass[r] = sum over the first r sorted logits of exp(x - max) / norm."""
    order = sorted(range(len(x)), key=lambda i: (-float(x[i]), i))
    v = np.asarray(x, np.float32)[order]
    t = np.exp(v - v[0]).astype(np.float32)
    norm = np.float32(0)
    for u in t:
        norm = np.float32(norm + u)
    mass, out = np.float32(0), [np.float32(0)]
    for u in t:
        mass = np.float32(mass + np.float32(u / norm))
        out.append(mass)
    return out


def test_top_p_mass_on_the_boundary(qmm, oracle):
    """Top-p where the reference's f32 prefix mass lands exactly on p (or one
    f32 step from it): the kept prefix must be the reference's, so the
    sampled tokens match over many seeds. Equal logits give terms of exactly 1
    (3 logits with p = f32(2/3): the f32 mass after two is f32(2/3), which
    stops there, while the exact mass 2/3 is below f32(2/3)); the random rows
    take p as the reference's own mass after r logits and the next f32 above."""
    rng = np.random.default_rng(77)
    batch = 96
    seeds = rng.integers(0, 2 ** 63, batch, dtype=np.uint64)
    cases = [(np.zeros(3, np.float32), np.float32(2.0 / 3.0)),
             (np.zeros(10, np.float32), np.float32(0.3)),
             (np.zeros(10, np.float32), np.float32(0.7)),
             (np.zeros(7, np.float32), np.float32(3.0 / 7.0))]
    for v in (50, 3000):
        x = rng.normal(0, 1.0, v).astype(np.float32)
        masses = _ref_masses(x)
        for r in (1, 2, 3):
            cases.append((x, masses[r]))
            cases.append((x, np.nextafter(masses[r], np.float32(2))))
    for x, p in cases:
        vocab = x.size
        rows = np.tile(x, batch)
        want = oracle.unified_sampling(rows, batch, vocab, seeds=seeds, top_p=float(p))
        got = _run(qmm, rows, F32, vocab, batch, qmm.SamplingMethod(stochastic=True, top_p=float(p)), seeds, None)
        assert np.array_equal(got, want), (vocab, float(p), got, want)
