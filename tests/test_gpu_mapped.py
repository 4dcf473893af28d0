"""GPU parity of the hybrid operator weight_metal::mapped_many
(crates/stark-engine/src/engine/hybrid/weight_metal.rs:376-545): GGUF Q8_0 and
Q4_K blocks (decode_block, weights.rs:2923-3012) and MLX-affine planes
(Weights::affine_row, weights.rs:1284-1309), f32 activations, against the
oracle's sequential f32 sums on the same seeded inputs."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu

F32, F16, BF16 = 0, 1, 30


def _x(rng, m, k, kind="normal"):
    if kind == "bf16":  # exactly bf16-representable (the bench's activations)
        return rng.normal(0, 1, (m, k)).astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000)
    return rng.normal(0, 1, (m, k)).astype(np.float32)


def _packed(oracle, rng, kind, n, k):
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    return oracle.quantize_q8_0(w) if kind == 8 else oracle.quantize_q4_k(w)


def _run_packed(qmm, oracle, kind, n, k, m, seed, xkind="normal"):
    rng = np.random.default_rng(seed)
    blocks = _packed(oracle, rng, kind, n, k)
    x = _x(rng, m, k, xkind)
    x = x.view(np.float32) if x.dtype == np.uint32 else x
    codes = H.to_dev(blocks.ravel())
    op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=codes)] * m, inputs=torch.from_numpy(x.ravel()).cuda(),
                             rows=n, columns=k, format=("packed", kind))
    (out,) = qmm.mapped_many([op])
    got = out.cpu().numpy().reshape(m, n)
    dec = oracle.decode_rows(kind, blocks, n, k)
    for i in range(m):
        want = oracle.hybrid_packed_matvec(kind, blocks, n, k, x[i])
        check(got[i], want, mag=np.abs(dec) @ np.abs(x[i]), label=f"kind{kind} n{n} k{k} m{m} row{i}")


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("n,k", [(64, 256), (48, 512), (300, 1024), (16, 4096), (40, 2304)])
def test_packed_matvec(qmm, oracle, kind, n, k):
    _run_packed(qmm, oracle, kind, n, k, 1, seed=n * 7 + k + kind)


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("m", [2, 3, 5, 8])
def test_packed_small_m(qmm, oracle, kind, m):
    """Views of one matrix with consecutive inputs: one product with M rows."""
    _run_packed(qmm, oracle, kind, 96, 1024, m, seed=m + kind)


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("n,k,m", [(16, 2304, 3), (40, 1280, 8), (300, 256, 6), (48, 4096, 4)])
def test_packed_small_m_ragged(qmm, oracle, kind, n, k, m):
    """Row counts that leave the last pair of 16-row tiles partial or shifted
    back, and K with a partial last pass."""
    _run_packed(qmm, oracle, kind, n, k, m, seed=n + k + m + kind)


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("m", [4, 8])
def test_packed_small_m_runs(qmm, oracle, kind, m):
    """More tile pairs than workgroup slots (N = 39990, K = 1024): a workgroup
    runs three pairs under one activation conversion; the last run holds two
    pairs, the last one shifted back to end at N."""
    _run_packed(qmm, oracle, kind, 39990, 1024, m, seed=500 + m + kind)


@pytest.mark.parametrize("kind", [8, 12])
def test_packed_runs_batch_matches_single(qmm, oracle, kind):
    """Two products of 8 rows in one mapped_many call (runs sized for the
    whole launch) give the bits of two calls of one product each."""
    rng = np.random.default_rng(61 + kind)
    made = []
    for n, k in [(12288, 4096), (24576, 1024)]:
        blocks = _packed(oracle, rng, kind, n, k)
        x = torch.from_numpy(_x(rng, 8, k).ravel()).cuda()
        made.append((n, k, H.to_dev(blocks.ravel()), x))

    def op(n, k, codes, x):
        return qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=codes)] * 8, inputs=x, rows=n, columns=k,
                                   format=("packed", kind))
    both = qmm.mapped_many([op(*t) for t in made])
    alone = [qmm.mapped_many([op(*t)])[0] for t in made]
    for (n, k, _, _), a, b in zip(made, both, alone):
        assert torch.equal(a, b), f"kind{kind} n{n} k{k}"


@pytest.mark.parametrize("kind", [8, 12])
def test_packed_batch_of_mixed_k(qmm, oracle, kind):
    """One mapped_many call with products of different K and M (the launch
    orders them longest K first; every output goes to its own operation)."""
    rng = np.random.default_rng(41 + kind)
    specs = [(96, 1024, 1), (64, 4096, 1), (48, 2048, 6), (80, 4096, 6)]
    ops, wants = [], []
    for n, k, m in specs:
        blocks = _packed(oracle, rng, kind, n, k)
        x = rng.normal(0, 1, (m, k)).astype(np.float32)
        ops.append(qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(blocks.ravel()))] * m,
                                       inputs=torch.from_numpy(x.ravel()).cuda(), rows=n, columns=k,
                                       format=("packed", kind)))
        dec = oracle.decode_rows(kind, blocks, n, k)
        wants.append([(oracle.hybrid_packed_matvec(kind, blocks, n, k, x[i]), np.abs(dec) @ np.abs(x[i]))
                      for i in range(m)])
    outs = qmm.mapped_many(ops)
    for (n, k, m), out, want in zip(specs, outs, wants):
        got = out.cpu().numpy().reshape(m, n)
        for i in range(m):
            check(got[i], want[i][0], mag=want[i][1], label=f"n{n} k{k} m{m} row{i}")


@pytest.mark.parametrize("kind", [8, 12])
def test_packed_bf16_exact_inputs(qmm, oracle, kind):
    _run_packed(qmm, oracle, kind, 256, 4096, 1, seed=5 + kind, xkind="bf16")


def test_packed_q8_0_short_rows(qmm, oracle):
    """Q8_0 rows of 3 blocks (K = 96): rows are not 16-byte aligned."""
    _run_packed(qmm, oracle, 8, 33, 96, 2, seed=3)


def test_empty_mapped_operations_are_rejected(qmm, oracle):
    """parameters_for_input rejects zero rows or columns as invalid dimensions
    (weight_metal.rs:456-466): INVALID_ARGUMENT, also next to a valid op."""
    rng = np.random.default_rng(13)
    blocks = _packed(oracle, rng, 8, 32, 256)
    x = torch.from_numpy(rng.normal(0, 1, 256).astype(np.float32)).cuda()

    def op(rows, columns):
        return qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(blocks.ravel()))], inputs=x,
                                   rows=rows, columns=columns, format=("packed", 8))
    for bad in (op(0, 256), op(32, 0)):
        with pytest.raises(qmm.MatmulError) as e:
            qmm.mapped_many([bad, op(32, 256)])
        assert e.value.status == qmm.INVALID_ARGUMENT


def test_packed_wide_range_inputs(qmm, oracle):
    """f32 activations far from bf16: the result must still hold the bar."""
    rng = np.random.default_rng(11)
    for kind in (8, 12):
        n, k = 64, 1024
        blocks = _packed(oracle, rng, kind, n, k)
        x = (rng.normal(0, 1, k) * np.exp(rng.uniform(-6, 6, k))).astype(np.float32)
        op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(blocks.ravel()))],
                                 inputs=torch.from_numpy(x).cuda(), rows=n, columns=k, format=("packed", kind))
        (out,) = qmm.mapped_many([op])
        want = oracle.hybrid_packed_matvec(kind, blocks, n, k, x)
        dec = oracle.decode_rows(kind, blocks, n, k)
        check(out.cpu().numpy(), want, mag=np.abs(dec) @ np.abs(x), label=f"wide kind{kind}")


def test_packed_rows_per_batch(qmm, oracle):
    """rows_per_batch: batch b of rows multiplies input segment b."""
    rng = np.random.default_rng(21)
    n, k, rpb = 96, 512, 32
    blocks = _packed(oracle, rng, 12, n, k)
    x = rng.normal(0, 1, (n // rpb, k)).astype(np.float32)
    op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(blocks.ravel()))],
                             inputs=torch.from_numpy(x.ravel()).cuda(), rows=n, columns=k, format=("packed", 12),
                             rows_per_batch=rpb)
    (out,) = qmm.mapped_many([op])
    got = out.cpu().numpy()
    rows = blocks.reshape(n, -1)
    for b in range(n // rpb):
        sub = np.ascontiguousarray(rows[b * rpb:(b + 1) * rpb])
        want = oracle.hybrid_packed_matvec(12, sub, rpb, k, x[b])
        dec = oracle.decode_rows(12, sub, rpb, k)
        check(got[b * rpb:(b + 1) * rpb], want, mag=np.abs(dec) @ np.abs(x[b]), label=f"rpb batch {b}")


@pytest.mark.parametrize("bits,group,sdt", [(4, 64, BF16), (8, 64, F16), (4, 128, F32), (8, 32, BF16)])
def test_affine_matvec(qmm, oracle, bits, group, sdt):
    rng = np.random.default_rng(bits * 100 + group + sdt)
    n, k = 80, 1024
    codes = rng.integers(0, 256, n * k * bits // 8, dtype=np.uint8)
    G = k // group
    s = rng.uniform(0.001, 0.01, (n, G)).astype(np.float32)
    b = rng.uniform(-0.05, 0.05, (n, G)).astype(np.float32)
    sp, bp = H.store(oracle, s.ravel(), sdt), H.store(oracle, b.ravel(), sdt)
    x = rng.normal(0, 1, k).astype(np.float32)
    op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(codes), scales=H.to_dev(sp),
                                                        biases=H.to_dev(bp))],
                             inputs=torch.from_numpy(x).cuda(), rows=n, columns=k, format=("affine", sdt, bits, group))
    (out,) = qmm.mapped_many([op])
    want = oracle.hybrid_affine_matvec(codes, sp, bp, sdt, bits, group, n, k, x)
    sf, bf = H.load(oracle, sp, sdt).reshape(n, G), H.load(oracle, bp, sdt).reshape(n, G)
    mag = (np.abs(sf).repeat(group, 1) * (2 ** bits) + np.abs(bf).repeat(group, 1)) @ np.abs(x)
    check(out.cpu().numpy(), want, mag=mag, label=f"affine b{bits} g{group} dt{sdt}")


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("m", [1, 8])
def test_non_finite_input_is_rejected(qmm, oracle, kind, m):
    """The reference's input finite check (weight_metal.rs:435-440) on the
    matrix-core path: an infinity or NaN anywhere in any activation row is
    rejected; the largest finite magnitudes are not."""
    rng = np.random.default_rng(4 + kind + m)
    n, k = 32, 512
    blocks = _packed(oracle, rng, kind, n, k)
    codes = H.to_dev(blocks.ravel())

    def run(x):
        op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=codes)] * m,
                                 inputs=torch.from_numpy(x.ravel()).cuda(), rows=n, columns=k, format=("packed", kind))
        qmm.mapped_many([op])
        torch.cuda.synchronize()

    for bad in (np.inf, -np.inf, np.nan):
        for row, col in ((0, 0), (m - 1, 77), (m // 2, k - 1)):
            x = rng.normal(0, 1, (m, k)).astype(np.float32)
            x[row, col] = bad
            with pytest.raises(qmm.MatmulError) as e:
                run(x)
            assert e.value.status == qmm.INVALID_ARGUMENT, (bad, row, col)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    x[0, 5] = np.finfo(np.float32).max
    x[m - 1, k - 2] = -np.finfo(np.float32).max
    run(x)  # finite: no error
