"""Activation dynamic range of the matrix-core kernels.

The matrix-core kernels stage each activation group as x * 2^E with a
per-group exponent E (the group's largest |x| lands in [2^62, 2^64)) and scale
the group's sum back with ldexp by 133 - E, so every finite activation is
handled: these tests drive activations from 2^-100 to 2^70, bf16 subnormals
and groups that mix magnitudes, on every matrix-core kernel, against the
oracle's sequential f32 sums (MatmulCpuKernel::encode,
crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:168-285; GGUF:
decode_block + the reference's f32 sum, weights.rs:2533-2550), to the usual
parity bar.

Non-finite activations: the kernels compute the reference GPU GEMV's factored
form per group, fma(b, sum(x), fma(s, sum(x*q), acc))
(crates/stark-engine/src/backends/metal/kernel/matmul/gemv/common/quant_slice.h:42-205),
so an infinite activation gives a non-finite output exactly where the CPU
reference's does, with the same sign where both are infinite, and NaN where
the factored form meets Inf - Inf or Inf * 0 (a zero code or a bias term of the
opposite sign) and the CPU reference's per-element product gives +-Inf.
"""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu


def wide_x(rng, m, k, lo=-100, hi=70, gs=64):
    """N(0,1) values scaled by a random power of two per 32 values, plus
    groups that mix the extremes and a few bf16 subnormals."""
    e = rng.integers(lo, hi + 1, (m, k // 32))
    x = rng.normal(0, 1, (m, k)) * np.exp2(np.repeat(e, 32, axis=1))
    x[:, :gs] = rng.normal(0, 1, (m, gs)) * np.exp2(rng.integers(lo, hi + 1, (m, gs)))  # mixed group
    x[:, gs:gs + 8] = rng.integers(1, 127, (m, 8)) * 2.0 ** -133 * rng.choice([-1, 1], (m, 8))  # subnormals
    return x.astype(np.float32).ravel()


def _affine(Q, O, x, *, m, n, k, bits=4, gs=64, layout=1, seed=0, label="", nonfinite=False):
    rng = np.random.default_rng(seed)
    W = H.affine_weights(O, rng, n, k, bits, gs, layout, 1, H.BF16, quantizer=False)
    xb = H.store(O, x, H.BF16)
    G = k // gs
    mode = Q.MODE_U4 if bits == 4 else Q.MODE_U8
    st, want = O.matmul(a=xb, m=m, n=n, k=k, codes=W["codes"], scales=W["scales"], correction_data=W["corr"],
                        layout=layout, row_count=n, group_count=G, bits=bits, group_size=gs, output_dt=H.F32,
                        threads=8)
    assert st == 0
    d = torch.zeros(m * n, dtype=torch.float32, device="cuda")
    args = Q.MatmulArguments(
        a=H.to_dev(xb), m=m, n=n, k=k, d=d,
        b=Q.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=Q.QuantParams(layout, n, G),
                       mode=mode, group_size=gs, correction_data=H.to_dev(W["corr"])))
    Q.MatmulKernel(H.BF16, H.BF16, H.F32).encode(args)
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    want = np.asarray(want, np.float32)
    if nonfinite:
        _check_nonfinite(got, want, label)
        return
    assert np.isfinite(want).all()
    mag = H.dequant_magnitude(O, W["codes"], W["scales"], W["corr"], n, k, bits, gs, layout, 1, H.BF16, xb, H.BF16, m)
    check(got, want, mag=mag, label=label)


def _check_nonfinite(got, want, label):
    fin_g, fin_w = np.isfinite(got), np.isfinite(want)
    assert np.array_equal(fin_g, fin_w), f"{label}: finite pattern differs"
    both_inf = np.isinf(got) & np.isinf(want)
    assert np.array_equal(np.sign(got[both_inf]), np.sign(want[both_inf])), f"{label}: infinity sign differs"
    assert (~fin_w).any()


KERNELS = [
    # (label, m, n, k, bits, gs): the dispatch picks the kernel named
    ("qmv_stream", 1, 96, 4096, 4, 64),
    ("qmv_mfma w4 m1", 1, 48, 2048, 4, 64),
    ("qmv_mfma w4 m1 g32", 1, 48, 2048, 4, 32),
    ("qmv_mfma w4 m1 g128", 1, 48, 2048, 4, 128),
    ("qmv_mfma w4 m2", 2, 48, 4096, 4, 64),
    ("qmv_mfma w4 m4", 4, 48, 4096, 4, 64),
    ("qmv_mfma w8 m1", 1, 64, 4096, 8, 64),
    ("qmv_mfma w8 m4", 4, 64, 4096, 8, 64),
    ("qmv_mfma w8 m16", 16, 64, 2048, 8, 64),
    ("qmv_small_m m8", 8, 96, 4096, 4, 64),
    ("qmv_small_m m16", 16, 96, 2048, 4, 64),
]


@pytest.mark.parametrize("label,m,n,k,bits,gs", KERNELS)
def test_affine_wide_range(qmm, oracle, label, m, n, k, bits, gs):
    rng = np.random.default_rng(sum(map(ord, label)))
    _affine(qmm, oracle, wide_x(rng, m, k, gs=gs), m=m, n=n, k=k, bits=bits, gs=gs, seed=m + k + bits, label=label)


@pytest.mark.parametrize("label,m,n,k,bits,gs", KERNELS)
@pytest.mark.parametrize("e", [-100, 70])
def test_affine_uniform_extreme_scale(qmm, oracle, label, m, n, k, bits, gs, e):
    """Every activation at 2^-100 or 2^70 times N(0,1) (the old fixed x * 2^64
    staging overflowed at |x| >= 2^64 and lost the products below 2^-57)."""
    rng = np.random.default_rng(e + 1000)
    x = (rng.normal(0, 1, m * k) * 2.0 ** e).astype(np.float32)
    _affine(qmm, oracle, x, m=m, n=n, k=k, bits=bits, gs=gs, seed=m + bits, label=f"{label} 2^{e}")


@pytest.mark.parametrize("label,m,n,k,bits,gs", KERNELS[:1] + KERNELS[4:6] + KERNELS[7:10])
def test_affine_infinite_activations(qmm, oracle, label, m, n, k, bits, gs):
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (m, k)).astype(np.float32)
    x[0, 5] = np.inf
    x[m - 1, k - 3] = -np.inf
    if m > 2:
        x[1, :] = rng.normal(0, 1, k)  # a finite row stays finite
    _affine(qmm, oracle, x.ravel(), m=m, n=n, k=k, bits=bits, gs=gs, seed=3, label=label, nonfinite=True)


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("m", [1, 8])
def test_gguf_wide_range(qmm, oracle, kind, m):
    """gguf_mfma with f32 activations from 2^-100 to 2^70 (and f32 subnormals)."""
    rng = np.random.default_rng(kind * 10 + m)
    n, k = 48, 2048
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    blocks = oracle.quantize_q8_0(w) if kind == 8 else oracle.quantize_q4_k(w)
    x = wide_x(rng, m, k, gs=32).reshape(m, k)
    x[:, 100:104] = np.float32(2.0 ** -140)
    op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(blocks.ravel()))] * m,
                             inputs=torch.from_numpy(x.ravel()).cuda(), rows=n, columns=k, format=("packed", kind))
    (out,) = qmm.mapped_many([op])
    got = out.cpu().numpy().reshape(m, n)
    dec = oracle.decode_rows(kind, blocks, n, k)
    for i in range(m):
        want = oracle.hybrid_packed_matvec(kind, blocks, n, k, x[i])
        check(got[i], want, mag=np.abs(dec).astype(np.float64) @ np.abs(x[i]).astype(np.float64),
              label=f"gguf kind {kind} m{m} row {i}")
