"""Benchmark config 2 at its own size: N = 12288, K = 4096, M = 1 and M = 8,
for MLX-affine 8-bit (group 64, bf16 planes, through MatmulKernel::encode)
and GGUF Q8_0 / Q4_K (through the hybrid operator mapped_many,
weight_metal.rs:376-545; decode_block weights.rs:2936-2941, 2993-3012).

Two checks per case:
* every output of the full product against the oracle (MatmulCpuKernel's
  sequential f32 sums, kernel.rs:219-265; the hybrid engine's f32 fold over
  decode_block values) at the bar of tests/tolerances.py;
* bit-exact dequantisation on a sample of columns at the full N: one-hot
  activation rows (x = e_j) make output n the weight dequantised at (n, j),
  compared bitwise with the oracle's s*q + bias_term / decode_block.
Weights are N(0, 0.02) quantized by each format's own rule (the oracle's
quantizers), activations N(0, 1) rounded to bf16 as in the benchmark."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu

N, K = 12288, 4096


@pytest.fixture(scope="module")
def weights():
    rng = np.random.default_rng(12288)
    return rng.normal(0, 0.02, (N, K)).astype(np.float32)


def _bf16_rows(O, rng, m):
    return H.activations(O, rng, m, K, H.BF16)


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("m", [1, 8])
def test_config2_mlx_u8_full(qmm, oracle, weights, m, layout):
    rng = np.random.default_rng(100 + m + layout)
    codes, s, b = oracle.quantize_affine(weights, 8, 64, layout)
    codes, s, b = codes.ravel(), s.ravel(), b.ravel()
    x = _bf16_rows(oracle, rng, m)
    G = K // 64
    st, want = oracle.matmul(a=x, m=m, n=N, k=K, codes=codes, scales=s, correction_data=b, layout=layout,
                             row_count=N, group_count=G, bits=8, group_size=64, output_dt=H.F32, threads=8)
    assert st == 0
    d = torch.full((m * N,), float("nan"), dtype=torch.float32, device="cuda")
    dcodes = H.to_dev(codes)
    args = qmm.MatmulArguments(a=H.to_dev(x), m=m, n=N, k=K, d=d, b=qmm.QuantizedB(
        codes=dcodes, scales=H.to_dev(s), params=qmm.QuantParams(layout, N, G), mode=qmm.MODE_U8,
        correction_data=H.to_dev(b)))
    qmm.MatmulKernel(H.BF16, H.BF16, H.F32).encode(args)
    torch.cuda.synchronize()
    # tolerance magnitude sum_k |w x|, |w| <= |s| q + |b| (8-bit codes are the bytes)
    sp = H.load(oracle, s, H.BF16).reshape((N, G) if layout == 0 else (G, N)).astype(np.float32)
    bp = H.load(oracle, b, H.BF16).reshape(sp.shape).astype(np.float32)
    sp, bp = (sp, bp) if layout == 0 else (sp.T, bp.T)
    wabs = np.abs(np.repeat(sp, 64, 1)) * codes.reshape(N, K) + np.abs(np.repeat(bp, 64, 1))
    mag = np.abs(H.load(oracle, x, H.BF16).reshape(m, K)) @ wabs.T
    check(H.from_dev(d, np.float32), want, mag=mag, label=f"config2 u8 m{m} layout{layout}")

    # bit-exact dequantisation on sampled columns, every output row
    cols = np.array(sorted(set([0, 1, 2, 3, 63, 64, 255, 256, K // 2, K - 2, K - 1]) |
                           set(rng.choice(K, 13, replace=False).tolist())), np.int64)
    cols = np.resize(cols, (len(cols) + m - 1) // m * m)
    onehot = np.zeros((len(cols), K), np.float32)
    onehot[np.arange(len(cols)), cols] = 1.0
    xb = H.store(oracle, onehot.ravel(), H.BF16)
    st, wexact = oracle.matmul(a=xb, m=len(cols), n=N, k=K, codes=codes, scales=s, correction_data=b, layout=layout,
                               row_count=N, group_count=G, bits=8, group_size=64, output_dt=H.F32, threads=8)
    assert st == 0
    xdev = H.to_dev(xb)
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.F32)
    outs = []
    for c0 in range(0, len(cols), m):
        o = torch.full((m * N,), float("nan"), dtype=torch.float32, device="cuda")
        kern.encode(qmm.MatmulArguments(a=xdev, a_offset=c0 * K, m=m, n=N, k=K, d=o, b=args.b))
        outs.append(o)
    torch.cuda.synchronize()
    got = torch.cat(outs).cpu().numpy()
    wexact = np.asarray(wexact, np.float32)
    bad = got.view(np.uint32) != wexact.view(np.uint32)
    assert not bad.any(), f"config2 u8 m{m}: {int(bad.sum())} dequantised weights differ"


def _gguf(qmm, oracle, kind, blocks, x):
    m = x.shape[0]
    op = qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=H.to_dev(blocks))] * m,
                             inputs=torch.from_numpy(np.ascontiguousarray(x).ravel()).cuda(), rows=N, columns=K,
                             format=("packed", kind))
    (out,) = qmm.mapped_many([op])
    return out.cpu().numpy().reshape(m, N)


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("m", [1, 8])
def test_config2_gguf_full(qmm, oracle, weights, kind, m):
    rng = np.random.default_rng(200 + kind + m)
    blocks = (oracle.quantize_q8_0(weights) if kind == 8 else oracle.quantize_q4_k(weights)).ravel()
    x = H.load(oracle, _bf16_rows(oracle, rng, m), H.BF16).astype(np.float32).reshape(m, K)
    got = _gguf(qmm, oracle, kind, blocks, x)
    dec = oracle.decode_rows(kind, blocks, N, K)
    absdec = np.abs(dec)
    for i in range(m):
        want = oracle.hybrid_packed_matvec(kind, blocks, N, K, x[i])
        check(got[i], want, mag=absdec @ np.abs(x[i]), label=f"config2 kind{kind} m{m} row{i}")

    # bit-exact dequantisation: identity blocks of m one-hot rows over sampled columns
    cols = np.array(sorted(set([0, 1, 31, 32, 33, 127, 128, 255, 256, K - 1]) |
                           set(rng.choice(K, 14, replace=False).tolist())), np.int64)
    cols = np.resize(cols, (len(cols) + m - 1) // m * m)
    codes = H.to_dev(blocks)
    ops = []
    for c0 in range(0, len(cols), m):
        oh = np.zeros((m, K), np.float32)
        oh[np.arange(m), cols[c0:c0 + m]] = 1.0
        ops.append(qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=codes)] * m,
                                       inputs=torch.from_numpy(oh.ravel()).cuda(), rows=N, columns=K,
                                       format=("packed", kind)))
    g = np.concatenate([o.cpu().numpy().reshape(m, N) for o in qmm.mapped_many(ops)])
    w = np.ascontiguousarray(dec[:, cols].T)
    # +0 and -0 weights reach no output differently (sums start at +0.0)
    bad = (g.view(np.uint32) != w.view(np.uint32)) & ~((g == 0) & (w == 0))
    assert not bad.any(), f"config2 kind{kind} m{m}: {int(bad.sum())} dequantised weights differ"
