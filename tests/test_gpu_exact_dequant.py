"""Bit-exact dequantisation on every production kernel.

An activation row that is one-hot at column j (x = e_j, f32 output) makes each
kernel's output row n equal to the weight it dequantised at (n, j), with no
summation rounding left: the matrix-core kernels compute per group
fma(s, sum(x*q), b*sum(x)) with an exact product, i.e. exactly the
reference's s*q + bias_term (one rounding), and every other group adds +0.
The tests compare those outputs BITWISE with the oracle:

* affine GEMV / verify kernels: the oracle's MatmulCpuKernel restatement with
  the same one-hot rows (kernel.rs:219-265: w = s*q + bias_term in f32; its
  sequential sum of a single nonzero product is that weight);
* the prefill dequant-GEMM: the oracle's bf16-effective linear
  (so_reference_affine_linear_bf16, vision.rs:249-336, whose tree of fmas over
  one nonzero product is bf16_rne(s*q + b)); for the signed / symmetric
  variants the oracle's f32 weight rounded by the oracle's bf16 RNE;
* GGUF Q8_0 / Q4_K (hybrid path): the oracle's decode_block
  (weights.rs:2936-2941, 2993-3012), itself pinned by the reference's SHA-256
  decode KATs.

For M > 1 the activation rows form an identity block (row m one-hot at its own
column), so every activation-row class of each kernel is covered. Which kernel
runs follows the dispatch rules of stark_qmm_encode; each test names it.
Scales and biases are drawn over wide exponent ranges so that the addition
s*q + b rounds in most outputs (a fused or reassociated form would differ).
"""
import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _wide_planes(O, rng, shape, w_dt):
    s = rng.uniform(0.5, 1.0, shape) * np.exp2(rng.integers(-12, 3, shape)) * rng.choice([-1.0, 1.0], shape)
    b = rng.normal(0, 1, shape) * np.exp2(rng.integers(-10, 2, shape))
    return (H.store(O, s.astype(np.float32).ravel(), w_dt), H.store(O, b.astype(np.float32).ravel(), w_dt))


def _weights(O, rng, n, k, bits, gs, layout, correction, w_dt):
    G = k // gs
    plane_shape = (n, G) if layout == 0 else (G, (n + 3) // 4 * 4)
    codes = rng.integers(0, 256, (n * k * bits + 7) // 8, dtype=np.uint8)
    s, b = _wide_planes(O, rng, plane_shape, w_dt)
    if correction == 0:
        b = None
    elif correction == 2:
        pd = 8 // bits
        zos, zgs = O.quant_strides(layout, n, G, pd)
        zlen = ((n - 1) * zos + (G - 1) * zgs) // pd + 1
        b = rng.integers(0, 256, zlen + 1, dtype=np.uint8)
    return codes, s, b


def _columns(rng, k, count):
    """Columns covering every position within a 32-bit word of 4-bit codes and
    of a 128-byte block, both ends of K, and random ones."""
    fixed = list(range(8)) + list(range(248, 264)) + [k // 2 - 1, k // 2, k - 8, k - 1]
    cols = [c for c in fixed if c < k]
    extra = rng.choice(k, size=min(k, count), replace=False)
    return np.array(sorted(set(cols) | set(int(c) for c in extra)), np.int64)


def _one_hot(k, cols, x_dt):
    x = np.zeros((len(cols), k), np.float32)
    x[np.arange(len(cols)), cols] = 1.0
    return x


def _mode(Q, bits):
    return {4: Q.MODE_U4, 8: Q.MODE_U8, 3: Q.MODE_U3, 5: Q.MODE_U5, 6: Q.MODE_U6}[bits]


def _affine_exact(Q, O, *, n, k, m, bits=4, gs=64, layout=1, correction=1, signed=False, w_dt=H.BF16, x_dt=H.BF16,
                  ncols=40, seed=0, label=""):
    """Columns in chunks of m one-hot rows; M = 1 chunks go through
    encode_many (eight products per call, shared weights)."""
    rng = np.random.default_rng(seed)
    codes, s, b = _weights(O, rng, n, k, bits, gs, layout, correction, w_dt)
    cols = _columns(rng, k, ncols)
    pad = (-len(cols)) % m
    cols = np.concatenate([cols, cols[:pad]]) if pad else cols
    G = k // gs
    xall = _one_hot(k, cols, x_dt)
    xbits = H.store(O, xall.ravel(), x_dt)
    st, want = O.matmul(a=xbits, m=len(cols), n=n, k=k, codes=codes, scales=s, correction=correction,
                        correction_data=b, layout=layout, row_count=n, group_count=G, bits=bits, group_size=gs,
                        signed_codes=signed, weights_dt=w_dt, input_dt=x_dt, output_dt=H.F32, threads=8)
    assert st == 0
    want = np.asarray(want, np.float32).reshape(len(cols), n)
    dcodes, ds = H.to_dev(codes), H.to_dev(s)
    db = None if b is None else H.to_dev(b)
    xdev = H.to_dev(xbits)
    outs = []
    args = []
    for c0 in range(0, len(cols), m):
        d = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
        # view into the device copy of all one-hot rows (a_offset in elements)
        a = Q.MatmulArguments(
            a=xdev, a_offset=c0 * k, m=m, n=n, k=k, d=d,
            b=Q.QuantizedB(codes=dcodes, scales=ds, params=Q.QuantParams(layout, n, G), mode=_mode(Q, bits),
                           group_size=gs, correction=correction, correction_data=db, signed_codes=signed))
        outs.append(d)
        args.append(a)
    kern = Q.MatmulKernel(w_dt, x_dt, H.F32)
    if m == 1:
        for i in range(0, len(args), 8):
            kern.encode_many(args[i:i + 8])
    else:
        for a in args:
            kern.encode(a)
    torch.cuda.synchronize()
    got = torch.cat(outs).cpu().numpy().reshape(len(cols), n)
    bad = got.view(np.uint32) != want.view(np.uint32)
    if bad.any():
        r, c = np.argwhere(bad)[0]
        raise AssertionError(f"{label}: {int(bad.sum())}/{bad.size} weights not bit-exact; first at column "
                             f"{cols[r]} row {c}: got {got[r, c]!r} want {want[r, c]!r}")


# ------------------------------------------------------------ qmv_stream (M = 1 decode)

@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("correction,signed", [(1, False), (0, False), (1, True), (0, True)])
def test_stream_exact(qmm, oracle, layout, correction, signed):
    """qmv_stream: 4-bit, M = 1, group 64, K % 4096 == 0, N >= 32 (N = 96 has a
    shifted last 32-row tile)."""
    _affine_exact(qmm, oracle, n=96, k=8192, m=1, layout=layout, correction=correction, signed=signed,
                  seed=layout * 8 + correction * 2 + signed, label="qmv_stream")


def test_stream_exact_f16_planes(qmm, oracle):
    _affine_exact(qmm, oracle, n=64, k=4096, m=1, w_dt=H.F16, seed=11, label="qmv_stream f16")


# ------------------------------------------------------------ qmv_mfma (slot form)

@pytest.mark.parametrize("gs", [32, 64, 128])
def test_mfma_4bit_m1_exact(qmm, oracle, gs):
    """qmv_mfma<1,1,gs,4>: K = 2048 is not a streaming shape."""
    _affine_exact(qmm, oracle, n=48, k=2048, m=1, gs=gs, seed=gs, label=f"qmv_mfma w4 m1 g{gs}")


@pytest.mark.parametrize("m", [2, 3, 4])
@pytest.mark.parametrize("layout", [0, 1])
def test_mfma_4bit_small_m_exact(qmm, oracle, m, layout):
    """qmv_mfma<2,1> (M = 2) and <4,1> (M = 3, 4; K % 1024 != 0 keeps them off
    the dense small-M kernel), identity activation blocks."""
    _affine_exact(qmm, oracle, n=48, k=4096 if m == 2 else 4032, m=m, layout=layout, ncols=24,
                  seed=m * 3 + layout, label=f"qmv_mfma w4 m{m}")


@pytest.mark.parametrize("m", [1, 2, 4, 8, 16])
def test_mfma_8bit_exact(qmm, oracle, m):
    """qmv_mfma<MP,MB,64,8> for every activation-row class at N = 1040 (N % 8 == 0)."""
    _affine_exact(qmm, oracle, n=1040, k=4096, m=m, bits=8, ncols=32, seed=80 + m, label=f"qmv_mfma w8 m{m}")


@pytest.mark.parametrize("signed,correction", [(True, 1), (False, 0)])
def test_mfma_8bit_signed_symmetric_exact(qmm, oracle, signed, correction):
    _affine_exact(qmm, oracle, n=64, k=2048, m=4, bits=8, signed=signed, correction=correction, ncols=16,
                  seed=90 + signed, label="qmv_mfma w8 variants")


# ------------------------------------------------------------ qmv_small_m (dense form, M = 3..16)

@pytest.mark.parametrize("m", [3, 4, 5, 8, 16])
@pytest.mark.parametrize("layout", [0, 1])
def test_small_m_exact(qmm, oracle, m, layout):
    _affine_exact(qmm, oracle, n=96, k=4096, m=m, layout=layout, ncols=32, seed=100 + m + layout,
                  label=f"qmv_small_m m{m}")


def test_small_m_signed_symmetric_exact(qmm, oracle):
    _affine_exact(qmm, oracle, n=48, k=2048, m=8, correction=0, signed=True, ncols=16, seed=120,
                  label="qmv_small_m signed symmetric")


# ------------------------------------------------------------ other GEMV kernels

@pytest.mark.parametrize("m", [1, 2])
def test_decode_kernel_exact(qmm, oracle, m):
    """qmv_w4_decode: K = 96 (K % 64 != 0 rules out the matrix-core kernels),
    group 32, group-output planes."""
    _affine_exact(qmm, oracle, n=64, k=96, m=m, gs=32, ncols=96, seed=130 + m, label=f"qmv_w4_decode m{m}")


@pytest.mark.parametrize("bits", [4, 8])
def test_tile_kernel_f32_activations_exact(qmm, oracle, bits):
    """qmv_affine_tile: f32 activations take the VALU tile kernel."""
    _affine_exact(qmm, oracle, n=40, k=1024, m=2, bits=bits, x_dt=H.F32, ncols=24, seed=140 + bits,
                  label=f"qmv_affine_tile w{bits}")


@pytest.mark.parametrize("m", [1, 2, 4])
def test_tile_kernel_bf16_activations_exact(qmm, oracle, m):
    """qmv_affine_tile, 4-bit codes as bf16 (1 + q/16) into v_dot2: per-row
    planes whose group count is not a multiple of 8 (K = 4032) keep the
    product off the matrix-core kernels."""
    _affine_exact(qmm, oracle, n=48, k=4032, m=m, layout=0, ncols=24, seed=170 + m, label=f"qmv_affine_tile dot2 m{m}")


@pytest.mark.parametrize("x_dt", [H.BF16, H.F32])
def test_tile_kernel_f32_planes_exact(qmm, oracle, x_dt):
    """qmv_affine_tile with f32 scale and bias planes (s*q is then rounded
    before b joins, as in the reference), dot2 and f32-FMA forms."""
    _affine_exact(qmm, oracle, n=40, k=1024, m=2, w_dt=H.F32, x_dt=x_dt, ncols=24, seed=175,
                  label=f"qmv_affine_tile f32 planes x{x_dt}")


@pytest.mark.parametrize("bits", [3, 5, 6])
def test_generic_kernel_exact(qmm, oracle, bits):
    """qmv_affine_generic: odd code widths (codes spill across bytes)."""
    _affine_exact(qmm, oracle, n=37, k=320, m=1, bits=bits, gs=32, ncols=24, seed=150 + bits,
                  label=f"qmv_affine_generic w{bits}")


@pytest.mark.parametrize("bits", [4, 8])
def test_zero_point_correction_exact(qmm, oracle, bits):
    _affine_exact(qmm, oracle, n=40, k=512, m=1, bits=bits, correction=2, ncols=24, seed=160 + bits,
                  label=f"zero points w{bits}")


# ------------------------------------------------------------ prefill dequant-GEMM

def _gemm_exact(Q, O, *, n, k, bits, correction=1, signed=False, layout=0, seed=0, m=72, label="qgemm_mfma"):
    rng = np.random.default_rng(seed)
    gs = 64
    codes, s, b = _weights(O, rng, n, k, bits, gs, layout, correction, H.BF16)
    cols = _columns(rng, k, 40)
    cols = np.resize(cols, m)  # M > 64 takes the GEMM, 17 .. 64 (4-bit g64, K % 512 == 0) the skinny product
    x = H.store(O, _one_hot(k, cols, H.BF16).ravel(), H.BF16)
    G = k // gs
    if correction == 1 and not signed and bits in (4, 8):
        sos, sgs = O.quant_strides(layout, n, G, 1)
        want = O.reference_affine_linear_bf16(x, codes, s, b, m, n, k, bits=bits, sos=sos, sgs=sgs, f32_out=True)
    else:
        st, w32 = O.matmul(a=x, m=m, n=n, k=k, codes=codes, scales=s, correction=correction, correction_data=b,
                           layout=layout, row_count=n, group_count=G, bits=bits, group_size=gs, signed_codes=signed,
                           output_dt=H.F32, threads=8)
        assert st == 0
        want = O.bf16_to_f32(O.f32_to_bf16(np.asarray(w32, np.float32)))
    want = np.asarray(want, np.float32).reshape(m, n)
    d = torch.full((m * n,), float("nan"), dtype=torch.float32, device="cuda")
    args = Q.MatmulArguments(
        a=H.to_dev(x), m=m, n=n, k=k, d=d,
        b=Q.QuantizedB(codes=H.to_dev(codes), scales=H.to_dev(s), params=Q.QuantParams(layout, n, G),
                       mode=_mode(Q, bits), group_size=gs, correction=correction,
                       correction_data=None if b is None else H.to_dev(b), signed_codes=signed))
    Q.MatmulKernel(H.BF16, H.BF16, H.F32).encode(args)
    torch.cuda.synchronize()
    got = d.cpu().numpy().reshape(m, n)
    bad = got.view(np.uint32) != want.view(np.uint32)
    assert not bad.any(), (f"{label} w{bits} m{m}: {int(bad.sum())} weights not bit-exact; first "
                           f"{np.argwhere(bad)[0]}: got {got[bad][0]!r} want {want[bad][0]!r}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", [0, 1])
def test_gemm_exact_against_bf16_effective_oracle(qmm, oracle, bits, layout):
    """qgemm_mfma's bf16 weight tiles equal the reference's bf16-effective
    weights bf16_rne(s*q + b) (vision.rs:301-305) bit for bit."""
    _gemm_exact(qmm, oracle, n=256, k=512, bits=bits, layout=layout, seed=170 + bits + layout)


@pytest.mark.parametrize("correction,signed", [(0, False), (1, True), (0, True)])
def test_gemm_exact_variants(qmm, oracle, correction, signed):
    _gemm_exact(qmm, oracle, n=128, k=256, bits=4, correction=correction, signed=signed, seed=180 + correction)


@pytest.mark.parametrize("m,k", [(65, 64), (130, 384), (200, 448), (384, 512), (96, 576), (300, 640), (128, 704),
                                 (72, 3136), (385, 448), (520, 320)])
@pytest.mark.parametrize("bits", [4, 8])
def test_gemm_exact_tile_classes(qmm, oracle, m, k, bits):
    """The three GEMM tile classes (128x64 tiles up to 128 rows, 128x128 up
    to 384, both of eight waves with three load stages; 256x128 above) at
    64-value step counts that leave every remainder of the six-step unrolled
    blocks (1, 6 .. 11 and 49 steps; odd and even counts in the 256-row
    class), ragged N: the bf16 weight tiles stay bit-exact."""
    _gemm_exact(qmm, oracle, n=136, k=k, bits=bits, seed=200 + m + bits, m=m)


@pytest.mark.parametrize("m", [17, 32, 40])
@pytest.mark.parametrize("layout", [0, 1])
def test_skinny_exact_against_bf16_effective_oracle(qmm, oracle, m, layout):
    """qgemm_skinny (4-bit, 17 .. 64 rows; 40 rows as blocks of 32 and 8)
    dequantises to the same bf16 weights as the GEMM, bit for bit."""
    _gemm_exact(qmm, oracle, n=96, k=512, bits=4, layout=layout, seed=190 + m + layout, m=m, label="qgemm_skinny")


@pytest.mark.parametrize("correction,signed", [(0, False), (1, True), (0, True)])
def test_skinny_exact_variants(qmm, oracle, correction, signed):
    _gemm_exact(qmm, oracle, n=48, k=1024, bits=4, correction=correction, signed=signed, seed=195 + correction,
                m=24, label="qgemm_skinny")


# ------------------------------------------------------------ GGUF blocks (hybrid path)

def _gguf_blocks(rng, kind, n, k):
    """Random blocks with finite f16 headers over a wide exponent range."""
    if kind == 8:
        nb = n * k // 32
        blk = np.zeros((nb, 34), np.uint8)
        d = (rng.uniform(0.5, 1, nb) * np.exp2(rng.integers(-14, 0, nb)) * rng.choice([-1, 1], nb))
        blk[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
        blk[:, 2:] = rng.integers(0, 256, (nb, 32), dtype=np.uint8)
    else:
        nb = n * k // 256
        blk = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
        d = rng.uniform(0.5, 1, nb) * np.exp2(rng.integers(-16, -4, nb))
        dm = rng.uniform(0.5, 1, nb) * np.exp2(rng.integers(-16, -4, nb))
        blk[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(nb, 2)
        blk[:, 2:4] = dm.astype(np.float16).view(np.uint8).reshape(nb, 2)
    return blk.ravel()


@pytest.mark.parametrize("kind", [8, 12])
@pytest.mark.parametrize("m", [1, 8])
def test_gguf_exact(qmm, oracle, kind, m):
    """gguf_mfma<kind> at M = 1 (slot form) and M = 8 (dense form), through
    mapped_many with f32 one-hot activations: output = decode_block value."""
    rng = np.random.default_rng(200 + kind + m)
    n, k = 48, 2048
    blocks = _gguf_blocks(rng, kind, n, k)
    dec = oracle.decode_rows(kind, blocks, n, k)
    cols = _columns(rng, k, 40)
    cols = np.concatenate([cols, cols[:(-len(cols)) % m]])
    codes = H.to_dev(blocks)
    ops = []
    for c0 in range(0, len(cols), m):
        x = _one_hot(k, cols[c0:c0 + m], H.F32)
        ops.append(qmm.MappedOperation(matrices=[qmm.MappedMatrix(codes=codes)] * m,
                                       inputs=torch.from_numpy(x.ravel()).cuda(), rows=n, columns=k,
                                       format=("packed", kind)))
    got = []
    for i in range(0, len(ops), 64):
        got += [o.cpu().numpy().reshape(m, n) for o in qmm.mapped_many(ops[i:i + 64])]
    got = np.concatenate(got)
    want = np.ascontiguousarray(dec[:, cols].T).astype(np.float32)
    # Q8_0 forms d*q as fma(d, q + 128, -128 d), which gives +0 where d*0 is -0
    # for a negative d; the sign of a zero weight reaches no output (the
    # reference's sums start at +0.0, and +0 + -0 = +0), so zeros compare equal
    bad = (got.view(np.uint32) != want.view(np.uint32)) & ~((got == 0) & (want == 0))
    assert not bad.any(), (f"gguf kind {kind} m{m}: {int(bad.sum())} weights not bit-exact; first "
                           f"{np.argwhere(bad)[0]}: got {got[bad][0]!r} want {want[bad][0]!r}")
