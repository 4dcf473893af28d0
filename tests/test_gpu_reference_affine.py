"""The BF16-effective affine reference dot (ReferenceAffineBF16Matmul,
encode_block/linear/reference_affine.rs:105-280; kernel vision.rs:249-336) on
the GPU, held BIT-EXACT to the oracle's restatement and to the reference's own
tests (encodable_block/linear/reference_affine/tests.rs):

* source_boundaries (tests.rs:92-170): the bank generator of tests.rs:40-73,
  every width (dense, 4, 5, 6, 8), both plane layouts, plain and gathered,
  BF16 and widened F32 output, an input offset; quantized == dense == oracle;
* cancellation_tree (tests.rs:176-222): [1.0, 1.0];
* malformed bounds and the NaN mask (tests.rs:253-340), source policies
  (tests.rs:224-251), the plan bounds (tests.rs:76-90);
* random banks at model widths against the oracle, bit for bit.
"""
import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu
F32, BF16 = H.F32, H.BF16
OG, GO = 0, 1  # OUTPUT_GROUP, GROUP_OUTPUT
MODES = {4: 0, 8: 2, 5: 3, 6: 4}


def _bank(O, rows, k, bits, layout):
    """tests.rs:40-73: codes (row*19 + inner*7 + inner/11) % 2^bits, scale
    0.1 + row/32 + group/64, bias -0.2 - row/16, NaN padding in the planes."""
    G = k // 64
    if layout == OG:
        shape, sos, sgs = (rows, G), G, 1
    else:
        shape, sos, sgs = (G, (rows + 3) // 4 * 4), 1, (rows + 3) // 4 * 4
    scales = np.full(shape[0] * shape[1], 0x7FC0, np.uint16)
    biases = scales.copy()
    codes = np.zeros(rows * k * bits // 8, np.uint8)
    dense = np.zeros(rows * k, np.uint16)
    bf = lambda v: O.f32_to_bf16(np.asarray([v], np.float32))[0]  # noqa: E731
    for row in range(rows):
        for inner in range(k):
            g = row * sos + inner // 64 * sgs
            s = bf(np.float32(0.1) + np.float32(row) / np.float32(32.0) + np.float32(inner // 64) / np.float32(64.0))
            b = bf(np.float32(-0.2) - np.float32(row) / np.float32(16.0))
            scales[g], biases[g] = s, b
            code = (row * 19 + inner * 7 + inner // 11) % (1 << bits)
            bit = inner * bits
            off = row * (k * bits // 8) + bit // 8
            codes[off] |= (code << (bit % 8)) & 0xFF
            if bit % 8 + bits > 8:
                codes[off + 1] |= code >> (8 - bit % 8)
            sf = O.bf16_to_f32(np.asarray([s], np.uint16))[0]
            bfl = O.bf16_to_f32(np.asarray([b], np.uint16))[0]
            dense[row * k + inner] = bf(np.float32(code) * sf + bfl)
    return codes, scales, biases, dense, sos, sgs


def _quantized(Q, codes, scales, biases, bits, layout, rows, k, gs=64, signed=False, row_count=None, groups=None,
               materialize=False):
    return Q.QuantizedB(codes=codes, scales=scales,
                        params=Q.QuantParams(layout=layout, row_count=rows if row_count is None else row_count,
                                             group_count=k // 64 if groups is None else groups,
                                             materialize_affine_input_sum=materialize),
                        mode=MODES[bits], group_size=gs, correction=Q.BIASES, correction_data=biases,
                        signed_codes=signed)


def _out(t, dt):
    a = t.cpu().numpy()
    return a.view(np.uint32) if dt == F32 else a.view(np.uint16)


def _oracle(O, x, weights, scales, biases, m, n, k, bits, idx, bank, sos, sgs, dt):
    got = O.reference_affine_linear_bf16(x, weights, scales, biases, m, n, k, bits=bits, indices=idx, bank_rows=bank,
                                         sos=sos, sgs=sgs, f32_out=dt == F32)
    return got.view(np.uint32) if dt == F32 else got


@pytest.mark.parametrize("layout", [OG, GO])
def test_source_boundaries(qmm, oracle, layout):
    m, rows, k = 3, 7, 128
    xs = np.array([(i % 31) / 16.0 - 1.0 for i in range(m * k)], np.float32)
    prefixed = np.concatenate([oracle.f32_to_bf16(np.full(2, -99.0, np.float32)), oracle.f32_to_bf16(xs)])
    x_dev = H.to_dev(prefixed)
    x_plain = oracle.f32_to_bf16(xs)
    for bits in (0, 4, 5, 6, 8):
        codes, scales, biases, dense, sos, sgs = _bank(oracle, rows, k, max(bits, 4), layout)
        d_dense = H.to_dev(dense)
        for gathered in (False, True):
            n = 5 if gathered else rows
            sel = np.array([(r * 3 + c * 2) % rows for r in range(m) for c in range(n)], np.uint32)
            idx = H.to_dev(sel) if gathered else None
            for dt in (BF16, F32):
                R = qmm.ReferenceAffineBF16Matmul(dt)
                if bits == 0:
                    w = qmm.FullPrecisionB(values=d_dense)
                else:
                    w = _quantized(qmm, H.to_dev(codes), H.to_dev(scales), H.to_dev(biases), bits, layout, rows, k)
                got = _out(R.encode(x_dev, 4, w, idx, m, n, k), dt)
                base = _out(R.encode(x_dev, 4, qmm.FullPrecisionB(values=d_dense), idx, m, n, k), dt)
                want = _oracle(oracle, x_plain, dense.view(np.uint8), np.zeros(1, np.uint16), np.zeros(1, np.uint16),
                               m, n, k, 0, sel if gathered else None, rows, 0, 0, dt)
                label = f"bits {bits} gathered {gathered} dt {dt}"
                assert np.array_equal(got, base), label
                assert np.array_equal(got, want), label
                if bits:
                    wq = _oracle(oracle, x_plain, codes, scales, biases, m, n, k, bits, sel if gathered else None,
                                 rows, sos, sgs, dt)
                    assert np.array_equal(got, wq), label


def test_cancellation_tree(qmm, oracle):
    """tests.rs:176-222: row 0's source tree returns 1 (sequential f32 gives 0);
    row 1 rounds 1 + 1/256 to bf16 before widening."""
    x = np.zeros(128, np.float32)
    x[0], x[4], x[8] = 67108864.0, 1.0, -67108864.0
    x[64], x[65] = 1.0, 1.0 / 256.0
    xd = H.to_dev(oracle.f32_to_bf16(x))
    one = oracle.f32_to_bf16(np.ones(1, np.float32))[0]
    for bits in (0, 4, 5, 6, 8):
        if bits == 0:
            w = qmm.FullPrecisionB(values=H.to_dev(np.full(64, one, np.uint16)))
        else:
            plane = H.to_dev(np.full(4, one, np.uint16))  # GroupOutput [1, 4]
            w = _quantized(qmm, H.to_dev(np.zeros(64 * bits // 8, np.uint8)), plane, plane, bits, GO, 1, 64)
        got = qmm.ReferenceAffineBF16Matmul(F32).encode(xd, 0, w, None, 2, 1, 64).cpu().numpy()
        assert got.tolist() == [1.0, 1.0], f"bits {bits}"


def test_malformed_and_nan_mask(qmm, oracle):
    codes, scales, biases, dense, sos, sgs = _bank(oracle, 7, 128, 4, GO)
    R = qmm.ReferenceAffineBF16Matmul(F32)
    one = oracle.f32_to_bf16(np.ones(1, np.float32))[0]
    x = H.to_dev(np.full(3 * 128, one, np.uint16))
    c, s, b = H.to_dev(codes), H.to_dev(scales), H.to_dev(biases)
    cases = [
        (H.to_dev(codes[:-1]), s, 64, False, dict(), 0),
        (c, H.to_dev(scales[:-2]), 64, False, dict(), 0),
        (c, s, 32, False, dict(), 0),
        (c, s, 64, True, dict(), 0),
        (c, s, 64, False, dict(row_count=9, groups=2), 0),
        (c, s, 64, False, dict(), 1),
        (c, s, 64, False, dict(), 2),
    ]
    for cc, ss, gs, signed, params, off in cases:
        w = _quantized(qmm, cc, ss, b, 4, GO, 7, 128, gs=gs, signed=signed, **params)
        with pytest.raises(qmm.MatmulError):
            R.encode(x, off, w, None, 3, 5, 128)
    w = _quantized(qmm, c, s, b, 4, GO, 7, 128)
    with pytest.raises(qmm.MatmulError):  # short indices
        R.encode(x, 0, w, H.to_dev(np.zeros(14, np.uint32)), 3, 5, 128)
    padded = torch.zeros(3 * 128 + 1, dtype=torch.int16, device="cuda")
    with pytest.raises(qmm.MatmulError):  # input at an odd byte address
        R.encode(padded.view(torch.uint8)[1:], 0, w, None, 3, 5, 128)
    with pytest.raises(qmm.MatmulError):  # indices off 4-byte alignment
        R.encode(x, 0, w, torch.zeros(16, dtype=torch.int32, device="cuda").view(torch.uint8)[2:], 3, 5, 128)
    sel = np.zeros(15, np.uint32)
    sel[0] = 0xFFFFFFFF
    got = R.encode(x, 0, w, H.to_dev(sel), 3, 5, 128).cpu().numpy()
    assert np.isnan(got[0]) and np.isfinite(got[1:]).all()
    # plain form: N beyond the bank
    with pytest.raises(qmm.MatmulError):
        R.encode(x, 0, w, None, 3, 8, 128)


def test_source_policies_keep_their_route(qmm, oracle):
    """tests.rs:224-251: materialized input sums and fused-source widths are refused."""
    one = oracle.f32_to_bf16(np.ones(1, np.float32))[0]
    plane = H.to_dev(np.full(4, one, np.uint16))
    codes = H.to_dev(np.zeros(32, np.uint8))
    x = H.to_dev(np.full(64, one, np.uint16))
    R = qmm.ReferenceAffineBF16Matmul(BF16)
    R.encode(x, 0, _quantized(qmm, codes, plane, plane, 4, GO, 1, 64), None, 1, 1, 64)
    with pytest.raises(qmm.MatmulError):
        R.encode(x, 0, _quantized(qmm, codes, plane, plane, 4, GO, 1, 64, materialize=True), None, 1, 1, 64)
    with pytest.raises(qmm.MatmulError):
        R.encode(x, 0, _quantized(qmm, codes, plane, plane, 4, GO, 1, 64), None, 1, 1, 64, source_output_widths=[1])
    with pytest.raises(qmm.MatmulError):
        qmm.ReferenceAffineBF16Matmul(H.F16)


def test_plan_bounds(qmm):
    """ReferenceAffinePlan (tests.rs:76-90): shapes outside the bounded work
    geometry are refused before anything runs."""
    one = torch.zeros(64, dtype=torch.int16, device="cuda")
    w = qmm.FullPrecisionB(values=one)
    R = qmm.ReferenceAffineBF16Matmul(F32)
    for m, n, k in [(0, 1, 64), (1, 0, 64), (1, 1, 0), (1, 1, 63), (32769, 1, 64), (4096, 1048576, 131072)]:
        with pytest.raises(qmm.MatmulError):
            R.encode(one, 0, w, None, m, n, k)


@pytest.mark.parametrize("bits", [0, 4, 5, 6, 8])
@pytest.mark.parametrize("layout", [OG, GO])
def test_random_banks_bit_exact(qmm, oracle, bits, layout):
    """Model-width banks (K = 2048) with N(0, 0.02) weights and N(0, 1) inputs,
    plain at M = 1, 5 and gathered expert rows, bitwise against the oracle."""
    rng = np.random.default_rng(bits * 2 + layout)
    rows, k = 160, 2048
    G = k // 64
    if bits:
        codes = rng.integers(0, 256, rows * k * bits // 8, dtype=np.uint8)
        plane = (rows, G) if layout == OG else (G, (rows + 3) // 4 * 4)
        sos, sgs = (G, 1) if layout == OG else (1, (rows + 3) // 4 * 4)
        scales = oracle.f32_to_bf16(rng.uniform(0.001, 0.01, plane).astype(np.float32).ravel())
        biases = oracle.f32_to_bf16(rng.uniform(-0.05, 0.0, plane).astype(np.float32).ravel())
        w = _quantized(qmm, H.to_dev(codes), H.to_dev(scales), H.to_dev(biases), bits, layout, rows, k)
        wb = codes
    else:
        dense = oracle.f32_to_bf16(rng.normal(0, 0.02, rows * k).astype(np.float32))
        scales = biases = np.zeros(1, np.uint16)
        sos = sgs = 0
        w = qmm.FullPrecisionB(values=H.to_dev(dense))
        wb = dense.view(np.uint8)
    for dt in (BF16, F32):
        R = qmm.ReferenceAffineBF16Matmul(dt)
        for m in (1, 5):
            x = oracle.f32_to_bf16(rng.normal(0, 1, m * k).astype(np.float32))
            got = _out(R.encode(H.to_dev(x), 0, w, None, m, rows, k), dt)
            want = _oracle(oracle, x, wb, scales, biases, m, rows, k, bits, None, rows, sos, sgs, dt)
            assert np.array_equal(got, want), f"plain m{m} dt {dt}"
        m, n = 8, 24
        sel = rng.integers(0, rows, m * n).astype(np.uint32)
        x = oracle.f32_to_bf16(rng.normal(0, 1, m * k).astype(np.float32))
        got = _out(R.encode(H.to_dev(x), 0, w, H.to_dev(sel), m, n, k), dt)
        want = _oracle(oracle, x, wb, scales, biases, m, n, k, bits, sel, rows, sos, sgs, dt)
        assert np.array_equal(got, want), f"gathered dt {dt}"


def test_full_width_rows(qmm, oracle):
    """A q4 projection at Qwen3-8B width (N = 4096, K = 4096), M = 3, bitwise."""
    rng = np.random.default_rng(99)
    n, k = 4096, 4096
    codes, s, b = oracle.quantize_affine(rng.normal(0, 0.02, (n, k)).astype(np.float32), 4, 64, oracle.OUTPUT_GROUP)
    x = oracle.f32_to_bf16(rng.normal(0, 1, 3 * k).astype(np.float32))
    w = _quantized(qmm, H.to_dev(codes.ravel()), H.to_dev(s.ravel()), H.to_dev(b.ravel()), 4, OG, n, k)
    got = _out(qmm.ReferenceAffineBF16Matmul(BF16).encode(H.to_dev(x), 0, w, None, 3, n, k), BF16)
    want = _oracle(oracle, x, codes.ravel(), s.ravel(), b.ravel(), 3, n, k, 4, None, n, k // 64, 1, BF16)
    assert np.array_equal(got, want)
