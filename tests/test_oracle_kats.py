"""Pins the CPU oracle against the reference's own known-answer tests, library
conversions and closed forms. No GPU. Each check is chosen so that a plausible
mistake in the restatement (nibble order, stride, sign, rounding) fails it."""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "kat_vectors.json")))
FORMATS = json.load(open(os.path.join(HERE, "golden", "ggml_formats.json")))


# ------------------------------------------------------------ conversions

def test_bf16_rounding_matches_torch(oracle):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.005859375, 1.001953125, 3.0e38, 3.4e38, -3.4e38, 1e-40,
                  np.inf, -np.inf], np.float32),
        # exact ties: lsb even stays, lsb odd rounds up
        (np.array([0x3F808000, 0x3F818000, 0x3F80C000, 0x7F7F8000], np.uint32)).view(np.float32),
    ])
    ours = oracle.f32_to_bf16(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    back = oracle.bf16_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(vals).to(torch.bfloat16).float().numpy())
    nan = oracle.f32_to_bf16(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0


def test_f16_rounding_matches_numpy(oracle):
    rng = np.random.default_rng(2)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 6.0e-8, 2.98e-8, 2.99e-8, 5.96e-8, 1e-10], np.float32),
    ]).astype(np.float32)
    ours = oracle.f32_to_f16(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    bits = np.arange(0, 0x10000, dtype=np.uint32).astype(np.uint16)
    f = oracle.f16_to_f32(bits)
    ref_f = bits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref_f)
    assert np.array_equal(f[finite], ref_f[finite])
    assert np.all(np.isnan(f[~finite & np.isnan(ref_f)]))


# ------------------------------------------------------------ packed codes

def test_packed_code_reference_kats(oracle):
    """reference.rs:196-219"""
    assert oracle.packed_code([0xD3], 8, 0) == 0xD3
    assert oracle.packed_code([0xD3], 4, 0) == 3
    assert oracle.packed_code([0xD3], 4, 1) == 13
    for bits in (3, 5, 6):
        expected = [(i * 17 + 3) & ((1 << bits) - 1) for i in range(64)]
        packed = np.zeros(len(expected) * bits // 8, np.uint8)
        for i, code in enumerate(expected):
            for b in range(bits):
                pos = i * bits + b
                packed[pos // 8] |= ((code >> b) & 1) << (pos % 8)
        assert all(oracle.packed_code(packed, bits, i) == c for i, c in enumerate(expected))
    codes = [0x10, 0x32, 0x54, 0x76, 0x98, 0xBA]
    assert [oracle.packed_code(codes, 4, i) for i in range(12)] == list(range(12))
    assert [oracle.packed_code([0x12, 0x34, 0x56, 0x78], 8, i) for i in range(4)] == [0x12, 0x34, 0x56, 0x78]


def test_quant_params_layout_table(oracle):
    """quant_dispatch_test.rs:53-70"""
    for case in KAT["quant_params_layout_table"]["cases"]:
        assert list(oracle.quant_strides(case["layout"], 5, 3, 1)) == case["scale_strides"]
        assert list(oracle.quant_strides(case["layout"], 5, 3, 2)) == case["u4_zero_point_strides"]


# ------------------------------------------------------------ MatmulCpuKernel

def test_cpu_matmul_exact_packed_tails(oracle):
    """reference.rs:222-298, including the undersized-codes error."""
    for c in KAT["packed_tails"]["cases"]:
        k, n = c["k"], c["n"]
        st, d = oracle.matmul(a=np.ones(k, np.float32), m=1, n=n, k=k, codes=np.array(c["codes"], np.uint8),
                              scales=np.ones(n, np.float32), correction=oracle.SYMMETRIC, bits=c["bits"],
                              group_size=k, group_count=1, weights_dt=oracle.F32, input_dt=oracle.F32,
                              output_dt=oracle.F32)
        assert st == 0
        assert d.tolist() == c["expected"]
    st, _ = oracle.matmul(a=np.ones(2, np.float32), m=1, n=1, k=2, codes=np.zeros(1, np.uint8),
                          scales=np.ones(1, np.float32), correction=oracle.SYMMETRIC, bits=8, group_size=2,
                          group_count=1, weights_dt=oracle.F32, input_dt=oracle.F32, output_dt=oracle.F32)
    assert st == 1


def materialized_case(oracle, scenario, materialize):
    """Inputs of affine_input_sum_test.rs:26-95 (bf16 everywhere, W4, g64, OutputGroup)."""
    k, n = {"quad": (64, 32), "fold": (1024, 32), "generic_output_tail": (1024, 33),
            "generic_input_tail": (768, 32), "grouped_partial": (512, 33)}[scenario]
    groups = k // 64
    x = np.zeros(k, np.float32)
    codes = np.zeros(k * n // 2, np.uint8)
    biases = np.zeros(groups * n, np.float32)
    if scenario == "quad":
        x = np.resize(np.array([1.0, 1.0 / 256, -1.0, 1.0 / 512], np.float32), k)
        biases[:] = 0.5
    elif scenario == "fold":
        x[0], x[512] = 1.0, 33554432.0
        for row in range(n):
            codes[row * k // 2] = 1
            codes[row * k // 2 + 256] = 1
            biases[row * groups + 8] = -1.0
    elif scenario.startswith("generic"):
        x[0], x[256], x[512] = 33554432.0, -33554432.0, 1.0
        for row in range(n):
            for idx in (0, 256, 512):
                codes[row * k // 2 + idx // 2] = 1
    else:
        x[0], x[1], x[4], x[5] = 33554432.0, 1.0, -33554432.0, 1.0
        for row in range(n):
            codes[row * k // 2] = 0x11
            codes[row * k // 2 + 2] = 0x11
    return dict(a=oracle.f32_to_bf16(x), m=1, n=n, k=k, codes=codes,
                scales=oracle.f32_to_bf16(np.ones(groups * n, np.float32)), correction=oracle.BIASES,
                correction_data=oracle.f32_to_bf16(biases), layout=oracle.OUTPUT_GROUP, group_count=groups, bits=4,
                group_size=64, materialize=materialize)


@pytest.mark.parametrize("case", KAT["materialized_affine_input_sum"]["cases"], ids=lambda c: c["scenario"] + str(c["materialize"]))
def test_materialized_affine_input_sum_exact_values(oracle, case):
    st, d = oracle.matmul(**materialized_case(oracle, case["scenario"], case["materialize"]))
    assert st == 0
    assert np.all(oracle.bf16_to_f32(d) == case["expected_all"])


def test_materialized_policy_rejections(oracle):
    """arguments.rs:36-61: F32 input or 8-bit codes with the flag set are rejected."""
    args = materialized_case(oracle, "quad", True)
    args["input_dt"] = oracle.F32
    args["a"] = oracle.bf16_to_f32(args["a"])
    assert oracle.matmul(**args)[0] == 1
    args = materialized_case(oracle, "quad", True)
    args["bits"] = 8
    args["codes"] = np.zeros(64 * 32, np.uint8)
    assert oracle.matmul(**args)[0] == 1


def _f64_dequant(codes, scales, biases_or_zp, k, n, bits, gs, layout, correction, signed, os_, gs_, zos=0, zgs=0):
    """Independent float64 dequant from first principles of the layout docs
    (mod.rs:19-25 layouts, matmul_b.rs:24-29 corrections)."""
    w = np.zeros((n, k))
    mid = 2 ** (bits - 1)
    for r in range(n):
        for kk in range(k):
            bit = (r * k + kk) * bits
            v = int(codes[bit // 8]) | (int(codes[bit // 8 + 1]) << 8 if bit // 8 + 1 < len(codes) else 0)
            q = (v >> (bit % 8)) & ((1 << bits) - 1)
            if signed:
                q ^= 1 << (bits - 1)
            g = kk // gs
            s = float(scales[r * os_ + g * gs_])
            if correction == 1:
                b = float(biases_or_zp[r * os_ + g * gs_])
            elif correction == 2:
                zi = r * zos + g * zgs
                if bits == 4:
                    byte = int(biases_or_zp[zi // 2])
                    zp = byte & 15 if zi % 2 == 0 else byte >> 4
                else:
                    zp = int(biases_or_zp[zi])
                b = -s * zp
            else:
                b = -s * mid
            w[r, kk] = s * q + b
    return w


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("correction", [0, 1, 2])
@pytest.mark.parametrize("bits", [4, 8])
def test_matmul_matches_float64_dequant(oracle, layout, correction, bits):
    rng = np.random.default_rng(10 + layout + 3 * correction + bits)
    m, n, k, gs = 3, 7, 128, 32
    G = k // gs
    codes = rng.integers(0, 256, n * k * bits // 8, dtype=np.uint8)
    os_, gs_ = oracle.quant_strides(layout, n, G, 1)
    plane = (n * G) if layout == 0 else G * ((n + 3) // 4 * 4)
    scales = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.uniform(0.01, 0.3, plane).astype(np.float32)))
    biases = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.uniform(-0.03, 0.03, plane).astype(np.float32)))
    zos = zgs = 0
    corr = None
    if correction == 1:
        corr = oracle.f32_to_bf16(biases)
        corr_f = biases
    elif correction == 2:
        pd = 8 // bits
        zos, zgs = oracle.quant_strides(layout, n, G, pd)
        zlen = (n * zos + G * zgs) // pd + 2
        corr = rng.integers(0, 256, zlen, dtype=np.uint8)
        corr_f = corr
    else:
        corr_f = None
    x = oracle.bf16_to_f32(oracle.f32_to_bf16(rng.uniform(-0.3, 0.3, m * k).astype(np.float32)))
    for signed in (False, True):
        st, d = oracle.matmul(a=oracle.f32_to_bf16(x), m=m, n=n, k=k, codes=codes, scales=oracle.f32_to_bf16(scales),
                              correction=correction, correction_data=corr, layout=layout, bits=bits, group_size=gs,
                              signed_codes=signed, output_dt=oracle.F32)
        assert st == 0
        w = _f64_dequant(codes, scales, corr_f, k, n, bits, gs, layout, correction, signed, os_, gs_, zos, zgs)
        ref = x.reshape(m, k).astype(np.float64) @ w.T
        mag = np.abs(x.reshape(m, k)) @ np.abs(w).T
        assert np.all(np.abs(d.reshape(m, n) - ref) <= 1e-5 * mag + 1e-7)


def test_matmul_d_ops_gather_and_layout_invariants(oracle):
    """Same matrix in both plane layouts gives bit-identical output; gather of
    permuted rows equals permuting outputs; D-ops follow kernel.rs:270-281."""
    rng = np.random.default_rng(5)
    m, n, k, gs = 2, 9, 256, 64
    w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
    c0, s0, b0 = oracle.quantize_affine(w, 4, gs, oracle.OUTPUT_GROUP)
    c1, s1, b1 = oracle.quantize_affine(w, 4, gs, oracle.GROUP_OUTPUT)
    assert np.array_equal(c0, c1)
    assert np.array_equal(s0, s1[:, :n].T) and np.array_equal(b0, b1[:, :n].T)
    x = oracle.f32_to_bf16(rng.normal(0, 1, m * k).astype(np.float32))
    common = dict(a=x, m=m, n=n, k=k, codes=c0, bits=4, group_size=gs, output_dt=oracle.F32)
    _, d0 = oracle.matmul(scales=s0, correction_data=b0, layout=oracle.OUTPUT_GROUP, **common)
    _, d1 = oracle.matmul(scales=s1, correction_data=b1, layout=oracle.GROUP_OUTPUT, **common)
    assert np.array_equal(d0, d1)
    perm = rng.permutation(n).astype(np.uint32)
    gather = np.concatenate([perm, perm[::-1]])
    _, dg = oracle.matmul(scales=s0, correction_data=b0, gather=gather, **common)
    assert np.array_equal(dg.reshape(m, n)[0], d0.reshape(m, n)[0][perm])
    assert np.array_equal(dg.reshape(m, n)[1], d0.reshape(m, n)[1][perm[::-1]])
    bias = oracle.f32_to_bf16(rng.normal(0, 1, n).astype(np.float32))
    prior = rng.normal(0, 1, m * n).astype(np.float32)
    _, dd = oracle.matmul(scales=s0, correction_data=b0, ab_scale=0.5, accumulate=True, d=prior, bias=bias,
                          soft_cap=3.0, **common)
    bf = oracle.bf16_to_f32(bias)
    v = (np.float32(0.5) * d0.reshape(m, n) + prior.reshape(m, n)).astype(np.float32) + bf[None, :]
    exp = (np.float32(3.0) * np.tanh(v.astype(np.float32) / np.float32(3.0))).astype(np.float32)
    assert np.allclose(dd.reshape(m, n), exp, rtol=1e-6, atol=1e-6)


def test_reference_affine_bf16_exact_on_integer_data(oracle):
    """vision.rs:249-336: with integer activations and weights whose dequant is
    exactly representable, every partial sum is exact, so the result equals the
    integer dot product rounded to bf16."""
    rng = np.random.default_rng(7)
    m, n, k = 2, 5, 128
    G = k // 64
    codes = rng.integers(0, 256, n * k // 2, dtype=np.uint8)
    scales = np.ones(n * G, np.float32)
    biases = rng.integers(-8, 8, n * G).astype(np.float32)
    x = rng.integers(-4, 5, m * k).astype(np.float32)
    out = oracle.reference_affine_linear_bf16(oracle.f32_to_bf16(x), codes, oracle.f32_to_bf16(scales),
                                              oracle.f32_to_bf16(biases), m, n, k, f32_out=True)
    q = np.array([[oracle.packed_code(codes, 4, r * k + kk) for kk in range(k)] for r in range(n)], np.float64)
    w = q + np.repeat(biases.reshape(n, G), 64, axis=1)
    ref = x.reshape(m, k).astype(np.float64) @ w.T
    assert np.array_equal(out.reshape(m, n), oracle.bf16_to_f32(oracle.f32_to_bf16(ref.astype(np.float32))))
    # a bank row beyond the bank is NaN
    out = oracle.reference_affine_linear_bf16(oracle.f32_to_bf16(x), codes, oracle.f32_to_bf16(scales),
                                              oracle.f32_to_bf16(biases), m, n, k, bank_rows=n - 1, f32_out=True)
    assert np.isnan(out.reshape(m, n)[:, n - 1]).all() and not np.isnan(out.reshape(m, n)[:, :n - 1]).any()


# ------------------------------------------------------------ GGUF

def test_block_layout_matches_upstream_headers(oracle):
    """weights.rs:3149-3164 against unit/fixtures/hybrid_ggml_formats.json."""
    for f in FORMATS["formats"]:
        assert oracle.block_layout(f["kind"]) == (f["block_elements"], f["block_bytes"]), f["name"]


@pytest.mark.parametrize("case", KAT["gguf_decode_sha256"]["cases"], ids=lambda c: str(c["kind"]))
def test_decode_block_matches_ggml_hashes(oracle, case):
    """weights.rs:3183-3220: SHA-256 of the f32 outputs of decode_block."""
    elems, size = oracle.block_layout(case["kind"])
    b = np.array([(i * 73 + 41) % 256 for i in range(size)], np.uint8)
    for i, at in enumerate(case["offsets"]):
        v = 0x3400 if i == 0 else 0x3000
        b[at], b[at + 1] = v & 0xFF, v >> 8
    out = oracle.decode_block(case["kind"], b)
    assert hashlib.sha256(out.astype("<f4").tobytes()).hexdigest() == case["sha256"]
    with pytest.raises(ValueError):
        oracle.decode_block(case["kind"], b[:-1])


def test_q4k_scale_min_round_trips_generator(oracle):
    """The generator packs 6-bit (scale, min) pairs; scale_min (weights.rs:2908-2921)
    must return exactly what was packed, for all 8 indices."""
    rng = np.random.default_rng(3)
    w = rng.normal(0, 0.02, (4, 512)).astype(np.float32)
    q = oracle.quantize_q4_k(w)
    for r in range(4):
        for blk in range(2):
            b = q[r, blk * 144:(blk + 1) * 144]
            d = oracle.f16_to_f32(np.array([int(b[0]) | (int(b[1]) << 8)], np.uint16))[0]
            dm = oracle.f16_to_f32(np.array([int(b[2]) | (int(b[3]) << 8)], np.uint16))[0]
            dec = oracle.decode_block(12, b)
            for j in range(8):
                sc, mn = oracle.scale_min(b[4:16], j)
                assert 0 <= sc < 64 and 0 <= mn < 64
                part, half = divmod(j, 2)
                qs = b[16 + part * 32:16 + part * 32 + 32]
                nib = (qs >> (4 * half)) & 15
                exp = (np.float32(d) * np.float32(sc) * nib.astype(np.float32) - np.float32(dm) * np.float32(mn))
                assert np.array_equal(dec[part * 64 + half * 32: part * 64 + half * 32 + 32], exp.astype(np.float32))
            # the quantizer is accurate: decode close to the source weights
            src = w[r, blk * 256:(blk + 1) * 256]
            assert np.max(np.abs(dec - src)) < 0.2 * np.max(np.abs(src))


def test_q8_0_decode_closed_form(oracle):
    rng = np.random.default_rng(4)
    w = rng.normal(0, 0.02, (3, 64)).astype(np.float32)
    q = oracle.quantize_q8_0(w)
    dec = oracle.decode_rows(8, q, 3, 64)
    for r in range(3):
        for blk in range(2):
            b = q[r, blk * 34:(blk + 1) * 34]
            d = np.float32(oracle.f16_to_f32(np.array([int(b[0]) | (int(b[1]) << 8)], np.uint16))[0])
            assert np.array_equal(dec[r, blk * 32:(blk + 1) * 32], (d * b[2:].view(np.int8).astype(np.float32)))
    assert np.max(np.abs(dec - w)) < 0.01 * np.abs(w).max() + 1e-6


@pytest.mark.parametrize("kind", [8, 12])
def test_hybrid_packed_matvec_vs_float64(oracle, kind):
    """f64 brute force of decode . x, the tolerance of weight_metal.rs:2390-2395."""
    rng = np.random.default_rng(kind)
    rows, cols = 6, 512
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    q = oracle.quantize_q8_0(w) if kind == 8 else oracle.quantize_q4_k(w)
    x = rng.normal(0, 1, cols).astype(np.float32)
    out = oracle.hybrid_packed_matvec(kind, q, rows, cols, x)
    dec = oracle.decode_rows(kind, q, rows, cols).astype(np.float64)
    ref = dec @ x.astype(np.float64)
    mag = np.abs(dec) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(out - ref) <= 2e-5 * np.maximum(mag, 1.0))


def test_hybrid_affine_matvec_vs_float64(oracle):
    rng = np.random.default_rng(9)
    rows, cols, gs = 5, 256, 64
    w = rng.normal(0, 0.02, (rows, cols)).astype(np.float32)
    codes, s, b = oracle.quantize_affine(w, 4, gs, oracle.OUTPUT_GROUP)
    x = rng.normal(0, 1, cols).astype(np.float32)
    out = oracle.hybrid_affine_matvec(codes, s, b, oracle.BF16, 4, gs, rows, cols, x)
    sf, bf = oracle.bf16_to_f32(s), oracle.bf16_to_f32(b)
    q = np.array([[oracle.packed_code(codes, 4, r * cols + c) for c in range(cols)] for r in range(rows)], np.float64)
    deq = q * np.repeat(sf, gs, axis=1) + np.repeat(bf, gs, axis=1)
    ref = deq @ x.astype(np.float64)
    mag = np.abs(deq) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(out - ref) <= 2e-5 * np.maximum(mag, 1.0))


# ------------------------------------------------------------ MoE

def test_moe_adjust_routes_kat(oracle):
    c = KAT["moe_adjust_routes"]
    ids = np.array(c["ids"], np.uint32)
    w = np.array(c["weights"], np.float32)
    oracle.moe_adjust_routes(ids, w, np.array(c["scales"], np.float32), 1, 4, 3, True)
    assert ids.tolist() == c["expected_ids"]
    assert w.tolist() == [np.float32(v) for v in c["expected_weights"]]


def test_moe_accumulate_bf16_kat(oracle):
    c = KAT["moe_accumulate_bf16"]
    inputs = oracle.f32_to_bf16(np.array(c["inputs"], np.float32))
    for rnd, exp in ((0, c["expected_round_accumulator_off"]), (1, c["expected_round_accumulator_on"])):
        acc = np.array([np.nan], np.float32)
        out = np.zeros(1, np.uint16)
        for rank in range(3):
            oracle.moe_accumulate(inputs[rank:rank + 1], np.ones(3, np.float32), acc, out, 1, rank, 0, rank == 0,
                                  rank == 2, 1, rnd)
        assert oracle.bf16_to_f32(out)[0] == exp


def test_moe_route_invariants(oracle):
    """Top-k by repeated argmax: ids are the k largest logits in descending
    order with ties to the lower id (numpy stable argsort of -logits); weights
    are the renormalised softmax exp(l_i - max) / sum_sel exp(l_j - max)."""
    rng = np.random.default_rng(11)
    rows, E, k = 6, 128, 8
    logits = rng.normal(0, 2, (rows, E)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = logits[0, 77] = 9.0  # ties
    ids, w = oracle.moe_route(logits, rows, E, k)
    ids, w = ids.reshape(rows, k), w.reshape(rows, k)
    for r in range(rows):
        exp_ids = np.argsort(-logits[r], kind="stable")[:k]
        assert ids[r].tolist() == exp_ids.tolist()
        e = np.exp(logits[r, exp_ids].astype(np.float64) - logits[r].max())
        assert np.allclose(w[r], e / e.sum(), rtol=1e-6, atol=0)
    assert ids[0, :3].tolist() == [5, 9, 77]
    bad = logits.copy()
    bad[2, 3] = np.inf
    ids2, w2 = oracle.moe_route(bad, rows, E, k)
    assert np.all(ids2.reshape(rows, k)[2] == 0) and np.all(np.isnan(w2.reshape(rows, k)[2]))
    _, wr = oracle.moe_route(logits, rows, E, k, round_weights=True)
    assert np.array_equal(wr, oracle.bf16_to_f32(oracle.f32_to_bf16(w.ravel())))


def test_gated_silu_closed_form(oracle):
    rng = np.random.default_rng(12)
    hidden = 64
    p = rng.normal(0, 2, 2 * hidden).astype(np.float32)
    pb = oracle.f32_to_bf16(p)
    out = oracle.bf16_to_f32(oracle.gated_silu_bf16(pb, hidden, 1))
    v, g = oracle.bf16_to_f32(pb[:hidden]).astype(np.float64), oracle.bf16_to_f32(pb[hidden:]).astype(np.float64)
    ref = v * g / (1 + np.exp(-g))
    assert np.all(np.abs(out - ref) <= 2 * 2.0 ** -8 * np.abs(ref) + 1e-30)
