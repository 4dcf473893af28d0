"""Pins of the oracle's activation transforms, gated activations, int8
activations and output RHT (oracle/stark_oracle.c) against the reference's own
test vectors and against closed forms:

* the Walsh-Hadamard butterfly: Sylvester's matrix H[i][j] = (-1)^popcount(i&j) / sqrt(32),
  an involution;
* Int8CodeLayout::GroupedByNibble maps [0..8) to [0, 4, 1, 5, 2, 6, 3, 7]
  (crates/stark-engine/src/backends/common/kernel/matmul/matmul_a.rs:38);
* symmetric int8 quantization (activation_transform/mod.rs:9-26) by its definition;
* GatedActMul KATs: the separate-operand case (gated_act_mul_test.rs:235-256),
  the MLX materialized-sigmoid boundaries against an independent f64 scalar
  restatement (gated_act_mul_test.rs:84-119), alpha and clipping (:304-367);
* int8 activations give the FullPrecision product of their dequantized values
  bit for bit (kernel.rs:193-205 computes q * scale first);
* output RHT (kernel.rs:287-300) against float64 brute force.
"""
import numpy as np
import pytest

F32, F16, BF16 = 0, 1, 30


def sylvester(n=32):
    i = np.arange(n)
    pc = np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    return np.where(pc % 2 == 0, 1.0, -1.0) / np.sqrt(n)


def test_hadamard_closed_form(oracle):
    H = sylvester()
    for i in range(32):
        e = np.zeros(32)
        e[i] = 1
        assert np.allclose(oracle.hadamard32(e), H[:, i], atol=1e-7)
    rng = np.random.default_rng(0)
    x = rng.normal(0, 1, 32).astype(np.float32)
    y = oracle.hadamard32(x)
    assert np.allclose(y, H @ x.astype(np.float64), rtol=1e-5, atol=1e-6)
    assert np.allclose(oracle.hadamard32(y), x, rtol=1e-5, atol=1e-6)  # H is its own inverse


def test_grouped_by_nibble_index(oracle):
    assert [oracle.int8_code_index(True, i) for i in range(8)] == [0, 4, 1, 5, 2, 6, 3, 7]
    assert [oracle.int8_code_index(True, i) for i in range(8, 16)] == [8, 12, 9, 13, 10, 14, 11, 15]
    assert [oracle.int8_code_index(False, i) for i in range(8)] == list(range(8))


def test_symmetric_divisor_and_quantize(oracle):
    L = oracle.lib()
    import ctypes as C

    def div(v):
        a = np.ascontiguousarray(v, np.float32)
        return L.so_min_max_symmetric_divisor(a.ctypes.data_as(C.c_void_p), a.size)
    assert div([-2.0, 1.0, 0.5]) == np.float32(2.0) / np.float32(127.0)
    assert div([0.0, 0.0]) == 1.0 and div([np.inf, 1.0]) == 1.0
    assert div([np.nan, -3.0]) == np.float32(3.0) / np.float32(127.0)  # f32::min/max skip NaN
    q = L.so_quantize_symmetric_i8
    assert q(2.5, 1.0) == 3 and q(-2.5, 1.0) == -3 and q(0.49, 1.0) == 0  # half away from zero
    assert q(1000.0, 1.0) == 127 and q(-1000.0, 1.0) == -127 and q(float("nan"), 1.0) == 0


@pytest.mark.parametrize("count", [32, 128, 2048])
def test_activation_transform_rht_brute_force(oracle, count):
    rng = np.random.default_rng(count)
    batch = 3
    x = rng.normal(0, 2, (batch, count)).astype(np.float32)
    f = np.where(np.arange(count) % 3 == 0, -1, 1).astype(np.int32)
    H = sylvester()
    blocks = x.reshape(batch, count // 32, 32).astype(np.float64)
    fin = (f.reshape(count // 32, 32)).astype(np.float64)
    want_in = np.einsum("ij,bsj->bsi", H, blocks * fin).reshape(batch, count)
    want_out = (np.einsum("ij,bsj->bsi", H, blocks) * fin).reshape(batch, count)
    got_in = oracle.activation_transform(x.ravel(), f, batch, count, oracle.INPUT_RHT).reshape(batch, count)
    got_out = oracle.activation_transform(x.ravel(), f, batch, count, oracle.OUTPUT_RHT).reshape(batch, count)
    assert np.allclose(got_in, want_in, rtol=1e-5, atol=1e-5)
    assert np.allclose(got_out, want_out, rtol=1e-5, atol=1e-5)
    # bf16 storage with a bias: the transformed value is rounded to bf16 before the bias
    xb = oracle.f32_to_bf16(x.ravel())
    bias = rng.normal(0, 0.1, count).astype(np.float32)
    got = oracle.bf16_to_f32(oracle.activation_transform(xb, f, batch, count, oracle.OUTPUT_RHT, t_dt=BF16,
                                                         bias=bias))
    plain = oracle.bf16_to_f32(oracle.activation_transform(xb, f, batch, count, oracle.OUTPUT_RHT, t_dt=BF16))
    want = oracle.bf16_to_f32(oracle.f32_to_bf16((plain.reshape(batch, count) + bias).astype(np.float32).ravel()))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("scale_group,sum_group", [(32, 32), (128, 64), (64, 64)])
def test_activation_quantize(oracle, grouped, scale_group, sum_group):
    rng = np.random.default_rng(scale_group + sum_group + grouped)
    batch, count = 2, 256
    x = rng.normal(0, 1, batch * count).astype(np.float32)
    f = rng.choice([-1, 1], count).astype(np.int32)
    t = oracle.activation_transform(x, f, batch, count, oracle.INPUT_RHT).reshape(batch, count)
    q, sc, sums = oracle.activation_transform(x, f, batch, count, oracle.QUANTIZE_WITH_GROUP_SUMS,
                                              scale_group=scale_group, sum_group=sum_group, grouped=grouped)
    q = q.reshape(batch, count)
    order = np.array([oracle.int8_code_index(grouped, i) for i in range(count)])
    codes = q[:, order]  # logical order
    sc = sc.reshape(batch, count // scale_group)
    for r in range(batch):
        for g in range(count // scale_group):
            seg = t[r, g * scale_group:(g + 1) * scale_group]
            assert sc[r, g] == np.float32(np.abs(seg).max()) / np.float32(127.0)
            assert np.abs(codes[r, g * scale_group:(g + 1) * scale_group] * sc[r, g] - seg).max() <= sc[r, g] * 0.5 + 1e-7
            assert np.abs(codes[r, g * scale_group:(g + 1) * scale_group]).max() == 127
    assert np.array_equal(sums.reshape(batch, -1), codes.reshape(batch, -1, sum_group).sum(-1))


def test_gated_act_mul_separate_kat(oracle):
    """gated_act_mul_test.rs:235-256: identity gate, per-layer value slices."""
    for dt in (F32, BF16):
        gate = oracle.to_dtype_bits(np.array([1.0, 2.0, 3.0, 4.0], np.float32), dt)
        value = oracle.to_dtype_bits(np.array([0, 0, 10, 20, 30, 40, 0, 0, 50, 60, 70, 80], np.float32), dt)
        out = oracle.gated_act_mul(gate, 2, 2, oracle.IDENTITY, value=value, value_offset=2, value_row_stride=6,
                                   interleaved=False, t_dt=dt)
        assert np.array_equal(oracle.from_dtype_bits(out, dt), [10.0, 40.0, 150.0, 240.0])


def test_gated_act_mul_materialized_sigmoid_boundaries(oracle):
    """gated_act_mul_test.rs:84-119: the MLX materialized sigmoid on bf16 gates
    against an independent f64 restatement rounded at the bf16 boundaries."""
    gated, batch = 128, 4
    fused = np.zeros(batch * 2 * gated, np.float32)
    want = []
    bf = lambda v: float(oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([v], np.float32)))[0])  # noqa: E731
    for row in range(batch):
        for ch in range(gated):
            idx = row * gated + ch
            gate = bf(np.float32((idx - 256.0) / 32.0))
            value = bf(np.float32(np.sin(np.float32(idx * 0.137))) * np.float32(2.0))
            base = row * 2 * gated + ch
            fused[base], fused[base + gated] = value, gate
            exponential = bf(np.exp(abs(gate)))
            lower = bf(1.0 / bf(1.0 + exponential))
            sigmoid = lower if gate < 0 else bf(1.0 - lower)
            activated = bf(gate * sigmoid)
            want.append(bf(value * activated))
    got = oracle.bf16_to_f32(oracle.gated_act_mul(oracle.f32_to_bf16(fused), gated, batch,
                                                  oracle.SILU_MATERIALIZED_SIGMOID, t_dt=BF16))
    assert np.array_equal(got, np.array(want, np.float32))


@pytest.mark.parametrize("gclip,vclip", [((-1.0, 2.0), (-2.0, 3.0)), ((-1.0, 3.4e38), (-3.4e38, 3.0))])
def test_gated_act_mul_alpha_and_clipping(oracle, gclip, vclip):
    """gated_act_mul_test.rs:304-367: SiLU with alpha 0.5 and clipped operands."""
    values = np.array([-4.0, -1.0, 2.0, 5.0], np.float32)
    gates = np.array([-3.0, -0.5, 1.0, 4.0], np.float32)
    want = []
    for v, g in zip(values, gates):
        v = np.clip(v, *vclip)
        g = np.float32(np.clip(g, *gclip))
        want.append(np.float32(v) * np.float32(g / (np.float32(1.0) + np.exp(np.float32(-0.5) * g))))
    got = oracle.gated_act_mul(np.concatenate([values, gates]), 4, 1, oracle.SILU, alpha=0.5, gate_clip=gclip,
                               value_clip=vclip)
    assert np.allclose(got, want, rtol=1e-6)


def test_activations_closed_forms(oracle):
    a = oracle.activate
    assert a(oracle.SILU, 0.0) == 0.0 and a(oracle.SILU, 100.0) == 100.0
    assert a(oracle.GELU_EXACT, 0.0) == 0.0 and abs(a(oracle.GELU_EXACT, 1.0) - 0.8413447) < 1e-6
    assert abs(a(oracle.GELU_APPROX, 1.0) - 0.8411920) < 1e-6
    assert a(oracle.SOFTPLUS, 25.0) == 25.0 and abs(a(oracle.SOFTPLUS, 0.0) - np.log(2.0)) < 1e-7
    assert a(oracle.IDENTITY, -3.5) == -3.5


def test_int8_activations_equal_dequantized_product(oracle):
    """kernel.rs:193-205: a = q * scale in f32, so the int8 product equals the
    FullPrecision product of the f32 values q * scale exactly."""
    rng = np.random.default_rng(9)
    m, n, k, g = 3, 40, 256, 64
    for grouped in (False, True):
        codes, s, b = oracle.quantize_affine(rng.normal(0, 0.02, (n, k)).astype(np.float32), 4, 64,
                                             oracle.GROUP_OUTPUT)
        q = rng.integers(-127, 128, (m, k)).astype(np.int8)
        sc = rng.uniform(0.001, 0.05, (m, k // g)).astype(np.float32)
        order = np.array([oracle.int8_code_index(grouped, i) for i in range(k)])
        stored = np.empty_like(q)
        stored[:, order] = q
        xf = (q.astype(np.float32) * np.repeat(sc, g, axis=1)).astype(np.float32)
        common = dict(m=m, n=n, k=k, codes=codes, scales=s, correction_data=b, layout=oracle.GROUP_OUTPUT, bits=4,
                      group_size=64, output_dt=F32)
        st1, y1 = oracle.matmul(a=np.zeros(m * k, np.uint16), a_codes=stored, a_scales=sc, a_scale_group_size=g,
                                a_grouped_by_nibble=grouped, **common)
        st2, y2 = oracle.matmul(a=xf.ravel(), input_dt=F32, **common)
        assert st1 == 0 and st2 == 0 and np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    st, _ = oracle.matmul(a=np.zeros(m * k, np.uint16), a_codes=stored, a_scales=sc, a_scale_group_size=16,
                          **common)
    assert st == 3  # unsupported activation group


def test_matmul_output_rht_brute_force(oracle):
    rng = np.random.default_rng(10)
    m, n, k = 2, 64, 128
    codes, s, b = oracle.quantize_affine(rng.normal(0, 0.02, (n, k)).astype(np.float32), 4, 64, oracle.GROUP_OUTPUT)
    x = oracle.f32_to_bf16(rng.normal(0, 1, m * k).astype(np.float32))
    f = rng.choice([-1, 1], n).astype(np.int32)
    bias = oracle.f32_to_bf16(rng.normal(0, 0.3, n).astype(np.float32))
    common = dict(a=x, m=m, n=n, k=k, codes=codes, scales=s, correction_data=b, layout=oracle.GROUP_OUTPUT, bits=4,
                  group_size=64, output_dt=F32)
    st, y = oracle.matmul(**common)
    st2, yr = oracle.matmul(rht_factors=f, bias=bias, **common)
    assert st == 0 and st2 == 0
    H = sylvester()
    want = (np.einsum("ij,bsj->bsi", H, y.reshape(m, n // 32, 32).astype(np.float64)).reshape(m, n) * f
            + oracle.bf16_to_f32(bias))
    assert np.allclose(yr.reshape(m, n), want, rtol=1e-5, atol=1e-5)
    st3, _ = oracle.matmul(rht_factors=f[:48], **{**common, "n": 48, "codes": codes[:48]})
    assert st3 == 4
