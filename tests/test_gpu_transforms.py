"""GPU parity of the activation side of the quantized products, through the C
ABI, against the oracle on the same bytes:

* ActivationTransform (activation_transform.rs; CPU twin
  backends/cpu/kernel/activation_transform/activation_transform.rs:48-156):
  input RHT, output RHT (+ bias, in place) and int8 quantization, bit-exact;
* GatedActMul (gated_act_mul.rs; CPU twin gated_act_mul.rs:17-152): bit-exact
  for the identity gate and clipping; for the transcendental activations the
  device's expf/tanhf/erff/logf may differ from the host's by an ulp, so the
  bar is 4 f32 ulps before storage rounding (one storage ulp after it) and, when
  quantized, codes within one step where the rounded value moved;
* int8-activation products (MatmulA::Int8Symmetric, kernel.rs:122-141, 193-205)
  for 4/8-bit weights, both code layouts, every activation and weight group,
  every correction, against the oracle within the accumulation tolerance, plus
  the incompatible-A statuses;
* the output-RHT D-op (kernel.rs:167, 287-300) on f32 and bf16 outputs.
"""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu
F32, F16, BF16 = H.F32, H.F16, H.BF16


def _signs(rng, n):
    return rng.choice([-1, 1], n).astype(np.int32)


def _dev_empty(n, dtype):
    return torch.zeros(n, dtype=dtype, device="cuda")


def _np_storage(t, dt):
    a = t.cpu().numpy()
    return a.view(np.uint16) if dt == BF16 else a


# ------------------------------------------------------------------ ActivationTransform

@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("count", [32, 256, 4096])
def test_rht_fp(qmm, oracle, dt, count):
    rng = np.random.default_rng(count + dt)
    batch = 5
    x = H.store(oracle, rng.normal(0, 2, batch * count).astype(np.float32), dt)
    f = _signs(rng, count)
    tdt = torch.float32 if dt == F32 else torch.int16
    for op in (oracle.INPUT_RHT, oracle.OUTPUT_RHT):
        want = oracle.activation_transform(x, f, batch, count, op, t_dt=dt)
        out = _dev_empty(batch * count, tdt)
        T = qmm.ActivationTransform.input_rht(dt) if op == 0 else qmm.ActivationTransform.output_rht(dt)
        T.encode_fp(H.to_dev(x), out, H.to_dev(f), batch, count)
        torch.cuda.synchronize()
        assert np.array_equal(_np_storage(out, dt), want), f"op {op} dt {dt} count {count}"


@pytest.mark.parametrize("dt,bias_dt", [(F32, F32), (BF16, BF16), (BF16, F32)])
def test_output_rht_in_place_bias(qmm, oracle, dt, bias_dt):
    rng = np.random.default_rng(7 + dt + bias_dt)
    batch, count = 3, 512
    x = H.store(oracle, rng.normal(0, 1, batch * count).astype(np.float32), dt)
    f = _signs(rng, count)
    bias = H.store(oracle, rng.normal(0, 0.3, count).astype(np.float32), bias_dt)
    want = oracle.activation_transform(x, f, batch, count, oracle.OUTPUT_RHT, t_dt=dt, bias=bias, bias_dt=bias_dt)
    d = H.to_dev(x)
    qmm.ActivationTransform.output_rht(dt, bias_dt, in_place=True).encode_fp_in_place(d, H.to_dev(f), H.to_dev(bias),
                                                                                        batch, count)
    torch.cuda.synchronize()
    assert np.array_equal(_np_storage(d, dt), want)


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("scale_group,sum_group", [(32, 32), (64, 32), (64, 64), (128, 32), (128, 128)])
def test_quantize(qmm, oracle, dt, grouped, scale_group, sum_group):
    rng = np.random.default_rng(scale_group * 3 + sum_group + grouped + dt)
    batch, count = 4, 1024
    xs = rng.normal(0, 1, batch * count).astype(np.float32)
    xs[5] = 40.0  # one outlier group
    xs[count:count + scale_group] = 0.0  # an all-zero group: divisor 1
    x = H.store(oracle, xs, dt)
    f = _signs(rng, count)
    for sums in (False, True):
        q = qmm.ActivationQuantization.new(scale_group, sum_group, sums, int(grouped))
        assert q is not None
        op = oracle.QUANTIZE_WITH_GROUP_SUMS if sums else oracle.QUANTIZE
        wq, ws, wsum = oracle.activation_transform(x, f, batch, count, op, t_dt=dt, scale_group=scale_group,
                                                   sum_group=sum_group, grouped=grouped)
        gq = _dev_empty(batch * count, torch.int8)
        gs = _dev_empty(batch * count // scale_group, torch.float32)
        gsum = _dev_empty(batch * count // sum_group, torch.int32) if sums else None
        qmm.ActivationTransform.quantize(dt, q).encode_quantize(H.to_dev(x), gq, gs, gsum, H.to_dev(f), batch, count)
        torch.cuda.synchronize()
        assert np.array_equal(gq.cpu().numpy(), wq)
        assert np.array_equal(gs.cpu().numpy().view(np.uint32), ws.view(np.uint32))
        if sums:
            assert np.array_equal(gsum.cpu().numpy(), wsum)


def test_quantization_rules(qmm):
    """ActivationQuantization::new (activation_transform.rs:27-42) and the ABI's checks."""
    assert qmm.ActivationQuantization.new(64, 128, True) is None
    assert qmm.ActivationQuantization.new(16, 16, False) is None
    assert qmm.ActivationQuantization.new(128, 64, True).sum_group_size == 64
    assert qmm.ActivationQuantization.new(128, 64, False).sum_group_size is None
    x = _dev_empty(48, torch.float32)
    with pytest.raises(RuntimeError):  # element_count not a multiple of 32
        qmm.ActivationTransform.input_rht(F32).encode_fp(x, _dev_empty(48, torch.float32),
                                                         _dev_empty(48, torch.int32), 1, 48)


# ------------------------------------------------------------------ GatedActMul

def _storage_ulp(v, dt):
    v = np.abs(np.asarray(v, np.float64))
    e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
    return 2.0 ** (e - (7 if dt == BF16 else 23))


def _gated_tolerance(oracle, fused, gated, batch, dt, want, rht):
    """Per-output bound for a transcendental gate: 4 f32 ulps of the activation,
    |value * gate| * 2^-21 for the cancellation in 1 + erf / 1 + tanh near -1,
    two storage ulps when the storage type rounds; through the RHT each output
    takes the block's summed bound / sqrt(32) plus one storage ulp."""
    f = H.load(oracle, fused, dt).astype(np.float64).reshape(batch, 2, gated)
    v, g = f[:, 0], f[:, 1]
    w = H.load(oracle, want, dt).astype(np.float64).reshape(batch, gated)
    pre = np.abs(v * g) * 2.0 ** -21 + (4 * _storage_ulp(w, F32) if not rht else 0)
    if dt == BF16:
        pre = pre + 2 * _storage_ulp(np.abs(v * g) if rht else w, BF16)
    if rht:
        pre = np.repeat(pre.reshape(batch, gated // 32, 32).sum(-1, keepdims=True), 32, -1).reshape(batch, gated)
        pre = pre / np.sqrt(32) + _storage_ulp(w, dt) + 4 * _storage_ulp(w, F32)
    return pre


def _close(oracle, got, want, dt, tol, label):
    gv = H.load(oracle, got, dt).astype(np.float64).ravel()
    wv = H.load(oracle, want, dt).astype(np.float64).ravel()
    assert np.array_equal(np.isnan(gv), np.isnan(wv)), label
    ok = ~np.isnan(wv)
    err = np.abs(gv[ok] - wv[ok])
    bad = err > tol.ravel()[ok]
    assert not bad.any(), f"{label}: {int(bad.sum())} outside; worst {err.max()}"


ACTS = ["SILU", "GELU_APPROX", "GELU_EXACT", "IDENTITY", "SOFTPLUS", "SILU_MATERIALIZED_SIGMOID",
        "GELU_MATERIALIZED_POLYNOMIAL"]


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("act", ACTS)
def test_gated_fp_interleaved(qmm, oracle, dt, act):
    rng = np.random.default_rng(ACTS.index(act) * 2 + dt)
    gated, batch = 256, 6
    fused = H.store(oracle, rng.normal(0, 3, batch * 2 * gated).astype(np.float32), dt)
    t = getattr(oracle, act)
    tdt = torch.float32 if dt == F32 else torch.int16
    for use_rht in (False, True):
        f = _signs(rng, gated) if use_rht else None
        want = oracle.gated_act_mul(fused, gated, batch, t, t_dt=dt, factors=f)
        out = _dev_empty(batch * gated, tdt)
        qmm.GatedActMul.full_precision(dt, True, use_rht).encode_fp(
            H.to_dev(fused), None, out, None if f is None else H.to_dev(f), gated, batch, 0, 0, t)
        torch.cuda.synchronize()
        got = _np_storage(out, dt)
        if act == "IDENTITY":
            assert np.array_equal(got, want)
        else:
            tol = _gated_tolerance(oracle, fused, gated, batch, dt, want, use_rht)
            _close(oracle, got, want, dt, tol, f"{act} rht={use_rht}")


def test_gated_separate_operand_kat(qmm, oracle):
    """gated_act_mul_test.rs:235-256: identity gate, values at value_offset in
    rows of value_row_stride."""
    for dt in (F32, BF16):
        gate = H.store(oracle, np.array([1.0, 2.0, 3.0, 4.0], np.float32), dt)
        value = H.store(oracle, np.array([0, 0, 10, 20, 30, 40, 0, 0, 50, 60, 70, 80], np.float32), dt)
        out = _dev_empty(4, torch.float32 if dt == F32 else torch.int16)
        qmm.GatedActMul.full_precision(dt, False, False).encode_fp(H.to_dev(gate), H.to_dev(value), out, None, 2, 2, 2,
                                                                   6, qmm.ACT_IDENTITY)
        torch.cuda.synchronize()
        assert np.array_equal(H.load(oracle, _np_storage(out, dt), dt), [10.0, 40.0, 150.0, 240.0])


@pytest.mark.parametrize("gclip,vclip", [((-1.0, 2.0), (-2.0, 3.0)), ((-1.0, 3.4e38), (-3.4e38, 3.0))])
def test_gated_alpha_and_clipping(qmm, oracle, gclip, vclip):
    """gated_act_mul_test.rs:304-367 shape: SiLU with alpha 0.5 and clipped operands."""
    rng = np.random.default_rng(11)
    gated, batch = 64, 3
    fused = rng.normal(0, 3, batch * 2 * gated).astype(np.float32)
    want = oracle.gated_act_mul(fused, gated, batch, oracle.SILU, alpha=0.5, gate_clip=gclip, value_clip=vclip)
    out = _dev_empty(batch * gated, torch.float32)
    s = qmm.GatedActMulSettings(activation_alpha=0.5, gate_clipping=gclip, value_clipping=vclip)
    qmm.GatedActMul.full_precision(F32, True, False, s).encode_fp(H.to_dev(fused), None, out, None, gated, batch, 0,
                                                                  0, qmm.ACT_SILU)
    torch.cuda.synchronize()
    tol = _gated_tolerance(oracle, fused, gated, batch, F32, want, False)
    _close(oracle, out.cpu().numpy(), want, F32, tol, "alpha/clip")


@pytest.mark.parametrize("dt", [F32, BF16])
@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("scale_group,sum_group", [(32, 32), (128, 64)])
def test_gated_quantized(qmm, oracle, dt, grouped, scale_group, sum_group):
    """The A8 producer: SwiGLU, RHT, int8 codes per scale group. Identity gates
    are bit-exact; SiLU codes may move by one step where a value sits on a
    rounding boundary."""
    rng = np.random.default_rng(scale_group + sum_group * 5 + grouped + dt)
    gated, batch = 512, 4
    fused = H.store(oracle, rng.normal(0, 2, batch * 2 * gated).astype(np.float32), dt)
    f = _signs(rng, gated)
    for act in (oracle.IDENTITY, oracle.SILU):
        for sums in (False, True):
            q = qmm.ActivationQuantization.new(scale_group, sum_group, sums, int(grouped))
            op = oracle.GAM_QUANTIZE_WITH_GROUP_SUMS if sums else oracle.GAM_QUANTIZE
            wq, ws, wsum = oracle.gated_act_mul(fused, gated, batch, act, t_dt=dt, op=op, factors=f,
                                                scale_group=scale_group, sum_group=sum_group, grouped=grouped)
            gq = _dev_empty(batch * gated, torch.int8)
            gs = _dev_empty(batch * gated // scale_group, torch.float32)
            gsum = _dev_empty(batch * gated // sum_group, torch.int32) if sums else None
            qmm.GatedActMul.quantized(dt, q).encode_quantized(H.to_dev(fused), gq, gs, gsum, H.to_dev(f), gated, batch,
                                                              act)
            torch.cuda.synchronize()
            label = f"act {act} sums {sums}"
            if act == oracle.IDENTITY:
                assert np.array_equal(gq.cpu().numpy(), wq), label
                assert np.array_equal(gs.cpu().numpy(), ws), label
                if sums:
                    assert np.array_equal(gsum.cpu().numpy(), wsum), label
            else:
                # a bf16 gate output that rounds the other way moves its block's
                # RHT values by ~2^-8 |v| / sqrt(32): scales within 2e-3 there
                assert np.allclose(gs.cpu().numpy(), ws, rtol=1e-5 if dt == F32 else 2e-3, atol=0), label
                dq = np.abs(gq.cpu().numpy().astype(np.int32) - wq.astype(np.int32))
                assert dq.max() <= 1 and (dq > 0).mean() < 0.05, label
                if sums:
                    assert np.abs(gsum.cpu().numpy() - wsum).max() <= sum_group // 8, label


# ------------------------------------------------------------------ int8-activation products

def _a8_inputs(oracle, rng, m, k, ag, grouped):
    x = rng.normal(0, 1, m * k).astype(np.float32)
    f = np.ones(k, np.int32)
    # codes and scales as the quantizing transform writes them (after an RHT)
    q, sc, _ = oracle.activation_transform(x, f, m, k, oracle.QUANTIZE, scale_group=ag, grouped=grouped)
    return q, sc


def _a8_case(qmm, oracle, rng, m, n, k, bits, wg, ag, grouped, correction=1, signed=False, out_dt=F32, w_dt=BF16,
             gather=None, bank=None, rht=False, bias=False, label=""):
    rows = bank or n
    w = H.affine_weights(oracle, rng, rows, k, bits=bits, gs=wg, layout=0, correction=correction, w_dt=w_dt,
                         quantizer=(correction == 1 and w_dt == BF16))
    q, sc = _a8_inputs(oracle, rng, m, k, ag, grouped)
    f = _signs(rng, n) if rht else None
    bv = H.store(oracle, rng.normal(0, 0.2, n).astype(np.float32), w_dt) if bias else None
    st, want = oracle.matmul(a=np.zeros(m * k, np.uint16), m=m, n=n, k=k, codes=w["codes"], scales=w["scales"],
                             correction=correction, correction_data=w["corr"], layout=0, row_count=rows,
                             group_count=k // wg, bits=bits, group_size=wg, signed_codes=signed, output_dt=out_dt,
                             weights_dt=w_dt, a_codes=q, a_scales=sc, a_scale_group_size=ag,
                             a_grouped_by_nibble=grouped, gather=gather, rht_factors=f, bias=bv, threads=8)
    assert st == 0, label
    d = _dev_empty(m * n, torch.float32 if out_dt == F32 else torch.int16)
    b = qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                       params=qmm.QuantParams(layout=0, row_count=rows, group_count=k // wg),
                       mode=qmm.MODE_U4 if bits == 4 else qmm.MODE_U8, group_size=wg, correction=correction,
                       correction_data=None if w["corr"] is None else H.to_dev(w["corr"]), signed_codes=signed)
    A = qmm.Int8SymmetricA(values=H.to_dev(q), scales=H.to_dev(sc), scale_group_size=ag,
                           code_layout=qmm.GROUPED_BY_NIBBLE if grouped else qmm.SEQUENTIAL)
    dops = qmm.MatmulDOps(rht_factors=None if f is None else H.to_dev(f), bias=None if bv is None else H.to_dev(bv))
    qmm.MatmulKernel(w_dt, BF16, out_dt).encode(qmm.MatmulArguments(
        a=A, b=b, d=d, m=m, n=n, k=k, d_transform=dops,
        gather_indices=None if gather is None else H.to_dev(np.asarray(gather, np.uint32))))
    torch.cuda.synchronize()
    got = _np_storage(d, out_dt)
    if out_dt == BF16:
        got, want = oracle.bf16_to_f32(got), oracle.bf16_to_f32(want)
    xf = (q.astype(np.float32).reshape(m, k)[:, [oracle.int8_code_index(grouped, i) for i in range(k)]]
          * np.repeat(sc.reshape(m, k // ag), ag, axis=1)).astype(np.float32)
    mag = H.dequant_magnitude(oracle, w["codes"], w["scales"], w["corr"], rows, k, bits, wg, 0, correction, w_dt,
                              xf.ravel(), F32, m, gather=gather, signed=signed, out_n=n)
    if rht:  # the RHT mixes 32 outputs: bound by the block's summed magnitude / sqrt(32)
        mag = np.repeat(mag.reshape(m, n // 32, 32).sum(-1, keepdims=True), 32, axis=-1) / np.sqrt(32)
    check(got, want, mag=mag, label=label)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("ag,wg", [(32, 32), (64, 32), (128, 64), (32, 128), (128, 128)])
def test_a8_products(qmm, oracle, bits, grouped, ag, wg):
    rng = np.random.default_rng(bits * 1000 + ag * 7 + wg + grouped)
    for m in (1, 5, 17):
        _a8_case(qmm, oracle, rng, m, 96, 512, bits, wg, ag, grouped, label=f"m{m}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("correction", [0, 1, 2])
def test_a8_corrections_and_signed(qmm, oracle, bits, correction):
    rng = np.random.default_rng(bits * 10 + correction)
    for signed in (False, True):
        _a8_case(qmm, oracle, rng, 3, 64, 256, bits, 64, 64, bits == 4, correction=correction, signed=signed,
                 label=f"corr {correction} signed {signed}")


def test_a8_generic_forms(qmm, oracle):
    """Gathered rows and rows whose packed length is not 16-byte aligned run
    the per-output kernel."""
    rng = np.random.default_rng(21)
    n, bank, k = 40, 70, 96
    gather = rng.integers(0, bank, 2 * n).astype(np.uint32)
    _a8_case(qmm, oracle, rng, 2, n, k, 4, 32, 32, True, gather=gather, bank=bank, label="gather")
    _a8_case(qmm, oracle, rng, 3, 33, 96, 4, 32, 32, False, label="k96")
    _a8_case(qmm, oracle, rng, 2, 31, 160, 8, 32, 32, True, label="k160 8-bit")


@pytest.mark.parametrize("out_dt", [F32, BF16])
def test_a8_output_dtypes_and_rht(qmm, oracle, out_dt):
    """The A8W4 layer shape: int8 activations, output RHT and a bias after it."""
    rng = np.random.default_rng(31 + out_dt)
    for m in (1, 4):
        _a8_case(qmm, oracle, rng, m, 128, 1024, 4, 64, 128, True, out_dt=out_dt, rht=True, bias=True,
                 label=f"rht m{m}")
        _a8_case(qmm, oracle, rng, m, 64, 512, 8, 128, 128, False, out_dt=out_dt, bias=True, label=f"bias m{m}")


def test_a8_full_width_row(qmm, oracle):
    """A full model row: K = 4096, N = 1024, M = 2 with the nibble-grouped layout."""
    rng = np.random.default_rng(41)
    _a8_case(qmm, oracle, rng, 2, 1024, 4096, 4, 64, 128, True, label="k4096")


def test_a8_incompatible(qmm, oracle):
    """kernel.rs:130-141: the activation group must be 32/64/128 and divide K,
    B a 4- or 8-bit quantized matrix with group 32/64/128."""
    rng = np.random.default_rng(51)
    m, n, k = 1, 32, 256
    w = H.affine_weights(oracle, rng, n, k, bits=4, gs=64)
    q, sc = _a8_inputs(oracle, rng, m, k, 64, False)
    d = _dev_empty(m * n, torch.float32)
    kern = qmm.MatmulKernel(BF16, BF16, F32)

    def b(mode=qmm.MODE_U4, gs=64):
        return qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                              params=qmm.QuantParams(layout=0, row_count=n, group_count=k // gs), mode=mode,
                              group_size=gs, correction=1, correction_data=H.to_dev(w["corr"]))

    def run(bb, ag=64):
        A = qmm.Int8SymmetricA(values=H.to_dev(q), scales=H.to_dev(sc), scale_group_size=ag)
        return qmm.lib().stark_qmm_encode(kern._h, qmm.C.byref(qmm._args(qmm.MatmulArguments(
            a=A, b=bb, d=d, m=m, n=n, k=k))), qmm._stream(None))
    assert run(b()) == qmm.OK
    assert run(b(), ag=16) == qmm.INCOMPATIBLE_A
    assert run(b(), ag=96) == qmm.INCOMPATIBLE_A
    assert run(b(gs=16)) == qmm.INCOMPATIBLE_A
    assert run(qmm.FullPrecisionB(values=_dev_empty(n * k, torch.int16))) == qmm.INCOMPATIBLE_A
    torch.cuda.synchronize()


def test_output_rht_statuses(qmm, oracle):
    rng = np.random.default_rng(61)
    m, n, k = 1, 48, 128
    w = H.affine_weights(oracle, rng, n, k, bits=4, gs=64)
    x = H.to_dev(H.activations(oracle, rng, m, k))
    b = qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                       params=qmm.QuantParams(layout=0, row_count=n, group_count=k // 64), mode=qmm.MODE_U4,
                       group_size=64, correction=1, correction_data=H.to_dev(w["corr"]))
    f = H.to_dev(np.ones(n, np.int32))
    for out_dt, nn in ((F16, 32), (F32, 48)):
        d = _dev_empty(m * nn, torch.float32)
        args = qmm.MatmulArguments(a=x, b=b, d=d, m=m, n=nn, k=k, d_transform=qmm.MatmulDOps(rht_factors=f))
        kern = qmm.MatmulKernel(BF16, BF16, out_dt)  # held: the handle lives as long as the object
        st = qmm.lib().stark_qmm_encode(kern._h, qmm.C.byref(qmm._args(args)), qmm._stream(None))
        assert st == qmm.UNSUPPORTED_D_OP


@pytest.mark.parametrize("out_dt", [F32, BF16])
@pytest.mark.parametrize("m", [1, 3, 40])
def test_output_rht_dop_full_precision_a(qmm, oracle, out_dt, m):
    """bf16 activations (GEMV and, at M = 40, the GEMM) followed by the output RHT and bias."""
    rng = np.random.default_rng(71 + m + out_dt)
    n, k = 256, 512
    w = H.affine_weights(oracle, rng, n, k, bits=4, gs=64)
    x = H.activations(oracle, rng, m, k)
    f = _signs(rng, n)
    bv = H.store(oracle, rng.normal(0, 0.2, n).astype(np.float32), BF16)
    kern = qmm.MatmulKernel(BF16, BF16, out_dt)
    kern.set_reference_accumulation(True)  # f32-dequant products, the oracle's semantics at every M
    st, want = oracle.matmul(a=x, m=m, n=n, k=k, codes=w["codes"], scales=w["scales"], correction=1,
                             correction_data=w["corr"], layout=0, row_count=n, group_count=k // 64, bits=4,
                             group_size=64, output_dt=out_dt, rht_factors=f, bias=bv, threads=8)
    assert st == 0
    d = _dev_empty(m * n, torch.float32 if out_dt == F32 else torch.int16)
    b = qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                       params=qmm.QuantParams(layout=0, row_count=n, group_count=k // 64), mode=qmm.MODE_U4,
                       group_size=64, correction=1, correction_data=H.to_dev(w["corr"]))
    kern.encode(qmm.MatmulArguments(a=H.to_dev(x), b=b, d=d, m=m, n=n, k=k,
                                    d_transform=qmm.MatmulDOps(rht_factors=H.to_dev(f), bias=H.to_dev(bv))))
    torch.cuda.synchronize()
    got = _np_storage(d, out_dt)
    if out_dt == BF16:
        got, want = oracle.bf16_to_f32(got), oracle.bf16_to_f32(want)
    mag = H.dequant_magnitude(oracle, w["codes"], w["scales"], w["corr"], n, k, 4, 64, 0, 1, BF16, x, BF16, m)
    mag = np.repeat(mag.reshape(m, n // 32, 32).sum(-1, keepdims=True), 32, axis=-1) / np.sqrt(32)
    check(got, want, mag=mag, label=f"rht m{m}")


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("ag,wg,grouped", [(128, 64, True), (64, 64, False), (32, 32, True), (128, 32, False),
                                           (32, 128, True)])
def test_a8_prefill_gemm(qmm, oracle, bits, ag, wg, grouped):
    """M > 16 runs the int8 GEMM on v_mfma_i32_16x16x64_i8 (partial tiles in
    M, N and K steps), against the oracle within the accumulation bar."""
    rng = np.random.default_rng(bits * 31 + ag + wg + grouped)
    for m, n, k in ((40, 136, 512), (130, 96, 384)):
        _a8_case(qmm, oracle, rng, m, n, k, bits, wg, ag, grouped, label=f"gemm m{m} n{n} k{k}")
    _a8_case(qmm, oracle, rng, 33, 64, 256, bits, wg, ag, grouped, correction=0, signed=True, label="sym signed")
    _a8_case(qmm, oracle, rng, 20, 64, 256, bits, wg, ag, grouped, bias=True, rht=True, out_dt=BF16, label="rht bf16")


def test_a8_prefill_full_width(qmm, oracle):
    """The A8W4 prefill shape: M = 2048, N = 4096, K = 4096 (activation groups
    128, weight groups 64, grouped codes), 24 sampled rows against the oracle."""
    rng = np.random.default_rng(77)
    m, n, k, ag, wg = 2048, 4096, 4096, 128, 64
    w = H.affine_weights(oracle, rng, n, k, bits=4, gs=wg)
    q, sc = _a8_inputs(oracle, rng, m, k, ag, True)
    d = _dev_empty(m * n, torch.float32)
    b = qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                       params=qmm.QuantParams(layout=0, row_count=n, group_count=k // wg), mode=qmm.MODE_U4,
                       group_size=wg, correction=qmm.BIASES, correction_data=H.to_dev(w["corr"]))
    A = qmm.Int8SymmetricA(values=H.to_dev(q), scales=H.to_dev(sc), scale_group_size=ag,
                           code_layout=qmm.GROUPED_BY_NIBBLE)
    qmm.MatmulKernel(BF16, BF16, F32).encode(qmm.MatmulArguments(a=A, b=b, d=d, m=m, n=n, k=k))
    torch.cuda.synchronize()
    got = d.cpu().numpy().reshape(m, n)
    rows = np.concatenate([[0, m - 1], rng.choice(np.arange(1, m - 1), 22, replace=False)])
    qs = q.reshape(m, k)[rows].ravel()
    ss = sc.reshape(m, k // ag)[rows].ravel()
    st, want = oracle.matmul(a=np.zeros(len(rows) * k, np.uint16), m=len(rows), n=n, k=k, codes=w["codes"],
                             scales=w["scales"], correction=1, correction_data=w["corr"], layout=0, row_count=n,
                             group_count=k // wg, bits=4, group_size=wg, output_dt=F32, a_codes=qs, a_scales=ss,
                             a_scale_group_size=ag, a_grouped_by_nibble=True, threads=8)
    assert st == 0
    xf = (qs.astype(np.float32).reshape(len(rows), k)[:, [oracle.int8_code_index(True, i) for i in range(k)]]
          * np.repeat(ss.reshape(len(rows), k // ag), ag, axis=1)).astype(np.float32)
    mag = H.dequant_magnitude(oracle, w["codes"], w["scales"], w["corr"], n, k, 4, wg, 0, 1, BF16, xf.ravel(), F32,
                              len(rows))
    check(got[rows].ravel(), want, mag=mag, label="a8 prefill full width")


def test_a8_prefill_batch_matches_single(qmm, oracle):
    """stark_qmm_encode_many with int8-activation products of M > 16: one GEMM
    grid per (bits, flush group, signed codes, code layout) class, each entry
    with its own activations, gives the bits of one launch per product.
    Ragged M, N and K; the D-ops on one entry; entries of three classes."""
    rng = np.random.default_rng(55)
    kern = qmm.MatmulKernel(BF16, BF16, BF16)
    # (m, n, k, bits, wg, ag, grouped, d-ops)
    specs = [(40, 136, 512, 4, 64, 128, True, False), (130, 96, 1024, 4, 64, 64, True, True),
             (300, 256, 256, 4, 64, 128, True, False), (17, 64, 384, 8, 64, 64, False, False),
             (64, 200, 512, 8, 64, 128, False, False), (33, 520, 256, 4, 64, 128, True, False)]
    made = []
    for m, n, k, bits, wg, ag, grouped, dops in specs:
        w = H.affine_weights(oracle, rng, n, k, bits=bits, gs=wg)
        q, sc = _a8_inputs(oracle, rng, m, k, ag, grouped)
        prior = H.to_dev(oracle.f32_to_bf16(rng.normal(0, 1, m * n).astype(np.float32))) if dops else None
        bias = H.to_dev(oracle.f32_to_bf16(rng.normal(0, 0.2, n).astype(np.float32))) if dops else None
        made.append((m, n, k, bits, wg, ag, grouped, w, H.to_dev(q), H.to_dev(sc), prior, bias))

    def args(m, n, k, bits, wg, ag, grouped, w, q, sc, prior, bias):
        b = qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                           params=qmm.QuantParams(layout=0, row_count=n, group_count=k // wg),
                           mode=qmm.MODE_U4 if bits == 4 else qmm.MODE_U8, group_size=wg, correction=qmm.BIASES,
                           correction_data=H.to_dev(w["corr"]))
        A = qmm.Int8SymmetricA(values=q, scales=sc, scale_group_size=ag,
                               code_layout=qmm.GROUPED_BY_NIBBLE if grouped else qmm.SEQUENTIAL)
        d = prior.clone() if prior is not None else _dev_empty(m * n, torch.int16)
        dops = qmm.MatmulDOps(ab_scale=0.5, accumulate=True, bias=bias) if prior is not None else qmm.MatmulDOps()
        return qmm.MatmulArguments(a=A, b=b, d=d, m=m, n=n, k=k, d_transform=dops)
    many = [args(*t) for t in made]
    kern.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        kern.encode(a)
    torch.cuda.synchronize()
    for a, b, t in zip(many, single, made):
        assert torch.equal(a.d, b.d), f"batched and single differ for m={t[0]} n={t[1]} k={t[2]} bits={t[3]}"
    assert any(bool((a.d != 0).any()) for a in many)


def test_a8_prefill_split_into_row_launches(qmm, oracle):
    """An int8-activation product too tall for one grid's 32-bit offsets
    (K = 12288: 174592 rows per grid) runs as launches of whole rows; rows on
    both sides of the split against the oracle."""
    m, n, k, ag, wg = 174592 + 300, 64, 12288, 128, 64
    rng = np.random.default_rng(174)
    w = H.affine_weights(oracle, rng, n, k, bits=4, gs=wg)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(174)
    q = torch.randint(-127, 128, (m * k,), generator=gen, device="cuda", dtype=torch.int8)
    sc = torch.rand(m * k // ag, generator=gen, device="cuda") * 0.02 + 1e-3
    d = _dev_empty(m * n, torch.float32)
    b = qmm.QuantizedB(codes=H.to_dev(w["codes"]), scales=H.to_dev(w["scales"]),
                       params=qmm.QuantParams(layout=0, row_count=n, group_count=k // wg), mode=qmm.MODE_U4,
                       group_size=wg, correction=qmm.BIASES, correction_data=H.to_dev(w["corr"]))
    A = qmm.Int8SymmetricA(values=q, scales=sc, scale_group_size=ag, code_layout=qmm.SEQUENTIAL)
    qmm.MatmulKernel(BF16, BF16, F32).encode(qmm.MatmulArguments(a=A, b=b, d=d, m=m, n=n, k=k))
    torch.cuda.synchronize()
    rows = np.array([0, 174591, 174592, m - 1])
    ri = torch.from_numpy(rows).cuda()
    qs = q.view(m, k)[ri].cpu().numpy().ravel()
    ss = sc.view(m, k // ag)[ri].cpu().numpy().ravel()
    got = d.view(m, n)[ri].cpu().numpy().ravel()
    st, want = oracle.matmul(a=np.zeros(len(rows) * k, np.uint16), m=len(rows), n=n, k=k, codes=w["codes"],
                             scales=w["scales"], correction=1, correction_data=w["corr"], layout=0, row_count=n,
                             group_count=k // wg, bits=4, group_size=wg, output_dt=F32, a_codes=qs, a_scales=ss,
                             a_scale_group_size=ag, a_grouped_by_nibble=False, threads=8)
    assert st == 0
    xf = (qs.astype(np.float32).reshape(len(rows), k) * np.repeat(ss.reshape(len(rows), k // ag), ag, axis=1))
    mag = H.dequant_magnitude(oracle, w["codes"], w["scales"], w["corr"], n, k, 4, wg, 0, 1, BF16,
                              xf.astype(np.float32).ravel(), F32, len(rows))
    check(got, want, mag=mag, label="row-split a8 gemm")
