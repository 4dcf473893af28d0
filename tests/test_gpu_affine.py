"""GPU parity of the affine (MLX-style) quantized matmul path against the CPU
oracle (restating MatmulCpuKernel::encode,
crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:58-303), through the
C ABI (stark_qmm_encode / stark_qmm_encode_many)."""
import json
import os

import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KAT = json.load(open(os.path.join(HERE, "golden", "kat_vectors.json")))


def np_dtype(dt):
    return np.float32 if dt == H.F32 else np.uint16


def torch_empty(n, dt):
    return torch.zeros(n, dtype=torch.float32 if dt == H.F32 else torch.int16, device="cuda")


def run_case(Q, O, *, m, n, k, bits=4, gs=64, layout=0, correction=1, w_dt=H.BF16, x_dt=H.BF16, d_dt=H.BF16,
             signed=False, gather=None, bank_rows=None, ab_scale=1.0, accumulate=False, with_bias=False,
             soft_cap=None, seed=0, quantizer=True, label=""):
    rng = np.random.default_rng(seed)
    rows = n if bank_rows is None else bank_rows
    W = H.affine_weights(O, rng, rows, k, bits, gs, layout, correction, w_dt, quantizer=quantizer)
    x = H.activations(O, rng, m, k, x_dt)
    prior = H.store(O, rng.normal(0, 1, m * n).astype(np.float32), d_dt) if accumulate else None
    bias = H.store(O, rng.normal(0, 0.5, n).astype(np.float32), w_dt) if with_bias else None
    G = k // gs
    mode = {4: Q.MODE_U4, 8: Q.MODE_U8}.get(bits, {3: Q.MODE_U3, 5: Q.MODE_U5, 6: Q.MODE_U6}.get(bits))
    st, want = O.matmul(a=x, m=m, n=n, k=k, codes=W["codes"], scales=W["scales"], correction=correction,
                        correction_data=W["corr"], layout=layout, row_count=rows, group_count=G, bits=bits,
                        group_size=gs, signed_codes=signed, d=prior, ab_scale=ab_scale, accumulate=accumulate,
                        bias=bias, soft_cap=soft_cap, gather=gather, weights_dt=w_dt, input_dt=x_dt, output_dt=d_dt,
                        threads=8)
    assert st == 0
    d = H.to_dev(prior) if prior is not None else torch_empty(m * n, d_dt)
    args = Q.MatmulArguments(
        a=H.to_dev(x), m=m, n=n, k=k, d=d,
        b=Q.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                       params=Q.QuantParams(layout, rows, G), mode=mode, group_size=gs, correction=correction,
                       correction_data=None if W["corr"] is None else H.to_dev(W["corr"]), signed_codes=signed),
        d_transform=Q.MatmulDOps(ab_scale=ab_scale, accumulate=accumulate,
                                 bias=None if bias is None else H.to_dev(bias), soft_cap=soft_cap),
        gather_indices=None if gather is None else H.to_dev(np.asarray(gather, np.uint32)))
    kern = Q.MatmulKernel(w_dt, x_dt, d_dt)
    kern.encode(args)
    torch.cuda.synchronize()
    got = H.load(O, H.from_dev(d, np_dtype(d_dt)), d_dt)
    mag = H.dequant_magnitude(O, W["codes"], W["scales"], W["corr"], rows, k, bits, gs, layout, correction, w_dt, x,
                              x_dt, m, gather=gather, signed=signed, out_n=n)
    if accumulate or with_bias:
        mag = mag * abs(ab_scale) + 4.0
    check(got, H.load(O, want, d_dt), mag=mag, label=label or f"m{m} n{n} k{k} b{bits} g{gs}")
    return got, H.load(O, want, d_dt)


# --------------------------------------------------------------- headline shapes

@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("d_dt", [H.BF16, H.F32])
def test_config0_w4_matvec(qmm, oracle, layout, d_dt):
    """Benchmark config 0 (the reference's CPU-runnable case): N=3072, K=1024, W4 g64, M=1."""
    run_case(qmm, oracle, m=1, n=3072, k=1024, layout=layout, d_dt=d_dt, seed=1)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
def test_qwen3_8b_shapes_small_m(qmm, oracle, m):
    """Config-1 widths at reduced N (full-size runs are in bench/property tests)."""
    for n, k in ((256, 4096), (96, 12288)):
        run_case(qmm, oracle, m=m, n=n, k=k, layout=1, seed=m * 7 + k)


@pytest.mark.parametrize("k", [32, 96, 2048, 4160, 8192 + 512])
def test_partial_passes_and_tails(qmm, oracle, k):
    run_case(qmm, oracle, m=2, n=45, k=k, gs=32, seed=k)


@pytest.mark.parametrize("bits,gs", [(4, 32), (4, 128), (8, 16), (8, 32), (8, 64), (8, 128)])
def test_bits_and_groups(qmm, oracle, bits, gs):
    run_case(qmm, oracle, m=1, n=70, k=1024, bits=bits, gs=gs, seed=bits * gs)
    run_case(qmm, oracle, m=5, n=33, k=2048, bits=bits, gs=gs, layout=1, seed=bits * gs + 1)


@pytest.mark.parametrize("correction", [0, 1, 2])
@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("signed", [False, True])
def test_corrections_layouts_signed(qmm, oracle, correction, layout, signed):
    for bits in (4, 8):
        run_case(qmm, oracle, m=2, n=37, k=512, bits=bits, layout=layout, correction=correction, signed=signed,
                 quantizer=False, seed=correction * 4 + layout * 2 + signed + bits)


@pytest.mark.parametrize("x_dt", [H.BF16, H.F16, H.F32])
@pytest.mark.parametrize("w_dt", [H.BF16, H.F16, H.F32])
@pytest.mark.parametrize("d_dt", [H.BF16, H.F16, H.F32])
def test_dtypes(qmm, oracle, x_dt, w_dt, d_dt):
    run_case(qmm, oracle, m=1, n=40, k=512, w_dt=w_dt, x_dt=x_dt, d_dt=d_dt, quantizer=False, seed=x_dt + w_dt + d_dt)


def test_d_ops(qmm, oracle):
    run_case(qmm, oracle, m=3, n=50, k=1024, ab_scale=0.75, accumulate=True, with_bias=True, soft_cap=4.0,
             d_dt=H.F32, seed=3)
    run_case(qmm, oracle, m=1, n=50, k=1024, ab_scale=2.0, with_bias=True, seed=4)


@pytest.mark.parametrize("m", [1, 3])
def test_gather(qmm, oracle, m):
    """gather_indices remap output (m, n) to weight row gather[m*n+n]
    (kernel.rs:172-176); a row outside the codes buffer gives NaN."""
    rng = np.random.default_rng(20 + m)
    bank, n, k = 200, 64, 1024
    g = rng.integers(0, bank, m * n).astype(np.uint32)
    run_case(qmm, oracle, m=m, n=n, k=k, gather=g, bank_rows=bank, seed=m)


def test_gather_out_of_bank_is_nan(qmm, oracle):
    rng = np.random.default_rng(0)
    bank, n, k = 64, 32, 512
    W = H.affine_weights(oracle, rng, bank, k)
    x = H.activations(oracle, rng, 1, k)
    g = np.arange(n, dtype=np.uint32)
    g[5] = 1000
    d = torch_empty(n, H.F32)
    args = qmm.MatmulArguments(a=H.to_dev(x), m=1, n=n, k=k, d=d, gather_indices=H.to_dev(g),
                               b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                                                params=qmm.QuantParams(0, bank, k // 64),
                                                correction_data=H.to_dev(W["corr"])))
    qmm.MatmulKernel(H.BF16, H.BF16, H.F32).encode(args)
    out = d.cpu().numpy()
    assert np.isnan(out[5]) and not np.isnan(np.delete(out, 5)).any()


# --------------------------------------------------------------- exact-value cases

def test_packed_tail_kats_on_gpu(qmm, oracle):
    """reference.rs:240-245 run through the GPU generic path: exact outputs."""
    for c in KAT["packed_tails"]["cases"]:
        k, n, bits = c["k"], c["n"], c["bits"]
        d = torch_empty(n, H.F32)
        args = qmm.MatmulArguments(
            a=torch.ones(k, dtype=torch.float32, device="cuda"), m=1, n=n, k=k, d=d,
            b=qmm.QuantizedB(codes=H.to_dev(np.array(c["codes"], np.uint8)),
                             scales=torch.ones(n, dtype=torch.float32, device="cuda"),
                             params=qmm.QuantParams(0, n, 1), mode=qmm.MODE_U8 if bits == 8 else qmm.MODE_U4,
                             group_size=k, correction=qmm.SYMMETRIC))
        qmm.MatmulKernel(H.F32, H.F32, H.F32).encode(args)
        assert d.cpu().tolist() == c["expected"]
    # undersized codes -> UnsupportedLayout, nothing launched
    args = qmm.MatmulArguments(
        a=torch.ones(2, dtype=torch.float32, device="cuda"), m=1, n=1, k=2, d=torch_empty(1, H.F32),
        b=qmm.QuantizedB(codes=torch.zeros(1, dtype=torch.uint8, device="cuda"),
                         scales=torch.ones(1, dtype=torch.float32, device="cuda"), params=qmm.QuantParams(0, 1, 1),
                         mode=qmm.MODE_U8, group_size=2, correction=qmm.SYMMETRIC))
    with pytest.raises(qmm.MatmulError) as e:
        qmm.MatmulKernel(H.F32, H.F32, H.F32).encode(args)
    assert e.value.status == qmm.UNSUPPORTED_LAYOUT


@pytest.mark.parametrize("bits", [3, 5, 6])
def test_odd_bit_widths_generic(qmm, oracle, bits):
    run_case(qmm, oracle, m=2, n=17, k=192, bits=bits, gs=64, correction=1, quantizer=False, seed=bits)


@pytest.mark.parametrize("case", KAT["materialized_affine_input_sum"]["cases"],
                         ids=lambda c: c["scenario"] + str(c["materialize"]))
def test_materialized_affine_input_sum_on_gpu(qmm, oracle, case):
    """affine_input_sum_test.rs:133-196: the CPU-backend exact values. The
    non-materialized 'quad' case runs the fast GEMV; its exact value holds
    because every partial sum there is exactly representable."""
    from tests.test_oracle_kats import materialized_case
    a = materialized_case(oracle, case["scenario"], case["materialize"])
    n, k = a["n"], a["k"]
    d = torch_empty(n, H.BF16)
    args = qmm.MatmulArguments(
        a=H.to_dev(a["a"]), m=1, n=n, k=k, d=d,
        b=qmm.QuantizedB(codes=H.to_dev(a["codes"]), scales=H.to_dev(a["scales"]),
                         params=qmm.QuantParams(0, n, k // 64, case["materialize"]), group_size=64,
                         correction_data=H.to_dev(a["correction_data"])))
    qmm.MatmulKernel(H.BF16, H.BF16, H.BF16).encode(args)
    got = oracle.bf16_to_f32(H.from_dev(d, np.uint16))
    assert np.all(got == case["expected_all"]), got[:4]


def test_error_paths(qmm, oracle):
    rng = np.random.default_rng(1)
    W = H.affine_weights(oracle, rng, 8, 128)
    base = dict(a=H.to_dev(H.activations(oracle, rng, 1, 128)), m=1, n=8, k=128, d=torch_empty(8, H.F32))

    def b(**kw):
        args = dict(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=qmm.QuantParams(0, 8, 2),
                    correction_data=H.to_dev(W["corr"]))
        args.update(kw)
        return qmm.QuantizedB(**args)

    k = qmm.MatmulKernel(H.BF16, H.BF16, H.F32)
    with pytest.raises(qmm.MatmulError) as e:
        k.encode(qmm.MatmulArguments(b=b(), d_transform=qmm.MatmulDOps(rht_factors=torch.zeros(8, device="cuda")),
                                     **base))
    assert e.value.status == qmm.UNSUPPORTED_D_OP
    with pytest.raises(qmm.MatmulError) as e:
        k.encode(qmm.MatmulArguments(b=b(params=qmm.QuantParams(0, 8, 2, True)), **base))
    assert e.value.status == qmm.UNSUPPORTED_LAYOUT  # materialize needs bf16 output
    with pytest.raises(qmm.MatmulError) as e:
        k.encode(qmm.MatmulArguments(b=b(group_size=0), **base))
    assert e.value.status == qmm.UNSUPPORTED_GROUP_SIZE
    with pytest.raises(qmm.MatmulError) as e:
        qmm.MatmulKernel(H.BF16, H.BF16, 2)
    assert e.value.status == qmm.UNSUPPORTED_DATA_TYPE


def test_empty_products_are_no_ops(qmm, oracle):
    """m = 0 or n = 0: the reference's loops run zero times and return Ok
    (kernel.rs:168-285); nothing is written (the output keeps its bits), alone
    and inside a batch with a real product."""
    rng = np.random.default_rng(3)
    W = H.affine_weights(oracle, rng, 64, 256)
    x = H.to_dev(H.activations(oracle, rng, 2, 256))
    k = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)

    def args(m, n, d):
        return qmm.MatmulArguments(
            a=x, m=m, n=n, k=256, d=d,
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(0, 64, 4), correction_data=H.to_dev(W["corr"])))
    for m, n in [(0, 64), (1, 0), (0, 0), (2, 0)]:
        d = torch_empty(128, H.BF16)
        d.fill_(0x1234)
        k.encode(args(m, n, d))
        torch.cuda.synchronize()
        assert bool((d == 0x1234).all()), (m, n)
    d0, d1 = torch_empty(64, H.BF16), torch_empty(64, H.BF16)
    d0.fill_(0x1234)
    k.encode_many([args(0, 64, d0), args(1, 64, d1)])
    torch.cuda.synchronize()
    assert bool((d0 == 0x1234).all())
    st, want = oracle.matmul(a=H.from_dev(x, np.uint16)[:256], m=1, n=64, k=256, codes=W["codes"],
                             scales=W["scales"], correction=1, correction_data=W["corr"], layout=0, row_count=64,
                             group_count=4, bits=4, group_size=64, output_dt=H.BF16, threads=1)
    assert st == 0
    assert np.array_equal(H.from_dev(d1, np.uint16), want) or np.allclose(
        H.load(oracle, H.from_dev(d1, np.uint16), H.BF16), H.load(oracle, want, H.BF16), rtol=2 ** -7, atol=1e-3)


def test_encode_many_matches_single(qmm, oracle):
    """stark_qmm_encode_many: one launch for several independent products
    (the config-1 layer set at reduced N) equals one encode per product."""
    rng = np.random.default_rng(9)
    shapes = [(256, 4096), (64, 4096), (64, 4096), (256, 4096), (512, 4096), (512, 4096), (256, 12288)]
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    many, single = [], []
    for n, k in shapes:
        W = H.affine_weights(oracle, rng, n, k, layout=1)
        x = H.to_dev(H.activations(oracle, rng, 1, k))
        mk = lambda d: qmm.MatmulArguments(
            a=x, m=1, n=n, k=k, d=d,
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(1, n, k // 64), correction_data=H.to_dev(W["corr"])))
        many.append(mk(torch_empty(n, H.BF16)))
        single.append(mk(torch_empty(n, H.BF16)))
    kern.encode_many(many)
    for a in single:
        kern.encode(a)
    torch.cuda.synchronize()
    for a, b in zip(many, single):
        assert torch.equal(a.d, b.d)


@pytest.mark.parametrize("n,k,gs", [(40, 4160, 32), (64, 8192 + 512, 64), (1000, 12288, 128), (3072, 1024, 64)])
@pytest.mark.parametrize("m", [1, 2])
@pytest.mark.parametrize("layout", [0, 1])
def test_streaming_kernel_shapes(qmm, oracle, n, k, gs, m, layout):
    """Shapes the persistent streaming kernel takes (4-bit, bf16 activations,
    N % 8 == 0): partial passes, a shifted last tile (N % 32 != 0), both plane
    layouts."""
    run_case(qmm, oracle, m=m, n=n, k=k, gs=gs, layout=layout, seed=n + k + m)


@pytest.mark.parametrize("correction,signed", [(0, False), (1, True), (0, True)])
def test_streaming_kernel_corrections(qmm, oracle, correction, signed):
    run_case(qmm, oracle, m=1, n=72, k=4096, correction=correction, signed=signed, quantizer=False, seed=5)
    run_case(qmm, oracle, m=2, n=72, k=4096, correction=correction, signed=signed, quantizer=False, w_dt=H.F16,
             seed=6)


def test_streaming_kernel_d_ops_on_shifted_tile(qmm, oracle):
    """N=40: the last 32-row tile overlaps the first; accumulate must add once."""
    run_case(qmm, oracle, m=1, n=40, k=2048, ab_scale=0.5, accumulate=True, with_bias=True, d_dt=H.F32, seed=8)
    run_case(qmm, oracle, m=2, n=40, k=2048, accumulate=True, soft_cap=2.0, d_dt=H.BF16, seed=9)


@pytest.mark.parametrize("n,k", [(16, 4096), (40, 4096), (72, 8192), (1000, 12288), (3072, 4096), (24, 16384)])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("layout", [0, 1])
def test_decode_stream_kernel_shapes(qmm, oracle, n, k, bits, layout):
    """Shapes of the one-row streaming kernel (M = 1, group 64, K % 4096 == 0):
    one to four 1024-k units per wave and tile (K = 16384 cycles the three
    activation regions), a shifted last tile (N % 16 != 0), both plane
    layouts, 4- and 8-bit codes."""
    run_case(qmm, oracle, m=1, n=n, k=k, bits=bits, layout=layout, seed=n + k + bits + 3 * layout)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("correction,signed", [(0, False), (1, True), (0, True)])
def test_decode_stream_kernel_corrections(qmm, oracle, bits, correction, signed):
    run_case(qmm, oracle, m=1, n=72, k=4096, bits=bits, correction=correction, signed=signed, quantizer=False,
             seed=15)
    run_case(qmm, oracle, m=1, n=72, k=8192, bits=bits, correction=correction, signed=signed, quantizer=False,
             w_dt=H.F16, layout=1, seed=16)


def test_decode_stream_kernel_d_ops_on_shifted_tile(qmm, oracle):
    """N=40: the last 16-row tile overlaps the previous one; accumulate must add once."""
    run_case(qmm, oracle, m=1, n=40, k=4096, ab_scale=0.5, accumulate=True, with_bias=True, d_dt=H.F32, seed=18)
    run_case(qmm, oracle, m=1, n=40, k=8192, bits=8, accumulate=True, soft_cap=2.0, d_dt=H.BF16, seed=19)
    # 12288-deep launch with fewer tiles than CUs: the twelve-wave workgroups
    run_case(qmm, oracle, m=1, n=40, k=12288, ab_scale=0.5, accumulate=True, with_bias=True, d_dt=H.F32, seed=20)
    run_case(qmm, oracle, m=1, n=4096, k=12288, correction=0, signed=True, quantizer=False, seed=21)


@pytest.mark.parametrize("bits", [4, 8])
def test_decode_stream_kernel_layer_set_against_oracle(qmm, oracle, bits):
    """One launch over a reduced layer set (q, k, v, o, gate, up, down): ops of
    one K with distinct activations and ops sharing one activation vector;
    every output against the oracle (the per-wave activation regions are tagged
    by op and chunk)."""
    rng = np.random.default_rng(21 + bits)
    shapes = [(256, 4096), (64, 4096), (64, 4096), (256, 4096), (512, 4096), (512, 4096), (256, 12288)]
    xs = {4096: H.activations(oracle, rng, 1, 4096), 12288: H.activations(oracle, rng, 1, 12288)}
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    args, wants = [], []
    for i, (n, k) in enumerate(shapes):
        W = H.affine_weights(oracle, rng, n, k, bits, 64, layout=i % 2)
        x = xs[k] if i in (1, 2) else H.activations(oracle, rng, 1, k)  # k_proj and v_proj share x
        st, want = oracle.matmul(a=x, m=1, n=n, k=k, codes=W["codes"], scales=W["scales"], correction=1,
                                 correction_data=W["corr"], layout=i % 2, row_count=n, group_count=k // 64,
                                 bits=bits, group_size=64, output_dt=H.BF16, threads=8)
        assert st == 0
        mode = qmm.MODE_U4 if bits == 4 else qmm.MODE_U8
        args.append(qmm.MatmulArguments(
            a=H.to_dev(x), m=1, n=n, k=k, d=torch_empty(n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(i % 2, n, k // 64), mode=mode,
                             correction_data=H.to_dev(W["corr"]))))
        mag = H.dequant_magnitude(oracle, W["codes"], W["scales"], W["corr"], n, k, bits, 64, i % 2, 1, H.BF16, x,
                                  H.BF16, 1, out_n=n)
        wants.append((want, mag))
    kern.encode_many(args)
    torch.cuda.synchronize()
    for i, (a, (want, mag)) in enumerate(zip(args, wants)):
        got = H.load(oracle, H.from_dev(a.d, np.uint16), H.BF16)
        check(got, H.load(oracle, want, H.BF16), mag=mag, label=f"op {i} bits {bits}")


@pytest.mark.parametrize("bits", [4])
def test_decode_stream_kernel_many_tiles_repeated(qmm, oracle, bits):
    """More 32-row tiles than the streaming kernel has workgroups (several
    tiles per workgroup list, ops of two K), three launches in a row, outputs
    pre-filled with NaN so that a tile no workgroup takes shows; a ragged last
    tile in every op."""
    rng = np.random.default_rng(77)
    shapes = [(20000 + 8, 4096, 1), (4000 + 24, 8192, 0), (1000 + 16, 4096, 1)]
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    ops = []
    for n, k, layout in shapes:
        W = H.affine_weights(oracle, rng, n, k, bits, 64, layout=layout)
        x = H.activations(oracle, rng, 1, k)
        st, want = oracle.matmul(a=x, m=1, n=n, k=k, codes=W["codes"], scales=W["scales"], correction=1,
                                 correction_data=W["corr"], layout=layout, row_count=n, group_count=k // 64,
                                 bits=bits, group_size=64, output_dt=H.BF16, threads=8)
        assert st == 0
        mag = H.dequant_magnitude(oracle, W["codes"], W["scales"], W["corr"], n, k, bits, 64, layout, 1, H.BF16,
                                  x, H.BF16, 1, out_n=n)
        ops.append((n, k, layout, W, x, want, mag))
    for rep in range(3):
        args = []
        for n, k, layout, W, x, _, _ in ops:
            d = torch_empty(n, H.BF16)
            d.fill_(0x7FC0)  # bf16 NaN bits
            args.append(qmm.MatmulArguments(
                a=H.to_dev(x), m=1, n=n, k=k, d=d,
                b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                                 params=qmm.QuantParams(layout, n, k // 64), mode=qmm.MODE_U4,
                                 correction_data=H.to_dev(W["corr"]))))
        kern.encode_many(args)
        torch.cuda.synchronize()
        for i, (a, (n, k, layout, W, x, want, mag)) in enumerate(zip(args, ops)):
            got = H.load(oracle, H.from_dev(a.d, np.uint16), H.BF16)
            check(got, H.load(oracle, want, H.BF16), mag=mag, label=f"launch {rep} op {i}")


@pytest.mark.parametrize("n,k,gs", [(80, 4160, 32), (64, 8192 + 512, 64), (1040, 12288, 128), (3072, 1024, 64),
                                    (96, 96, 32)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16])
@pytest.mark.parametrize("layout", [0, 1])
def test_matrix_core_kernel_shapes(qmm, oracle, n, k, gs, m, layout):
    """Shapes the 4-bit matrix-core kernel takes (bf16 activations, N % 16 == 0,
    N >= 64, M <= 16): every activation-row class (1, 2, 4, 8 and two blocks of
    8), partial steps and passes, a shifted last 64-row tile."""
    run_case(qmm, oracle, m=m, n=n, k=k, gs=gs, layout=layout, seed=n + k + m + 7 * layout)


@pytest.mark.parametrize("n,k", [(16, 1024), (40, 4096), (1000, 2048), (96, 12288)])
@pytest.mark.parametrize("m", [3, 4, 5, 8, 9, 12, 16])
@pytest.mark.parametrize("layout", [0, 1])
def test_small_m_dense_kernel_shapes(qmm, oracle, n, k, m, layout):
    """M = 3 .. 16, 4-bit, group 64, K % 1024 == 0 takes the dense small-M
    kernel (all 16 activation rows per MFMA, two 16-row tiles per step): one
    tile, a pair with a shifted second tile, ragged N, long K."""
    run_case(qmm, oracle, m=m, n=n, k=k, gs=64, layout=layout, seed=n + k + 3 * m + layout)


@pytest.mark.parametrize("correction,signed,w_dt", [(0, False, H.BF16), (1, True, H.F16), (0, True, H.F16)])
def test_small_m_dense_kernel_corrections(qmm, oracle, correction, signed, w_dt):
    run_case(qmm, oracle, m=11, n=72, k=2048, gs=64, correction=correction, signed=signed, w_dt=w_dt,
             seed=17 + correction + 2 * signed)


def test_small_m_dense_kernel_d_ops(qmm, oracle):
    run_case(qmm, oracle, m=16, n=40, k=1024, gs=64, ab_scale=0.75, accumulate=True, with_bias=True,
             soft_cap=30.0, seed=5)


def test_small_m_dense_kernel_batch_matches_single(qmm, oracle):
    """Three dense-eligible ops (N = 48, 17, 64) in one launch give the bits
    of three single launches (the op search by first block)."""
    rng = np.random.default_rng(31)
    k = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    specs = [(12, 48, 1024), (12, 17, 1024), (12, 64, 2048)]
    made = []
    for m, n, kk in specs:
        W = H.affine_weights(oracle, rng, n, kk, 4, 64, layout=1)
        x = H.to_dev(H.activations(oracle, rng, m, kk))
        made.append((m, n, kk, W, x))

    def args(m, n, kk, W, x):
        return qmm.MatmulArguments(
            a=x, m=m, n=n, k=kk, d=torch_empty(m * n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(1, n, kk // 64), correction_data=H.to_dev(W["corr"])))
    many = [args(*t) for t in made]
    k.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        k.encode(a)
    torch.cuda.synchronize()
    for a, b in zip(many, single):
        assert torch.equal(a.d, b.d)


@pytest.mark.parametrize("n,k", [(9000, 4096), (32010, 1024)])
@pytest.mark.parametrize("m", [8, 16])
def test_small_m_dense_kernel_runs(qmm, oracle, n, k, m):
    """Launches with more tile pairs than resident workgroups: a workgroup
    runs several pairs pass by pass (three at N = 9000, K = 4096; two at
    N = 32010, K = 1024, whose last run holds one pair with a shifted tile)."""
    run_case(qmm, oracle, m=m, n=n, k=k, gs=64, layout=1, seed=n + k + m)


@pytest.mark.parametrize("variant", ["symmetric", "f16_planes", "signed", "output_group", "m3", "d_ops"])
def test_small_m_dense_kernel_runs_variants(qmm, oracle, variant):
    """The multi-pair runs (N = 9000, K = 4096: three pairs per workgroup)
    with each plane, code and output variant: symmetric codes (no bias
    plane), f16 planes, signed codes, per-row planes, an odd M, and the
    D-ops on a run's shifted last tile."""
    kw = dict(m=8, n=9000, k=4096, gs=64, layout=1, seed=300 + len(variant))
    kw.update({"symmetric": dict(correction=0), "f16_planes": dict(w_dt=H.F16), "signed": dict(signed=True),
               "output_group": dict(layout=0), "m3": dict(m=3),
               "d_ops": dict(m=5, ab_scale=0.5, accumulate=True, with_bias=True, soft_cap=20.0)}[variant])
    run_case(qmm, oracle, **kw)


def test_small_m_dense_kernel_run_length_keeps_bits(qmm, oracle):
    """A K = 12288 product and a K = 4096 product in one launch run one pair
    per workgroup; alone, the K = 4096 product runs three. Every output row
    keeps its bits."""
    rng = np.random.default_rng(37)
    k = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    made = []
    for n, kk in [(4096, 12288), (12288, 4096)]:
        W = H.affine_weights(oracle, rng, n, kk, 4, 64, layout=1)
        x = H.to_dev(H.activations(oracle, rng, 8, kk))
        made.append((n, kk, W, x))

    def args(n, kk, W, x):
        return qmm.MatmulArguments(
            a=x, m=8, n=n, k=kk, d=torch_empty(8 * n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(1, n, kk // 64), correction_data=H.to_dev(W["corr"])))
    many = [args(*t) for t in made]
    k.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        k.encode(a)
    torch.cuda.synchronize()
    for a, b in zip(many, single):
        assert torch.equal(a.d, b.d)


@pytest.mark.parametrize("correction,signed", [(0, False), (1, True), (0, True)])
@pytest.mark.parametrize("m", [1, 4, 16])
def test_matrix_core_kernel_corrections(qmm, oracle, correction, signed, m):
    run_case(qmm, oracle, m=m, n=144, k=4096, correction=correction, signed=signed, quantizer=False, seed=5 + m)
    run_case(qmm, oracle, m=m, n=144, k=4096, correction=correction, signed=signed, quantizer=False, w_dt=H.F16,
             seed=6 + m)


@pytest.mark.parametrize("m", [1, 2, 6, 12])
def test_matrix_core_kernel_d_ops_on_shifted_tile(qmm, oracle, m):
    """N=80: the last 64-row tile overlaps the first; accumulate must add once."""
    run_case(qmm, oracle, m=m, n=80, k=2048, ab_scale=0.5, accumulate=True, with_bias=True, d_dt=H.F32, seed=8)
    run_case(qmm, oracle, m=m, n=80, k=2048, accumulate=True, soft_cap=2.0, d_dt=H.BF16, seed=9)


# --------------------------------------------------------------- prefill GEMM

def bf16_effective_reference(O, W, x, m, n, k, bits, gs, layout, correction, w_dt, signed):
    """f64 product with the weights the GEMM multiplies: w = bf16_rne(f32(q)*s + bias_term)
    (backends/cpu/kernel/matmul/vision.rs:249-336 for biases; the symmetric bias
    term -s*2^(bits-1) and the signed-code XOR as kernel.rs:219-265)."""
    codes = W["codes"][: n * k * bits // 8]
    if bits == 4:
        q = np.stack([codes & 15, codes >> 4], axis=-1).reshape(n, k).astype(np.int64)
    else:
        q = codes.reshape(n, k).astype(np.int64)
    if signed:
        q ^= 1 << (bits - 1)
    G = k // gs
    s = H.load(O, W["scales"], w_dt).astype(np.float32)
    s = s.reshape(n, G) if layout == 0 else s.reshape(G, -1)[:, :n].T
    if correction == 1:
        b = H.load(O, W["corr"], w_dt).astype(np.float32)
        b = b.reshape(n, G) if layout == 0 else b.reshape(G, -1)[:, :n].T
    else:
        b = -s * np.float32(1 << (bits - 1))
    w = q.astype(np.float32) * np.repeat(s, gs, 1) + np.repeat(b, gs, 1)  # exact product, one rounding
    w = O.bf16_to_f32(O.f32_to_bf16(w.astype(np.float32).ravel())).reshape(n, k).astype(np.float64)
    xf = H.load(O, x, H.BF16).astype(np.float64).reshape(m, k)
    return xf @ w.T, np.abs(xf) @ np.abs(w).T


def _ref_strides(layout, n, k):
    return (k // 64, 1) if layout == 0 else (1, (n + 3) // 4 * 4)


def test_prefill_gemm_full_width(qmm, oracle):
    """Config-4 prefill at full width: M = 2048, N = 12288, K = 4096, 4-bit g64
    with GroupOutput planes (the converted artifact's layout), bf16 output.
    Rows 0, 2047 and 14 random rows against the oracle's BF16-effective
    reference dot (vision.rs:249-336) on every column."""
    m, n, k = 2048, 12288, 4096
    rng = np.random.default_rng(2048)
    W = H.affine_weights(oracle, rng, n, k, 4, 64, 1, 1, H.BF16)
    x = H.activations(oracle, rng, m, k, H.BF16)
    d = torch_empty(m * n, H.BF16)
    qmm.MatmulKernel(H.BF16, H.BF16, H.BF16).encode(qmm.MatmulArguments(a=H.to_dev(x), m=m, n=n, k=k, d=d, b=qmm.QuantizedB(
        codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=qmm.QuantParams(1, n, k // 64),
        mode=qmm.MODE_U4, correction_data=H.to_dev(W["corr"]))))
    torch.cuda.synchronize()
    got = oracle.bf16_to_f32(H.from_dev(d, np.uint16)).reshape(m, n)
    rows = np.concatenate([[0, m - 1], rng.choice(np.arange(1, m - 1), 14, replace=False)])
    xs = x.reshape(m, k)[rows].ravel()
    sos, sgs = _ref_strides(1, n, k)
    ref = oracle.reference_affine_linear_bf16(xs, W["codes"], W["scales"], W["corr"], len(rows), n, k, bits=4,
                                              sos=sos, sgs=sgs, f32_out=True).reshape(len(rows), n)
    _, mag = bf16_effective_reference(oracle, W, xs, len(rows), n, k, 4, 64, 1, 1, H.BF16, False)
    check(got[rows].ravel(), ref.ravel(), mag=mag.ravel(), label="full-width prefill")


@pytest.mark.parametrize("m,n,k", [(17, 96, 512), (64, 256, 1024), (200, 300, 4096), (2048, 128, 256), (520, 136, 320),
                                   (130, 1000, 192)])
@pytest.mark.parametrize("bits", [4, 8])
def test_prefill_gemm_shapes(qmm, oracle, m, n, k, bits):
    """M > 16 runs the matrix-core dequant-GEMM (4-bit g64 products of at most
    32 rows with K % 512 == 0 the skinny product, same arithmetic):
    bf16-effective weights, f32 accumulation. Checked against the f64 product of the same bf16 weights, and
    against the exact-f32 CPU kernel at the reference's own GPU/CPU bar
    (quant_dispatch_test.rs:189: rel 0.05 / abs 0.4)."""
    rng = np.random.default_rng(m * 7 + n + bits)
    layout = 1 if (m + bits) % 2 else 0
    W = H.affine_weights(oracle, rng, n, k, bits, 64, layout, 1, H.BF16)
    x = H.activations(oracle, rng, m, k, H.BF16)
    d = torch_empty(m * n, H.F32)
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.F32)
    mode = qmm.MODE_U4 if bits == 4 else qmm.MODE_U8
    kern.encode(qmm.MatmulArguments(a=H.to_dev(x), m=m, n=n, k=k, d=d, b=qmm.QuantizedB(
        codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=qmm.QuantParams(layout, n, k // 64),
        mode=mode, correction_data=H.to_dev(W["corr"]))))
    torch.cuda.synchronize()
    got = H.from_dev(d, np.float32).reshape(m, n)
    want, mag = bf16_effective_reference(oracle, W, x, m, n, k, bits, 64, layout, 1, H.BF16, False)
    check(got.ravel(), want.ravel(), mag=mag.ravel(), label=f"gemm m{m} n{n} k{k} b{bits}")
    # the oracle's restatement of the reference's BF16-effective dot (vision.rs:249-336)
    sos, sgs = _ref_strides(layout, n, k)
    ref = oracle.reference_affine_linear_bf16(x, W["codes"], W["scales"], W["corr"], m, n, k, bits=bits, sos=sos,
                                              sgs=sgs, f32_out=True)
    check(got.ravel(), ref, mag=mag.ravel(), label=f"gemm vs reference dot m{m} n{n} k{k} b{bits}")
    st, exact = oracle.matmul(a=x, m=m, n=n, k=k, codes=W["codes"], scales=W["scales"], correction_data=W["corr"],
                              layout=layout, bits=bits, group_size=64, output_dt=H.F32, threads=8)
    assert st == 0
    assert np.all(np.abs(got.ravel() - exact) <= 0.05 * np.abs(exact) + 0.4)


def _skinny_case(qmm, oracle, m, n, k, *, layout=1, correction=1, signed=False, w_dt=H.BF16, seed=0, d_dt=H.F32,
                 ab_scale=1.0, accumulate=False, with_bias=False, soft_cap=None):
    """A 4-bit g64 product of 17 .. 32 rows (the skinny product) against the
    f64 product of the bf16-effective weights, at the prefill bar."""
    rng = np.random.default_rng(seed)
    W = H.affine_weights(oracle, rng, n, k, 4, 64, layout, correction, w_dt)
    x = H.activations(oracle, rng, m, k, H.BF16)
    prior = rng.normal(0, 1, m * n).astype(np.float32) if accumulate else None
    bias = H.store(oracle, rng.normal(0, 0.5, n).astype(np.float32), w_dt) if with_bias else None
    d = H.to_dev(H.store(oracle, prior, d_dt)) if accumulate else torch_empty(m * n, d_dt)
    kern = qmm.MatmulKernel(w_dt, H.BF16, d_dt)
    kern.encode(qmm.MatmulArguments(a=H.to_dev(x), m=m, n=n, k=k, d=d, b=qmm.QuantizedB(
        codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=qmm.QuantParams(layout, n, k // 64),
        mode=qmm.MODE_U4, correction=correction, signed_codes=signed,
        correction_data=None if W["corr"] is None else H.to_dev(W["corr"])),
        d_transform=qmm.MatmulDOps(ab_scale=ab_scale, accumulate=accumulate,
                                   bias=None if bias is None else H.to_dev(bias), soft_cap=soft_cap)))
    torch.cuda.synchronize()
    got = H.load(oracle, H.from_dev(d, np_dtype(d_dt)), d_dt).reshape(m, n).astype(np.float64)
    want, mag = bf16_effective_reference(oracle, W, x, m, n, k, 4, 64, layout, correction, w_dt, signed)
    want = want * ab_scale
    if accumulate:
        want = want + H.load(oracle, H.store(oracle, prior, d_dt), d_dt).reshape(m, n)
    if with_bias:
        want = want + H.load(oracle, bias, w_dt)[None, :n]
        mag = mag + 4.0
    if soft_cap is not None:
        want = soft_cap * np.tanh(want / soft_cap)
    check(got.ravel(), want.ravel(), mag=(mag * abs(ab_scale) + (4.0 if accumulate else 0.0)).ravel(),
          label=f"skinny m{m} n{n} k{k}")


@pytest.mark.parametrize("m,n,k", [(17, 16, 512), (24, 40, 1536), (32, 1000, 4096), (20, 9000, 4096),
                                   (32, 96, 12288), (31, 32010, 512), (33, 72, 1024), (48, 1000, 4096),
                                   (64, 9000, 4096)])
@pytest.mark.parametrize("layout", [0, 1])
def test_skinny_product_shapes(qmm, oracle, m, n, k, layout):
    """17 .. 64 rows, 4-bit g64, K % 512 == 0: the skinny product (one tile
    pair; ragged N; runs of several pairs at N = 9000 and 32010; deep K;
    33 .. 64 rows as two 32-row blocks, the second one short)."""
    _skinny_case(qmm, oracle, m, n, k, layout=layout, seed=m + n + k + layout)


@pytest.mark.parametrize("variant", ["symmetric", "signed", "signed_symmetric", "f16_planes", "bf16_out", "d_ops"])
def test_skinny_product_variants(qmm, oracle, variant):
    kw = {"symmetric": dict(correction=0), "signed": dict(signed=True),
          "signed_symmetric": dict(correction=0, signed=True),
          "f16_planes": dict(w_dt=H.F16), "bf16_out": dict(d_dt=H.BF16),
          "d_ops": dict(ab_scale=0.75, accumulate=True, with_bias=True, soft_cap=30.0)}[variant]
    _skinny_case(qmm, oracle, 27, 9000, 4096, seed=400 + len(variant), **kw)


def test_skinny_product_batch_matches_single(qmm, oracle):
    """A K = 12288 and a K = 4096 product of 32 rows in one launch (one pair
    per workgroup) give the bits of two single launches (three pairs per
    workgroup for the K = 4096 one)."""
    rng = np.random.default_rng(41)
    k = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    made = []
    for n, kk in [(4096, 12288), (12288, 4096)]:
        W = H.affine_weights(oracle, rng, n, kk, 4, 64, layout=1)
        x = H.to_dev(H.activations(oracle, rng, 32, kk))
        made.append((n, kk, W, x))

    def args(n, kk, W, x):
        return qmm.MatmulArguments(
            a=x, m=32, n=n, k=kk, d=torch_empty(32 * n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(1, n, kk // 64), correction_data=H.to_dev(W["corr"])))
    many = [args(*t) for t in made]
    k.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        k.encode(a)
    torch.cuda.synchronize()
    for a, b in zip(many, single):
        assert torch.equal(a.d, b.d)


def test_encode_many_mixed_row_classes_match_single(qmm, oracle):
    """One encode_many call over products of 1, 2, 8, 24, 48 and 100 rows (the
    streaming kernel, the slot form, the small-M kernel, both skinny classes
    and the GEMM) gives each product the bits of its own encode call."""
    rng = np.random.default_rng(43)
    k = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    made = []
    for m, n, kk in [(1, 4096, 4096), (2, 1000, 4096), (8, 96, 4096), (24, 1000, 4096), (48, 96, 1024),
                     (100, 256, 1024)]:
        W = H.affine_weights(oracle, rng, n, kk, 4, 64, layout=1)
        x = H.to_dev(H.activations(oracle, rng, m, kk))
        made.append((m, n, kk, W, x))

    def args(m, n, kk, W, x):
        return qmm.MatmulArguments(
            a=x, m=m, n=n, k=kk, d=torch_empty(m * n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(1, n, kk // 64), correction_data=H.to_dev(W["corr"])))
    many = [args(*t) for t in made]
    k.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        k.encode(a)
    torch.cuda.synchronize()
    for (m, n, kk, _, _), a, b in zip(made, many, single):
        assert torch.equal(a.d, b.d), f"m{m} n{n} k{kk}"


def test_encode_many_row_classes_in_graph_replays(qmm, oracle):
    """encode_many over products of 1, 8, 24 and 48 rows recorded in a HIP graph:
    three replays, with eager launches and synchronizations between them, each
    give the eager call's bits."""
    rng = np.random.default_rng(47)
    k = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    made = []
    for m, n, kk in [(1, 2080, 4096), (8, 1000, 4096), (24, 1000, 2048), (48, 136, 1024)]:
        W = H.affine_weights(oracle, rng, n, kk, 4, 64, layout=1)
        made.append((m, n, kk, W, H.to_dev(H.activations(oracle, rng, m, kk))))

    def args(m, n, kk, W, x):
        return qmm.MatmulArguments(
            a=x, m=m, n=n, k=kk, d=torch_empty(m * n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(1, n, kk // 64), correction_data=H.to_dev(W["corr"])))
    eager = [args(*t) for t in made]
    k.encode_many(eager)
    torch.cuda.synchronize()
    cap = [args(*t) for t in made]
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        k.encode_many(cap, stream=s)
    for rep in range(3):
        for a in cap:
            a.d.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for (m, n, kk, _, _), a, b in zip(made, cap, eager):
            assert torch.equal(a.d, b.d), f"replay {rep}: m{m} n{n} k{kk}"
        k.encode_many([args(*made[0])])  # eager work between the replays


@pytest.mark.parametrize("correction,signed,w_dt,gs", [(0, False, H.BF16, 64), (1, True, H.F16, 32),
                                                       (0, True, H.BF16, 128), (1, False, H.F16, 64)])
@pytest.mark.parametrize("m", [40, 200])  # 40: skinny (group 64) or 128x64 GEMM tiles; 200: 128x128 tiles
def test_prefill_gemm_corrections(qmm, oracle, correction, signed, w_dt, gs, m):
    n, k = 160, 512
    rng = np.random.default_rng(gs + correction)
    for layout in (0, 1):
        W = H.affine_weights(oracle, rng, n, k, 4, gs, layout, correction, w_dt, quantizer=False)
        x = H.activations(oracle, rng, m, k, H.BF16)
        d = torch_empty(m * n, H.BF16)
        kern = qmm.MatmulKernel(w_dt, H.BF16, H.BF16)
        kern.encode(qmm.MatmulArguments(a=H.to_dev(x), m=m, n=n, k=k, d=d, b=qmm.QuantizedB(
            codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=qmm.QuantParams(layout, n, k // gs),
            group_size=gs, correction=correction, signed_codes=signed,
            correction_data=None if W["corr"] is None else H.to_dev(W["corr"]))))
        torch.cuda.synchronize()
        got = H.load(oracle, H.from_dev(d, np.uint16), H.BF16)
        want, mag = bf16_effective_reference(oracle, W, x, m, n, k, 4, gs, layout, correction, w_dt, signed)
        check(got, want.ravel(), mag=mag.ravel(), label=f"gemm corr{correction} s{signed} l{layout}")


def test_prefill_gemm_d_ops_and_reference_mode(qmm, oracle):
    """D-ops in the GEMM epilogue; with set_reference_accumulation the same
    product takes the f32-dequant path and meets the exact oracle's bar."""
    m, n, k = 33, 130, 256
    rng = np.random.default_rng(3)
    W = H.affine_weights(oracle, rng, n, k, 4, 64, 1, 1, H.BF16)
    x = H.activations(oracle, rng, m, k, H.BF16)
    prior = rng.normal(0, 1, m * n).astype(np.float32)
    bias = oracle.f32_to_bf16(rng.normal(0, 0.5, n).astype(np.float32))
    for reference in (False, True):
        d = H.to_dev(prior.copy())
        kern = qmm.MatmulKernel(H.BF16, H.BF16, H.F32)
        kern.set_reference_accumulation(reference)
        kern.encode(qmm.MatmulArguments(a=H.to_dev(x), m=m, n=n, k=k, d=d, b=qmm.QuantizedB(
            codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]), params=qmm.QuantParams(1, n, k // 64),
            correction_data=H.to_dev(W["corr"])), d_transform=qmm.MatmulDOps(ab_scale=0.5, accumulate=True,
                                                                              bias=H.to_dev(bias), soft_cap=3.0)))
        torch.cuda.synchronize()
        got = H.from_dev(d, np.float32)
        st, want = oracle.matmul(a=x, m=m, n=n, k=k, codes=W["codes"], scales=W["scales"],
                                 correction_data=W["corr"], layout=1, bits=4, group_size=64, output_dt=H.F32,
                                 d=prior.copy(), ab_scale=0.5, accumulate=True, bias=bias, soft_cap=3.0)
        assert st == 0
        if reference:
            mag = H.dequant_magnitude(oracle, W["codes"], W["scales"], W["corr"], n, k, 4, 64, 1, 1, H.BF16, x,
                                      H.BF16, m, out_n=n)
            check(got, want, mag=mag * 0.5 + 4.0, label="reference mode")
        else:
            assert np.all(np.abs(got - want) <= 0.05 * np.abs(want) + 0.4)


def test_prefill_gemm_batch_matches_single(qmm, oracle):
    """stark_qmm_encode_many with M > 16 products: one dequant-GEMM grid per
    (bits, signed codes, correction, plane type) class, ops longest K first,
    gives the bits of one launch per product (the same tile code, found by
    block index). Ragged M, N and K, both layouts, 4- and 8-bit, both
    corrections, signed codes, and the D-ops on one entry."""
    rng = np.random.default_rng(77)
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    # (m, n, k, bits, layout, correction, signed, d-ops)
    specs = [(200, 300, 512, 4, 1, 1, False, False), (40, 1024, 1536, 4, 0, 1, False, True),
             (130, 96, 256, 4, 1, 1, False, False), (17, 136, 320, 8, 0, 1, False, False),
             (300, 256, 1024, 8, 1, 1, False, False), (64, 64, 512, 4, 1, 0, True, False),
             (72, 520, 192, 4, 0, 0, True, False), (256, 128, 2048, 4, 1, 1, False, False)]
    made = []
    for m, n, kk, bits, layout, corr, signed, dops in specs:
        W = H.affine_weights(oracle, rng, n, kk, bits, 64, layout, corr, H.BF16, quantizer=False)
        x = H.to_dev(H.activations(oracle, rng, m, kk))
        prior = H.to_dev(oracle.f32_to_bf16(rng.normal(0, 1, m * n).astype(np.float32))) if dops else None
        bias = H.to_dev(oracle.f32_to_bf16(rng.normal(0, 0.5, n).astype(np.float32))) if dops else None
        made.append((m, n, kk, bits, layout, corr, signed, W, x, prior, bias))

    def args(m, n, kk, bits, layout, corr, signed, W, x, prior, bias):
        d = prior.clone() if prior is not None else torch_empty(m * n, H.BF16)
        return qmm.MatmulArguments(
            a=x, m=m, n=n, k=kk, d=d,
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(layout, n, kk // 64), mode=qmm.MODE_U4 if bits == 4 else qmm.MODE_U8,
                             correction=corr, signed_codes=signed,
                             correction_data=None if W["corr"] is None else H.to_dev(W["corr"])),
            d_transform=qmm.MatmulDOps(ab_scale=0.75, accumulate=True, bias=bias) if prior is not None else qmm.MatmulDOps())
    many = [args(*t) for t in made]
    kern.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        kern.encode(a)
    torch.cuda.synchronize()
    for a, b, t in zip(many, single, made):
        assert torch.equal(a.d, b.d), f"batched and single differ for m={t[0]} n={t[1]} k={t[2]} bits={t[3]}"
    # and the batch against the f64 product of the bf16-effective weights
    for a, t in zip(many, made):
        m, n, kk, bits, layout, corr, signed, W, x, prior, bias = t
        if prior is not None:
            continue
        got = H.load(oracle, H.from_dev(a.d, np.uint16), H.BF16)
        want, mag = bf16_effective_reference(oracle, W, H.from_dev(x, np.uint16), m, n, kk, bits, 64, layout, corr,
                                             H.BF16, signed)
        check(got, want.ravel(), mag=mag.ravel(), label=f"batched gemm m{m} n{n} k{kk} b{bits}")


@pytest.mark.parametrize("w_dt,gs", [(H.F16, 32), (H.F16, 128), (H.BF16, 128), (H.BF16, 32)])
def test_prefill_gemm_batch_plane_types_and_groups(qmm, oracle, w_dt, gs):
    """One-grid prefill batches with f16 or bf16 planes and group sizes 32 and
    128 (the group of a thread's codes found from the step's k and its offset
    in the step): the bits of one launch per product, and the bf16-effective
    f64 product within the accumulation bar."""
    rng = np.random.default_rng(gs * 3 + (w_dt == H.F16))
    kern = qmm.MatmulKernel(w_dt, H.BF16, H.BF16)
    specs = [(300, 260, 768, 4, 1, 1, False), (40, 128, 1024, 4, 0, 0, True), (257, 96, 384, 8, 1, 1, False)]
    made = []
    for m, n, kk, bits, layout, corr, signed in specs:
        W = H.affine_weights(oracle, rng, n, kk, bits, gs, layout, corr, w_dt, quantizer=False)
        x = H.to_dev(H.activations(oracle, rng, m, kk))
        made.append((m, n, kk, bits, layout, corr, signed, W, x))

    def args(m, n, kk, bits, layout, corr, signed, W, x):
        return qmm.MatmulArguments(
            a=x, m=m, n=n, k=kk, d=torch_empty(m * n, H.BF16),
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(layout, n, kk // gs), mode=qmm.MODE_U4 if bits == 4 else qmm.MODE_U8,
                             group_size=gs, correction=corr, signed_codes=signed,
                             correction_data=None if W["corr"] is None else H.to_dev(W["corr"])))
    many = [args(*t) for t in made]
    kern.encode_many(many)
    single = [args(*t) for t in made]
    for a in single:
        kern.encode(a)
    torch.cuda.synchronize()
    for a, b, t in zip(many, single, made):
        assert torch.equal(a.d, b.d), f"batched and single differ for m={t[0]} n={t[1]} k={t[2]}"
        m, n, kk, bits, layout, corr, signed, W, x = t
        got = H.load(oracle, H.from_dev(a.d, np.uint16), H.BF16)
        want, mag = bf16_effective_reference(oracle, W, H.from_dev(x, np.uint16), m, n, kk, bits, gs, layout, corr,
                                             w_dt, signed)
        check(got, want.ravel(), mag=mag.ravel(), label=f"batched gemm gs{gs} m{m} n{n} k{kk} b{bits}")


def test_prefill_gemm_split_into_row_launches(qmm, oracle):
    """A product too tall for one grid's 32-bit offsets (K = 12288: 87040 rows
    per grid) runs as launches of whole rows: rows on both sides of the split
    against the bf16-effective f64 product, the D-ops on the second part."""
    m, n, k = 87040 + 300, 136, 12288
    rng = np.random.default_rng(87)
    W = H.affine_weights(oracle, rng, n, k, 4, 64, 1, 1, H.BF16)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(87)
    x = torch.randn(m * k, generator=gen, device="cuda").to(torch.bfloat16).view(torch.int16)
    prior = torch.randn(m * n, generator=gen, device="cuda")
    d = prior.clone()
    qmm.MatmulKernel(H.BF16, H.BF16, H.F32).encode(qmm.MatmulArguments(
        a=x, m=m, n=n, k=k, d=d, b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                                                  params=qmm.QuantParams(1, n, k // 64), mode=qmm.MODE_U4,
                                                  correction_data=H.to_dev(W["corr"])),
        d_transform=qmm.MatmulDOps(accumulate=True)))
    torch.cuda.synchronize()
    rows = np.array([0, 87039, 87040, 87041, m - 1])
    xs = x.view(m, k)[torch.from_numpy(rows).cuda()].cpu().numpy().view(np.uint16).ravel()
    want, mag = bf16_effective_reference(oracle, W, xs, len(rows), n, k, 4, 64, 1, 1, H.BF16, False)
    got = d.view(m, n)[torch.from_numpy(rows).cuda()].cpu().numpy() - prior.view(m, n)[torch.from_numpy(rows).cuda()].cpu().numpy()
    check(got.ravel(), want.ravel(), mag=mag.ravel() + 4.0, label="row-split gemm")


@pytest.mark.parametrize("layout", [0, 1])
def test_decode_stream_kernel_tile_heights_agree(qmm, oracle, layout):
    """A launch with fewer 32-row tiles than CUs runs 16-row tiles; batched
    with a large product it runs 32-row tiles. The per-row arithmetic is the
    same, so the product's outputs are the same bits either way (ragged N)."""
    rng = np.random.default_rng(91 + layout)
    n, k = 1000 + 8, 8192
    W = H.affine_weights(oracle, rng, n, k, 4, 64, layout=layout)
    x = H.activations(oracle, rng, 1, k)
    F = H.affine_weights(oracle, rng, 12288, 4096, 4, 64, layout=1)
    fx = H.activations(oracle, rng, 1, 4096)
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)

    def product(d):
        return qmm.MatmulArguments(
            a=H.to_dev(x), m=1, n=n, k=k, d=d,
            b=qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                             params=qmm.QuantParams(layout, n, k // 64), mode=qmm.MODE_U4,
                             correction_data=H.to_dev(W["corr"])))

    alone = torch_empty(n, H.BF16)
    kern.encode_many([product(alone)])  # 32 tiles of 32 rows: the 16-row form
    batched = torch_empty(n, H.BF16)
    filler = qmm.MatmulArguments(
        a=H.to_dev(fx), m=1, n=12288, k=4096, d=torch_empty(12288, H.BF16),
        b=qmm.QuantizedB(codes=H.to_dev(F["codes"]), scales=H.to_dev(F["scales"]),
                         params=qmm.QuantParams(1, 12288, 64), mode=qmm.MODE_U4, correction_data=H.to_dev(F["corr"])))
    kern.encode_many([product(batched), filler])  # 416 tiles of 32 rows
    torch.cuda.synchronize()
    assert torch.equal(alone, batched)
