"""GPU tests of stark_qmm_encode_many_prologue: the streaming kernel with the
RMS norm or the gated SiLU applied to the shared activation row as it is
staged. The prologue has no counterpart in the reference (its decoder runs
both as kernels of their own), so the bar is the unfused sequence on the same
inputs: the separate kernel writes the row, stark_qmm_encode_many reads it,
and the fused product must equal that output bit for bit. The unfused
products are held to the oracle elsewhere; the fused output is also checked
against the oracle on the transformed row here."""
import ctypes as C

import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dec():
    from stark_amd import decode
    decode.lib()
    return decode


def _p(t):
    return C.c_void_p(t.data_ptr())


def _s():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).astype(np.float32)).cuda().to(torch.bfloat16)


def _ops(qmm, oracle, rng, x, shapes, layout, correction, signed, w_dt, d_dt, accumulate=False, bias=False):
    """Products over the row x: (args for the fused call, args for the unfused
    call, oracle inputs). The unfused args read a placeholder row, set later."""
    k = x.numel()
    fused, plain, ref = [], [], []
    for n in shapes:
        W = H.affine_weights(oracle, rng, n, k, 4, 64, layout, correction, w_dt, quantizer=False)
        prior = rng.normal(0, 1, n).astype(np.float32) if accumulate else None
        bv = H.store(oracle, rng.normal(0, 0.5, n).astype(np.float32), w_dt) if bias else None
        corr = None if W["corr"] is None else H.to_dev(W["corr"])
        b = qmm.QuantizedB(codes=H.to_dev(W["codes"]), scales=H.to_dev(W["scales"]),
                           params=qmm.QuantParams(layout, n, k // 64), mode=qmm.MODE_U4, group_size=64,
                           correction=correction, correction_data=corr, signed_codes=signed)

        def mk(a, n=n, b=b, prior=prior, bv=bv):
            d = (H.to_dev(H.store(oracle, prior, d_dt)) if prior is not None else
                 torch.zeros(n, dtype=torch.float32 if d_dt == H.F32 else torch.int16, device="cuda"))
            return qmm.MatmulArguments(a=a, m=1, n=n, k=k, d=d, b=b,
                                       d_transform=qmm.MatmulDOps(accumulate=accumulate,
                                                                  bias=None if bv is None else H.to_dev(bv)))
        fused.append(mk(x))
        plain.append(mk)
        ref.append(dict(W=W, n=n, prior=prior, bias=bv))
    return fused, plain, ref


def _check_oracle(qmm, oracle, row, got_args, ref, layout, correction, signed, w_dt, d_dt, accumulate):
    x = row.view(torch.int16).cpu().numpy().view(np.uint16)
    k = x.size
    for a, r in zip(got_args, ref):
        n, W = r["n"], r["W"]
        prior = None if r["prior"] is None else H.store(oracle, r["prior"], d_dt)
        st, want = oracle.matmul(a=x, m=1, n=n, k=k, codes=W["codes"], scales=W["scales"], correction=correction,
                                 correction_data=W["corr"], layout=layout, row_count=n, group_count=k // 64, bits=4,
                                 group_size=64, signed_codes=signed, d=prior, accumulate=accumulate, bias=r["bias"],
                                 weights_dt=w_dt, input_dt=H.BF16, output_dt=d_dt, threads=8)
        assert st == 0
        got = H.load(oracle, H.from_dev(a.d, np.float32 if d_dt == H.F32 else np.uint16), d_dt)
        mag = H.dequant_magnitude(oracle, W["codes"], W["scales"], W["corr"], n, k, 4, 64, layout, correction, w_dt,
                                  x, H.BF16, 1, signed=signed)
        if accumulate or r["bias"] is not None:
            mag = mag + 4.0
        check(got, H.load(oracle, want, d_dt), mag=mag, label=f"prologue n{n} k{k}")


NORM_CASES = [
    # (shapes sharing the row, K, layout, correction, signed, w_dt, d_dt, accumulate, bias, row scale)
    ((512, 128, 128), 4096, 0, 1, False, H.BF16, H.BF16, False, False, 1.0),  # q/k/v-like
    ((96, 40), 4096, 1, 1, False, H.BF16, H.BF16, False, False, 1.0),        # shifted last tile
    ((256,), 8192, 0, 0, True, H.BF16, H.F32, True, True, 300.0),
    ((64, 200), 12288, 1, 1, True, H.F16, H.BF16, True, False, 1e-3),
    ((1024, 1024), 4096, 0, 1, False, H.BF16, H.BF16, False, False, 1e4),   # gate/up-like
]


@pytest.mark.parametrize("case", range(len(NORM_CASES)))
def test_rms_norm_prologue_equals_norm_then_product(qmm, oracle, dec, case):
    shapes, k, layout, corr, signed, w_dt, d_dt, acc, bias, scale = NORM_CASES[case]
    rng = np.random.default_rng(100 + case)
    x = _bf16(rng.normal(0, scale, k))
    w = _bf16(1 + 0.1 * rng.normal(0, 1, k))
    eps = 1e-6
    fused, plain, ref = _ops(qmm, oracle, rng, x, shapes, layout, corr, signed, w_dt, d_dt, acc, bias)
    kern = qmm.MatmulKernel(w_dt, H.BF16, d_dt)
    kern.encode_many_prologue(fused, qmm.PROLOGUE_RMS_NORM, w, eps)
    h = torch.empty_like(x)
    assert dec.lib().stark_decode_rms_norm(_p(x), _p(w), _p(h), k, eps, _s()) == 0
    unfused = [mk(h) for mk in plain]
    kern.encode_many(unfused)
    torch.cuda.synchronize()
    for a, b in zip(fused, unfused):
        assert torch.equal(a.d, b.d), f"fused and unfused differ for n={a.n}"
    # the normalised row itself against the torch statement of the norm
    xf = x.float()
    want_h = (xf * torch.rsqrt((xf * xf).mean() + eps)).to(torch.bfloat16).float() * w.float()
    torch.testing.assert_close(h.float(), want_h.to(torch.bfloat16).float(), rtol=2 ** -7, atol=0)
    _check_oracle(qmm, oracle, h, fused, ref, layout, corr, signed, w_dt, d_dt, acc)


SILU_CASES = [
    ((4096,), 12288, 0, 1, False, H.BF16, H.BF16, True, 1.0),    # down-like, residual accumulate
    ((96,), 4096, 1, 0, True, H.F16, H.F32, False, 4.0),
    ((64, 64), 8192, 0, 1, False, H.BF16, H.BF16, False, 30.0),  # saturating gates: exp overflow, silu -> 0 / x
]


@pytest.mark.parametrize("case", range(len(SILU_CASES)))
def test_silu_gate_prologue_equals_gated_act_mul_then_product(qmm, oracle, dec, case):
    shapes, k, layout, corr, signed, w_dt, d_dt, acc, scale = SILU_CASES[case]
    rng = np.random.default_rng(200 + case)
    g = _bf16(rng.normal(0, scale, k))
    u = _bf16(rng.normal(0, 1, k))
    fused, plain, ref = _ops(qmm, oracle, rng, g, shapes, layout, corr, signed, w_dt, d_dt, acc)
    kern = qmm.MatmulKernel(w_dt, H.BF16, d_dt)
    kern.encode_many_prologue(fused, qmm.PROLOGUE_SILU_GATE, u)
    # the decode stand-in's silu_mul writes the row the prologue stages; the
    # library's GatedActMul (SiLU, separate value operand: expf and a
    # division) is within one bf16 ulp of it
    a = torch.empty_like(g)
    assert dec.lib().stark_decode_silu_mul(_p(g), _p(u), _p(a), k, _s()) == 0
    ga = torch.empty_like(g)
    qmm.GatedActMul.full_precision(H.BF16, False, False).encode_fp(g.view(torch.int16), u.view(torch.int16),
                                                                   ga.view(torch.int16), None, k, 1, 0, k,
                                                                   qmm.ACT_SILU)
    unfused = [mk(a) for mk in plain]
    kern.encode_many(unfused)
    torch.cuda.synchronize()
    # (gates below about -87 put 1 + e^-g past 2^126, where the hardware
    # reciprocal flushes: silu(g) * up is then below 2^-100 on both sides)
    tiny = 2.0 ** -100
    big = torch.maximum(a.float().abs(), ga.float().abs()) >= tiny
    ulp = (a.view(torch.int16).int() - ga.view(torch.int16).int()).abs()
    assert bool((a.float() * ga.float() >= 0)[big].all()) and int(ulp[big].max()) <= 1
    assert bool(((a.float() - ga.float()).abs() <= tiny)[~big].all())
    assert int((ulp[big] > 0).sum()) <= k // 64, "more one-ulp differences than the exp2/reciprocal error allows"
    for x, y in zip(fused, unfused):
        assert torch.equal(x.d, y.d), f"fused and unfused differ for n={x.n}"
    _check_oracle(qmm, oracle, a, fused, ref, layout, corr, signed, w_dt, d_dt, acc)


def test_prologue_repeated_and_graph_replay(qmm, oracle, dec):
    """A layer's three prologue launches (norm -> q/k/v, norm -> gate/up,
    SiLU -> down) captured in a graph and replayed with eager work between the
    replays: every replay equals the eager result."""
    rng = np.random.default_rng(7)
    k, inter = 4096, 12288
    x = _bf16(rng.normal(0, 1, k))
    w1, w2 = _bf16(1 + 0.1 * rng.normal(0, 1, k)), _bf16(1 + 0.1 * rng.normal(0, 1, k))
    qkv, _, _ = _ops(qmm, oracle, rng, x, (512, 128, 128), 0, 1, False, H.BF16, H.BF16)
    gu, _, _ = _ops(qmm, oracle, rng, x, (inter, inter), 0, 1, False, H.BF16, H.BF16)
    g, u = gu[0].d.view(torch.bfloat16), gu[1].d.view(torch.bfloat16)
    down, _, _ = _ops(qmm, oracle, rng, g, (k,), 0, 1, False, H.BF16, H.BF16)
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.BF16)
    b1 = kern.prepare_many_prologue(qkv, qmm.PROLOGUE_RMS_NORM, w1, 1e-6)
    b2 = kern.prepare_many_prologue(gu, qmm.PROLOGUE_RMS_NORM, w2, 1e-6)
    b3 = kern.prepare_many_prologue(down, qmm.PROLOGUE_SILU_GATE, u)

    def layer(s=None):
        kern.encode_prepared(b1, s)
        kern.encode_prepared(b2, s)
        kern.encode_prepared(b3, s)

    layer()
    torch.cuda.synchronize()
    want = [a.d.clone() for a in qkv + gu + down]
    assert down[0].d.view(torch.bfloat16).float().abs().max().item() > 0
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            layer(s)
    torch.cuda.current_stream().wait_stream(s)
    for _ in range(3):
        for a in qkv + gu + down:
            a.d.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, w in zip(qkv + gu + down, want):
            assert torch.equal(a.d, w)
