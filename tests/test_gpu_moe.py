"""GPU parity of the MoE kernels (moe.rs:24-184 restated in the oracle) and of
the fused routed-experts pipeline (routed.rs:154-257) through the C ABI."""

import numpy as np
import pytest
import torch

from tests import helpers as H
from tests import moe_cases as MC

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,experts,active,rw,rl", [(1, 128, 8, False, False), (16, 128, 8, True, False),
                                                      (7, 64, 4, False, True), (33, 1024, 32, True, True),
                                                      (4, 8, 8, False, False)])
def test_route(qmm, oracle, rows, experts, active, rw, rl):
    rng = np.random.default_rng(rows * experts + active)
    logits = rng.normal(0, 2, rows * experts).astype(np.float32)
    logits[: experts // 2] = logits[experts // 2: experts]  # exact ties: the lower id wins
    want_ids, want_w = oracle.moe_route(logits, rows, experts, active, rw, rl)
    ids, w = qmm.moe_route(H.to_dev(logits), rows, experts, active, rw, rl)
    torch.cuda.synchronize()
    # ids depend only on comparisons of the (optionally bf16-rounded) logits: exact
    assert np.array_equal(H.from_dev(ids, np.uint32), want_ids)
    # weights go through expf and the softmax denominator, whose last bits are
    # libm's (the reference's own f32::exp is the platform's): a few f32 ulp, or
    # one bf16 ulp once rounded to bf16
    got_w = H.from_dev(w, np.float32)
    rtol = 2.0 ** -7 if rw else 4e-7 * 8
    assert np.allclose(got_w, want_w, rtol=rtol, atol=0)


@pytest.mark.parametrize("sort_ids", [False, True])
def test_adjust_exact(qmm, oracle, sort_ids):
    rng = np.random.default_rng(5)
    rows, E, A = 9, 16, 5
    ids = np.stack([rng.permutation(E)[:A] for _ in range(rows)]).astype(np.uint32).ravel()
    ids[3] = E + 2  # out of range: weight becomes NaN
    w = rng.uniform(0, 1, rows * A).astype(np.float32)
    g = rng.uniform(0.5, 2, E).astype(np.float32)
    di, dw = H.to_dev(ids), H.to_dev(w.copy())
    qmm.moe_adjust_routes(di, dw, H.to_dev(g), rows, E, A, sort_ids)
    oracle.moe_adjust_routes(ids, w, g, rows, E, A, sort_ids)
    torch.cuda.synchronize()
    assert np.array_equal(H.from_dev(di, np.uint32), ids)
    assert np.array_equal(H.from_dev(dw, np.float32).view(np.uint32), w.view(np.uint32))


def test_gather_and_accumulate_exact(qmm, oracle):
    rng = np.random.default_rng(11)
    ids = np.array([3, 1, 7, 99], np.uint32)
    for route in range(4):
        want = oracle.moe_gather_rows(ids, route, 24, 8, 24)
        got = qmm.moe_gather_rows(H.to_dev(ids), route, 24, 8, 24)
        assert np.array_equal(H.from_dev(got, np.uint32), want)
    L = 300
    inp = oracle.f32_to_bf16(rng.normal(0, 1, L).astype(np.float32))
    wts = rng.uniform(0, 1, 4).astype(np.float32)
    for flags in [(1, 0, 0, 0), (0, 1, 1, 0), (0, 1, 0, 1), (1, 1, 1, 1)]:
        init, fin, rp, ra = flags
        acc = rng.normal(0, 1, L + 10).astype(np.float32)
        out = np.zeros(L + 10, np.uint16)
        da, do = H.to_dev(acc.copy()), H.to_dev(out.copy())
        qmm.moe_accumulate(H.to_dev(inp), H.to_dev(wts), da, do, L, 2, 10, init, fin, rp, ra)
        oracle.moe_accumulate(inp, wts, acc, out, L, 2, 10, init, fin, rp, ra)
        torch.cuda.synchronize()
        assert np.array_equal(H.from_dev(da, np.float32).view(np.uint32), acc.view(np.uint32))
        assert np.array_equal(H.from_dev(do, np.uint16), out)


def routed_want(O, c, **flags):
    R, M, Hd, E, A = c["rows"], c["model"], c["hidden"], c["experts"], c["active"]
    return O.bf16_to_f32(O.routed_experts(c["x"], c["logits"], c["up"], c["down"], R, M, Hd, E, A,
                                          expert_scales=c["scales"], layout=c["layout"], group=c["group"],
                                          round_logits=flags.get("rl", False), round_weights=flags.get("rw", False),
                                          round_products=flags.get("rp", False),
                                          round_accumulator=flags.get("ra", False),
                                          sort_ids=flags.get("si", False)))


def routed_check(qmm, O, c, workspace=None, **flags):
    want = routed_want(O, c, **flags)
    got = routed_run(qmm, c, workspace, **flags)
    check_routed(O, c, got, want, flags)
    return got, want


def routed_run(qmm, c, workspace=None, **flags):
    R, M, Hd, E, A = c["rows"], c["model"], c["hidden"], c["experts"], c["active"]
    corr = qmm.BIASES if c["up"]["biases"] is not None else qmm.SYMMETRIC

    def qb(b, rows, cols):
        return qmm.QuantizedB(codes=H.to_dev(b["codes"]), scales=H.to_dev(b["scales"]), correction=corr,
                              correction_data=None if b["biases"] is None else H.to_dev(b["biases"]),
                              params=qmm.QuantParams(c["layout"], rows, cols // c["group"]),
                              group_size=c["group"])

    out = qmm.routed_experts(H.to_dev(c["x"]), H.to_dev(c["logits"]), qb(c["up"], E * 2 * Hd, M),
                             qb(c["down"], E * M, Hd), R, M, Hd, E, A,
                             expert_scales=None if c["scales"] is None else H.to_dev(c["scales"]),
                             round_logits=flags.get("rl", False), round_weights=flags.get("rw", False),
                             round_products=flags.get("rp", False), round_accumulator=flags.get("ra", False),
                             sort_expert_ids=flags.get("si", False), workspace=workspace)
    torch.cuda.synchronize()
    return (H.from_dev(out.view(torch.int16), np.uint16).astype(np.uint32) << 16).view(np.float32)


def _dequant4(O, bank, r0, rows, cols, total_rows, layout, group):
    """s*q + b (float64) of bank rows r0 .. r0+rows (4-bit, bf16 planes)."""
    codes = np.asarray(bank["codes"], np.uint8).reshape(total_rows, cols // 2)[r0:r0 + rows]
    q = np.empty((rows, cols), np.float64)
    q[:, 0::2] = codes & 15
    q[:, 1::2] = codes >> 4
    G = cols // group
    os_, gs_ = O.quant_strides(layout, total_rows, G, 1)
    idx = (r0 + np.arange(rows))[:, None] * os_ + (np.arange(cols) // group)[None, :] * gs_
    s = O.bf16_to_f32(np.asarray(bank["scales"], np.uint16)).astype(np.float64)[idx]
    if bank["biases"] is None:
        return s * q - 8.0 * s
    return s * q + O.bf16_to_f32(np.asarray(bank["biases"], np.uint16)).astype(np.float64)[idx]


def routed_magnitude(O, c, flags):
    """Per output, sum over its routes of p_r * sum_i |w_down[n, i] * act_r[i]|,
    with act_r the oracle's gated activation of route r (its up product
    through MatmulCpuKernel and the gated SiLU, both restated in the oracle)."""
    R, M, Hd, E, A = c["rows"], c["model"], c["hidden"], c["experts"], c["active"]
    ids, w = O.moe_route(c["logits"], R, E, A, flags.get("rw", False), flags.get("rl", False))
    if c["scales"] is not None:
        O.moe_adjust_routes(ids, w, c["scales"], R, E, A, flags.get("si", False))
    corr = 1 if c["up"]["biases"] is not None else 0
    mag = np.zeros((R, M))
    for r in range(R):
        for k in range(A):
            e = int(ids[r * A + k]) % E
            up = c["up"]
            rows = np.arange(e * 2 * Hd, (e + 1) * 2 * Hd, dtype=np.uint32)
            st, proj = O.matmul(a=c["x"][r * M:(r + 1) * M], m=1, n=2 * Hd, k=M, codes=up["codes"],
                                scales=up["scales"], correction=corr, correction_data=up["biases"],
                                layout=c["layout"], row_count=E * 2 * Hd, group_count=M // c["group"], bits=4,
                                group_size=c["group"], gather=rows, output_dt=H.BF16)
            assert st == 0
            act = np.abs(O.bf16_to_f32(O.gated_silu_bf16(proj, Hd, 1))).astype(np.float64)
            wd = _dequant4(O, c["down"], e * M, M, Hd, E * M, c["layout"], c["group"])
            mag[r] += abs(float(w[r * A + k])) * (np.abs(wd) @ act)
    return mag


def check_routed(O, c, got, want, flags):
    """Parity bar of the routed pipeline. Each (token, rank) passes through the
    reference's bf16 rounding points (value and gate rows of the up product,
    the gated activation, the down product; routed.rs:208-239 writes bf16 at
    each). The GPU's f32 sums differ from the oracle's sequential ones only in
    summation order, but a sum that lands on the other side of a bf16 rounding
    boundary moves that intermediate by one bf16 ulp (<= 2^-7 relative); a
    flipped value or gate moves the activation by at most about 4 * 2^-7 of
    itself. So every output is held to
        max(1e-2 |want|, 2 bf16 ulps, 2^-5 * sum_r p_r sum_i |w_down act_r,i|)
    the last term bounding what one-ulp flips of the bf16 intermediates can
    move an output (it only exceeds the others where the down product
    cancels), and at least 99% of the outputs must meet the north-star bar
    max(1e-2 |want|, 2 bf16 ulps) outright."""
    from tests.tolerances import bf16_ulp
    R, M = c["rows"], c["model"]
    want2, got2 = want.reshape(R, M).astype(np.float64), got.reshape(R, M).astype(np.float64)
    base = np.maximum(1e-2 * np.abs(want2), 2 * bf16_ulp(want2))
    mag = routed_magnitude(O, c, flags)
    tol = np.maximum(base, 2.0 ** -5 * mag)
    err = np.abs(got2 - want2)
    bad = err > tol
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} outside the bound; worst excess "
                           f"{float((err - tol).max())}")
    strict = float((err <= base).mean())
    assert strict >= 0.99, f"only {strict:.4f} of outputs within 1e-2 rel / 2 bf16 ulp"


@pytest.mark.parametrize("rows", [1, 3, 16, 40])
@pytest.mark.parametrize("layout", [0, 1])
def test_routed_experts_pipeline(qmm, oracle, rows, layout):
    """Qwen3-MoE-like geometry at reduced size: every route-count class, GO and
    OG planes, rows > 16 (experts split into several slots)."""
    c = MC.case(oracle, 100 + rows + 7 * layout, rows, model=256, hidden=128, experts=16, active=4, layout=layout)
    routed_check(qmm, oracle, c)


@pytest.mark.parametrize("biased,gains,flags", [(False, False, dict(rp=True, ra=True)),
                                                (True, True, dict(si=True, rw=True)),
                                                (True, False, dict(si=True, rl=True))])
def test_routed_experts_options(qmm, oracle, biased, gains, flags):
    c = MC.case(oracle, 55, 6, model=256, hidden=128, experts=8, active=3, biased=biased, gains=gains)
    routed_check(qmm, oracle, c, **flags)


@pytest.mark.parametrize("rows,experts,flags", [(16, 128, {}), (9, 96, dict(si=True, rw=True)), (4, 128, {}),
                                                (5, 128, dict(rl=True))])
def test_routed_experts_route_paths(qmm, oracle, rows, experts, flags):
    """Both routing paths: the one-workgroup route + compaction (rows * E^2 up
    to 65536 compares) and the per-row route kernel with a separate compaction
    above it (16 x 128, 9 x 96, 5 x 128)."""
    c = MC.case(oracle, 300 + rows + experts, rows, model=256, hidden=128, experts=experts, active=8,
                gains=bool(flags.get("si")))
    routed_check(qmm, oracle, c, **flags)


@pytest.mark.parametrize("rows", [1, 4, 16])
def test_routed_experts_qwen3_moe_geometry(qmm, oracle, rows):
    """Config-3 widths (H=2048, I=768, E=128, top-8) at 1, 4 and 16 tokens:
    the K=2048 grouped up kernels of every route-count class run."""
    c = MC.case(oracle, 9 + rows, rows, model=2048, hidden=768, experts=128, active=8)
    routed_check(qmm, oracle, c)


def _workspace_routes(oracle, c, ws, flags):
    """(ids, weights) the call left at the start of its workspace, and the
    oracle's route (+ adjust, as routed.rs:188-209 applies it) of the same logits."""
    R, E, A = c["rows"], c["experts"], c["active"]
    n = R * A
    raw = ws.cpu().numpy()
    ids = raw[: 4 * n].view(np.uint32)
    w = raw[(4 * n + 255) // 256 * 256:][: 4 * n].view(np.float32)
    want_ids, want_w = oracle.moe_route(c["logits"], R, E, A, flags.get("rw", False), flags.get("rl", False))
    gains = c["scales"]
    if gains is not None or flags.get("si", False):
        g = gains if gains is not None else np.ones(E, np.float32)
        oracle.moe_adjust_routes(want_ids, want_w, g, R, E, A, flags.get("si", False) if gains is not None else True)
    return ids, w, want_ids, want_w


@pytest.mark.parametrize("experts,active,flags", [(128, 8, {}), (256, 8, dict(si=True)),
                                                  (64, 4, dict(rl=True, rp=True)), (16, 4, dict(si=True)),
                                                  (256, 8, dict(rw=True, ra=True)), (257, 8, {}), (96, 12, {})])
def test_routed_experts_one_token(qmm, oracle, experts, active, flags):
    """One token (E <= 256) routes inside the up launch (every workgroup ranks
    the token's logits itself; workgroup 0 files the slots), and up to 8
    routes take the down products and the rank accumulation in one launch.
    Its ids equal the oracle's route + adjust bit for bit, the weights meet the
    route kernels' bar and the outputs the routed bar. With bf16-rounded
    weights a last-bit difference of expf (the device's against the oracle's
    libm) can move a weight by one bf16 ulp, so there the bar also admits
    2^-7 of each output's magnitude. E = 257 takes the separate route launch;
    12 routes take the grouped down launch and the accumulation launch."""
    c = MC.case(oracle, 700 + experts + active, 1, model=1024, hidden=256, experts=experts, active=active,
                gains=bool(flags.get("si")) and experts != 16)
    c["logits"][: experts // 4] = c["logits"][experts // 4: experts // 2]  # exact ties: the lower id wins
    need = qmm.routed_experts_workspace_size(1, 1024, 256, experts, active)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    got = routed_run(qmm, c, ws, **flags)
    ids, w, want_ids, want_w = _workspace_routes(oracle, c, ws, flags)
    assert np.array_equal(ids, want_ids)
    rtol = 2.0 ** -7 if flags.get("rw") else 4e-7 * 8
    assert np.allclose(w, want_w, rtol=rtol, atol=0)
    want = routed_want(oracle, c, **flags)
    if flags.get("rw"):
        mag = routed_magnitude(oracle, c, flags).ravel()
        err = np.abs(got.astype(np.float64) - want)
        assert np.all(err <= np.maximum(np.maximum(1e-2 * np.abs(want), 2.0 ** -7 * mag), 1e-30))
    else:
        check_routed(oracle, c, got, want, flags)


def test_routed_experts_one_token_non_finite_logit(qmm, oracle):
    """A non-finite logit: every route of the token reads expert 0 with a NaN
    weight (moe.rs:52-84), in the fused one-token launch as in the route kernels."""
    c = MC.case(oracle, 812, 1, model=256, hidden=128, experts=32, active=4)
    c["logits"][5] = np.nan
    b = lambda bank, rows, cols: qmm.QuantizedB(
        codes=H.to_dev(bank["codes"]), scales=H.to_dev(bank["scales"]), correction_data=H.to_dev(bank["biases"]),
        params=qmm.QuantParams(c["layout"], rows, cols // c["group"]))
    need = qmm.routed_experts_workspace_size(1, 256, 128, 32, 4)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    qmm.routed_experts(H.to_dev(c["x"]), H.to_dev(c["logits"]), b(c["up"], 32 * 2 * 128, 256), b(c["down"], 32 * 256, 128),
                       1, 256, 128, 32, 4, workspace=ws)
    torch.cuda.synchronize()
    ids, w, want_ids, want_w = _workspace_routes(oracle, c, ws, {})
    assert np.array_equal(ids, want_ids) and not ids.any()
    assert np.isnan(w).all() and np.isnan(want_w).all()


def test_routed_experts_rejections(qmm, oracle):
    c = MC.case(oracle, 1, 2, model=256, hidden=128, experts=8, active=2)
    b = qmm.QuantizedB(codes=H.to_dev(c["up"]["codes"]), scales=H.to_dev(c["up"]["scales"]),
                       correction_data=H.to_dev(c["up"]["biases"]), params=qmm.QuantParams(1, 8 * 256, 256 // 64))
    d = qmm.QuantizedB(codes=H.to_dev(c["down"]["codes"]), scales=H.to_dev(c["down"]["scales"]),
                       correction_data=H.to_dev(c["down"]["biases"]), params=qmm.QuantParams(1, 8 * 256, 128 // 64))
    x, lg = H.to_dev(c["x"]), H.to_dev(c["logits"])
    with pytest.raises(qmm.MatmulError) as e:
        qmm.routed_experts(x, lg, b, d, 2, 256, 128, 8, 2, workspace=torch.empty(16, dtype=torch.uint8,
                                                                                  device="cuda"))
    assert e.value.status == qmm.WORKSPACE_TOO_SMALL
    with pytest.raises(qmm.MatmulError):
        qmm.routed_experts(x, lg, b, d, 2, 256, 128, 8, 9)  # active > experts
