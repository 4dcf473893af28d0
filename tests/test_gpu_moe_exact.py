"""Bit-exact dequantisation inside the routed-experts pipeline
(RoutedExperts::encode_scaled, crates/stark-engine/src/encodable_block/mlp/routed.rs:154-257).

The reference writes bf16 at its rounding points: the up product's value and
gate rows, the gated activation and the down product (routed.rs:208-239), and
each product's f32 sum over one nonzero term is the dequantised weight
s*q + bias_term of MatmulCpuKernel (kernel.rs:219-265). With one active
expert the route weight is score / score = 1 exactly, so the output row is
the down product of that route, and weights built so that every sum has one
nonzero term make the output a dequantised weight, bf16-rounded:

* up exactness: x = e_c (one-hot at column c), gate rows all equal to 16
  (codes 0, bias 16: silu(16) rounds to 16 in bf16), the down bank the
  identity (w = 1 where output row n equals hidden index i). Output n < hidden
  is then bf16(bf16(w_value[n, c]) * 16) = 16 * bf16_rne(s*q + b) of the
  value row;
* down exactness: value rows one-hot (w = 1/16 at hidden index f(c) = c mod
  hidden, else 0), gate 16 again, so the activation row is e_{f(c)}; output n
  is bf16_rne(s*q + b) of down row n at column f(c).

Both are compared BITWISE with the oracle's dequantisation (f32 s*q + b, then
bf16 round-to-nearest-even), on every route-count class of the grouped
kernels: one token (the fused route + up launch), 3 and 16 tokens (slots of
up to 4 routes of one expert), both plane layouts, K = 256 and 2048."""
import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _planes(O, rows, G, layout, s, b):
    """[rows, G] float arrays -> bf16 planes in the layout (0: [rows, G], 1: [G, roundup4(rows)])."""
    if layout == 1:
        n4 = (rows + 3) // 4 * 4
        ps = np.zeros((G, n4), np.float32)
        pb = np.zeros((G, n4), np.float32)
        ps[:, :rows] = s.T
        pb[:, :rows] = b.T
        s, b = ps, pb
    return H.store(O, s.astype(np.float32).ravel(), H.BF16), H.store(O, b.astype(np.float32).ravel(), H.BF16)


def _pack(q):
    """[rows, cols] 4-bit codes -> bytes, low nibble first."""
    q = np.asarray(q, np.uint8)
    return np.ascontiguousarray((q[:, 0::2] | (q[:, 1::2] << 4)).ravel())


def _wide(rng, shape):
    s = rng.uniform(0.5, 1.0, shape) * np.exp2(rng.integers(-12, 1, shape)) * rng.choice([-1.0, 1.0], shape)
    b = rng.normal(0, 1, shape) * np.exp2(rng.integers(-10, 1, shape))
    return s.astype(np.float32), b.astype(np.float32)


def _dequant(O, codes_q, s_rows, b_rows, group):
    """f32 s*q + b per weight from [rows, cols] codes and [rows, G] bf16-exact planes."""
    s = np.repeat(O.bf16_to_f32(O.f32_to_bf16(s_rows)), group, 1).astype(np.float64)
    b = np.repeat(O.bf16_to_f32(O.f32_to_bf16(b_rows)), group, 1).astype(np.float64)
    return (s * codes_q + b).astype(np.float32)  # s*q is exact; one rounding of the sum


def _run(qmm, O, *, x_cols, logits_experts, up, down, rows, model, hidden, experts, layout, group):
    xs = np.zeros((rows, model), np.float32)
    xs[np.arange(rows), x_cols] = 1.0
    logits = np.full((rows, experts), -4.0, np.float32)
    logits[np.arange(rows), logits_experts] = 4.0
    qb = lambda bank, nrows, cols: qmm.QuantizedB(
        codes=H.to_dev(bank[0]), scales=H.to_dev(bank[1]), correction_data=H.to_dev(bank[2]),
        params=qmm.QuantParams(layout, nrows, cols // group), group_size=group)
    out = qmm.routed_experts(H.to_dev(H.store(O, xs.ravel(), H.BF16)), H.to_dev(logits.ravel()),
                             qb(up, experts * 2 * hidden, model), qb(down, experts * model, hidden), rows, model,
                             hidden, experts, 1)
    torch.cuda.synchronize()
    return H.from_dev(out.view(torch.int16), np.uint16).reshape(rows, model)


CASES = [(1, 256, 128, 4), (3, 256, 128, 4), (16, 256, 128, 4), (16, 2048, 768, 8), (1, 2048, 768, 16)]


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("rows,model,hidden,experts", CASES)
def test_routed_up_product_exact(qmm, oracle, rows, model, hidden, experts, layout):
    O, group = oracle, 64
    rng = np.random.default_rng(1000 + rows + model + layout)
    Gu, Gd = model // group, hidden // group
    # up bank: per expert [value rows (random codes, wide planes) | gate rows (= 16)]
    qv = rng.integers(0, 16, (experts, hidden, model), dtype=np.uint8)
    sv, bv = _wide(rng, (experts, hidden, Gu))
    q = np.zeros((experts, 2 * hidden, model), np.uint8)
    q[:, :hidden] = qv
    s = np.ones((experts, 2 * hidden, Gu), np.float32)
    b = np.full((experts, 2 * hidden, Gu), 16.0, np.float32)
    s[:, :hidden], b[:, :hidden] = sv, bv
    up = (_pack(q.reshape(-1, model)),) + _planes(O, experts * 2 * hidden, Gu, layout, s.reshape(-1, Gu),
                                                   b.reshape(-1, Gu))
    # down bank: identity (row n, column i: 1 where n == i)
    qd = np.zeros((experts, model, hidden), np.uint8)
    qd[:, np.arange(hidden), np.arange(hidden)] = 1
    down = (_pack(qd.reshape(-1, hidden)),) + _planes(O, experts * model, Gd, layout,
                                                       np.ones((experts * model, Gd), np.float32),
                                                       np.zeros((experts * model, Gd), np.float32))
    cols = rng.integers(0, model, rows)
    ex = rng.integers(0, experts, rows)
    got = _run(qmm, O, x_cols=cols, logits_experts=ex, up=up, down=down, rows=rows, model=model, hidden=hidden,
               experts=experts, layout=layout, group=group)
    want = np.zeros((rows, model), np.uint16)
    for t in range(rows):
        w = _dequant(O, qv[ex[t]][:, cols[t]:cols[t] + 1], sv[ex[t]][:, cols[t] // group:cols[t] // group + 1],
                     bv[ex[t]][:, cols[t] // group:cols[t] // group + 1], 1)[:, 0]
        want[t, :hidden] = O.f32_to_bf16(O.bf16_to_f32(O.f32_to_bf16(w)) * np.float32(16.0))
    bad = got != want
    bad &= ~(((got & 0x7FFF) == 0) & ((want & 0x7FFF) == 0))  # +0 / -0 of a zero weight
    assert not bad.any(), (f"{int(bad.sum())} up-product weights not bit-exact; first {np.argwhere(bad)[0]}: "
                           f"got {got[bad][0]:#06x} want {want[bad][0]:#06x}")


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("rows,model,hidden,experts", CASES)
def test_routed_down_product_exact(qmm, oracle, rows, model, hidden, experts, layout):
    O, group = oracle, 64
    rng = np.random.default_rng(2000 + rows + model + layout)
    Gu, Gd = model // group, hidden // group
    # up bank: value rows one-hot (1/16 at hidden index c mod hidden), gate rows 16
    q = np.zeros((experts, 2 * hidden, model), np.uint8)
    c_all = np.arange(model)
    q[:, c_all % hidden, c_all] = 1
    s = np.ones((experts, 2 * hidden, Gu), np.float32)
    b = np.full((experts, 2 * hidden, Gu), 16.0, np.float32)
    s[:, :hidden], b[:, :hidden] = 1.0 / 16.0, 0.0
    up = (_pack(q.reshape(-1, model)),) + _planes(O, experts * 2 * hidden, Gu, layout, s.reshape(-1, Gu),
                                                   b.reshape(-1, Gu))
    # down bank: random codes, wide planes
    qd = rng.integers(0, 16, (experts, model, hidden), dtype=np.uint8)
    sd, bd = _wide(rng, (experts, model, Gd))
    down = (_pack(qd.reshape(-1, hidden)),) + _planes(O, experts * model, Gd, layout, sd.reshape(-1, Gd),
                                                       bd.reshape(-1, Gd))
    cols = rng.integers(0, model, rows)
    ex = rng.integers(0, experts, rows)
    got = _run(qmm, O, x_cols=cols, logits_experts=ex, up=up, down=down, rows=rows, model=model, hidden=hidden,
               experts=experts, layout=layout, group=group)
    want = np.zeros((rows, model), np.uint16)
    for t in range(rows):
        j = cols[t] % hidden
        w = _dequant(O, qd[ex[t]][:, j:j + 1], sd[ex[t]][:, j // group:j // group + 1],
                     bd[ex[t]][:, j // group:j // group + 1], 1)[:, 0]
        want[t] = O.f32_to_bf16(w)
    bad = got != want
    bad &= ~(((got & 0x7FFF) == 0) & ((want & 0x7FFF) == 0))
    assert not bad.any(), (f"{int(bad.sum())} down-product weights not bit-exact; first {np.argwhere(bad)[0]}: "
                           f"got {got[bad][0]:#06x} want {want[bad][0]:#06x}")
