"""CPU checks of the routed-experts oracle (RoutedExperts::encode_scaled,
crates/stark-engine/src/encodable_block/mlp/routed.rs:154-257): the composite
so_routed_experts must equal the reference's loop written out over the
already-pinned oracle pieces (route, adjust, gathered matmul, gated SiLU,
accumulate), bit for bit, and the result must agree with an f64 evaluation of
the same dequantised weights."""
import numpy as np
import pytest

from tests import moe_cases as MC


def loop_composition(O, c, round_logits=False, round_weights=False, round_products=False, round_acc=False,
                     sort_ids=False):
    R, M, H, E, A = c["rows"], c["model"], c["hidden"], c["experts"], c["active"]
    ids, w = O.moe_route(c["logits"], R, E, A, round_weights, round_logits)
    if c["scales"] is not None or sort_ids:
        gains = c["scales"] if c["scales"] is not None else np.ones(E, np.float32)
        O.moe_adjust_routes(ids, w, gains, R, E, A, sort_ids if c["scales"] is not None else True)
    acc = np.zeros(R * M, np.float32)
    out = np.zeros(R * M, np.uint16)
    up, down = c["up"], c["down"]
    corr = O.BIASES if up["biases"] is not None else O.SYMMETRIC
    for row in range(R):
        for rank in range(A):
            route = row * A + rank
            up_ids = O.moe_gather_rows(ids, route, 2 * H, E, 2 * H)
            st, proj = O.matmul(a=c["x"][row * M:(row + 1) * M], m=1, n=2 * H, k=M, codes=up["codes"],
                                scales=up["scales"], correction=corr, correction_data=up["biases"],
                                layout=c["layout"], row_count=E * 2 * H, group_count=M // c["group"], bits=4,
                                group_size=c["group"], gather=up_ids, output_dt=O.BF16)
            assert st == 0
            act = O.gated_silu_bf16(proj, H, 1)
            down_ids = O.moe_gather_rows(ids, route, M, E, M)
            st, dproj = O.matmul(a=act, m=1, n=M, k=H, codes=down["codes"], scales=down["scales"], correction=corr,
                                 correction_data=down["biases"], layout=c["layout"], row_count=E * M,
                                 group_count=H // c["group"], bits=4, group_size=c["group"], gather=down_ids,
                                 output_dt=O.BF16)
            assert st == 0
            O.moe_accumulate(dproj, w, acc, out, M, route, row * M, rank == 0, rank + 1 == A, round_products,
                             round_acc)
    return out


@pytest.mark.parametrize("rows,layout,biased,gains,flags", [
    (1, 1, True, False, (False, False, False, False, False)),
    (3, 0, True, True, (True, True, False, False, True)),
    (5, 1, False, False, (False, False, True, True, True)),
])
def test_routed_oracle_is_the_reference_loop(oracle, rows, layout, biased, gains, flags):
    O = oracle
    c = MC.case(O, 7 + rows, rows, model=128, hidden=64, experts=8, active=3, layout=layout, biased=biased,
                gains=gains)
    rl, rw, rp, ra, si = flags
    got = O.routed_experts(c["x"], c["logits"], c["up"], c["down"], rows, 128, 64, 8, 3, expert_scales=c["scales"],
                           layout=layout, round_logits=rl, round_weights=rw, round_products=rp,
                           round_accumulator=ra, sort_ids=si)
    want = loop_composition(O, c, rl, rw, rp, ra, si)
    assert np.array_equal(got, want)


def test_routed_oracle_against_f64(oracle):
    """Closed form in f64 from the dequantised banks (bf16 rounding only where
    the reference writes bf16 is left out, so the bound is loose)."""
    O = oracle
    R, M, H, E, A = 2, 128, 64, 8, 2
    c = MC.case(O, 3, R, M, H, E, A, layout=0)
    got = O.bf16_to_f32(O.routed_experts(c["x"], c["logits"], c["up"], c["down"], R, M, H, E, A, layout=0))
    ids, w = O.moe_route(c["logits"], R, E, A)

    def deq(b, rows, cols):
        codes = b["codes"].reshape(rows, cols // 2)
        q = np.stack([codes & 15, codes >> 4], axis=-1).reshape(rows, cols).astype(np.float64)
        s = O.bf16_to_f32(b["scales"]).reshape(rows, cols // 64).astype(np.float64)
        bb = O.bf16_to_f32(b["biases"]).reshape(rows, cols // 64).astype(np.float64)
        return q * np.repeat(s, 64, 1) + np.repeat(bb, 64, 1)

    Wu, Wd = deq(c["up"], E * 2 * H, M), deq(c["down"], E * M, H)
    x = O.bf16_to_f32(c["x"]).astype(np.float64).reshape(R, M)
    want = np.zeros((R, M))
    for r in range(R):
        for k in range(A):
            e = ids[r * A + k]
            p = Wu[e * 2 * H:(e + 1) * 2 * H] @ x[r]
            v, g = p[:H], p[H:]
            act = v * g / (1 + np.exp(-g))
            want[r] += w[r * A + k] * (Wd[e * M:(e + 1) * M] @ act)
    err = np.abs(got.reshape(R, M) - want)
    assert err.max() <= 0.03 * np.abs(want).max() + 1e-3
