"""stark_qmm_routed_experts_static (the allocation-free entry point) against
stark_qmm_routed_experts on the same inputs: two calls in a row, the second
with a smaller input, both bit-identical to the workspace entry point (the two
entry points run the same kernels; only where the workspace lives differs).
Also: a call whose workspace would exceed the fixed scratch is rejected."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests import moe_cases as MC

pytestmark = pytest.mark.gpu


def _banks(qmm, c):
    E, M, Hd = c["experts"], c["model"], c["hidden"]

    def qb(b, rows, cols):
        return qmm.QuantizedB(codes=H.to_dev(b["codes"]), scales=H.to_dev(b["scales"]),
                              correction_data=H.to_dev(b["biases"]),
                              params=qmm.QuantParams(c["layout"], rows, cols // c["group"]), group_size=c["group"])

    return qb(c["up"], E * 2 * Hd, M), qb(c["down"], E * M, Hd)


def _both(qmm, c):
    R, M, Hd, E, A = c["rows"], c["model"], c["hidden"], c["experts"], c["active"]
    up, down = _banks(qmm, c)
    x, lg = H.to_dev(c["x"]), H.to_dev(c["logits"])
    want = qmm.routed_experts(x, lg, up, down, R, M, Hd, E, A)
    out = torch.full((R * M,), float("nan"), dtype=torch.bfloat16, device="cuda")
    got = qmm.routed_experts_static(x, lg, up, down, R, M, Hd, E, A, output=out)
    torch.cuda.synchronize()
    return got.view(torch.int16).cpu().numpy(), want.view(torch.int16).cpu().numpy()


def test_static_matches_workspace_entry_point_twice(qmm, oracle):
    big = MC.case(oracle, 71, 16, model=2048, hidden=768, experts=128, active=8)
    small = MC.case(oracle, 72, 3, model=256, hidden=128, experts=16, active=4)
    for c in (big, small):  # the second call is smaller and reuses the scratch
        got, want = _both(qmm, c)
        assert np.array_equal(got, want), f"rows {c['rows']}: {int((got != want).sum())} outputs differ"


def test_static_rejects_workspace_beyond_scratch(qmm, oracle):
    rows, model, hidden, experts, active = 1024, 4096, 1536, 128, 8
    assert qmm.routed_experts_workspace_size(rows, model, hidden, experts, active) > qmm.ROUTED_STATIC_SCRATCH_BYTES
    c = MC.case(oracle, 73, 2, model=256, hidden=128, experts=8, active=2)
    up, down = _banks(qmm, c)
    x = torch.zeros(rows * model, dtype=torch.int16, device="cuda")
    lg = torch.zeros(rows * experts, dtype=torch.float32, device="cuda")
    out = torch.empty(rows * model, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(qmm.MatmulError) as e:
        qmm.routed_experts_static(x, lg, up, down, rows, model, hidden, experts, active, output=out)
    assert e.value.status == qmm.WORKSPACE_TOO_SMALL
