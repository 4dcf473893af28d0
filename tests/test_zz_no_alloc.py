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
    # one token at the config-3 geometry: the fused route + up launch and the
    # fused down + accumulation launch, the decode case
    one = MC.case(oracle, 73, 1, model=2048, hidden=768, experts=128, active=8)
    for c in (big, small, one):  # each call is smaller than the first and reuses the scratch
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


def test_static_one_token_matches(qmm, oracle):
    """One token at the Qwen3-30B-A3B geometry: the fused route + up launch
    and the fused down + accumulation launch, on the static scratch."""
    c = MC.case(oracle, 74, 1, model=2048, hidden=768, experts=128, active=8)
    got, want = _both(qmm, c)
    assert np.array_equal(got, want), f"{int((got != want).sum())} outputs differ"


def test_static_under_graph_capture(qmm, oracle):
    """The allocation-free entry point recorded in a HIP graph: every replay
    with new inputs copied into the captured buffers equals an eager call of
    the workspace entry point on those inputs, with eager work and
    synchronizations between the replays."""
    R, M, Hd, E, A = 1, 2048, 768, 128, 8
    base = MC.case(oracle, 75, R, model=M, hidden=Hd, experts=E, active=A)
    up, down = _banks(qmm, base)
    x = H.to_dev(base["x"])
    lg = H.to_dev(base["logits"])
    out = torch.empty(R * M, dtype=torch.bfloat16, device="cuda")
    qmm.routed_experts_static(x, lg, up, down, R, M, Hd, E, A, output=out)  # eager first call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            qmm.routed_experts_static(x, lg, up, down, R, M, Hd, E, A, output=out, stream=s)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    rng = np.random.default_rng(76)
    for rep in range(4):
        nx = oracle.f32_to_bf16(rng.normal(0, 1, R * M).astype(np.float32))
        nl = rng.normal(0, 2, R * E).astype(np.float32)
        x.copy_(H.to_dev(nx))
        lg.copy_(H.to_dev(nl))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.view(torch.int16).cpu().numpy().copy()
        want = qmm.routed_experts(H.to_dev(nx), H.to_dev(nl), up, down, R, M, Hd, E, A)
        torch.cuda.synchronize()
        want = want.view(torch.int16).cpu().numpy()
        assert np.array_equal(got, want), f"replay {rep}: {int((got != want).sum())} outputs differ"
