"""GPU parity of MatmulB::FullPrecision products (the MoE router and other
bf16 matrices; reference MatmulCpuKernel::encode,
crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:206-218)."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from tests.tolerances import check

pytestmark = pytest.mark.gpu


def run(qmm, O, m, n, k, w_dt=H.BF16, x_dt=H.BF16, d_dt=H.F32, transpose=True, ld=0, gather=None, seed=0,
        **dops):
    rng = np.random.default_rng(seed)
    rows = n if gather is None else int(max(gather)) + 1
    wshape = (rows, ld or k) if transpose else (k, ld or n)
    w = H.store(O, rng.normal(0, 0.05, wshape).astype(np.float32).ravel(), w_dt)
    x = H.store(O, rng.normal(0, 1, m * k).astype(np.float32), x_dt)
    st, want = O.matmul(a=x, m=m, n=n, k=k, b_values=w, b_leading_dimension=ld, b_transpose=transpose,
                        weights_dt=w_dt, input_dt=x_dt, output_dt=d_dt, gather=gather, codes=None, **dops)
    assert st == 0
    d = torch.zeros(m * n, dtype=torch.float32 if d_dt == H.F32 else torch.int16, device="cuda")
    kern = qmm.MatmulKernel(w_dt, x_dt, d_dt)
    kern.encode(qmm.MatmulArguments(a=H.to_dev(x), b=qmm.FullPrecisionB(values=H.to_dev(w)), d=d, m=m, n=n, k=k,
                                    b_leading_dimension=ld, b_transpose=transpose,
                                    gather_indices=None if gather is None else H.to_dev(np.asarray(gather,
                                                                                                   np.uint32))))
    torch.cuda.synchronize()
    got = H.load(O, H.from_dev(d, np.float32 if d_dt == H.F32 else np.uint16), d_dt)
    wf = H.load(O, w, w_dt).reshape(wshape)
    xf = np.abs(H.load(O, x, x_dt).reshape(m, k))
    wm = wf if transpose else wf.T
    if gather is not None:
        mag = np.stack([np.abs(wm[np.asarray(gather[i * n:(i + 1) * n])][:, :k]) @ xf[i] for i in range(m)])
    else:
        mag = xf @ np.abs(wm[:n, :k]).T
    check(got, H.load(O, want, d_dt), mag=mag.ravel(), label=f"dense m{m} n{n} k{k}")


@pytest.mark.parametrize("m", [1, 2, 4, 8, 9, 16])
def test_router_shape_bf16(qmm, oracle, m):
    """The Qwen3-MoE router: [128, 2048] bf16, f32 logits (fast bf16 path)."""
    run(qmm, oracle, m, 128, 2048, seed=m)


def test_other_dtypes_and_layouts(qmm, oracle):
    run(qmm, oracle, 3, 96, 520, w_dt=H.F32, x_dt=H.F32, seed=1)
    run(qmm, oracle, 2, 70, 256, w_dt=H.F16, x_dt=H.BF16, d_dt=H.BF16, seed=2)
    run(qmm, oracle, 2, 64, 128, transpose=False, seed=3)
    run(qmm, oracle, 1, 40, 256, ld=264, seed=4)
    run(qmm, oracle, 2, 24, 256, gather=list(np.random.default_rng(5).integers(0, 50, 48)), seed=5)
