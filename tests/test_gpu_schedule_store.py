"""The matvec schedule store filled past its capacity, from two streams.

Every shape set (the ops' tile counts and depths, the grid) gets a device
schedule in a fixed 4 MiB array per GPU. When it is full, an eager call
synchronizes the device and drops the schedules no captured graph holds, so
no pending launch still reads words that a new upload writes. These calls run
about 2.5 fills' worth of distinct shape sets, alternating two streams with no
synchronization between calls, repeating each earlier shape set once more; each
product must equal, bit for bit, the same rows of one product computed before
(a row's sum is computed by one tile in a fixed order, whatever the schedule)."""
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu

K, G = 4096, 4096 // 64
N_MAX = 65536
STORE_WORDS = 1 << 20


def _args(qmm, codes, scales, biases, x, n, d):
    b = qmm.QuantizedB(codes=codes[: n * K // 2], scales=scales[: n * G], correction_data=biases[: n * G],
                       params=qmm.QuantParams(0, n, G))
    return qmm.MatmulArguments(a=x, m=1, n=n, k=K, d=d, b=b)


def test_store_refills_across_streams(qmm):
    g = torch.Generator(device="cuda").manual_seed(5)
    codes = torch.randint(0, 256, (N_MAX * K // 2,), dtype=torch.uint8, device="cuda", generator=g)
    scales = (torch.rand(N_MAX * G, device="cuda", generator=g) * 0.01).to(torch.bfloat16).view(torch.int16)
    biases = (torch.rand(N_MAX * G, device="cuda", generator=g) - 0.5).to(torch.bfloat16).view(torch.int16)
    x = torch.randn(K, device="cuda", generator=g).to(torch.bfloat16).view(torch.int16)
    kern = qmm.MatmulKernel(H.BF16, H.BF16, H.F32)
    full = torch.empty(N_MAX, dtype=torch.float32, device="cuda")
    kern.encode(_args(qmm, codes, scales, biases, x, N_MAX, full))
    torch.cuda.synchronize()

    # distinct row counts (multiples of 32): a schedule holds about grid + 1 + n / 32 words
    ns = [N_MAX - 32 * i for i in range(1, 1101)]
    words = sum((513 + n // 32 + 63) // 64 * 64 for n in ns)
    assert words > 2 * STORE_WORDS, words
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = []
    for i, n in enumerate(ns):
        for rep in ((n,) if i % 2 else (n, ns[i // 2])):  # every other call repeats an earlier shape set
            d = torch.empty(rep, dtype=torch.float32, device="cuda")
            s = streams[len(outs) % 2]
            d.record_stream(s)
            kern.encode(_args(qmm, codes, scales, biases, x, rep, d), stream=s)
            outs.append((rep, d))
    for s in streams:
        torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want = full.view(torch.int32)
    bad = [(n, int((d.view(torch.int32) != want[:n]).sum().item())) for n, d in outs]
    bad = [b for b in bad if b[1]]
    assert not bad, f"{len(bad)} of {len(outs)} products differ; first (rows, outputs): {bad[:4]}"
