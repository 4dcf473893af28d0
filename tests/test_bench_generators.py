"""The bench's synthetic-weight generators must produce valid encodings:
decoding them with the oracle (decode_block, pinned by the reference's SHA-256
KATs) gives back the source weights to within each format's step."""
import numpy as np
import torch

import bench


def test_q8_0_generator_decodes(oracle):
    w = torch.randn(6, 256, generator=torch.Generator().manual_seed(1)) * 0.02
    blocks = bench.quantize_gguf_gpu(torch, w, 8).numpy()
    dec = oracle.decode_rows(8, blocks, 6, 256)
    step = np.abs(w.numpy()).reshape(6, 8, 32).max(axis=2, keepdims=True) / 127
    assert np.all(np.abs(dec.reshape(6, 8, 32) - w.numpy().reshape(6, 8, 32)) <= 0.51 * step + 1e-6)


def test_q4_k_generator_decodes(oracle):
    w = torch.randn(5, 512, generator=torch.Generator().manual_seed(2)) * 0.02
    blocks = bench.quantize_gguf_gpu(torch, w, 12).numpy()
    dec = oracle.decode_rows(12, blocks, 5, 512)
    g = w.numpy().reshape(5, 16, 32)
    span = g.max(axis=2, keepdims=True) - np.minimum(g.min(axis=2, keepdims=True), 0)
    # 4-bit step plus the 6-bit rounding of the sub-block scale and min
    assert np.all(np.abs(dec.reshape(5, 16, 32) - g) <= span / 15 * 0.75 + span / 63 * 2 + 1e-4)


def test_affine_u8_generator_decodes(oracle):
    w = torch.randn(4, 128, generator=torch.Generator().manual_seed(3)) * 0.02
    q, s, b = bench.quantize_gpu_bits(torch, w, 8)
    s = oracle.bf16_to_f32(s.numpy().view(np.uint16)).reshape(2, 4).T
    b = oracle.bf16_to_f32(b.numpy().view(np.uint16)).reshape(2, 4).T
    dec = q.numpy().reshape(4, 2, 64) * s[:, :, None] + b[:, :, None]
    # half a step, plus the bf16 rounding of the scale (x up to 255 steps) and of the bias
    bound = s[:, :, None] * (0.51 + 255 * 2.0 ** -9) + np.abs(b[:, :, None]) * 2.0 ** -8 + 1e-6
    assert np.all(np.abs(dec - w.numpy().reshape(4, 2, 64)) <= bound)
