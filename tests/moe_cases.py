"""Seeded routed-expert cases shared by the CPU oracle test and the GPU parity
test: banks flatten [experts, rows, cols] (routed.rs:1-5): up
[E*2*hidden, model] with rows [value(hidden) | gate(hidden)] per expert, down
[E*model, hidden]; MLX affine 4-bit with bf16 planes."""
import numpy as np


def bank(O, rng, rows, cols, group, layout, biased, scale=0.05):
    w = rng.normal(0, scale, (rows, cols)).astype(np.float32)
    codes, s, b = O.quantize_affine(w, 4, group, layout)
    return dict(codes=np.ascontiguousarray(codes.ravel()), scales=np.ascontiguousarray(s.ravel()),
                biases=np.ascontiguousarray(b.ravel()) if biased else None)


def case(O, seed, rows, model, hidden, experts, active, layout=1, group=64, biased=True, gains=False):
    rng = np.random.default_rng(seed)
    x = O.f32_to_bf16(rng.normal(0, 1, rows * model).astype(np.float32))
    logits = rng.normal(0, 2, rows * experts).astype(np.float32)
    up = bank(O, rng, experts * 2 * hidden, model, group, layout, biased)
    down = bank(O, rng, experts * model, hidden, group, layout, biased)
    scales = rng.uniform(0.5, 1.5, experts).astype(np.float32) if gains else None
    return dict(x=x, logits=logits, up=up, down=down, scales=scales, rows=rows, model=model, hidden=hidden,
                experts=experts, active=active, layout=layout, group=group)
