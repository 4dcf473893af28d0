"""Shared builders for the parity tests: seeded inputs as numpy storage arrays
(uint16 bits for bf16/f16, float32 for f32) and their GPU copies."""
import numpy as np

F32, F16, BF16 = 0, 1, 30


def to_dev(a):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16))
    elif a.dtype == np.uint32:
        t = torch.from_numpy(a.view(np.int32))
    else:
        t = torch.from_numpy(a)
    return t.cuda()


def from_dev(t, dtype):
    a = t.cpu().numpy()
    return a.view(dtype) if a.dtype != dtype else a


def store(O, x, dt):
    return O.to_dtype_bits(x, dt)


def load(O, x, dt):
    return O.from_dtype_bits(x, dt)


def affine_weights(O, rng, n, k, bits=4, gs=64, layout=0, correction=1, w_dt=BF16, quantizer=True):
    """Returns dict(codes, scales, corr, zos/zgs...) as storage arrays. With
    quantizer=True weights are N(0, 0.02) quantized MLX-affine (scale = (max-min)/(2^bits-1), bias = min);
    otherwise codes/scales/biases are drawn like the reference's QuantInput
    (unit/common/matmul/quant.rs:132-186)."""
    G = k // gs
    if layout == 0:
        plane_shape = (n, G)
    else:
        plane_shape = (G, (n + 3) // 4 * 4)
    if quantizer and bits in (4, 8) and correction == 1 and w_dt == BF16:
        w = rng.normal(0, 0.02, (n, k)).astype(np.float32)
        codes, s, b = O.quantize_affine(w, bits, gs, layout)
        return dict(codes=codes.ravel(), scales=s.ravel(), corr=b.ravel(), plane_shape=plane_shape)
    codes = rng.integers(0, 256, (n * k * bits + 7) // 8, dtype=np.uint8)
    s = rng.uniform(0.01, 0.3, plane_shape).astype(np.float32)
    out = dict(codes=codes, scales=store(O, s.ravel(), w_dt), plane_shape=plane_shape)
    if correction == 1:
        out["corr"] = store(O, rng.uniform(-0.03, 0.03, plane_shape).astype(np.float32).ravel(), w_dt)
    elif correction == 2:
        pd = 8 // bits
        zos, zgs = O.quant_strides(layout, n, G, pd)
        zlen = ((n - 1) * zos + (G - 1) * zgs) // pd + 1
        out["corr"] = rng.integers(0, 256, zlen + 1, dtype=np.uint8)
    else:
        out["corr"] = None
    return out


def activations(O, rng, m, k, x_dt=BF16, scale=1.0):
    x = (rng.normal(0, 1, m * k) * scale).astype(np.float32)
    return store(O, x, x_dt)


def dequant_magnitude(O, codes, scales, corr, n, k, bits, gs, layout, correction, w_dt, x, x_dt, m, gather=None,
                      signed=False, out_n=None):
    """sum_k |w x| per output via the oracle itself on |x| and |w| is not available;
    compute |w| from a float64 decode instead (used only for the tolerance floor)."""
    G = k // gs
    os_, gs_ = O.quant_strides(layout, n, G, 1)
    sf = load(O, scales, w_dt).astype(np.float64)
    rows = n if gather is None else min(n, int(np.max(gather)) + 1)
    q = np.zeros((rows, k))
    c = np.asarray(codes, np.uint8)
    for r in range(rows):
        idx = (r * k + np.arange(k)) * bits
        lo = c[idx // 8].astype(np.int64)
        hi = np.where(idx // 8 + 1 < c.size, c[np.minimum(idx // 8 + 1, c.size - 1)], 0).astype(np.int64)
        v = (lo | (hi << 8)) >> (idx % 8)
        q[r] = v & ((1 << bits) - 1)
    if signed:
        q = np.bitwise_xor(q.astype(np.int64), 1 << (bits - 1)).astype(np.float64)
    g = np.arange(k) // gs
    s = sf[np.arange(rows)[:, None] * os_ + g[None, :] * gs_]
    if correction == 1:
        b = load(O, corr, w_dt).astype(np.float64)[np.arange(rows)[:, None] * os_ + g[None, :] * gs_]
    else:
        b = s * 2 ** bits  # generous bound for symmetric / zero-point offsets
    w = np.abs(s * q) + np.abs(b)
    xa = np.abs(load(O, x, x_dt).astype(np.float64)).reshape(m, k)
    mag = xa @ w.T  # [m, rows]
    if gather is None:
        return mag[:, :n]
    gi = np.asarray(gather).reshape(m, out_n if out_n is not None else n)
    return np.take_along_axis(mag, np.minimum(gi, rows - 1), axis=1)
