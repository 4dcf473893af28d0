"""numpy/ctypes wrapper over the C oracle (oracle/stark_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, and only as the checker. The product package
(stark_amd) never imports this module.

Every wrapped function restates a reference function; the citations live in
stark_oracle.c next to each definition.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libstark_oracle.so")

F32, F16, BF16 = 0, 1, 30
OUTPUT_GROUP, GROUP_OUTPUT = 0, 1
SYMMETRIC, BIASES, ZERO_POINTS = 0, 1, 2


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class MatmulArgs(C.Structure):
    _fields_ = [
        ("a", C.c_void_p), ("a_offset", C.c_size_t),
        ("b_values", C.c_void_p), ("b_leading_dimension", C.c_uint32),
        ("codes", C.c_void_p), ("codes_size", C.c_size_t),
        ("scales", C.c_void_p), ("correction", C.c_int), ("correction_data", C.c_void_p),
        ("layout", C.c_int), ("row_count", C.c_uint32), ("group_count", C.c_uint32),
        ("materialize_affine_input_sum", C.c_int), ("bits", C.c_int), ("group_size", C.c_uint32),
        ("signed_codes", C.c_int), ("b_transpose", C.c_int),
        ("d", C.c_void_p), ("ab_scale", C.c_float), ("accumulate", C.c_int), ("bias", C.c_void_p),
        ("has_soft_cap", C.c_int), ("soft_cap", C.c_float),
        ("gather_indices", C.c_void_p), ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32),
        ("weights_dt", C.c_int), ("input_dt", C.c_int), ("output_dt", C.c_int),
        ("a_codes", C.c_void_p), ("a_scales", C.c_void_p), ("a_scale_group_size", C.c_uint32),
        ("a_grouped_by_nibble", C.c_int), ("rht_factors", C.c_void_p),
    ]


def _declare(l):
    vp, sz, u32, u16, u8, i32, f = C.c_void_p, C.c_size_t, C.c_uint32, C.c_uint16, C.c_uint8, C.c_int, C.c_float
    sig = {
        "so_bf16_to_f32": (f, [u16]), "so_f32_to_bf16": (u16, [f]),
        "so_f16_to_f32": (f, [u16]), "so_f32_to_f16": (u16, [f]),
        "so_f32_to_bf16_n": (None, [vp, vp, sz]), "so_bf16_to_f32_n": (None, [vp, vp, sz]),
        "so_f32_to_f16_n": (None, [vp, vp, sz]), "so_f16_to_f32_n": (None, [vp, vp, sz]),
        "so_packed_code": (u8, [vp, i32, sz]),
        "so_quant_strides": (None, [i32, u32, u32, u32, vp, vp]),
        "so_matmul": (i32, [C.POINTER(MatmulArgs)]),
        "so_matmul_parallel": (i32, [C.POINTER(MatmulArgs), i32]),
        "so_reference_affine_linear_bf16": (None, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32]),
        "so_block_layout": (i32, [u32, vp, vp]),
        "so_scale_min": (None, [vp, i32, vp, vp]),
        "so_decode_block": (i32, [u32, vp, sz, vp, sz]),
        "so_hybrid_packed_matvec": (i32, [u32, vp, sz, sz, vp, vp]),
        "so_decode_rows": (i32, [u32, vp, sz, sz, vp]),
        "so_hybrid_affine_matvec": (i32, [vp, vp, vp, i32, i32, sz, sz, sz, vp, vp]),
        "so_moe_route": (None, [vp, vp, vp, u32, u32, u32, u32, u32]),
        "so_moe_gather_rows": (None, [vp, vp, u32, u32, u32, u32]),
        "so_moe_accumulate": (None, [vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32]),
        "so_moe_adjust_routes": (None, [vp, vp, vp, u32, u32, u32, u32]),
        "so_gated_silu_bf16": (None, [vp, vp, u32, u32]),
        "so_routed_experts": (i32, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, u32, i32, u32, u32, u32, u32,
                                    u32, i32, i32, i32, i32, i32, vp]),
        "so_quantize_affine": (None, [vp, sz, sz, i32, sz, i32, vp, vp, vp]),
        "so_quantize_q8_0": (None, [vp, sz, sz, vp]),
        "so_quantize_q4_k": (None, [vp, sz, sz, vp]),
        "so_hadamard32": (None, [vp]),
        "so_min_max_symmetric_divisor": (f, [vp, sz]),
        "so_quantize_symmetric_i8": (C.c_int8, [f, f]),
        "so_int8_code_index": (sz, [i32, sz]),
        "so_activation_transform": (i32, [vp, vp, vp, vp, vp, vp, vp, u32, u32, i32, i32, i32, u32, u32, i32, i32]),
        "so_activate": (f, [i32, f, i32, i32, f]),
        "so_gated_act_mul": (i32, [vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, i32, i32, f, i32, f, f, i32, f, f,
                                   i32, i32, i32, i32, u32, u32, i32]),
        "so_philox4x32_10": (None, [vp, vp, vp]),
        "so_unit_interval": (f, [u32]),
        "so_gumbel": (f, [C.c_uint64, u32, u32]),
        "so_unified_sampling": (i32, [vp, i32, vp, vp, vp, i32, f, i32, u32, i32, f, i32, f, u32, u32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args


def _p(a):
    return None if a is None else a.ctypes.data


# ----------------------------------------------------------------- conversions

def f32_to_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().so_f32_to_bf16_n(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().so_bf16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().so_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def f16_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().so_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def to_dtype_bits(x, dt) -> np.ndarray:
    """f32 values -> storage array of dtype id `dt` (uint16 bits or float32)."""
    if dt == F32:
        return np.ascontiguousarray(x, dtype=np.float32)
    return f32_to_bf16(x) if dt == BF16 else f32_to_f16(x)


def from_dtype_bits(x, dt) -> np.ndarray:
    if dt == F32:
        return np.asarray(x, dtype=np.float32)
    return bf16_to_f32(x) if dt == BF16 else f16_to_f32(x)


def packed_code(codes, bits: int, index: int) -> int:
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    return int(lib().so_packed_code(_p(codes), bits, index))


def quant_strides(layout: int, row_count: int, group_count: int, packing_divisor: int = 1):
    os_, gs = C.c_uint32(), C.c_uint32()
    lib().so_quant_strides(layout, row_count, group_count, packing_divisor, C.byref(os_), C.byref(gs))
    return os_.value, gs.value


# ----------------------------------------------------------------- matmul

def matmul(*, a, m, n, k, codes=None, scales=None, correction=BIASES, correction_data=None,
           layout=OUTPUT_GROUP, row_count=None, group_count=None, bits=4, group_size=64,
           signed_codes=False, materialize=False, b_values=None, b_leading_dimension=0, b_transpose=True,
           d=None, ab_scale=1.0, accumulate=False, bias=None, soft_cap=None, gather=None,
           weights_dt=BF16, input_dt=BF16, output_dt=BF16, a_offset=0, threads=0, a_codes=None, a_scales=None,
           a_scale_group_size=0, a_grouped_by_nibble=False, rht_factors=None):
    """MatmulCpuKernel::encode restated. Arrays are storage arrays (uint16 bits
    for bf16/f16, float32 for f32). Returns (status, d)."""
    keep = []

    def arr(x, dtype=None):
        if x is None:
            return None
        x = np.ascontiguousarray(x, dtype=dtype) if dtype is not None else np.ascontiguousarray(x)
        keep.append(x)
        return x

    out_np = np.float32 if output_dt == F32 else np.uint16
    if d is None:
        d = np.zeros(m * n, out_np)
    d = np.ascontiguousarray(d, dtype=out_np).copy()
    args = MatmulArgs()
    args.a = _p(arr(a))
    args.a_offset = a_offset
    args.b_values = _p(arr(b_values))
    args.b_leading_dimension = b_leading_dimension
    c = arr(codes, np.uint8)
    args.codes = _p(c)
    args.codes_size = 0 if c is None else c.size
    args.scales = _p(arr(scales))
    args.correction = correction
    args.correction_data = _p(arr(correction_data))
    args.layout = layout
    args.row_count = n if row_count is None else row_count
    args.group_count = (k // group_size if group_size else 0) if group_count is None else group_count
    args.materialize_affine_input_sum = int(materialize)
    args.bits = bits
    args.group_size = group_size
    args.signed_codes = int(signed_codes)
    args.b_transpose = int(b_transpose)
    args.d = _p(d)
    args.ab_scale = ab_scale
    args.accumulate = int(accumulate)
    args.bias = _p(arr(bias))
    args.has_soft_cap = int(soft_cap is not None)
    args.soft_cap = 0.0 if soft_cap is None else soft_cap
    args.gather_indices = _p(arr(gather, np.uint32))
    args.m, args.n, args.k = m, n, k
    args.a_codes = _p(arr(a_codes, np.int8))
    args.a_scales = _p(arr(a_scales, np.float32))
    args.a_scale_group_size = a_scale_group_size
    args.a_grouped_by_nibble = int(a_grouped_by_nibble)
    args.rht_factors = _p(arr(rht_factors, np.int32))
    args.weights_dt, args.input_dt, args.output_dt = weights_dt, input_dt, output_dt
    if threads:
        st = lib().so_matmul_parallel(C.byref(args), threads)
    else:
        st = lib().so_matmul(C.byref(args))
    return st, d


def reference_affine_linear_bf16(input_bits, codes, scales, biases, m, n, k, bits=4, indices=None,
                                 bank_rows=None, sos=None, sgs=None, f32_out=False):
    G = k // 64
    if sos is None:
        sos, sgs = G, 1
    bank_rows = n if bank_rows is None else bank_rows
    input_bits = np.ascontiguousarray(input_bits, np.uint16)
    codes = np.ascontiguousarray(codes, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    biases = np.ascontiguousarray(biases, np.uint16)
    idx = None if indices is None else np.ascontiguousarray(indices, np.uint32)
    ob = None if f32_out else np.zeros(m * n, np.uint16)
    of = np.zeros(m * n, np.float32) if f32_out else None
    lib().so_reference_affine_linear_bf16(_p(input_bits), _p(codes), _p(scales), _p(biases), _p(idx), _p(ob),
                                          _p(of), m, n, k, bank_rows, bits, sos, sgs)
    return of if f32_out else ob


# ----------------------------------------------------------------- activation transforms

INPUT_RHT, OUTPUT_RHT, QUANTIZE, QUANTIZE_WITH_GROUP_SUMS = 0, 1, 2, 3
SILU, GELU_APPROX, GELU_EXACT, IDENTITY, SOFTPLUS, SILU_MATERIALIZED_SIGMOID, GELU_MATERIALIZED_POLYNOMIAL = range(7)
GAM_FULL_PRECISION, GAM_QUANTIZE, GAM_QUANTIZE_WITH_GROUP_SUMS = 0, 1, 2


def hadamard32(v) -> np.ndarray:
    v = np.array(v, np.float32)
    assert v.size == 32
    lib().so_hadamard32(_p(v))
    return v


def int8_code_index(grouped: bool, index: int) -> int:
    return int(lib().so_int8_code_index(int(grouped), index))


def activation_transform(x, factors, batch, count, op, t_dt=F32, bias=None, bias_dt=F32, scale_group=0,
                         sum_group=0, grouped=False):
    """ActivationTransform (activation_transform.rs:48-156) out of place.
    Returns fp output (storage array) or (codes int8, scales f32, sums int32)."""
    x = np.ascontiguousarray(x)
    f = np.ascontiguousarray(factors, np.int32)
    quantize = op in (QUANTIZE, QUANTIZE_WITH_GROUP_SUMS)
    fp = None if quantize else np.zeros(batch * count, np.float32 if t_dt == F32 else np.uint16)
    q = np.zeros(batch * count, np.int8) if quantize else None
    sc = np.zeros(batch * (count // scale_group), np.float32) if quantize else None
    sums = np.zeros(batch * (count // sum_group), np.int32) if op == QUANTIZE_WITH_GROUP_SUMS else None
    b = None if bias is None else np.ascontiguousarray(bias)
    st = lib().so_activation_transform(_p(x), _p(fp), _p(b), _p(q), _p(sc), _p(sums), _p(f), batch, count, op,
                                       int(grouped), 0, scale_group, sum_group, t_dt, bias_dt)
    if st:
        raise ValueError(f"so_activation_transform status {st}")
    return (q, sc, sums) if quantize else fp


def activate(act_type, x, t_dt=F32, alpha=None) -> float:
    return float(lib().so_activate(act_type, float(x), t_dt, int(alpha is not None), 1.0 if alpha is None else alpha))


def gated_act_mul(act, gated_dim, batch, act_type=SILU, value=None, value_offset=0, value_row_stride=0,
                  interleaved=True, t_dt=F32, alpha=None, gate_clip=None, value_clip=None, op=GAM_FULL_PRECISION,
                  factors=None, scale_group=0, sum_group=0, grouped=False):
    """GatedActMul (gated_act_mul.rs:17-152). act: interleaved [batch, value|gate]
    or gates [batch, gated_dim] with value [.. value_row_stride]; storage arrays."""
    act = np.ascontiguousarray(act)
    val = None if value is None else np.ascontiguousarray(value)
    f = None if factors is None else np.ascontiguousarray(factors, np.int32)
    quantize = op != GAM_FULL_PRECISION
    fp = None if quantize else np.zeros(batch * gated_dim, np.float32 if t_dt == F32 else np.uint16)
    q = np.zeros(batch * gated_dim, np.int8) if quantize else None
    sc = np.zeros(batch * (gated_dim // scale_group), np.float32) if quantize else None
    sums = np.zeros(batch * (gated_dim // sum_group), np.int32) if op == GAM_QUANTIZE_WITH_GROUP_SUMS else None
    gmin, gmax = gate_clip if gate_clip else (0.0, 0.0)
    vmin, vmax = value_clip if value_clip else (0.0, 0.0)
    st = lib().so_gated_act_mul(_p(act), _p(val), _p(fp), _p(q), _p(sc), _p(sums), _p(f), gated_dim, batch,
                                value_offset, value_row_stride, act_type, int(alpha is not None),
                                1.0 if alpha is None else alpha, int(gate_clip is not None), gmin, gmax,
                                int(value_clip is not None), vmin, vmax, op, int(grouped), int(interleaved),
                                int(f is not None), scale_group, sum_group, t_dt)
    if st:
        raise ValueError(f"so_gated_act_mul status {st}")
    return (q, sc, sums) if quantize else fp


# ----------------------------------------------------------------- sampling

def philox4x32_10(ctr, key):
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.zeros(4, np.uint32)
    lib().so_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def gumbel(seed: int, index: int, vocab: int) -> float:
    return float(lib().so_gumbel(seed, index, vocab))


def unified_sampling(logits, batch, vocab, t_dt=F32, seeds=None, bitmask=None, temperature=None, top_k=None,
                     top_p=None, min_p=None):
    """UnifiedSampling (unified_sampling.rs:14-117). logits: storage array
    [batch, vocab]; returns uint32 token ids (0xFFFFFFFF: none)."""
    lg = np.ascontiguousarray(logits)
    sd = None if seeds is None else np.ascontiguousarray(seeds, np.uint64)
    bm = None if bitmask is None else np.ascontiguousarray(bitmask, np.uint32)
    out = np.zeros(batch, np.uint32)
    st = lib().so_unified_sampling(_p(lg), t_dt, _p(out), _p(sd), _p(bm), int(temperature is not None),
                                   0.0 if temperature is None else temperature, int(top_k is not None),
                                   0 if top_k is None else top_k, int(top_p is not None),
                                   0.0 if top_p is None else top_p, int(min_p is not None),
                                   0.0 if min_p is None else min_p, vocab, batch)
    if st:
        raise MemoryError("so_unified_sampling")
    return out


# ----------------------------------------------------------------- GGUF

def block_layout(kind: int):
    e, b = C.c_size_t(), C.c_size_t()
    if lib().so_block_layout(kind, C.byref(e), C.byref(b)):
        raise ValueError(f"unsupported kind {kind}")
    return e.value, b.value


def scale_min(scales12, index):
    s = np.ascontiguousarray(scales12, np.uint8)
    a, b = C.c_uint8(), C.c_uint8()
    lib().so_scale_min(_p(s), index, C.byref(a), C.byref(b))
    return a.value, b.value


def decode_block(kind: int, block_bytes) -> np.ndarray:
    e, _ = block_layout(kind)
    b = np.ascontiguousarray(block_bytes, np.uint8)
    out = np.zeros(e, np.float32)
    st = lib().so_decode_block(kind, _p(b), b.size, _p(out), e)
    if st:
        raise ValueError("invalid quantization block size")
    return out


def decode_rows(kind: int, data, rows: int, cols: int) -> np.ndarray:
    """decode_block over every block of `rows` rows of `cols` values."""
    e, bb = block_layout(kind)
    data = np.ascontiguousarray(data, np.uint8)
    if data.size != rows * (cols // e) * bb or cols % e:
        raise ValueError("data does not hold rows x cols values")
    out = np.zeros((rows, cols), np.float32)
    if lib().so_decode_rows(kind, _p(data), rows, cols, _p(out)):
        raise ValueError("invalid quantization block")
    return out


def hybrid_packed_matvec(kind, data, rows, cols, x) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(rows, np.float32)
    st = lib().so_hybrid_packed_matvec(kind, _p(data), rows, cols, _p(x), _p(out))
    if st:
        raise ValueError(f"status {st}")
    return out


def hybrid_affine_matvec(codes, scales, biases, scale_dt, bits, group, rows, cols, x) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint8)
    scales = np.ascontiguousarray(scales)
    biases = np.ascontiguousarray(biases)
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(rows, np.float32)
    st = lib().so_hybrid_affine_matvec(_p(codes), _p(scales), _p(biases), scale_dt, bits, group, rows, cols,
                                       _p(x), _p(out))
    if st:
        raise ValueError(f"status {st}")
    return out


# ----------------------------------------------------------------- MoE

def moe_route(logits, rows, experts, active, round_weights=False, round_logits=False):
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.zeros(rows * active, np.uint32)
    w = np.zeros(rows * active, np.float32)
    lib().so_moe_route(_p(logits), _p(ids), _p(w), rows, experts, active, int(round_weights), int(round_logits))
    return ids, w


def moe_gather_rows(ids, route_offset, rows_per_expert, experts, length):
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.zeros(length, np.uint32)
    lib().so_moe_gather_rows(_p(ids), _p(out), route_offset, rows_per_expert, experts, length)
    return out


def moe_accumulate(input_bits, weights, accumulator, output, length, weight_offset, output_offset, initialize,
                   finalize, round_product, round_accumulator):
    """In-place on accumulator (float32) and output (uint16 bf16 bits)."""
    lib().so_moe_accumulate(_p(np.ascontiguousarray(input_bits, np.uint16)),
                            _p(np.ascontiguousarray(weights, np.float32)), _p(accumulator), _p(output), length,
                            weight_offset, output_offset, int(initialize), int(finalize), int(round_product),
                            int(round_accumulator))


def moe_adjust_routes(ids, weights, scales, rows, experts, active, sort_ids):
    """In-place on ids (uint32) and weights (float32)."""
    lib().so_moe_adjust_routes(_p(ids), _p(weights), _p(np.ascontiguousarray(scales, np.float32)), rows, experts,
                               active, int(sort_ids))


def gated_silu_bf16(projected_bits, hidden, batch):
    p = np.ascontiguousarray(projected_bits, np.uint16)
    out = np.zeros(batch * hidden, np.uint16)
    lib().so_gated_silu_bf16(_p(p), _p(out), hidden, batch)
    return out


def routed_experts(input_bits, logits, up, down, rows, model, hidden, experts, active, expert_scales=None,
                   layout=GROUP_OUTPUT, bits=4, group=64, plane_dt=BF16, round_logits=False, round_weights=False,
                   round_products=False, round_accumulator=False, sort_ids=False) -> np.ndarray:
    """RoutedExperts::encode_scaled restated (routed.rs:154-257). up/down are
    dicts with codes, scales, biases (None = symmetric). Returns bf16 bits."""
    out = np.zeros(rows * model, np.uint16)
    keep = [np.ascontiguousarray(input_bits, np.uint16), np.ascontiguousarray(logits, np.float32)]
    gains = None if expert_scales is None else np.ascontiguousarray(expert_scales, np.float32)
    st = lib().so_routed_experts(_p(keep[0]), _p(keep[1]), _p(gains) if gains is not None else None,
                                 _p(up["codes"]), _p(up["scales"]), _p(up["biases"]) if up["biases"] is not None else None,
                                 _p(down["codes"]), _p(down["scales"]),
                                 _p(down["biases"]) if down["biases"] is not None else None, layout, bits, group,
                                 plane_dt, rows, model, hidden, experts, active, int(round_logits), int(round_weights),
                                 int(round_products), int(round_accumulator), int(sort_ids), _p(out))
    if st:
        raise ValueError(f"so_routed_experts status {st}")
    return out


# ----------------------------------------------------------------- generators

def quantize_affine(w, bits=4, group=64, layout=OUTPUT_GROUP):
    """Returns (codes u8 [rows, cols*bits/8], scales bf16 bits, biases bf16 bits)."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    G = cols // group
    codes = np.zeros((rows, cols * bits // 8), np.uint8)
    if layout == OUTPUT_GROUP:
        shape = (rows, G)
    else:
        shape = (G, (rows + 3) // 4 * 4)
    scales = np.zeros(shape, np.uint16)
    biases = np.zeros(shape, np.uint16)
    lib().so_quantize_affine(_p(w), rows, cols, bits, group, layout, _p(codes), _p(scales), _p(biases))
    return codes, scales, biases


def quantize_q8_0(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.zeros((rows, cols // 32 * 34), np.uint8)
    lib().so_quantize_q8_0(_p(w), rows, cols, _p(out))
    return out


def quantize_q4_k(w):
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    out = np.zeros((rows, cols // 256 * 144), np.uint8)
    lib().so_quantize_q4_k(_p(w), rows, cols, _p(out))
    return out
