"""Python mirror of the reference's quantized-matmul operator API over the C ABI.

The classes keep the reference's names and argument meaning:

* ``MatmulKernel`` -- trait MatmulKernel
  (crates/stark-engine/src/backends/common/kernel/matmul/kernel.rs:15-79)
* ``MatmulArguments`` / ``QuantizedB`` / ``QuantParams`` / ``MatmulDOps`` --
  crates/stark-engine/src/backends/common/kernel/matmul/{arguments.rs:7-25,
  matmul_b.rs:6-29, mod.rs:19-41, d_ops.rs:3-9}
* ``MatmulError`` -- crates/stark-engine/src/backends/common/kernel/matmul/error.rs:10-31
* ``mapped_many`` -- crates/stark-engine/src/engine/hybrid/weight_metal.rs:539-545
* ``moe_*`` -- crates/stark-engine/src/backends/cpu/kernel/moe.rs

Tensors are torch tensors on the GPU (torch is used only for device memory
and the current stream); every call goes through libstark_qmm.so. There is no
CPU fallback: if the library cannot be loaded the import fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("QMM_LIB_OVERRIDE") or os.path.join(HERE, "libstark_qmm.so")

# ---------------------------------------------------------------- constants

ABI_VERSION = 2
OK = 0
INVALID_ARGUMENT = 1
ABI_MISMATCH = 2
UNSUPPORTED_DATA_TYPE = 3
UNSUPPORTED_GROUP_SIZE = 4
UNSUPPORTED_D_OP = 5
UNSUPPORTED_LAYOUT = 6
INCOMPATIBLE_A = 7
UNSUPPORTED = 8
OUT_OF_MEMORY = 9
DEVICE_FAILURE = 10
WORKSPACE_TOO_SMALL = 11
KEY_NOT_FOUND = 12
INVALID_TENSOR = 13
HEADER_ERROR = 14
IO_ERROR = 15
UNSUPPORTED_CONFIGURATION = 16

F32, F16, BF16 = 0, 1, 30
U32, I64, I32, U8, I8, U64 = 101, 102, 103, 104, 105, 106
OUTPUT_GROUP, GROUP_OUTPUT = 0, 1
SYMMETRIC, BIASES, ZERO_POINTS = 0, 1, 2
MODE_U4, MODE_I8, MODE_U8, MODE_U5, MODE_U6, MODE_U3 = 0, 1, 2, 3, 4, 5
KIND_Q8_0, KIND_Q4_K = 8, 12
FORMAT_PACKED, FORMAT_AFFINE = 0, 1

_TORCH_DT = {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}


class MatmulError(RuntimeError):
    def __init__(self, status: int, where: str = ""):
        self.status = status
        super().__init__(f"{where}: {status_string(status)} ({status})")


# ---------------------------------------------------------------- ctypes ABI

class _QuantParams(C.Structure):
    _fields_ = [("layout", C.c_uint32), ("row_count", C.c_uint32), ("group_count", C.c_uint32),
                ("materialize_affine_input_sum", C.c_uint32)]


class _B(C.Structure):
    _fields_ = [("values", C.c_void_p), ("codes", C.c_void_p), ("codes_size", C.c_uint64),
                ("scales", C.c_void_p), ("correction", C.c_uint32), ("correction_data", C.c_void_p),
                ("params", _QuantParams), ("mode", C.c_uint32), ("group_size", C.c_uint32),
                ("signed_codes", C.c_uint32)]


class _DOps(C.Structure):
    _fields_ = [("ab_scale", C.c_float), ("accumulate", C.c_uint32), ("bias", C.c_void_p),
                ("rht_factors", C.c_void_p), ("has_soft_cap", C.c_uint32), ("soft_cap", C.c_float)]


class _Args(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("a", C.c_void_p), ("a_offset", C.c_uint64), ("a_kind", C.c_uint32),
                ("a_scales", C.c_void_p), ("a_group_sums", C.c_void_p), ("a_scale_group_size", C.c_uint32),
                ("a_code_layout", C.c_uint32), ("b", _B),
                ("b_leading_dimension", C.c_uint32), ("b_transpose", C.c_uint32), ("d", C.c_void_p),
                ("d_ops", _DOps), ("gather_indices", C.c_void_p), ("m", C.c_uint32), ("n", C.c_uint32),
                ("k", C.c_uint32)]


class _MappedMatrix(C.Structure):
    _fields_ = [("codes", C.c_void_p), ("codes_length", C.c_uint64), ("scales", C.c_void_p),
                ("biases", C.c_void_p), ("plane_length", C.c_uint64)]


class _MappedOp(C.Structure):
    _fields_ = [("matrices", C.POINTER(_MappedMatrix)), ("matrix_count", C.c_uint32), ("inputs", C.c_void_p),
                ("input_length", C.c_uint64), ("rows", C.c_uint64), ("columns", C.c_uint64),
                ("rows_per_batch", C.c_uint64), ("format", C.c_uint32), ("packed_kind", C.c_uint32),
                ("scale_dtype", C.c_uint32), ("bits", C.c_uint32), ("group", C.c_uint32)]


class _RoutedArgs(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("input", C.c_void_p), ("router_logits", C.c_void_p),
                ("expert_scales", C.c_void_p), ("up", _B), ("down", _B), ("output", C.c_void_p),
                ("rows", C.c_uint32), ("model", C.c_uint32), ("hidden", C.c_uint32), ("experts", C.c_uint32),
                ("active", C.c_uint32), ("round_logits_bf16", C.c_uint32), ("round_weights_bf16", C.c_uint32),
                ("round_products_bf16", C.c_uint32), ("round_accumulator_bf16", C.c_uint32),
                ("sort_expert_ids", C.c_uint32), ("workspace", C.c_void_p), ("workspace_size", C.c_uint64)]


class _TensorInfo(C.Structure):
    _fields_ = [("dtype", C.c_uint32), ("rank", C.c_uint32), ("shape", C.c_uint64 * 8), ("offset", C.c_uint64),
                ("size", C.c_uint64), ("host", C.c_void_p)]


class _WeightSpec(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("kind", C.c_uint32), ("bits", C.c_uint32), ("group_size", C.c_uint32),
                ("layout", C.c_uint32), ("is_symmetric", C.c_uint32), ("materialize_affine_input_sum", C.c_uint32),
                ("source_output_widths", C.c_uint32 * 4), ("source_output_count", C.c_uint32)]


class _WeightMatrix(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("b", _B), ("rows", C.c_uint32), ("columns", C.c_uint32),
                ("source_output_widths", C.c_uint32 * 4), ("source_output_count", C.c_uint32),
                ("device", C.c_void_p * 3)]


class _RefAffineArgs(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("input", C.c_void_p), ("input_offset", C.c_uint64),
                ("input_size", C.c_uint64), ("weights", _B), ("values_size", C.c_uint64), ("scales_size", C.c_uint64),
                ("biases_size", C.c_uint64), ("source_output_width_count", C.c_uint32), ("indices", C.c_void_p),
                ("indices_size", C.c_uint64), ("output", C.c_void_p), ("output_dtype", C.c_uint32),
                ("m", C.c_uint32), ("n", C.c_uint32), ("k", C.c_uint32)]


class _SamplingArgs(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("logits", C.c_void_p), ("data_type", C.c_uint32),
                ("output", C.c_void_p), ("seeds", C.c_void_p), ("bitmask", C.c_void_p),
                ("has_temperature", C.c_uint32), ("temperature", C.c_float), ("has_top_k", C.c_uint32),
                ("top_k", C.c_uint32), ("has_top_p", C.c_uint32), ("top_p", C.c_float), ("has_min_p", C.c_uint32),
                ("min_p", C.c_float), ("vocab_size", C.c_uint32), ("batch_size", C.c_uint32)]


class _TransformArgs(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("op", C.c_uint32), ("data_type", C.c_uint32), ("in_place", C.c_uint32),
                ("input", C.c_void_p), ("output", C.c_void_p), ("bias", C.c_void_p), ("bias_data_type", C.c_uint32),
                ("q_out", C.c_void_p), ("scales_out", C.c_void_p), ("group_sums_out", C.c_void_p),
                ("rht_factors", C.c_void_p), ("batch_size", C.c_uint32), ("element_count", C.c_uint32),
                ("scale_group_size", C.c_uint32), ("sum_group_size", C.c_uint32),
                ("grouped_by_nibble", C.c_uint32)]


class _GatedArgs(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("op", C.c_uint32), ("data_type", C.c_uint32), ("act_type", C.c_uint32),
                ("interleaved", C.c_uint32), ("act_operand", C.c_void_p), ("value_operand", C.c_void_p),
                ("fp_out", C.c_void_p), ("q_out", C.c_void_p), ("scales_out", C.c_void_p),
                ("group_sums_out", C.c_void_p), ("hadamard_factors", C.c_void_p), ("gated_dim", C.c_uint32),
                ("batch_dim", C.c_uint32), ("value_offset", C.c_uint32), ("value_row_stride", C.c_uint32),
                ("has_activation_alpha", C.c_uint32), ("activation_alpha", C.c_float), ("clip_gate", C.c_uint32),
                ("gate_clip_min", C.c_float), ("gate_clip_max", C.c_float), ("clip_value", C.c_uint32),
                ("value_clip_min", C.c_float), ("value_clip_max", C.c_float), ("scale_group_size", C.c_uint32),
                ("sum_group_size", C.c_uint32), ("grouped_by_nibble", C.c_uint32)]


class _Prologue(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("kind", C.c_uint32), ("data", C.c_void_p), ("eps", C.c_float)]


# Input prologues of stark_qmm_encode_many_prologue (no counterpart in the
# reference: its decoder launches the RMS norm and the gated SiLU separately).
PROLOGUE_NONE, PROLOGUE_RMS_NORM, PROLOGUE_SILU_GATE = 0, 1, 2


class _ChainProduct(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("stage", C.c_uint32), ("args", C.POINTER(_Args)),
                ("prologue", C.c_uint32), ("prologue_data", C.c_void_p), ("eps", C.c_float),
                ("in_tag", C.c_uint32), ("out_tag", C.c_uint32), ("acc_tag", C.c_uint32), ("k_slices", C.c_uint32),
                ("part_tag", C.c_uint32)]


# Every symbol include/stark_qmm.h declares, with its ctypes signature.
SIGNATURES = {
    "stark_qmm_abi_version": (C.c_uint32, []),
    "stark_qmm_status_string": (C.c_char_p, [C.c_uint32]),
    "stark_qmm_create": (C.c_uint32, [C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_void_p)]),
    "stark_qmm_encode": (C.c_uint32, [C.c_void_p, C.POINTER(_Args), C.c_void_p]),
    "stark_qmm_encode_many": (C.c_uint32, [C.c_void_p, C.POINTER(_Args), C.c_uint32, C.c_void_p]),
    "stark_qmm_encode_many_prologue": (C.c_uint32, [C.c_void_p, C.POINTER(_Args), C.c_uint32, C.POINTER(_Prologue),
                                                    C.c_void_p]),
    "stark_qmm_set_reference_accumulation": (C.c_uint32, [C.c_void_p, C.c_uint32]),
    "stark_qmm_chain_workspace_size": (C.c_uint32, [C.POINTER(_ChainProduct), C.c_uint32, C.POINTER(C.c_uint64)]),
    "stark_qmm_encode_chain": (C.c_uint32, [C.c_void_p, C.POINTER(_ChainProduct), C.c_uint32, C.c_void_p, C.c_void_p,
                                            C.c_uint64, C.c_void_p]),
    "stark_qmm_destroy": (None, [C.c_void_p]),
    "stark_qmm_mapped_many": (C.c_uint32, [C.POINTER(_MappedOp), C.c_uint32, C.POINTER(C.c_void_p), C.c_void_p]),
    "stark_qmm_mapped_many_async": (C.c_uint32, [C.POINTER(_MappedOp), C.c_uint32, C.POINTER(C.c_void_p),
                                                 C.c_void_p, C.c_void_p]),
    "stark_qmm_moe_route": (C.c_uint32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
                                         C.c_uint32, C.c_uint32, C.c_void_p]),
    "stark_qmm_moe_adjust_routes": (C.c_uint32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32,
                                                 C.c_uint32, C.c_uint32, C.c_void_p]),
    "stark_qmm_moe_gather_rows": (C.c_uint32, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, C.c_uint32,
                                               C.c_uint32, C.c_void_p]),
    "stark_qmm_moe_accumulate": (C.c_uint32, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32,
                                              C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                              C.c_uint32, C.c_void_p]),
    "stark_qmm_routed_experts_workspace_size": (C.c_uint64, [C.c_uint32] * 5),
    "stark_qmm_routed_experts": (C.c_uint32, [C.POINTER(_RoutedArgs), C.c_void_p]),
    "stark_qmm_routed_experts_static": (C.c_uint32, [C.POINTER(_RoutedArgs), C.c_void_p]),
    "stark_qmm_last_error": (C.c_char_p, []),
    "stark_qmm_file_open": (C.c_uint32, [C.c_char_p, C.POINTER(C.c_void_p)]),
    "stark_qmm_file_close": (None, [C.c_void_p]),
    "stark_qmm_file_kind": (C.c_uint32, [C.c_void_p]),
    "stark_qmm_file_tensor_count": (C.c_uint64, [C.c_void_p]),
    "stark_qmm_file_tensor_name": (C.c_char_p, [C.c_void_p, C.c_uint64]),
    "stark_qmm_file_tensor": (C.c_uint32, [C.c_void_p, C.c_char_p, C.POINTER(_TensorInfo)]),
    "stark_qmm_file_metadata": (C.c_uint32, [C.c_void_p, C.c_char_p, C.POINTER(C.c_char_p)]),
    "stark_qmm_file_upload": (C.c_uint32, [C.c_void_p, C.c_char_p, C.POINTER(C.c_void_p), C.c_void_p]),
    "stark_qmm_device_free": (C.c_uint32, [C.c_void_p]),
    "stark_qmm_weight_matrix_load": (C.c_uint32, [C.c_void_p, C.c_char_p, C.POINTER(_WeightSpec), C.c_uint32,
                                                  C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(_WeightMatrix),
                                                  C.c_void_p]),
    "stark_qmm_weight_matrix_free": (None, [C.POINTER(_WeightMatrix)]),
    "stark_qmm_reference_affine_bf16": (C.c_uint32, [C.POINTER(_RefAffineArgs), C.c_void_p]),
    "stark_qmm_unified_sampling": (C.c_uint32, [C.POINTER(_SamplingArgs), C.c_void_p]),
    "stark_qmm_activation_transform": (C.c_uint32, [C.POINTER(_TransformArgs), C.c_void_p]),
    "stark_qmm_gated_act_mul": (C.c_uint32, [C.POINTER(_GatedArgs), C.c_void_p]),
}

_lib = None


def library_path() -> str:
    return LIB_PATH


def lib():
    """Load libstark_qmm.so, building it first if it is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _build
            _build.build()
        l = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        if l.stark_qmm_abi_version() != ABI_VERSION:
            raise RuntimeError("libstark_qmm ABI mismatch")
        _lib = l
    return _lib


def status_string(status: int) -> str:
    return lib().stark_qmm_status_string(status).decode()


def _check(status: int, where: str):
    if status != OK:
        raise MatmulError(status, where)


def _ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("stark_qmm operands must be GPU tensors")
    return t.data_ptr()


def _nbytes(t: Optional[torch.Tensor]) -> int:
    return 0 if t is None else t.numel() * t.element_size()


def _stream(stream) -> int:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


# ---------------------------------------------------------------- operator API

@dataclass
class QuantParams:
    layout: int
    row_count: int
    group_count: int
    materialize_affine_input_sum: bool = False


@dataclass
class QuantizedB:
    codes: torch.Tensor
    scales: torch.Tensor
    params: QuantParams
    mode: int = MODE_U4
    group_size: int = 64
    correction: int = BIASES
    correction_data: Optional[torch.Tensor] = None
    signed_codes: bool = False


@dataclass
class FullPrecisionB:
    values: torch.Tensor


@dataclass
class MatmulDOps:
    ab_scale: float = 1.0
    accumulate: bool = False
    bias: Optional[torch.Tensor] = None
    rht_factors: Optional[torch.Tensor] = None
    soft_cap: Optional[float] = None


# Int8CodeLayout (matmul_a.rs:6-9)
SEQUENTIAL, GROUPED_BY_NIBBLE = 0, 1


@dataclass
class Int8SymmetricA:
    """MatmulA::Int8Symmetric (matmul_a.rs:51-61): activation a[m, k] =
    values[m, index(k)] * scales[m, k // scale_group_size] with int8 values in
    `code_layout` order (as ActivationTransform::encode_quantize writes them)."""
    values: torch.Tensor
    scales: torch.Tensor
    scale_group_size: int
    group_sums: Optional[torch.Tensor] = None
    code_layout: int = SEQUENTIAL


@dataclass
class MatmulArguments:
    a: object  # torch.Tensor (MatmulA::FullPrecision) | Int8SymmetricA
    b: object  # QuantizedB | FullPrecisionB
    d: torch.Tensor
    m: int
    n: int
    k: int
    a_offset: int = 0
    b_leading_dimension: int = 0
    b_transpose: bool = True
    d_transform: MatmulDOps = field(default_factory=MatmulDOps)
    gather_indices: Optional[torch.Tensor] = None


def _fill_b(dst: _B, b) -> None:
    if isinstance(b, LoadedB):
        C.memmove(C.byref(dst), C.byref(b.raw), C.sizeof(_B))
        return
    if isinstance(b, FullPrecisionB):
        dst.values = _ptr(b.values)
        dst.codes = None
        return
    dst.codes = _ptr(b.codes)
    dst.codes_size = _nbytes(b.codes)
    dst.scales = _ptr(b.scales)
    dst.correction = b.correction
    dst.correction_data = _ptr(b.correction_data)
    dst.params.layout = b.params.layout
    dst.params.row_count = b.params.row_count
    dst.params.group_count = b.params.group_count
    dst.params.materialize_affine_input_sum = int(b.params.materialize_affine_input_sum)
    dst.mode = b.mode
    dst.group_size = b.group_size
    dst.signed_codes = int(b.signed_codes)


def _args(a: MatmulArguments) -> _Args:
    s = _Args()
    s.struct_size = C.sizeof(_Args)
    if isinstance(a.a, Int8SymmetricA):
        q = a.a
        s.a = _ptr(q.values)
        s.a_kind = 1
        s.a_scales = _ptr(q.scales)
        s.a_group_sums = _ptr(q.group_sums)
        s.a_scale_group_size = q.scale_group_size
        s.a_code_layout = q.code_layout
    else:
        s.a = _ptr(a.a)
        s.a_offset = a.a_offset
    _fill_b(s.b, a.b)
    s.b_leading_dimension = a.b_leading_dimension
    s.b_transpose = int(a.b_transpose)
    s.d = _ptr(a.d)
    t = a.d_transform
    s.d_ops.ab_scale = t.ab_scale
    s.d_ops.accumulate = int(t.accumulate)
    s.d_ops.bias = _ptr(t.bias)
    s.d_ops.rht_factors = _ptr(t.rht_factors)
    s.d_ops.has_soft_cap = int(t.soft_cap is not None)
    s.d_ops.soft_cap = 0.0 if t.soft_cap is None else t.soft_cap
    s.gather_indices = _ptr(a.gather_indices)
    s.m, s.n, s.k = a.m, a.n, a.k
    return s


@dataclass
class PreparedBatch:
    array: object  # ctypes array of stark_qmm_args
    keep: list     # the MatmulArguments whose tensors the array points into
    prologue: object = None  # _Prologue, for batches issued through stark_qmm_encode_many_prologue
    prologue_data: object = None  # the tensor the prologue reads


@dataclass
class ChainProduct:
    """One product of a chained launch (stark_qmm_chain_product). Tagged rows
    are int32 tensors of words bf16 | tag << 16; tag 0 = plain bf16 row."""
    arguments: MatmulArguments
    stage: int
    prologue: int = PROLOGUE_NONE
    prologue_data: Optional[torch.Tensor] = None
    eps: float = 0.0
    in_tag: int = 0
    out_tag: int = 0
    acc_tag: int = 0
    k_slices: int = 1
    part_tag: int = 0


@dataclass
class PreparedChain:
    array: object      # ctypes array of stark_qmm_chain_product
    args: object       # the stark_qmm_args they point to
    keep: list         # the ChainProducts whose tensors they point into
    workspace_bytes: int


def tag_rows(values: torch.Tensor, tag: int) -> torch.Tensor:
    """bf16 values -> tagged words (int32): bits | tag << 16."""
    hi = (int(tag) & 0xffff) << 16
    return (values.contiguous().view(torch.int16).to(torch.int32) & 0xffff) | (hi - (1 << 32) if hi >= 1 << 31 else hi)


def untag_rows(words: torch.Tensor) -> torch.Tensor:
    """tagged words -> (bf16 values, tags)."""
    w = words.to(torch.int64) & 0xffffffff
    return (w & 0xffff).to(torch.int16).view(torch.bfloat16), (w >> 16).to(torch.int32)


class MatmulKernel:
    """trait MatmulKernel (kernel.rs:15-79) over stark_qmm_create/encode."""

    def __init__(self, weights_data_type: int, input_data_type: int, output_data_type: int):
        h = C.c_void_p()
        _check(lib().stark_qmm_create(weights_data_type, input_data_type, output_data_type, C.byref(h)),
               "MatmulKernel::new")
        self._h = h
        self.weights_data_type = weights_data_type
        self.input_data_type = input_data_type
        self.output_data_type = output_data_type

    def set_reference_accumulation(self, enabled: bool = True) -> None:
        _check(lib().stark_qmm_set_reference_accumulation(self._h, int(enabled)), "set_reference_accumulation")

    def encode(self, arguments: MatmulArguments, stream=None) -> None:
        s = _args(arguments)
        _check(lib().stark_qmm_encode(self._h, C.byref(s), _stream(stream)), "MatmulKernel::encode")

    def encode_many(self, arguments: Sequence[MatmulArguments], stream=None) -> None:
        arr = (_Args * len(arguments))(*[_args(a) for a in arguments])
        _check(lib().stark_qmm_encode_many(self._h, arr, len(arguments), _stream(stream)), "encode_many")

    def prepare_many(self, arguments: Sequence[MatmulArguments]) -> "PreparedBatch":
        """Marshal a batch of arguments once (the C structs and the tensors they
        point into are kept alive) so that encode_prepared() issues it with no
        per-call Python conversion, as a compiled caller would."""
        return PreparedBatch((_Args * len(arguments))(*[_args(a) for a in arguments]), list(arguments))

    def encode_prepared(self, batch: "PreparedBatch", stream=None) -> None:
        if batch.prologue is not None:
            _check(lib().stark_qmm_encode_many_prologue(self._h, batch.array, len(batch.keep), C.byref(batch.prologue),
                                                        _stream(stream)), "encode_many_prologue")
            return
        _check(lib().stark_qmm_encode_many(self._h, batch.array, len(batch.keep), _stream(stream)), "encode_many")

    @staticmethod
    def _prologue(kind: int, data, eps: float):
        if data is None or data.dtype != torch.bfloat16 or not data.is_contiguous():
            raise ValueError("the prologue operand must be a contiguous bf16 tensor")
        return _Prologue(C.sizeof(_Prologue), kind, data.data_ptr(), float(eps))

    def encode_many_prologue(self, arguments: Sequence[MatmulArguments], kind: int, data, eps: float = 0.0,
                             stream=None) -> None:
        """encode_many with an input prologue on the row every entry reads:
        PROLOGUE_RMS_NORM (data = norm weights [K], eps) or PROLOGUE_SILU_GATE
        (the row is the gate, data = up [K])."""
        arr = (_Args * len(arguments))(*[_args(a) for a in arguments])
        pro = self._prologue(kind, data, eps)
        _check(lib().stark_qmm_encode_many_prologue(self._h, arr, len(arguments), C.byref(pro), _stream(stream)),
               "encode_many_prologue")

    def prepare_many_prologue(self, arguments: Sequence[MatmulArguments], kind: int, data,
                              eps: float = 0.0) -> "PreparedBatch":
        return PreparedBatch((_Args * len(arguments))(*[_args(a) for a in arguments]), list(arguments),
                             self._prologue(kind, data, eps), data)

    def prepare_chain(self, products: Sequence["ChainProduct"]) -> "PreparedChain":
        """Marshal the products of a chained launch (stark_qmm_encode_chain) once;
        returns the batch and the workspace bytes it needs."""
        args = (_Args * len(products))(*[_args(p.arguments) for p in products])
        arr = (_ChainProduct * len(products))()
        for i, p in enumerate(products):
            if p.prologue != PROLOGUE_NONE and (p.prologue_data is None or not p.prologue_data.is_contiguous()):
                raise ValueError("a prologue needs a contiguous operand")
            arr[i] = _ChainProduct(C.sizeof(_ChainProduct), p.stage, C.pointer(args[i]), p.prologue,
                                   _ptr(p.prologue_data), float(p.eps), p.in_tag, p.out_tag, p.acc_tag, p.k_slices,
                                   p.part_tag)
        need = C.c_uint64()
        _check(lib().stark_qmm_chain_workspace_size(arr, len(products), C.byref(need)), "chain_workspace_size")
        return PreparedChain(arr, args, list(products), need.value)

    def encode_chain(self, chain: "PreparedChain", workspace: torch.Tensor, seq: Optional[torch.Tensor] = None,
                     stream=None) -> None:
        _check(lib().stark_qmm_encode_chain(self._h, chain.array, len(chain.keep), _ptr(seq), _ptr(workspace),
                                            _nbytes(workspace), _stream(stream)), "encode_chain")

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().stark_qmm_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# ---------------------------------------------------------------- BF16-effective reference dot

class ReferenceAffineBF16Matmul:
    """ReferenceAffineBF16Matmul (reference_affine.rs:105-280) over
    stark_qmm_reference_affine_bf16. encode() returns the [m, n] output it
    allocates, as the reference returns its scratch buffer."""

    def __init__(self, output_type: int):
        if output_type not in (BF16, F32):
            raise MatmulError(UNSUPPORTED_DATA_TYPE, "ReferenceAffineBF16Matmul::new")
        self.output_type = output_type

    def encode(self, input: torch.Tensor, input_offset: int, weights, indices: Optional[torch.Tensor], m: int,
               n: int, k: int, stream=None, source_output_widths: Sequence[int] = ()) -> torch.Tensor:
        s = _RefAffineArgs()
        s.struct_size = C.sizeof(_RefAffineArgs)
        s.input, s.input_offset, s.input_size = _ptr(input), input_offset, _nbytes(input)
        _fill_b(s.weights, weights)
        if isinstance(weights, FullPrecisionB):
            s.values_size = _nbytes(weights.values)
        elif isinstance(weights, QuantizedB):
            s.scales_size = _nbytes(weights.scales)
            s.biases_size = _nbytes(weights.correction_data)
        s.source_output_width_count = len(source_output_widths)
        s.indices, s.indices_size = _ptr(indices), _nbytes(indices)
        out = torch.empty(m * n, dtype=torch.float32 if self.output_type == F32 else torch.int16,
                          device=input.device)
        s.output, s.output_dtype = _ptr(out), self.output_type
        s.m, s.n, s.k = m, n, k
        _check(lib().stark_qmm_reference_affine_bf16(C.byref(s), _stream(stream)), "ReferenceAffineBF16Matmul::encode")
        return out


# ---------------------------------------------------------------- sampling

@dataclass
class SamplingMethod:
    """SamplingMethod (src/encodable_block/sampling/mod.rs:28-40): greedy when
    `stochastic` is False (no seeds), else Gumbel sampling with the filters."""
    stochastic: bool = False
    temperature: Optional[float] = None
    top_k: Optional[int] = None
    top_p: Optional[float] = None
    min_p: Optional[float] = None


def unified_sampling(logits: torch.Tensor, data_type: int, vocab_size: int, batch_size: int,
                     method: SamplingMethod = SamplingMethod(), seeds: Optional[torch.Tensor] = None,
                     bitmask: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """UnifiedSampling over stark_qmm_unified_sampling; returns [batch] uint32
    token ids as an int32 tensor (0xFFFFFFFF reads as -1)."""
    out = torch.empty(batch_size, dtype=torch.int32, device=logits.device)
    s = _SamplingArgs()
    s.struct_size = C.sizeof(_SamplingArgs)
    s.logits, s.data_type, s.output = _ptr(logits), data_type, _ptr(out)
    if method.stochastic and seeds is None:
        raise ValueError("stochastic sampling needs seeds")
    s.seeds = _ptr(seeds) if method.stochastic else None
    s.bitmask = _ptr(bitmask)
    for name in ("temperature", "top_k", "top_p", "min_p"):
        v = getattr(method, name)
        if v is not None:
            setattr(s, "has_" + name, 1)
            setattr(s, name, v)
    s.vocab_size, s.batch_size = vocab_size, batch_size
    _check(lib().stark_qmm_unified_sampling(C.byref(s), _stream(stream)), "Sampling::encode")
    return out


# ---------------------------------------------------------------- activation transforms

# ActivationTransformOp / ActivationType / GatedActMulOp ids of the C ABI
INPUT_RHT, OUTPUT_RHT, QUANTIZE, QUANTIZE_WITH_GROUP_SUMS = 0, 1, 2, 3
(ACT_SILU, ACT_GELU_APPROX, ACT_GELU_EXACT, ACT_IDENTITY, ACT_SOFTPLUS, ACT_SILU_MATERIALIZED_SIGMOID,
 ACT_GELU_MATERIALIZED_POLYNOMIAL) = range(7)
GATED_FULL_PRECISION, GATED_QUANTIZE, GATED_QUANTIZE_WITH_GROUP_SUMS = 0, 1, 2
HADAMARD_BLOCK = 32


@dataclass(frozen=True)
class ActivationQuantization:
    """ActivationQuantization (activation_transform.rs:18-55); build with new()."""
    scale_group_size: int
    sum_group_size: Optional[int]
    code_layout: int

    @staticmethod
    def new(scale_group_size: int, weight_group_size: int, emit_group_sums: bool,
            code_layout: int = SEQUENTIAL) -> Optional["ActivationQuantization"]:
        ok = scale_group_size in (32, 64, 128) and weight_group_size in (32, 64, 128) and \
            scale_group_size >= weight_group_size
        return ActivationQuantization(scale_group_size, weight_group_size if emit_group_sums else None,
                                      code_layout) if ok else None


class ActivationTransform:
    """ActivationTransform (activation_transform.rs:57-260) over
    stark_qmm_activation_transform."""

    def __init__(self, data_type: int, op: int, in_place: bool = False, bias_data_type: Optional[int] = None,
                 quantization: Optional[ActivationQuantization] = None):
        self.data_type, self.op, self.in_place = data_type, op, in_place
        self.bias_data_type, self.quantization = bias_data_type, quantization

    @classmethod
    def input_rht(cls, data_type: int, in_place: bool = False):
        return cls(data_type, INPUT_RHT, in_place)

    @classmethod
    def output_rht(cls, data_type: int, bias_data_type: Optional[int] = None, in_place: bool = False):
        return cls(data_type, OUTPUT_RHT, in_place, bias_data_type)

    @classmethod
    def quantize(cls, data_type: int, quantization: ActivationQuantization):
        op = QUANTIZE if quantization.sum_group_size is None else QUANTIZE_WITH_GROUP_SUMS
        return cls(data_type, op, False, None, quantization)

    def _base(self, factors, batch_size, element_count) -> _TransformArgs:
        s = _TransformArgs()
        s.struct_size = C.sizeof(_TransformArgs)
        s.op, s.data_type = self.op, self.data_type
        s.rht_factors = _ptr(factors)
        s.batch_size, s.element_count = batch_size, element_count
        return s

    def _run(self, s, stream, where):
        _check(lib().stark_qmm_activation_transform(C.byref(s), _stream(stream)), where)

    def encode_fp(self, input: torch.Tensor, output: torch.Tensor, rht_factors: torch.Tensor, batch_size: int,
                  element_count: int, stream=None) -> None:
        assert self.quantization is None and not self.in_place and self.bias_data_type is None
        s = self._base(rht_factors, batch_size, element_count)
        s.input, s.output = _ptr(input), _ptr(output)
        self._run(s, stream, "ActivationTransform::encode_fp")

    def encode_fp_in_place(self, data: torch.Tensor, rht_factors: torch.Tensor, bias: Optional[torch.Tensor],
                           batch_size: int, element_count: int, stream=None) -> None:
        assert self.quantization is None and self.in_place and (bias is None) == (self.bias_data_type is None)
        s = self._base(rht_factors, batch_size, element_count)
        s.in_place = 1
        s.output = _ptr(data)
        s.bias = _ptr(bias)
        s.bias_data_type = self.bias_data_type or 0
        self._run(s, stream, "ActivationTransform::encode_fp_in_place")

    def encode_quantize(self, input: torch.Tensor, q_out: torch.Tensor, scales_out: torch.Tensor,
                        group_sums_out: Optional[torch.Tensor], rht_factors: torch.Tensor, batch_size: int,
                        element_count: int, stream=None) -> None:
        q = self.quantization
        assert q is not None and (q.sum_group_size is None) == (group_sums_out is None)
        s = self._base(rht_factors, batch_size, element_count)
        s.input, s.q_out, s.scales_out, s.group_sums_out = _ptr(input), _ptr(q_out), _ptr(scales_out), \
            _ptr(group_sums_out)
        s.scale_group_size = q.scale_group_size
        s.sum_group_size = q.sum_group_size or 0
        s.grouped_by_nibble = int(q.code_layout == GROUPED_BY_NIBBLE)
        self._run(s, stream, "ActivationTransform::encode_quantize")


@dataclass
class GatedActMulSettings:
    """GatedActMulSettings (gated_act_mul.rs:21-27): clip bounds are (min, max) or None."""
    activation_alpha: Optional[float] = None
    gate_clipping: Optional[tuple] = None
    value_clipping: Optional[tuple] = None


class GatedActMul:
    """GatedActMul (gated_act_mul.rs:29-190) over stark_qmm_gated_act_mul."""

    def __init__(self, data_type: int, interleaved: bool, use_hadamard: bool, settings: GatedActMulSettings,
                 quantization: Optional[ActivationQuantization]):
        self.data_type, self.interleaved, self.use_hadamard = data_type, interleaved, use_hadamard
        self.settings, self.quantization = settings, quantization

    @classmethod
    def full_precision(cls, data_type: int, interleaved: bool, use_hadamard: bool,
                       settings: GatedActMulSettings = GatedActMulSettings()):
        return cls(data_type, interleaved, use_hadamard, settings, None)

    @classmethod
    def quantized(cls, data_type: int, quantization: ActivationQuantization,
                  settings: GatedActMulSettings = GatedActMulSettings()):
        return cls(data_type, True, True, settings, quantization)

    def _base(self, act_operand, factors, gated_dim, batch_dim, act_type) -> _GatedArgs:
        s = _GatedArgs()
        s.struct_size = C.sizeof(_GatedArgs)
        s.data_type, s.act_type, s.interleaved = self.data_type, act_type, int(self.interleaved)
        s.act_operand = _ptr(act_operand)
        s.hadamard_factors = _ptr(factors)
        s.gated_dim, s.batch_dim = gated_dim, batch_dim
        st = self.settings
        if st.activation_alpha is not None:
            s.has_activation_alpha, s.activation_alpha = 1, st.activation_alpha
        if st.gate_clipping is not None:
            s.clip_gate, (s.gate_clip_min, s.gate_clip_max) = 1, st.gate_clipping
        if st.value_clipping is not None:
            s.clip_value, (s.value_clip_min, s.value_clip_max) = 1, st.value_clipping
        return s

    def encode_fp(self, act_operand: torch.Tensor, value_operand: Optional[torch.Tensor], output: torch.Tensor,
                  hadamard_factors: Optional[torch.Tensor], gated_dim: int, batch_dim: int, value_offset: int,
                  value_row_stride: int, act_type: int, stream=None) -> None:
        assert self.quantization is None and self.interleaved == (value_operand is None)
        assert self.use_hadamard == (hadamard_factors is not None)
        s = self._base(act_operand, hadamard_factors, gated_dim, batch_dim, act_type)
        s.op = GATED_FULL_PRECISION
        s.value_operand, s.fp_out = _ptr(value_operand), _ptr(output)
        s.value_offset, s.value_row_stride = value_offset, value_row_stride
        _check(lib().stark_qmm_gated_act_mul(C.byref(s), _stream(stream)), "GatedActMul::encode_fp")

    def encode_quantized(self, act_operand: torch.Tensor, values: torch.Tensor, scales: torch.Tensor,
                         group_sums: Optional[torch.Tensor], hadamard_factors: torch.Tensor, gated_dim: int,
                         batch_dim: int, act_type: int, stream=None) -> None:
        q = self.quantization
        assert q is not None and (q.sum_group_size is None) == (group_sums is None)
        s = self._base(act_operand, hadamard_factors, gated_dim, batch_dim, act_type)
        s.op = GATED_QUANTIZE if q.sum_group_size is None else GATED_QUANTIZE_WITH_GROUP_SUMS
        s.q_out, s.scales_out, s.group_sums_out = _ptr(values), _ptr(scales), _ptr(group_sums)
        s.scale_group_size = q.scale_group_size
        s.sum_group_size = q.sum_group_size or q.scale_group_size
        s.grouped_by_nibble = int(q.code_layout == GROUPED_BY_NIBBLE)
        _check(lib().stark_qmm_gated_act_mul(C.byref(s), _stream(stream)), "GatedActMul::encode_quantized")


# ---------------------------------------------------------------- hybrid engine

@dataclass
class MappedMatrix:
    codes: torch.Tensor
    scales: Optional[torch.Tensor] = None
    biases: Optional[torch.Tensor] = None


@dataclass
class MappedOperation:
    """MappedOperation (weight_metal.rs:385-392); format is ("packed", kind) or
    ("affine", scale_dtype, bits, group)."""
    matrices: Sequence[MappedMatrix]
    inputs: torch.Tensor
    rows: int
    columns: int
    format: tuple
    rows_per_batch: int = 0


def _mapped_structs(operations):
    ops = (_MappedOp * len(operations))()
    keep = []
    for i, op in enumerate(operations):
        mats = (_MappedMatrix * len(op.matrices))()
        for j, mm in enumerate(op.matrices):
            mats[j].codes = _ptr(mm.codes)
            mats[j].codes_length = _nbytes(mm.codes)
            mats[j].scales = _ptr(mm.scales)
            mats[j].biases = _ptr(mm.biases)
            mats[j].plane_length = 0 if mm.scales is None else _nbytes(mm.scales)
        keep.append(mats)
        o = ops[i]
        o.matrices = mats
        o.matrix_count = len(op.matrices)
        o.inputs = _ptr(op.inputs)
        o.input_length = op.inputs.numel()
        o.rows, o.columns, o.rows_per_batch = op.rows, op.columns, op.rows_per_batch
        if op.format[0] == "packed":
            o.format = FORMAT_PACKED
            o.packed_kind = op.format[1]
        else:
            o.format = FORMAT_AFFINE
            o.scale_dtype, o.bits, o.group = op.format[1], op.format[2], op.format[3]
    return ops, keep


def mapped_many(operations: Sequence[MappedOperation], stream=None) -> list:
    """weight_metal::mapped_many: returns one f32 tensor per operation; raises
    MatmulError(INVALID_ARGUMENT) for invalid shapes or non-finite inputs."""
    ops, keep = _mapped_structs(operations)
    outs = [torch.empty(len(op.matrices) * op.rows, dtype=torch.float32, device=op.inputs.device)
            for op in operations]
    ptrs = (C.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    _check(lib().stark_qmm_mapped_many(ops, len(operations), ptrs, _stream(stream)), "mapped_many")
    del keep
    return outs


# ---------------------------------------------------------------- MoE

def moe_route(logits: torch.Tensor, rows: int, experts: int, active: int, round_weights=False,
              round_logits=False, stream=None):
    ids = torch.empty(rows * active, dtype=torch.int32, device=logits.device)
    w = torch.empty(rows * active, dtype=torch.float32, device=logits.device)
    _check(lib().stark_qmm_moe_route(_ptr(logits), _ptr(ids), _ptr(w), rows, experts, active, int(round_weights),
                                     int(round_logits), _stream(stream)), "moe_route")
    return ids, w


def moe_adjust_routes(ids, weights, scales, rows, experts, active, sort_ids, stream=None):
    _check(lib().stark_qmm_moe_adjust_routes(_ptr(ids), _ptr(weights), _ptr(scales), rows, experts, active,
                                             int(sort_ids), _stream(stream)), "moe_adjust_routes")


def moe_gather_rows(ids, route_offset, rows_per_expert, experts, length, stream=None):
    out = torch.empty(length, dtype=torch.int32, device=ids.device)
    _check(lib().stark_qmm_moe_gather_rows(_ptr(ids), _ptr(out), route_offset, rows_per_expert, experts, length,
                                           _stream(stream)), "moe_gather_rows")
    return out


def moe_accumulate(inp, weights, accumulator, output, length, weight_offset, output_offset, initialize, finalize,
                   round_product, round_accumulator, stream=None):
    _check(lib().stark_qmm_moe_accumulate(_ptr(inp), _ptr(weights), _ptr(accumulator), _ptr(output), length,
                                          weight_offset, output_offset, int(initialize), int(finalize),
                                          int(round_product), int(round_accumulator), _stream(stream)),
           "moe_accumulate")


def routed_experts_workspace_size(rows, model, hidden, experts, active) -> int:
    return int(lib().stark_qmm_routed_experts_workspace_size(rows, model, hidden, experts, active))


def mapped_prepare(operations: Sequence[MappedOperation]):
    """Marshal a mapped batch once; returns (prepared, outputs) for mapped_many_async."""
    ops, keep = _mapped_structs(operations)
    outs = [torch.empty(len(op.matrices) * op.rows, dtype=torch.float32, device=op.inputs.device)
            for op in operations]
    ptrs = (C.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    return (ops, len(operations), ptrs, keep, list(operations)), outs


def mapped_many_async(prepared, status_word: torch.Tensor, stream=None) -> None:
    """stark_qmm_mapped_many_async: stream-ordered; ORs 1 into status_word
    (device int32, caller-zeroed) when an input is not finite."""
    ops, n, ptrs = prepared[0], prepared[1], prepared[2]
    _check(lib().stark_qmm_mapped_many_async(ops, n, ptrs, _ptr(status_word), _stream(stream)), "mapped_many_async")


_NO_WORKSPACE = object()  # routed_experts_static: the library supplies the workspace


def routed_experts(input: torch.Tensor, router_logits: torch.Tensor, up: QuantizedB, down: QuantizedB, rows: int,
                   model: int, hidden: int, experts: int, active: int, expert_scales=None, round_logits=False,
                   round_weights=False, round_products=False, round_accumulator=False, sort_expert_ids=False,
                   workspace: Optional[torch.Tensor] = None, output: Optional[torch.Tensor] = None, stream=None,
                   prepare_only: bool = False):
    """RoutedExperts::encode_scaled (routed.rs:154-257) as one device pipeline."""
    need = routed_experts_workspace_size(rows, model, hidden, experts, active)
    if workspace is _NO_WORKSPACE:
        workspace = None
    elif workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=input.device)
    if output is None:
        output = torch.empty(rows * model, dtype=torch.bfloat16, device=input.device)
    s = _RoutedArgs()
    s.struct_size = C.sizeof(_RoutedArgs)
    s.input = _ptr(input)
    s.router_logits = _ptr(router_logits)
    s.expert_scales = _ptr(expert_scales)
    _fill_b(s.up, up)
    _fill_b(s.down, down)
    s.output = _ptr(output)
    s.rows, s.model, s.hidden, s.experts, s.active = rows, model, hidden, experts, active
    s.round_logits_bf16, s.round_weights_bf16 = int(round_logits), int(round_weights)
    s.round_products_bf16, s.round_accumulator_bf16 = int(round_products), int(round_accumulator)
    s.sort_expert_ids = int(sort_expert_ids)
    s.workspace = _ptr(workspace)
    s.workspace_size = 0 if workspace is None else _nbytes(workspace)
    if prepare_only:
        return s, (input, router_logits, expert_scales, up, down, workspace, output)
    _check(lib().stark_qmm_routed_experts(C.byref(s), _stream(stream)), "routed_experts")
    return output


ROUTED_STATIC_SCRATCH_BYTES = 8 << 20


def routed_experts_static(input: torch.Tensor, router_logits: torch.Tensor, up: QuantizedB, down: QuantizedB,
                          rows: int, model: int, hidden: int, experts: int, active: int, output: torch.Tensor,
                          expert_scales=None, round_logits=False, round_weights=False, round_products=False,
                          round_accumulator=False, sort_expert_ids=False, stream=None) -> torch.Tensor:
    """stark_qmm_routed_experts_static: routed_experts with the library's fixed
    per-GPU scratch as its workspace (no device allocation; `output` is the
    caller's). Calls that overlap on one GPU race on that scratch."""
    s, keep = routed_experts(input, router_logits, up, down, rows, model, hidden, experts, active,
                             expert_scales=expert_scales, round_logits=round_logits, round_weights=round_weights,
                             round_products=round_products, round_accumulator=round_accumulator,
                             sort_expert_ids=sort_expert_ids, workspace=_NO_WORKSPACE, output=output,
                             prepare_only=True)
    _check(lib().stark_qmm_routed_experts_static(C.byref(s), _stream(stream)), "routed_experts_static")
    del keep
    return output


def routed_experts_prepared(prepared, stream=None) -> None:
    """Issue a routed_experts call whose arguments were marshalled with
    routed_experts(..., prepare_only=True)."""
    _check(lib().stark_qmm_routed_experts(C.byref(prepared[0]), _stream(stream)), "routed_experts")


# ---------------------------------------------------------------- weight files

class WeightFileError(MatmulError):
    """A weight-file call failed: status plus the library's detail text."""

    def __init__(self, status: int, where: str, detail: str):
        super().__init__(status, f"{where}: {detail}")
        self.detail = detail


def _wcheck(status: int, where: str):
    if status != OK:
        raise WeightFileError(status, where, lib().stark_qmm_last_error().decode())


class DeviceBuffer:
    """Device memory returned by the library (stark_qmm_file_upload); usable
    wherever the mirror takes a device tensor (its bytes as uint8 elements)."""
    is_cuda = True

    def __init__(self, ptr: int, nbytes: int):
        self._ptr, self._n = ptr, nbytes

    def data_ptr(self) -> int:
        return self._ptr

    def numel(self) -> int:
        return self._n

    def element_size(self) -> int:
        return 1

    def free(self) -> None:
        if self._ptr:
            lib().stark_qmm_device_free(C.c_void_p(self._ptr))
            self._ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class TensorInfo:
    dtype: int
    shape: tuple
    offset: int
    size: int
    host: int  # address of the read-only mapping


class WeightFile:
    """stark_qmm_file: a Stark artifact (.safetensors, as ParameterLoader) or a
    GGUF v3 file / split directory (as the hybrid Weights::open)."""
    SAFETENSORS, GGUF = 0, 1

    def __init__(self, path: str):
        h = C.c_void_p()
        _wcheck(lib().stark_qmm_file_open(os.fsencode(path), C.byref(h)), "open")
        self._h = h

    @property
    def kind(self) -> int:
        return lib().stark_qmm_file_kind(self._h)

    def names(self) -> list:
        n = lib().stark_qmm_file_tensor_count(self._h)
        return [lib().stark_qmm_file_tensor_name(self._h, i).decode() for i in range(n)]

    def tensor(self, name: str) -> TensorInfo:
        info = _TensorInfo()
        _wcheck(lib().stark_qmm_file_tensor(self._h, name.encode(), C.byref(info)), f"tensor {name}")
        return TensorInfo(info.dtype, tuple(info.shape[:info.rank]), info.offset, info.size, info.host or 0)

    def host_bytes(self, name: str) -> bytes:
        t = self.tensor(name)
        return C.string_at(t.host, t.size)

    def metadata(self, key: str) -> str:
        v = C.c_char_p()
        _wcheck(lib().stark_qmm_file_metadata(self._h, key.encode(), C.byref(v)), f"metadata {key}")
        return v.value.decode()

    def upload(self, name: str, stream=None) -> DeviceBuffer:
        d = C.c_void_p()
        _wcheck(lib().stark_qmm_file_upload(self._h, name.encode(), C.byref(d), _stream(stream)), f"upload {name}")
        return DeviceBuffer(d.value, self.tensor(name).size)

    def close(self) -> None:
        if getattr(self, "_h", None):
            lib().stark_qmm_file_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


SPEC_FULL_PRECISION, SPEC_MLX, SPEC_INT = 0, 1, 2
OUTPUT_INPUT, INPUT_OUTPUT = 0, 1


@dataclass
class WeightMatrixSpec:
    """AnyWeightMatrixSpec: kind SPEC_FULL_PRECISION / SPEC_MLX / SPEC_INT."""
    kind: int
    bits: int = 4
    group_size: int = 64
    layout: int = OUTPUT_INPUT
    is_symmetric: bool = False
    materialize_affine_input_sum: bool = False
    source_output_widths: Sequence[int] = ()


class LoadedB:
    """The stark_qmm_b of a loaded weight matrix (device memory owned by the
    WeightMatrix that produced it)."""

    def __init__(self, raw: _B, owner):
        self.raw, self.owner = raw, owner


class WeightMatrix:
    """WeightMatrix::load (weight_matrix.rs:114-216) through
    stark_qmm_weight_matrix_load; `.b` goes into MatmulArguments."""

    def __init__(self, file: WeightFile, prefix: str, spec: WeightMatrixSpec, required_layout: int,
                 output_dim: int, input_dim: int, data_type: int, stream=None):
        s = _WeightSpec()
        s.struct_size = C.sizeof(_WeightSpec)
        s.kind, s.bits, s.group_size, s.layout = spec.kind, spec.bits, spec.group_size, spec.layout
        s.is_symmetric = int(spec.is_symmetric)
        s.materialize_affine_input_sum = int(spec.materialize_affine_input_sum)
        w = list(spec.source_output_widths)
        s.source_output_count = len(w)
        for i, v in enumerate(w[:4]):
            s.source_output_widths[i] = v
        m = _WeightMatrix()
        m.struct_size = C.sizeof(_WeightMatrix)
        st = lib().stark_qmm_weight_matrix_load(file._h, prefix.encode(), C.byref(s), required_layout, output_dim,
                                                input_dim, data_type, C.byref(m),
                                                None if stream is None and not torch.cuda.is_available()
                                                else _stream(stream))
        _wcheck(st, f"WeightMatrix::load {prefix}")
        self._m = m
        self.rows, self.columns = m.rows, m.columns
        self.source_output_widths = tuple(m.source_output_widths[:m.source_output_count])
        self.b = LoadedB(m.b, self)

    def free(self) -> None:
        if getattr(self, "_m", None) is not None:
            lib().stark_qmm_weight_matrix_free(C.byref(self._m))
            self._m = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
