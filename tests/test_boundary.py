"""The C-ABI library loads here (no GPU) and exports every symbol that
include/stark_qmm.h declares; argument validation that needs no device runs
on the CPU. No compute call is made."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "stark_qmm.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(stark_qmm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("stark_qmm_create", "stark_qmm_encode", "stark_qmm_mapped_many", "stark_qmm_moe_route",
              "stark_qmm_routed_experts"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from stark_amd import qmm
    lib = qmm.lib()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(declared_symbols()) == set(qmm.SIGNATURES), "python mirror out of sync with header"


def test_library_exports_only_the_c_abi():
    """Hidden visibility plus a version script: internal C++ symbols (kernel
    launchers, eligibility checks, std:: instantiations) stay local."""
    import subprocess
    from stark_amd import qmm
    qmm.lib()
    out = subprocess.run(["nm", "-D", "--defined-only", qmm.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    names = [ln.split()[-1] for ln in out.splitlines() if ln.strip()]
    extra = [n for n in names if not n.startswith("stark_qmm_") and not n.startswith("__hip_cuid_")]
    assert not extra, extra[:10]
    assert set(n for n in names if n.startswith("stark_qmm_")) == set(declared_symbols())


def test_abi_version_and_status_strings():
    from stark_amd import qmm
    assert qmm.lib().stark_qmm_abi_version() == qmm.ABI_VERSION == 2
    for s in range(17):
        assert qmm.status_string(s) and qmm.status_string(s) != "unknown status"
    assert qmm.status_string(999) == "unknown status"


def test_create_validates_dtypes_like_reference():
    """MatmulCpuKernel::new accepts only F32/F16/BF16 (kernel.rs:37-41)."""
    from stark_amd import qmm
    for dts in ((qmm.BF16, qmm.BF16, qmm.BF16), (qmm.F32, qmm.F16, qmm.BF16)):
        k = qmm.MatmulKernel(*dts)
        k.close()
    with pytest.raises(qmm.MatmulError) as e:
        qmm.MatmulKernel(qmm.BF16, 7, qmm.BF16)
    assert e.value.status == qmm.UNSUPPORTED_DATA_TYPE


def _raw_args(qmm, **over):
    s = qmm._Args()
    s.struct_size = C.sizeof(qmm._Args)
    s.a = 0x1000
    s.b.codes = 0x2000
    s.b.codes_size = 64
    s.b.scales = 0x3000
    s.b.correction = qmm.BIASES
    s.b.correction_data = 0x4000
    s.b.params.layout = 0
    s.b.params.row_count = 1
    s.b.params.group_count = 2
    s.b.mode = qmm.MODE_U4
    s.b.group_size = 64
    s.b_transpose = 1
    s.d = 0x5000
    s.d_ops.ab_scale = 1.0
    s.m, s.n, s.k = 1, 1, 128
    for key, v in over.items():
        obj = s
        parts = key.split(".")
        for p in parts[:-1]:
            obj = getattr(obj, p)
        setattr(obj, parts[-1], v)
    return s


def _raw_encode(qmm, **over):
    """Encode with raw device-free pointers: every case below must be rejected
    before any HIP call."""
    s = _raw_args(qmm, **over)
    h = C.c_void_p()
    assert qmm.lib().stark_qmm_create(qmm.BF16, qmm.BF16, qmm.BF16, C.byref(h)) == 0
    st = qmm.lib().stark_qmm_encode(h, C.byref(s), None)
    qmm.lib().stark_qmm_destroy(h)
    return st


def test_encode_rejections_without_device():
    from stark_amd import qmm
    assert _raw_encode(qmm, struct_size=8) == qmm.ABI_MISMATCH
    assert _raw_encode(qmm, **{"d_ops.rht_factors": 0x6000}) == qmm.UNSUPPORTED_D_OP
    # reference.rs:62-71: 1*128*4/8 = 64 bytes required
    assert _raw_encode(qmm, **{"b.codes_size": 63}) == qmm.UNSUPPORTED_LAYOUT
    assert _raw_encode(qmm, **{"b.group_size": 0}) == qmm.UNSUPPORTED_GROUP_SIZE
    assert _raw_encode(qmm, **{"b.mode": 77}) == qmm.INVALID_ARGUMENT
    # materialize policy (arguments.rs:36-61): signed codes / 8-bit / k%4 rejected
    assert _raw_encode(qmm, **{"b.params.materialize_affine_input_sum": 1, "b.signed_codes": 1}) == qmm.UNSUPPORTED_LAYOUT
    assert _raw_encode(qmm, **{"b.params.materialize_affine_input_sum": 1, "b.mode": qmm.MODE_U8,
                               "b.codes_size": 128}) == qmm.UNSUPPORTED_LAYOUT
    assert _raw_encode(qmm, **{"b.correction": qmm.BIASES, "b.correction_data": None}) == qmm.INVALID_ARGUMENT
    # empty products are a no-op
    assert _raw_encode(qmm, m=0) == qmm.OK


def test_encode_many_prologue_rejections_without_device():
    """stark_qmm_encode_many_prologue takes only batches the streaming kernel
    runs (one shared bf16 row, M = 1, 4-bit g64, K % 4096 == 0, N >= 32)."""
    from stark_amd import qmm
    big = dict(k=4096, n=64, **{"b.codes_size": 64 * 2048, "b.params.row_count": 64, "b.params.group_count": 64})

    def run(entries, kind=qmm.PROLOGUE_RMS_NORM, data=0x7000, size=None, ref_acc=False, x_dt=qmm.BF16):
        arr = (qmm._Args * len(entries))(*entries)
        pro = qmm._Prologue(C.sizeof(qmm._Prologue) if size is None else size, kind, data, 1e-6)
        h = C.c_void_p()
        assert qmm.lib().stark_qmm_create(qmm.BF16, x_dt, qmm.BF16, C.byref(h)) == 0
        if ref_acc:
            qmm.lib().stark_qmm_set_reference_accumulation(h, 1)
        st = qmm.lib().stark_qmm_encode_many_prologue(h, arr, len(entries), C.byref(pro), None)
        qmm.lib().stark_qmm_destroy(h)
        return st

    ok = _raw_args(qmm, **big)
    assert run([ok], size=8) == qmm.ABI_MISMATCH
    assert run([_raw_args(qmm, struct_size=8, **big)]) == qmm.ABI_MISMATCH
    assert run([ok], kind=qmm.PROLOGUE_NONE) == qmm.UNSUPPORTED
    assert run([ok], kind=9) == qmm.UNSUPPORTED
    assert run([ok], data=None) == qmm.INVALID_ARGUMENT
    assert run([ok], data=0x7008) == qmm.INVALID_ARGUMENT  # 16-byte alignment
    assert run([ok], ref_acc=True) == qmm.UNSUPPORTED
    assert run([ok], x_dt=qmm.F32) == qmm.UNSUPPORTED
    assert run([_raw_args(qmm)]) == qmm.UNSUPPORTED  # K = 128
    assert run([_raw_args(qmm, m=2, **big)]) == qmm.UNSUPPORTED
    assert run([_raw_args(qmm, **dict(big, n=16))]) == qmm.UNSUPPORTED
    assert run([ok, _raw_args(qmm, a=0x1100, **big)]) == qmm.UNSUPPORTED  # two different rows
    assert run([ok, _raw_args(qmm, **dict(big, k=8192, **{"b.codes_size": 64 * 4096}))]) == qmm.UNSUPPORTED
    assert run([_raw_args(qmm, **{"b.mode": qmm.MODE_U8, **big})]) == qmm.UNSUPPORTED
    assert run([_raw_args(qmm, **{"d_ops.rht_factors": 0x6000, **big})]) == qmm.UNSUPPORTED
    assert run([_raw_args(qmm, gather_indices=0x6000, **big)]) == qmm.UNSUPPORTED
    assert run([ok] * 9) == qmm.UNSUPPORTED
    assert run([_raw_args(qmm, **dict(big, **{"b.codes_size": 100}))]) == qmm.UNSUPPORTED_LAYOUT
    assert run([]) == qmm.OK


def test_mapped_many_validation_without_device():
    """parameters_for_input (weight_metal.rs:442-537) rejections."""
    from stark_amd import qmm
    lib = qmm.lib()
    mats = (qmm._MappedMatrix * 1)()
    mats[0].codes = 0x1000
    mats[0].codes_length = 4 * 64 // 2
    mats[0].scales = 0x2000
    mats[0].biases = 0x3000
    mats[0].plane_length = 4 * 1 * 2
    op = (qmm._MappedOp * 1)()
    op[0].matrices = mats
    op[0].matrix_count = 1
    op[0].inputs = 0x4000
    op[0].input_length = 64
    op[0].rows, op[0].columns = 4, 64
    op[0].format = qmm.FORMAT_AFFINE
    op[0].scale_dtype, op[0].bits, op[0].group = qmm.BF16, 4, 64
    outs = (C.c_void_p * 1)(0x5000)

    # validation is reached before any launch only for invalid descriptors;
    # the size bounds are parameters_for_input's (weight_metal.rs:456-466)
    big = 8_000_001
    for kw in ({"input_length": 63}, {"group": 16}, {"bits": 5}, {"scale_dtype": 9}, {"rows": 0},
               {"columns": 0}, {"rows_per_batch": 3}, {"format": 7}, {"rows": big},
               {"columns": big, "input_length": big}, {"input_length": big},
               {"rows": 4_000_004, "matrix_count": 2, "input_length": 128}):
        saved = {k: getattr(op[0], k) for k in kw}
        for k, v in kw.items():
            setattr(op[0], k, v)
        assert lib.stark_qmm_mapped_many_async(op, 1, outs, C.c_void_p(0x6000), None) == qmm.INVALID_ARGUMENT, kw
        for k, v in saved.items():
            setattr(op[0], k, v)
    op[0].format = qmm.FORMAT_PACKED
    op[0].packed_kind = 99
    assert lib.stark_qmm_mapped_many_async(op, 1, outs, C.c_void_p(0x6000), None) == qmm.UNSUPPORTED
    assert lib.stark_qmm_mapped_many_async(op, 0, outs, C.c_void_p(0x6000), None) == qmm.INVALID_ARGUMENT
    assert lib.stark_qmm_mapped_many_async(op, 65, outs, C.c_void_p(0x6000), None) == qmm.INVALID_ARGUMENT



def _chain_product(qmm, n, k, stage=0, prologue=0, in_tag=0, out_tag=0, acc_tag=0, k_slices=1, part_tag=0):
    """A chained product over fake (aligned, never dereferenced) addresses."""
    a = qmm._Args()
    a.struct_size = C.sizeof(qmm._Args)
    a.a, a.d = 0x10000, 0x20000
    a.b.codes, a.b.codes_size = 0x30000, n * k // 2
    a.b.scales, a.b.correction_data = 0x40000, 0x50000
    a.b.correction = 1  # biases
    a.b.params.layout, a.b.params.row_count, a.b.params.group_count = qmm.GROUP_OUTPUT, n, k // 64
    a.b.mode, a.b.group_size = qmm.MODE_U4, 64
    a.b_transpose = 1
    a.d_ops.ab_scale = 1.0
    a.m, a.n, a.k = 1, n, k
    p = qmm._ChainProduct(C.sizeof(qmm._ChainProduct), stage, C.pointer(a), prologue, 0x60000 if prologue else 0,
                          1e-6, in_tag, out_tag, acc_tag, k_slices, part_tag)
    return p, a


def _chain_bytes(qmm, *prods):
    arr = (qmm._ChainProduct * len(prods))(*[p for p, _ in prods])
    need = C.c_uint64()
    st = qmm.lib().stark_qmm_chain_workspace_size(arr, len(prods), C.byref(need))
    return st, need.value


def test_chain_validation_on_host():
    """stark_qmm_chain_workspace_size validates a chain without a device:
    the workspace of a 3-slice product, and the shapes, tags and stage order
    it refuses (STARK_QMM_UNSUPPORTED = 8, STARK_QMM_INVALID_ARGUMENT = 1)."""
    from stark_amd import qmm
    qmm.lib()
    assert qmm.PROLOGUE_SILU_GATE == 2
    down = dict(n=4096, k=12288, prologue=2, in_tag=3, out_tag=4, k_slices=3, part_tag=4)
    assert _chain_bytes(qmm, _chain_product(qmm, **down)) == (0, 256 + 2 * 4096 * 8)
    assert _chain_bytes(qmm, _chain_product(qmm, **{**down, "k_slices": 1})) == (0, 256)
    for bad in (dict(part_tag=0), dict(part_tag=0x8000), dict(k_slices=5), dict(in_tag=0x8000), dict(k_slices=1, out_tag=0, acc_tag=2),
                dict(prologue=1)):
        st, _ = _chain_bytes(qmm, _chain_product(qmm, **{**down, **bad}))
        assert st == 8, bad
    assert _chain_bytes(qmm, _chain_product(qmm, 4096 + 16, 4096))[0] == 8  # N % 32
    assert _chain_bytes(qmm, _chain_product(qmm, 4096, 2048))[0] == 8       # K % 4096
    st, _ = _chain_bytes(qmm, _chain_product(qmm, 4096, 4096, stage=1), _chain_product(qmm, 4096, 4096, stage=0))
    assert st == 1  # stages must not decrease
