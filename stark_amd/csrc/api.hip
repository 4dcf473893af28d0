// C ABI of the quantized matrix-product path (include/stark_qmm.h).
//
// Argument validation mirrors the reference so that a caller sees the same
// error for the same bad input:
// * MatmulCpuKernel::new dtype check (crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:37-41)
// * validate_affine_input_sum_policy (crates/stark-engine/src/backends/common/kernel/matmul/arguments.rs:36-61)
// * WeightData::from_b codes-size check (crates/stark-engine/src/backends/cpu/kernel/matmul/reference.rs:62-71)
// * MappedOperation::parameters_for_input (crates/stark-engine/src/engine/hybrid/weight_metal.rs:442-537)
#include <new>
#include <vector>

#include "qmm_common.h"
#include "stream_common.h"

struct stark_qmm_kernel {
    uint32_t w_dt, x_dt, d_dt;
    uint32_t reference_accumulation;
};

namespace {

using namespace qmm;

bool dtype_ok(uint32_t dt) { return dt == STARK_QMM_F32 || dt == STARK_QMM_F16 || dt == STARK_QMM_BF16; }

int mode_bits(uint32_t mode) {
    switch (mode) {
    case STARK_QMM_MODE_U4: return 4;
    case STARK_QMM_MODE_I8:
    case STARK_QMM_MODE_U8: return 8;
    case STARK_QMM_MODE_U5: return 5;
    case STARK_QMM_MODE_U6: return 6;
    case STARK_QMM_MODE_U3: return 3;
    default: return -1;
    }
}

// QuantParams::strides (crates/stark-engine/src/backends/common/kernel/matmul/mod.rs:131-156).
void quant_strides(uint32_t layout, uint32_t rows, uint32_t groups, uint32_t pd, uint32_t* os, uint32_t* gs) {
    if (layout == STARK_QMM_LAYOUT_OUTPUT_GROUP) {
        *os = (groups + pd - 1) / pd * pd;
        *gs = 1;
    } else {
        *os = 1;
        *gs = (rows + 3u) / 4u * 4u;
    }
}

stark_qmm_status build_affine_op(const stark_qmm_kernel* kr, const stark_qmm_b& b, uint32_t m, uint32_t n, uint32_t k,
                                 const void* x, void* d, const stark_qmm_d_ops& dops, const uint32_t* gather,
                                 AffineOp* op, int* bits_out) {
    const int bits = mode_bits(b.mode);
    if (bits < 0) return STARK_QMM_INVALID_ARGUMENT;
    if (b.group_size == 0) return STARK_QMM_UNSUPPORTED_GROUP_SIZE;
    if (b.params.layout > STARK_QMM_LAYOUT_GROUP_OUTPUT || b.correction > STARK_QMM_CORRECTION_ZERO_POINTS)
        return STARK_QMM_INVALID_ARGUMENT;
    // reference.rs:62-71: n*k*bits/8 (rounded up) bytes must be present
    const unsigned __int128 need = ((unsigned __int128)n * k * (unsigned)bits + 7) / 8;
    if (need > b.codes_size) return STARK_QMM_UNSUPPORTED_LAYOUT;
    if (!b.scales) return STARK_QMM_INVALID_ARGUMENT;
    if (b.correction != STARK_QMM_CORRECTION_SYMMETRIC && !b.correction_data) return STARK_QMM_INVALID_ARGUMENT;
    if (b.correction == STARK_QMM_CORRECTION_ZERO_POINTS && 8 % bits) return STARK_QMM_UNSUPPORTED_LAYOUT;
    AffineOp o{};
    o.codes = (const uint8_t*)b.codes;
    o.scales = b.scales;
    o.corr = b.correction_data;
    o.x = x;
    o.d = d;
    o.bias = dops.bias;
    o.gather = gather;
    o.n = n;
    o.k = k;
    o.m = m;
    quant_strides(b.params.layout, b.params.row_count, b.params.group_count, 1, &o.os, &o.gs);
    if (b.correction == STARK_QMM_CORRECTION_ZERO_POINTS)
        quant_strides(b.params.layout, b.params.row_count, b.params.group_count, 8u / bits, &o.zos, &o.zgs);
    o.group_size = b.group_size;
    o.corr_kind = b.correction;
    o.w_dt = kr->w_dt;
    o.x_dt = kr->x_dt;
    o.d_dt = kr->d_dt;
    o.flags = (dops.accumulate ? FLAG_ACCUMULATE : 0u) | (dops.has_soft_cap ? FLAG_SOFT_CAP : 0u) |
              (b.signed_codes ? FLAG_SIGNED : 0u);
    o.ab_scale = dops.ab_scale;
    o.soft_cap = dops.soft_cap;
    const uint64_t rowbits = (uint64_t)k * (uint64_t)bits;
    o.bank_rows = k == 0 ? n : (uint32_t)std::min<uint64_t>(0xffffffffull, b.codes_size * 8ull / rowbits);
    *op = o;
    *bits_out = bits;
    return STARK_QMM_OK;
}

}  // namespace

extern "C" {

uint32_t stark_qmm_abi_version(void) { return STARK_QMM_ABI_VERSION; }

const char* stark_qmm_status_string(stark_qmm_status s) {
    switch (s) {
    case STARK_QMM_OK: return "ok";
    case STARK_QMM_INVALID_ARGUMENT: return "invalid argument";
    case STARK_QMM_ABI_MISMATCH: return "ABI mismatch";
    case STARK_QMM_UNSUPPORTED_DATA_TYPE: return "unsupported data type";
    case STARK_QMM_UNSUPPORTED_GROUP_SIZE: return "unsupported group size";
    case STARK_QMM_UNSUPPORTED_D_OP: return "unsupported D-transform op";
    case STARK_QMM_UNSUPPORTED_LAYOUT: return "unsupported B layout";
    case STARK_QMM_INCOMPATIBLE_A: return "incompatible A operand";
    case STARK_QMM_UNSUPPORTED: return "unsupported";
    case STARK_QMM_OUT_OF_MEMORY: return "out of memory";
    case STARK_QMM_DEVICE_FAILURE: return "device failure";
    case STARK_QMM_WORKSPACE_TOO_SMALL: return "workspace too small";
    case STARK_QMM_KEY_NOT_FOUND: return "key not found";
    case STARK_QMM_INVALID_TENSOR: return "invalid tensor";
    case STARK_QMM_HEADER_ERROR: return "header loading error";
    case STARK_QMM_IO_ERROR: return "failed to read data";
    case STARK_QMM_UNSUPPORTED_CONFIGURATION: return "unsupported weight matrix configuration";
    default: return "unknown status";
    }
}

stark_qmm_status stark_qmm_create(uint32_t w_dt, uint32_t x_dt, uint32_t d_dt, stark_qmm_kernel** out) {
    if (!out) return STARK_QMM_INVALID_ARGUMENT;
    *out = nullptr;
    if (!dtype_ok(w_dt) || !dtype_ok(x_dt) || !dtype_ok(d_dt)) return STARK_QMM_UNSUPPORTED_DATA_TYPE;
    stark_qmm_kernel* k = new (std::nothrow) stark_qmm_kernel{w_dt, x_dt, d_dt, 0};
    if (!k) return STARK_QMM_OUT_OF_MEMORY;
    *out = k;
    return STARK_QMM_OK;
}

void stark_qmm_destroy(stark_qmm_kernel* k) { delete k; }

stark_qmm_status stark_qmm_set_reference_accumulation(stark_qmm_kernel* k, uint32_t enabled) {
    if (!k) return STARK_QMM_INVALID_ARGUMENT;
    k->reference_accumulation = enabled ? 1u : 0u;
    return STARK_QMM_OK;
}

}  // extern "C"

namespace {

// The product of MatmulCpuKernel::encode (kernel.rs:58-282) with the D ops in
// `dops` (the output RHT, when requested, runs after it).
stark_qmm_status encode_product(stark_qmm_kernel* kr, const stark_qmm_args* args, const stark_qmm_d_ops& dops,
                                hipStream_t stream) {
    const stark_qmm_b& b = args->b;
    const uint32_t m = args->m, n = args->n, k = args->k;
    const size_t xsz = kr->x_dt == STARK_QMM_F32 ? 4 : 2;
    if (args->a_kind > STARK_QMM_A_INT8_SYMMETRIC || args->a_code_layout > STARK_QMM_CODES_GROUPED_BY_NIBBLE)
        return STARK_QMM_INVALID_ARGUMENT;
    const bool a8 = args->a_kind == STARK_QMM_A_INT8_SYMMETRIC;
    const void* x = args->a && !a8 ? (const uint8_t*)args->a + args->a_offset * xsz : nullptr;

    if (!b.codes) {
        if (a8) return STARK_QMM_INCOMPATIBLE_A;
        // MatmulB::FullPrecision
        if (b.params.materialize_affine_input_sum) return STARK_QMM_UNSUPPORTED_LAYOUT;
        if (!b.values || (!x && m && n && k) || (!args->d && m && n)) return STARK_QMM_INVALID_ARGUMENT;
        DenseOp o{};
        o.w = b.values;
        o.x = x;
        o.d = args->d;
        o.bias = dops.bias;
        o.gather = args->gather_indices;
        o.n = n;
        o.k = k;
        o.m = m;
        o.transpose = args->b_transpose ? 1u : 0u;
        o.ld = args->b_leading_dimension ? args->b_leading_dimension : (args->b_transpose ? k : n);
        o.w_dt = kr->w_dt;
        o.x_dt = kr->x_dt;
        o.d_dt = kr->d_dt;
        o.flags = (dops.accumulate ? FLAG_ACCUMULATE : 0u) | (dops.has_soft_cap ? FLAG_SOFT_CAP : 0u);
        o.ab_scale = dops.ab_scale;
        o.soft_cap = dops.soft_cap;
        o.bank_rows = 0xffffffffu;
        return launch_dense_gemv(o, stream);
    }

    // validate_affine_input_sum_policy (arguments.rs:36-61)
    const bool materialize = b.params.materialize_affine_input_sum != 0;
    if (materialize) {
        const uint32_t gs = b.group_size;
        if (kr->w_dt != STARK_QMM_BF16 || kr->x_dt != STARK_QMM_BF16 || kr->d_dt != STARK_QMM_BF16 ||
            b.mode != STARK_QMM_MODE_U4 || b.correction != STARK_QMM_CORRECTION_BIASES || b.signed_codes ||
            !args->b_transpose || a8 || !(gs == 16 || gs == 32 || gs == 64 || gs == 128) || (k % 4) != 0)
            return STARK_QMM_UNSUPPORTED_LAYOUT;
    }
    if (a8) {
        // MatmulA::Int8Symmetric compatibility (kernel.rs:130-141)
        const uint32_t ag = args->a_scale_group_size, gs = b.group_size;
        if (!(ag == 32 || ag == 64 || ag == 128) || k % ag != 0 || !(gs == 32 || gs == 64 || gs == 128) ||
            !(b.mode == STARK_QMM_MODE_U4 || b.mode == STARK_QMM_MODE_U8))
            return STARK_QMM_INCOMPATIBLE_A;
    }
    AffineOp op;
    int bits;
    stark_qmm_status st = build_affine_op(kr, b, m, n, k, x, args->d, dops, args->gather_indices, &op, &bits);
    if (st != STARK_QMM_OK) return st;
    if (m == 0 || n == 0) return STARK_QMM_OK;
    if (a8) {
        if (!args->d || (k && (!args->a || !args->a_scales))) return STARK_QMM_INVALID_ARGUMENT;
        A8Operand q{(const int8_t*)args->a, args->a_scales, args->a_scale_group_size,
                    args->a_code_layout == STARK_QMM_CODES_GROUPED_BY_NIBBLE ? 1u : 0u};
        return launch_affine_a8(op, q, bits, stream);
    }
    if (!args->d || (!x && k)) return STARK_QMM_INVALID_ARGUMENT;
    if (materialize && m == 1) return launch_affine_materialized(op, stream);
    // Prefill-sized products run the dequant-GEMM (bf16-rounded weight tiles, as
    // the reference's Metal GEMM); the reference-accumulation mode keeps the
    // f32-dequant GEMV kernels for every M (kernel.rs:34-37, metal mod.rs:341-357).
    if (!kr->reference_accumulation && !materialize && bits == 4 && skinny_eligible(&op, 1))
        return launch_skinny(&op, 1, (op.flags & FLAG_SIGNED) != 0, stream);
    if (!kr->reference_accumulation && !materialize && gemm_eligible(op, bits))
        return launch_affine_gemm(op, bits, stream);
    if (affine_fast_eligible(op, bits)) return launch_affine_gemv(&op, 1, bits, stream);
    return launch_affine_generic(op, bits, stream);
}

// The int8-activation GEMM operands of args when the product takes that grid
// with the same validation as encode_product (else false: the entry then
// goes through stark_qmm_encode, which reports any error).
bool a8_gemm_entry(const stark_qmm_kernel* kr, const stark_qmm_args* a, AffineOp* op, A8Operand* q, int* bits) {
    const stark_qmm_b& b = a->b;
    if (a->a_kind != STARK_QMM_A_INT8_SYMMETRIC || a->a_code_layout > STARK_QMM_CODES_GROUPED_BY_NIBBLE || !b.codes ||
        a->d_ops.rht_factors || b.params.materialize_affine_input_sum || a->gather_indices || a->m <= 16 || a->n == 0)
        return false;
    const uint32_t ag = a->a_scale_group_size, gs = b.group_size;
    if (!(ag == 32 || ag == 64 || ag == 128) || a->k % ag != 0 || !(gs == 32 || gs == 64 || gs == 128) ||
        !(b.mode == STARK_QMM_MODE_U4 || b.mode == STARK_QMM_MODE_U8))
        return false;
    if (build_affine_op(kr, b, a->m, a->n, a->k, nullptr, a->d, a->d_ops, nullptr, op, bits) != STARK_QMM_OK)
        return false;
    if (!a->d || (a->k && (!a->a || !a->a_scales))) return false;
    *q = A8Operand{(const int8_t*)a->a, a->a_scales, a->a_scale_group_size,
                   a->a_code_layout == STARK_QMM_CODES_GROUPED_BY_NIBBLE ? 1u : 0u};
    return a8_gemm_eligible(*op, *q, *bits);
}

}  // namespace

extern "C" {

stark_qmm_status stark_qmm_encode(stark_qmm_kernel* kr, const stark_qmm_args* args, void* stream_ptr) {
    if (!kr || !args) return STARK_QMM_INVALID_ARGUMENT;
    if (args->struct_size != sizeof(stark_qmm_args)) return STARK_QMM_ABI_MISMATCH;
    hipStream_t stream = (hipStream_t)stream_ptr;
    stark_qmm_d_ops dops = args->d_ops;
    const int32_t* rht = (const int32_t*)args->d_ops.rht_factors;
    if (rht) {
        // Output RHT over each 32 outputs of a row, then the bias (kernel.rs:167, 287-300).
        if (kr->d_dt == STARK_QMM_F16 || args->n % 32 != 0) return STARK_QMM_UNSUPPORTED_D_OP;
        dops.bias = nullptr;
    }
    stark_qmm_status st = encode_product(kr, args, dops, stream);
    if (st != STARK_QMM_OK || !rht || args->m == 0 || args->n == 0) return st;
    return launch_output_rht(args->d, kr->d_dt, args->d_ops.bias, kr->w_dt, rht, args->m, args->n, stream);
}

stark_qmm_status stark_qmm_encode_many(stark_qmm_kernel* kr, const stark_qmm_args* args, uint32_t count,
                                       void* stream_ptr) {
    if (!kr || (!args && count)) return STARK_QMM_INVALID_ARGUMENT;
    hipStream_t stream = (hipStream_t)stream_ptr;
    std::vector<AffineOp> fast4, fast8;
    // prefill-sized products by (bits, signed codes, biases, bf16 planes): one grid each
    std::vector<AffineOp> gemm[2][2][2][2];
    std::vector<AffineOp> skinny[2];  // by signedness
    // int8-activation prefill products by grid class
    std::vector<AffineOp> a8_ops[16];
    std::vector<A8Operand> a8_as[16];
    std::vector<size_t> rest;
    const size_t xsz = kr->x_dt == STARK_QMM_F32 ? 4 : 2;
    for (uint32_t i = 0; i < count; ++i) {
        const stark_qmm_args* a = &args[i];
        if (a->struct_size != sizeof(stark_qmm_args)) return STARK_QMM_ABI_MISMATCH;
        {
            AffineOp op;
            A8Operand q;
            int bits;
            if (a8_gemm_entry(kr, a, &op, &q, &bits)) {
                const uint32_t c = a8_gemm_class(op, q, bits);
                a8_ops[c].push_back(op);
                a8_as[c].push_back(q);
                continue;
            }
        }
        if (a->d_ops.rht_factors || a->a_kind != STARK_QMM_A_FULL_PRECISION || !a->b.codes || a->b.params.materialize_affine_input_sum || a->m == 0 || a->n == 0) {
            rest.push_back(i);
            continue;
        }
        const void* x = a->a ? (const uint8_t*)a->a + a->a_offset * xsz : nullptr;
        AffineOp op;
        int bits;
        stark_qmm_status st = build_affine_op(kr, a->b, a->m, a->n, a->k, x, a->d, a->d_ops, a->gather_indices, &op, &bits);
        if (st != STARK_QMM_OK) return st;
        if (!a->d || (!x && a->k)) return STARK_QMM_INVALID_ARGUMENT;
        if (op.m > 16 && !kr->reference_accumulation && bits == 4 && skinny_eligible(&op, 1)) {
            skinny[(op.flags & FLAG_SIGNED) != 0].push_back(op);
        } else if (op.m > 16 && !kr->reference_accumulation && gemm_eligible(op, bits) && op.m <= gemm_rows(op.k)) {
            gemm[bits == 8][(op.flags & FLAG_SIGNED) != 0][op.corr_kind == STARK_QMM_CORRECTION_BIASES]
                [op.w_dt == STARK_QMM_BF16].push_back(op);
        } else if (!affine_fast_eligible(op, bits) || op.gather || (op.m > 16 && !kr->reference_accumulation)) {
            rest.push_back(i);
        } else if (bits == 4) {
            fast4.push_back(op);
        } else {
            fast8.push_back(op);
        }
    }
    // Group by M class so one launch never mixes one- and two-row kernels.
    for (auto* v : {&fast4, &fast8}) {
        const int bits = v == &fast4 ? 4 : 8;
        std::vector<AffineOp> one, many;
        for (const AffineOp& o : *v) (o.m == 1 ? one : many).push_back(o);
        stark_qmm_status st = launch_affine_gemv(one.data(), (uint32_t)one.size(), bits, stream);
        if (st != STARK_QMM_OK) return st;
        st = launch_affine_gemv(many.data(), (uint32_t)many.size(), bits, stream);
        if (st != STARK_QMM_OK) return st;
    }
    for (int sg = 0; sg < 2; ++sg)
        for (size_t s = 0; s < skinny[sg].size(); s += kMaxBatchOps) {
            const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, skinny[sg].size() - s);
            const stark_qmm_status st = launch_skinny(skinny[sg].data() + s, n, sg != 0, stream);
            if (st != STARK_QMM_OK) return st;
        }
    for (int b8 = 0; b8 < 2; ++b8)
        for (auto& a : gemm[b8])
            for (auto& c : a)
                for (auto& v : c)
                    for (size_t s = 0; s < v.size(); s += kMaxBatchOps) {
                        const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, v.size() - s);
                        const stark_qmm_status st = launch_affine_gemm_group(v.data() + s, n, b8 ? 8 : 4, stream);
                        if (st != STARK_QMM_OK) return st;
                    }
    for (uint32_t c = 0; c < 16; ++c)
        for (size_t s = 0; s < a8_ops[c].size(); s += kMaxBatchOps) {
            const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, a8_ops[c].size() - s);
            const stark_qmm_status st =
                launch_affine_a8_gemm_group(a8_ops[c].data() + s, a8_as[c].data() + s, n, (c & 8) ? 8 : 4, stream);
            if (st != STARK_QMM_OK) return st;
        }
    for (size_t i : rest) {
        stark_qmm_status st = stark_qmm_encode(kr, &args[i], stream_ptr);
        if (st != STARK_QMM_OK) return st;
    }
    return STARK_QMM_OK;
}


stark_qmm_status stark_qmm_encode_many_prologue(stark_qmm_kernel* kr, const stark_qmm_args* args, uint32_t count,
                                                const stark_qmm_prologue* pro, void* stream_ptr) {
    if (!kr || !pro || (!args && count)) return STARK_QMM_INVALID_ARGUMENT;
    if (pro->struct_size != sizeof(stark_qmm_prologue)) return STARK_QMM_ABI_MISMATCH;
    if (pro->kind != STARK_QMM_PROLOGUE_RMS_NORM && pro->kind != STARK_QMM_PROLOGUE_SILU_GATE)
        return STARK_QMM_UNSUPPORTED;
    if (!pro->data || ((uintptr_t)pro->data & 15)) return STARK_QMM_INVALID_ARGUMENT;
    if (kr->reference_accumulation || kr->x_dt != STARK_QMM_BF16 || count > (uint32_t)kMaxBatchOps)
        return STARK_QMM_UNSUPPORTED;
    std::vector<AffineOp> ops;
    for (uint32_t i = 0; i < count; ++i) {
        const stark_qmm_args* a = &args[i];
        if (a->struct_size != sizeof(stark_qmm_args)) return STARK_QMM_ABI_MISMATCH;
        if (a->d_ops.rht_factors || a->a_kind != STARK_QMM_A_FULL_PRECISION || !a->b.codes ||
            a->b.params.materialize_affine_input_sum || a->gather_indices || a->m != 1 ||
            a->b.mode != STARK_QMM_MODE_U4 || a->a != args[0].a || a->a_offset != args[0].a_offset ||
            a->k != args[0].k)
            return STARK_QMM_UNSUPPORTED;
        const void* x = a->a ? (const uint8_t*)a->a + a->a_offset * 2 : nullptr;
        if (!x || !a->d) return STARK_QMM_INVALID_ARGUMENT;
        AffineOp op;
        int bits;
        const stark_qmm_status st =
            build_affine_op(kr, a->b, a->m, a->n, a->k, x, a->d, a->d_ops, nullptr, &op, &bits);
        if (st != STARK_QMM_OK) return st;
        if (a->n == 0) continue;
        ops.push_back(op);
    }
    const StreamPrologue p{pro->kind, pro->data, pro->eps};
    return launch_stream_prologue(ops.data(), (uint32_t)ops.size(), p, (hipStream_t)stream_ptr);
}

}  // extern "C"


// Chained products (stream_common.h, qmv_chain.hip): validation, K slices and
// the workspace layout -- a 256-byte status header, then for each product of
// k_slices > 1 (in order) (k_slices - 1) x N 64-bit partial words.
static stark_qmm_status chain_validate(const stark_qmm_chain_product* p, uint32_t count, uint64_t* bytes) {
    if (!p && count) return STARK_QMM_INVALID_ARGUMENT;
    uint64_t need = 256;
    uint32_t lists = 0, stage = 0;
    for (uint32_t i = 0; i < count; ++i) {
        if (p[i].struct_size != sizeof(stark_qmm_chain_product)) return STARK_QMM_ABI_MISMATCH;
        const stark_qmm_args* a = p[i].args;
        if (!a) return STARK_QMM_INVALID_ARGUMENT;
        if (a->struct_size != sizeof(stark_qmm_args)) return STARK_QMM_ABI_MISMATCH;
        if (i && p[i].stage < stage) return STARK_QMM_INVALID_ARGUMENT;  // stages in increasing order
        stage = p[i].stage;
        const uint32_t sl = p[i].k_slices ? p[i].k_slices : 1;
        if (a->a_kind != STARK_QMM_A_FULL_PRECISION || !a->b.codes || a->m != 1 || a->b.mode != STARK_QMM_MODE_U4 ||
            a->b.group_size != 64 || a->k == 0 || a->k % 4096 || a->n == 0 || a->n % 32 || a->gather_indices ||
            a->d_ops.bias || a->d_ops.rht_factors || a->d_ops.has_soft_cap || a->b.params.materialize_affine_input_sum ||
            a->b.correction != STARK_QMM_CORRECTION_BIASES || (a->k / 4096) % sl || p[i].in_tag > 0x7fff ||
            p[i].out_tag > 0x7fff || p[i].acc_tag > 0x7fff || p[i].part_tag > 0x7fff || (sl > 1 && !p[i].part_tag) ||
            (p[i].acc_tag && !p[i].out_tag) || p[i].prologue > STARK_QMM_PROLOGUE_SILU_GATE ||
            (p[i].prologue == STARK_QMM_PROLOGUE_RMS_NORM && a->k != 4096))
            return STARK_QMM_UNSUPPORTED;
        if (!a->a || !a->d || (p[i].prologue && (!p[i].prologue_data || ((uintptr_t)p[i].prologue_data & 15))))
            return STARK_QMM_INVALID_ARGUMENT;
        lists += sl;
        if (sl > 1) need += (uint64_t)(sl - 1) * a->n * 8;
    }
    if (lists > (uint32_t)kMaxChainOps) return STARK_QMM_UNSUPPORTED;
    *bytes = need;
    return STARK_QMM_OK;
}

extern "C" {

stark_qmm_status stark_qmm_chain_workspace_size(const stark_qmm_chain_product* products, uint32_t count,
                                               uint64_t* bytes) {
    if (!bytes) return STARK_QMM_INVALID_ARGUMENT;
    return chain_validate(products, count, bytes);
}

stark_qmm_status stark_qmm_encode_chain(stark_qmm_kernel* kr, const stark_qmm_chain_product* p, uint32_t count,
                                        const uint32_t* seq, void* workspace, uint64_t workspace_bytes,
                                        void* stream_ptr) {
    if (!kr) return STARK_QMM_INVALID_ARGUMENT;
    if (kr->reference_accumulation || kr->x_dt != STARK_QMM_BF16 || kr->d_dt != STARK_QMM_BF16 ||
        kr->w_dt != STARK_QMM_BF16)
        return STARK_QMM_UNSUPPORTED;
    uint64_t need = 0;
    const stark_qmm_status vs = chain_validate(p, count, &need);
    if (vs != STARK_QMM_OK) return vs;
    if (!workspace || ((uintptr_t)workspace & 255)) return STARK_QMM_INVALID_ARGUMENT;
    if (workspace_bytes < need) return STARK_QMM_WORKSPACE_TOO_SMALL;
    std::vector<ChainOp> ops;
    uint64_t* part = (uint64_t*)((uint8_t*)workspace + 256);
    for (uint32_t i = 0; i < count; ++i) {
        const stark_qmm_args* a = p[i].args;
        const uint32_t esz = p[i].in_tag ? 4 : 2;
        const void* x = (const uint8_t*)a->a + a->a_offset * esz;
        AffineOp op;
        int bits;
        const stark_qmm_status st = build_affine_op(kr, a->b, 1, a->n, a->k, x, a->d, a->d_ops, nullptr, &op, &bits);
        if (st != STARK_QMM_OK) return st;
        if ((((uintptr_t)op.codes | (uintptr_t)x | (uintptr_t)op.scales | (uintptr_t)op.corr) & 15) ||
            (op.os == 1 ? op.gs % 8 : op.os % 8))
            return STARK_QMM_UNSUPPORTED;
        const uint32_t sl = p[i].k_slices ? p[i].k_slices : 1, ks = a->k / sl;
        for (uint32_t j = 0; j < sl; ++j) {
            ChainOp c{};
            const size_t g0 = (size_t)j * (ks / 64);  // first group of the slice
            const size_t poff = op.os == 1 ? g0 * op.gs : g0;
            c.codes = op.codes + (size_t)j * (ks / 2);
            c.scales = (const uint16_t*)op.scales + poff;
            c.corr = (const uint16_t*)op.corr + poff;
            c.x = (const uint8_t*)x + (size_t)j * ks * esz;
            c.d = a->d;
            c.pro = p[i].prologue;
            c.pro_data = p[i].prologue == STARK_QMM_PROLOGUE_SILU_GATE
                             ? (const void*)((const uint8_t*)p[i].prologue_data + (size_t)j * ks * esz)
                             : p[i].prologue_data;
            c.eps = p[i].eps;
            c.n = a->n;
            c.k = ks;
            c.ldc = a->k / 2;
            c.os = op.os;
            c.gs = op.gs;
            c.ab_scale = op.ab_scale;
            c.in_tag = p[i].in_tag;
            c.out_tag = p[i].out_tag;
            c.acc_tag = p[i].acc_tag;
            c.part_tag = p[i].part_tag;
            c.flags = op.flags & (FLAG_ACCUMULATE | FLAG_SIGNED);
            c.order = 2 * p[i].stage;
            if (sl == 1) {
                c.out = p[i].out_tag ? CHAIN_OUT_TAGGED : CHAIN_OUT_PLAIN;
            } else if (j + 1 < sl) {
                c.out = CHAIN_OUT_PARTIAL;
                c.part = part + (size_t)j * a->n;
            } else {
                c.out = CHAIN_OUT_COMBINE;
                c.part = part;
                c.nparts = sl - 1;
                c.order = 2 * p[i].stage + 1;  // after the other slices in every list
            }
            ops.push_back(c);
        }
        if (sl > 1) part += (size_t)(sl - 1) * a->n;
    }
    return launch_chain(ops.data(), (uint32_t)ops.size(), seq, (uint32_t*)workspace, (hipStream_t)stream_ptr);
}

}  // extern "C"
