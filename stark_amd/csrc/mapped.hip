// Hybrid-engine matrix operations: weight_metal::mapped_many
// (crates/stark-engine/src/engine/hybrid/weight_metal.rs:376-545).
//
// Validation follows MappedOperation::parameters_for_input (weight_metal.rs:442-537)
// line for line so that the same descriptors are accepted and rejected. Execution
// turns every (matrix, input batch) pair into a matvec op; views of the same
// matrix with several inputs become one op with M > 1 so the weights stream once.
#include <mutex>
#include <vector>

#include "qmm_common.h"

namespace qmm {

namespace {

// engine/hybrid/weights.rs:2565-2584
bool block_layout(uint32_t kind, uint64_t* elements, uint64_t* bytes) {
    switch (kind) {
    case 0: *elements = 1; *bytes = 4; return true;
    case 1: case 30: *elements = 1; *bytes = 2; return true;
    case 8: *elements = 32; *bytes = 34; return true;
    case 10: *elements = 256; *bytes = 84; return true;
    case 11: *elements = 256; *bytes = 110; return true;
    case 12: *elements = 256; *bytes = 144; return true;
    case 13: *elements = 256; *bytes = 176; return true;
    case 14: *elements = 256; *bytes = 210; return true;
    case 16: *elements = 256; *bytes = 66; return true;
    case 17: *elements = 256; *bytes = 74; return true;
    case 18: *elements = 256; *bytes = 98; return true;
    case 23: *elements = 256; *bytes = 136; return true;
    default: return false;
    }
}

constexpr uint64_t kMaxDim = 8000000;

stark_qmm_status validate(const stark_qmm_mapped_op& op) {
    if (!op.matrices && op.matrix_count) return STARK_QMM_INVALID_ARGUMENT;
    const uint64_t rows = op.rows, columns = op.columns;
    uint64_t batches;
    if (op.rows_per_batch == 0) {
        batches = op.matrix_count;
    } else {
        if (op.matrix_count != 1 || rows % op.rows_per_batch) return STARK_QMM_INVALID_ARGUMENT;
        batches = rows / op.rows_per_batch;
    }
    if (rows == 0 || columns == 0 || rows > kMaxDim || columns > kMaxDim || op.matrix_count == 0 ||
        (uint64_t)op.matrix_count * rows > kMaxDim || batches * columns != op.input_length ||
        op.input_length > kMaxDim)
        return STARK_QMM_INVALID_ARGUMENT;
    uint64_t matrix_bytes, plane_bytes;
    if (op.format == STARK_QMM_FORMAT_PACKED) {
        uint64_t block, bytes;
        if (!block_layout(op.packed_kind, &block, &bytes)) return STARK_QMM_UNSUPPORTED;
        if (columns % block) return STARK_QMM_INVALID_ARGUMENT;
        matrix_bytes = rows * (columns / block) * bytes;
        plane_bytes = 0;
    } else if (op.format == STARK_QMM_FORMAT_AFFINE) {
        uint64_t item;
        if (op.scale_dtype == STARK_QMM_F32) item = 4;
        else if (op.scale_dtype == STARK_QMM_F16 || op.scale_dtype == STARK_QMM_BF16) item = 2;
        else return STARK_QMM_INVALID_ARGUMENT;
        if (!(op.bits == 4 || op.bits == 8) || !(op.group == 32 || op.group == 64 || op.group == 128) ||
            columns % op.group)
            return STARK_QMM_INVALID_ARGUMENT;
        matrix_bytes = rows * columns * op.bits / 8;
        plane_bytes = rows * (columns / op.group) * item;
    } else {
        return STARK_QMM_INVALID_ARGUMENT;
    }
    for (uint32_t i = 0; i < op.matrix_count; ++i) {
        const stark_qmm_mapped_matrix& mm = op.matrices[i];
        const bool has_planes = mm.scales || mm.biases;
        if (mm.codes_length != matrix_bytes || !mm.codes) return STARK_QMM_INVALID_ARGUMENT;
        if (!has_planes) {
            if (plane_bytes != 0) return STARK_QMM_INVALID_ARGUMENT;
        } else if (plane_bytes == 0 || mm.plane_length != plane_bytes || !mm.scales || !mm.biases) {
            return STARK_QMM_INVALID_ARGUMENT;
        }
    }
    if (!op.inputs) return STARK_QMM_INVALID_ARGUMENT;
    return STARK_QMM_OK;
}

__global__ void finite_check_kernel(const float* x, uint64_t n, uint32_t* status) {
    bool bad = false;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        bad |= !isfinite(x[i]);
    if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(status, 1u);
}

__global__ void zero_word_kernel(uint32_t* w) { *w = 0; }

}  // namespace

stark_qmm_status launch_finite_check(const float* x, uint64_t n, uint32_t* status, hipStream_t stream) {
    hipLaunchKernelGGL(finite_check_kernel, dim3(64), dim3(256), 0, stream, x, n, status);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

namespace {

// Build the matvec ops for one mapped operation.
void expand(const stark_qmm_mapped_op& op, float* out, std::vector<AffineOp>* affine4,
            std::vector<AffineOp>* affine8, std::vector<GgufOp>* gguf) {
    const uint64_t rows = op.rows, cols = op.columns;
    auto add = [&](const uint8_t* codes, const void* scales, const void* biases, const float* x, float* d,
                   uint32_t n, uint32_t m) {
        if (op.format == STARK_QMM_FORMAT_AFFINE) {
            AffineOp o{};
            o.codes = codes;
            o.scales = scales;
            o.corr = biases;
            o.corr_kind = STARK_QMM_CORRECTION_BIASES;
            o.x = x;
            o.d = d;
            o.n = n;
            o.k = (uint32_t)cols;
            o.m = m;
            o.os = (uint32_t)(cols / op.group);
            o.gs = 1;
            o.group_size = op.group;
            o.w_dt = op.scale_dtype;
            o.x_dt = STARK_QMM_F32;
            o.d_dt = STARK_QMM_F32;
            o.ab_scale = 1.0f;
            o.bank_rows = n;
            (op.bits == 4 ? affine4 : affine8)->push_back(o);
        } else {
            GgufOp g{};
            g.blocks = codes;
            g.kind = op.packed_kind;
            g.x = x;
            g.d = d;
            g.n = n;
            g.k = (uint32_t)cols;
            g.m = m;
            gguf->push_back(g);
        }
    };
    uint64_t row_bytes, plane_row_bytes = 0;
    if (op.format == STARK_QMM_FORMAT_AFFINE) {
        row_bytes = cols * op.bits / 8;
        plane_row_bytes = (cols / op.group) * (op.scale_dtype == STARK_QMM_F32 ? 4 : 2);
    } else {
        uint64_t block, bytes;
        block_layout(op.packed_kind, &block, &bytes);
        row_bytes = cols / block * bytes;
    }
    if (op.rows_per_batch) {
        const stark_qmm_mapped_matrix& mm = op.matrices[0];
        const uint64_t rpb = op.rows_per_batch;
        for (uint64_t b = 0; b < rows / rpb; ++b)
            add((const uint8_t*)mm.codes + b * rpb * row_bytes,
                mm.scales ? (const uint8_t*)mm.scales + b * rpb * plane_row_bytes : nullptr,
                mm.biases ? (const uint8_t*)mm.biases + b * rpb * plane_row_bytes : nullptr, op.inputs + b * cols,
                out + b * rpb, (uint32_t)rpb, 1);
        return;
    }
    // views of one matrix with consecutive inputs -> one op with M rows
    uint32_t j = 0;
    while (j < op.matrix_count) {
        uint32_t e = j + 1;
        while (e < op.matrix_count && op.matrices[e].codes == op.matrices[j].codes &&
               op.matrices[e].scales == op.matrices[j].scales && op.matrices[e].biases == op.matrices[j].biases)
            ++e;
        const stark_qmm_mapped_matrix& mm = op.matrices[j];
        add((const uint8_t*)mm.codes, mm.scales, mm.biases, op.inputs + (uint64_t)j * cols, out + (uint64_t)j * rows,
            (uint32_t)rows, e - j);
        j = e;
    }
}

// Status word of the synchronous form, one per device. The whole synchronous
// call (zero, launches, wait, read) holds the device's lock, so concurrent
// callers on different streams never share a word in flight.
struct SyncWord {
    std::mutex mu;
    uint32_t* word = nullptr;
};

SyncWord* sync_word(int dev) {
    static SyncWord words[64];
    return dev >= 0 && dev < 64 ? &words[dev] : nullptr;
}

stark_qmm_status run(const stark_qmm_mapped_op* ops, uint32_t count, float* const* outputs, uint32_t* status,
                     hipStream_t stream) {
    if (!ops || !outputs || count == 0 || count > 64) return STARK_QMM_INVALID_ARGUMENT;
    for (uint32_t i = 0; i < count; ++i) {
        stark_qmm_status st = validate(ops[i]);
        if (st != STARK_QMM_OK) return st;
        if (!outputs[i]) return STARK_QMM_INVALID_ARGUMENT;
        if (ops[i].format == STARK_QMM_FORMAT_PACKED && !gguf_supported(ops[i].packed_kind))
            return STARK_QMM_UNSUPPORTED;
    }
    // input finite check (weight_metal.rs:435-440); the GGUF kernels check
    // the activations they stage themselves
    for (uint32_t i = 0; i < count; ++i) {
        if (ops[i].format == STARK_QMM_FORMAT_PACKED) continue;
        stark_qmm_status st = launch_finite_check(ops[i].inputs, ops[i].input_length, status, stream);
        if (st != STARK_QMM_OK) return st;
    }
    std::vector<AffineOp> a4, a8;
    std::vector<GgufOp> gg;
    for (uint32_t i = 0; i < count; ++i) expand(ops[i], outputs[i], &a4, &a8, &gg);
    for (int bits : {4, 8}) {
        std::vector<AffineOp>& v = bits == 4 ? a4 : a8;
        std::vector<AffineOp> fast;
        for (const AffineOp& o : v) {
            if (affine_fast_eligible(o, bits)) {
                fast.push_back(o);
            } else {
                stark_qmm_status st = launch_affine_generic(o, bits, stream);
                if (st != STARK_QMM_OK) return st;
            }
        }
        std::vector<AffineOp> one, many;
        for (const AffineOp& o : fast) (o.m == 1 ? one : many).push_back(o);
        stark_qmm_status st = launch_affine_gemv(one.data(), (uint32_t)one.size(), bits, stream);
        if (st != STARK_QMM_OK) return st;
        st = launch_affine_gemv(many.data(), (uint32_t)many.size(), bits, stream);
        if (st != STARK_QMM_OK) return st;
    }
    return launch_gguf_gemv(gg.data(), (uint32_t)gg.size(), status, stream);
}

}  // namespace

}  // namespace qmm

using namespace qmm;

extern "C" {

stark_qmm_status stark_qmm_mapped_many_async(const stark_qmm_mapped_op* ops, uint32_t count, float* const* outputs,
                                             uint32_t* status_word, void* stream) {
    if (!status_word) return STARK_QMM_INVALID_ARGUMENT;
    return run(ops, count, outputs, status_word, (hipStream_t)stream);
}

stark_qmm_status stark_qmm_mapped_many(const stark_qmm_mapped_op* ops, uint32_t count, float* const* outputs,
                                       void* stream_ptr) {
    hipStream_t stream = (hipStream_t)stream_ptr;
    int dev = 0;
    QMM_HIP_CHECK(hipGetDevice(&dev));
    SyncWord* sw = sync_word(dev);
    if (!sw) return STARK_QMM_DEVICE_FAILURE;
    std::lock_guard<std::mutex> hold(sw->mu);
    if (!sw->word) {
        void* p = nullptr;
        QMM_HIP_CHECK(hipMalloc(&p, 256));
        sw->word = (uint32_t*)p;
    }
    uint32_t* word = sw->word;
    hipLaunchKernelGGL(zero_word_kernel, dim3(1), dim3(1), 0, stream, word);
    QMM_HIP_CHECK(hipGetLastError());
    stark_qmm_status st = run(ops, count, outputs, word, stream);
    QMM_HIP_CHECK(hipStreamSynchronize(stream));
    if (st != STARK_QMM_OK) return st;
    uint32_t host = 0;
    QMM_HIP_CHECK(hipMemcpy(&host, word, sizeof(host), hipMemcpyDeviceToHost));
    return host ? STARK_QMM_INVALID_ARGUMENT : STARK_QMM_OK;
}

}  // extern "C"
