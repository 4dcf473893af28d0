// The BF16-effective affine reference dot (ReferenceAffineBF16Matmul,
// crates/stark-engine/src/encodable_block/linear/reference_affine.rs:105-280;
// kernel reference_affine_linear_bf16,
// crates/stark-engine/src/backends/cpu/kernel/matmul/vision.rs:249-336), bit for
// bit:
//   w = bf16_rne(f32(code) * scale + bias)       (dense bf16 weights when bits == 0)
//   32 partial sums p[r][l] (r < 8, l < 4) each take inner = start + 4r + l
//   for start = 0, 32, .. in order, by fma(x, w, p);
//   p[r] += p[r + o] for o = 4, 2, 1; result = bf16((p00 + p01) + (p02 + p03)).
// On gfx950 the 32 partial sums are the 32 lanes of a half-wave (lane = 4r + l),
// so each lane runs its own sum in the reference's order, and the tree is three
// cross-lane adds within the half-wave followed by the final pairwise add: the
// same IEEE operations on the same operands, hence the same bits. A half-wave
// owns one weight row; for the plain form it reuses each decoded chunk for
// kRows activation rows at a time. Gathered rows come from `indices` per
// output; a row outside the bank gives NaN (vision.rs:292-297).
#include "qmm_common.h"

#pragma clang fp contract(off)

namespace qmm {
namespace {

constexpr int kHalfWaves = 8;  // 256 threads
constexpr int kRows = 4;       // activation rows per pass (plain form)

struct RefArgs {
    const uint16_t* input;    // [M, K] bf16
    const uint8_t* weights;   // packed codes, or bf16 [bank, K] when bits == 0
    const uint16_t* scales;
    const uint16_t* biases;
    const uint32_t* indices;  // [M*N] or NULL
    void* out;
    uint32_t m, n, k, bank_rows, bits, sos, sgs, f32_out;
};

__device__ __forceinline__ float weight_value(const RefArgs& a, size_t row, uint32_t inner) {
    if (a.bits == 0) return bf16_bits_to_f32(((const uint16_t*)a.weights)[row * a.k + inner]);
    const size_t bit = (size_t)inner * a.bits;
    const uint32_t shift = (uint32_t)(bit % 8);
    const size_t off = row * ((size_t)a.k * a.bits / 8) + bit / 8;
    uint32_t packed = a.weights[off];
    if (shift + a.bits > 8) packed |= (uint32_t)a.weights[off + 1] << 8;
    const uint32_t code = (packed >> shift) & ((1u << a.bits) - 1u);
    const size_t g = row * a.sos + (size_t)(inner / 64) * a.sgs;
    const float v = (float)code * bf16_bits_to_f32(a.scales[g]) + bf16_bits_to_f32(a.biases[g]);
    return bf16_bits_to_f32(f32_to_bf16_bits(v));
}

// The reference's tree over the half-wave; lane 0 of the half returns the sum.
__device__ __forceinline__ float tree(float v) {
    v += __shfl_down(v, 16, 32);
    v += __shfl_down(v, 8, 32);
    v += __shfl_down(v, 4, 32);
    const float pair = v + __shfl_down(v, 1, 32);  // lane 0: p00 + p01, lane 2: p02 + p03
    return pair + __shfl_down(pair, 2, 32);
}

__device__ __forceinline__ void store(const RefArgs& a, size_t o, float v) {
    const uint16_t h = f32_to_bf16_bits(v);
    if (a.f32_out)
        ((float*)a.out)[o] = bf16_bits_to_f32(h);
    else
        ((uint16_t*)a.out)[o] = h;
}

__global__ __launch_bounds__(256) void ref_affine_plain(RefArgs a) {
    const uint32_t lane = threadIdx.x & 31;
    const uint32_t column = blockIdx.x * kHalfWaves + (threadIdx.x >> 5);
    const uint32_t m0 = blockIdx.y * kRows;
    if (column >= a.n) return;  // uniform over the half-wave
    const uint32_t rows = min((uint32_t)kRows, a.m - m0);
    float p[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) p[r] = 0.0f;
    for (uint32_t start = 0; start < a.k; start += 32) {
        const uint32_t inner = start + lane;
        const float w = weight_value(a, column, inner);
#pragma unroll
        for (int r = 0; r < kRows; ++r)
            if ((uint32_t)r < rows) p[r] = fmaf(bf16_bits_to_f32(a.input[(size_t)(m0 + r) * a.k + inner]), w, p[r]);
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        if ((uint32_t)r >= rows) break;
        const float v = tree(p[r]);
        if (lane == 0) store(a, (size_t)(m0 + r) * a.n + column, v);
    }
}

__global__ __launch_bounds__(256) void ref_affine_gathered(RefArgs a) {
    const uint32_t lane = threadIdx.x & 31;
    const size_t item = (size_t)blockIdx.x * kHalfWaves + (threadIdx.x >> 5);
    if (item >= (size_t)a.m * a.n) return;
    const size_t row = item / a.n;
    const uint32_t source = a.indices[item];
    if (source >= a.bank_rows) {
        if (lane == 0) store(a, item, __int_as_float(0x7fc00000));
        return;
    }
    float p = 0.0f;
    for (uint32_t start = 0; start < a.k; start += 32) {
        const uint32_t inner = start + lane;
        p = fmaf(bf16_bits_to_f32(a.input[row * a.k + inner]), weight_value(a, source, inner), p);
    }
    const float v = tree(p);
    if (lane == 0) store(a, item, v);
}

int mode_bits_ref(uint32_t mode) {
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

// ReferenceAffinePlan::with_limits (reference_affine.rs:55-96) with the
// production limits.
bool plan_ok(uint32_t m, uint32_t n, uint32_t k) {
    constexpr uint64_t per_dispatch = 1ull << 30, total = 1ull << 38, max_dispatches = 1024;
    const uint64_t outputs = (uint64_t)m * n, terms = outputs * k;
    if (m == 0 || m > 32768 || n == 0 || n > 1048576 || k == 0 || k > 131072 || k % 32 || outputs > (64ull << 20) ||
        terms > total || k > per_dispatch)
        return false;
    const uint64_t tile = std::min<uint64_t>(per_dispatch / k, 65536);
    const uint64_t tile_columns = std::min<uint64_t>(n, tile);
    const uint64_t tile_rows = std::min<uint64_t>(m, tile / tile_columns);
    const uint64_t dispatches = ((m + tile_rows - 1) / tile_rows) * ((n + tile_columns - 1) / tile_columns);
    return dispatches != 0 && dispatches <= max_dispatches;
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

stark_qmm_status stark_qmm_reference_affine_bf16(const stark_qmm_reference_affine_args* args, void* stream) {
    if (!args) return STARK_QMM_INVALID_ARGUMENT;
    if (args->struct_size != sizeof(stark_qmm_reference_affine_args)) return STARK_QMM_ABI_MISMATCH;
    const stark_qmm_reference_affine_args& x = *args;
    // ReferenceAffineBF16Matmul::new: BF16 or widened-BF16 (F32) output
    if (x.output_dtype != STARK_QMM_BF16 && x.output_dtype != STARK_QMM_F32) return STARK_QMM_UNSUPPORTED_DATA_TYPE;
    const uint32_t m = x.m, n = x.n, k = x.k;
    if (!plan_ok(m, n, k)) return STARK_QMM_INVALID_ARGUMENT;
    const stark_qmm_b& b = x.weights;
    RefArgs a{};
    uint64_t weight_bytes;
    uint32_t bits = 0;
    if (!b.codes) {
        a.weights = (const uint8_t*)b.values;
        weight_bytes = x.values_size;
    } else {
        // explicit source policies keep their own route (reference_affine.rs:20-25, 130-132)
        if (b.params.materialize_affine_input_sum || x.source_output_width_count) return STARK_QMM_UNSUPPORTED_LAYOUT;
        const int mb = mode_bits_ref(b.mode);
        if (b.group_size != 64 || b.signed_codes || !(mb == 4 || mb == 5 || mb == 6 || mb == 8) || k % 64 ||
            b.correction != STARK_QMM_CORRECTION_BIASES || !b.correction_data || !b.scales)
            return STARK_QMM_INVALID_ARGUMENT;
        bits = (uint32_t)mb;
        const uint64_t row_bytes = (uint64_t)k * bits / 8;
        if (b.codes_size == 0 || b.codes_size % row_bytes) return STARK_QMM_INVALID_ARGUMENT;
        const uint64_t rows = b.codes_size / row_bytes;
        if (rows > (1u << 28)) return STARK_QMM_INVALID_ARGUMENT;
        // QuantParams::new(layout, rows, k / 64).scale_shape() must equal the given params' shape
        auto shape = [](uint32_t layout, uint64_t r, uint64_t g, uint64_t* s0, uint64_t* s1) {
            if (layout == STARK_QMM_LAYOUT_OUTPUT_GROUP) {
                *s0 = r;
                *s1 = g;
            } else {
                *s0 = g;
                *s1 = (r + 3) / 4 * 4;
            }
        };
        if (b.params.layout > STARK_QMM_LAYOUT_GROUP_OUTPUT) return STARK_QMM_INVALID_ARGUMENT;
        uint64_t e0, e1, g0, g1;
        shape(b.params.layout, rows, k / 64, &e0, &e1);
        shape(b.params.layout, b.params.row_count, b.params.group_count, &g0, &g1);
        if (e0 != g0 || e1 != g1) return STARK_QMM_INVALID_ARGUMENT;
        a.weights = (const uint8_t*)b.codes;
        weight_bytes = b.codes_size;
        if (b.params.layout == STARK_QMM_LAYOUT_OUTPUT_GROUP) {
            a.sos = b.params.group_count;
            a.sgs = 1;
        } else {
            a.sos = 1;
            a.sgs = (b.params.row_count + 3) / 4 * 4;
        }
    }
    const uint64_t row_bytes = bits == 0 ? (uint64_t)k * 2 : (uint64_t)k * bits / 8;
    if (!a.weights || weight_bytes == 0 || weight_bytes % row_bytes) return STARK_QMM_INVALID_ARGUMENT;
    const uint64_t bank_rows = weight_bytes / row_bytes;
    if (bank_rows > (1u << 28)) return STARK_QMM_INVALID_ARGUMENT;
    // input / index extents and alignment (reference_affine.rs:190-205)
    const uint64_t input_bytes = (uint64_t)m * k * 2, outputs = (uint64_t)m * n;
    const uintptr_t input_start = (uintptr_t)x.input + x.input_offset;
    if (!x.input || input_start % 2 || (bits == 0 && (uintptr_t)a.weights % 2) ||
        (bits != 0 && (((uintptr_t)b.scales % 2) || ((uintptr_t)b.correction_data % 2))) ||
        x.input_offset + input_bytes > x.input_size ||
        (x.indices && (x.indices_size < outputs * 4 || (uintptr_t)x.indices % 4)) || (!x.indices && n > bank_rows))
        return STARK_QMM_INVALID_ARGUMENT;
    if (bits != 0) {
        const uint64_t end = ((bank_rows - 1) * a.sos + (uint64_t)(k / 64 - 1) * a.sgs + 1) * 2;
        if (end > x.scales_size || end > x.biases_size) return STARK_QMM_INVALID_ARGUMENT;
    }
    if (!x.output || (uintptr_t)x.output % (x.output_dtype == STARK_QMM_F32 ? 4 : 2)) return STARK_QMM_INVALID_ARGUMENT;
    a.input = (const uint16_t*)input_start;
    a.scales = (const uint16_t*)b.scales;
    a.biases = (const uint16_t*)b.correction_data;
    a.indices = x.indices;
    a.out = x.output;
    a.m = m;
    a.n = n;
    a.k = k;
    a.bank_rows = (uint32_t)bank_rows;
    a.bits = bits;
    a.f32_out = x.output_dtype == STARK_QMM_F32;
    hipStream_t s = (hipStream_t)stream;
    if (x.indices) {
        hipLaunchKernelGGL(ref_affine_gathered, dim3((unsigned)((outputs + kHalfWaves - 1) / kHalfWaves)), dim3(256), 0,
                           s, a);
    } else {
        hipLaunchKernelGGL(ref_affine_plain, dim3((n + kHalfWaves - 1) / kHalfWaves, (m + kRows - 1) / kRows),
                           dim3(256), 0, s, a);
    }
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // extern "C"
