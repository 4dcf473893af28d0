// MoE routing kernels (reference: crates/stark-engine/src/backends/cpu/kernel/moe.rs and
// crates/stark-engine/src/backends/metal/kernel/moe.metal).
#include "qmm_common.h"

namespace qmm {

namespace {

QMM_DEVICE float round_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// MoeRoute (moe.rs:23-85): one wave per token row, experts striped over lanes.
// Top-k is a repeated argmax where a strictly greater value wins and ties go to
// the lowest expert id (moe.rs:61-66). The softmax denominator is a wave
// reduction and exp is the device expf (the reference sums sequentially with
// the platform's libm exp): ids are exact, weights agree to a few ulp.
__global__ __launch_bounds__(64) void moe_route_kernel(const float* logits, uint32_t* ids, float* weights,
                                                        uint32_t rows, uint32_t experts, uint32_t active,
                                                        uint32_t round_weights, uint32_t round_logits) {
    const uint32_t row = blockIdx.x;
    const int lane = threadIdx.x;
    if (row >= rows) return;
    constexpr int kMaxPerLane = 1024 / 64;
    float x[kMaxPerLane];
    uint32_t used = 0;  // bit j: expert lane + 64*j already selected
    bool valid = experts >= 1 && experts <= 1024 && active >= 1 && active <= 32 && active <= experts;
    const uint32_t E = experts > 1024 ? 1024 : experts;
    float mx = -INFINITY;
    bool finite = true;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j) {
        const uint32_t e = lane + 64 * j;
        float v = -INFINITY;
        if (e < E) {
            v = logits[(size_t)row * experts + e];
            if (round_logits) v = round_bf16(v);
            finite = finite && isfinite(v);
            mx = fmaxf(mx, v);
        } else {
            used |= 1u << j;
        }
        x[j] = v;
    }
    valid = valid && __all(finite) && experts <= 1024;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    float den = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxPerLane; ++j)
        if (lane + 64 * j < E) den += expf(x[j] - mx);
    den = wave_sum(den);
    float selected_sum = 0.0f;
    float w_rank = 0.0f;  // lane r keeps the weight of rank r
    for (uint32_t rank = 0; rank < active && rank < 32; ++rank) {
        float best = -INFINITY;
        uint32_t sel = 0xffffffffu;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j) {
            if (!(used & (1u << j)) && x[j] > best) {
                best = x[j];
                sel = lane + 64 * j;
            }
        }
        // wave argmax: larger value wins; equal values -> lower id
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            float ob = __shfl_xor(best, off, 64);
            uint32_t os = __shfl_xor(sel, off, 64);
            if (ob > best || (ob == best && os < sel)) {
                best = ob;
                sel = os;
            }
        }
        // nothing left that is > -inf: the reference keeps expert 0
        const uint32_t chosen = sel == 0xffffffffu ? 0u : sel;
        if (sel != 0xffffffffu && (sel & 63u) == (uint32_t)lane) used |= 1u << (sel >> 6);
        const float score = expf(best - mx) / den;
        selected_sum += score;
        if ((uint32_t)lane == rank) w_rank = score;
        if (lane == 0) ids[(size_t)row * active + rank] = valid ? chosen : 0u;
    }
    if ((uint32_t)lane < active) {
        float s = w_rank / selected_sum;
        if (round_weights) s = round_bf16(s);
        weights[(size_t)row * active + lane] = valid ? s : __builtin_nanf("");
    }
}

// MoeAdjustRoutes (moe.rs:147-184): gains, then a stable insertion sort by id.
__global__ void moe_adjust_kernel(uint32_t* ids, float* weights, const float* scales, uint32_t rows,
                                  uint32_t experts, uint32_t active, uint32_t sort_ids) {
    const uint32_t row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const size_t base = (size_t)row * active;
    for (uint32_t r = 0; r < active; ++r) {
        const uint32_t id = ids[base + r];
        weights[base + r] = id < experts ? weights[base + r] * (scales ? scales[id] : 1.0f) : __builtin_nanf("");
    }
    if (sort_ids) {
        for (uint32_t r = 1; r < active; ++r) {
            uint32_t i = r;
            while (i > 0 && ids[base + i] < ids[base + i - 1]) {
                uint32_t t = ids[base + i];
                ids[base + i] = ids[base + i - 1];
                ids[base + i - 1] = t;
                float w = weights[base + i];
                weights[base + i] = weights[base + i - 1];
                weights[base + i - 1] = w;
                --i;
            }
        }
    }
}

// MoeGatherRows (moe.rs:87-107).
__global__ void moe_gather_rows_kernel(const uint32_t* ids, uint32_t* indices, uint32_t route_offset,
                                       uint32_t rows_per_expert, uint32_t experts, uint32_t length) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= length) return;
    uint32_t e = ids[route_offset];
    if (e >= experts) e = 0;
    indices[p] = e * rows_per_expert + p;
}

// MoeAccumulate (moe.rs:109-145).
__global__ void moe_accumulate_kernel(const uint16_t* input, const float* weights, float* acc, uint16_t* output,
                                      uint32_t length, uint32_t weight_offset, uint32_t output_offset,
                                      uint32_t initialize, uint32_t finalize, uint32_t round_product,
                                      uint32_t round_accumulator) {
    const uint32_t p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= length) return;
    const float w = weights[weight_offset];
    float product = __fmul_rn(bf16_bits_to_f32(input[p]), w);
    if (round_product) product = round_bf16(product);
    const size_t out = (size_t)output_offset + p;
    float v = __fadd_rn(initialize ? 0.0f : acc[out], product);
    if (round_accumulator) v = round_bf16(v);
    acc[out] = v;
    if (finalize) output[out] = f32_to_bf16_bits(v);
}

}  // namespace

// Adjust with optional gains: NULL scales stand for the unit gains the
// reference allocates when only the id sort is requested (routed.rs:205-208).
stark_qmm_status launch_moe_adjust(uint32_t* ids, float* weights, const float* scales, uint32_t rows,
                                   uint32_t experts, uint32_t active, uint32_t sort_ids, hipStream_t stream) {
    if (rows == 0) return STARK_QMM_OK;
    hipLaunchKernelGGL(moe_adjust_kernel, dim3((rows + 63) / 64), dim3(64), 0, stream, ids, weights, scales, rows,
                       experts, active, sort_ids);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm

using namespace qmm;

extern "C" {

stark_qmm_status stark_qmm_moe_route(const float* logits, uint32_t* ids, float* weights, uint32_t rows,
                                     uint32_t experts, uint32_t active, uint32_t round_weights,
                                     uint32_t round_logits, void* stream) {
    if (rows == 0) return STARK_QMM_OK;
    if (!logits || !ids || !weights || active == 0 || active > 32 || experts == 0 || experts > 1024)
        return STARK_QMM_INVALID_ARGUMENT;
    hipLaunchKernelGGL(moe_route_kernel, dim3(rows), dim3(64), 0, (hipStream_t)stream, logits, ids, weights, rows,
                       experts, active, round_weights, round_logits);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

stark_qmm_status stark_qmm_moe_adjust_routes(uint32_t* ids, float* weights, const float* scales, uint32_t rows,
                                             uint32_t experts, uint32_t active, uint32_t sort_ids, void* stream) {
    if (rows == 0 || active == 0) return STARK_QMM_OK;
    if (!ids || !weights || !scales) return STARK_QMM_INVALID_ARGUMENT;
    hipLaunchKernelGGL(moe_adjust_kernel, dim3((rows + 63) / 64), dim3(64), 0, (hipStream_t)stream, ids, weights,
                       scales, rows, experts, active, sort_ids);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

stark_qmm_status stark_qmm_moe_gather_rows(const uint32_t* ids, uint32_t* indices, uint32_t route_offset,
                                           uint32_t rows_per_expert, uint32_t experts, uint32_t length,
                                           void* stream) {
    if (length == 0) return STARK_QMM_OK;
    if (!ids || !indices) return STARK_QMM_INVALID_ARGUMENT;
    hipLaunchKernelGGL(moe_gather_rows_kernel, dim3((length + 255) / 256), dim3(256), 0, (hipStream_t)stream, ids,
                       indices, route_offset, rows_per_expert, experts, length);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

stark_qmm_status stark_qmm_moe_accumulate(const void* input, const float* weights, float* accumulator, void* output,
                                          uint32_t length, uint32_t weight_offset, uint32_t output_offset,
                                          uint32_t initialize, uint32_t finalize, uint32_t round_product,
                                          uint32_t round_accumulator, void* stream) {
    if (length == 0) return STARK_QMM_OK;
    if (!input || !weights || !accumulator || (finalize && !output)) return STARK_QMM_INVALID_ARGUMENT;
    hipLaunchKernelGGL(moe_accumulate_kernel, dim3((length + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)input, weights, accumulator, (uint16_t*)output, length, weight_offset,
                       output_offset, initialize, finalize, round_product, round_accumulator);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // extern "C"
