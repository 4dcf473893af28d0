// MoE routing kernels (reference: crates/stark-engine/src/backends/cpu/kernel/moe.rs and
// crates/stark-engine/src/backends/metal/kernel/moe.metal).
#include "qmm_common.h"

namespace qmm {

namespace {

QMM_DEVICE float round_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// MoeRoute (moe.rs:23-85): one 256-thread workgroup per token row. The
// reference's top-k is a repeated argmax where a strictly greater value wins
// and ties go to the lowest expert id (moe.rs:61-66), i.e. expert e lands at
// rank #{e' : x[e'] > x[e] or (x[e'] == x[e] and e' < e)}. Each thread counts
// that for its experts against the row staged in LDS: one pass, no
// cross-lane argmax rounds. The softmax denominator is a tree sum and exp is
// the device expf (the reference sums sequentially with the platform's libm
// exp): ids are exact, weights agree to a few ulp.
constexpr int kRouteThreads = 256;

__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(const float* logits, uint32_t* ids, float* weights,
                                                                  uint32_t rows, uint32_t experts, uint32_t active,
                                                                  uint32_t round_weights, uint32_t round_logits) {
    __shared__ float xs[1024];
    __shared__ float wred[kRouteThreads / 64];
    __shared__ uint32_t sel[32];
    __shared__ int all_finite;
    const uint32_t row = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (row >= rows) return;
    const bool shape_ok = experts >= 1 && experts <= 1024 && active >= 1 && active <= 32 && active <= experts;
    const uint32_t E = experts > 1024 ? 1024 : experts;
    if (t == 0) all_finite = 1;
    if (t < 32) sel[t] = 0;
    __syncthreads();
    float mx = -INFINITY;
    bool finite = true;
    for (uint32_t e = t; e < E; e += kRouteThreads) {
        float v = logits[(size_t)row * experts + e];
        if (round_logits) v = round_bf16(v);
        xs[e] = v;
        finite = finite && isfinite(v);
        mx = fmaxf(mx, v);
    }
    if (!finite) all_finite = 0;  // benign race: every writer stores 0
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
    if (lane == 0) wred[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(wred[0], wred[1]), fmaxf(wred[2], wred[3]));
    const bool valid = shape_ok && all_finite;
    float den = 0.0f;
    for (uint32_t e = t; e < E; e += kRouteThreads) den += expf(xs[e] - mx);
    den = wave_sum(den);
    __syncthreads();  // every thread has read wred (max) before it is reused
    if (lane == 0) wred[wave] = den;
    // ranks by counting
    for (uint32_t e = t; e < E; e += kRouteThreads) {
        const float v = xs[e];
        uint32_t rank = 0;
        for (uint32_t f = 0; f < E; ++f) {
            const float u = xs[f];
            rank += (u > v || (u == v && f < e)) ? 1u : 0u;
        }
        if (rank < active) sel[rank] = e;
    }
    __syncthreads();
    den = (wred[0] + wred[1]) + (wred[2] + wred[3]);
    // scores of the selected experts, then their sum in rank order (as the
    // reference accumulates), then the renormalised weights
    __shared__ float score[32];
    __shared__ float selected_sum;
    if (t < active && t < 32) score[t] = expf(xs[sel[t]] - mx) / den;
    __syncthreads();
    if (t == 0) {
        float sum = 0.0f;
        for (uint32_t r = 0; r < active && r < 32; ++r) sum += score[r];
        selected_sum = sum;
    }
    __syncthreads();
    if (t < active && t < 32) {
        float s = score[t] / selected_sum;
        if (round_weights) s = round_bf16(s);
        ids[(size_t)row * active + t] = valid ? sel[t] : 0u;
        weights[(size_t)row * active + t] = valid ? s : __builtin_nanf("");
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
    hipLaunchKernelGGL(moe_route_kernel, dim3(rows), dim3(kRouteThreads), 0, (hipStream_t)stream, logits, ids, weights, rows,
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
