// Full-precision GEMV used for MatmulB::FullPrecision operands (e.g. the MoE
// router, a bf16 [experts, model] matrix; crates/stark-engine/src/encodable_block/mlp/qwen_moe.rs:64).
// Per output the reference multiplies and adds sequentially in f32
// (crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:206-218, 267); here one
// wave owns a row and reduces 64 lane-partials (sums agree to f32 rounding).
#include "qmm_common.h"

namespace qmm {

namespace {

__global__ __launch_bounds__(256) void gemv_dense_rows(DenseOp op) {
    const int lane = threadIdx.x & 63;
    const uint32_t n = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t m = blockIdx.y;
    if (n >= op.n) return;
    const size_t row = op.gather ? op.gather[(size_t)m * op.n + n] : n;
    const size_t o = (size_t)m * op.n + n;
    if (row >= op.bank_rows) {
        if (lane == 0) store_from_f32(op.d, op.d_dt, o, __builtin_nanf(""));
        return;
    }
    float acc = 0.0f;
    for (uint32_t k = lane; k < op.k; k += 64) {
        const float a = load_as_f32(op.x, op.x_dt, (size_t)m * op.k + k);
        const float w = load_as_f32(op.w, op.w_dt, row * op.ld + k);
        acc = fmaf(a, w, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) {
        float v = op.ab_scale * acc;
        if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
        if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
        if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
        store_from_f32(op.d, op.d_dt, o, v);
    }
}

// bf16 x and w, no gather, 16-byte aligned rows: one workgroup per weight row;
// its four waves split K (8 values per lane per load, the row read once for up
// to MT activation rows) and meet in LDS.
template <int MT>
__global__ __launch_bounds__(256) void gemv_dense_bf16(DenseOp op) {
    __shared__ float part[4][MT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t n = blockIdx.x;
    const uint32_t m0 = blockIdx.y * MT;
    const uint16_t* w = (const uint16_t*)op.w + (size_t)n * op.ld;
    const uint16_t* x = (const uint16_t*)op.x;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (uint32_t k = (wave * 64 + lane) * 8; k < op.k; k += 2048) {
        const u32x4 wv = *(const u32x4*)(w + k);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (m0 + t < op.m) {
                const u32x4 xv = *(const u32x4*)(x + (size_t)(m0 + t) * op.k + k);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t] = dot2_bf16(wv[e], xv[e], acc[t]);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const float sum = wave_sum(acc[t]);
        if (lane == 0) part[wave][t] = sum;
    }
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < (uint32_t)MT && m0 + t < op.m) {
        const float sum = (part[0][t] + part[1][t]) + (part[2][t] + part[3][t]);
        const size_t o = (size_t)(m0 + t) * op.n + n;
        float v = op.ab_scale * sum;
        if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
        if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
        if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
        store_from_f32(op.d, op.d_dt, o, v);
    }
}

// B stored [K, ld] (b_transpose = false): thread per output.
__global__ __launch_bounds__(256) void gemv_dense_cols(DenseOp op) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t m = blockIdx.y;
    if (n >= op.n) return;
    const size_t col = op.gather ? op.gather[(size_t)m * op.n + n] : n;
    const size_t o = (size_t)m * op.n + n;
    if (col >= op.bank_rows) {
        store_from_f32(op.d, op.d_dt, o, __builtin_nanf(""));
        return;
    }
    float acc = 0.0f;
    for (uint32_t k = 0; k < op.k; ++k)
        acc = fmaf(load_as_f32(op.x, op.x_dt, (size_t)m * op.k + k), load_as_f32(op.w, op.w_dt, k * op.ld + col), acc);
    float v = op.ab_scale * acc;
    if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
    if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
    if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
    store_from_f32(op.d, op.d_dt, o, v);
}

}  // namespace

stark_qmm_status launch_dense_gemv(const DenseOp& op, hipStream_t stream) {
    if (op.n == 0 || op.m == 0) return STARK_QMM_OK;
    const bool fast = op.transpose && op.w_dt == STARK_QMM_BF16 && op.x_dt == STARK_QMM_BF16 && !op.gather &&
                      op.k % 8 == 0 && op.ld % 8 == 0 && (((uintptr_t)op.w | (uintptr_t)op.x) & 15) == 0;
    if (fast) {
        hipLaunchKernelGGL(gemv_dense_bf16<8>, dim3(op.n, (op.m + 7) / 8), dim3(256), 0, stream, op);
    } else if (op.transpose) {
        hipLaunchKernelGGL(gemv_dense_rows, dim3((op.n + 3) / 4, op.m), dim3(256), 0, stream, op);
    } else {
        hipLaunchKernelGGL(gemv_dense_cols, dim3((op.n + 255) / 256, op.m), dim3(256), 0, stream, op);
    }
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm
