// Products with int8 activations (MatmulA::Int8Symmetric, the A8W4 / A8W8
// path): a = q_a * scale_a per activation group (32/64/128 values), weights
// 4- or 8-bit affine. Reference: MatmulCpuKernel::encode
// (crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:122-141, 193-205),
// which forms a = q * scale and w = s * q + bias_term in f32 and accumulates
// a * w in order.
//
// Fast form (qmv_a8): per 16-byte piece of a weight row (32 4-bit or 16 8-bit
// values, inside one weight group and one activation group)
//   sum a*w = scale_a * (s * sum(q_a * q_w) + bias_term * sum(q_a))
// with both sums exact in int32 on v_dot4_i32_i8. 4-bit codes unpack to the
// bytes (q0, q2, q4, q6) and (q1, q3, q5, q7) of each word, which is how the
// grouped-by-nibble activation layout stores its codes
// (Int8CodeLayout::GroupedByNibble, matmul_a.rs:31-46); sequential codes are
// permuted into that order with v_perm_b32. 8-bit codes enter as q - 128 and
// the sum gets 128 * sum(q_a) back. One wave per weight row, lanes over its
// pieces, up to 16 activation rows per pass over the weights; the f32 sums
// meet in a wave reduction. Generic form (qmv_a8_generic): one thread per
// output in the reference's order, for gathers and unaligned rows.
#include "qmm_common.h"

namespace qmm {
namespace {

constexpr int kA8Rows = 16;  // activation rows per pass over a weight row
constexpr int kA8Wg = 256;   // 4 waves = 4 weight rows per workgroup

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// bias_term of weight row n, group h (kernel.rs:226-262)
__device__ __forceinline__ void affine_terms(const AffineOp& op, int bits, uint32_t n, uint32_t h, float* s, float* b) {
    const size_t md = (size_t)n * op.os + (size_t)h * op.gs;
    *s = load_as_f32(op.scales, op.w_dt, md);
    if (op.corr_kind == STARK_QMM_CORRECTION_BIASES) {
        *b = load_as_f32(op.corr, op.w_dt, md);
    } else if (op.corr_kind == STARK_QMM_CORRECTION_ZERO_POINTS) {
        const size_t zi = (size_t)n * op.zos + (size_t)h * op.zgs;
        const uint8_t* z = (const uint8_t*)op.corr;
        const float zp = bits == 4 ? (float)((zi % 2 == 0) ? (z[zi / 2] & 15) : (z[zi / 2] >> 4)) : (float)z[zi];
        *b = -*s * zp;
    } else {
        *b = -*s * (float)(1 << (bits - 1));
    }
}

__device__ __forceinline__ void epilogue(const AffineOp& op, uint32_t m, uint32_t n, float acc) {
    const size_t o = (size_t)m * op.n + n;
    float v = op.ab_scale * acc;
    if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
    if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
    if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
    store_from_f32(op.d, op.d_dt, o, v);
}

template <int BITS>
__global__ __launch_bounds__(kA8Wg) void qmv_a8(AffineOp op, A8Operand a) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = blockIdx.x * (kA8Wg / 64) + (threadIdx.x >> 6);
    const uint32_t m0 = blockIdx.y * kA8Rows;
    if (n >= op.n) return;  // wave-uniform
    constexpr uint32_t VPP = BITS == 4 ? 32 : 16;  // values per 16-byte piece
    const uint32_t K = op.k, pieces = K / VPP, GA = K / a.group;
    const uint8_t* wrow = op.codes + (size_t)n * (K * BITS / 8);
    const uint32_t rows = min((uint32_t)kA8Rows, op.m - m0);
    float acc[kA8Rows];
#pragma unroll
    for (int i = 0; i < kA8Rows; ++i) acc[i] = 0.0f;
    for (uint32_t p = lane; p < pieces; p += 64) {
        u32x4 w = load_stream(wrow + (size_t)p * 16);
        if (op.flags & FLAG_SIGNED) {
#pragma unroll
            for (int t = 0; t < 4; ++t) w[t] ^= BITS == 4 ? 0x88888888u : 0x80808080u;
        }
        const uint32_t k0 = p * VPP;
        float s, b;
        affine_terms(op, BITS, n, k0 / op.group_size, &s, &b);
        // weight bytes in the activation code order: BITS 4: per word
        // (q0,q2,q4,q6), (q1,q3,q5,q7); BITS 8: q - 128 in value order
        uint32_t wb[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (BITS == 4) {
                wb[2 * t] = w[t] & 0x0F0F0F0Fu;
                wb[2 * t + 1] = (w[t] >> 4) & 0x0F0F0F0Fu;
            } else {
                wb[t] = w[t] ^ 0x80808080u;
            }
        }
        const uint32_t g = k0 / a.group;
#pragma unroll
        for (uint32_t i = 0; i < (uint32_t)kA8Rows; ++i) {
            if (i >= rows) break;
            const uint32_t m = m0 + i;
            const uint32_t* aw = (const uint32_t*)(a.codes + (size_t)m * K + k0);
            int dot = 0, sum = 0;
#pragma unroll
            for (int t = 0; t < (int)VPP / 8; ++t) {
                uint32_t x0 = aw[2 * t], x1 = aw[2 * t + 1];  // stored codes of values 8t .. 8t+7
                if (BITS == 4 && !a.grouped) {  // sequential -> (v0,v2,v4,v6), (v1,v3,v5,v7)
                    const uint32_t e = __builtin_amdgcn_perm(x1, x0, 0x06040200u);
                    const uint32_t o = __builtin_amdgcn_perm(x1, x0, 0x07050301u);
                    x0 = e;
                    x1 = o;
                } else if (BITS == 8 && a.grouped) {  // grouped -> value order
                    const uint32_t lo = __builtin_amdgcn_perm(x1, x0, 0x05010400u);
                    const uint32_t hi = __builtin_amdgcn_perm(x1, x0, 0x07030602u);
                    x0 = lo;
                    x1 = hi;
                }
                dot = sdot4(x0, wb[2 * t], dot);
                dot = sdot4(x1, wb[2 * t + 1], dot);
                sum = sdot4(x0, 0x01010101u, sum);
                sum = sdot4(x1, 0x01010101u, sum);
            }
            if (BITS == 8) dot += 128 * sum;
            const float sa = a.scales[(size_t)m * GA + g];
            acc[i] = fmaf(sa, fmaf(s, (float)dot, b * (float)sum), acc[i]);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < (uint32_t)kA8Rows; ++i) {
        if (i >= rows) break;
        const float v = wave_sum(acc[i]);
        if (lane == 0) epilogue(op, m0 + i, n, v);
    }
}

// One thread per output, kernel.rs:170-282 order with the int8 A (gathers,
// any aligned or unaligned row).
__global__ __launch_bounds__(256) void qmv_a8_generic(AffineOp op, A8Operand a, int bits) {
    const uint32_t n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
    if (n >= op.n || m >= op.m) return;
    const uint32_t K = op.k, GA = K / a.group;
    uint32_t row = n;
    if (op.gather) {
        row = op.gather[(size_t)m * op.n + n];
        if (row >= op.bank_rows) {
            epilogue(op, m, n, __int_as_float(0x7fc00000));
            return;
        }
    }
    float acc = 0.0f;
    for (uint32_t k = 0; k < K; ++k) {
        const uint32_t ci = a.grouped ? (k - (k & 7u) + (k & 1u) * 4u + (k & 7u) / 2u) : k;
        const float av = (float)a.codes[(size_t)m * K + ci] * a.scales[(size_t)m * GA + k / a.group];
        const size_t bit = ((size_t)row * K + k) * bits;
        uint32_t code = op.codes[bit / 8] >> (bit % 8);
        code &= (1u << bits) - 1u;
        if (op.flags & FLAG_SIGNED) code ^= 1u << (bits - 1);
        float s, b;
        affine_terms(op, bits, row, k / op.group_size, &s, &b);
        acc += av * (s * (float)code + b);
    }
    epilogue(op, m, n, acc);
}

}  // namespace

stark_qmm_status launch_affine_a8(const AffineOp& op, const A8Operand& a, int bits, hipStream_t stream) {
    if (op.m == 0 || op.n == 0) return STARK_QMM_OK;
    const uint32_t vpp = bits == 4 ? 32 : 16;
    const bool fast = !op.gather && op.k % vpp == 0 && ((uintptr_t)op.codes & 15) == 0 &&
                      ((size_t)op.k * bits / 8) % 16 == 0 && ((uintptr_t)a.codes & 3) == 0 && op.k % 4 == 0;
    if (fast) {
        const dim3 grid((op.n + kA8Wg / 64 - 1) / (kA8Wg / 64), (op.m + kA8Rows - 1) / kA8Rows);
        if (bits == 4)
            hipLaunchKernelGGL(qmv_a8<4>, grid, dim3(kA8Wg), 0, stream, op, a);
        else
            hipLaunchKernelGGL(qmv_a8<8>, grid, dim3(kA8Wg), 0, stream, op, a);
    } else {
        hipLaunchKernelGGL(qmv_a8_generic, dim3((op.n + 255) / 256, op.m), dim3(256), 0, stream, op, a, bits);
    }
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm
