// Shared device/host helpers for the gfx950 quantized matrix-product kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "../../include/stark_qmm.h"

#define QMM_DEVICE __device__ __forceinline__

namespace qmm {

// ---------------------------------------------------------------- numerics

QMM_DEVICE float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// f32 -> bf16 round-to-nearest-even with quiet-NaN forcing; the same rule the
// reference's `half` crate applies when writing bf16 outputs.
QMM_DEVICE uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

QMM_DEVICE float f16_bits_to_f32(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// v_cvt_f16_f32: round-to-nearest-even, overflow to infinity.
QMM_DEVICE uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Load element `i` of a dtype-tagged array as f32.
QMM_DEVICE float load_as_f32(const void* p, uint32_t dt, size_t i) {
    if (dt == STARK_QMM_F32) return ((const float*)p)[i];
    uint32_t h = ((const uint16_t*)p)[i];
    return dt == STARK_QMM_BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

QMM_DEVICE void store_from_f32(void* p, uint32_t dt, size_t i, float v) {
    if (dt == STARK_QMM_F32) {
        ((float*)p)[i] = v;
    } else if (dt == STARK_QMM_BF16) {
        ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
    } else {
        ((uint16_t*)p)[i] = f32_to_f16_bits(v);
    }
}

// Full 64-lane sum; every lane receives the total.
QMM_DEVICE float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte nontemporal load of weight codes that are read exactly once per launch.
QMM_DEVICE u32x4 load_stream(const void* p) { return __builtin_nontemporal_load((const u32x4*)p); }

// (a & mask) | orv in one VALU op: gfx950 VOP3 takes no literal, so the mask
// rides in an SGPR and the or-value in a VGPR.
QMM_DEVICE uint32_t and_or(uint32_t a, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(orv));
    return r;
}

// Sum each of 8 per-lane values over the wave with a transposed butterfly
// (10 shuffles instead of 48). Returns, in every lane, the total of value
// r = 4*bit5 + 2*bit4 + bit3 of the lane id.
QMM_DEVICE float wave_sum8(const float (&v)[8], int lane) {
    const bool h32 = lane & 32, h16 = lane & 16, h8 = lane & 8;
    float a[4], b[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] = (h32 ? v[4 + j] : v[j]) + __shfl_xor(h32 ? v[j] : v[4 + j], 32, 64);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = (h16 ? a[2 + j] : a[j]) + __shfl_xor(h16 ? a[j] : a[2 + j], 16, 64);
    float c = (h8 ? b[1] : b[0]) + __shfl_xor(h8 ? b[0] : b[1], 8, 64);
    c += __shfl_xor(c, 4, 64);
    c += __shfl_xor(c, 2, 64);
    c += __shfl_xor(c, 1, 64);
    return c;
}

// ---- Lane exchanges inside a row of 16 lanes through DPP (no LDS traffic,
// unlike __shfl_xor's ds_bpermute). Every lane receives the result.
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140 };

template <int CTRL>
QMM_DEVICE uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
QMM_DEVICE float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum / max over aligned groups of L consecutive lanes (L = 1, 2, 4, 8, 16).
template <int L>
QMM_DEVICE float group_sum(float v) {
    if (L >= 2) v += dpp_f32<DPP_XOR1>(v);
    if (L >= 4) v += dpp_f32<DPP_XOR2>(v);
    if (L >= 8) v += dpp_f32<DPP_HALF_MIRROR>(v);
    if (L >= 16) v += dpp_f32<DPP_MIRROR>(v);
    return v;
}
template <int L>
QMM_DEVICE uint32_t group_max(uint32_t v) {
    if (L >= 2) v = max(v, dpp_u32<DPP_XOR1>(v));
    if (L >= 4) v = max(v, dpp_u32<DPP_XOR2>(v));
    if (L >= 8) v = max(v, dpp_u32<DPP_HALF_MIRROR>(v));
    if (L >= 16) v = max(v, dpp_u32<DPP_MIRROR>(v));
    return v;
}

// ---- Per-group activation exponent of the matrix-core kernels. Their codes
// enter the MFMA as raw bf16 bit patterns (a pattern p < 256 is exactly
// p * 2^-133), so each group's activations are staged as x * 2^E with
// E = min(189 - f, 127), f the largest exponent field in the group: the
// group's largest |x| lands in [2^62, 2^64), every product x * 2^E * q * 2^-133
// is exact and in f32's normal range (for |x| >= 2^-120 or so), and the group's
// accumulated sum is brought back with one v_ldexp_f32 by 133 - E. This holds
// for every finite activation (E = -66 for Inf/NaN keeps them as they are).

// Largest exponent field among the 8 bf16 values of a 16-byte vector.
QMM_DEVICE uint32_t bf16x8_exp_max(const u32x4& t) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const auto h = [](uint32_t w) { return __builtin_bit_cast(u16x2, w & 0x7f807f80u); };
    const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(h(t[0]), h(t[1])),
                                              __builtin_elementwise_max(h(t[2]), h(t[3])));
    return (uint32_t)max(m[0], m[1]) >> 7;
}

// Largest f32 exponent field among 8 f32 values (two 16-byte vectors).
QMM_DEVICE uint32_t f32x8_exp_max(const u32x4& a, const u32x4& b) {
    uint32_t m = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) m = max(m, max(a[e] & 0x7f800000u, b[e] & 0x7f800000u));
    return m >> 23;
}

// Staging exponent E of a group whose largest exponent field is f.
QMM_DEVICE int group_shift(uint32_t f) { return min(189 - (int)f, 127); }

// 2^e as f32 for e in [-126, 127].
QMM_DEVICE float pow2i(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

// c * 2^n, exact unless the result leaves f32's range.
QMM_DEVICE float ldexp_f32(float c, int n) { return __builtin_amdgcn_ldexpf(c, n); }

// D = a.lo*b.lo + a.hi*b.hi + c (products exact for bf16, f32 accumulate).
QMM_DEVICE float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

}  // namespace qmm

// ------------------------------------------------------------------ host side

#define QMM_HIP_CHECK(expr)                                   \
    do {                                                      \
        hipError_t qmm_err_ = (expr);                         \
        if (qmm_err_ != hipSuccess) return STARK_QMM_DEVICE_FAILURE; \
    } while (0)

namespace qmm {

// Epilogue and correction flags shared by the matvec kernels.
enum : uint32_t {
    FLAG_ACCUMULATE = 1u << 0,
    FLAG_SOFT_CAP = 1u << 1,
    FLAG_SIGNED = 1u << 2,
};

// One affine matrix product d[m, n] = sum_k a[m, k] * (s * q + bias_term).
struct AffineOp {
    const uint8_t* codes;    // [N, K*bits/8]
    const void* scales;      // plane in w_dt
    const void* corr;        // biases (w_dt) / zero points (u8) / NULL
    const void* x;           // [M, K] in x_dt
    void* d;                 // [M, N] in d_dt
    const void* bias;        // [N] in w_dt or NULL
    const uint32_t* gather;  // [M*N] or NULL
    uint32_t n, k, m;
    uint32_t os, gs;         // scale/bias plane strides (elements)
    uint32_t zos, zgs;       // zero-point strides (nibbles for 4-bit, bytes for 8-bit)
    uint32_t group_size;
    uint32_t corr_kind;      // STARK_QMM_CORRECTION_*
    uint32_t w_dt, x_dt, d_dt;
    uint32_t flags;
    float ab_scale, soft_cap;
    uint32_t bank_rows;      // weight rows present in the codes buffer (gather bound)
    uint32_t block_begin;    // first blockIdx.x of this op inside a batched launch
    uint32_t xid;            // streaming kernel: ops with the same activations (x, K) share an id;
                             // small-M kernel: tile pairs per workgroup
};

constexpr int kMaxBatchOps = 8;

struct AffineBatch {
    AffineOp op[kMaxBatchOps];
    uint32_t count;
    uint32_t total;     // work tiles over all ops
    uint32_t nib_mask;  // 0x00780078: nibble-pair mask, passed in so it stays in an SGPR
    uint32_t nib_one;   // 0x3F803F80: bf16 1.0 pair, likewise
    // streaming kernel's input prologue (every op of the launch reads the same row)
    const void* pro_data;  // RMS-norm weights or the gated product's up values, [K] bf16
    float pro_eps;
};

// Input prologue of a streaming launch: the activation row is transformed
// while it is staged (kind: STARK_QMM_PROLOGUE_*).
struct StreamPrologue {
    uint32_t kind;
    const void* data;
    float eps;
};

// Launch helpers implemented in qmv_affine.hip.
stark_qmm_status launch_affine_gemv(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream);
stark_qmm_status launch_affine_generic(const AffineOp& op, int bits, hipStream_t stream);
bool affine_fast_eligible(const AffineOp& op, int bits);
// Wave-independent kernel for decode-shaped 4-bit products (qmv_decode.hip).
bool decode_eligible(const AffineOp& op, int bits);
stark_qmm_status launch_affine_decode(const AffineOp* ops, uint32_t count, hipStream_t stream);
stark_qmm_status launch_affine_materialized(const AffineOp& op, hipStream_t stream);
// Prefill dequant-GEMM on the matrix cores for M > 16 (qgemm_mfma.hip).
bool gemm_eligible(const AffineOp& op, int bits);
uint32_t gemm_rows(uint32_t k);  // activation rows one dequant-GEMM grid takes at K
stark_qmm_status launch_affine_gemm(const AffineOp& op, int bits, hipStream_t stream);
stark_qmm_status launch_affine_gemm_group(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream);
// Route adjustment with optional gains (moe.hip).
stark_qmm_status launch_moe_adjust(uint32_t* ids, float* weights, const float* scales, uint32_t rows,
                                   uint32_t experts, uint32_t active, uint32_t sort_ids, hipStream_t stream);
// Dense small-M kernel: 4-bit, group 64, M = 3 .. 16, K % 1024 == 0 (qmv_small_m.hip).
bool small_m_eligible(const AffineOp* ops, uint32_t count);
stark_qmm_status launch_small_m(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream);
// Skinny dequant product: 4-bit, group 64, M = 17 .. 64, K % 512 == 0, the
// dequant-GEMM's bf16-effective arithmetic (qgemm_skinny.hip).
bool skinny_eligible(const AffineOp* ops, uint32_t count);
stark_qmm_status launch_skinny(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream);
// Matrix-core kernel for 4/8-bit products with M <= 16 (qmv_mfma.hip).
bool mfma_eligible(const AffineOp& op, int bits);
stark_qmm_status launch_affine_mfma(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream);
// Streaming kernel with an input prologue: ops that all read one bf16 row
// (same x and K), each mfma_eligible for 4 bits, m == 1, group 64, K % 4096 == 0,
// N >= 32; otherwise STARK_QMM_UNSUPPORTED.
stark_qmm_status launch_stream_prologue(const AffineOp* ops, uint32_t count, const StreamPrologue& pro,
                                        hipStream_t stream);
// Full-precision B operand (MatmulB::FullPrecision).
struct DenseOp {
    const void* w;           // [N, ld] (transpose) or [K, ld]
    const void* x;           // [M, K]
    void* d;                 // [M, N]
    const void* bias;
    const uint32_t* gather;
    uint32_t n, k, m, ld, transpose;
    uint32_t w_dt, x_dt, d_dt, flags;
    float ab_scale, soft_cap;
    uint32_t bank_rows;
};
stark_qmm_status launch_dense_gemv(const DenseOp& op, hipStream_t stream);

// GGUF packed-block matvec (kinds 8 = Q8_0, 12 = Q4_K).
struct GgufOp {
    const uint8_t* blocks;   // [N, K/block * block_bytes]
    uint32_t kind;
    const void* x;           // [M, K] in x_dt (f32 on the hybrid path)
    void* d;                 // [M, N] in d_dt
    uint32_t n, k, m;
    uint32_t x_dt, d_dt;     // 0/0 means f32/f32
    uint32_t block_begin;
    uint32_t run;            // dense matrix-core form: tile pairs per workgroup (set by the launch)
};
struct GgufBatch {
    GgufOp op[kMaxBatchOps];
    uint32_t count;
    uint32_t* status;  // ORed with 1 when an activation is not finite
};
bool gguf_supported(uint32_t kind);
// Every op's activations are checked for non-finite values (status |= 1).
stark_qmm_status launch_gguf_gemv(const GgufOp* ops, uint32_t count, uint32_t* status, hipStream_t stream);
// status |= 1 when any of x[0..n) is not finite (mapped.hip).
stark_qmm_status launch_finite_check(const float* x, uint64_t n, uint32_t* status, hipStream_t stream);

// Output RHT of a product (transforms.hip): d <- RHT(d) * factors, then + bias.
stark_qmm_status launch_output_rht(void* d, uint32_t d_dt, const void* bias, uint32_t bias_dt,
                                   const int32_t* factors, uint32_t rows, uint32_t n, hipStream_t stream);
// Int8-activation products (qmv_a8.hip).
struct A8Operand {
    const int8_t* codes;   // [M, K] in code layout order
    const float* scales;   // [M, K / group]
    uint32_t group;        // activation scale group
    uint32_t grouped;      // Int8CodeLayout::GroupedByNibble
};
stark_qmm_status launch_affine_a8(const AffineOp& op, const A8Operand& a, int bits, hipStream_t stream);
// int8-activation products of one grid (prefill sizes)
struct A8Batch {
    AffineOp op[kMaxBatchOps];
    A8Operand a[kMaxBatchOps];
    uint32_t count;
};
bool a8_gemm_eligible(const AffineOp& op, const A8Operand& a, int bits);
uint32_t a8_gemm_class(const AffineOp& op, const A8Operand& a, int bits);
stark_qmm_status launch_affine_a8_gemm_group(const AffineOp* ops, const A8Operand* as, uint32_t count, int bits,
                                             hipStream_t stream);

// Largest M the GEMV kernel handles in one weight pass.
constexpr uint32_t kGemvMaxM = 2;

}  // namespace qmm
