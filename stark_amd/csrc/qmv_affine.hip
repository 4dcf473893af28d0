// Affine (MLX-style) quantized matvec for small M on gfx950.
//
// d[m, n] = sum_k a[m, k] * (s[n, g] * q[n, k] + bias_term[n, g]),  g = k / group_size
//
// Semantics follow the reference CPU kernel
// (crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:170-282); the
// summation is reassociated per group as the reference's Metal GEMV does
// (crates/stark-engine/src/backends/metal/kernel/matmul/gemv/common/quant_metadata.h:103-114):
//   acc += s * sum_{k in g} x*q + bias_term * sum_{k in g} x
//
// Design (HBM-bound streaming):
// * one workgroup = 4 wave64s = a tile of 32 weight rows; the K axis is walked in
//   passes of 4096 values; within a pass lane L of a wave owns 16-byte code
//   chunks L, L+64, ... so every load instruction reads 1 KiB contiguous;
// * the activation slice of the pass and the tile's per-group (scale, bias)
//   are staged once per workgroup in LDS, then each lane keeps its activation
//   chunks in registers for all 8 rows of its wave;
// * 4-bit x bf16: nibbles become bf16 (1 + q/16) with one shift and one
//   and-or per pair and feed v_dot2_f32_bf16 (products exact, f32 sums);
//   the offset is folded into the group's (scale, bias):
//     s*sum(x*q) + b*sum(x) = 16s * sum(x*(1+q/16)) + (b - 16s) * sum(x)
// * other types: v_cvt_f32_ubyte + f32 FMA;
// * rows are reduced across the wave at the end.
#include "qmm_common.h"

namespace qmm {

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = 32;
constexpr int kRowsPerWave = kRowsPerBlock / (kThreads / 64);
constexpr int kPassValues = 4096;

// Byte B of a dword as f32 (selects v_cvt_f32_ubyteB).
template <int B>
__device__ __forceinline__ float ubyte(uint32_t w) {
    return (float)((w >> (8 * B)) & 0xffu);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Generic slow path: one thread per output, the reference's exact per-element
// order (kernel.rs:185-268): w = s*q + bias_term; acc += a*w with separate
// roundings. Handles every shape the fast kernel does not (odd K, 3/5/6-bit
// codes, misaligned buffers, tiny groups).
__global__ __launch_bounds__(256) void qmv_affine_generic(AffineOp op, int bits) {
    uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t m = blockIdx.y;
    if (n >= op.n || m >= op.m) return;
    uint32_t wrow = op.gather ? op.gather[(size_t)m * op.n + n] : n;
    size_t oi = (size_t)m * op.n + n;
    if (wrow >= op.bank_rows) {
        store_from_f32(op.d, op.d_dt, oi, __builtin_nanf(""));
        return;
    }
    float acc = 0.0f;
    float midpoint = (float)(1u << (bits - 1));
    for (uint32_t k = 0; k < op.k; ++k) {
        float a = load_as_f32(op.x, op.x_dt, (size_t)m * op.k + k);
        size_t bit = ((size_t)wrow * op.k + k) * (size_t)bits;
        size_t off = bit >> 3;
        uint32_t shift = (uint32_t)(bit & 7);
        uint32_t v = op.codes[off];
        if (shift + bits > 8) v |= (uint32_t)op.codes[off + 1] << 8;
        uint32_t code = (v >> shift) & ((1u << bits) - 1u);
        if (op.flags & FLAG_SIGNED) code ^= 1u << (bits - 1);
        uint32_t g = k / op.group_size;
        size_t md = (size_t)wrow * op.os + (size_t)g * op.gs;
        float s = load_as_f32(op.scales, op.w_dt, md);
        float bt;
        if (op.corr_kind == STARK_QMM_CORRECTION_BIASES) {
            bt = load_as_f32(op.corr, op.w_dt, md);
        } else if (op.corr_kind == STARK_QMM_CORRECTION_ZERO_POINTS) {
            size_t zi = (size_t)wrow * op.zos + (size_t)g * op.zgs;
            uint32_t zb;
            if (bits == 4) {
                uint32_t byte = ((const uint8_t*)op.corr)[zi >> 1];
                zb = (zi & 1) ? (byte >> 4) & 15u : byte & 15u;
            } else {
                zb = ((const uint8_t*)op.corr)[zi];
            }
            bt = __fmul_rn(-s, (float)zb);
        } else {
            bt = __fmul_rn(-s, midpoint);
        }
        float w = __fadd_rn(__fmul_rn(s, (float)code), bt);
        acc = __fadd_rn(acc, __fmul_rn(a, w));
    }
    float v = __fmul_rn(op.ab_scale, acc);
    if (op.flags & FLAG_ACCUMULATE) v = __fadd_rn(v, load_as_f32(op.d, op.d_dt, oi));
    if (op.bias) v = __fadd_rn(v, load_as_f32(op.bias, op.w_dt, n));
    if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
    store_from_f32(op.d, op.d_dt, oi, v);
}

// MLX-source-compatible single-row W4 dot (MLXSpec.materialize_affine_input_sum),
// restating crates/stark-engine/src/backends/cpu/kernel/matmul/reference.rs:109-154:
// per 16-value chunk, products summed in quads, activations summed as bf16
// quads, `result += s*dot + b*sum`. One thread per output; bf16 in/out, biases.
__global__ __launch_bounds__(256) void qmv_affine_materialized(AffineOp op) {
    uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= op.n) return;
    uint32_t col = op.gather ? op.gather[n] : n;
    if (col >= op.bank_rows) {
        store_from_f32(op.d, op.d_dt, n, __builtin_nanf(""));
        return;
    }
    const uint16_t* x = (const uint16_t*)op.x;
    const uint32_t K = op.k;
    float result = 0.0f;
    for (uint32_t begin = 0; begin < K; begin += 16) {
        uint32_t end = min(begin + 16, K);
        float dot = 0.0f, sum = 0.0f;
        for (uint32_t quad = begin; quad < end; quad += 4) {
            uint32_t v[4] = {0, 0, 0, 0};
            float subtotal = 0.0f;
            for (uint32_t i = 0; i < 4; ++i) {
                if (quad + i < end) {
                    v[i] = x[quad + i];
                    size_t idx = (size_t)col * K + quad + i;
                    uint32_t code = (op.codes[idx >> 1] >> (4 * (idx & 1))) & 15u;
                    subtotal = __fadd_rn(subtotal, __fmul_rn(bf16_bits_to_f32(v[i]), (float)code));
                }
            }
            dot = __fadd_rn(dot, subtotal);
            uint32_t s01 = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(v[0]), bf16_bits_to_f32(v[1])));
            uint32_t s012 = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(s01), bf16_bits_to_f32(v[2])));
            uint32_t s0123 = f32_to_bf16_bits(__fadd_rn(bf16_bits_to_f32(s012), bf16_bits_to_f32(v[3])));
            sum = __fadd_rn(sum, bf16_bits_to_f32(s0123));
        }
        size_t md = (size_t)col * op.os + (size_t)(begin / op.group_size) * op.gs;
        float s = bf16_bits_to_f32(((const uint16_t*)op.scales)[md]);
        float b = bf16_bits_to_f32(((const uint16_t*)op.corr)[md]);
        result = __fadd_rn(result, __fadd_rn(__fmul_rn(s, dot), __fmul_rn(b, sum)));
    }
    float v = __fmul_rn(op.ab_scale, result);
    if (op.flags & FLAG_ACCUMULATE) v = __fadd_rn(v, load_as_f32(op.d, op.d_dt, n));
    if (op.bias) v = __fadd_rn(v, load_as_f32(op.bias, op.w_dt, n));
    if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
    store_from_f32(op.d, op.d_dt, n, v);
}

// Per-lane activation registers for one pass.
template <int BITS, int MT, bool DOT2>
struct XRegs {
    static constexpr int VPC = 128 / BITS;                // values per 16-byte chunk
    static constexpr int CPL = kPassValues / (64 * VPC);  // chunks per lane per pass
    // DOT2: 16 bf16 pairs per 32-value chunk; else VPC floats per chunk.
    static constexpr int WORDS = DOT2 ? 16 : VPC;
    uint32_t v[MT][CPL][WORDS];
    float sum[MT][CPL];
};

template <int BITS, int MT, bool DOT2>
__global__ __launch_bounds__(kThreads) void qmv_affine_fast(AffineBatch batch) {
    using X = XRegs<BITS, MT, DOT2>;
    constexpr int VPC = X::VPC;
    constexpr int CPL = X::CPL;
    constexpr int RBATCH = BITS == 4 ? 8 : 4;  // rows whose codes are in flight together

    extern __shared__ __align__(16) uint8_t smem[];

    // ---- locate this block's op (uniform scalar select; no dynamic kernarg indexing)
    const uint32_t bid = blockIdx.x;
    int oi = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatchOps; ++i)
        if (i < (int)batch.count && bid >= batch.op[i].block_begin) oi = i;
    AffineOp op = batch.op[0];
#pragma unroll
    for (int i = 1; i < kMaxBatchOps; ++i)
        if (oi == i) op = batch.op[i];

    const uint32_t N = op.n, K = op.k;
    const uint32_t nrb = (N + kRowsPerBlock - 1) / kRowsPerBlock;
    const uint32_t lb = bid - op.block_begin;
    const uint32_t mtile = lb / nrb;
    const uint32_t n0 = (lb - mtile * nrb) * kRowsPerBlock;
    const uint32_t m0 = mtile * MT;
    const int mcount = min((int)MT, (int)(op.m - m0));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const size_t row_bytes = (size_t)K * BITS / 8;
    const uint32_t gsz = op.group_size;
    const uint32_t G = K / gsz;
    const uint32_t gpp = kPassValues / gsz;  // groups per pass

    uint32_t* s_wrow = (uint32_t*)smem;                                   // [32]
    float2* s_meta = (float2*)(smem + 128);                               // [32 * gpp]
    uint8_t* s_x = smem + 128 + (size_t)kRowsPerBlock * gpp * sizeof(float2);  // [MT][4096] bf16 or f32

    if (tid < kRowsPerBlock) {
        uint32_t n = n0 + tid;
        uint32_t w = 0xffffffffu;
        if (n < N) {
            w = op.gather ? op.gather[(size_t)m0 * N + n] : n;
            if (w >= op.bank_rows) w = 0xffffffffu;  // out-of-bank gathered row: NaN output below
        }
        s_wrow[tid] = w;
    }

    float acc[kRowsPerWave][MT];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    const uint32_t npass = (K + kPassValues - 1) / kPassValues;
    const float midpoint = (float)(1u << (BITS - 1));
    const bool go_layout = op.os == 1;  // group-output planes: consecutive rows are contiguous

    for (uint32_t p = 0; p < npass; ++p) {
        const uint32_t kbase = p * kPassValues;
        const uint32_t kvals = min((uint32_t)kPassValues, K - kbase);
        const uint32_t g0 = kbase / gsz;
        const uint32_t gcnt = min(gpp, G - g0);
        __syncthreads();

        // ---- stage activations (as bf16 bits for DOT2, else as f32)
        for (uint32_t i = tid; i < (uint32_t)mcount * kvals; i += kThreads) {
            uint32_t m = i / kvals, kk = i - m * kvals;
            size_t src = (size_t)(m0 + m) * K + kbase + kk;
            if (DOT2) {
                ((uint16_t*)s_x)[m * kPassValues + kk] = ((const uint16_t*)op.x)[src];
            } else {
                ((float*)s_x)[m * kPassValues + kk] = load_as_f32(op.x, op.x_dt, src);
            }
        }
        // ---- stage (scale, bias_term) of the tile's rows for this pass
        for (uint32_t i = tid; i < (uint32_t)kRowsPerBlock * gcnt; i += kThreads) {
            uint32_t r, g;
            if (go_layout) {
                g = i / kRowsPerBlock;
                r = i - g * kRowsPerBlock;
            } else {
                r = i / gcnt;
                g = i - r * gcnt;
            }
            uint32_t w = s_wrow[r];
            float2 e = make_float2(0.0f, 0.0f);
            if (w != 0xffffffffu) {
                size_t md = (size_t)w * op.os + (size_t)(g0 + g) * op.gs;
                float s = load_as_f32(op.scales, op.w_dt, md);
                float bt;
                if (op.corr_kind == STARK_QMM_CORRECTION_BIASES) {
                    bt = load_as_f32(op.corr, op.w_dt, md);
                } else if (op.corr_kind == STARK_QMM_CORRECTION_ZERO_POINTS) {
                    size_t zi = (size_t)w * op.zos + (size_t)(g0 + g) * op.zgs;
                    uint32_t zb;
                    if (BITS == 4) {
                        uint32_t byte = ((const uint8_t*)op.corr)[zi >> 1];
                        zb = (zi & 1) ? (byte >> 4) & 15u : byte & 15u;
                    } else {
                        zb = ((const uint8_t*)op.corr)[zi];
                    }
                    bt = -s * (float)zb;
                } else {
                    bt = -s * midpoint;
                }
                if (DOT2) {
                    float s16 = 16.0f * s;
                    e = make_float2(s16, bt - s16);
                } else {
                    e = make_float2(s, bt);
                }
            }
            s_meta[r * gpp + g] = e;
        }
        __syncthreads();

        // ---- activation registers for this lane's chunks
        X xr;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const uint32_t c = lane + 64 * i;
                const bool ok = m < mcount && c * VPC < kvals;
                if (DOT2) {
                    uint32_t v[16];
                    if (ok) {
                        const uint4* src = (const uint4*)((const uint16_t*)s_x + m * kPassValues + c * 32);
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            uint4 t = src[q];
                            v[4 * q + 0] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
                        }
                    } else {
#pragma unroll
                        for (int q = 0; q < 16; ++q) v[q] = 0;
                    }
                    float s = 0.0f;
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        xr.v[m][i][4 * d + 0] = perm(v[4 * d + 2], v[4 * d + 0], 0x05040100u);
                        xr.v[m][i][4 * d + 1] = perm(v[4 * d + 2], v[4 * d + 0], 0x07060302u);
                        xr.v[m][i][4 * d + 2] = perm(v[4 * d + 3], v[4 * d + 1], 0x05040100u);
                        xr.v[m][i][4 * d + 3] = perm(v[4 * d + 3], v[4 * d + 1], 0x07060302u);
                    }
#pragma unroll
                    for (int q = 0; q < 16; ++q) s = dot2_bf16(v[q], 0x3F803F80u, s);
                    xr.sum[m][i] = s;
                } else {
                    const float* src = (const float*)s_x + m * kPassValues + c * VPC;
                    float s = 0.0f;
#pragma unroll
                    for (int q = 0; q < VPC; ++q) {
                        // 4-bit: per dword the unpack yields values in order 0,2,4,6,1,3,5,7
                        int srcq = q;
                        if (BITS == 4) {
                            int d = q / 8, e = q % 8;
                            srcq = 8 * d + (e < 4 ? 2 * e : 2 * (e - 4) + 1);
                        }
                        float xv = ok ? src[srcq] : 0.0f;
                        xr.v[m][i][q] = __float_as_uint(xv);
                        s += xv;
                    }
                    xr.sum[m][i] = s;
                }
            }
        }

        // ---- stream the wave's rows
        const uint8_t* pass_codes = op.codes + (size_t)kbase * BITS / 8;
#pragma unroll
        for (int rb = 0; rb < kRowsPerWave; rb += RBATCH) {
            u32x4 w[RBATCH][CPL];
#pragma unroll
            for (int r = 0; r < RBATCH; ++r) {
                const uint32_t wrow = s_wrow[wave * kRowsPerWave + rb + r];
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    const uint32_t c = lane + 64 * i;
                    if (wrow != 0xffffffffu && c * VPC < kvals) {
                        w[r][i] = load_stream(pass_codes + (size_t)wrow * row_bytes + (size_t)c * 16);
                    } else {
                        w[r][i] = u32x4{0, 0, 0, 0};
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < RBATCH; ++r) {
                const int row = wave * kRowsPerWave + rb + r;
#pragma unroll
                for (int i = 0; i < CPL; ++i) {
                    const uint32_t c = lane + 64 * i;
                    const uint32_t g = min((c * VPC) / gsz, gpp - 1);
                    const float2 e = s_meta[row * gpp + g];
                    uint32_t wd[4] = {w[r][i][0], w[r][i][1], w[r][i][2], w[r][i][3]};
                    if (op.flags & FLAG_SIGNED) {
#pragma unroll
                        for (int d = 0; d < 4; ++d) wd[d] ^= BITS == 4 ? 0x88888888u : 0x80808080u;
                    }
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        float dsum = 0.0f;
                        if (DOT2) {
#pragma unroll
                            for (int d = 0; d < 4; ++d) {
                                const uint32_t u = wd[d];
                                const uint32_t p0 = ((u << 3) & 0x00780078u) | 0x3F803F80u;
                                const uint32_t p1 = ((u >> 1) & 0x00780078u) | 0x3F803F80u;
                                const uint32_t p2 = ((u >> 5) & 0x00780078u) | 0x3F803F80u;
                                const uint32_t p3 = ((u >> 9) & 0x00780078u) | 0x3F803F80u;
                                dsum = dot2_bf16(p0, xr.v[m][i][4 * d + 0], dsum);
                                dsum = dot2_bf16(p1, xr.v[m][i][4 * d + 1], dsum);
                                dsum = dot2_bf16(p2, xr.v[m][i][4 * d + 2], dsum);
                                dsum = dot2_bf16(p3, xr.v[m][i][4 * d + 3], dsum);
                            }
                        } else if (BITS == 4) {
#pragma unroll
                            for (int d = 0; d < 4; ++d) {
                                const uint32_t lo = wd[d] & 0x0F0F0F0Fu;
                                const uint32_t hi = (wd[d] >> 4) & 0x0F0F0F0Fu;
                                const float* xv = (const float*)&xr.v[m][i][8 * d];
                                dsum = fmaf(ubyte<0>(lo), xv[0], dsum);
                                dsum = fmaf(ubyte<1>(lo), xv[1], dsum);
                                dsum = fmaf(ubyte<2>(lo), xv[2], dsum);
                                dsum = fmaf(ubyte<3>(lo), xv[3], dsum);
                                dsum = fmaf(ubyte<0>(hi), xv[4], dsum);
                                dsum = fmaf(ubyte<1>(hi), xv[5], dsum);
                                dsum = fmaf(ubyte<2>(hi), xv[6], dsum);
                                dsum = fmaf(ubyte<3>(hi), xv[7], dsum);
                            }
                        } else {
#pragma unroll
                            for (int d = 0; d < 4; ++d) {
                                const float* xv = (const float*)&xr.v[m][i][4 * d];
                                dsum = fmaf(ubyte<0>(wd[d]), xv[0], dsum);
                                dsum = fmaf(ubyte<1>(wd[d]), xv[1], dsum);
                                dsum = fmaf(ubyte<2>(wd[d]), xv[2], dsum);
                                dsum = fmaf(ubyte<3>(wd[d]), xv[3], dsum);
                            }
                        }
                        acc[rb + r][m] = fmaf(e.x, dsum, fmaf(e.y, xr.sum[m][i], acc[rb + r][m]));
                    }
                }
            }
        }
    }

    // ---- reduce across the wave and apply the D-ops (kernel.rs:270-281)
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int row = wave * kRowsPerWave + r;
        const uint32_t n = n0 + row;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = wave_sum(acc[r][m]);
            if (lane == 0 && n < N && m < mcount) {
                const size_t o = (size_t)(m0 + m) * N + n;
                if (s_wrow[row] == 0xffffffffu) {
                    store_from_f32(op.d, op.d_dt, o, __builtin_nanf(""));
                    continue;
                }
                v = op.ab_scale * v;
                if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
                if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
                if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
                store_from_f32(op.d, op.d_dt, o, v);
            }
        }
    }
}

template <int BITS, int MT, bool DOT2>
stark_qmm_status launch_fast(const AffineOp* ops, uint32_t count, hipStream_t stream) {
    AffineBatch batch{};
    uint32_t blocks = 0;
    size_t lds = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = ops[i];
        batch.op[i].block_begin = blocks;
        const uint32_t nrb = (ops[i].n + kRowsPerBlock - 1) / kRowsPerBlock;
        const uint32_t mt = ops[i].gather ? ops[i].m : (ops[i].m + MT - 1) / MT;
        blocks += nrb * mt;
        const size_t gpp = kPassValues / ops[i].group_size;
        const size_t need = 128 + kRowsPerBlock * gpp * sizeof(float2) +
                            (size_t)MT * kPassValues * (DOT2 ? 2 : 4);
        if (need > lds) lds = need;
    }
    batch.count = count;
    if (blocks == 0) return STARK_QMM_OK;
    hipLaunchKernelGGL((qmv_affine_fast<BITS, MT, DOT2>), dim3(blocks), dim3(kThreads), lds, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace

bool affine_fast_eligible(const AffineOp& op, int bits) {
    if (bits != 4 && bits != 8) return false;
    const uint32_t vpc = 128 / bits;
    if (op.k == 0 || op.k % vpc) return false;
    if (op.group_size % vpc || kPassValues % op.group_size) return false;
    if (((uintptr_t)op.codes & 15) || ((size_t)op.k * bits / 8) % 16) return false;
    return true;
}

stark_qmm_status launch_affine_generic(const AffineOp& op, int bits, hipStream_t stream) {
    if (op.n == 0 || op.m == 0) return STARK_QMM_OK;
    dim3 grid((op.n + 255) / 256, op.m);
    hipLaunchKernelGGL(qmv_affine_generic, grid, dim3(256), 0, stream, op, bits);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

stark_qmm_status launch_affine_materialized(const AffineOp& op, hipStream_t stream) {
    if (op.n == 0) return STARK_QMM_OK;
    hipLaunchKernelGGL(qmv_affine_materialized, dim3((op.n + 255) / 256), dim3(256), 0, stream, op);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

// ops: same bits; each op must be affine_fast_eligible. M per op arbitrary
// (weights are re-streamed once per pair of M rows).
stark_qmm_status launch_affine_gemv(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream) {
    if (count == 0) return STARK_QMM_OK;
    uint32_t max_m = 0;
    bool dot2 = true;
    for (uint32_t i = 0; i < count; ++i) {
        max_m = ops[i].m > max_m ? ops[i].m : max_m;
        if (ops[i].x_dt != STARK_QMM_BF16) dot2 = false;
        if (ops[i].gather) max_m = max_m > 1 ? max_m : 1;
    }
    bool gathered = false;
    for (uint32_t i = 0; i < count; ++i) gathered |= ops[i].gather != nullptr;
    const bool mt2 = max_m >= 2 && !gathered;
    for (uint32_t start = 0; start < count; start += kMaxBatchOps) {
        uint32_t c = count - start < (uint32_t)kMaxBatchOps ? count - start : (uint32_t)kMaxBatchOps;
        stark_qmm_status st;
        if (bits == 4) {
            if (dot2) st = mt2 ? launch_fast<4, 2, true>(ops + start, c, stream) : launch_fast<4, 1, true>(ops + start, c, stream);
            else st = mt2 ? launch_fast<4, 2, false>(ops + start, c, stream) : launch_fast<4, 1, false>(ops + start, c, stream);
        } else {
            st = mt2 ? launch_fast<8, 2, false>(ops + start, c, stream) : launch_fast<8, 1, false>(ops + start, c, stream);
        }
        if (st != STARK_QMM_OK) return st;
    }
    return STARK_QMM_OK;
}

}  // namespace qmm
