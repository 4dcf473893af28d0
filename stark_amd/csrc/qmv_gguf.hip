// GGUF block-format matvec (Q8_0 = kind 8, Q4_K = kind 12) on gfx950.
//
// Dequantisation is the reference's decode_block
// (crates/stark-engine/src/engine/hybrid/weights.rs:2923-3012):
//   Q8_0: w_i = f16(d) * int8(q_i)                          (32 values, 34 bytes)
//   Q4_K: w   = f16(d) * sc * q - f16(dmin) * m, (sc, m) = scale_min(scales, j)
//         (weights.rs:2908-2921), 8 sub-blocks of 32 values, 144 bytes
// Both products are exact in f32, so the factored per-block form
//   sum_i w_i x_i = d * sum_i q_i x_i              (Q8_0)
//   sum_j (d*sc_j) * sum_{i in j} q_i x_i - (dmin*m_j) * sum_{i in j} x_i   (Q4_K)
// reassociates only the additions, as the reference Metal kernels do
// (crates/stark-engine/src/engine/hybrid/packed_q8_grouped8_matvec.metal:11-82).
//
// Q4_K super-blocks are 16-byte aligned: lanes read them directly (8 lanes per
// super-block, one 16-byte quant piece each plus the shared 16-byte header).
// Q8_0 blocks are 34 bytes, so a tile of rows is first copied into LDS with
// 16-byte loads and each thread then decodes whole blocks from LDS.
#include "qmm_common.h"

namespace qmm {

namespace {

constexpr int kThreads = 256;
constexpr int kRows = 32;  // rows per workgroup tile

template <int B>
__device__ __forceinline__ float ubyte(uint32_t w) {
    return (float)((w >> (8 * B)) & 0xffu);
}

__device__ __forceinline__ uint32_t byte_of(const uint32_t* w, uint32_t i) { return (w[i >> 2] >> (8 * (i & 3))) & 0xffu; }

// weights.rs:2908-2921 on the 12 packed scale bytes held in 3 dwords.
__device__ __forceinline__ void scale_min(const uint32_t* s, uint32_t j, float* sc, float* mn) {
    if (j < 4) {
        *sc = (float)(byte_of(s, j) & 63u);
        *mn = (float)(byte_of(s, j + 4) & 63u);
    } else {
        *sc = (float)((byte_of(s, j + 4) & 15u) | ((byte_of(s, j - 4) >> 6) << 4));
        *mn = (float)((byte_of(s, j + 4) >> 4) | ((byte_of(s, j) >> 6) << 4));
    }
}

__device__ __forceinline__ const GgufOp& pick(const GgufBatch& b, uint32_t bid, GgufOp* tmp) {
    int oi = 0;
#pragma unroll
    for (int i = 1; i < kMaxBatchOps; ++i)
        if (i < (int)b.count && bid >= b.op[i].block_begin) oi = i;
    *tmp = b.op[0];
#pragma unroll
    for (int i = 1; i < kMaxBatchOps; ++i)
        if (oi == i) *tmp = b.op[i];
    return *tmp;
}

// ------------------------------------------------------------------ Q4_K
// Pass = 8 super-blocks (2048 values); lane = 8*sb + piece.
template <int MT>
__global__ __launch_bounds__(kThreads) void q4k_gemv(GgufBatch batch) {
    GgufOp tmp;
    const GgufOp& op = pick(batch, blockIdx.x, &tmp);
    const uint32_t N = op.n, K = op.k;
    const uint32_t nrb = (N + kRows - 1) / kRows;
    const uint32_t lb = blockIdx.x - op.block_begin;
    const uint32_t mtile = lb / nrb;
    const uint32_t n0 = (lb - mtile * nrb) * kRows;
    const uint32_t m0 = mtile * MT;
    const int mcount = min((int)MT, (int)(op.m - m0));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nsb = K / 256;
    const size_t row_bytes = (size_t)nsb * 144;
    const int sbl = lane >> 3, piece = lane & 7;
    const int part = piece >> 1;
    const int l0 = 16 * (piece & 1);
    const uint32_t j_lo = 2 * part, j_hi = 2 * part + 1;
    constexpr int RW = kRows / 4;

    float acc[RW][MT];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    for (uint32_t sb0 = 0; sb0 < nsb; sb0 += 8) {
        const uint32_t sb = sb0 + sbl;
        const bool ok = sb < nsb;
        // activations of this lane: 16 values for the low nibbles, 16 for the high
        float xl[MT][16], xh[MT][16], sl[MT], sh[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            sl[m] = sh[m] = 0.0f;
            const size_t base = (size_t)(m0 + m) * K + (size_t)sb * 256 + part * 64 + l0;
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const bool v = ok && m < mcount;
                xl[m][t] = v ? load_as_f32(op.x, op.x_dt, base + t) : 0.0f;
                xh[m][t] = v ? load_as_f32(op.x, op.x_dt, base + 32 + t) : 0.0f;
                sl[m] += xl[m][t];
                sh[m] += xh[m][t];
            }
        }
#pragma unroll 2
        for (int r = 0; r < RW; ++r) {
            const uint32_t n = n0 + wave * RW + r;
            if (n >= N || !ok) continue;
            const uint8_t* blk = op.blocks + (size_t)n * row_bytes + (size_t)sb * 144;
            const u32x4 hdr = load_stream(blk);
            const u32x4 q = load_stream(blk + 16 + 16 * piece);
            const float d = f16_bits_to_f32(hdr[0] & 0xffffu);
            const float dmin = f16_bits_to_f32(hdr[0] >> 16);
            const uint32_t sc3[3] = {hdr[1], hdr[2], hdr[3]};
            float sc_lo, m_lo, sc_hi, m_hi;
            scale_min(sc3, j_lo, &sc_lo, &m_lo);
            scale_min(sc3, j_hi, &sc_hi, &m_hi);
            const float dl = d * sc_lo, dh = d * sc_hi, ml = dmin * m_lo, mh = dmin * m_hi;
            const uint32_t qw[4] = {q[0], q[1], q[2], q[3]};
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float dot_lo = 0.0f, dot_hi = 0.0f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t lo = qw[w] & 0x0F0F0F0Fu, hi = (qw[w] >> 4) & 0x0F0F0F0Fu;
                    dot_lo = fmaf(ubyte<0>(lo), xl[m][4 * w + 0], dot_lo);
                    dot_lo = fmaf(ubyte<1>(lo), xl[m][4 * w + 1], dot_lo);
                    dot_lo = fmaf(ubyte<2>(lo), xl[m][4 * w + 2], dot_lo);
                    dot_lo = fmaf(ubyte<3>(lo), xl[m][4 * w + 3], dot_lo);
                    dot_hi = fmaf(ubyte<0>(hi), xh[m][4 * w + 0], dot_hi);
                    dot_hi = fmaf(ubyte<1>(hi), xh[m][4 * w + 1], dot_hi);
                    dot_hi = fmaf(ubyte<2>(hi), xh[m][4 * w + 2], dot_hi);
                    dot_hi = fmaf(ubyte<3>(hi), xh[m][4 * w + 3], dot_hi);
                }
                float a = acc[r][m];
                a = fmaf(dl, dot_lo, a);
                a = fmaf(-ml, sl[m], a);
                a = fmaf(dh, dot_hi, a);
                a = fmaf(-mh, sh[m], a);
                acc[r][m] = a;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const uint32_t n = n0 + wave * RW + r;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float v = wave_sum(acc[r][m]);
            if (lane == 0 && n < N && m < mcount) store_from_f32(op.d, op.d_dt, (size_t)(m0 + m) * N + n, v);
        }
    }
}

// ------------------------------------------------------------------ Q8_0
// Pass = 32 blocks (1024 values, 1088 bytes per row); the 32-row tile of the
// pass is staged in LDS (34 KiB) with 16-byte loads. Thread t decodes block
// t % 32 of rows t/32 + 8i.
constexpr int kQ8PassBlocks = 32;
constexpr int kQ8PassBytes = kQ8PassBlocks * 34;

template <int MT>
__global__ __launch_bounds__(kThreads) void q8_0_gemv(GgufBatch batch) {
    __shared__ __align__(16) uint32_t tile[kRows * kQ8PassBytes / 4];
    GgufOp tmp;
    const GgufOp& op = pick(batch, blockIdx.x, &tmp);
    const uint32_t N = op.n, K = op.k;
    const uint32_t nrb = (N + kRows - 1) / kRows;
    const uint32_t lb = blockIdx.x - op.block_begin;
    const uint32_t mtile = lb / nrb;
    const uint32_t n0 = (lb - mtile * nrb) * kRows;
    const uint32_t m0 = mtile * MT;
    const int mcount = min((int)MT, (int)(op.m - m0));
    const int tid = threadIdx.x;
    const uint32_t nb = K / 32;
    const size_t row_bytes = (size_t)nb * 34;
    const int b = tid & 31;
    const int r0 = tid >> 5;

    float acc[4][MT];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[i][m] = 0.0f;

    for (uint32_t blk0 = 0; blk0 < nb; blk0 += kQ8PassBlocks) {
        const uint32_t nblk = min((uint32_t)kQ8PassBlocks, nb - blk0);
        const uint32_t pass_bytes = nblk * 34;  // multiple of 16 when nblk % 8 == 0
        const uint32_t vecs = (pass_bytes + 15) / 16;
        __syncthreads();
        for (uint32_t i = tid; i < kRows * vecs; i += kThreads) {
            const uint32_t r = i / vecs, v = i - r * vecs;
            const uint32_t n = n0 + r;
            u32x4 val = {0, 0, 0, 0};
            if (n < N) val = load_stream(op.blocks + (size_t)n * row_bytes + (size_t)blk0 * 34 + (size_t)v * 16);
            *(u32x4*)(tile + (r * kQ8PassBytes + v * 16) / 4) = val;
        }
        __syncthreads();
        const bool ok = (uint32_t)b < nblk;
        float x[MT][32], xs[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            xs[m] = 0.0f;
            const size_t base = (size_t)(m0 + m) * K + (size_t)(blk0 + b) * 32;
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                x[m][t] = (ok && m < mcount) ? load_as_f32(op.x, op.x_dt, base + t) : 0.0f;
                xs[m] += x[m][t];
            }
        }
        if (!ok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = r0 + 8 * i;
            const uint32_t off = r * kQ8PassBytes + b * 34;  // byte offset; even
            const uint32_t* p = tile + (off >> 2);
            uint32_t dw[9];
#pragma unroll
            for (int q = 0; q < 9; ++q) dw[q] = p[q];
            float d;
            uint32_t qs[8];
            if ((off & 3) == 0) {
                d = f16_bits_to_f32(dw[0] & 0xffffu);
#pragma unroll
                for (int q = 0; q < 8; ++q) qs[q] = __builtin_amdgcn_alignbyte(dw[q + 1], dw[q], 2);
            } else {
                d = f16_bits_to_f32(dw[0] >> 16);
#pragma unroll
                for (int q = 0; q < 8; ++q) qs[q] = dw[q + 1];
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                // signed bytes: q = u - 128 with u = byte ^ 0x80
                float dot = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t u = qs[q] ^ 0x80808080u;
                    dot = fmaf(ubyte<0>(u), x[m][4 * q + 0], dot);
                    dot = fmaf(ubyte<1>(u), x[m][4 * q + 1], dot);
                    dot = fmaf(ubyte<2>(u), x[m][4 * q + 2], dot);
                    dot = fmaf(ubyte<3>(u), x[m][4 * q + 3], dot);
                }
                dot = fmaf(-128.0f, xs[m], dot);
                acc[i][m] = fmaf(d, dot, acc[i][m]);
            }
        }
    }
    // reduce the 32 block-threads of each row (lanes b = 0..31 of a half-wave)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t n = n0 + r0 + 8 * i;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            float v = acc[i][m];
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
            if (b == 0 && n < N && m < mcount) store_from_f32(op.d, op.d_dt, (size_t)(m0 + m) * N + n, v);
        }
    }
}

// Any row layout / any K: one thread per output, the reference's order
// (decode_values then a sequential f32 sum, weights.rs:2533-2550).
__global__ void gguf_generic(GgufOp op) {
    const uint32_t n = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t m = blockIdx.y;
    if (n >= op.n || m >= op.m) return;
    const uint32_t be = op.kind == 8 ? 32 : 256, bb = op.kind == 8 ? 34 : 144;
    const size_t row_bytes = (size_t)(op.k / be) * bb;
    const uint8_t* row = op.blocks + (size_t)n * row_bytes;
    float s = -0.0f;
    for (uint32_t blk = 0; blk < op.k / be; ++blk) {
        const uint8_t* p = row + (size_t)blk * bb;
        const float d = f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
        const size_t xb = (size_t)m * op.k + (size_t)blk * be;
        if (op.kind == 8) {
            for (int i = 0; i < 32; ++i) {
                const float w = __fmul_rn(d, (float)(int8_t)p[2 + i]);
                s = __fadd_rn(s, __fmul_rn(w, load_as_f32(op.x, op.x_dt, xb + i)));
            }
        } else {
            const float dmin = f16_bits_to_f32((uint32_t)p[2] | ((uint32_t)p[3] << 8));
            uint32_t sc3[3];
            for (int i = 0; i < 3; ++i)
                sc3[i] = (uint32_t)p[4 + 4 * i] | ((uint32_t)p[5 + 4 * i] << 8) | ((uint32_t)p[6 + 4 * i] << 16) |
                         ((uint32_t)p[7 + 4 * i] << 24);
            for (int part = 0; part < 4; ++part)
                for (int half = 0; half < 2; ++half) {
                    float sc, mn;
                    scale_min(sc3, part * 2 + half, &sc, &mn);
                    for (int l = 0; l < 32; ++l) {
                        const float q = (float)((p[16 + part * 32 + l] >> (4 * half)) & 15);
                        const float w = __fsub_rn(__fmul_rn(__fmul_rn(d, sc), q), __fmul_rn(dmin, mn));
                        s = __fadd_rn(s, __fmul_rn(w, load_as_f32(op.x, op.x_dt, xb + part * 64 + half * 32 + l)));
                    }
                }
        }
    }
    store_from_f32(op.d, op.d_dt, (size_t)m * op.n + n, s);
}

template <typename F>
stark_qmm_status launch_batched(const GgufOp* ops, uint32_t count, int mt, F launch) {
    GgufBatch batch{};
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = ops[i];
        batch.op[i].block_begin = blocks;
        blocks += ((ops[i].n + kRows - 1) / kRows) * ((ops[i].m + mt - 1) / mt);
    }
    batch.count = count;
    if (blocks) launch(batch, blocks);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

bool fast_eligible(const GgufOp& o) {
    if (((uintptr_t)o.blocks & 15) != 0) return false;
    if (o.kind == 12) return o.k % 256 == 0;
    return o.k % 256 == 0;  // Q8_0: rows of 8-block multiples stay 16-byte aligned
}

}  // namespace

bool gguf_supported(uint32_t kind) { return kind == 8 || kind == 12; }

stark_qmm_status launch_gguf_gemv(const GgufOp* ops, uint32_t count, hipStream_t stream) {
    std::vector<GgufOp> q4, q8;
    for (uint32_t i = 0; i < count; ++i) {
        GgufOp o = ops[i];
        if (o.x_dt == 0 && o.d_dt == 0) {
            o.x_dt = STARK_QMM_F32;
            o.d_dt = STARK_QMM_F32;
        }
        if (o.n == 0 || o.m == 0) continue;
        if (!fast_eligible(o)) {
            hipLaunchKernelGGL(gguf_generic, dim3((o.n + 255) / 256, o.m), dim3(256), 0, stream, o);
            QMM_HIP_CHECK(hipGetLastError());
            continue;
        }
        (o.kind == 12 ? q4 : q8).push_back(o);
    }
    for (int kind : {12, 8}) {
        std::vector<GgufOp>& v = kind == 12 ? q4 : q8;
        for (size_t s = 0; s < v.size(); s += kMaxBatchOps) {
            const uint32_t c = (uint32_t)std::min<size_t>(kMaxBatchOps, v.size() - s);
            bool mt2 = false;
            for (uint32_t i = 0; i < c; ++i) mt2 |= v[s + i].m >= 2;
            const int mt = mt2 ? 2 : 1;
            stark_qmm_status st = launch_batched(v.data() + s, c, mt, [&](const GgufBatch& b, uint32_t blocks) {
                if (kind == 12) {
                    if (mt2) hipLaunchKernelGGL(q4k_gemv<2>, dim3(blocks), dim3(kThreads), 0, stream, b);
                    else hipLaunchKernelGGL(q4k_gemv<1>, dim3(blocks), dim3(kThreads), 0, stream, b);
                } else {
                    if (mt2) hipLaunchKernelGGL(q8_0_gemv<2>, dim3(blocks), dim3(kThreads), 0, stream, b);
                    else hipLaunchKernelGGL(q8_0_gemv<1>, dim3(blocks), dim3(kThreads), 0, stream, b);
                }
            });
            if (st != STARK_QMM_OK) return st;
        }
    }
    return STARK_QMM_OK;
}

}  // namespace qmm
