// Decode-shaped 4-bit affine matvec (M <= 2, bf16 activations) on gfx950.
//
// Arithmetic: per group g of a weight row,
//   s*sum(x*q) + b*sum(x) = (16s * sum x*(1 + q/16) - 16s * sum x) + b * sum x
// where (1 + q/16) is a bf16 built from a code nibble by one shift and one
// v_and_or_b32, and the sums run on v_dot2_f32_bf16 (exact bf16 products, f32
// accumulation). This reassociates only additions of the reference's per-element
// loop (crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:185-268).
//
// Schedule: every wave64 is independent (no LDS, no barriers). A wave owns 8
// consecutive weight rows over the whole K axis, walked in passes of 4096 values;
// in a pass lane L owns 16-byte code chunks L and L+64, so each load instruction
// reads 1 KiB contiguous of a row. The (scale, bias) of the 8 rows of one group
// are 16 contiguous bytes in the converter's group-output planes [G][N], so a
// lane fetches them with one 16-byte load per plane; activations come straight
// from L1/L2. All loads of a pass are issued before any arithmetic.
//
// Eligibility (decode_eligible): 4-bit codes, bf16 activations, no gather,
// biases or symmetric correction, bf16/f16 group-output planes, N % 8 == 0,
// 16-byte aligned buffers, M <= 2.
#include "qmm_common.h"

namespace qmm {

namespace {

constexpr int kWgThreads = 512;  // 8 waves
constexpr int kWaveRows = 4;
constexpr int kTileRows = kWaveRows * kWgThreads / 64;  // 32
constexpr int kPass = 4096;
constexpr int kCpl = 2;  // 16-byte code chunks per lane per pass

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// (a & mask) | orv as one v_and_or_b32. Volatile keeps these in program
// order, so the scheduler cannot hoist every item's unpack ahead of its use
// (which it does to non-volatile asm, with a large register cost).
__device__ __forceinline__ uint32_t and_or_v(uint32_t a, uint32_t mask, uint32_t orv) {
    uint32_t r;
    asm volatile("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(mask), "v"(orv));
    return r;
}

// 16-bit float bits -> f32 (bf16: shift; f16: hardware convert)
template <bool BF>
__device__ __forceinline__ float h2f(uint32_t h) {
    return BF ? __uint_as_float(h << 16) : f16_bits_to_f32(h);
}


// LDS per workgroup: (16s, bias term) per (tile row, group of the pass),
// activation pairs stored [d][chunk] (16-byte units) so that a wave reading
// vector d of chunks L, L+64 touches consecutive addresses, and chunk sums.
template <int MT>
struct DecodeLds {
    float2 meta[kTileRows][kPass / 32];  // sized for the smallest group (32)
    u32x4 xp[MT][4][kPass / 32];
    float xs[MT][kPass / 32];
};

template <int MT, bool SIGNED, bool BIASED, bool BF_PLANES>
__global__ __launch_bounds__(kWgThreads) void qmv_w4_decode(AffineBatch batch) {
    (void)batch;
    __shared__ DecodeLds<MT> lds;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t bid = blockIdx.x;
    uint32_t oi = 0;
    for (uint32_t i = 1; i < kb->count; ++i)
        if (bid >= kb->op[i].block_begin) oi = i;
    const AffineOp& op = kb->op[oi];
    const uint32_t N = op.n, K = op.k;
    // the last tile of an op is moved back to end at N (N % 8 == 0, N >= 32); its
    // leading rows repeat the previous tile and are not stored again
    const uint32_t t0 = (bid - op.block_begin) * kTileRows;
    const uint32_t n0 = min(t0, N - kTileRows);
    const uint32_t wrow0 = n0 + wave * kWaveRows;
    const size_t row_bytes = (size_t)K / 2;
    const uint32_t gsz = op.group_size;
    const uint32_t gshift = 31 - __builtin_clz(gsz);
    const uint32_t gpp = kPass >> gshift;  // groups per pass
    // nibble mask and bf16 1.0 pair from kernel arguments: SGPR operands, so each
    // unpack is a shift plus v_and_or_b32 / v_and + v_or without literals
    const uint32_t nib = kb->nib_mask;
    const uint32_t one2 = kb->nib_one;

    float acc[kWaveRows][MT];
#pragma unroll
    for (int r = 0; r < kWaveRows; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

    const uint8_t* codes = op.codes + (size_t)wrow0 * row_bytes;
    for (uint32_t kbase = 0; kbase < K; kbase += kPass) {
        const uint32_t kvals = min((uint32_t)kPass, K - kbase);
        const uint32_t g0 = kbase >> gshift;
        const uint32_t gcnt = min(gpp, (K >> gshift) - g0);
        // ---- 1. this wave's codes: the HBM stream starts before any staging
        u32x4 w[kCpl][kWaveRows];
#pragma unroll
        for (int i = 0; i < kCpl; ++i) {
            const uint32_t c = lane + 64 * i;
            const bool ok = c * 32 < kvals;
#pragma unroll
            for (int r = 0; r < kWaveRows; ++r)
                w[i][r] = ok ? load_stream(codes + (size_t)r * row_bytes + kbase / 2 + (size_t)c * 16)
                             : u32x4{0, 0, 0, 0};
        }
        if (kbase) __syncthreads();  // the previous pass is done reading LDS
        // ---- 2. staging: threads [0, 4*gcnt) take (group, 8-row block) metadata
        //      vectors, the rest take activation vectors (8 values each)
        {
            const uint32_t nmeta = gcnt * (kTileRows / 8);
            if ((uint32_t)tid < nmeta) {
                const uint32_t g = tid >> 2, r8 = (tid & 3) * 8;
                const size_t off = (size_t)(g0 + g) * op.gs + n0 + r8;
                const u32x4 sv = *(const u32x4*)((const uint16_t*)op.scales + off);
                u32x4 bv = u32x4{0, 0, 0, 0};
                if (BIASED) bv = *(const u32x4*)((const uint16_t*)op.corr + off);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float sc = h2f<BF_PLANES>((sv[e >> 1] >> (16 * (e & 1))) & 0xffffu);
                    const float s16 = 16.0f * sc;
                    const float b = BIASED ? h2f<BF_PLANES>((bv[e >> 1] >> (16 * (e & 1))) & 0xffffu)
                                           : -8.0f * sc;  // symmetric: -s * 2^(bits-1)
                    lds.meta[r8 + e][g] = make_float2(s16, b);
                }
            }
            // activations: MT * 512 vectors over all threads
            for (uint32_t v = tid; v < MT * (kPass / 8); v += kWgThreads) {
                const uint32_t m = v / (kPass / 8), vi = v % (kPass / 8);  // vi: chunk vi/4, dword vi%4
                u32x4 t = u32x4{0, 0, 0, 0};
                if (m < op.m && vi * 8 < kvals)
                    t = *(const u32x4*)((const uint16_t*)op.x + (size_t)m * K + kbase + vi * 8);
                u32x4 pq;
                pq[0] = perm(t[2], t[0], 0x05040100u);  // (x0, x4)
                pq[1] = perm(t[2], t[0], 0x07060302u);  // (x1, x5)
                pq[2] = perm(t[3], t[1], 0x05040100u);  // (x2, x6)
                pq[3] = perm(t[3], t[1], 0x07060302u);  // (x3, x7)
                lds.xp[m][vi & 3][vi >> 2] = pq;
                float sm = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) sm = dot2_bf16(t[e], 0x3F803F80u, sm);
                sm = group_sum<4>(sm);  // the 4 vectors of a chunk are 4 consecutive lanes
                if ((vi & 3) == 0) lds.xs[m][vi >> 2] = sm;
            }
        }
        __syncthreads();
        // ---- 3. dot products, chunk by chunk
#pragma unroll
        for (int i = 0; i < kCpl; ++i) {
            const uint32_t c = lane + 64 * i;
            const uint32_t g = min((c * 32) >> gshift, gcnt - 1);
            uint32_t xr[MT][16];
            float xs[MT];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const u32x4 t = lds.xp[m][q][c];
#pragma unroll
                    for (int e = 0; e < 4; ++e) xr[m][4 * q + e] = t[e];
                }
                xs[m] = lds.xs[m][c];
            }
#pragma unroll
            for (int r = 0; r < kWaveRows; ++r) {
                const float2 e = lds.meta[wave * kWaveRows + r][g];
                uint32_t pr[4][4];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    uint32_t u = w[i][r][d];
                    if (SIGNED) u ^= 0x88888888u;
                    pr[d][0] = ((u << 3) & nib) | one2;
                    pr[d][1] = ((u >> 1) & nib) | one2;
                    pr[d][2] = ((u >> 5) & nib) | one2;
                    pr[d][3] = ((u >> 9) & nib) | one2;
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    float d0 = dot2_bf16(pr[0][0], xr[m][0], 0.0f);
                    float d1 = dot2_bf16(pr[1][0], xr[m][4], 0.0f);
#pragma unroll
                    for (int q = 1; q < 4; ++q) {
                        d0 = dot2_bf16(pr[0][q], xr[m][q], d0);
                        d1 = dot2_bf16(pr[1][q], xr[m][4 + q], d1);
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        d0 = dot2_bf16(pr[2][q], xr[m][8 + q], d0);
                        d1 = dot2_bf16(pr[3][q], xr[m][12 + q], d1);
                    }
                    // (16s * sum x(1 + q/16) - 16s * sum x) is s * sum x*q exactly for
                    // a single term, so a one-hot row yields s*q + b with one
                    // rounding, the reference's dequantised weight
                    acc[r][m] = fmaf(e.y, xs[m], fmaf(e.x, d0 + d1, fmaf(-e.x, xs[m], acc[r][m])));
                }
            }
        }
    }

    // ---- reduce the 4 rows across the wave; one lane per row applies the D-ops
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const bool h32 = lane & 32, h16 = lane & 16;
        const float a0 = (h32 ? acc[2][m] : acc[0][m]) + __shfl_xor(h32 ? acc[0][m] : acc[2][m], 32, 64);
        const float a1 = (h32 ? acc[3][m] : acc[1][m]) + __shfl_xor(h32 ? acc[1][m] : acc[3][m], 32, 64);
        float b = (h16 ? a1 : a0) + __shfl_xor(h16 ? a0 : a1, 16, 64);
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) b += __shfl_xor(b, off, 64);
        const uint32_t rrow = ((lane >> 5) & 1) * 2 + ((lane >> 4) & 1);
        const uint32_t n = wrow0 + rrow;
        if ((lane & 15) == 0 && m < (int)op.m && n >= t0) {
            const size_t o = (size_t)m * N + n;
            float v = op.ab_scale * b;
            if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
            if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
            if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
            store_from_f32(op.d, op.d_dt, o, v);
        }
    }
}

template <int MT, bool SIGNED, bool BIASED, bool BF>
stark_qmm_status launch_decode(const AffineOp* ops, uint32_t count, hipStream_t stream) {
    AffineBatch batch{};
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = ops[i];
        batch.op[i].block_begin = blocks;
        blocks += (ops[i].n + kTileRows - 1) / kTileRows;
    }
    batch.count = count;
    batch.total = blocks;
    batch.nib_mask = 0x00780078u;
    batch.nib_one = 0x3F803F80u;
    if (blocks == 0) return STARK_QMM_OK;
    hipLaunchKernelGGL((qmv_w4_decode<MT, SIGNED, BIASED, BF>), dim3(blocks), dim3(kWgThreads), 0, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

template <int MT, bool SIGNED>
stark_qmm_status launch_decode_corr(const AffineOp* o, uint32_t c, hipStream_t stream) {
    const bool biased = o[0].corr_kind == STARK_QMM_CORRECTION_BIASES;
    const bool bf = o[0].w_dt == STARK_QMM_BF16;
    if (biased) return bf ? launch_decode<MT, SIGNED, true, true>(o, c, stream) : launch_decode<MT, SIGNED, true, false>(o, c, stream);
    return bf ? launch_decode<MT, SIGNED, false, true>(o, c, stream) : launch_decode<MT, SIGNED, false, false>(o, c, stream);
}

}  // namespace

bool decode_eligible(const AffineOp& o, int bits) {
    if (bits != 4 || o.x_dt != STARK_QMM_BF16 || o.gather || o.m == 0 || o.m > 2) return false;
    if (!(o.corr_kind == STARK_QMM_CORRECTION_BIASES || o.corr_kind == STARK_QMM_CORRECTION_SYMMETRIC)) return false;
    if (o.w_dt == STARK_QMM_F32) return false;
    if (o.group_size != 32 && o.group_size != 64 && o.group_size != 128) return false;
    if (o.k == 0 || o.k % 32 || o.n < (uint32_t)kTileRows || o.n % 8) return false;
    if (((uintptr_t)o.codes | (uintptr_t)o.x | (uintptr_t)o.scales) & 15) return false;
    if (o.corr_kind == STARK_QMM_CORRECTION_BIASES && ((uintptr_t)o.corr & 15)) return false;
    return o.os == 1 && o.gs % 8 == 0;  // group-output planes [G][N4]
}

// ops: all decode_eligible; one launch per (M class, signedness, correction, plane type).
stark_qmm_status launch_affine_decode(const AffineOp* ops, uint32_t count, hipStream_t stream) {
    std::vector<AffineOp> cls[2][2][2][2];
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        cls[o.m >= 2][(o.flags & FLAG_SIGNED) != 0][o.corr_kind == STARK_QMM_CORRECTION_BIASES]
           [o.w_dt == STARK_QMM_BF16].push_back(o);
    }
    for (int mt = 0; mt < 2; ++mt)
        for (int sg = 0; sg < 2; ++sg)
            for (int bi = 0; bi < 2; ++bi)
                for (int bf = 0; bf < 2; ++bf) {
                    const std::vector<AffineOp>& v = cls[mt][sg][bi][bf];
                    for (size_t s = 0; s < v.size(); s += kMaxBatchOps) {
                        const uint32_t c = (uint32_t)std::min<size_t>(kMaxBatchOps, v.size() - s);
                        const AffineOp* o = v.data() + s;
                        stark_qmm_status st;
                        if (mt) st = sg ? launch_decode_corr<2, true>(o, c, stream) : launch_decode_corr<2, false>(o, c, stream);
                        else st = sg ? launch_decode_corr<1, true>(o, c, stream) : launch_decode_corr<1, false>(o, c, stream);
                        if (st != STARK_QMM_OK) return st;
                    }
                }
    return STARK_QMM_OK;
}

}  // namespace qmm
