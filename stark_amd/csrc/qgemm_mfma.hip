// Prefill dequant-GEMM (M > 16) for MLX-affine 4/8-bit weights on the gfx950
// matrix cores: D[M,N] = X[M,K] * W[N,K]^T with W dequantised per tile.
//
// Reference: the Metal GEMM with its dequantising B loader
// (crates/stark-engine/src/backends/metal/kernel/matmul/gemm/gemm.metal:122-203,
// gemm/common/quant_scale_bias.h:23-138) dequantises each B tile into
// threadgroup memory in the activation type and multiplies there; the CPU
// twin of that rounding is reference_affine_linear_bf16
// (backends/cpu/kernel/matmul/vision.rs:249-336): w = bf16_rne(f32(q)*s + b).
// Here: a workgroup (8 waves) owns a 256x128, 128x128 or 128x64 output tile; per
// 64-wide K step the X tile is staged in LDS as is and the W tile is
// dequantised into LDS as bf16 (w = s*q + bias_term rounded to nearest even),
// double-buffered so the next steps' global loads overlap the current step's
// v_mfma_f32_16x16x32_bf16 work (each wave: a 64x64 block = 4x4 MFMA tiles,
// 32 MFMAs per K step, or 32x64 / 32x32 in the 128-row tiles). The
// D-ops (ab_scale, accumulate, bias, soft-cap) and the output rounding follow
// kernel.rs:270-281.
#include "qmm_common.h"

namespace qmm {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Tiles of BM rows (256, or 128 for products of at most kBM128Rows rows) x
// BN columns (128, or 64 for products of at most kBN64Rows rows), eight
// waves each; kBM and kBN are the largest.
constexpr int kBM = 256, kBN = 128, kBK = 64, kThreads = 512;
// Products of few rows have few tiles, and the serial K loop of the deepest
// (the Qwen3-8B down product's, K = 12288) sets their time. The 128-row
// tile keeps eight waves (two per SIMD, so one wave's dequantisation and LDS
// traffic overlap the other's MFMAs) and three register stages of loads in
// flight. Qwen3-8B set at 65 / 128 / 256 / 384 rows: 161 / 165 / 183 / 240
// us with 256-row tiles above 128 rows and 128-row tiles of four waves and
// two stages; 124 / 132 / 153 / 223 us now (eight waves alone 135 / 150 at
// 65 / 128; four or six stages 128-136; three stages in the 256-row tile
// lost 6% at 256 and 2048 rows). From 512 rows the 256-row tile is faster.
// Up to 128 rows, 64-column tiles halve each step's dequantisation and MFMA
// work and double the tiles: 125 / 134 -> 97 / 112 us at 65 / 128 rows
// (151 -> 169 us at 256 rows, where the 128-column tile stays).
constexpr uint32_t kBM128Rows = 384, kBN64Rows = 128;
__host__ __device__ constexpr uint32_t gemm_bm(uint32_t m) { return m <= kBM128Rows ? 128 : 256; }
__host__ __device__ constexpr uint32_t gemm_bn(uint32_t m) { return m <= kBN64Rows ? 64 : 128; }

// LDS tiles: rows of 64 bf16 (128 bytes, 8 chunks of 16 bytes), chunk c of
// row r stored at chunk c ^ (r & 7). Every access here moves 16 bytes per
// lane, and any 8 consecutive lanes then cover all 32 banks once: the MFMA
// operand reads (rows r..r+7, one chunk), the X stores (one row, 8 chunks)
// and the dequantised W stores (4 rows x 2 chunks). (Measured against
// c ^ ((r >> 1) & 7), which spreads 16 lanes over 64 banks: 611 vs 604
// TFLOP/s on the Qwen3-8B prefill set; 144-byte padded rows: 597.)
template <int BM, int BN>
struct GemmLds {
    u32x4 a[2][BM][kBK / 8];
    u32x4 b[2][BN][kBK / 8];
};
__device__ __forceinline__ uint32_t swz(uint32_t r, uint32_t c) { return c ^ (r & 7); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t gemm_rsrc(const void* p, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)min(bytes, (uint64_t)0x7fffffffu), 0x00020000);
}

// Output tile (bx, by) of one product: columns BN bx.., rows BM by...
// BITS: 4 or 8. CORR: 0 symmetric, 1 biases. BF: bf16 (else f16) planes.
template <int BITS, int CORR, bool SIGNED, bool BF, int BM, int BN>
__device__ __forceinline__ void gemm_tile(const AffineOp& op, uint32_t bx, uint32_t by) {
    constexpr int XI = BM * 8 / kThreads;  // X chunks per thread
    constexpr int MI = BM / 64;            // 16-row blocks per wave
    constexpr int NS = BM == 128 ? 3 : 2;  // register stages of loads
    constexpr int MJ = BN / 32;            // 16-column blocks per wave
    __shared__ GemmLds<BM, BN> lds;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t M = op.m, N = op.n, K = op.k;
    const uint32_t m0 = by * BM, n0 = bx * BN;
    const uint32_t row_bytes = K * BITS / 8;

    // ---- per-thread load assignment
    // X tile [BM][64] bf16: XI x 16 B per thread (row v / 8, column 8 * (v % 8)).
    // W tile: BN rows x (64*BITS/8) bytes, 4 threads per row, 16 codes each
    // (8 bytes of 4-bit codes, 16 of 8-bit; 64-column tiles: 8 threads per
    // row, 8 codes each). Each dequantised weight serves the
    // tile's 256 rows: against 128x128 tiles of four waves (two workgroups per
    // CU), half the dequantisation per MFMA, 869-871 vs 792-795 TFLOP/s on the
    // Qwen3-8B prefill set.
    constexpr int CB = BN * kBK * BITS / 8 / kThreads;  // code bytes per thread
    constexpr int WPT = (CB > 16 ? 16 : CB) * 8 / BITS;  // codes per thread per pass
    constexpr int TPR = kBK / WPT;                       // threads per row
    constexpr int WPASS = CB > 16 ? CB / 16 : 1;         // passes over the rows
    constexpr int WW = WPT * BITS / 32;  // code words per thread
    struct Stage {
        u32x4 xa[XI];
        uint32_t wc[WPASS][4];
        float ws[WPASS], wb[WPASS];
    };

    // Buffer loads with per-thread offsets fixed here (the step adds k0):
    // X rows past M and W rows past N lie past their resources and read
    // zeros (with no branch around the load); a W row past N takes its plane
    // entries from row N - 1 (its outputs are never stored). The plane group
    // of a thread's codes is k0 / gs + (its offset in the step) / gs: group
    // sizes are 32, 64 or 128 and k0 a multiple of 64. A step reads 32 bytes
    // (4-bit) or 64 bytes (8-bit) of each W row's 128-byte line and the next
    // steps the rest, so the W loads are ordinary (cached) loads: with the
    // nontemporal hint L2 dropped the line between steps and fetched it again
    // (Qwen3-8B set: 253 -> 167 MB fetched at 128 rows, 115 -> 102 us; 929 ->
    // 993 TFLOP/s at 2048 rows).
    const __amdgpu_buffer_rsrc_t rx = gemm_rsrc(op.x, (uint64_t)M * K * 2);
    const __amdgpu_buffer_rsrc_t rw = gemm_rsrc(op.codes, (uint64_t)N * row_bytes);
    const __amdgpu_buffer_rsrc_t rs = gemm_rsrc(op.scales, 0x7fffffffu);
    const __amdgpu_buffer_rsrc_t rb = gemm_rsrc(op.corr, 0x7fffffffu);
    const uint32_t lgs = 31 - __builtin_clz(op.group_size);
    uint32_t xo[XI], wo[WPASS], po[WPASS];
#pragma unroll
    for (int i = 0; i < XI; ++i) {
        const uint32_t v = tid + kThreads * i, r = v / 8, c = (v % 8) * 8;
        xo[i] = ((m0 + r) * K + c) * 2;
    }
#pragma unroll
    for (int p = 0; p < WPASS; ++p) {
        const uint32_t v = tid + kThreads * p, r = v / TPR, part = v % TPR;
        const uint32_t n = n0 + r;
        wo[p] = n * row_bytes + part * WPT * BITS / 8;
        po[p] = (min(n, N - 1) * op.os + ((part * WPT) >> lgs) * op.gs) * 2;
    }
    auto load_step = [&](Stage& st, uint32_t k0) {
#pragma unroll
        for (int i = 0; i < XI; ++i)
            st.xa[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i] + k0 * 2, 0, 0));
        const uint32_t pg = (k0 >> lgs) * op.gs * 2;  // bytes of the step's first plane group
#pragma unroll
        for (int p = 0; p < WPASS; ++p) {
            if constexpr (WW == 1) {
                st.wc[p][0] = __builtin_amdgcn_raw_buffer_load_b32(rw, wo[p] + k0 * BITS / 8, 0, 0);
                st.wc[p][1] = st.wc[p][2] = st.wc[p][3] = 0;
            } else if constexpr (WW == 4) {
                const u32x4 t = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, wo[p] + k0 * BITS / 8, 0, 0));
                st.wc[p][0] = t[0]; st.wc[p][1] = t[1]; st.wc[p][2] = t[2]; st.wc[p][3] = t[3];
            } else {
                typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
                const u32x2v t = __builtin_bit_cast(u32x2v, __builtin_amdgcn_raw_buffer_load_b64(rw, wo[p] + k0 * BITS / 8, 0, 0));
                st.wc[p][0] = t[0]; st.wc[p][1] = t[1]; st.wc[p][2] = 0; st.wc[p][3] = 0;
            }
            const uint32_t hs = __builtin_amdgcn_raw_buffer_load_b16(rs, po[p], pg, 0);
            st.ws[p] = BF ? bf16_bits_to_f32(hs) : f16_bits_to_f32(hs);
            if (CORR == 1) {
                const uint32_t hb = __builtin_amdgcn_raw_buffer_load_b16(rb, po[p], pg, 0);
                st.wb[p] = BF ? bf16_bits_to_f32(hb) : f16_bits_to_f32(hb);
            } else {
                st.wb[p] = 0.0f;
            }
        }
    };
    // X to LDS as is; W dequantised: w = s*q + bias_term (exact in f32: bf16/f16
    // s times a <= 8-bit q), rounded to bf16 by v_cvt_pk_bf16_f32 (nearest even).
    auto store_step = [&](const Stage& st, int buf) {
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t v = tid + kThreads * i, r = v / 8, c = (v % 8) * 8;
            lds.a[buf][r][swz(r, c / 8)] = st.xa[i];
        }
#pragma unroll
        for (int p = 0; p < WPASS; ++p) {
            const uint32_t v = tid + kThreads * p, r = v / TPR, part = v % TPR;
            // (never true with kThreads threads; the compiler cannot tell, and the
            // branch keeps the dequantisation below the MFMA block in its
            // schedule: removing it measured 746 vs 791-797 TFLOP/s, a
            // sched_barrier in its place 712-721, with 128x128 tiles)
            if (r >= (uint32_t)BN) continue;
            const float s = st.ws[p];
            // bias term: biases, or -s * 2^(bits-1) for the symmetric correction
            const float b = CORR == 1 ? st.wb[p] : -s * (float)(1 << (BITS - 1));
            uint32_t bytes[WPT / 4];  // code e of this thread sits in byte e % 4 of bytes[e / 4]
#pragma unroll
            for (int d = 0; d < WW; ++d) {
                uint32_t u = st.wc[p][d];
                if (BITS == 4) {
                    if (SIGNED) u ^= 0x88888888u;
                    const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
                    // codes 8d..8d+7: low nibbles are the even codes, high nibbles the odd
                    bytes[2 * d] = __builtin_amdgcn_perm(hi, lo, 0x05010400u);      // codes 8d..8d+3
                    bytes[2 * d + 1] = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // codes 8d+4..8d+7
                } else {
                    bytes[d] = SIGNED ? u ^ 0x80808080u : u;
                }
            }
            uint32_t packed[WPT / 2];
#pragma unroll
            for (int e = 0; e < WPT; e += 2) {
                const uint32_t word = bytes[e / 4];
                const float q0 = (float)((word >> (8 * (e % 4))) & 255u);
                const float q1 = (float)((word >> (8 * (e % 4 + 1))) & 255u);
                const bf16x2 pr = {(__bf16)fmaf(q0, s, b), (__bf16)fmaf(q1, s, b)};
                packed[e / 2] = __builtin_bit_cast(uint32_t, pr);
            }
#pragma unroll
            for (int q = 0; q < WPT / 8; ++q)
                lds.b[buf][r][swz(r, (part * WPT + 8 * q) / 8)] =
                    u32x4{packed[4 * q], packed[4 * q + 1], packed[4 * q + 2], packed[4 * q + 3]};
        }
    };

    // wave (wm, wn) owns rows wm*16MI.., cols wn*BN/2.. of the tile
    const int wm = wave >> 1, wn = wave & 1;  // wm 0..3
    const uint32_t li = lane & 15, lk = (lane >> 4) * 8;
    f32x4 acc[MI][MJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32) {
            u32x4 af[MI], bfr[MJ];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const uint32_t r = wm * (16 * MI) + 16 * i + li;
                af[i] = lds.a[buf][r][swz(r, (kk + lk) / 8)];
            }
#pragma unroll
            for (int j = 0; j < MJ; ++j) {
                const uint32_t r = wn * (BN / 2) + 16 * j + li;
                bfr[j] = lds.b[buf][r][swz(r, (kk + lk) / 8)];
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < MJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, af[i]), __builtin_bit_cast(bf16x8, bfr[j]), acc[i][j], 0, 0, 0);
        }
    };

    // NS register stages: step s computes from LDS buffer s%2 while step s+1
    // (loaded NS - 1 steps earlier) is dequantised into the other buffer and
    // the loads of steps s+2 .. s+NS fly; the barriers order LDS only, so
    // those loads stay in flight across them.
    const auto lds_barrier = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    const uint32_t steps = K / kBK;
    // Branch-free body (a conditional load would make the compiler wait for
    // every load before the next dequantisation): the step indices of the
    // prefetches are clamped, so the last ones re-read the final step's tile
    // into a buffer that is not computed again.
    if constexpr (NS == 2) {
        Stage sa, sb;
        load_step(sa, 0);
        load_step(sb, min(1u, steps - 1) * kBK);
        store_step(sa, 0);
        lds_barrier();
        uint32_t s = 0;
        for (; s + 2 <= steps; s += 2) {
            load_step(sa, min(s + 2, steps - 1) * kBK);
            compute(0);
            store_step(sb, 1);
            lds_barrier();
            load_step(sb, min(s + 3, steps - 1) * kBK);
            compute(1);
            store_step(sa, 0);
            lds_barrier();
        }
        if (s < steps) compute(0);  // odd step count: the last step sits in buffer 0
    } else {
        // step s + u of an unrolled block uses stage u % NS and LDS buffer
        // u % 2, constants (a run-time stage index makes the compiler join
        // the stages with copies that wait for their loads); fewer than U
        // steps left take the same bodies, their extra loads clamped
        constexpr int U = NS % 2 ? 2 * NS : NS;
        Stage st[NS];
#pragma unroll
        for (int i = 0; i < NS; ++i) load_step(st[i], min((uint32_t)i, steps - 1) * kBK);
        store_step(st[0], 0);
        lds_barrier();
        uint32_t s = 0;
        for (; s + U <= steps; s += U) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                load_step(st[u % NS], min(s + u + NS, steps - 1) * kBK);
                compute(u % 2);
                store_step(st[(u + 1) % NS], (u + 1) % 2);
                lds_barrier();
            }
        }
#pragma unroll
        for (int u = 0; u < U - 1; ++u) {
            if (s + u >= steps) break;
            load_step(st[u % NS], min(s + u + NS, steps - 1) * kBK);
            compute(u % 2);
            store_step(st[(u + 1) % NS], (u + 1) % 2);
            lds_barrier();
        }
    }

    // ---- epilogue: C[i][j] of a 16x16 block sits in lane j + 16*(i/4), element i%4
    // Full tiles with a plain bf16 store (no D-op past ab_scale): one row
    // pointer per (i, e), the column blocks at fixed offsets from it.
    if (!(op.flags & (FLAG_ACCUMULATE | FLAG_SOFT_CAP)) && !op.bias && op.d_dt == STARK_QMM_BF16 &&
        m0 + BM <= M && n0 + BN <= N) {
        uint16_t* const d = (uint16_t*)op.d;
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + wm * (16 * MI) + 16 * i + 4 * (lane >> 4) + e;
                uint16_t* const row = d + (size_t)m * N + n0 + wn * (BN / 2) + (lane & 15);
#pragma unroll
                for (int j = 0; j < MJ; ++j) row[16 * j] = f32_to_bf16_bits(op.ab_scale * acc[i][j][e]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < MJ; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + wm * (16 * MI) + 16 * i + 4 * (lane >> 4) + e;
                const uint32_t n = n0 + wn * (BN / 2) + 16 * j + (lane & 15);
                if (m >= M || n >= N) continue;
                const size_t o = (size_t)m * N + n;
                float v = op.ab_scale * acc[i][j][e];
                if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
                if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
                if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
                store_from_f32(op.d, op.d_dt, o, v);
            }
}

template <int BITS, int CORR, bool SIGNED, bool BF, int BM, int BN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_mfma(AffineOp op) {
    gemm_tile<BITS, CORR, SIGNED, BF, BM, BN>(op, blockIdx.x, blockIdx.y);
}

__host__ __device__ inline uint32_t gemm_tiles(const AffineOp& o, uint32_t bm, uint32_t bn) {
    return ((o.n + bn - 1) / bn) * ((o.m + bm - 1) / bm);
}

// Several products in one grid (ops of one template class): the tiles of op
// i follow those of op i - 1, each op's row-major over (row block, column
// block), so that the column blocks that share a weight tile keep one XCD
// while the op's column-block count is a multiple of 8. Ops come longest K
// first, so the costliest tiles are dispatched first.
template <int BITS, int CORR, bool SIGNED, bool BF, int BM, int BN>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_group(AffineBatch batch) {
    (void)batch;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t t = blockIdx.x, i = 0;
    for (; i + 1 < kb->count; ++i) {
        const uint32_t nt = gemm_tiles(kb->op[i], BM, BN);
        if (t < nt) break;
        t -= nt;
    }
    const AffineOp& op = kb->op[i];
    const uint32_t gx = (op.n + BN - 1) / BN;
    gemm_tile<BITS, CORR, SIGNED, BF, BM, BN>(op, t % gx, t / gx);
}

}  // namespace

bool gemm_eligible(const AffineOp& o, int bits) {
    if (bits != 4 && bits != 8) return false;
    if (o.x_dt != STARK_QMM_BF16 || o.gather || o.m <= 16) return false;
    if (o.w_dt == STARK_QMM_F32) return false;
    if (!(o.corr_kind == STARK_QMM_CORRECTION_BIASES || o.corr_kind == STARK_QMM_CORRECTION_SYMMETRIC)) return false;
    if (o.group_size != 32 && o.group_size != 64 && o.group_size != 128) return false;
    if (o.k == 0 || o.k % kBK) return false;
    // 32-bit buffer offsets into the codes (with a tile of rows to spare);
    // the activation rows are split into launches that fit (gemm_rows)
    if ((uint64_t)(o.n + kBN) * o.k * bits / 8 >= (1ull << 31) || gemm_rows(o.k) == 0) return false;
    return (((uintptr_t)o.codes | (uintptr_t)o.x) & 15) == 0;
}

// Activation rows one grid takes at K: a multiple of the tile rows whose
// 32-bit byte offsets (with a tile of rows to spare) stay below 2^31.
uint32_t gemm_rows(uint32_t k) {
    const uint64_t rows = ((1ull << 31) - 1) / ((uint64_t)k * 2);
    return rows <= (uint64_t)kBM ? 0u : (uint32_t)std::min<uint64_t>((rows - kBM) / kBM * kBM, 0x80000000u);
}

stark_qmm_status launch_affine_gemm_rows(const AffineOp& op, int bits, hipStream_t stream);

stark_qmm_status launch_affine_gemm(const AffineOp& op, int bits, hipStream_t stream) {
    // products too tall for 32-bit offsets run as several launches of whole rows
    const uint32_t R = gemm_rows(op.k);
    if (R == 0) return STARK_QMM_UNSUPPORTED;
    const size_t dsz = op.d_dt == STARK_QMM_F32 ? 4 : 2;
    for (uint32_t m0 = 0; m0 < op.m; m0 += R) {
        AffineOp part = op;
        part.m = std::min(R, op.m - m0);
        part.x = (const uint8_t*)op.x + (size_t)m0 * op.k * 2;
        part.d = (uint8_t*)op.d + (size_t)m0 * op.n * dsz;
        const stark_qmm_status st = launch_affine_gemm_rows(part, bits, stream);
        if (st != STARK_QMM_OK) return st;
    }
    return STARK_QMM_OK;
}

stark_qmm_status launch_affine_gemm_rows(const AffineOp& op, int bits, hipStream_t stream) {
    const uint32_t bm = gemm_bm(op.m), bn = gemm_bn(op.m);
    const dim3 grid((op.n + bn - 1) / bn, (op.m + bm - 1) / bm);
    if (grid.x == 0 || grid.y == 0) return STARK_QMM_OK;
    const bool sg = (op.flags & FLAG_SIGNED) != 0, bi = op.corr_kind == STARK_QMM_CORRECTION_BIASES;
    const bool bf = op.w_dt == STARK_QMM_BF16;
#define QMM_G(B, C, S, F)                                                                        \
    do {                                                                                         \
        if (bm == 256) hipLaunchKernelGGL((qgemm_mfma<B, C, S, F, 256, 128>), grid, dim3(kThreads), 0, stream, op); \
        else if (bn == 64) hipLaunchKernelGGL((qgemm_mfma<B, C, S, F, 128, 64>), grid, dim3(kThreads), 0, stream, op); \
        else hipLaunchKernelGGL((qgemm_mfma<B, C, S, F, 128, 128>), grid, dim3(kThreads), 0, stream, op);        \
    } while (0)
#define QMM_G_BITS(B)                                                      \
    if (bi) {                                                              \
        if (sg) { if (bf) QMM_G(B, 1, true, true); else QMM_G(B, 1, true, false); } \
        else { if (bf) QMM_G(B, 1, false, true); else QMM_G(B, 1, false, false); }  \
    } else {                                                               \
        if (sg) { if (bf) QMM_G(B, 0, true, true); else QMM_G(B, 0, true, false); } \
        else { if (bf) QMM_G(B, 0, false, true); else QMM_G(B, 0, false, false); }  \
    }
    if (bits == 4) {
        QMM_G_BITS(4)
    } else {
        QMM_G_BITS(8)
    }
#undef QMM_G_BITS
#undef QMM_G
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm

namespace qmm {

// ops: gemm_eligible, M > 16, of one (bits, signedness, correction, plane
// type) class; at most kMaxBatchOps.
stark_qmm_status launch_affine_gemm_group(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream) {
    if (count == 0) return STARK_QMM_OK;
    if (count == 1) return launch_affine_gemm(ops[0], bits, stream);
    if (count > (uint32_t)kMaxBatchOps) return STARK_QMM_UNSUPPORTED;
    std::vector<AffineOp> sorted(ops, ops + count);
    std::stable_sort(sorted.begin(), sorted.end(), [](const AffineOp& a, const AffineOp& b) { return a.k > b.k; });
    AffineBatch batch{};
    uint32_t mmax = 0;
    for (uint32_t i = 0; i < count; ++i) mmax = std::max(mmax, sorted[i].m);
    const uint32_t bm = gemm_bm(mmax), bn = gemm_bn(mmax);  // as launch_affine_gemm_rows
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = sorted[i];
        tiles += gemm_tiles(sorted[i], bm, bn);
    }
    batch.count = count;
    batch.total = (uint32_t)tiles;
    if (tiles == 0) return STARK_QMM_OK;
    if (tiles > 0x7fffffffu) return STARK_QMM_UNSUPPORTED;
    const AffineOp& op = sorted[0];
    const bool sg = (op.flags & FLAG_SIGNED) != 0, bi = op.corr_kind == STARK_QMM_CORRECTION_BIASES;
    const bool bf = op.w_dt == STARK_QMM_BF16;
    const dim3 grid((uint32_t)tiles);
#define QMM_GG(B, C, S, F)                                                                          \
    do {                                                                                            \
        if (bm == 256) hipLaunchKernelGGL((qgemm_group<B, C, S, F, 256, 128>), grid, dim3(kThreads), 0, stream, batch); \
        else if (bn == 64) hipLaunchKernelGGL((qgemm_group<B, C, S, F, 128, 64>), grid, dim3(kThreads), 0, stream, batch); \
        else hipLaunchKernelGGL((qgemm_group<B, C, S, F, 128, 128>), grid, dim3(kThreads), 0, stream, batch);        \
    } while (0)
#define QMM_GG_BITS(B)                                                                 \
    if (bi) {                                                                          \
        if (sg) { if (bf) QMM_GG(B, 1, true, true); else QMM_GG(B, 1, true, false); } \
        else { if (bf) QMM_GG(B, 1, false, true); else QMM_GG(B, 1, false, false); }  \
    } else {                                                                           \
        if (sg) { if (bf) QMM_GG(B, 0, true, true); else QMM_GG(B, 0, true, false); } \
        else { if (bf) QMM_GG(B, 0, false, true); else QMM_GG(B, 0, false, false); }  \
    }
    if (bits == 4) {
        QMM_GG_BITS(4)
    } else {
        QMM_GG_BITS(8)
    }
#undef QMM_GG_BITS
#undef QMM_GG
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm
