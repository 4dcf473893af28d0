// mfma_tile.h -- one 16-row tile of a 4-bit affine product on the gfx950
// matrix cores (activation rows M <= 16), shared by the plain product kernel
// (qmv_mfma.hip) and the grouped MoE kernels (moe_routed.hip).
//
// Per group g of a weight row (reference per-element loop:
// crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:185-268)
//   sum x*w = s * sum(x*q) + bias_term * sum(x),  bias_term = b or -s*2^(bits-1)
// sum(x*q) runs on v_mfma_f32_16x16x32_bf16 with the codes used as raw bf16
// bit patterns: a pattern p < 256 (exponent field 0 or 1) is exactly
// p * 2^-133, so a code needs only a mask to become an operand (4-bit: the odd
// nibble is left at bit 4, i.e. 16q, and its activation is scaled by 2^-4).
// The activations are staged as bf16 x * 2^64 (exact), which puts the products
// x*q*2^-69 in f32's normal range; the flush multiplies by s * 2^69. Products
// are exact and accumulate in f32.
//
// Schedule: a workgroup (4 waves) owns a 16-row tile (two 8-row halves that
// may sit anywhere in the bank, e.g. an expert's value and gate rows). K is walked in passes; each wave takes a contiguous quarter of a pass.
// A wave loads its quarter of the 16 rows with 16-byte lanes laid out row-major
// (one load instruction covers whole 128-512 byte row segments, which HBM
// streams far better than the 64-byte pieces of the MFMA operand layout),
// writes it to a private padded LDS block and reads it back in operand layout.
// Activations (as bf16 pairs in the MFMA's k order, with per-group sums) and
// the raw (scale, bias) pairs of the tile are staged in LDS once per pass; the
// next pass's code loads are in flight while the current pass computes. The
// four waves' partial sums meet in LDS and are added in a fixed order before
// the D-ops.
#pragma once
#include "qmm_common.h"

#ifndef QMM_MFMA_PASS_SMALL_M
#define QMM_MFMA_PASS_SMALL_M 4096
#endif

namespace qmm {
namespace mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWg = 256;
constexpr int kRows = 16;   // tile rows (MFMA B columns)
constexpr int kStep = 128;  // k values per step (4 MFMAs, 64 bytes of a row)
constexpr int kBufNt = 2;   // buffer-load cache policy: nontemporal (streamed once)


// P1: pass length (k values) when MP*MB <= 2; wider activation tiles use
// shorter passes so the staged activations fit LDS.
template <int MP, int MB, int P1 = QMM_MFMA_PASS_SMALL_M, int BITS = 4>
struct Cfg {
    static constexpr int S = 16 / MP;  // group slots per activation row
    static constexpr int MR = MP * MB;
    static constexpr int PASS = MR <= 2 ? P1 : (MR <= 8 ? 2048 : 1024);
    static constexpr int Q = PASS / 4;             // k values per wave per pass
    static constexpr int SEGB = Q * BITS / 8;      // bytes of a row per wave per pass
    static constexpr int NI = SEGB / 64;           // 16-byte code loads per lane per pass
    static constexpr int NSTEP = Q / kStep;        // MFMA steps per pass
    static constexpr int ROWB = SEGB + 16;         // padded LDS row: the 16 operand rows hit distinct banks
};

template <int MP, int MB, int P1 = QMM_MFMA_PASS_SMALL_M, int BITS = 4>
struct MfmaLds {
    using C = Cfg<MP, MB, P1, BITS>;
    u32x4 stage[4][kRows * C::ROWB / 16];    // per-wave code block [16][ROWB bytes]
    uint32_t meta[kRows][C::PASS / 32 + 4];  // raw 16-bit (scale | bias << 16) per (row, group)
    u32x4 xp[C::MR][C::PASS / 8];            // activation pairs (x0,x4)(x1,x5)(x2,x6)(x3,x7) per 8 values
    float xs[C::MR][C::PASS / 32 + 4];       // activation sum per group
    float red[4][C::MR][kRows];              // per-wave partial outputs
    u32x4 zero[4];
};

template <bool BF>
__device__ __forceinline__ float h2f(uint32_t h) {
    return BF ? __uint_as_float(h << 16) : f16_bits_to_f32(h);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// Tile engine: one 16-row tile of a 4-bit affine product on the matrix cores,
// run pass by pass, with the loads of the next pass -- or of the next tile --
// issued into the same registers as soon as the current pass sits in LDS.
// A tile is described by
//   op     : codes / planes / activation base, K, group size, plane strides
//   nA, nB : bank rows of tile rows 0..7 and 8..15 (multiples of 8, nB >= nA)
//   M      : activation rows (<= MP*MB); xrow(m) = element offset of row m in op.x
// run() leaves the per-(activation row, tile row) sums in lds.red[wave][m][r]
// (add the four waves in order (0+1)+(2+3)) behind a barrier.
template <int MP, int MB, bool SIGNED, bool BIASED, bool BF, int P1 = QMM_MFMA_PASS_SMALL_M, int BITS = 4>
struct TileEngine {
    using Cf = Cfg<MP, MB, P1, BITS>;
    static constexpr int S = Cf::S, MR = Cf::MR, PASS = Cf::PASS, Q = Cf::Q, SEGB = Cf::SEGB, NI = Cf::NI;
    static constexpr int NSTEP = Cf::NSTEP;
    static constexpr int ROWB = Cf::ROWB;
    static constexpr int LPR = SEGB / 16;         // lanes per row segment of a code load
    static constexpr int RPI = 64 / LPR;          // rows per code load instruction (divides 8)
    static constexpr int XV = MR * (PASS / 8);    // activation vectors per pass
    static constexpr int XI = (XV + kWg - 1) / kWg;

    MfmaLds<MP, MB, P1, BITS>& lds;
    int tid, lane;
    uint32_t wave, j, kq, am, aslot, qbase, lcol, nib, one2;
    uint8_t* wstage;
    u32x4 w[NI];       // codes of the loaded pass
    u32x4 xv[XI];      // activations of the loaded pass
    u32x4 msv, mbv;    // scale / bias vectors of the loaded pass

    __device__ __forceinline__ TileEngine(MfmaLds<MP, MB, P1, BITS>& l, uint32_t nib_s, uint32_t one2_s) : lds(l) {
        tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        j = lane & 15;  // B/C column (tile row)
        kq = lane >> 4; // k quarter of a step
        am = j / S;     // A row j -> (activation row, slot)
        aslot = j % S;
        qbase = wave * Q;  // wave's first k within a pass
        lcol = (lane % LPR) * 16;
        wstage = (uint8_t*)lds.stage[wave];
        nib = nib_s;
        one2 = one2_s;
        if (tid < 4) lds.zero[tid] = u32x4{0, 0, 0, 0};
    }

    static __device__ __forceinline__ uint32_t gshift_of(const AffineOp& op) {
        return 31 - __builtin_clz(op.group_size);
    }
    // output-group rows start 16-byte aligned only when the group count is a
    // multiple of 8 (passes start at multiples of 8 groups)
    static __device__ __forceinline__ bool og_vec_of(const AffineOp& op) {
        return op.os % 8 == 0 && (((uintptr_t)op.scales | (uintptr_t)op.corr) & 15) == 0;
    }

    // Issue every global load of pass `kbase` of a tile: codes through a buffer
    // resource starting at row nA (16-byte piece i*64 + lane of the wave's
    // row-major [16][SEGB] block; pieces past K get an offset beyond the
    // resource and read as zero), activations (vector v = tid + i*256 of the
    // [MR][PASS/8] table) and one scale and one bias vector per thread.
    template <class XRow>
    __device__ __forceinline__ void load(const AffineOp& op, uint32_t nA, uint32_t nB, uint32_t M, XRow xrow,
                                         uint32_t kbase) {
        const uint32_t K = op.k, kvals = min((uint32_t)PASS, K - kbase);
        const uint32_t gshift = gshift_of(op), g0 = kbase >> gshift, gcnt = kvals >> gshift;
        const uint32_t row_bytes = K * BITS / 8;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t v = tid + i * kWg, m = v / (PASS / 8), vi = v % (PASS / 8);
            const bool ok = v < (uint32_t)XV && m < M && vi * 8 < kvals;
            const u32x4 t = *(const u32x4*)((const uint16_t*)op.x + (ok ? xrow(m) + kbase + vi * 8 : 0));
            xv[i] = ok ? t : u32x4{0, 0, 0, 0};
        }
        bool ok;
        size_t off;
        if (op.os == 1) {  // group-output planes [G][N4]: 8 rows of group tid/2 per vector
            ok = (uint32_t)tid < gcnt * 2;
            off = (size_t)(g0 + (tid >> 1)) * op.gs + ((tid & 1) ? nB : nA);
        } else {  // output-group planes [N][G]: 8 groups of a row per vector
            const uint32_t per_row = og_vec_of(op) ? gcnt / 8 : 0;  // 0: staged element by element
            ok = (uint32_t)tid < kRows * per_row;
            const uint32_t r = per_row ? tid / per_row : 0, g8 = per_row ? (tid % per_row) * 8 : 0;
            off = (size_t)(r < 8 ? nA + r : nB + r - 8) * op.os + g0 + g8;
        }
        off = ok ? off : 0;
        const u32x4 sv = *(const u32x4*)((const uint16_t*)op.scales + off);
        msv = ok ? sv : u32x4{0, 0, 0, 0};
        if (BIASED) {
            const u32x4 bv = *(const u32x4*)((const uint16_t*)op.corr + off);
            mbv = ok ? bv : u32x4{0, 0, 0, 0};
        } else {
            mbv = u32x4{0, 0, 0, 0};
        }
        const uint32_t hi_skip = nB - nA - 8;  // extra rows between the two halves
        const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(op.codes + (size_t)nA * row_bytes), 0, (int)((nB - nA + 8) * row_bytes), 0x00020000);
        const uint32_t voff = (lane / LPR) * row_bytes + wave * SEGB + lcol;
        const uint32_t vo = qbase + lcol * 8 / BITS < kvals ? voff : 0x80000000u;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            w[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           crs, vo, (i * RPI + (i * RPI >= 8 ? hi_skip : 0)) * row_bytes + kbase / 2, kBufNt));
    }

    // Run every pass of a tile whose first pass has been load()ed. After the
    // last pass is staged, next() is called to issue the next tile's loads.
    template <class XRow, class Next>
    __device__ __forceinline__ void run(const AffineOp& op, uint32_t nA, uint32_t nB, uint32_t M, XRow xrow,
                                        Next next) {
        const uint32_t K = op.k;
        const uint32_t gshift = gshift_of(op);
        const bool og_vec = og_vec_of(op);
        const uint32_t gps_shift = 7 - gshift;             // log2(groups per step)
        const uint32_t period = (uint32_t)S >> gps_shift;  // steps per accumulator period
        const uint32_t gw = qbase >> gshift;                // wave's first group within a pass

        f32x4 acc[MB], C[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[b] = C[b] = f32x4{0, 0, 0, 0};

        for (uint32_t kbase = 0; kbase < K; kbase += PASS) {
            const uint32_t kvals = min((uint32_t)PASS, K - kbase);
            const uint32_t gcnt = kvals >> gshift;  // K % group_size == 0

            if (kbase) __syncthreads();  // every wave finished the previous pass's LDS
            // ---- stage activations: bf16 x * 2^64 (4-bit odd codes: x * 2^60), in
            // the operand order of the code masks, and per-group sums of x
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const uint32_t v = tid + i * kWg, m = v / (PASS / 8), vi = v % (PASS / 8);
                const u32x4 t = xv[i];
                float f[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    f[2 * e] = __uint_as_float(t[e] << 16) * 0x1p64f;
                    f[2 * e + 1] = __uint_as_float(t[e] & 0xffff0000u) * (BITS == 4 ? 0x1p60f : 0x1p64f);
                }
                // 4-bit pairs (x0,x4)(x1,x5)(x2,x6)(x3,x7); 8-bit pairs (x0,x2)(x1,x3)(x4,x6)(x5,x7)
                constexpr int p0 = 0, p1 = BITS == 4 ? 4 : 2, p2 = 1, p3 = BITS == 4 ? 5 : 3;
                constexpr int p4 = BITS == 4 ? 2 : 4, p5 = 6, p6 = BITS == 4 ? 3 : 5, p7 = 7;
                u32x4 pq;
                pq[0] = perm(__float_as_uint(f[p1]), __float_as_uint(f[p0]), 0x07060302u);
                pq[1] = perm(__float_as_uint(f[p3]), __float_as_uint(f[p2]), 0x07060302u);
                pq[2] = perm(__float_as_uint(f[p5]), __float_as_uint(f[p4]), 0x07060302u);
                pq[3] = perm(__float_as_uint(f[p7]), __float_as_uint(f[p6]), 0x07060302u);
                if (v < (uint32_t)XV) lds.xp[m][vi] = pq;
                float sm = 0.0f;
#pragma unroll
                for (int e = 0; e < 4; ++e) sm = dot2_bf16(t[e], 0x3F803F80u, sm);
                // the gs/8 vectors of a group sit in consecutive lanes (whole waves
                // take part in the shuffles; lanes past the table add zeros)
                for (uint32_t off = 1; off < (op.group_size >> 3); off <<= 1) sm += __shfl_xor(sm, off, 64);
                if (v < (uint32_t)XV && (vi & ((op.group_size >> 3) - 1)) == 0) lds.xs[m][(vi * 8) >> gshift] = sm;
            }
            // ---- stage raw (scale, bias) pairs of the 16 tile rows
            if (op.os == 1) {
                if ((uint32_t)tid < gcnt * 2) {
                    const uint32_t g = tid >> 1, r8 = (tid & 1) * 8;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        lds.meta[r8 + e][g] = ((msv[e >> 1] >> (16 * (e & 1))) & 0xffffu) |
                                              (((mbv[e >> 1] >> (16 * (e & 1))) & 0xffffu) << 16);
                }
            } else if (og_vec) {
                const uint32_t per_row = gcnt / 8;
                if ((uint32_t)tid < kRows * per_row) {
                    const uint32_t r = tid / per_row, g8 = (tid % per_row) * 8;
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        lds.meta[r][g8 + e] = ((msv[e >> 1] >> (16 * (e & 1))) & 0xffffu) |
                                              (((mbv[e >> 1] >> (16 * (e & 1))) & 0xffffu) << 16);
                }
            } else {  // output-group planes whose rows are not 16-byte aligned: one element per step
                const uint32_t g0 = kbase >> gshift;
                for (uint32_t q = tid; q < kRows * gcnt; q += kWg) {
                    const uint32_t r = q / gcnt, g = q % gcnt;
                    const size_t o = (size_t)(r < 8 ? nA + r : nB + r - 8) * op.os + g0 + g;
                    const uint32_t sv = ((const uint16_t*)op.scales)[o];
                    const uint32_t bv = BIASED ? ((const uint16_t*)op.corr)[o] : 0u;
                    lds.meta[r][g] = sv | (bv << 16);
                }
            }
            // ---- this pass's codes to the wave's LDS block (row-major, padded rows)
#pragma unroll
            for (int i = 0; i < NI; ++i) *(u32x4*)(wstage + (i * RPI + lane / LPR) * ROWB + lcol) = w[i];
            __syncthreads();
            // the registers are free: the next pass's (or tile's) loads fly while this pass computes
            if (kbase + PASS < K)
                load(op, nA, nB, M, xrow, kbase + PASS);
            else
                next();

            // Fold the period's accumulator rows into acc: row i = (m, slot) with
            // wave-local group pidx*S + slot; adds s * 2^69 * C + bias_term * xsum.
            // Slots past the wave's groups or past K hold nothing and are skipped.
            const uint32_t* rmeta = lds.meta[j];
            const uint32_t glim = min(gcnt, gw + (uint32_t)(Q >> gshift));
            auto flush = [&](uint32_t pidx) {
                const uint32_t gb = gw + pidx * S;
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    uint32_t raw[4], g[4];
                    float xsum[4];
                    if (S >= 4) {
                        const uint32_t g4 = gb + (4 * kq) % S;
                        const uint32_t m = b * MP + (4 * kq) / S;
                        const u32x4 r4 = *(const u32x4*)&rmeta[g4];
                        const f32x4 x4 = *(const f32x4*)&lds.xs[m][g4];
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) {
                            raw[jj] = r4[jj];
                            xsum[jj] = x4[jj];
                            g[jj] = g4 + jj;
                        }
                    } else {  // S == 2: rows (2kq, gb), (2kq, gb+1), (2kq+1, gb), (2kq+1, gb+1)
                        const uint32_t m = b * MP + 2 * kq;
                        raw[0] = raw[2] = rmeta[gb];
                        raw[1] = raw[3] = rmeta[gb + 1];
                        xsum[0] = lds.xs[m][gb];
                        xsum[1] = lds.xs[m][gb + 1];
                        xsum[2] = lds.xs[m + 1][gb];
                        xsum[3] = lds.xs[m + 1][gb + 1];
                        g[0] = g[2] = gb;
                        g[1] = g[3] = gb + 1;
                    }
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const float sc = h2f<BF>(raw[jj] & 0xffffu);
                        const float bi = BIASED ? h2f<BF>(raw[jj] >> 16) : -(float)(1 << (BITS - 1)) * sc;
                        const float nv = fmaf(sc * 0x1p69f, C[b][jj], fmaf(bi, xsum[jj], acc[b][jj]));
                        acc[b][jj] = g[jj] < glim ? nv : acc[b][jj];
                    }
                    C[b] = f32x4{0, 0, 0, 0};
                }
            };
#pragma unroll
            for (int s = 0; s < NSTEP; ++s) {
                const uint32_t kloc = s * kStep + 32 * kq;  // wave-local k of this lane's 32 values
                const uint32_t kpos = qbase + kloc;         // pass-relative k
                const uint32_t lg = kloc >> gshift;         // wave-local group
                u32x4 a[MB][4];
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    const uint32_t m = b * MP + am;
                    const bool act = m < M && (lg % S) == aslot && kpos < kvals;
                    const u32x4* src = act ? &lds.xp[m][kpos / 8] : lds.zero;
#pragma unroll
                    for (int t = 0; t < 4; ++t) a[b][t] = src[t];
                }
                // this lane's 32 codes: 16 bytes (4-bit) or 32 bytes (8-bit)
                u32x4 wv[BITS / 4];
#pragma unroll
                for (int h = 0; h < BITS / 4; ++h)
                    wv[h] = *(const u32x4*)(wstage + j * ROWB + s * (kStep * BITS / 8) + 4 * BITS * kq + 16 * h);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    u32x4 bq;
                    if (BITS == 4) {
                        uint32_t u = wv[0][t];
                        if (SIGNED) u ^= 0x88888888u;
                        const uint32_t u8 = u >> 8;
                        bq[0] = u & 0x000F000Fu;   // (q0, q4)
                        bq[1] = u & 0x00F000F0u;   // (16 q1, 16 q5)
                        bq[2] = u8 & 0x000F000Fu;  // (q2, q6)
                        bq[3] = u8 & 0x00F000F0u;  // (16 q3, 16 q7)
                    } else {
                        uint32_t u0 = wv[t >> 1][2 * (t & 1)], u1 = wv[t >> 1][2 * (t & 1) + 1];
                        if (SIGNED) {
                            u0 ^= 0x80808080u;
                            u1 ^= 0x80808080u;
                        }
                        bq[0] = u0 & 0x00FF00FFu;         // (q0, q2)
                        bq[1] = (u0 >> 8) & 0x00FF00FFu;  // (q1, q3)
                        bq[2] = u1 & 0x00FF00FFu;         // (q4, q6)
                        bq[3] = (u1 >> 8) & 0x00FF00FFu;  // (q5, q7)
                    }
                    const bf16x8 bv = __builtin_bit_cast(bf16x8, bq);
#pragma unroll
                    for (int b = 0; b < MB; ++b)
                        C[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[b][t]), bv,
                                                                      C[b], 0, 0, 0);
                }
                if ((s + 1) % period == 0) flush(s / period);
            }
            if (NSTEP % period) flush(NSTEP / period);  // partial last period of the pass
        }

        // ---- reduce accumulator rows of the same activation row, then across waves
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            if (S >= 4) {
                float v = (acc[b][0] + acc[b][1]) + (acc[b][2] + acc[b][3]);
                if (S == 16) {
                    v += __shfl_xor(v, 16, 64);
                    v += __shfl_xor(v, 32, 64);
                } else if (S == 8) {
                    v += __shfl_xor(v, 16, 64);
                }
                const uint32_t m = b * MP + (4 * kq) / S;
                const bool owner = S == 16 ? kq == 0 : (S == 8 ? (kq & 1) == 0 : true);
                if (owner) lds.red[wave][m][j] = v;
            } else {  // S == 2: rows 4kq..4kq+3 are (m, slot) = (2kq, 0), (2kq, 1), (2kq+1, 0), (2kq+1, 1)
                lds.red[wave][b * MP + 2 * kq][j] = acc[b][0] + acc[b][1];
                lds.red[wave][b * MP + 2 * kq + 1][j] = acc[b][2] + acc[b][3];
            }
        }
        __syncthreads();
    }

    // Sum over the four waves of (activation row m, tile row r), in a fixed order.
    __device__ __forceinline__ float sum(uint32_t m, uint32_t r) const {
        return (lds.red[0][m][r] + lds.red[1][m][r]) + (lds.red[2][m][r] + lds.red[3][m][r]);
    }
};

// One tile, loads included (the grouped MoE kernels).
template <int MP, int MB, bool SIGNED, bool BIASED, bool BF, int P1 = QMM_MFMA_PASS_SMALL_M, int BITS = 4,
          class XRow>
__device__ __forceinline__ void mfma_tile(const AffineOp& op, uint32_t nA, uint32_t nB, uint32_t M, XRow xrow,
                                          MfmaLds<MP, MB, P1, BITS>& lds, uint32_t nib_s, uint32_t one2) {
    TileEngine<MP, MB, SIGNED, BIASED, BF, P1, BITS> e(lds, nib_s, one2);
    e.load(op, nA, nB, M, xrow, 0);
    e.run(op, nA, nB, M, xrow, [] {});
}

}  // namespace mfma
}  // namespace qmm
