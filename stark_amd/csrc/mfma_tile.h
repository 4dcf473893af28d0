// mfma_tile.h -- one 16-row tile of a 4-bit affine product on the gfx950
// matrix cores (activation rows M <= 16), shared by the plain product kernel
// (qmv_mfma.hip) and the grouped MoE kernels (moe_routed.hip).
//
// Per group g of a weight row (reference per-element loop:
// crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:185-268)
//   s*sum(x*q) + b*sum(x) = 128s * sum x*(1 + q/128) + (b - 128s) * sum(x)
// (1 + q/128) is the bf16 whose low mantissa bits are the code nibble, built by
// a shift, an and and an or per pair of codes; sum x*(1 + q/128) runs on
// v_mfma_f32_16x16x32_bf16 (exact bf16 products, f32 accumulation).
//
// MFMA roles: B[k][j] = weight row (n0 + j) dequantised as above, A[i][k] =
// activations, where accumulator row i stands for (activation row m, group
// slot): A[i][k] = x[m][k] when k's group maps to slot i, else 0. One
// accumulator period therefore collects S = 16/MP groups separately; at the end
// of a period each lane scales its 4 accumulator rows by the (row, group)
// scale/bias from LDS. MP = padded activation rows per A block (1, 2, 4, 8); M
// up to 16 uses two A blocks sharing every dequantised B operand.
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

// v_and_or_b32 with the mask in a VGPR and the or-value in an SGPR: the
// compiler splits (a & m) | c into two instructions on its own.
__device__ __forceinline__ uint32_t and_or_vs(uint32_t a, uint32_t vmask, uint32_t sor) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(vmask), "s"(sor));
    return r;
}

// P1: pass length (k values) when MP*MB <= 2; wider activation tiles use
// shorter passes so the staged activations fit LDS.
template <int MP, int MB, int P1 = QMM_MFMA_PASS_SMALL_M>
struct Cfg {
    static constexpr int S = 16 / MP;  // group slots per activation row
    static constexpr int MR = MP * MB;
    static constexpr int PASS = MR <= 2 ? P1 : (MR <= 8 ? 2048 : 1024);
    static constexpr int Q = PASS / 4;      // k values per wave per pass
    static constexpr int SEGB = Q / 2;      // bytes of a row per wave per pass
    static constexpr int NI = SEGB / 64;    // 16-byte loads per lane per pass == steps per pass
    static constexpr int ROWB = SEGB + 16;  // padded LDS row: the 16 operand rows hit distinct banks
};

template <int MP, int MB, int P1 = QMM_MFMA_PASS_SMALL_M>
struct MfmaLds {
    using C = Cfg<MP, MB, P1>;
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

// One 16-row tile of a 4-bit affine product on the matrix cores, up to the
// per-(activation row, tile row) sums, which are left in lds.red[wave][m][r]
// (add the four waves in order 0+1, 2+3) behind a barrier.
//   op     : codes / planes / activation base, K, group size, plane strides
//   nA, nB : bank rows of tile rows 0..7 and 8..15 (multiples of 8, nB >= nA)
//   M      : activation rows (<= MP*MB); xrow(m) = element offset of row m in op.x
//   nib_s  : 0x000F000F, one2 : 0x3F803F80 (kernel arguments, scalar)
template <int MP, int MB, bool SIGNED, bool BIASED, bool BF, int P1 = QMM_MFMA_PASS_SMALL_M, class XRow>
__device__ __forceinline__ void mfma_tile(const AffineOp& op, uint32_t nA, uint32_t nB, uint32_t M, XRow xrow,
                                          MfmaLds<MP, MB, P1>& lds, uint32_t nib_s, uint32_t one2) {
    using Cf = Cfg<MP, MB, P1>;
    constexpr int S = Cf::S, MR = Cf::MR, PASS = Cf::PASS, Q = Cf::Q, SEGB = Cf::SEGB, NI = Cf::NI;
    constexpr int ROWB = Cf::ROWB;

    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t K = op.k;
    const size_t row_bytes = (size_t)K / 2;
    const uint32_t gshift = 31 - __builtin_clz(op.group_size);
    // output-group rows start 16-byte aligned only when the group count is a
    // multiple of 8 (passes start at multiples of 8 groups)
    const bool og_vec = op.os % 8 == 0 && (((uintptr_t)op.scales | (uintptr_t)op.corr) & 15) == 0;
    const uint32_t gps_shift = 7 - gshift;             // log2(groups per step)
    const uint32_t period = (uint32_t)S >> gps_shift;  // steps per accumulator period
    uint32_t nib;  // 0x000F000F, held in a VGPR so v_and_or_b32 can take one2 from an SGPR
    asm volatile("v_mov_b32 %0, %1" : "=v"(nib) : "s"(nib_s));

    const uint32_t j = lane & 15, kq = lane >> 4;  // B/C column (tile row), k quarter of a step
    const uint32_t am = j / S, aslot = j % S;      // A row j -> (activation row, slot)
    const uint32_t qbase = wave * Q;               // wave's first k within a pass
    const uint32_t gw = qbase >> gshift;           // wave's first group within a pass
    uint8_t* wstage = (uint8_t*)lds.stage[wave];

    if (tid < 4) lds.zero[tid] = u32x4{0, 0, 0, 0};

    // Code loads of one pass through a buffer resource starting at row nA:
    // 16-byte piece i*64 + lane of the wave's row-major [16][SEGB] block. The
    // lane part of the offset is fixed, the piece part (row, pass) is a scalar;
    // pieces past K get an offset beyond the resource and read as zero.
    constexpr int LPR = SEGB / 16;  // lanes per row segment
    constexpr int RPI = 64 / LPR;   // rows per load instruction (divides 8)
    const uint32_t hi_skip = nB - nA - 8;  // extra rows between the two halves
    const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(op.codes + (size_t)nA * row_bytes), 0, (int)((nB - nA + 8) * row_bytes), 0x00020000);
    const uint32_t lcol = (lane % LPR) * 16;
    const uint32_t voff = (lane / LPR) * (uint32_t)row_bytes + wave * SEGB + lcol;
    u32x4 w[NI];
    auto load_codes = [&](uint32_t kbase) {
        const uint32_t kvals = min((uint32_t)PASS, K - kbase);
        const uint32_t vo = qbase + 2 * lcol < kvals ? voff : 0x80000000u;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            w[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           crs, vo, (i * RPI + (i * RPI >= 8 ? hi_skip : 0)) * (uint32_t)row_bytes + kbase / 2,
                           kBufNt));
    };
    // Activation and metadata loads of one pass, all issued at once so that a
    // pass costs one memory round trip: activation vector v = tid + i*256 of
    // the [MR][PASS/8] table; one scale and one bias vector per thread.
    constexpr int XV = MR * (PASS / 8);             // activation vectors per pass
    constexpr int XI = (XV + kWg - 1) / kWg;        // per thread
    u32x4 xv[XI], msv, mbv;
    auto load_aux = [&](uint32_t kbase) {
        const uint32_t kvals = min((uint32_t)PASS, K - kbase);
        const uint32_t g0 = kbase >> gshift, gcnt = kvals >> gshift;
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
            const uint32_t per_row = og_vec ? gcnt / 8 : 0;  // 0: staged element by element below
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
    };
    load_aux(0);
    load_codes(0);

    f32x4 acc[MB], C[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b) acc[b] = C[b] = f32x4{0, 0, 0, 0};

    for (uint32_t kbase = 0; kbase < K; kbase += PASS) {
        const uint32_t kvals = min((uint32_t)PASS, K - kbase);
        const uint32_t gcnt = kvals >> gshift;  // K % group_size == 0

        if (kbase) __syncthreads();  // every wave finished the previous pass's LDS
        // ---- stage activations: pairs in MFMA k order and per-group sums
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t v = tid + i * kWg, m = v / (PASS / 8), vi = v % (PASS / 8);
            const u32x4 t = xv[i];
            u32x4 pq;
            pq[0] = perm(t[2], t[0], 0x05040100u);
            pq[1] = perm(t[2], t[0], 0x07060302u);
            pq[2] = perm(t[3], t[1], 0x05040100u);
            pq[3] = perm(t[3], t[1], 0x07060302u);
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
        for (int i = 0; i < NI; ++i) {
            *(u32x4*)(wstage + (i * RPI + lane / LPR) * ROWB + lcol) = w[i];
        }
        __syncthreads();
        if (kbase + PASS < K) {  // next pass's loads are in flight while this pass computes
            load_aux(kbase + PASS);
            load_codes(kbase + PASS);
        }

        // Fold the period's accumulator rows into acc: row i = (m, slot) with
        // wave-local group pidx*S + slot; weight = 128s * C + (b - 128s) * xsum.
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
                    const float bi = BIASED ? h2f<BF>(raw[jj] >> 16) : -8.0f * sc;
                    const float s128 = 128.0f * sc;
                    const float nv = fmaf(s128, C[b][jj], fmaf(bi - s128, xsum[jj], acc[b][jj]));
                    acc[b][jj] = g[jj] < glim ? nv : acc[b][jj];
                }
                C[b] = f32x4{0, 0, 0, 0};
            }
        };
#pragma unroll
        for (int s = 0; s < NI; ++s) {
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
            const u32x4 wv = *(const u32x4*)(wstage + j * ROWB + s * 64 + 16 * kq);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t u = wv[t];
                if (SIGNED) u ^= 0x88888888u;
                u32x4 bq;
                bq[0] = and_or_vs(u, nib, one2);        // (q0, q4)
                bq[1] = and_or_vs(u >> 4, nib, one2);   // (q1, q5)
                bq[2] = and_or_vs(u >> 8, nib, one2);   // (q2, q6)
                bq[3] = and_or_vs(u >> 12, nib, one2);  // (q3, q7)
                const bf16x8 bv = __builtin_bit_cast(bf16x8, bq);
#pragma unroll
                for (int b = 0; b < MB; ++b)
                    C[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[b][t]), bv, C[b],
                                                                  0, 0, 0);
            }
            if ((s + 1) % period == 0) flush(s / period);
        }
        if (NI % period) flush(NI / period);  // partial last period of the pass
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

}  // namespace mfma
}  // namespace qmm
