// mfma_tile.h -- one 16-row tile of a 4- or 8-bit affine product on the gfx950
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
// The activations are staged as bf16 x * 2^E (exact) with a per-group exponent
// E (group_shift, qmm_common.h), which puts the products x*q*2^(E-133) in f32's
// normal range for every finite x; the flush brings a group's sum back with
// ldexp by 133 - E and multiplies by s. Products are exact and accumulate in f32.
//
// MFMA roles: B columns are the 16 weight rows of the tile; A rows are
// (activation row, group slot) pairs -- A holds x where the k position's group
// maps to the row's slot and 0 elsewhere -- so the accumulator keeps S = 16/MP
// groups apart and each group's scale and bias are applied once, in f32, when
// its period of steps ends (the "flush"). The group geometry (group size,
// slots, flush points) is fixed at compile time.
//
// Schedule: a workgroup (4 waves) owns a 16-row tile (two 8-row halves that
// may sit anywhere in the bank, e.g. an expert's value and gate rows). K is
// walked in passes; each wave takes a contiguous quarter of a pass. A wave
// loads its quarter of the 16 rows with 16-byte lanes laid out row-major (one
// load instruction covers whole 128-512 byte row segments), writes it to a
// private padded LDS block and reads it back in operand layout. Activations
// (as bf16 pairs in the MFMA's k order, with per-group sums) and the raw scale
// and bias planes of the tile are staged in LDS once per pass; the next pass's
// loads -- or the next tile's -- are issued into the same registers as soon as
// the current pass sits in LDS. The four waves' partial sums meet in LDS and
// are added in a fixed order before the D-ops.
#pragma once
#include "qmm_common.h"

namespace qmm {
namespace mfma {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kWg = 256;
constexpr int kRows = 16;   // tile rows (MFMA B columns)
constexpr int kStep = 128;  // k values per step (4 MFMAs)
constexpr int kBufNt = 2;   // buffer-load cache policy: nontemporal (streamed once)

// Plane flags of a tile op (runtime: they only touch staging and the flush).
enum : uint32_t {
    PLANE_BF16 = 1u << 0,      // scale/bias planes are bf16 (else f16)
    PLANE_BIASED = 1u << 1,    // bias plane present (else symmetric: -s * 2^(bits-1))
    PLANE_GROUP_OUT = 1u << 2  // group-output planes [G][N4] (else output-group [N][G])
};

__host__ __device__ inline uint32_t plane_flags(const AffineOp& op) {
    return (op.w_dt == STARK_QMM_BF16 ? PLANE_BF16 : 0u) |
           (op.corr_kind == STARK_QMM_CORRECTION_BIASES ? PLANE_BIASED : 0u) | (op.os == 1 ? PLANE_GROUP_OUT : 0u);
}

// Compile-time geometry. P1: pass length (k values of 4-bit codes) when
// MP*MB <= 2; wider activation tiles use shorter passes so the staged
// activations fit LDS. 8-bit codes take half the k per pass (same bytes).
template <int MP, int MB, int GS, int BITS, int P1>
struct Geo {
    static constexpr int S = 16 / MP;        // group slots per activation row
    static constexpr int MR = MP * MB;       // activation rows of the tile
    static constexpr int GPS = kStep / GS;   // groups per step
    static_assert(GS == 32 || GS == 64 || GS == 128, "group size");
    static_assert(S >= GPS, "a step's groups must fit the slots");
    static constexpr int PERIOD = S / GPS;   // steps between flushes
    static constexpr int PASS = (MR <= 2 ? P1 : (MR <= 8 ? 2048 : 1024)) * 4 / BITS;
    static constexpr int Q = PASS / 4;       // k values per wave per pass
    static constexpr int SEGB = Q * BITS / 8;  // bytes of a row per wave per pass
    static constexpr int NI = SEGB / 64;     // 16-byte code loads per lane per pass
    static constexpr int NSTEP = Q / kStep;  // MFMA steps per wave per pass
    static constexpr int ROWB = SEGB + 16;   // padded LDS row: the 16 operand rows hit distinct banks
    static constexpr int GPP = PASS / GS;    // groups per pass
    static constexpr int GPW = Q / GS;       // groups per wave per pass
    static constexpr int LPR = SEGB / 16;    // lanes per row segment of a code load
    static constexpr int RPI = 64 / LPR;     // rows per code load instruction
    // Activation window: one activation row stages the x of two passes at
    // once, so a K of up to XK is staged once per op and kept across the
    // tile's passes and the workgroup's next tiles of the same op.
    static constexpr int XK = (MR == 1 ? 2 : 1) * PASS;
    static constexpr int XV = MR * (XK / 8);  // activation vectors of a window
    static constexpr int XI = (XV + kWg - 1) / kWg;
    static_assert(NI >= 1 && RPI <= 8 && 8 % RPI == 0, "pass too short for 16 rows");
};

template <int MP, int MB, int GS, int BITS, int P1>
struct MfmaLds {
    using G = Geo<MP, MB, GS, BITS, P1>;
    u32x4 stage[4][kRows * G::ROWB / 16];     // per-wave code block [16][ROWB bytes]
    // a flush reads S slots from the wave's first group on; slots past the
    // wave's groups are read (and discarded), hence the S extra entries
    uint16_t sc[G::GPP + G::S][kRows];        // raw scale plane of the tile [group][row]
    uint16_t bi[G::GPP + G::S][kRows];        // raw bias plane
    // activation pairs per 8 values, in MFMA k order; rows padded by 16 bytes
    // so that the A rows one MFMA read touches (up to 8) start on distinct banks
    u32x4 xp[G::MR][G::XK / 8 + 1];
    float xs[G::MR][G::XK / GS + G::S];       // activation sum per group
    alignas(16) int xe[G::MR][G::XK / GS + G::S];  // 133 - E per group (activations staged as x * 2^E)
    float red[4][G::MR][kRows];               // per-wave partial outputs
    u32x4 zero[4];
};

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ float plane_f32(uint32_t h, bool bf) {
    return bf ? __uint_as_float(h << 16) : f16_bits_to_f32(h);
}

// Tile engine. A tile is described by
//   op     : codes / planes / activation base, K, group size, plane strides
//   nA, nB : bank rows of tile rows 0..7 and 8..15 (multiples of 8, nB >= nA)
//   M      : activation rows (<= MP*MB); xrow(m) = element offset of row m in op.x
// load() issues one pass's global loads into registers; run() walks every pass
// of the tile (calling next() once the last pass is in LDS, to issue the next
// tile's loads) and leaves the per-(activation row, tile row) sums in
// lds.red[wave][m][r] behind a barrier (add the four waves in order (0+1)+(2+3)).
// keep_x: the activations staged for the previous tile are this tile's too
// (same op, one pass): they are neither loaded nor staged.
template <int MP, int MB, int GS, int BITS, bool SIGNED, int P1>
struct TileEngine {
    using G = Geo<MP, MB, GS, BITS, P1>;
    static constexpr int S = G::S, MR = G::MR, PASS = G::PASS, Q = G::Q, SEGB = G::SEGB, NI = G::NI;
    static constexpr int NSTEP = G::NSTEP, PERIOD = G::PERIOD, GPS = G::GPS, GPP = G::GPP, GPW = G::GPW;
    static constexpr int ROWB = G::ROWB, LPR = G::LPR, RPI = G::RPI, XK = G::XK, XV = G::XV, XI = G::XI;
    static constexpr int GSH = GS == 32 ? 5 : GS == 64 ? 6 : 7;

    MfmaLds<MP, MB, GS, BITS, P1>& lds;
    uint32_t tid, lane, wave, j, kq, am, aslot, lcol;
    uint8_t* wstage;
    u32x4 w[NI];     // codes of the loaded pass
    u32x4 xv[XI];    // activations of the loaded window
    u32x4 msv, mbv;  // scale / bias vectors of the loaded pass

    __device__ __forceinline__ explicit TileEngine(MfmaLds<MP, MB, GS, BITS, P1>& l) : lds(l) {
        tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        j = lane & 15;   // B/C column (tile row)
        kq = lane >> 4;  // k quarter of a step
        am = j / S;      // A row j -> (activation row, slot)
        aslot = j % S;
        lcol = (lane % LPR) * 16;
        wstage = (uint8_t*)lds.stage[wave];
        if (tid < 4) lds.zero[tid] = u32x4{0, 0, 0, 0};
    }

    // Whether a pass stages activations, and which: the whole K when it fits
    // the window (at the first pass, unless kept from the previous tile),
    // else the pass's own k range.
    static __device__ __forceinline__ bool x_window(uint32_t K, uint32_t kbase, bool keep_x, uint32_t kvals,
                                                    uint32_t& xk0, uint32_t& xcnt) {
        const bool whole = K <= (uint32_t)XK;
        xk0 = whole ? 0 : kbase;
        xcnt = whole ? K : kvals;
        return !keep_x && (!whole || kbase == 0);
    }
    // first k of the staged window for a pass at kbase
    static __device__ __forceinline__ uint32_t x_offset(uint32_t K, uint32_t kbase) {
        return K <= (uint32_t)XK ? kbase : 0;
    }

    // Output-group plane rows are read as 16-byte vectors when every row of a
    // pass starts 16-byte aligned (8 groups at a time); otherwise the planes
    // are staged element by element.
    static __device__ __forceinline__ bool og_vec(const AffineOp& op, uint32_t gcnt) {
        return op.os % 8 == 0 && gcnt % 8 == 0 && (((uintptr_t)op.scales | (uintptr_t)op.corr) & 15) == 0;
    }

    // Issue every global load of pass `kbase` of a tile: codes through a buffer
    // resource starting at row nA (16-byte piece i*64 + lane of the wave's
    // row-major [16][SEGB] block; pieces past K get an offset beyond the
    // resource and read as zero), activations (vector v = tid + i*256 of the
    // [MR][PASS/8] table) and one scale and one bias vector per thread. No
    // value is selected here (a select would wait for the load): loads whose
    // slot is unused read from the array base and are never staged.
    template <class XRow>
    __device__ __forceinline__ void load(const AffineOp& op, uint32_t pf, uint32_t nA, uint32_t nB, uint32_t M,
                                         XRow xrow, uint32_t kbase, bool keep_x = false) {
        const uint32_t K = op.k, kvals = min((uint32_t)PASS, K - kbase);
        const uint32_t g0 = kbase >> GSH;
        const uint32_t row_bytes = K * BITS / 8;
        uint32_t xk0, xcnt;
        if (x_window(K, kbase, keep_x, kvals, xk0, xcnt)) {
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const uint32_t v = tid + i * kWg, m = v / (XK / 8), vi = v % (XK / 8);
                const bool ok = v < (uint32_t)XV && m < M && vi * 8 < xcnt;
                xv[i] = *(const u32x4*)((const uint16_t*)op.x + (ok ? xrow(m) + xk0 + vi * 8 : 0));
            }
        }
        const uint32_t gcnt = kvals >> GSH;
        size_t off;
        bool ok;
        if (pf & PLANE_GROUP_OUT) {  // [G][N4]: 8 rows of group tid/2 per vector
            ok = tid < gcnt * 2;
            off = (size_t)(g0 + (tid >> 1)) * op.gs + ((tid & 1) ? nB : nA);
        } else {  // [N][G]: 8 groups of row tid/(gcnt/8) per vector
            const uint32_t per_row = og_vec(op, gcnt) ? gcnt / 8 : 0;
            ok = per_row && tid < kRows * per_row;
            const uint32_t r = per_row ? tid / per_row : 0, g8 = per_row ? (tid % per_row) * 8 : 0;
            off = (size_t)(r < 8 ? nA + r : nB + r - 8) * op.os + g0 + g8;
        }
        off = ok ? off : 0;
        msv = *(const u32x4*)((const uint16_t*)op.scales + off);
        if (pf & PLANE_BIASED) mbv = *(const u32x4*)((const uint16_t*)op.corr + off);
        const uint32_t hi_skip = nB - nA - 8;  // extra rows between the two halves
        const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(op.codes + (size_t)nA * row_bytes), 0, (int)((nB - nA + 8) * row_bytes), 0x00020000);
        const uint32_t voff = (lane / LPR) * row_bytes + wave * SEGB + lcol;
        const uint32_t vo = wave * Q + lcol * 8 / BITS < kvals ? voff : 0x80000000u;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            w[i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           crs, vo, (i * RPI + (i * RPI >= 8 ? hi_skip : 0)) * row_bytes + kbase * BITS / 8, kBufNt));
    }

    // Stage the loaded pass into LDS (after a barrier when the previous pass's
    // LDS may still be read).
    __device__ __forceinline__ void stage(const AffineOp& op, uint32_t pf, uint32_t nA, uint32_t nB, uint32_t kbase,
                                          uint32_t gcnt, bool keep_x) {
        uint32_t xk0, xcnt;
        if (x_window(op.k, kbase, keep_x, min((uint32_t)PASS, op.k - kbase), xk0, xcnt)) {
#pragma unroll
            for (int i = 0; i < XI; ++i) {
                const uint32_t v = tid + i * kWg, m = v / (XK / 8), vi = v % (XK / 8);
                const u32x4 t = xv[i];
                // the group's exponent: its GS/8 vectors sit in consecutive lanes
                const int E = group_shift(group_max<GS / 8>(bf16x8_exp_max(t)));
                const float se = pow2i(E), so = BITS == 4 ? pow2i(E - 4) : se;
                float f[8];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    f[2 * e] = __uint_as_float(t[e] << 16) * se;
                    f[2 * e + 1] = __uint_as_float(t[e] & 0xffff0000u) * so;
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
                // the GS/8 vectors of a group sit in consecutive lanes
                sm = group_sum<GS / 8>(sm);
                if (v < (uint32_t)XV && (vi & (GS / 8 - 1)) == 0) {
                    lds.xs[m][(vi * 8) >> GSH] = sm;
                    lds.xe[m][(vi * 8) >> GSH] = 133 - E;
                }
            }
        }
        if (pf & PLANE_GROUP_OUT) {
            if (tid < gcnt * 2) {
                const uint32_t g = tid >> 1, h = (tid & 1) * 8;
                *(u32x4*)&lds.sc[g][h] = msv;
                if (pf & PLANE_BIASED) *(u32x4*)&lds.bi[g][h] = mbv;
            }
        } else if (!og_vec(op, gcnt)) {  // unaligned output-group rows: one element at a time
            const uint32_t g0 = kbase >> GSH;
            for (uint32_t q = tid; q < kRows * gcnt; q += kWg) {
                const uint32_t r = q / gcnt, g = q % gcnt;
                const size_t o = (size_t)(r < 8 ? nA + r : nB + r - 8) * op.os + g0 + g;
                lds.sc[g][r] = ((const uint16_t*)op.scales)[o];
                if (pf & PLANE_BIASED) lds.bi[g][r] = ((const uint16_t*)op.corr)[o];
            }
        } else {
            const uint32_t per_row = gcnt / 8;
            if (tid < kRows * per_row) {
                const uint32_t r = tid / per_row, g8 = (tid % per_row) * 8;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    lds.sc[g8 + e][r] = (uint16_t)(msv[e >> 1] >> (16 * (e & 1)));
                    if (pf & PLANE_BIASED) lds.bi[g8 + e][r] = (uint16_t)(mbv[e >> 1] >> (16 * (e & 1)));
                }
            }
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) *(u32x4*)(wstage + (i * RPI + lane / LPR) * ROWB + lcol) = w[i];
    }

    // One step: 4 MFMAs over this lane's 32 codes of row j (16 or 32 bytes).
    __device__ __forceinline__ void step(int s, const u32x4* const (&asrc)[MB], f32x4 (&C0)[MB], f32x4 (&C1)[MB]) {
        u32x4 wv[BITS / 4];
#pragma unroll
        for (int h = 0; h < BITS / 4; ++h)
            wv[h] = *(const u32x4*)(wstage + j * ROWB + s * (kStep * BITS / 8) + 4 * BITS * kq + 16 * h);
        u32x4 a[MB][4];
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int t = 0; t < 4; ++t) a[b][t] = asrc[b][t];
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
            for (int b = 0; b < MB; ++b) {
                f32x4& c = (t & 1) ? C1[b] : C0[b];
                c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[b][t]), bv, c, 0, 0, 0);
            }
        }
    }

    // Fold one period's accumulator rows into acc: C row i = (m, slot) holds
    // wave-pass group gbase + slot; acc += s * ldexp(C, 133 - E) + bias_term * xsum.
    // Groups at or past glim (past the wave's quarter or the K tail) are not
    // this wave's and are skipped.
    __device__ __forceinline__ void flush(uint32_t pf, uint32_t gbase, uint32_t glim, uint32_t xg0, f32x4 (&C0)[MB],
                                          f32x4 (&C1)[MB], f32x4 (&acc)[MB]) {
        const bool bf = pf & PLANE_BF16, biased = pf & PLANE_BIASED;
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const f32x4 c = C0[b] + C1[b];
            uint32_t g[4];
            float xsum[4];
            int xn[4];
            if (S >= 4) {
                const uint32_t g4 = gbase + (4 * kq) % S;
                const uint32_t m = b * MP + (4 * kq) / S;
                const f32x4 x4 = *(const f32x4*)&lds.xs[m][xg0 + g4];
                const i32x4 e4 = *(const i32x4*)&lds.xe[m][xg0 + g4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    g[q] = g4 + q;
                    xsum[q] = x4[q];
                    xn[q] = e4[q];
                }
            } else {  // S == 2: rows (2kq, gbase), (2kq, gbase+1), (2kq+1, gbase), (2kq+1, gbase+1)
                const uint32_t m = b * MP + 2 * kq;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    g[q] = gbase + (q & 1);
                    xsum[q] = lds.xs[m + (q >> 1)][xg0 + g[q]];
                    xn[q] = lds.xe[m + (q >> 1)][xg0 + g[q]];
                }
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float sc = plane_f32(lds.sc[g[q]][j], bf);
                const float bias = biased ? plane_f32(lds.bi[g[q]][j], bf) : -(float)(1 << (BITS - 1)) * sc;
                const float nv = fmaf(sc, ldexp_f32(c[q], xn[q]), fmaf(bias, xsum[q], acc[b][q]));
                acc[b][q] = g[q] < glim ? nv : acc[b][q];
            }
            C0[b] = C1[b] = f32x4{0, 0, 0, 0};
        }
    }

    // Compute one staged pass: NSTEP steps with flushes at period ends.
    // koff: first k of the pass within the staged activation window
    template <bool TAIL>
    __device__ __forceinline__ void compute(uint32_t pf, uint32_t M, uint32_t kvals, uint32_t gcnt, uint32_t koff,
                                            f32x4 (&acc)[MB]) {
        f32x4 C0[MB], C1[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) C0[b] = C1[b] = f32x4{0, 0, 0, 0};
        const uint32_t qbase = wave * Q;
        const uint32_t gw = qbase >> GSH;  // wave's first group within the pass
        const uint32_t glim = TAIL ? min(gcnt, gw + GPW) : gw + GPW;
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) {
            const uint32_t kloc = s * kStep + 32 * kq;  // wave-local k of this lane's 32 values
            const uint32_t lg = kloc >> GSH;            // wave-local group
            const u32x4* asrc[MB];
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                const uint32_t m = b * MP + am;
                bool act = (lg % S) == aslot && m < M;
                if (TAIL) act = act && qbase + kloc < kvals;
                asrc[b] = act ? &lds.xp[m][(koff + qbase + kloc) / 8] : lds.zero;
            }
            step(s, asrc, C0, C1);
            if ((s + 1) % PERIOD == 0 || s == NSTEP - 1)
                flush(pf, gw + (s / PERIOD) * S, glim, koff >> GSH, C0, C1, acc);
        }
    }

    // Parameters of the loads issued after a pass is staged: the tile's next
    // pass, or the first pass of the workgroup's next tile.
    struct NextLoad {
        const AffineOp* op;
        uint32_t pf, nA, nB, M, kbase;
        bool keep_x, other_op;  // other_op: activation rows are m * op->k, not xrow(m)
    };

    // Walk every pass of a tile whose first pass has been load()ed. next(nl)
    // fills nl with the next tile's first pass and returns true, or returns
    // false. Both kinds of refill go through one load() call: loads written
    // to the same registers from two call sites make the compiler join the
    // two sets of values with copies, and a copy waits for its load, which
    // would drain the prefetch.
    template <class XRow, class Next>
    __device__ __forceinline__ void run(const AffineOp& op, uint32_t pf, uint32_t nA, uint32_t nB, uint32_t M,
                                        XRow xrow, Next next, bool keep_x = false) {
        const uint32_t K = op.k;
        f32x4 acc[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) acc[b] = f32x4{0, 0, 0, 0};
        for (uint32_t kbase = 0; kbase < K; kbase += PASS) {
            const uint32_t kvals = min((uint32_t)PASS, K - kbase);
            const uint32_t gcnt = kvals >> GSH;  // K % GS == 0
            if (kbase) __syncthreads();          // every wave finished the previous pass's LDS
            stage(op, pf, nA, nB, kbase, gcnt, keep_x && kbase == 0);
            __syncthreads();
            // the registers are free: the next pass's (or tile's) loads fly while this pass computes
            NextLoad nl{&op, pf, nA, nB, M, kbase + PASS, false, false};
            if (kbase + PASS < K || next(nl))
                load(*nl.op, nl.pf, nl.nA, nl.nB, nl.M,
                     [&](uint32_t m) { return nl.other_op ? (size_t)m * nl.op->k : xrow(m); }, nl.kbase, nl.keep_x);
            const uint32_t koff = x_offset(K, kbase);
            if (kvals == (uint32_t)PASS)
                compute<false>(pf, M, kvals, gcnt, koff, acc);
            else
                compute<true>(pf, M, kvals, gcnt, koff, acc);
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
template <int MP, int MB, int GS, int BITS, bool SIGNED, int P1, class XRow>
__device__ __forceinline__ void mfma_tile(const AffineOp& op, uint32_t pf, uint32_t nA, uint32_t nB, uint32_t M,
                                          XRow xrow, MfmaLds<MP, MB, GS, BITS, P1>& lds) {
    TileEngine<MP, MB, GS, BITS, SIGNED, P1> e(lds);
    e.load(op, pf, nA, nB, M, xrow, 0);
    e.run(op, pf, nA, nB, M, xrow, [](typename TileEngine<MP, MB, GS, BITS, SIGNED, P1>::NextLoad&) { return false; });
}

}  // namespace mfma
}  // namespace qmm
