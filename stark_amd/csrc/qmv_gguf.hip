// GGUF block-format matvec / small-M product (Q8_0 = kind 8, Q4_K = kind 12)
// on the gfx950 matrix cores, for the hybrid operator's f32 activations.
//
// Dequantisation is the reference's decode_block
// (crates/stark-engine/src/engine/hybrid/weights.rs:2923-3012):
//   Q8_0: w_i = f16(d) * int8(q_i)                          (32 values, 34 bytes)
//   Q4_K: w   = f16(d) * sc * q - f16(dmin) * m, (sc, m) = scale_min(scales, j)
//         (weights.rs:2908-2921), 8 sub-blocks of 32 values, 144 bytes
// Both products are exact in f32, so the factored per-group form
//   sum_i w_i x_i = d * sum_i q_i x_i                                          (Q8_0)
//   (d*sc_j) * sum_{i in j} q_i x_i - (dmin*m_j) * sum_{i in j} x_i            (Q4_K)
// reassociates only the additions, as the reference Metal kernels do
// (crates/stark-engine/src/engine/hybrid/packed_q8_grouped8_matvec.metal:11-82).
//
// Matrix-core form (the affine engine's, mfma_tile.h): sum(q * x) per group on
// v_mfma_f32_16x16x32_bf16 with the codes as raw bf16 bit patterns (p < 256 is
// p * 2^-133; Q8_0 codes enter as q + 128, the -128 folded into the bias
// term; Q4_K high nibbles enter as 16 q with their activations scaled by
// 2^-4), B columns = the 16 weight rows of a tile, A rows = (activation part,
// group slot). The activations are f32, staged per group as x * 2^E (a
// per-group exponent, group_shift in qmm_common.h): each row enters as two
// bf16 rows, hi = bf16(x 2^E) and lo = bf16(x 2^E - hi), so
// |x 2^E - hi - lo| <= 2^-18 |x 2^E| and the products stay exact; the two
// parts' sums meet in the reduction, brought back by ldexp(., 133 - E). Groups are
// the 32-value (sub-)blocks; per-group scale and bias are applied once in f32
// when a period of steps ends.
//
// Schedule: one workgroup (4 waves) per 16-row tile; K in passes, each wave a
// quarter of a pass; a wave loads its quarter of the 16 rows' raw block bytes
// with 16-byte loads (row-major), writes them to a padded LDS block and reads
// its operands from there (Q8_0 code runs start 2 bytes into a block and are
// realigned with v_alignbyte). Block headers are decoded to per-group f32
// scale and bias in LDS once per pass. The next pass's loads are issued as
// soon as the current pass sits in LDS.
#include <algorithm>
#include "mfma_tile.h"

namespace qmm {

namespace {

using mfma::bf16x8;
using mfma::f32x4;
using mfma::kBufNt;
using mfma::kRows;
using mfma::kStep;
using mfma::kWg;
using mfma::perm;

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


// ------------------------------------------------------------------ geometry
constexpr int kGgMaxRun = 3;  // dense form: tile pairs per workgroup, at most
// M real rows take MR = 2M activation rows (hi/lo); MP rows per MFMA block.
template <int KIND, int MP, int MB>
struct GGeo {
    static constexpr int BE = KIND == 12 ? 256 : 32;   // values per block
    static constexpr int BB = KIND == 12 ? 144 : 34;   // bytes per block
    static constexpr int MR = MP * MB;
    static constexpr int RR = MR / 2;                  // real rows
    // MP == 16 is the dense form: all 16 activation rows in every MFMA, one
    // MFMA per 32-value group (no slots; S only sizes the LDS arrays)
    static constexpr bool DENSE = MP == 16;
    static constexpr int S = DENSE ? 4 : 16 / MP;      // group slots per activation row
    // the dense form runs TPW 16-row tiles per pass under one activation stage
    static constexpr int TPW = DENSE ? 2 : 1;
    static constexpr int GS = 32;
    static constexpr int GPS = kStep / GS;             // 4 groups per step
    static_assert(S >= GPS, "slots");
    static constexpr int PERIOD = S / GPS;
    // k values per pass; Q8_0 at M = 1 takes 1024 (four passes at K = 4096,
    // so less of the last pass's compute trails the loads: +5%; Q4_K lost 10%)
    static constexpr int PASS = (MR <= 2 && KIND == 8) ? 1024 : MR <= 4 ? 2048 : 1024;
    static constexpr int Q = PASS / 4;                  // per wave
    static constexpr int BPW = Q / BE;                  // blocks per wave per pass
    static constexpr int SEGB = BPW * BB;               // bytes of a row per wave per pass
    static constexpr int PPR = SEGB / 16;               // 16-byte pieces per row
    static constexpr int NI = (kRows * PPR + 63) / 64;  // loads per lane
    // LDS row: an odd number of 16-byte chunks, so that 8 rows read at one
    // offset (a column of the code tile) fall on 8 distinct groups of 4 banks
    static constexpr int ROWB = (SEGB / 16) % 2 ? SEGB : SEGB + 16;
    static constexpr int NSTEP = Q / kStep;
    static constexpr int GPP = PASS / GS, GPW = Q / GS;
    static constexpr int GX = DENSE ? GPP : GPP + S;    // group entries of the LDS tables
    static constexpr int XV = RR * (PASS / 8);          // 8-value activation chunks per pass
    static constexpr int XI = (XV + kWg - 1) / kWg;
    static_assert(SEGB % 16 == 0 && BPW >= 1, "pass geometry");
};

template <int KIND, int MP, int MB>
struct GLds {
    using G = GGeo<KIND, MP, MB>;
    union {
        u32x4 stage[G::TPW][4][kRows * G::ROWB / 16];  // raw block bytes, per tile and wave [16][ROWB]
        float red[G::TPW][4][G::RR][kRows];            // per-wave results, after the last pass
    };
    float sc[G::TPW][G::GX][kRows];  // per (group, row) scale
    float bi[G::TPW][G::GX][kRows];  // per (group, row) bias term
    // activation rows (hi, lo per real row), 8-bit pair order; rows padded by
    // 64 bytes (16 banks) so that the 16 rows one MFMA A read touches fall on
    // two bank offsets instead of one
    u32x4 xp[G::MR][G::PASS / 8 + 4];
    // per-group activation sums and 133 - E (activations staged as x * 2^E):
    // per A row in the slot form; per real row (hi + lo) in the dense form,
    // whose flush adds the two parts anyway (this keeps two workgroups per CU),
    // with rows padded to an odd length there (the dense flush reads rows 2kq
    // and 2kq + 1 of one group: four banks, not one)
    float xs[G::DENSE ? G::RR : G::MR][G::GX + (G::DENSE ? 1 : 0)];
    alignas(16) int xe[G::DENSE ? G::RR : G::MR][G::GX + (G::DENSE ? 1 : 0)];
    u32x4 zero[4];
};

// two f32 to bf16 (round to nearest even) in one word, the first in the low half
__device__ __forceinline__ uint32_t bf16_pack(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// One tile of a GGUF product: op rows n0..n0+15, real activation rows 0..M-1.
template <int KIND, int MP, int MB>
struct GEngine {
    using G = GGeo<KIND, MP, MB>;
    static constexpr int S = G::S, MR = G::MR, RR = G::RR, PASS = G::PASS, Q = G::Q, BE = G::BE, BB = G::BB;
    static constexpr int SEGB = G::SEGB, PPR = G::PPR, NI = G::NI, ROWB = G::ROWB, NSTEP = G::NSTEP;
    static constexpr int PERIOD = G::PERIOD, GPP = G::GPP, GPW = G::GPW, XV = G::XV, XI = G::XI, BPW = G::BPW;
    static constexpr int TPW = G::TPW;

    GLds<KIND, MP, MB>& lds;
    uint32_t tid, lane, wave, j, kq, am, aslot;
    u32x4 w[TPW][NI];
    u32x4 xa[XI], xb[XI];  // 8 f32 activations per chunk

    __device__ __forceinline__ explicit GEngine(GLds<KIND, MP, MB>& l) : lds(l) {
        tid = threadIdx.x;
        lane = tid & 63;
        wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        j = lane & 15;
        kq = lane >> 4;
        am = j / S;
        aslot = j % S;
        if (tid < 4) lds.zero[tid] = u32x4{0, 0, 0, 0};
    }

    // Issue the pass's loads: raw block bytes of the wave's quarter of the 16
    // rows (pieces past the pass's blocks read as zero through the buffer
    // resource) and the f32 activation chunks.
    __device__ __forceinline__ void load(const GgufOp& op, const uint32_t (&n0)[TPW], uint32_t M, uint32_t kbase) {
        load_codes(op, n0, kbase);
        load_x(op, M, kbase);
    }
    __device__ __forceinline__ void load_codes(const GgufOp& op, const uint32_t (&n0)[TPW], uint32_t kbase) {
        const uint32_t K = op.k, kvals = min((uint32_t)PASS, K - kbase);
        const uint32_t row_bytes = K / BE * BB;
        const uint32_t vbytes = kvals / BE * BB;  // valid bytes of a row in this pass
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const __amdgpu_buffer_rsrc_t crs = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(op.blocks + (size_t)n0[tt] * row_bytes), 0, (int)(kRows * row_bytes), 0x00020000);
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t p = i * 64 + lane, r = p / PPR, c = (p % PPR) * 16;
                const uint32_t col = wave * SEGB + c;
                const uint32_t vo = p < (uint32_t)(kRows * PPR) && col < vbytes
                                        ? r * row_bytes + col + kbase / BE * BB
                                        : 0x80000000u;
                w[tt][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(crs, vo, 0, kBufNt));
            }
        }
    }
    __device__ __forceinline__ void load_x(const GgufOp& op, uint32_t M, uint32_t kbase) {
        const uint32_t K = op.k, kvals = min((uint32_t)PASS, K - kbase);
        // activations: chunks past the rows, the pass or K read zeros from past the resource
        const __amdgpu_buffer_rsrc_t xrs =
            __builtin_amdgcn_make_buffer_rsrc((void*)op.x, 0, (int)min((uint64_t)M * K * 4, (uint64_t)0x7fffffffu), 0x00020000);
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t v = tid + i * kWg, r = v / (PASS / 8), c = v % (PASS / 8);
            const bool ok = v < (uint32_t)XV && r < M && c * 8 < kvals;
            const uint32_t xo = ok ? (r * K + kbase + c * 8) * 4 : 0x80000000u;
            xa[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0));
            xb[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 16, 0, 0));
        }
    }

    // Stage codes and activations, then (after a barrier) decode the pass's
    // block headers into per-group scale and bias.
    __device__ __forceinline__ void stage(uint32_t kvals, uint32_t M, uint32_t* status) {
        stage_codes();
        stage_x(kvals, M, status);
    }
    __device__ __forceinline__ void stage_codes() {
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            uint8_t* ws = (uint8_t*)lds.stage[tt][wave];
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const uint32_t p = i * 64 + lane;
                if (p < (uint32_t)(kRows * PPR)) *(u32x4*)(ws + (p / PPR) * ROWB + (p % PPR) * 16) = w[tt][i];
            }
        }
    }
    __device__ __forceinline__ void stage_x(uint32_t kvals, uint32_t M, uint32_t* status) {
        bool bad = false;
#pragma unroll
        for (int i = 0; i < XI; ++i) {
            const uint32_t v = tid + i * kWg, r = v / (PASS / 8), c = v % (PASS / 8);
            float x[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = __uint_as_float(xa[i][e]);
                x[4 + e] = __uint_as_float(xb[i][e]);
            }
            // per-group exponent E (group_shift): the 4 chunks of a 32-value
            // group sit in consecutive lanes; Q4_K values 32..63 of every 64
            // meet the high nibbles (16 q) and are staged at x * 2^(E-4)
            const uint32_t fe = f32x8_exp_max(xa[i], xb[i]);
            const int E = group_shift(group_max<4>(fe));
            const int Es = (KIND == 12 && ((c * 8) & 32)) ? E - 4 : E;
            const float sc = pow2i(Es);
            // a value is infinite or NaN exactly when its exponent field is 255
            bad |= v < (uint32_t)XV && r < M && c * 8 < kvals && fe == 255u;
            // hi = bf16(x sc) = bf16(x) sc and lo = bf16(x sc - hi) through the
            // hardware round-to-nearest-even pack; sc is a power of two, so the
            // sums of the scaled parts times 1/sc are the sums of the parts
            float shi = 0.0f, slo = 0.0f;
            u32x4 ph, pl;  // 8-bit pair order (x0,x2)(x1,x3)(x4,x6)(x5,x7)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e0 = (q & 1) + 4 * (q >> 1), e1 = e0 + 2;
                const float a0 = x[e0] * sc, a1 = x[e1] * sc;
                const uint32_t hb = bf16_pack(a0, a1);
                const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xffff0000u);
                const float l0 = a0 - h0, l1 = a1 - h1;
                ph[q] = hb;
                pl[q] = bf16_pack(l0, l1);
                shi += h0 + h1;
                slo += __uint_as_float(pl[q] << 16) + __uint_as_float(pl[q] & 0xffff0000u);
            }
            shi = ldexp_f32(shi, -Es);
            slo = ldexp_f32(slo, -Es);
            // the 4 chunks of a 32-value group sit in consecutive lanes
            shi = group_sum<4>(shi);
            slo = group_sum<4>(slo);
            if (v < (uint32_t)XV) {
                lds.xp[2 * r][c] = ph;
                lds.xp[2 * r + 1][c] = pl;
                if ((c & 3) == 0) {
                    if constexpr (G::DENSE) {
                        lds.xs[r][c >> 2] = shi + slo;
                        lds.xe[r][c >> 2] = 133 - E;
                    } else {
                        lds.xs[2 * r][c >> 2] = shi;
                        lds.xs[2 * r + 1][c >> 2] = slo;
                        lds.xe[2 * r][c >> 2] = 133 - E;
                        lds.xe[2 * r + 1][c >> 2] = 133 - E;
                    }
                }
            }
        }
        // the reference's input finite check (weight_metal.rs:435-440)
        if (__any(bad) && lane == 0) atomicOr(status, 1u);
    }

    // Per-group scale and bias of the pass from the staged block headers.
    __device__ __forceinline__ void decode_meta(uint32_t kvals) {
        const uint32_t nblk = kvals / BE;  // blocks of a row in this pass
        if (KIND == 12) {
            for (uint32_t t = tid; t < kRows * nblk * TPW; t += kWg) {
                const uint32_t r = t % kRows, b = (t / kRows) % nblk, tt = t / (kRows * nblk);
                const uint8_t* blk = (const uint8_t*)lds.stage[tt][b / BPW] + r * ROWB + (b % BPW) * BB;
                const u32x4 h = *(const u32x4*)blk;
                const float d = f16_bits_to_f32(h[0] & 0xffffu), dmin = f16_bits_to_f32(h[0] >> 16);
                const uint32_t q3[3] = {h[1], h[2], h[3]};
#pragma unroll
                for (uint32_t jj = 0; jj < 8; ++jj) {
                    float scj, mj;
                    scale_min(q3, jj, &scj, &mj);
                    lds.sc[tt][b * 8 + jj][r] = d * scj;
                    lds.bi[tt][b * 8 + jj][r] = -(dmin * mj);
                }
            }
        } else {
            for (uint32_t t = tid; t < kRows * nblk * TPW; t += kWg) {
                const uint32_t r = t % kRows, b = (t / kRows) % nblk, tt = t / (kRows * nblk);
                const uint8_t* blk = (const uint8_t*)lds.stage[tt][b / BPW] + r * ROWB + (b % BPW) * BB;
                const float d = f16_bits_to_f32(*(const uint16_t*)blk);
                lds.sc[tt][b][r] = d;
                lds.bi[tt][b][r] = -128.0f * d;  // codes enter as q + 128
            }
        }
    }

    // This lane's 32 codes of step s as 4 MFMA operands, and each operand's
    // wave-local group and first value.
    __device__ __forceinline__ void codes(int s, u32x4 (&bq)[4], uint32_t (&grp)[4], uint32_t (&e0)[4]) const {
        const uint8_t* row = (const uint8_t*)lds.stage[0][wave] + j * ROWB;
        if (KIND == 12) {
            const uint32_t sb = s / 2, p = 2 * (s % 2) + kq / 2, l0 = 16 * (kq % 2);
            const u32x4 u = *(const u32x4*)(row + sb * BB + 16 + p * 32 + l0);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t a = u[2 * (t >> 1)], b = u[2 * (t >> 1) + 1];
                const uint32_t m = (t & 1) ? 0x00F000F0u : 0x000F000Fu;
                bq[t][0] = a & m;
                bq[t][1] = (a >> 8) & m;
                bq[t][2] = b & m;
                bq[t][3] = (b >> 8) & m;
                grp[t] = sb * 8 + 2 * p + (t & 1);
                e0[t] = sb * 256 + p * 64 + 32 * (t & 1) + l0 + 8 * (t >> 1);
            }
        } else {
            const uint32_t lb = s * 4 + kq;                 // block of this lane
            const uint32_t start = lb * BB + 2;             // first code byte
            const uint32_t* base = (const uint32_t*)(row + (start & ~3u));
            const uint32_t sh = start & 3u;                 // 0 or 2
            uint32_t d9[9];
#pragma unroll
            for (int q = 0; q < 9; ++q) d9[q] = base[q];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t a = __builtin_amdgcn_alignbyte(d9[2 * t + 1], d9[2 * t], sh) ^ 0x80808080u;
                uint32_t b = __builtin_amdgcn_alignbyte(d9[2 * t + 2], d9[2 * t + 1], sh) ^ 0x80808080u;
                bq[t][0] = a & 0x00FF00FFu;
                bq[t][1] = (a >> 8) & 0x00FF00FFu;
                bq[t][2] = b & 0x00FF00FFu;
                bq[t][3] = (b >> 8) & 0x00FF00FFu;
                grp[t] = lb;
                e0[t] = lb * 32 + 8 * t;
            }
        }
    }

    __device__ __forceinline__ void flush(uint32_t gbase, uint32_t glim, f32x4 (&C0)[MB], f32x4 (&C1)[MB],
                                          f32x4 (&acc)[MB]) {
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const f32x4 c = C0[b] + C1[b];
            const uint32_t g4 = gbase + (4 * kq) % S;
            const uint32_t a = b * MP + (4 * kq) / S;
            const f32x4 x4 = *(const f32x4*)&lds.xs[a][g4];
            const mfma::i32x4 e4 = *(const mfma::i32x4*)&lds.xe[a][g4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float nv = fmaf(lds.sc[0][g4 + q][j], ldexp_f32(c[q], e4[q]),
                                      fmaf(lds.bi[0][g4 + q][j], x4[q], acc[b][q]));
                acc[b][q] = g4 + q < glim ? nv : acc[b][q];
            }
            C0[b] = C1[b] = f32x4{0, 0, 0, 0};
        }
    }

    // Dense form: this lane's 8 codes (values 8*kq .. 8*kq+7) of wave-local
    // group gl as one MFMA B operand in 8-bit pair order.
    __device__ __forceinline__ u32x4 codes_dense(int tt, uint32_t gl) const {
        const uint8_t* row = (const uint8_t*)lds.stage[tt][wave] + j * ROWB;
        uint32_t a, b, m;
        if (KIND == 12) {
            const uint32_t sb = gl / 8, jj = gl % 8;  // super-block, sub-block
            const uint2 u = *(const uint2*)(row + sb * BB + 16 + (jj / 2) * 32 + 8 * kq);
            a = u.x;
            b = u.y;
            m = (jj & 1) ? 0x00F000F0u : 0x000F000Fu;  // high nibbles stay at bit 4 (16 q)
        } else {
            const uint32_t start = gl * BB + 2 + 8 * kq;  // first code byte
            const uint32_t* base = (const uint32_t*)(row + (start & ~3u));
            const uint32_t sh = start & 3u;               // 0 or 2
            a = __builtin_amdgcn_alignbyte(base[1], base[0], sh) ^ 0x80808080u;  // q + 128
            b = __builtin_amdgcn_alignbyte(base[2], base[1], sh) ^ 0x80808080u;
            m = 0x00FF00FFu;
        }
        return u32x4{a & m, (a >> 8) & m, b & m, (b >> 8) & m};
    }

    // Dense form: per step and tile 4 groups, one MFMA each over all 16
    // activation rows (A row i = real row i/2, hi or lo; the A operand serves
    // every tile), flushed at once: lane (j, kq) holds C rows 4kq .. 4kq+3,
    // i.e. real rows 2kq and 2kq+1 with their hi and lo parts, which it adds
    // before the group's scale and bias.
    template <bool TAIL>
    __device__ __forceinline__ void compute_dense(uint32_t kvals, f32x4 (&acc)[TPW]) {
        const uint32_t qbase = wave * Q, gw = wave * GPW;
        const uint32_t glim = TAIL ? min(kvals / 32, gw + GPW) : gw + GPW;
        const uint32_t ar = j;  // A row of this lane
        const uint32_t m0 = 2 * kq, m1 = 2 * kq + 1;
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) {
            u32x4 a[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t gl = 4 * s + t;
                const bool act = !TAIL || gw + gl < glim;
                a[t] = act ? lds.xp[ar][(qbase + gl * 32 + 8 * kq) / 8] : lds.zero[0];
            }
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                f32x4 c[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const u32x4 bq = codes_dense(tt, 4 * s + t);
                    c[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[t]),
                                                                 __builtin_bit_cast(bf16x8, bq), f32x4{0, 0, 0, 0},
                                                                 0, 0, 0);
                }
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t g = gw + 4 * s + t;
                    if (TAIL && g >= glim) continue;
                    const float sc = lds.sc[tt][g][j], bi = lds.bi[tt][g][j];
                    const float x0 = lds.xs[m0][g], x1 = lds.xs[m1][g];
                    const int n0 = lds.xe[m0][g], n1 = lds.xe[m1][g];
                    acc[tt][0] = fmaf(sc, ldexp_f32(c[t][0] + c[t][1], n0), fmaf(bi, x0, acc[tt][0]));
                    acc[tt][1] = fmaf(sc, ldexp_f32(c[t][2] + c[t][3], n1), fmaf(bi, x1, acc[tt][1]));
                }
            }
        }
    }

    template <bool TAIL>
    __device__ __forceinline__ void compute(uint32_t M, uint32_t kvals, f32x4 (&acc)[MB]) {
        f32x4 C0[MB], C1[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) C0[b] = C1[b] = f32x4{0, 0, 0, 0};
        const uint32_t qbase = wave * Q, gw = wave * GPW;
        const uint32_t glim = TAIL ? min(kvals / 32, gw + GPW) : gw + GPW;
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) {
            u32x4 bq[4];
            uint32_t grp[4], e0[4];
            codes(s, bq, grp, e0);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int b = 0; b < MB; ++b) {
                    const uint32_t r = b * (MP / 2) + am / 2;  // real row of A row j
                    bool act = grp[t] % S == aslot && r < M;
                    if (TAIL) act = act && qbase + e0[t] < kvals;
                    const u32x4 a = act ? lds.xp[b * MP + am][(qbase + e0[t]) / 8] : lds.zero[0];
                    f32x4& cc = (t & 1) ? C1[b] : C0[b];
                    cc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                               __builtin_bit_cast(bf16x8, bq[t]), cc, 0, 0, 0);
                }
            }
            if ((s + 1) % PERIOD == 0 || s == NSTEP - 1) flush(gw + (s / PERIOD) * S, glim, C0, C1, acc);
        }
    }

    // Dense form, a run of cnt tile pairs (pair0 ..) pass-major: step s is
    // pass s / cnt of pair s % cnt; a pass's activations are converted and
    // staged at its first step and serve every pair of the run (their loads
    // are issued right after that staging, a pass ahead); a step's codes are
    // issued a step ahead. Pair t accumulates in acc[t]. Runs of more than one
    // pair need K % PASS == 0 (only a one-pair run has a tail pass).
    template <int RUN>
    __device__ __forceinline__ void run_runs(const GgufOp& op, uint32_t pair0, uint32_t cnt, uint32_t M,
                                             uint32_t* status, f32x4 (&acc)[RUN][TPW]) {
        static_assert(G::DENSE, "runs are the dense form's");
        const uint32_t K = op.k, N = op.n, passes = (K + PASS - 1) / PASS, steps = passes * cnt;
        const auto rows = [&](uint32_t t, uint32_t (&n0)[TPW]) {
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) n0[tt] = min(kRows * (TPW * (pair0 + t) + tt), N - kRows);
        };
#pragma unroll
        for (int r = 0; r < RUN; ++r)
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) acc[r][tt] = f32x4{0, 0, 0, 0};
        uint32_t n0[TPW];
        rows(0, n0);
        load_codes(op, n0, 0);
        load_x(op, M, 0);
        uint32_t p = 0, t = 0;
        for (uint32_t s = 0; s < steps; ++s) {
            const uint32_t kbase = p * PASS, kvals = min((uint32_t)PASS, K - kbase);
            if (s) __syncthreads();  // every wave finished the previous step's LDS
            stage_codes();
            if (t == 0) {
                stage_x(kvals, M, status);
                if (p + 1 < passes) load_x(op, M, kbase + PASS);
            }
            __syncthreads();
            if (s + 1 < steps) {
                uint32_t m0[TPW];
                rows(t + 1 < cnt ? t + 1 : 0, m0);
                load_codes(op, m0, (t + 1 < cnt ? p : p + 1) * PASS);
            }
            decode_meta(kvals);
            __syncthreads();
            if (t == 0) {
                if (kvals == (uint32_t)PASS)
                    compute_dense<false>(kvals, acc[0]);
                else
                    compute_dense<true>(kvals, acc[0]);
            } else {
#pragma unroll
                for (int r = 1; r < RUN; ++r)
                    if (t == (uint32_t)r) compute_dense<false>(kvals, acc[r]);
            }
            if (++t == cnt) t = 0, ++p;
        }
    }

    __device__ __forceinline__ void run(const GgufOp& op, const uint32_t (&n0)[TPW], uint32_t M, uint32_t* status) {
        const uint32_t K = op.k;
        f32x4 acc[MB * TPW];
#pragma unroll
        for (int b = 0; b < MB * TPW; ++b) acc[b] = f32x4{0, 0, 0, 0};
        load(op, n0, M, 0);
        for (uint32_t kbase = 0; kbase < K; kbase += PASS) {
            const uint32_t kvals = min((uint32_t)PASS, K - kbase);
            if (kbase) __syncthreads();
            stage(kvals, M, status);
            __syncthreads();
            if (kbase + PASS < K) load(op, n0, M, kbase + PASS);
            decode_meta(kvals);
            __syncthreads();
            if constexpr (G::DENSE) {
                if (kvals == (uint32_t)PASS)
                    compute_dense<false>(kvals, acc);
                else
                    compute_dense<true>(kvals, acc);
            } else {
                if (kvals == (uint32_t)PASS)
                    compute<false>(M, kvals, acc);
                else
                    compute<true>(M, kvals, acc);
            }
        }
        __syncthreads();  // the results overwrite the code stage
        if constexpr (G::DENSE) {  // real rows 2kq and 2kq+1 of column j
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                lds.red[tt][wave][2 * kq][j] = acc[tt][0];
                lds.red[tt][wave][2 * kq + 1][j] = acc[tt][1];
            }
            __syncthreads();
            return;
        }
        // lane's slots sum to one activation row's share; hi and lo rows meet
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            float v = (acc[b][0] + acc[b][1]) + (acc[b][2] + acc[b][3]);
            if (S == 8) {  // kq 0,1: hi; kq 2,3: lo
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                if (kq == 0) lds.red[0][wave][b * (MP / 2)][j] = v;
            } else {  // S == 4: lane row a = kq; real row kq / 2
                v += __shfl_xor(v, 16, 64);
                if ((kq & 1) == 0) lds.red[0][wave][b * (MP / 2) + kq / 2][j] = v;
            }
        }
        __syncthreads();
    }
};

template <int KIND, int MP, int MB>
__global__ __launch_bounds__(kWg) __attribute__((amdgpu_waves_per_eu(MB >= 4 ? 2 : (MB >= 2 || MP >= 4 || KIND == 8) ? 2 : 3))) void gguf_mfma(GgufBatch batch) {
    (void)batch;
    __shared__ GLds<KIND, MP, MB> lds;
    const GgufBatch* kb = (const GgufBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t oi = 0;
    for (uint32_t i = 1; i < kb->count; ++i)
        if (blockIdx.x >= kb->op[i].block_begin) oi = i;
    const GgufOp& op = kb->op[oi];
    const uint32_t N = op.n;
    constexpr int TPW = GGeo<KIND, MP, MB>::TPW, RR = MP * MB / 2;
    if constexpr (GGeo<KIND, MP, MB>::DENSE) {
        // a run of up to kGgMaxRun tile pairs per workgroup (op.run pairs; the
        // last run of an op may be shorter)
        const uint32_t pair0 = (blockIdx.x - op.block_begin) * op.run;
        const uint32_t cnt = min(op.run, (N + kRows * TPW - 1) / (kRows * TPW) - pair0);
        GEngine<KIND, MP, MB> e(lds);
        f32x4 acc[kGgMaxRun][TPW];
        e.template run_runs<kGgMaxRun>(op, pair0, cnt, op.m, kb->status, acc);
#pragma unroll
        for (int r = 0; r < kGgMaxRun; ++r) {
            if ((uint32_t)r >= cnt) break;
            __syncthreads();  // the results overwrite the code stage / the previous pair's results
            const uint32_t j = threadIdx.x & 15, kq = (threadIdx.x & 63) >> 4, wave = threadIdx.x >> 6;
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {  // real rows 2kq and 2kq+1 of column j
                lds.red[tt][wave][2 * kq][j] = acc[r][tt][0];
                lds.red[tt][wave][2 * kq + 1][j] = acc[r][tt][1];
            }
            __syncthreads();
            const uint32_t t0 = kRows * TPW * (pair0 + r);
            for (uint32_t t = threadIdx.x; t < (uint32_t)(TPW * RR * kRows); t += kWg) {
                const uint32_t tt = t / (RR * kRows), m = (t / kRows) % RR, rr = t % kRows;
                const uint32_t n = min(t0 + kRows * tt, N - kRows) + rr;
                if (m >= op.m || n < t0 + kRows * tt) continue;
                const float v = (lds.red[tt][0][m][rr] + lds.red[tt][1][m][rr]) +
                                (lds.red[tt][2][m][rr] + lds.red[tt][3][m][rr]);
                store_from_f32(op.d, op.d_dt, (size_t)m * N + n, v);
            }
        }
        return;
    }
    // tile tt covers rows n0[tt] .. +15 and writes those from t0 + 16 tt on; a
    // tile past N moves back to end at N, so every row is written once
    const uint32_t t0 = (blockIdx.x - op.block_begin) * kRows * TPW;
    uint32_t n0[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) n0[tt] = min(t0 + kRows * tt, N - kRows);
    GEngine<KIND, MP, MB> e(lds);
    e.run(op, n0, op.m, kb->status);
    for (uint32_t t = threadIdx.x; t < (uint32_t)(TPW * RR * kRows); t += kWg) {
        const uint32_t tt = t / (RR * kRows), m = (t / kRows) % RR, r = t % kRows;
        const uint32_t n = min(t0 + kRows * tt, N - kRows) + r;
        if (m >= op.m || n < t0 + kRows * tt) continue;
        const float v = (lds.red[tt][0][m][r] + lds.red[tt][1][m][r]) + (lds.red[tt][2][m][r] + lds.red[tt][3][m][r]);
        store_from_f32(op.d, op.d_dt, (size_t)m * N + n, v);
    }
}

template <int KIND, int MP, int MB>
stark_qmm_status launch_mfma(const GgufOp* ops, uint32_t count, uint32_t* status, hipStream_t stream) {
    if (count > (uint32_t)kMaxBatchOps) return STARK_QMM_INVALID_ARGUMENT;  // the batch holds kMaxBatchOps
    // longest K first: the workgroups with the most passes are dispatched first
    std::vector<GgufOp> sorted(ops, ops + count);
    std::stable_sort(sorted.begin(), sorted.end(), [](const GgufOp& a, const GgufOp& b) { return a.k > b.k; });
    using G = GGeo<KIND, MP, MB>;
    GgufBatch batch{};
    batch.status = status;
    // Dense form: runs of tile pairs, so that one activation conversion serves
    // up to kGgMaxRun pairs. The run length of an op is the launch's pass
    // count per resident workgroup (two per CU) over the op's passes, as in
    // the small-M kernel: a launch with fewer pairs than workgroup slots (one
    // product of N = 12288) keeps one pair per workgroup.
    uint64_t per_wg = 1;
    if constexpr (G::DENSE) {
        int dev = 0, cus = 0;
        QMM_HIP_CHECK(hipGetDevice(&dev));
        QMM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        uint64_t units = 0;
        for (uint32_t i = 0; i < count; ++i)
            units += (uint64_t)((sorted[i].n + kRows * G::TPW - 1) / (kRows * G::TPW)) *
                     ((sorted[i].k + G::PASS - 1) / G::PASS);
        const uint64_t slots = 2 * (uint64_t)std::max(cus, 1);
        per_wg = (units + slots - 1) / slots;
    }
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = sorted[i];
        batch.op[i].block_begin = blocks;
        const uint32_t pairs = (sorted[i].n + kRows * G::TPW - 1) / (kRows * G::TPW);
        uint32_t run = 1;
        if (G::DENSE && sorted[i].k % G::PASS == 0)
            run = (uint32_t)std::min<uint64_t>(kGgMaxRun, std::max<uint64_t>(1, per_wg / (sorted[i].k / G::PASS)));
        batch.op[i].run = run;
        blocks += (pairs + run - 1) / run;
    }
    batch.count = count;
    if (blocks) hipLaunchKernelGGL((gguf_mfma<KIND, MP, MB>), dim3(blocks), dim3(kWg), 0, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

template <int KIND>
stark_qmm_status launch_class(int c, const GgufOp* ops, uint32_t count, uint32_t* status, hipStream_t stream) {
    switch (c) {
    case 0: return launch_mfma<KIND, 2, 1>(ops, count, status, stream);
    case 1: return launch_mfma<KIND, 4, 1>(ops, count, status, stream);
    default: return launch_mfma<KIND, 16, 1>(ops, count, status, stream);  // M = 3 .. 8: dense
    }
}

// matrix-core kernel: f32 activations, 16-byte aligned rows, at least one tile
bool mfma_ok(const GgufOp& o) {
    if (((uintptr_t)o.blocks & 15) || ((uintptr_t)o.x & 15) || o.k % 256 || o.n < (uint32_t)kRows) return false;
    if ((uint64_t)o.k * 8 * 4 >= (1ull << 31)) return false;  // 32-bit offsets into 8 activation rows
    return o.x_dt == STARK_QMM_F32;
}

int m_class(uint32_t m) { return m <= 1 ? 0 : m <= 2 ? 1 : m <= 4 ? 2 : 3; }

}  // namespace

bool gguf_supported(uint32_t kind) { return kind == 8 || kind == 12; }

stark_qmm_status launch_gguf_gemv(const GgufOp* ops, uint32_t count, uint32_t* status, hipStream_t stream) {
    std::vector<GgufOp> cls[2][4];
    for (uint32_t i = 0; i < count; ++i) {
        GgufOp o = ops[i];
        if (o.x_dt == 0 && o.d_dt == 0) {
            o.x_dt = STARK_QMM_F32;
            o.d_dt = STARK_QMM_F32;
        }
        if (o.n == 0 || o.m == 0) continue;
        if (!mfma_ok(o)) {
            if (o.x_dt == STARK_QMM_F32) {
                const stark_qmm_status st = launch_finite_check((const float*)o.x, (uint64_t)o.m * o.k, status, stream);
                if (st != STARK_QMM_OK) return st;
            }
            hipLaunchKernelGGL(gguf_generic, dim3((o.n + 255) / 256, o.m), dim3(256), 0, stream, o);
            QMM_HIP_CHECK(hipGetLastError());
            continue;
        }
        // up to 8 activation rows per product; more rows are split
        const size_t xsz = 4, dsz = o.d_dt == STARK_QMM_F32 ? 4 : 2;
        for (uint32_t m0 = 0; m0 < o.m; m0 += 8) {
            GgufOp p = o;
            p.m = std::min<uint32_t>(8, o.m - m0);
            p.x = (const uint8_t*)o.x + (size_t)m0 * o.k * xsz;
            p.d = (uint8_t*)o.d + (size_t)m0 * o.n * dsz;
            cls[o.kind == 12][m_class(p.m)].push_back(p);
        }
    }
    for (int q4 = 0; q4 < 2; ++q4)
        for (int c = 0; c < 4; ++c) {
            std::vector<GgufOp>& v = cls[q4][c];
            for (size_t s = 0; s < v.size(); s += kMaxBatchOps) {
                const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, v.size() - s);
                const stark_qmm_status st = q4 ? launch_class<12>(c, v.data() + s, n, status, stream)
                                               : launch_class<8>(c, v.data() + s, n, status, stream);
                if (st != STARK_QMM_OK) return st;
            }
        }
    return STARK_QMM_OK;
}

}  // namespace qmm
