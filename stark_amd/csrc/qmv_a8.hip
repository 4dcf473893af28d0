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


// ---- Prefill form (M > 16): int8 GEMM on the matrix cores.
// A 128x128 output tile per workgroup (4 waves, 64x64 each, 4x4 blocks of
// v_mfma_i32_16x16x64_i8; a 32-wide chunk masks the other half's activations). K is
// walked in steps of 64; each step's activation codes and weight codes (4-bit
// unpacked to bytes, 8-bit as q - 128) are staged in LDS as int8 in the same
// k order, so every MFMA sums q_a * q_w exactly in int32 over one flush chunk
// of G = min(activation group, weight group, 64) values. Per chunk and output
//   acc += (scale_a * s) * C + (scale_a * sum q_a) * bias_term
// (8-bit weights: bias_term + 128 s, for the q - 128 offset), in f32. The
// chunk sums of q_a come from v_dot4 during staging. The k order inside a
// chunk does not matter (integer sums), so sequential activation codes meet
// weight bytes permuted to sequential order and grouped-by-nibble codes meet
// the nibble split as it falls out of the weight word.
#ifndef QMM_A8_WPE
#define QMM_A8_WPE 2
#endif
constexpr int kGB = 128;         // tile rows (M) and columns (N)
constexpr int kGK = 64;          // k per step
// LDS rows of 64 int8 codes (4 chunks of 16 bytes), chunk c of row r stored
// at chunk c ^ ((r >> 1) & 3): any 8 consecutive lanes moving 16 bytes each
// then cover the 32 banks once -- the MFMA operand reads (rows r..r+7, one
// chunk), the activation stores (2 rows x 4 chunks) and the 4-bit weight
// stores (4 rows x 2 chunks).
__device__ __forceinline__ uint32_t swz8(uint32_t r, uint32_t c) { return c ^ ((r >> 1) & 3); }

struct A8GemmLds {
    u32x4 a[2][kGB][kGK / 16];  // int8 codes, 16 per element
    u32x4 b[2][kGB][kGK / 16];
    float sa[2][2][kGB];  // [buf][chunk][row] activation scale
    // rings of 8 chunks; rows padded to 144 floats so that the four lane
    // groups of a bias read (four slots) fall on disjoint banks
    float ur[8][kGB + 16];  // [chunk % 8][row] activation scale * chunk sum of codes
    float ws[2][2][kGB];  // [buf][chunk][col] weight scale
    float br[8][kGB + 16];  // [chunk % 8][col] bias term (8-bit: + 128 s)
};

typedef int i32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t a8_rsrc(const void* p, size_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)min(bytes, (size_t)0x7fffffff), 0x00020000);
}

template <int AUX = 0>
__device__ __forceinline__ u32x4 a8_load16_impl(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}
// aux 2: nontemporal (weights are streamed once per output tile row)
__device__ __forceinline__ u32x4 a8_load16(__amdgpu_buffer_rsrc_t r, uint32_t off, int nt = 0) {
    return nt ? a8_load16_impl<2>(r, off) : a8_load16_impl<0>(r, off);
}
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Output tile (bx, by) of one product: columns kGB bx.., rows kGB by...
template <int BITS, int G, bool SIGNED, bool GROUPED>
__device__ __forceinline__ void a8_tile(const AffineOp& op, const A8Operand& a, uint32_t bx, uint32_t by) {
    __shared__ A8GemmLds lds;
    constexpr int NCH = kGK / G;  // flush chunks per step
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t M = op.m, N = op.n, K = op.k, GA = K / a.group;
    const uint32_t m0 = by * kGB, n0 = bx * kGB;
    const size_t wrow = (size_t)K * BITS / 8;

    // staging roles: activation rows ar and 64 + ar, 16 bytes at aq * 16;
    // 4-bit weights: row tid / 2, 16 bytes (32 codes) at (tid % 2) * 16;
    // 8-bit weights: rows ar and 64 + ar, 16 bytes at aq * 16;
    // weight metadata: column tid (tid < 128).
    // Every load is a buffer load whose resource ends at the operand's last
    // byte: rows past M or N read zeros, with no branch around any load.
    const uint32_t ar = tid >> 2, aq = tid & 3;
    const uint32_t lga = 31 - __builtin_clz(a.group), lgw = 31 - __builtin_clz(op.group_size);
    const __amdgpu_buffer_rsrc_t ra = a8_rsrc(a.codes, (size_t)M * K);
    const __amdgpu_buffer_rsrc_t rsa = a8_rsrc(a.scales, (size_t)M * GA * 4);
    const __amdgpu_buffer_rsrc_t rw = a8_rsrc(op.codes, (size_t)N * wrow);
    const __amdgpu_buffer_rsrc_t rps = a8_rsrc(op.scales, 0x7fffffffu);
    const __amdgpu_buffer_rsrc_t rpb = a8_rsrc(op.corr, 0x7fffffffu);
    const bool biased = op.corr_kind == STARK_QMM_CORRECTION_BIASES, bfp = op.w_dt == STARK_QMM_BF16;
    struct Stage {
        u32x4 xa[2];
        u32x4 wc[BITS / 4];
        float sa[2];
        uint32_t s[NCH], b[NCH];  // raw plane values
    };
    auto load = [&](Stage& st, uint32_t k0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t m = m0 + ar + 64 * h;
            st.xa[h] = a8_load16(ra, m * K + k0 + aq * 16);
            st.sa[h] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                     rsa, (m * GA + ((k0 + aq * 16) >> lga)) * 4, 0, 0));
        }
#pragma unroll
        for (int h = 0; h < BITS / 4; ++h) {
            const uint32_t r = BITS == 4 ? (uint32_t)tid >> 1 : ar + 64 * h;
            const uint32_t off = BITS == 4 ? ((uint32_t)tid & 1) * 16 : aq * 16;
            // ordinary (cached) loads: a step reads 32 bytes (4-bit) of each
            // row's 128-byte line and the next steps the rest; with the
            // nontemporal hint L2 fetched the line again for each (Qwen3-8B
            // prefill set: 710 -> 824 TOP/s)
            st.wc[h] = a8_load16(rw, (n0 + r) * (uint32_t)wrow + k0 * BITS / 8 + off, 0);
        }
        // plane entries of column n0 + tid (threads past 128 read a valid
        // entry too and never store it); past N they are ignored
        const uint32_t n = min(n0 + ((uint32_t)tid & (kGB - 1)), N - 1);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const uint32_t md = n * op.os + ((k0 + c * G) >> lgw) * op.gs;
            st.s[c] = __builtin_amdgcn_raw_buffer_load_b16(rps, md * 2, 0, 0);
            st.b[c] = __builtin_amdgcn_raw_buffer_load_b16(rpb, biased ? md * 2 : 0x80000000u, 0, 0);
        }
    };
    // (st: the step whose chunks this stage holds)
    auto store = [&](const Stage& st, int buf, uint32_t step) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t r = ar + 64 * h;
            lds.a[buf][r][swz8(r, aq)] = st.xa[h];
            int sum = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t) sum = __builtin_amdgcn_sdot4((int)st.xa[h][t], 0x01010101, sum, false);
            sum += __shfl_xor(sum, 1, 64);
            if (G == 64) sum += __shfl_xor(sum, 2, 64);
            if (G == 64 ? aq == 0 : (aq & 1) == 0) {
                const uint32_t c = G == 64 ? 0 : aq >> 1;
                lds.sa[buf][c][r] = st.sa[h];
                lds.ur[(step * NCH + c) & 7][r] = st.sa[h] * (float)sum;
            }
        }
        if (BITS == 4) {
            const uint32_t r = (uint32_t)tid >> 1, off = ((uint32_t)tid & 1) * 32;
            uint32_t out[8];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t w = st.wc[0][t];
                if (SIGNED) w ^= 0x88888888u;
                const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;  // (v0,v2,v4,v6), (v1,v3,v5,v7)
                out[2 * t] = GROUPED ? lo : __builtin_amdgcn_perm(hi, lo, 0x05010400u);
                out[2 * t + 1] = GROUPED ? hi : __builtin_amdgcn_perm(hi, lo, 0x07030602u);
            }
            lds.b[buf][r][swz8(r, off / 16)] = u32x4{out[0], out[1], out[2], out[3]};
            lds.b[buf][r][swz8(r, off / 16 + 1)] = u32x4{out[4], out[5], out[6], out[7]};
        } else {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                u32x4 w = st.wc[h];
#pragma unroll
                for (int t = 0; t < 4; ++t) w[t] ^= SIGNED ? 0u : 0x80808080u;  // q - 128 as int8
                if (GROUPED) {
                    const uint32_t e0 = __builtin_amdgcn_perm(w[1], w[0], 0x06040200u);
                    const uint32_t o0 = __builtin_amdgcn_perm(w[1], w[0], 0x07050301u);
                    const uint32_t e1 = __builtin_amdgcn_perm(w[3], w[2], 0x06040200u);
                    const uint32_t o1 = __builtin_amdgcn_perm(w[3], w[2], 0x07050301u);
                    w = u32x4{e0, o0, e1, o1};
                }
                lds.b[buf][ar + 64 * h][swz8(ar + 64 * h, aq)] = w;
            }
        }
        if (tid < kGB) {
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const float sc = bfp ? bf16_bits_to_f32(st.s[c]) : f16_bits_to_f32(st.s[c]);
                const float bt = biased ? (bfp ? bf16_bits_to_f32(st.b[c]) : f16_bits_to_f32(st.b[c]))
                                        : -sc * (float)(1 << (BITS - 1));
                lds.ws[buf][c][tid] = sc;
                lds.br[(step * NCH + c) & 7][tid] = BITS == 8 ? bt + 128.0f * sc : bt;
            }
        }
    };

    const int wm = wave >> 1, wn = wave & 1;
    const uint32_t li = lane & 15, lq = lane >> 4;
    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0, 0, 0, 0};
    // per chunk: the wave's B fragments and weight metadata once, then each
    // row block's 4 MFMAs and its flush (16 int32 accumulators live at a time)
    auto compute = [&](int buf) {
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll 1
        for (int c = 0; c < NCH; ++c) {
            float s4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) s4[j] = lds.ws[buf][c][wn * 64 + 16 * j + li];
            u32x4 bfr[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t r = wn * 64 + 16 * j + li;
                bfr[j] = lds.b[buf][r][swz8(r, lq)];
            }
            i32x4_t cz = i32x4_t{0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t ra = wm * 64 + 16 * i + li;
                u32x4 af = lds.a[buf][ra][swz8(ra, lq)];
                // a 32-wide chunk keeps the activation bytes of its own half of
                // the step (lanes 16 lq read bytes 16 lq ..), the other half zero
                if (G == 32 && (lq >> 1) != (uint32_t)c) af = u32x4{0, 0, 0, 0};
                i32x4_t C[4];
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    C[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i32x4_t, af),
                                                                 __builtin_bit_cast(i32x4_t, bfr[j]),
                                                                 cz, 0, 0, 0);
                // C element e of block (i, j): row 4 lq + e, column li
                const f32x4 sa = *(const f32x4*)&lds.sa[buf][c][wm * 64 + 16 * i + 4 * lq];
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(sa[e] * s4[j], (float)C[j][e], acc[i][j][e]);
                // the next row block's MFMAs start after this flush: their zero
                // accumulator input is tied to this block's results, so only one
                // block's 16 int32 sums are live (two waves per SIMD fit the registers)
                asm volatile("" : "+v"(cz) : "v"(acc[i][0]), "v"(acc[i][1]), "v"(acc[i][2]), "v"(acc[i][3]));
            }
            // keep the chunks apart: hoisting the next chunk's fragments and
            // MFMAs above this flush would not fit the register budget
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // The bias terms sum_c (s_a * sum q_a)[row, c] * bias_term[col, c] of four
    // chunks as one f32 product per 16x16 block (v_mfma_f32_16x16x4_f32: A
    // row = lane % 16, k = lane / 16; B k = lane / 16, column = lane % 16; D in
    // the int8 product's C layout), chunks q0 .. q0 + 3 from the LDS rings
    // (k entries at or past `valid` read as zero).
    auto bias4 = [&](uint32_t q0, uint32_t valid) {
        const uint32_t sl = (q0 + lq) & 7;
        const bool ok = lq < valid;
        float av[4], bv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) av[i] = ok ? lds.ur[sl][wm * 64 + 16 * i + li] : 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) bv[j] = ok ? lds.br[sl][wn * 64 + 16 * j + li] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    };

    const auto barrier = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    };
    // one register stage: step s computes from LDS buffer s % 2 while step
    // s + 1's loads fly; they are staged into the other buffer after the compute
    // (the last step's re-read of its own tile lands in a buffer not read again)
    const uint32_t steps = K / kGK;
    Stage stg;
    load(stg, 0);
    store(stg, 0, 0);
    barrier();
    for (uint32_t st = 0; st < steps; ++st) {
        load(stg, min(st + 1, steps - 1) * kGK);
        compute(st & 1);
        // every fourth chunk: the bias terms of the last four (the ring of 8
        // holds them while the next step's chunks are stored beside them)
        if (NCH == 2 ? (st & 1) : ((st & 3) == 3)) bias4((st + 1) * NCH - 4, 4);
        store(stg, (st & 1) ^ 1, st + 1);
        barrier();
    }
    {
        const uint32_t q = steps * NCH, rem = q & 3;
        if (rem) bias4(q - rem, rem);
    }

    // full tiles with a plain bf16 store (no D-op past ab_scale): one row
    // pointer per (i, e), the column blocks at fixed offsets from it
    if (!(op.flags & (FLAG_ACCUMULATE | FLAG_SOFT_CAP)) && !op.bias && op.d_dt == STARK_QMM_BF16 &&
        m0 + kGB <= M && n0 + kGB <= N) {
        uint16_t* const d = (uint16_t*)op.d;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint16_t* const row = d + (size_t)(m0 + wm * 64 + 16 * i + 4 * lq + e) * N + n0 + wn * 64 + li;
#pragma unroll
                for (int j = 0; j < 4; ++j) row[16 * j] = f32_to_bf16_bits(op.ab_scale * acc[i][j][e]);
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t m = m0 + wm * 64 + 16 * i + 4 * lq + e;
                const uint32_t n = n0 + wn * 64 + 16 * j + li;
                if (m < M && n < N) epilogue(op, m, n, acc[i][j][e]);
            }
}

template <int BITS, int G, bool SIGNED, bool GROUPED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(QMM_A8_WPE))) void qgemm_a8(AffineOp op, A8Operand a) {
    a8_tile<BITS, G, SIGNED, GROUPED>(op, a, blockIdx.x, blockIdx.y);
}

__host__ __device__ inline uint32_t a8_tiles(const AffineOp& o) {
    return ((o.n + kGB - 1) / kGB) * ((o.m + kGB - 1) / kGB);
}

// Several products in one grid (one template class), as qgemm_group: op i's
// tiles follow op i - 1's, row-major over (row block, column block).
template <int BITS, int G, bool SIGNED, bool GROUPED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(QMM_A8_WPE))) void qgemm_a8_group(A8Batch batch) {
    (void)batch;
    const A8Batch* kb = (const A8Batch*)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t t = blockIdx.x, i = 0;
    for (; i + 1 < kb->count; ++i) {
        const uint32_t nt = a8_tiles(kb->op[i]);
        if (t < nt) break;
        t -= nt;
    }
    const AffineOp& op = kb->op[i];
    const uint32_t gx = (op.n + kGB - 1) / kGB;
    a8_tile<BITS, G, SIGNED, GROUPED>(op, kb->a[i], t % gx, t / gx);
}

template <int BITS, int G>
void launch_gemm_a8_group(const A8Batch& b, uint32_t tiles, hipStream_t stream) {
    const bool sg = (b.op[0].flags & FLAG_SIGNED) != 0, gr = b.a[0].grouped != 0;
    const dim3 grid(tiles);
    if (sg && gr)
        hipLaunchKernelGGL((qgemm_a8_group<BITS, G, true, true>), grid, dim3(256), 0, stream, b);
    else if (sg)
        hipLaunchKernelGGL((qgemm_a8_group<BITS, G, true, false>), grid, dim3(256), 0, stream, b);
    else if (gr)
        hipLaunchKernelGGL((qgemm_a8_group<BITS, G, false, true>), grid, dim3(256), 0, stream, b);
    else
        hipLaunchKernelGGL((qgemm_a8_group<BITS, G, false, false>), grid, dim3(256), 0, stream, b);
}

template <int BITS, int G>
void launch_gemm_a8(const AffineOp& op, const A8Operand& a, hipStream_t stream) {
    const dim3 grid((op.n + kGB - 1) / kGB, (op.m + kGB - 1) / kGB);
    const bool sg = (op.flags & FLAG_SIGNED) != 0, gr = a.grouped != 0;
    if (sg && gr)
        hipLaunchKernelGGL((qgemm_a8<BITS, G, true, true>), grid, dim3(256), 0, stream, op, a);
    else if (sg)
        hipLaunchKernelGGL((qgemm_a8<BITS, G, true, false>), grid, dim3(256), 0, stream, op, a);
    else if (gr)
        hipLaunchKernelGGL((qgemm_a8<BITS, G, false, true>), grid, dim3(256), 0, stream, op, a);
    else
        hipLaunchKernelGGL((qgemm_a8<BITS, G, false, false>), grid, dim3(256), 0, stream, op, a);
}

}  // namespace

// Prefill sizes take the int8 GEMM on the matrix cores.
bool a8_gemm_eligible(const AffineOp& op, const A8Operand& a, int bits) {
    return op.m > 16 && !op.gather && op.k % kGK == 0 && (((uintptr_t)op.codes | (uintptr_t)a.codes) & 15) == 0 &&
           op.corr_kind != STARK_QMM_CORRECTION_ZERO_POINTS && op.w_dt != STARK_QMM_F32 &&
           (uint64_t)op.m * op.k < (1ull << 31) && (uint64_t)op.n * op.k * bits / 8 < (1ull << 31);
}

// Grid class of an a8_gemm_eligible product: (bits, flush group 32, signed codes, grouped activation codes).
uint32_t a8_gemm_class(const AffineOp& op, const A8Operand& a, int bits) {
    return (bits == 8 ? 8u : 0u) | (a.group == 32 || op.group_size == 32 ? 4u : 0u) |
           ((op.flags & FLAG_SIGNED) ? 2u : 0u) | (a.grouped ? 1u : 0u);
}

stark_qmm_status launch_affine_a8_gemm_group(const AffineOp* ops, const A8Operand* as, uint32_t count, int bits,
                                             hipStream_t stream) {
    if (count == 0) return STARK_QMM_OK;
    if (count == 1) return launch_affine_a8(ops[0], as[0], bits, stream);
    if (count > (uint32_t)kMaxBatchOps) return STARK_QMM_UNSUPPORTED;
    std::vector<uint32_t> idx(count);
    for (uint32_t i = 0; i < count; ++i) idx[i] = i;
    std::stable_sort(idx.begin(), idx.end(), [&](uint32_t x, uint32_t y) { return ops[x].k > ops[y].k; });
    A8Batch b{};
    uint64_t tiles = 0;
    for (uint32_t i = 0; i < count; ++i) {
        b.op[i] = ops[idx[i]];
        b.a[i] = as[idx[i]];
        tiles += a8_tiles(b.op[i]);
    }
    b.count = count;
    if (tiles == 0) return STARK_QMM_OK;
    if (tiles > 0x7fffffffu) return STARK_QMM_UNSUPPORTED;
    const bool g32 = (a8_gemm_class(b.op[0], b.a[0], bits) & 4u) != 0;
    if (bits == 4 && g32)
        launch_gemm_a8_group<4, 32>(b, (uint32_t)tiles, stream);
    else if (bits == 4)
        launch_gemm_a8_group<4, 64>(b, (uint32_t)tiles, stream);
    else if (g32)
        launch_gemm_a8_group<8, 32>(b, (uint32_t)tiles, stream);
    else
        launch_gemm_a8_group<8, 64>(b, (uint32_t)tiles, stream);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

stark_qmm_status launch_affine_a8(const AffineOp& op, const A8Operand& a, int bits, hipStream_t stream) {
    if (op.m == 0 || op.n == 0) return STARK_QMM_OK;
    // a product too tall for one grid's 32-bit offsets: launches of whole rows
    // (the activation codes, their scales and d advanced per part)
    if (op.m > 16 && op.k > 0 && (uint64_t)op.m * op.k >= (1ull << 31)) {
        const uint64_t fit = ((1ull << 31) - 1) / op.k;
        const uint32_t R = fit > (uint64_t)kGB ? (uint32_t)((fit - kGB) / kGB * kGB) : 0u;
        AffineOp part = op;
        A8Operand pa = a;
        part.m = R;
        if (R > 16 && a8_gemm_eligible(part, a, bits)) {
            const size_t dsz = op.d_dt == STARK_QMM_F32 ? 4 : 2;
            for (uint32_t m0 = 0; m0 < op.m; m0 += R) {
                part.m = std::min(R, op.m - m0);
                part.d = (uint8_t*)op.d + (size_t)m0 * op.n * dsz;
                pa.codes = a.codes + (size_t)m0 * op.k;
                pa.scales = a.scales + (size_t)m0 * (op.k / a.group);
                const stark_qmm_status st = launch_affine_a8(part, pa, bits, stream);
                if (st != STARK_QMM_OK) return st;
            }
            return STARK_QMM_OK;
        }
    }
    // prefill sizes: the int8 GEMM on the matrix cores
    if (a8_gemm_eligible(op, a, bits)) {
        const bool g32 = a.group == 32 || op.group_size == 32;
        if (bits == 4 && g32)
            launch_gemm_a8<4, 32>(op, a, stream);
        else if (bits == 4)
            launch_gemm_a8<4, 64>(op, a, stream);
        else if (g32)
            launch_gemm_a8<8, 32>(op, a, stream);
        else
            launch_gemm_a8<8, 64>(op, a, stream);
        QMM_HIP_CHECK(hipGetLastError());
        return STARK_QMM_OK;
    }
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
