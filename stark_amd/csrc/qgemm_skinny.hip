// Skinny dequant product: 17 .. 64 activation rows (short prefill chunks and
// speculative-verify batches above the small-M matvec; products of more than
// 32 rows run as 32-row blocks), 4-bit MLX-affine codes, group size 64, bf16
// activations.
//
// Same arithmetic as the dequant-GEMM (qgemm_mfma.hip) that every product of
// more than 16 rows takes: each weight is dequantised once to
// w = bf16_rne(fma(q, s, bias_term)) -- an exact product and one f32 rounding,
// then bf16 (the reference's BF16-effective dot, vision.rs:249-336) -- and
// enters v_mfma_f32_16x16x32_bf16 as the B operand; the activation rows enter
// as plain bf16 in two 16-row blocks (one dequantised operand serves both);
// the sums accumulate in f32 over the whole K. The GEMM runs 128-column tiles
// through 64-value K steps, so a product of few rows costs the serial K loop
// of its deepest tiles (the Qwen3-8B set: 155 us at 17 to 32 rows, as at
// 128). Here the layout is the small-M kernel's (qmv_small_m.hip): a
// workgroup runs a run of 1-3 pairs of 16-row weight tiles of one op,
// pass-major under one activation stage, the four waves split each 512-value
// pass, and every prefetch buffer is indexed by a constant (a run-time index
// makes the compiler join the buffers with copies that wait for the loads).
#include <algorithm>
#include <type_traits>
#include <vector>

#include "mfma_tile.h"

namespace qmm {

namespace {

using namespace mfma;

constexpr int kSkPass = 512;             // k per pass: 4 waves x 128
constexpr int kSkQ = kSkPass / 4;        // k per wave per pass: 2 groups, 4 chunks of 32
constexpr int kSkTiles = 2;              // 16-row weight tiles per pair
constexpr int kSkRowB = kSkQ / 2 + 16;   // LDS row of a wave's codes: 80 bytes, 5 chunks (odd: no column conflicts)
constexpr int kSkGroups = kSkPass / 64;  // groups per pass
constexpr int kSkMB = 2;                 // 16-row activation blocks
constexpr int kSkRows = 16 * kSkMB;      // activation rows (M <= 32)
constexpr int kSkMaxRun = 3;             // tile pairs per workgroup, at most
constexpr int kSkMaxM = 2 * kSkRows;     // products of more rows run as blocks of kSkRows

struct SkLds {
    union {
        u32x4 stage[kSkTiles][4][kRows * kSkRowB / 16];  // codes [tile][wave][row][80 bytes]
        float red[kSkTiles][4][kSkRows][kRows];          // per-wave partial outputs, after the last pass
    };
    float2 pl[kSkTiles][kSkGroups][kRows];  // (scale, bias term) [tile][group][row]
    // activation rows as bf16 in k order, padded by 64 bytes so that the 16
    // rows of one A read alternate between the two halves of the banks
    u32x4 xp[kSkRows][kSkPass / 8 + 4];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sk_rsrc(const void* p, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)min(bytes, (uint64_t)0x7fffffffu), 0x00020000);
}

// Eight 4-bit codes (one word, k order: low nibble of byte b is value 2b, its
// high nibble 2b + 1) dequantised to bf16 as the GEMM rounds them.
template <bool SIGNED>
__device__ __forceinline__ u32x4 dequant8(uint32_t u, float s, float bt) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    if (SIGNED) u ^= 0x88888888u;
    const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
    u32x4 w;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const float w0 = fmaf((float)((lo >> (8 * b)) & 255u), s, bt);
        const float w1 = fmaf((float)((hi >> (8 * b)) & 255u), s, bt);
        const bf16x2 pr = {(__bf16)w0, (__bf16)w1};
        w[b] = __builtin_bit_cast(uint32_t, pr);
    }
    return w;
}

template <bool SIGNED>
__global__ __launch_bounds__(kWg) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_skinny(AffineBatch batch) {
    (void)batch;
    __shared__ SkLds lds;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    // workgroup b runs run b: up to kSkMaxRun consecutive tile pairs of one op
    // (op.xid pairs; the last run of an op may be shorter)
    const uint32_t L = blockIdx.x;
    if (L >= kb->total) return;
    uint32_t oi = 0;
    for (uint32_t i = 1; i < kb->count; ++i)
        if (L >= kb->op[i].block_begin) oi = i;
    const AffineOp& op = kb->op[oi];
    const uint32_t N = op.n, K = op.k, M = op.m;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t j = lane & 15, kq = lane >> 4;
    const uint32_t pair0 = (L - op.block_begin) * op.xid;
    const uint32_t cnt = min(op.xid, (N + kRows * kSkTiles - 1) / (kRows * kSkTiles) - pair0);
    const uint32_t passes = K / kSkPass, steps = passes * cnt;
    // tile tt of the run's pair t covers rows n0(t, tt) .. +15 and writes
    // those from 32 (pair0 + t) + 16 tt on; a tile past N moves back to end
    // at N, so every row is written once
    const auto tile_begin = [&](uint32_t t, int tt) { return kRows * (kSkTiles * (pair0 + t) + tt); };
    const auto n0_of = [&](uint32_t t, int tt) { return min(tile_begin(t, tt), N - kRows); };
    const uint32_t row_bytes = K / 2;
    const bool bf = op.w_dt == STARK_QMM_BF16, biased = op.corr_kind == STARK_QMM_CORRECTION_BIASES;
    // Buffer loads at per-thread offsets (a step adds its pair's rows and its
    // pass's k): activation rows past M lie past their resource and read zeros.
    const __amdgpu_buffer_rsrc_t rc = sk_rsrc(op.codes, (uint64_t)N * row_bytes);
    const __amdgpu_buffer_rsrc_t rx = sk_rsrc(op.x, (uint64_t)M * K * 2);
    const __amdgpu_buffer_rsrc_t rs = sk_rsrc(op.scales, 0x7fffffffu);
    const __amdgpu_buffer_rsrc_t rb = biased ? sk_rsrc(op.corr, 0x7fffffffu) : rs;
    // a tile's pass is 16 rows x 256 bytes: thread tid loads chunk tid % 16 of row tid / 16
    const uint32_t co = (tid / 16) * row_bytes + 16 * (tid % 16);
    // plane entry (group pt / 16, row pt % 16); threads 128.. repeat 0..127 and do not stage
    const uint32_t pt = tid & 127;
    const uint32_t po = ((pt % 16) * op.os + (pt / 16) * op.gs) * 2;
    uint32_t xo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t v = tid + 256 * i, m = v / 64, c = v % 64;
        xo[i] = (m * K + 8 * c) * 2;
    }

    // Steps run pass-major: step s is pass s / cnt of pair s % cnt, and a
    // pass's activations are staged at its first step. Two register buffers
    // for codes (a step's codes are issued two steps before it is staged) and
    // two for activations.
    u32x4 wc[2][kSkTiles];  // codes: chunk tid % 16 of row tid / 16 of a tile's pass
    u32x4 xv[2][8];         // activations: vector v = tid + 256 i is row v / 64, values 8 (v % 64)
    uint32_t ps[2][kSkTiles], pb[2][kSkTiles];  // raw plane values of (group pt / 16, row pt % 16)
    const auto load_codes = [&](auto buf, uint32_t t, uint32_t kbase) {
        constexpr int B = decltype(buf)::value;
        const uint32_t pg = (kbase / 64) * op.gs * 2;  // bytes of the pass's first plane group
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt) {
            const uint32_t n0 = n0_of(t, tt);
            wc[B][tt] = __builtin_bit_cast(u32x4,
                                           __builtin_amdgcn_raw_buffer_load_b128(rc, co + kbase / 2, n0 * row_bytes, 2));
            const uint32_t pr = pg + n0 * op.os * 2;
            ps[B][tt] = __builtin_amdgcn_raw_buffer_load_b16(rs, po, pr, 0);
            pb[B][tt] = __builtin_amdgcn_raw_buffer_load_b16(rb, po, pr, 0);  // unused without biases
        }
    };
    const auto load_x = [&](auto buf, uint32_t kbase) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            xv[B][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i] + kbase * 2, 0, 0));
    };
    const auto stage_codes = [&](auto buf) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt) {
            const uint32_t r = tid / 16, c = tid % 16;  // chunk c of the row belongs to wave c / 4
            *(u32x4*)((uint8_t*)lds.stage[tt][c / 4] + r * kSkRowB + 16 * (c % 4)) = wc[B][tt];
            if (tid < 128) {
                const float sc = plane_f32(ps[B][tt], bf);
                lds.pl[tt][pt / 16][pt % 16] = float2{sc, biased ? plane_f32(pb[B][tt], bf) : -8.0f * sc};
            }
        }
    };
    const auto stage_x = [&](auto buf) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = tid + 256 * i, m = v / 64, c = v % 64;
            if (m < M) lds.xp[m][c] = xv[B][i];  // rows past M stay zero (cleared once)
        }
    };

    f32x4 acc[kSkMaxRun][kSkTiles][kSkMB];
#pragma unroll
    for (int r = 0; r < kSkMaxRun; ++r)
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt)
#pragma unroll
            for (int b = 0; b < kSkMB; ++b) acc[r][tt][b] = f32x4{0, 0, 0, 0};
    // the wave's 128 k of a step: 4 chunks of 32 (two per group); lane (j, kq)
    // dequantises the 8 codes k = 8kq .. 8kq+7 of a chunk of tile row j, the
    // B operand of both activation blocks
    const auto compute = [&](f32x4 (&a_acc)[kSkTiles][kSkMB]) {
#pragma unroll
        for (int cc = 0; cc < kSkQ / 32; ++cc) {
            const uint32_t gp = wave * (kSkQ / 64) + cc / 2;  // group within the pass
            u32x4 a[kSkMB];
#pragma unroll
            for (int b = 0; b < kSkMB; ++b) a[b] = lds.xp[16 * b + j][wave * (kSkQ / 8) + 4 * cc + kq];
#pragma unroll
            for (int tt = 0; tt < kSkTiles; ++tt) {
                const uint32_t u =
                    *(const uint32_t*)((const uint8_t*)lds.stage[tt][wave] + j * kSkRowB + 16 * cc + 4 * kq);
                const float2 p = lds.pl[tt][gp][j];
                const u32x4 w = dequant8<SIGNED>(u, p.x, p.y);
#pragma unroll
                for (int b = 0; b < kSkMB; ++b)
                    a_acc[tt][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, a[b]), __builtin_bit_cast(bf16x8, w), a_acc[tt][b], 0, 0, 0);
            }
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    // activation rows past M: zero once (their products are zero)
    for (uint32_t v = tid; v < kSkRows * (kSkPass / 8); v += kWg) {
        const uint32_t m = v / (kSkPass / 8);
        if (m >= M) lds.xp[m][v % (kSkPass / 8)] = u32x4{0, 0, 0, 0};
    }
    // The step loop is unrolled over two steps, so that a step's code buffer
    // is its parity, a constant. A run of one pair (ONE) takes its activations
    // two passes ahead into the buffer of the pass's parity (also the step's);
    // a longer run takes them one pass (cnt steps) ahead into one buffer,
    // issued right after that buffer is staged on the same path.
    const auto run = [&](auto one_c) {
        constexpr bool ONE = decltype(one_c)::value;
        constexpr uint32_t XA = ONE ? 2 : 1;  // passes ahead of the activation loads
        load_codes(B0{}, 0, 0);
        uint32_t lp = 0, lt = 1;  // load cursor: pass and pair of step s + 2
        if (lt == cnt) lt = 0, lp = 1;
        if (steps > 1) load_codes(B1{}, lt, lp * kSkPass);
        if (++lt == cnt) lt = 0, ++lp;
        load_x(B0{}, 0);
        if (ONE && passes > 1) load_x(B1{}, kSkPass);
        uint32_t p = 0, t = 0;
        const auto step = [&](auto b_c, uint32_t s) {
            constexpr int SB = decltype(b_c)::value;
            using BS = std::integral_constant<int, SB>;
            using BX = std::integral_constant<int, ONE ? SB : 0>;
            if (s) __syncthreads();  // every wave finished the previous step's LDS
            stage_codes(BS{});
            if (ONE || t == 0) {
                stage_x(BX{});
                if (p + XA < passes) load_x(BX{}, (p + XA) * kSkPass);
            }
            __syncthreads();
            if (s + 2 < steps) {
                load_codes(BS{}, lt, lp * kSkPass);
                if (++lt == cnt) lt = 0, ++lp;
            }
            if (ONE) {
                compute(acc[0]);
            } else {
#pragma unroll
                for (int r = 0; r < kSkMaxRun; ++r)
                    if (t == (uint32_t)r) compute(acc[r]);
            }
            if (++t == cnt) t = 0, ++p;
        };
        for (uint32_t s = 0; s < steps; s += 2) {
            step(B0{}, s);
            if (s + 1 < steps) step(B1{}, s + 1);
        }
    };
    if (cnt == 1) run(std::true_type{});
    else run(std::false_type{});

#pragma unroll
    for (int r = 0; r < kSkMaxRun; ++r) {
        if ((uint32_t)r >= cnt) break;
        __syncthreads();  // the results overwrite the code stage / the previous pair's results
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt)
#pragma unroll
            for (int b = 0; b < kSkMB; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) lds.red[tt][wave][16 * b + 4 * kq + q][j] = acc[r][tt][b][q];
        __syncthreads();
        for (uint32_t v = tid; v < (uint32_t)(kSkTiles * kSkRows * kRows); v += kWg) {
            const uint32_t tt = v / (kSkRows * kRows), m = (v / kRows) % kSkRows, rr = v % kRows;
            const uint32_t n = n0_of(r, tt) + rr;
            if (m >= M || n < tile_begin(r, tt)) continue;
            const size_t o = (size_t)m * N + n;
            float y = op.ab_scale * ((lds.red[tt][0][m][rr] + lds.red[tt][1][m][rr]) +
                                     (lds.red[tt][2][m][rr] + lds.red[tt][3][m][rr]));
            if (op.flags & FLAG_ACCUMULATE) y += load_as_f32(op.d, op.d_dt, o);
            if (op.bias) y += load_as_f32(op.bias, op.w_dt, n);
            if (op.flags & FLAG_SOFT_CAP) y = op.soft_cap * tanhf(y / op.soft_cap);
            store_from_f32(op.d, op.d_dt, o, y);
        }
    }
}

}  // namespace

bool skinny_eligible(const AffineOp* ops, uint32_t count) {
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        if (o.m <= 16 || o.m > (uint32_t)kSkMaxM || o.group_size != 64 || o.k % kSkPass || o.n < (uint32_t)kRows ||
            o.gather)
            return false;
        if (o.x_dt != STARK_QMM_BF16 || !(o.w_dt == STARK_QMM_BF16 || o.w_dt == STARK_QMM_F16)) return false;
        if (!(o.corr_kind == STARK_QMM_CORRECTION_BIASES || o.corr_kind == STARK_QMM_CORRECTION_SYMMETRIC))
            return false;
        if (((uintptr_t)o.codes | (uintptr_t)o.x) & 15) return false;
        // 32-bit buffer offsets
        if ((uint64_t)o.n * o.k / 2 >= (1ull << 31) || (uint64_t)kSkRows * o.k * 2 >= (1ull << 31)) return false;
    }
    return count > 0;
}

namespace {

// One launch of at most kMaxBatchOps ops of at most kSkRows rows each.
stark_qmm_status launch_skinny_blocks(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream) {
    int dev = 0, cus = 0;
    QMM_HIP_CHECK(hipGetDevice(&dev));
    QMM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // Run lengths as in the small-M kernel: the launch's pass count per
    // resident workgroup (two per CU) over the op's passes, 1 .. kSkMaxRun.
    uint64_t units = 0;
    for (uint32_t i = 0; i < count; ++i)
        units += (uint64_t)((ops[i].n + kRows * kSkTiles - 1) / (kRows * kSkTiles)) * (ops[i].k / kSkPass);
    const uint64_t slots = 2 * (uint64_t)std::max(cus, 1);
    const uint64_t per_wg = (units + slots - 1) / slots;
    std::vector<AffineOp> sorted(ops, ops + count);  // longest K first: its runs take the low indices
    std::stable_sort(sorted.begin(), sorted.end(), [](const AffineOp& a, const AffineOp& b) { return a.k > b.k; });
    AffineBatch batch{};
    uint32_t runs = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t pairs = (sorted[i].n + kRows * kSkTiles - 1) / (kRows * kSkTiles);
        const uint32_t run =
            (uint32_t)std::min<uint64_t>(kSkMaxRun, std::max<uint64_t>(1, per_wg / (sorted[i].k / kSkPass)));
        batch.op[i] = sorted[i];
        batch.op[i].block_begin = runs;
        batch.op[i].xid = run;  // tile pairs per run
        runs += (pairs + run - 1) / run;
    }
    batch.count = count;
    batch.total = runs;
    if (runs == 0) return STARK_QMM_OK;
    if (signed_codes)
        hipLaunchKernelGGL(qgemm_skinny<true>, dim3(runs), dim3(kWg), 0, stream, batch);
    else
        hipLaunchKernelGGL(qgemm_skinny<false>, dim3(runs), dim3(kWg), 0, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace

// Products of 33 .. 64 rows run as blocks of kSkRows rows (the rows' own
// activations and outputs; every block reads the weights once): against the
// GEMM's 156-161 us on the Qwen3-8B set at 33 .. 64 rows.
stark_qmm_status launch_skinny(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream) {
    std::vector<AffineOp> blocks;
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        const size_t dsz = o.d_dt == STARK_QMM_F32 ? 4 : 2;
        for (uint32_t m0 = 0; m0 < o.m; m0 += kSkRows) {
            AffineOp b = o;
            b.m = std::min<uint32_t>(kSkRows, o.m - m0);
            b.x = (const uint8_t*)o.x + (size_t)m0 * o.k * 2;
            b.d = (uint8_t*)o.d + (size_t)m0 * o.n * dsz;
            blocks.push_back(b);
        }
    }
    for (size_t s = 0; s < blocks.size(); s += kMaxBatchOps) {
        const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, blocks.size() - s);
        const stark_qmm_status st = launch_skinny_blocks(blocks.data() + s, n, signed_codes, stream);
        if (st != STARK_QMM_OK) return st;
    }
    return STARK_QMM_OK;
}

}  // namespace qmm
