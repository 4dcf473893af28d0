// Skinny dequant product: 17 .. 64 activation rows (short prefill chunks and
// speculative-verify batches above the small-M matvec), 4-bit MLX-affine
// codes, group size 64, bf16 activations.
//
// Same arithmetic as the dequant-GEMM (qgemm_mfma.hip) that every product of
// more than 16 rows takes: each weight is dequantised once to
// w = bf16_rne(fma(q, s, bias_term)) -- an exact product and one f32 rounding,
// then bf16 (the reference's BF16-effective dot, vision.rs:249-336) -- and
// enters v_mfma_f32_16x16x32_bf16 as the B operand; the activation rows enter
// as plain bf16 in 16-row blocks (one dequantised operand serves them all);
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

constexpr int kSkTiles = 2;  // 16-row weight tiles per pair

// Geometry of a class: MB 16-row activation blocks, P-value passes (four
// waves of P / 4), runs of up to RUN tile pairs. Two classes: 17 .. 32 rows
// (MB 2, P 512, RUN 3) and 33 .. 64 rows (MB 4, P 256, RUN 1: the activation
// stage and the accumulators of four blocks fit two workgroups per CU only so).
template <int MB, int P, int RUN>
struct SkGeo {
    static constexpr int Q = P / 4;                  // k per wave per pass
    static constexpr int CH = Q / 32;                // 32-value chunks per wave per pass
    static constexpr int GW = Q / 64;                // groups per wave per pass
    static constexpr int GP = P / 64;                // groups per pass
    static constexpr int CPR = P / 32;               // 16-byte code chunks of a row per pass
    static constexpr int CPW = CPR / 4;              // of them per wave
    static constexpr int CT = kRows * CPR;           // code chunks of a tile per pass (threads that load one)
    static constexpr int PT = kRows * GP;            // plane entries of a tile per pass
    static constexpr int ROWB = Q / 2 + 16;          // LDS row of a wave's codes (an odd number of chunks)
    static constexpr int ROWS = 16 * MB;             // activation rows
    static constexpr int XI = ROWS * (P / 8) / kWg;  // activation vectors per thread
    static_assert(CT <= kWg && PT <= kWg && (ROWB / 16) % 2 == 1 && XI * kWg == ROWS * (P / 8), "geometry");
};

template <int MB, int P, int RUN>
struct SkLds {
    using G = SkGeo<MB, P, RUN>;
    union {
        u32x4 stage[kSkTiles][4][kRows * G::ROWB / 16];  // codes [tile][wave][row][ROWB bytes]
        float red[4][G::ROWS][kRows];                    // one tile's per-wave partial outputs, after the last pass
    };
    float2 pl[kSkTiles][G::GP][kRows];  // (scale, bias term) [tile][group][row]
    // activation rows as bf16 in k order, padded by 64 bytes so that the 16
    // rows of one A read alternate between the two halves of the banks
    u32x4 xp[G::ROWS][P / 8 + 4];
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

template <bool SIGNED, int MB, int P, int RUN>
__global__ __launch_bounds__(kWg) __attribute__((amdgpu_waves_per_eu(2))) void qgemm_skinny(AffineBatch batch) {
    (void)batch;
    using G = SkGeo<MB, P, RUN>;
    __shared__ SkLds<MB, P, RUN> lds;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    // workgroup b runs run b: up to RUN consecutive tile pairs of one op
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
    const uint32_t passes = K / P, steps = passes * cnt;
    // tile tt of the run's pair t covers rows n0(t, tt) .. +15 and writes
    // those from 32 (pair0 + t) + 16 tt on; a tile past N moves back to end
    // at N, so every row is written once
    const auto tile_begin = [&](uint32_t t, int tt) { return kRows * (kSkTiles * (pair0 + t) + tt); };
    const auto n0_of = [&](uint32_t t, int tt) { return min(tile_begin(t, tt), N - kRows); };
    const uint32_t row_bytes = K / 2;
    const bool bf = op.w_dt == STARK_QMM_BF16, biased = op.corr_kind == STARK_QMM_CORRECTION_BIASES;
    // Buffer loads at per-thread offsets (a step adds its pair's rows and its
    // pass's k): activation rows past M lie past their resource and read zeros,
    // and so do the code chunks of threads past a tile's pass.
    const __amdgpu_buffer_rsrc_t rc = sk_rsrc(op.codes, (uint64_t)N * row_bytes);
    const __amdgpu_buffer_rsrc_t rx = sk_rsrc(op.x, (uint64_t)M * K * 2);
    const __amdgpu_buffer_rsrc_t rs = sk_rsrc(op.scales, 0x7fffffffu);
    const __amdgpu_buffer_rsrc_t rb = biased ? sk_rsrc(op.corr, 0x7fffffffu) : rs;
    // thread tid < CT loads chunk tid % CPR of row tid / CPR of a tile's pass
    const uint32_t co = tid < (uint32_t)G::CT ? (tid / G::CPR) * row_bytes + 16 * (tid % G::CPR) : 0x80000000u;
    // plane entry (group pt / 16, row pt % 16); threads past PT repeat and do not stage
    const uint32_t pt = tid % G::PT;
    const uint32_t po = ((pt % 16) * op.os + (pt / 16) * op.gs) * 2;
    uint32_t xo[G::XI];
#pragma unroll
    for (int i = 0; i < G::XI; ++i) {
        const uint32_t v = tid + kWg * i, m = v / (P / 8), c = v % (P / 8);
        xo[i] = (m * K + 8 * c) * 2;
    }

    // Steps run pass-major: step s is pass s / cnt of pair s % cnt, and a
    // pass's activations are staged at its first step. Two register buffers
    // for codes (a step's codes are issued two steps before it is staged) and
    // two for activations.
    u32x4 wc[2][kSkTiles];  // codes: chunk tid % CPR of row tid / CPR of a tile's pass
    u32x4 xv[2][G::XI];     // activations: vector v = tid + 256 i is row v / (P / 8), values 8 (v % (P / 8))
    uint32_t ps[2][kSkTiles], pb[2][kSkTiles];  // raw plane values of (group pt / 16, row pt % 16)
    const auto load_codes = [&](auto buf, uint32_t t, uint32_t kbase) {
        constexpr int B = decltype(buf)::value;
        const uint32_t pg = (kbase / 64) * op.gs * 2;  // bytes of the pass's first plane group
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt) {
            const uint32_t n0 = n0_of(t, tt);
            wc[B][tt] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, co + kbase / 2, n0 * row_bytes, 2));
            const uint32_t pr = pg + n0 * op.os * 2;
            ps[B][tt] = __builtin_amdgcn_raw_buffer_load_b16(rs, po, pr, 0);
            pb[B][tt] = __builtin_amdgcn_raw_buffer_load_b16(rb, po, pr, 0);  // unused without biases
        }
    };
    const auto load_x = [&](auto buf, uint32_t kbase) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int i = 0; i < G::XI; ++i)
            xv[B][i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, xo[i] + kbase * 2, 0, 0));
    };
    const auto stage_codes = [&](auto buf) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt) {
            if (tid < (uint32_t)G::CT) {
                const uint32_t r = tid / G::CPR, c = tid % G::CPR;  // chunk c of the row belongs to wave c / CPW
                *(u32x4*)((uint8_t*)lds.stage[tt][c / G::CPW] + r * G::ROWB + 16 * (c % G::CPW)) = wc[B][tt];
            }
            if (tid < (uint32_t)G::PT) {
                const float sc = plane_f32(ps[B][tt], bf);
                lds.pl[tt][pt / 16][pt % 16] = float2{sc, biased ? plane_f32(pb[B][tt], bf) : -8.0f * sc};
            }
        }
    };
    const auto stage_x = [&](auto buf) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int i = 0; i < G::XI; ++i) {
            const uint32_t v = tid + kWg * i, m = v / (P / 8), c = v % (P / 8);
            if (m < M) lds.xp[m][c] = xv[B][i];  // rows past M stay zero (cleared once)
        }
    };

    f32x4 acc[RUN][kSkTiles][MB];
#pragma unroll
    for (int r = 0; r < RUN; ++r)
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt)
#pragma unroll
            for (int b = 0; b < MB; ++b) acc[r][tt][b] = f32x4{0, 0, 0, 0};
    // the wave's Q values of a step: CH chunks of 32 (two per group); lane
    // (j, kq) dequantises the 8 codes k = 8kq .. 8kq+7 of a chunk of tile row
    // j, the B operand of every activation block
    const auto compute = [&](f32x4 (&a_acc)[kSkTiles][MB]) {
#pragma unroll
        for (int cc = 0; cc < G::CH; ++cc) {
            const uint32_t gp = wave * G::GW + cc / 2;  // group within the pass
            u32x4 a[MB];
#pragma unroll
            for (int b = 0; b < MB; ++b) a[b] = lds.xp[16 * b + j][wave * (G::Q / 8) + 4 * cc + kq];
#pragma unroll
            for (int tt = 0; tt < kSkTiles; ++tt) {
                const uint32_t u =
                    *(const uint32_t*)((const uint8_t*)lds.stage[tt][wave] + j * G::ROWB + 16 * cc + 4 * kq);
                const float2 p = lds.pl[tt][gp][j];
                const u32x4 w = dequant8<SIGNED>(u, p.x, p.y);
#pragma unroll
                for (int b = 0; b < MB; ++b)
                    a_acc[tt][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(bf16x8, a[b]), __builtin_bit_cast(bf16x8, w), a_acc[tt][b], 0, 0, 0);
            }
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    // activation rows past M: zero once (their products are zero)
    for (uint32_t v = tid; v < (uint32_t)G::ROWS * (P / 8); v += kWg) {
        const uint32_t m = v / (P / 8);
        if (m >= M) lds.xp[m][v % (P / 8)] = u32x4{0, 0, 0, 0};
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
        if (steps > 1) load_codes(B1{}, lt, lp * P);
        if (++lt == cnt) lt = 0, ++lp;
        load_x(B0{}, 0);
        if (ONE && passes > 1) load_x(B1{}, P);
        uint32_t p = 0, t = 0;
        const auto step = [&](auto b_c, uint32_t s) {
            constexpr int SB = decltype(b_c)::value;
            using BS = std::integral_constant<int, SB>;
            using BX = std::integral_constant<int, ONE ? SB : 0>;
            if (s) __syncthreads();  // every wave finished the previous step's LDS
            stage_codes(BS{});
            if (ONE || t == 0) {
                stage_x(BX{});
                if (p + XA < passes) load_x(BX{}, (p + XA) * P);
            }
            __syncthreads();
            if (s + 2 < steps) {
                load_codes(BS{}, lt, lp * P);
                if (++lt == cnt) lt = 0, ++lp;
            }
            if (ONE) {
                compute(acc[0]);
            } else {
#pragma unroll
                for (int r = 0; r < RUN; ++r)
                    if (t == (uint32_t)r) compute(acc[r]);
            }
            if (++t == cnt) t = 0, ++p;
        };
        for (uint32_t s = 0; s < steps; s += 2) {
            step(B0{}, s);
            if (s + 1 < steps) step(B1{}, s + 1);
        }
    };
    if constexpr (RUN == 1) {
        run(std::true_type{});
    } else {
        if (cnt == 1) run(std::true_type{});
        else run(std::false_type{});
    }

    // results, one tile at a time: the four waves' sums meet in LDS (over the
    // code stage) and the rows go out with the D-ops
#pragma unroll
    for (int r = 0; r < RUN; ++r) {
        if ((uint32_t)r >= cnt) break;
#pragma unroll
        for (int tt = 0; tt < kSkTiles; ++tt) {
            __syncthreads();  // the code stage / the previous results are read
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) lds.red[wave][16 * b + 4 * kq + q][j] = acc[r][tt][b][q];
            __syncthreads();
            for (uint32_t v = tid; v < (uint32_t)(G::ROWS * kRows); v += kWg) {
                const uint32_t m = v / kRows, rr = v % kRows;
                const uint32_t n = n0_of(r, tt) + rr;
                if (m >= M || n < tile_begin(r, tt)) continue;
                const size_t o = (size_t)m * N + n;
                float y = op.ab_scale * ((lds.red[0][m][rr] + lds.red[1][m][rr]) + (lds.red[2][m][rr] + lds.red[3][m][rr]));
                if (op.flags & FLAG_ACCUMULATE) y += load_as_f32(op.d, op.d_dt, o);
                if (op.bias) y += load_as_f32(op.bias, op.w_dt, n);
                if (op.flags & FLAG_SOFT_CAP) y = op.soft_cap * tanhf(y / op.soft_cap);
                store_from_f32(op.d, op.d_dt, o, y);
            }
        }
    }
}

// the two classes: rows 17 .. 32 and 33 .. 64
using Small = SkGeo<2, 512, 3>;
using Wide = SkGeo<4, 256, 1>;
constexpr uint32_t kSkMaxM = Wide::ROWS;

}  // namespace

bool skinny_eligible(const AffineOp* ops, uint32_t count) {
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        if (o.m <= 16 || o.m > kSkMaxM || o.group_size != 64 || o.k % 512 || o.n < (uint32_t)kRows || o.gather)
            return false;
        if (o.x_dt != STARK_QMM_BF16 || !(o.w_dt == STARK_QMM_BF16 || o.w_dt == STARK_QMM_F16)) return false;
        if (!(o.corr_kind == STARK_QMM_CORRECTION_BIASES || o.corr_kind == STARK_QMM_CORRECTION_SYMMETRIC))
            return false;
        if (((uintptr_t)o.codes | (uintptr_t)o.x) & 15) return false;
        // 32-bit buffer offsets
        if ((uint64_t)o.n * o.k / 2 >= (1ull << 31) || (uint64_t)kSkMaxM * o.k * 2 >= (1ull << 31)) return false;
    }
    return count > 0;
}

namespace {

// One launch of a class's ops (at most kMaxBatchOps, each of at most the
// class's rows). Run lengths as in the small-M kernel: the launch's pass count
// per resident workgroup (two per CU) over the op's passes, 1 .. RUN.
template <int MB, int P, int RUN>
stark_qmm_status launch_class(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream) {
    if (count > (uint32_t)kMaxBatchOps) return STARK_QMM_INVALID_ARGUMENT;  // the batch holds kMaxBatchOps
    int dev = 0, cus = 0;
    QMM_HIP_CHECK(hipGetDevice(&dev));
    QMM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    uint64_t units = 0;
    for (uint32_t i = 0; i < count; ++i)
        units += (uint64_t)((ops[i].n + kRows * kSkTiles - 1) / (kRows * kSkTiles)) * (ops[i].k / P);
    const uint64_t slots = 2 * (uint64_t)std::max(cus, 1);
    const uint64_t per_wg = (units + slots - 1) / slots;
    std::vector<AffineOp> sorted(ops, ops + count);  // longest K first: its runs take the low indices
    std::stable_sort(sorted.begin(), sorted.end(), [](const AffineOp& a, const AffineOp& b) { return a.k > b.k; });
    AffineBatch batch{};
    uint32_t runs = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t pairs = (sorted[i].n + kRows * kSkTiles - 1) / (kRows * kSkTiles);
        const uint32_t run = (uint32_t)std::min<uint64_t>(RUN, std::max<uint64_t>(1, per_wg / (sorted[i].k / P)));
        batch.op[i] = sorted[i];
        batch.op[i].block_begin = runs;
        batch.op[i].xid = run;  // tile pairs per run
        runs += (pairs + run - 1) / run;
    }
    batch.count = count;
    batch.total = runs;
    if (runs == 0) return STARK_QMM_OK;
    if (signed_codes)
        hipLaunchKernelGGL((qgemm_skinny<true, MB, P, RUN>), dim3(runs), dim3(kWg), 0, stream, batch);
    else
        hipLaunchKernelGGL((qgemm_skinny<false, MB, P, RUN>), dim3(runs), dim3(kWg), 0, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace

stark_qmm_status launch_skinny(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream) {
    std::vector<AffineOp> cls[2];  // rows 17 .. 32, 33 .. 64
    for (uint32_t i = 0; i < count; ++i) cls[ops[i].m > (uint32_t)Small::ROWS].push_back(ops[i]);
    for (int c = 0; c < 2; ++c)
        for (size_t s = 0; s < cls[c].size(); s += kMaxBatchOps) {
            const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, cls[c].size() - s);
            const stark_qmm_status st = c ? launch_class<4, 256, 1>(cls[c].data() + s, n, signed_codes, stream)
                                          : launch_class<2, 512, 3>(cls[c].data() + s, n, signed_codes, stream);
            if (st != STARK_QMM_OK) return st;
        }
    return STARK_QMM_OK;
}

}  // namespace qmm
