// Dense small-M form of the 4-bit MLX-affine product (speculative verify:
// M = 3 .. 16 activation rows, group size 64, bf16 activations; M = 3 and 4
// measured 3.18 -> 3.50 TB/s against the slot form on the Qwen3-8B layer set,
// M = 2 stays on the slot form, 4.18 against 3.61 TB/s here).
//
// Same arithmetic as the tile engine (mfma_tile.h): codes enter
// v_mfma_f32_16x16x32_bf16 as raw bf16 bit patterns (p < 256 is p * 2^-133),
// activations are staged as bf16 x * 2^E with a per-group exponent E
// (x * 2^(E-4) where the code is the high nibble, i.e. 16 q), and each group's
// scale and bias are applied once, in f32:
// acc += s * ldexp(C, 133 - E) + bias_term * sum(x) (kernel.rs:219-265 per
// element, regrouped). The layout differs: every MFMA takes all 16 activation
// rows (A row = activation row, no group slots), covers 32 k of one group and
// accumulates the group's two halves before its flush, and a workgroup runs
// two 16-row weight tiles per pass under one activation stage (the A operand
// serves both tiles). The slot form instead needs one MFMA per 8 activation
// rows and re-stages the activations for every tile. Measured on the Qwen3-8B
// layer set against the slot form: M = 16 1.0 -> 1.94 TB/s, M = 8 1.69 ->
// 2.02 TB/s (at 8 rows half the A rows are empty and it still wins).
//
// A workgroup runs a run of 1 .. 3 tile pairs of one op pass-major, so one
// activation stage serves up to 96 weight rows. The register buffers of the
// code and activation prefetch are indexed by constants only: a buffer
// picked at run time makes the compiler merge the buffers with copies, and a
// load into registers whose previous load may be pending on another path
// waits for every load in flight, which drains the prefetch. Measured on the
// Qwen3-8B layer set: one pair per workgroup with run-time buffer choice
// 2.44 / 2.08 TB/s at M = 8 / 16, runs of three with constant buffers
// 3.27 / 2.90 TB/s.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "mfma_tile.h"

namespace qmm {

namespace {

using namespace mfma;

constexpr int kSmPass = 1024;            // k per pass: 4 waves x 256
constexpr int kSmQ = kSmPass / 4;        // k per wave per pass (4 groups)
constexpr int kSmTiles = 2;              // 16-row tiles per workgroup pass
constexpr int kSmRowB = kSmQ / 2 + 16;   // padded LDS row of a wave's codes (bytes)
constexpr int kSmGroups = kSmPass / 64;  // groups per pass
constexpr int kSmMaxRun = 3;             // tile pairs per workgroup, at most

struct SmLds {
    union {
        u32x4 stage[kSmTiles][4][kRows * kSmRowB / 16];  // codes [tile][wave][row][kSmRowB bytes]
        float red[kSmTiles][4][16][kRows];               // per-wave partial outputs, after the last pass
    };
    float2 pl[kSmTiles][kSmGroups][kRows];  // (scale, bias term) [tile][group][row]
    // activation rows, MFMA pair order, scaled; rows padded by 64 bytes so that
    // the 16 rows of one A read alternate between the two halves of the banks
    u32x4 xp[16][kSmPass / 8 + 4];
    // per-group activation sums and 133 - E (activations staged as x * 2^E);
    // rows of odd length: the flush reads rows 4kq + i of one group
    float xs[16][kSmGroups + 1];
    int xe[16][kSmGroups + 1];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t sm_rsrc(const void* p, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)min(bytes, (uint64_t)0x7fffffffu), 0x00020000);
}

template <bool SIGNED>
__global__ __launch_bounds__(kWg) __attribute__((amdgpu_waves_per_eu(2))) void qmv_small_m(AffineBatch batch) {
    (void)batch;
    __shared__ SmLds lds;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    // Workgroup b runs run b: up to kSmMaxRun consecutive tile pairs of one op
    // (op.xid pairs; the last run of an op may be shorter). A run's rows
    // already share the 64-row lines of the group-output planes; consecutive
    // runs on one XCD measured slower than this plain order.
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
    const uint32_t cnt = min(op.xid, (N + kRows * kSmTiles - 1) / (kRows * kSmTiles) - pair0);
    const uint32_t passes = K / kSmPass, steps = passes * cnt;
    // tile tt of the run's pair t covers rows n0(t, tt) .. +15 and writes
    // those from 32 (pair0 + t) + 16 tt on; a tile past N moves back to end
    // at N, so every row is written once
    const auto tile_begin = [&](uint32_t t, int tt) { return kRows * (kSmTiles * (pair0 + t) + tt); };
    const auto n0_of = [&](uint32_t t, int tt) { return min(tile_begin(t, tt), N - kRows); };
    const uint32_t row_bytes = K / 2;
    const bool bf = op.w_dt == STARK_QMM_BF16, biased = op.corr_kind == STARK_QMM_CORRECTION_BIASES;
    // Buffer loads at per-thread offsets (a step adds its pair's rows and its
    // pass's k): activation rows past M lie past their resource and read zeros.
    const __amdgpu_buffer_rsrc_t rc = sm_rsrc(op.codes, (uint64_t)N * row_bytes);
    const __amdgpu_buffer_rsrc_t rx = sm_rsrc(op.x, (uint64_t)M * K * 2);
    const __amdgpu_buffer_rsrc_t rs = sm_rsrc(op.scales, 0x7fffffffu);
    const __amdgpu_buffer_rsrc_t rb = biased ? sm_rsrc(op.corr, 0x7fffffffu) : rs;
    uint32_t co[2], xo[8];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t p = tid + 256 * i, r = p / 32, c = p % 32;
        co[i] = r * row_bytes + 16 * c;
    }
    const uint32_t po = ((tid % 16) * op.os + (tid / 16) * op.gs) * 2;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t v = tid + 256 * i, m = v / 128, c = v % 128;
        xo[i] = (m * K + 8 * c) * 2;
    }

    // Steps run pass-major: step s is pass s / cnt of pair s % cnt, and a
    // pass's activations are staged at its first step. Two register buffers
    // for codes (a step's codes are issued two steps before it is staged) and
    // two for activations.
    u32x4 wc[2][kSmTiles][2];  // codes: piece p = tid + 256 i of a tile's [16 rows][512 bytes]
    u32x4 xv[2][8];            // activations: vector v = tid + 256 i is row v / 128, values 8 (v % 128)
    uint32_t ps[2][kSmTiles], pb[2][kSmTiles];  // raw plane values of (group tid / 16, row tid % 16)
    const auto load_codes = [&](auto buf, uint32_t t, uint32_t kbase) {
        constexpr int B = decltype(buf)::value;
        const uint32_t pg = (kbase / 64) * op.gs * 2;  // bytes of the pass's first plane group
#pragma unroll
        for (int tt = 0; tt < kSmTiles; ++tt) {
            const uint32_t n0 = n0_of(t, tt);
#pragma unroll
            for (int i = 0; i < 2; ++i)
                wc[B][tt][i] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(rc, co[i] + kbase / 2, n0 * row_bytes, 2));
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
        for (int tt = 0; tt < kSmTiles; ++tt) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const uint32_t p = tid + 256 * i, r = p / 32, c = p % 32;
                *(u32x4*)((uint8_t*)lds.stage[tt][c / 8] + r * kSmRowB + 16 * (c % 8)) = wc[B][tt][i];
            }
            const float sc = plane_f32(ps[B][tt], bf);
            lds.pl[tt][tid / 16][tid % 16] = float2{sc, biased ? plane_f32(pb[B][tt], bf) : -8.0f * sc};
        }
    };
    const auto stage_x = [&](auto buf) {
        constexpr int B = decltype(buf)::value;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t v = tid + 256 * i, m = v / 128, c = v % 128;
            if (m >= M) continue;  // rows past M stay zero (cleared once); a row's 8-lane groups agree
            const u32x4 t = xv[B][i];
            // the group's exponent: its 8 vectors sit in 8 consecutive lanes
            const int E = group_shift(group_max<8>(bf16x8_exp_max(t)));
            const float se = pow2i(E), so = pow2i(E - 4);
            float f[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                f[2 * e] = __uint_as_float(t[e] << 16) * se;           // even values meet q
                f[2 * e + 1] = __uint_as_float(t[e] & 0xffff0000u) * so;  // odd values meet 16 q
            }
            u32x4 pq;  // (x0,x4)(x1,x5)(x2,x6)(x3,x7), as the codes unpack
            pq[0] = perm(__float_as_uint(f[4]), __float_as_uint(f[0]), 0x07060302u);
            pq[1] = perm(__float_as_uint(f[5]), __float_as_uint(f[1]), 0x07060302u);
            pq[2] = perm(__float_as_uint(f[6]), __float_as_uint(f[2]), 0x07060302u);
            pq[3] = perm(__float_as_uint(f[7]), __float_as_uint(f[3]), 0x07060302u);
            lds.xp[m][c] = pq;
            float sm = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) sm = dot2_bf16(t[e], 0x3F803F80u, sm);
            sm = group_sum<8>(sm);  // the 8 vectors of a group sit in consecutive lanes
            if ((c & 7) == 0) {
                lds.xs[m][c / 8] = sm;
                lds.xe[m][c / 8] = 133 - E;
            }
        }
    };

    f32x4 acc[kSmMaxRun][kSmTiles];
#pragma unroll
    for (int r = 0; r < kSmMaxRun; ++r)
#pragma unroll
        for (int tt = 0; tt < kSmTiles; ++tt) acc[r][tt] = f32x4{0, 0, 0, 0};
    // the wave's 256 k of a step: 8 chunks of 32, two per group
    const auto compute = [&](f32x4 (&a_acc)[kSmTiles]) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f32x4 C[kSmTiles];
#pragma unroll
            for (int tt = 0; tt < kSmTiles; ++tt) C[tt] = f32x4{0, 0, 0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int cc = 2 * g + h;
                const u32x4 a = lds.xp[j][wave * 32 + 4 * cc + kq];  // A row j = activation row j
#pragma unroll
                for (int tt = 0; tt < kSmTiles; ++tt) {
                    uint32_t u = *(const uint32_t*)((const uint8_t*)lds.stage[tt][wave] + j * kSmRowB + 16 * cc +
                                                    4 * kq);
                    if (SIGNED) u ^= 0x88888888u;
                    const uint32_t u8 = u >> 8;
                    const u32x4 bq{u & 0x000F000Fu, u & 0x00F000F0u, u8 & 0x000F000Fu, u8 & 0x00F000F0u};
                    C[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                                  __builtin_bit_cast(bf16x8, bq), C[tt], 0, 0, 0);
                }
            }
            // flush: lane (j, kq) holds activation rows 4kq .. 4kq+3 of tile row j
            const uint32_t gp = wave * 4 + g;  // group within the pass
            const f32x4 x4 = f32x4{lds.xs[4 * kq][gp], lds.xs[4 * kq + 1][gp], lds.xs[4 * kq + 2][gp],
                                   lds.xs[4 * kq + 3][gp]};
            const int e4[4] = {lds.xe[4 * kq][gp], lds.xe[4 * kq + 1][gp], lds.xe[4 * kq + 2][gp],
                               lds.xe[4 * kq + 3][gp]};
#pragma unroll
            for (int tt = 0; tt < kSmTiles; ++tt) {
                const float2 p = lds.pl[tt][gp][j];
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    a_acc[tt][q] = fmaf(p.x, ldexp_f32(C[tt][q], e4[q]), fmaf(p.y, x4[q], a_acc[tt][q]));
            }
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    // activation rows past M: zero once (their products and sums are zero)
    for (uint32_t v = tid; v < 16 * (kSmPass / 8); v += kWg) {
        const uint32_t m = v / (kSmPass / 8);
        if (m >= M) lds.xp[m][v % (kSmPass / 8)] = u32x4{0, 0, 0, 0};
    }
    for (uint32_t v = tid; v < 16 * kSmGroups; v += kWg)
        if (v / kSmGroups >= M) {
            lds.xs[v / kSmGroups][v % kSmGroups] = 0.0f;
            lds.xe[v / kSmGroups][v % kSmGroups] = 0;
        }
    // The step loop is unrolled over two steps, so that a step's code buffer
    // is its parity, a constant. A run of one pair (ONE) takes its activations
    // two passes ahead into the buffer of the pass's parity (also the step's);
    // a longer run takes them one pass (cnt steps) ahead into one buffer.
    const auto run = [&](auto one_c) {
        constexpr bool ONE = decltype(one_c)::value;
        constexpr uint32_t XA = ONE ? 2 : 1;  // passes ahead of the activation loads
        load_codes(B0{}, 0, 0);
        uint32_t lp = 0, lt = 1;  // load cursor: pass and pair of step s + 2
        if (lt == cnt) lt = 0, lp = 1;
        if (steps > 1) load_codes(B1{}, lt, lp * kSmPass);
        if (++lt == cnt) lt = 0, ++lp;
        load_x(B0{}, 0);
        if (ONE && passes > 1) load_x(B1{}, kSmPass);
        uint32_t p = 0, t = 0;
        const auto step = [&](auto b_c, uint32_t s) {
            constexpr int SB = decltype(b_c)::value;
            using BS = std::integral_constant<int, SB>;
            using BX = std::integral_constant<int, ONE ? SB : 0>;
            if (s) __syncthreads();  // every wave finished the previous step's LDS
            stage_codes(BS{});
            // a buffer's next activation loads are issued right after it is
            // staged, on the same path (a load into registers whose previous
            // load may still be pending on another path waits for every load)
            if (ONE || t == 0) {
                stage_x(BX{});
                if (p + XA < passes) load_x(BX{}, (p + XA) * kSmPass);
            }
            __syncthreads();
            if (s + 2 < steps) {
                load_codes(BS{}, lt, lp * kSmPass);
                if (++lt == cnt) lt = 0, ++lp;
            }
            if (ONE) {
                compute(acc[0]);
            } else {
#pragma unroll
                for (int r = 0; r < kSmMaxRun; ++r)
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
    for (int r = 0; r < kSmMaxRun; ++r) {
        if ((uint32_t)r >= cnt) break;
        __syncthreads();  // the results overwrite the code stage / the previous pair's results
#pragma unroll
        for (int tt = 0; tt < kSmTiles; ++tt)
#pragma unroll
            for (int q = 0; q < 4; ++q) lds.red[tt][wave][4 * kq + q][j] = acc[r][tt][q];
        __syncthreads();
        for (uint32_t v = tid; v < (uint32_t)(kSmTiles * 16 * kRows); v += kWg) {
            const uint32_t tt = v / (16 * kRows), m = (v / kRows) % 16, rr = v % kRows;
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

bool small_m_eligible(const AffineOp* ops, uint32_t count) {
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        if (o.m < 3 || o.m > 16 || o.group_size != 64 || o.k % kSmPass || o.n < (uint32_t)kRows || o.gather)
            return false;
        if (o.x_dt != STARK_QMM_BF16 || !(o.w_dt == STARK_QMM_BF16 || o.w_dt == STARK_QMM_F16)) return false;
        if (!(o.corr_kind == STARK_QMM_CORRECTION_BIASES || o.corr_kind == STARK_QMM_CORRECTION_SYMMETRIC))
            return false;
        if (((uintptr_t)o.codes | (uintptr_t)o.x) & 15) return false;
        // 32-bit buffer offsets
        if ((uint64_t)o.n * o.k / 2 >= (1ull << 31) || (uint64_t)16 * o.k * 2 >= (1ull << 31)) return false;
    }
    return count > 0;
}

stark_qmm_status launch_small_m(const AffineOp* ops, uint32_t count, bool signed_codes, hipStream_t stream) {
    if (count > (uint32_t)kMaxBatchOps) return STARK_QMM_INVALID_ARGUMENT;  // the batch holds kMaxBatchOps
    int dev = 0, cus = 0;
    QMM_HIP_CHECK(hipGetDevice(&dev));
    QMM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // Runs: a workgroup takes up to kSmMaxRun tile pairs of one op, so one
    // activation stage serves that many pairs. The run length of an op is the
    // launch's pass count per resident workgroup (two per CU) over the op's
    // passes: a launch of deep and shallow products then gives every
    // workgroup about the same number of steps (the Qwen3-8B layer set: one
    // pair of the K = 12288 down product or three pairs of the K = 4096
    // products, 12 steps each, 492 workgroups), and a launch of few pairs
    // keeps one pair per workgroup.
    uint64_t units = 0;
    for (uint32_t i = 0; i < count; ++i)
        units += (uint64_t)((ops[i].n + kRows * kSmTiles - 1) / (kRows * kSmTiles)) * (ops[i].k / kSmPass);
    const uint64_t slots = 2 * (uint64_t)std::max(cus, 1);
    const uint64_t per_wg = (units + slots - 1) / slots;
    // longest K first: its runs take the low run indices
    std::vector<AffineOp> sorted(ops, ops + count);
    std::stable_sort(sorted.begin(), sorted.end(), [](const AffineOp& a, const AffineOp& b) { return a.k > b.k; });
    AffineBatch batch{};
    uint32_t runs = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t pairs = (sorted[i].n + kRows * kSmTiles - 1) / (kRows * kSmTiles);
        const uint32_t run =
            (uint32_t)std::min<uint64_t>(kSmMaxRun, std::max<uint64_t>(1, per_wg / (sorted[i].k / kSmPass)));
        batch.op[i] = sorted[i];
        batch.op[i].block_begin = runs;
        batch.op[i].xid = run;  // tile pairs per run
        runs += (pairs + run - 1) / run;
    }
    batch.count = count;
    batch.total = runs;
    if (runs == 0) return STARK_QMM_OK;
    if (signed_codes)
        hipLaunchKernelGGL(qmv_small_m<true>, dim3(runs), dim3(kWg), 0, stream, batch);
    else
        hipLaunchKernelGGL(qmv_small_m<false>, dim3(runs), dim3(kWg), 0, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm
