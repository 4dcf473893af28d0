// Affine 4/8-bit matvec / small-M product (M <= 16) on the gfx950 matrix
// cores: one workgroup per 16-row output tile of an op; the tile math is
// mfma::TileEngine (mfma_tile.h). Reference semantics: MatmulCpuKernel::encode,
// crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:168-285 (sum,
// then ab_scale, accumulate, bias, soft-cap, output rounding).
#include "mfma_tile.h"

namespace qmm {

namespace {

using namespace mfma;

// Pass length for one or two activation rows: 4096 values for 4-bit codes,
// 2048 for 8-bit (same bytes per pass, same registers).
template <int BITS>
struct PassFor {
    static constexpr int P1 = BITS == 4 ? QMM_MFMA_PASS_SMALL_M : QMM_MFMA_PASS_SMALL_M / 2;
};

template <int MP, int MB, bool SIGNED, bool BIASED, bool BF, int BITS>
__global__ __launch_bounds__(kWg) void qmv_mfma(AffineBatch batch) {
    (void)batch;
    constexpr int P1 = PassFor<BITS>::P1;
    __shared__ MfmaLds<MP, MB, P1, BITS> lds;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    // Workgroups are dealt to the 8 XCDs round-robin (id % 8), each XCD with
    // its own L2. Four neighbouring 16-row tiles share the 128-byte lines of
    // the group-output scale/bias planes, so within every 32 ids the tiles are
    // permuted to put four neighbours on one XCD: one HBM fetch per line.
    const uint32_t bid = (blockIdx.x & ~31u) + 32 <= kb->total
                             ? (blockIdx.x & ~31u) + (blockIdx.x & 7) * 4 + ((blockIdx.x >> 3) & 3)
                             : blockIdx.x;
    uint32_t oi = 0;
    for (uint32_t i = 1; i < kb->count; ++i)
        if (bid >= kb->op[i].block_begin) oi = i;
    const AffineOp& op = kb->op[oi];
    const uint32_t N = op.n, K = op.k, M = op.m;
    const uint32_t t0 = (bid - op.block_begin) * kRows;
    const uint32_t n0 = min(t0, N - kRows);  // last tile moved back to end at N
    TileEngine<MP, MB, SIGNED, BIASED, BF, P1, BITS> e(lds, kb->nib_mask, kb->nib_one);
    const auto xrow = [&](uint32_t m) { return (size_t)m * K; };
    e.load(op, n0, n0 + 8, M, xrow, 0);
    e.run(op, n0, n0 + 8, M, xrow, [] {});
    constexpr int MR = MP * MB;
    for (uint32_t t = threadIdx.x; t < (uint32_t)MR * kRows; t += kWg) {
        const uint32_t m = t / kRows, r = t % kRows;
        const uint32_t n = n0 + r;
        if (m >= M || n < t0) continue;  // padding rows; rows of the previous tile (shifted last tile)
        const size_t o = (size_t)m * N + n;
        float v = op.ab_scale * e.sum(m, r);
        if (op.flags & FLAG_ACCUMULATE) v += load_as_f32(op.d, op.d_dt, o);
        if (op.bias) v += load_as_f32(op.bias, op.w_dt, n);
        if (op.flags & FLAG_SOFT_CAP) v = op.soft_cap * tanhf(v / op.soft_cap);
        store_from_f32(op.d, op.d_dt, o, v);
    }
}

template <int MP, int MB, bool SIGNED, bool BIASED, bool BF, int BITS>
stark_qmm_status launch_one(const AffineOp* ops, uint32_t count, hipStream_t stream) {
    AffineBatch batch{};
    uint32_t blocks = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = ops[i];
        batch.op[i].block_begin = blocks;
        blocks += (ops[i].n + kRows - 1) / kRows;
    }
    batch.count = count;
    batch.total = blocks;
    if (blocks == 0) return STARK_QMM_OK;
    hipLaunchKernelGGL((qmv_mfma<MP, MB, SIGNED, BIASED, BF, BITS>), dim3(blocks), dim3(kWg), 0, stream, batch);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

template <int MP, int MB, int BITS>
stark_qmm_status launch_mp(const AffineOp* o, uint32_t c, hipStream_t st) {
    const bool sg = (o[0].flags & FLAG_SIGNED) != 0;
    const bool bi = o[0].corr_kind == STARK_QMM_CORRECTION_BIASES;
    const bool bf = o[0].w_dt == STARK_QMM_BF16;
#define QMM_L(SG, BI, BF_) launch_one<MP, MB, SG, BI, BF_, BITS>(o, c, st)
    if (sg) {
        if (bi) return bf ? QMM_L(true, true, true) : QMM_L(true, true, false);
        return bf ? QMM_L(true, false, true) : QMM_L(true, false, false);
    }
    if (bi) return bf ? QMM_L(false, true, true) : QMM_L(false, true, false);
    return bf ? QMM_L(false, false, true) : QMM_L(false, false, false);
#undef QMM_L
}

// (MP, MB) class of an activation-row count
int m_class(uint32_t m) { return m <= 1 ? 0 : m <= 2 ? 1 : m <= 4 ? 2 : m <= 8 ? 3 : 4; }

template <int BITS>
stark_qmm_status launch_class(int c, const AffineOp* o, uint32_t n, hipStream_t stream) {
    switch (c) {
    case 0: return launch_mp<1, 1, BITS>(o, n, stream);
    case 1: return launch_mp<2, 1, BITS>(o, n, stream);
    case 2: return launch_mp<4, 1, BITS>(o, n, stream);
    case 3: return launch_mp<8, 1, BITS>(o, n, stream);
    default: return launch_mp<8, 2, BITS>(o, n, stream);
    }
}

}  // namespace

bool mfma_eligible(const AffineOp& o, int bits) {
    if ((bits != 4 && bits != 8) || o.x_dt != STARK_QMM_BF16 || o.gather || o.m == 0 || o.m > 16) return false;
    if (!(o.corr_kind == STARK_QMM_CORRECTION_BIASES || o.corr_kind == STARK_QMM_CORRECTION_SYMMETRIC)) return false;
    if (o.w_dt == STARK_QMM_F32) return false;
    if (o.group_size != 32 && o.group_size != 64 && o.group_size != 128) return false;
    const int cls = m_class(o.m);
    const uint32_t mp = cls == 0 ? 1 : cls == 1 ? 2 : cls == 2 ? 4 : 8;
    if (16 / mp < 128 / o.group_size) return false;  // a step's groups must fit the slots
    if (o.k == 0 || o.k % 64 || o.n < (uint32_t)kRows || o.n % 8) return false;  // 16-byte code rows
    if (((uintptr_t)o.codes | (uintptr_t)o.x | (uintptr_t)o.scales) & 15) return false;
    if (o.corr_kind == STARK_QMM_CORRECTION_BIASES && ((uintptr_t)o.corr & 15)) return false;
    const uint32_t G = o.k / o.group_size;
    if (o.os == 1) return o.gs % 8 == 0;
    return o.gs == 1 && o.os % 8 == 0 && G % 8 == 0;
}

// ops: all mfma_eligible for `bits`; one launch per (M class, signedness,
// correction, plane type).
stark_qmm_status launch_affine_mfma(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream) {
    std::vector<AffineOp> cls[5][2][2][2];
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        cls[m_class(o.m)][(o.flags & FLAG_SIGNED) != 0][o.corr_kind == STARK_QMM_CORRECTION_BIASES]
           [o.w_dt == STARK_QMM_BF16].push_back(o);
    }
    for (int c = 0; c < 5; ++c)
        for (auto& a : cls[c])
            for (auto& b : a)
                for (auto& v : b)
                    for (size_t s = 0; s < v.size(); s += kMaxBatchOps) {
                        const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, v.size() - s);
                        const stark_qmm_status st = bits == 4 ? launch_class<4>(c, v.data() + s, n, stream)
                                                              : launch_class<8>(c, v.data() + s, n, stream);
                        if (st != STARK_QMM_OK) return st;
                    }
    return STARK_QMM_OK;
}

}  // namespace qmm
