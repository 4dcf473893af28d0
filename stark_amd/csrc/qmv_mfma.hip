// Affine 4/8-bit matvec / small-M product (M <= 16) on the gfx950 matrix
// cores: one workgroup per 16-row output tile of an op; the tile math is
// mfma::TileEngine (mfma_tile.h). Reference semantics: MatmulCpuKernel::encode,
// crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:168-285 (sum,
// then ab_scale, accumulate, bias, soft-cap, output rounding).
#include <map>
#include <mutex>

#include "mfma_tile.h"

namespace qmm {

namespace {

using namespace mfma;

// Pass length (in 4-bit k values) for one or two activation rows. 4-bit:
// 2048 values, 1 KiB of every tile row, which keeps LDS and registers at four
// workgroups per CU. 8-bit: 2048 values, 2 KiB of every row, so that a wave's
// quarter still spans 4 steps between flushes.
template <int BITS>
constexpr int kP1 = BITS == 4 ? 2048 : 4096;
// Waves per SIMD the register budget is sized for (no spills).
template <int MR, int BITS, int GS>
constexpr int kWavesPerEu = MR >= 8 || (GS == 32 && MR >= 4) ? 2 : (MR >= 4 || BITS == 8 || (GS == 32 && MR >= 2)) ? 3 : 4;

// Work distribution. The grid is persistent: as many workgroups as fit the
// chip at once, a multiple of 8. Workgroups are dealt to the 8 XCDs
// round-robin (blockIdx % 8), each XCD with its own L2. The 16-row tiles of
// all ops are cut into quads of 4 neighbouring tiles -- the four tiles that
// share the 128-byte lines of the group-output scale/bias planes -- and quad g
// belongs to XCD g % 8, so each plane line is fetched from HBM once. Within an
// XCD the tiles are dealt longest first to the least-loaded workgroup (cost =
// K), which bounds the tail by one short tile. The host builds that schedule
// once per shape set and keeps it on the device: workgroup b walks
// tiles[begin[b] .. begin[b+1]) in order, each entry (op << 24) | tile. A
// workgroup issues the next tile's loads as soon as the current tile sits in
// LDS, so HBM streams across tile boundaries; there are no atomics and no
// per-launch state.
struct Schedule {
    const uint32_t* begin;  // [grid + 1] offsets into tiles
    const uint32_t* tiles;  // [total tiles]
};

template <int MP, int MB, int GS, int BITS, bool SIGNED>
__global__ __launch_bounds__(kWg) __attribute__((amdgpu_waves_per_eu(kWavesPerEu<MP * MB, BITS, GS>))) void qmv_mfma(
    AffineBatch batch, Schedule sched) {
    (void)batch;
    constexpr int PASS = Geo<MP, MB, GS, BITS, kP1<BITS>>::PASS;
    __shared__ MfmaLds<MP, MB, GS, BITS, kP1<BITS>> lds;
    const AffineBatch* kb = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    const uint32_t lo = sched.begin[blockIdx.x], hi = sched.begin[blockIdx.x + 1];
    if (lo >= hi) return;
    TileEngine<MP, MB, GS, BITS, SIGNED, kP1<BITS>> e(lds);
    const auto rows_of = [&](uint32_t t, uint32_t& t0, uint32_t& n0) {
        const AffineOp& op = kb->op[t >> 24];
        t0 = (t & 0xffffffu) * kRows;
        n0 = min(t0, op.n - kRows);  // last tile moved back to end at N
    };
    uint32_t cur = sched.tiles[lo];
    {
        uint32_t t0, n0;
        rows_of(cur, t0, n0);
        const AffineOp& op = kb->op[cur >> 24];
        e.load(op, plane_flags(op), n0, n0 + 8, op.m, [&](uint32_t m) { return (size_t)m * op.k; }, 0);
    }
    bool keep_x = false;
    for (uint32_t i = lo; i < hi; ++i) {
        const AffineOp& op = kb->op[cur >> 24];
        const uint32_t N = op.n, M = op.m, pf = plane_flags(op);
        uint32_t t0, n0;
        rows_of(cur, t0, n0);
        const uint32_t nxt = i + 1 < hi ? sched.tiles[i + 1] : 0u;
        bool next_keep_x = false;
        e.run(op, pf, n0, n0 + 8, M, [&](uint32_t m) { return (size_t)m * op.k; }, [&] {
            if (i + 1 < hi) {
                uint32_t u0, m0;
                rows_of(nxt, u0, m0);
                const AffineOp& nop = kb->op[nxt >> 24];
                next_keep_x = (nxt >> 24) == (cur >> 24) && nop.k <= (uint32_t)Geo<MP, MB, GS, BITS, kP1<BITS>>::XK;
                e.load(nop, plane_flags(nop), m0, m0 + 8, nop.m, [&](uint32_t m) { return (size_t)m * nop.k; }, 0,
                       next_keep_x);
            }
        }, keep_x);
        keep_x = next_keep_x;
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
        cur = nxt;
    }
}

template <class Kern>
uint32_t persistent_grid(Kern kern) {
    static int cached = 0;
    if (!cached) {
        int dev = 0, cus = 0, per_cu = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kWg, 0) != hipSuccess)
            return 0;
        cached = std::max(8, cus * std::max(per_cu, 1) / 8 * 8);
    }
    return (uint32_t)cached;
}

// Device copy of the schedule of a shape set (ops in launch order: tile
// count and K each) for `grid` workgroups, built on first use and kept for
// the life of the process (a few KiB per distinct shape set and device).
bool schedule_for(const AffineOp* ops, uint32_t count, uint32_t grid, Schedule* out) {
    static std::mutex mu;
    static std::map<std::vector<uint32_t>, Schedule> cache;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    std::vector<uint32_t> key{(uint32_t)dev, grid};
    for (uint32_t i = 0; i < count; ++i) {
        key.push_back((ops[i].n + kRows - 1) / kRows);
        key.push_back(ops[i].k);
    }
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(key);
    if (it != cache.end()) {
        *out = it->second;
        return true;
    }
    const uint32_t per_xcd = grid / 8;
    std::vector<std::vector<uint32_t>> lists(grid);
    std::vector<uint64_t> load(grid, 0);
    // tiles per XCD in quad order; ops are already longest-K first, so a
    // stable walk deals the costliest tiles first
    std::vector<std::vector<std::pair<uint32_t, uint32_t>>> xcd_tiles(8);  // (entry, cost)
    uint32_t quad = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t tiles = (ops[i].n + kRows - 1) / kRows;
        for (uint32_t t0 = 0; t0 < tiles; t0 += 4, ++quad)
            for (uint32_t t = t0; t < std::min(tiles, t0 + 4); ++t) xcd_tiles[quad % 8].push_back({(i << 24) | t, ops[i].k});
    }
    for (uint32_t x = 0; x < 8; ++x) {
        for (const auto& et : xcd_tiles[x]) {
            uint32_t best = 0;
            for (uint32_t w = 1; w < per_xcd; ++w)
                if (load[x + 8 * w] < load[x + 8 * best]) best = w;
            lists[x + 8 * best].push_back(et.first);
            load[x + 8 * best] += et.second;
        }
    }
    std::vector<uint32_t> host(grid + 1);
    uint32_t total = 0;
    for (uint32_t b = 0; b < grid; ++b) {
        host[b] = total;
        total += (uint32_t)lists[b].size();
    }
    host[grid] = total;
    for (uint32_t b = 0; b < grid; ++b) host.insert(host.end(), lists[b].begin(), lists[b].end());
    void* d = nullptr;
    if (hipMalloc(&d, host.size() * sizeof(uint32_t)) != hipSuccess) return false;
    if (hipMemcpy(d, host.data(), host.size() * sizeof(uint32_t), hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        return false;
    }
    Schedule s{(const uint32_t*)d, (const uint32_t*)d + grid + 1};
    cache.emplace(std::move(key), s);
    *out = s;
    return true;
}

template <int MP, int MB, int GS, int BITS, bool SIGNED>
stark_qmm_status launch_one(const AffineOp* ops, uint32_t count, hipStream_t stream) {
    // longest K first (stable)
    std::vector<AffineOp> sorted(ops, ops + count);
    std::stable_sort(sorted.begin(), sorted.end(), [](const AffineOp& a, const AffineOp& b) { return a.k > b.k; });
    AffineBatch batch{};
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = sorted[i];
        tiles += (sorted[i].n + kRows - 1) / kRows;
    }
    batch.count = count;
    batch.total = tiles;
    if (tiles == 0) return STARK_QMM_OK;
    auto kern = qmv_mfma<MP, MB, GS, BITS, SIGNED>;
    const uint32_t grid = std::min(persistent_grid(kern), (tiles + 7) / 8 * 8);
    Schedule sched;
    if (grid == 0 || !schedule_for(sorted.data(), count, grid, &sched)) return STARK_QMM_DEVICE_FAILURE;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kWg), 0, stream, batch, sched);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

// (MP, MB) class of an activation-row count
int m_class(uint32_t m) { return m <= 1 ? 0 : m <= 2 ? 1 : m <= 4 ? 2 : m <= 8 ? 3 : 4; }

template <int MP, int MB, int BITS>
stark_qmm_status launch_gs(const AffineOp* o, uint32_t n, hipStream_t st) {
    const bool sg = (o[0].flags & FLAG_SIGNED) != 0;
    switch (o[0].group_size) {
    case 32:
        if constexpr (16 / MP >= 4) return sg ? launch_one<MP, MB, 32, BITS, true>(o, n, st)
                                              : launch_one<MP, MB, 32, BITS, false>(o, n, st);
        return STARK_QMM_UNSUPPORTED_GROUP_SIZE;
    case 64:
        return sg ? launch_one<MP, MB, 64, BITS, true>(o, n, st) : launch_one<MP, MB, 64, BITS, false>(o, n, st);
    default:
        return sg ? launch_one<MP, MB, 128, BITS, true>(o, n, st) : launch_one<MP, MB, 128, BITS, false>(o, n, st);
    }
}

template <int BITS>
stark_qmm_status launch_class(int c, const AffineOp* o, uint32_t n, hipStream_t stream) {
    switch (c) {
    case 0: return launch_gs<1, 1, BITS>(o, n, stream);
    case 1: return launch_gs<2, 1, BITS>(o, n, stream);
    case 2: return launch_gs<4, 1, BITS>(o, n, stream);
    case 3: return launch_gs<8, 1, BITS>(o, n, stream);
    default: return launch_gs<8, 2, BITS>(o, n, stream);
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
// group size). Plane type, correction and layout are per op.
stark_qmm_status launch_affine_mfma(const AffineOp* ops, uint32_t count, int bits, hipStream_t stream) {
    std::vector<AffineOp> cls[5][2][3];
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        cls[m_class(o.m)][(o.flags & FLAG_SIGNED) != 0][o.group_size == 32 ? 0 : o.group_size == 64 ? 1 : 2]
            .push_back(o);
    }
    for (int c = 0; c < 5; ++c)
        for (auto& a : cls[c])
            for (auto& v : a)
                for (size_t s = 0; s < v.size(); s += kMaxBatchOps) {
                    const uint32_t n = (uint32_t)std::min<size_t>(kMaxBatchOps, v.size() - s);
                    const stark_qmm_status st = bits == 4 ? launch_class<4>(c, v.data() + s, n, stream)
                                                          : launch_class<8>(c, v.data() + s, n, stream);
                    if (st != STARK_QMM_OK) return st;
                }
    return STARK_QMM_OK;
}

}  // namespace qmm
