// Affine 4/8-bit matvec / small-M product (M <= 16) on the gfx950 matrix
// cores: one workgroup per 16-row output tile of an op; the tile math is
// mfma::TileEngine (mfma_tile.h). Reference semantics: MatmulCpuKernel::encode,
// crates/stark-engine/src/backends/cpu/kernel/matmul/kernel.rs:168-285 (sum,
// then ab_scale, accumulate, bias, soft-cap, output rounding).
#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>

#include "stream_common.h"

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
        e.run(op, pf, n0, n0 + 8, M, [&](uint32_t m) { return (size_t)m * op.k; }, [&](auto& nl) {
            if (i + 1 >= hi) return false;
            uint32_t u0, m0;
            rows_of(nxt, u0, m0);
            const AffineOp& nop = kb->op[nxt >> 24];
            next_keep_x = (nxt >> 24) == (cur >> 24) && nop.k <= (uint32_t)Geo<MP, MB, GS, BITS, kP1<BITS>>::XK;
            nl = {&nop, plane_flags(nop), m0, m0 + 8, nop.m, 0u, next_keep_x, true};
            return true;
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

// Workgroups of `kern` that fit the device at once (a multiple of 8), cached
// per (kernel, device).
template <class Kern>
uint32_t persistent_grid(Kern kern, int block = kWg) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, uint32_t> cache;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair((const void*)kern, dev);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, block, 0) != hipSuccess)
        return 0;
    const uint32_t grid = (uint32_t)std::max(8, cus * std::max(per_cu, 1) / 8 * 8);
    cache.emplace(key, grid);
    return grid;
}

// ---- Schedule store. The host-built schedules live in a file-scope device
// array (one copy per GPU, no allocation on any call) and are written by a
// stream-ordered upload kernel whose payload travels in its kernel arguments,
// so a first call on a new shape set neither allocates nor waits for the
// device: it enqueues one or more small upload launches ahead of the product
// on the caller's stream. Entries are immutable once written.
//  - Another stream that uses an entry before its upload has completed waits
//    for it on the device (hipStreamWaitEvent), never on the host.
//  - Under stream capture the upload becomes part of the graph (every replay
//    rewrites the same words); such an entry is pinned for the life of the
//    process, and the next eager call uploads it once more for eager use.
//  - When the store is full, an eager call synchronizes the device once and
//    drops every unpinned entry (the only blocking case; a capturing call
//    gets STARK_QMM_OUT_OF_MEMORY instead).
constexpr uint32_t kStoreWords = 1u << 20;   // 4 MiB per device
constexpr uint32_t kUploadWords = 960;       // payload words per upload launch (3.8 KB of arguments)
__device__ __align__(256) uint32_t sched_store[kStoreWords];

struct UploadChunk {
    uint32_t offset, count;
    uint32_t w[kUploadWords];
};

__global__ __launch_bounds__(256) void sched_upload(uint32_t* store, UploadChunk c) {
    for (uint32_t i = threadIdx.x; i < c.count; i += 256) store[c.offset + i] = c.w[i];
}

struct StoreEntry {
    std::vector<uint32_t> host;  // begin[grid + 1] then the tile lists
    uint32_t offset = 0;
    hipEvent_t done = nullptr;   // recorded after the eager upload
    bool eager = false;          // uploaded outside capture
    bool landed = false;         // the eager upload has been seen complete
    bool pinned = false;         // referenced by a captured graph
    hipStream_t stream = nullptr;  // stream of the eager upload
};

struct DeviceStore {
    uint32_t* base = nullptr;
    uint32_t used = 0;
    std::map<std::vector<uint32_t>, StoreEntry> entries;
};

stark_qmm_status upload(uint32_t* base, const StoreEntry& e, hipStream_t stream) {
    UploadChunk c;
    for (size_t s = 0; s < e.host.size(); s += kUploadWords) {
        c.offset = e.offset + (uint32_t)s;
        c.count = (uint32_t)std::min<size_t>(kUploadWords, e.host.size() - s);
        std::copy(e.host.begin() + s, e.host.begin() + s + c.count, c.w);
        hipLaunchKernelGGL(sched_upload, dim3(1), dim3(256), 0, stream, base, c);
        QMM_HIP_CHECK(hipGetLastError());
    }
    return STARK_QMM_OK;
}

// Tile lists of a shape set (ops in launch order: tile count and K each) for
// `grid` workgroups and tiles of `rows` rows. The tiles that share the
// 128-byte lines of the group-output planes (64 rows) go to one XCD.
std::vector<uint32_t> build_schedule(const AffineOp* ops, uint32_t count, uint32_t grid, uint32_t rows) {
    const uint32_t per_xcd = grid / 8;
    std::vector<std::vector<uint32_t>> lists(grid);
    std::vector<uint64_t> load(grid, 0);
    // tiles per XCD in line-group order; ops are already longest-K first, so
    // a stable walk deals the costliest tiles first
    std::vector<std::vector<std::pair<uint32_t, uint32_t>>> xcd_tiles(8);  // (entry, cost)
    const uint32_t per_line = std::max(1u, 64 / rows);
    uint32_t quad = 0;
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t tiles = (ops[i].n + rows - 1) / rows;
        for (uint32_t t0 = 0; t0 < tiles; t0 += per_line, ++quad)
            for (uint32_t t = t0; t < std::min(tiles, t0 + per_line); ++t)
                xcd_tiles[quad % 8].push_back({(i << 24) | t, ops[i].k});
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
    // Streaming kernel (32-row tiles): within each XCD the lists with the most
    // tiles go to the workgroups dispatched first. Workgroups dispatched late
    // queue behind everyone's first loads; a list of one long tile (no tile
    // switches) absorbs that best (measured: launch median 25.6 -> 24.3 us on
    // the Qwen3-8B layer set).
    if (rows == 32) {
        for (uint32_t x = 0; x < 8; ++x) {
            std::vector<uint32_t> idx(per_xcd);
            for (uint32_t w = 0; w < per_xcd; ++w) idx[w] = w;
            std::stable_sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) {
                return lists[x + 8 * a].size() > lists[x + 8 * b].size();
            });
            std::vector<std::vector<uint32_t>> sorted_lists(per_xcd);
            for (uint32_t w = 0; w < per_xcd; ++w) sorted_lists[w] = std::move(lists[x + 8 * idx[w]]);
            for (uint32_t w = 0; w < per_xcd; ++w) lists[x + 8 * w] = std::move(sorted_lists[w]);
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
    return host;
}

// Device schedule of a shape set, uploaded on `stream` on first use (see the
// store above).
stark_qmm_status store_schedule(const std::vector<uint32_t>& key, uint32_t grid,
                                const std::function<std::vector<uint32_t>()>& build, Schedule* out,
                                hipStream_t stream) {
    static std::mutex mu;
    static std::map<int, DeviceStore> stores;
    int dev = 0;
    QMM_HIP_CHECK(hipGetDevice(&dev));
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    QMM_HIP_CHECK(hipStreamIsCapturing(stream, &cap));
    const bool capturing = cap != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(mu);
    DeviceStore& ds = stores[dev];
    if (!ds.base) QMM_HIP_CHECK(hipGetSymbolAddress((void**)&ds.base, HIP_SYMBOL(sched_store)));
    auto it = ds.entries.find(key);
    if (it == ds.entries.end()) {
        StoreEntry e;
        e.host = build();
        const uint32_t words = ((uint32_t)e.host.size() + 63) / 64 * 64;
        if (words > kStoreWords) return STARK_QMM_OUT_OF_MEMORY;
        if (ds.used + words > kStoreWords) {
            if (capturing) return STARK_QMM_OUT_OF_MEMORY;
            QMM_HIP_CHECK(hipDeviceSynchronize());
            uint32_t end = 0;
            for (auto jt = ds.entries.begin(); jt != ds.entries.end();) {
                if (jt->second.pinned) {
                    end = std::max(end, jt->second.offset + ((uint32_t)jt->second.host.size() + 63) / 64 * 64);
                    ++jt;
                } else {
                    if (jt->second.done) (void)hipEventDestroy(jt->second.done);
                    jt = ds.entries.erase(jt);
                }
            }
            ds.used = end;
            if (ds.used + words > kStoreWords) return STARK_QMM_OUT_OF_MEMORY;
        }
        e.offset = ds.used;
        ds.used += words;
        it = ds.entries.emplace(std::move(key), std::move(e)).first;
    }
    StoreEntry& e = it->second;
    if (capturing) {
        // An eager upload that has completed serves the graph too. One still
        // in flight (or of unknown state: nothing here may wait while a
        // stream captures) is repeated inside the graph, ordered before the
        // product; the words are the same.
        // (an event recorded on the capturing stream itself is not queried:
        // that would invalidate the capture)
        if (e.eager && !e.landed && e.stream != stream) {
            if (hipEventQuery(e.done) == hipSuccess)
                e.landed = true;
            else
                (void)hipGetLastError();
        }
        if (!e.landed) {
            const stark_qmm_status st = upload(ds.base, e, stream);
            if (st != STARK_QMM_OK) return st;
        }
        e.pinned = true;
    } else if (!e.eager) {
        const stark_qmm_status st = upload(ds.base, e, stream);
        if (st != STARK_QMM_OK) return st;
        if (!e.done) QMM_HIP_CHECK(hipEventCreateWithFlags(&e.done, hipEventDisableTiming));
        QMM_HIP_CHECK(hipEventRecord(e.done, stream));
        e.eager = true;
        e.stream = stream;
    } else if (!e.landed) {
        const hipError_t q = hipEventQuery(e.done);
        if (q == hipSuccess)
            e.landed = true;
        else if (q == hipErrorNotReady)
            QMM_HIP_CHECK(hipStreamWaitEvent(stream, e.done, 0));
        else
            return STARK_QMM_DEVICE_FAILURE;
    }
    *out = Schedule{ds.base + e.offset, ds.base + e.offset + grid + 1};
    return STARK_QMM_OK;
}

// Schedule of a shape set for `grid` workgroups and tiles of `rows` rows.
stark_qmm_status schedule_for(const AffineOp* ops, uint32_t count, uint32_t grid, Schedule* out, hipStream_t stream,
                              uint32_t rows = kRows) {
    std::vector<uint32_t> key{grid, rows};
    for (uint32_t i = 0; i < count; ++i) {
        key.push_back((ops[i].n + rows - 1) / rows);
        key.push_back(ops[i].k);
    }
    return store_schedule(key, grid, [&] { return build_schedule(ops, count, grid, rows); }, out, stream);
}


// BF: bf16 planes (else f16); BIASED: bias plane (else symmetric). Both are
// compile-time so that the per-unit plane conversion is straight-line code.
// PRO: input prologue (STARK_QMM_PROLOGUE_*; every op reads the same row).
// WV: waves per workgroup, each taking every WV-th unit of a tile (4: two
// workgroups per CU; 12: one workgroup of three waves per SIMD, for launches
// of 12288-deep products with fewer tiles than CUs, whose tiles then keep
// three times the loads in flight).
template <bool SIGNED, bool BF, bool BIASED, int PRO = STARK_QMM_PROLOGUE_NONE, int WV = 4, int TR = kTR>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(WV == 4 ? 2 : WV / 4))) void qmv_stream(
    AffineBatch batch, Schedule sched) {
    (void)batch;
    static_assert(TR == 32 || TR == 16, "tile rows");
    constexpr int NS = TR / 8;             // 8-row subtiles of a tile
    constexpr int NSTEP = 4 * NS;          // steps of a unit: 4 k blocks x NS subtiles
    constexpr uint32_t UB = kUnitK / 2;    // bytes of a row per unit
    constexpr uint32_t OOB = 0x80000000u;  // buffer offset past every resource: reads zero, no traffic
    constexpr uint32_t PLANE = 0x7fffffffu;  // plane resources: addressed by the op's strides
    __shared__ StreamLds<WV> lds;
    const AffineBatch* kb_ = (const AffineBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    typedef const __attribute__((address_space(4))) uint32_t cu32;
    const uint32_t lo = ((cu32*)sched.begin)[blockIdx.x], hi = ((cu32*)sched.begin)[blockIdx.x + 1];
    if (lo >= hi) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // lane roles: c16 = B/C column = (byte half hh, subtile row r), kb = k block
    const uint32_t c16 = lane & 15, kb = lane >> 4, hh = c16 >> 3, r = lane & 7;
    const uint32_t piece = 16 * (4 * hh + kb);  // this lane's 16 bytes of a row's 128-byte block
    if (lane < 4) lds.zero[wave][lane] = u32x4{0, 0, 0, 0};
    // The workgroup's schedule entries go to LDS once, so that no unit waits on
    // a scalar miss for its successor. Their load is issued first and written
    // to LDS after the first unit's loads are on their way (by the first kListLds threads).
    const uint32_t list_v = tid < min(hi - lo, (uint32_t)kListLds) ? sched.tiles[lo + tid] : 0u;
    const auto entry = [&](uint32_t t) {
        return t - lo < (uint32_t)kListLds ? __builtin_amdgcn_readfirstlane(lds.list[t - lo])
                                           : ((cu32*)sched.tiles)[t];
    };
    const auto tile_row = [&](const AffineOp& op, uint32_t e) {  // first bank row of the tile
        return min((e & 0xffffffu) * TR, op.n - TR);
    };

    // RMS-norm prologue. The sum of squares runs in chunk-major order: the
    // first four waves' lane l sums, for chunks c = wave, wave + 4, ... (1024
    // values each), the 8-value vectors 128c + l and 128c + 64 + l -- the two
    // vectors a wave stages of its chunk -- then the wave sums (xor butterfly)
    // and the four waves in order (the decode loop's RMS-norm kernel sums in
    // the same order). With K = 4096 and four waves every wave computes all
    // four waves' sums itself (eight vectors per lane, L2 hits after the
    // first), so that no wave waits for another's loads; otherwise the row's
    // first two chunks per wave are loaded before the first unit's loads (so
    // that waiting for them waits for nothing else), summed after those are
    // issued and combined through LDS at the list barrier.
    u32x4 q4[4], q8[8];
    const AffineOp& o0 = kb_->op[((cu32*)sched.tiles)[lo] >> 24];
    const __amdgpu_buffer_rsrc_t x0r = rsrc(o0.x, o0.k * 2);
    const bool ss_from_stage = WV == 4 && o0.k == 4 * kUnitK;
    const auto ss_offset = [&](uint32_t c, int half) {  // byte offset of vector 128c + 64 half + lane
        return wave < 4 ? (c * kUnitK + 512 * half + lane * 8) * 2 : OOB;
    };
    if constexpr (PRO == STARK_QMM_PROLOGUE_RMS_NORM) {
        if (ss_from_stage) {
#pragma unroll
            for (int j = 0; j < 8; ++j) q8[j] = buf_load(x0r, ((j >> 1) * kUnitK + 512 * (j & 1) + lane * 8) * 2);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) q4[j] = buf_load(x0r, ss_offset(wave + 4 * (j >> 1), j & 1));
        }
    }

    u32x4 ring[8];
    u32x4 xv[2], pls, plb;  // plb reads zero when the op has no bias plane
    u32x4 pv[2];            // prologue operand at the activations' positions
    // Activations (when need_x) and plane vectors of unit (op, tile at n0, chunk c).
    const auto issue_aux = [&](const AffineOp& op, uint32_t n0, uint32_t c, bool need_x) {
        const __amdgpu_buffer_rsrc_t xr = rsrc(op.x, op.k * 2);
        const uint32_t xo = need_x ? (c * kUnitK + lane * 8) * 2 : OOB;
        xv[0] = buf_load(xr, xo);
        xv[1] = buf_load(xr, xo + 1024);
        if constexpr (PRO != STARK_QMM_PROLOGUE_NONE) {
            const __amdgpu_buffer_rsrc_t pr = rsrc(kb_->pro_data, op.k * 2);
            pv[0] = buf_load(pr, xo);
            pv[1] = buf_load(pr, xo + 1024);
        }
        // group-output [G][N4]: lane = (group, 8-row part of the TR rows);
        // output-group [N][G]: lane = (row, half of the 16 groups); with
        // 16-row tiles lanes 32..63 repeat lanes 0..31
        const size_t off = op.os == 1 ? (size_t)(c * 16 + ((lane / NS) & 15)) * op.gs + n0 + 8 * (lane % NS)
                                      : (size_t)(n0 + ((lane >> 1) & (TR - 1))) * op.os + c * 16 + 8 * (lane & 1);
        pls = buf_load(rsrc(op.scales, PLANE), (uint32_t)off * 2);
        plb = buf_load(rsrc(op.corr, PLANE), BIASED ? (uint32_t)off * 2 : OOB);
    };
    const auto code_rsrc = [&](const AffineOp& op, uint32_t n0) {
        return rsrc(op.codes + (size_t)n0 * (op.k / 2), TR * (op.k / 2));
    };
    // step v of a unit: k block v / NS of subtile v % NS
    const auto step_soff = [&](const AffineOp& op, int v) { return (uint32_t)(8 * (v % NS)) * (op.k / 2) + (v / NS) * 128; };

    uint32_t i = lo, ri = 0, e = ((cu32*)sched.tiles)[lo];
    const AffineOp* opp = &kb_->op[e >> 24];
    __amdgpu_buffer_rsrc_t cr;
    uint32_t vo;
    {
        const uint32_t n0 = tile_row(*opp, e);
        issue_aux(*opp, n0, wave, true);
        cr = code_rsrc(*opp, n0);
        vo = r * (opp->k / 2) + wave * UB + piece;
#pragma unroll
        for (int s = 0; s < 8; ++s) ring[s] = buf_load<kBufNt>(cr, vo, step_soff(*opp, s));
    }
    float inv = 0.0f;
    if (PRO == STARK_QMM_PROLOGUE_RMS_NORM && ss_from_stage) {
        float p[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            float ss = 0.0f;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float a = __uint_as_float(q8[2 * w + h][q] << 16);
                    const float b = __uint_as_float(q8[2 * w + h][q] & 0xffff0000u);
                    ss = fmaf(a, a, fmaf(b, b, ss));
                }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
            p[w] = ss;
        }
        inv = 1.0f / sqrtf((p[0] + p[1] + p[2] + p[3]) / (float)o0.k + kb_->pro_eps);
    }
    if (PRO == STARK_QMM_PROLOGUE_RMS_NORM && !ss_from_stage && wave < 4) {
        // (loads past the row read zero and add nothing)
        float ss = 0.0f;
        const auto sq = [&](const u32x4& u) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float a = __uint_as_float(u[q] << 16), b = __uint_as_float(u[q] & 0xffff0000u);
                ss = fmaf(a, a, fmaf(b, b, ss));
            }
        };
        {
            const uint32_t nch = o0.k / kUnitK;
            for (uint32_t c = wave;;) {
#pragma unroll
                for (int j = 0; j < 4; ++j) sq(q4[j]);
                c += 8;
                if (c >= nch) break;
#pragma unroll
                for (int j = 0; j < 4; ++j) q4[j] = buf_load(x0r, ss_offset(c + 4 * (j >> 1), j & 1));
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (lane == 0) lds.ssq[wave] = ss;
    }
    if (tid < (uint32_t)kListLds) lds.list[tid] = list_v;
    lds_barrier();
    if (PRO == STARK_QMM_PROLOGUE_RMS_NORM && !ss_from_stage)
        inv = 1.0f / sqrtf((lds.ssq[0] + lds.ssq[1] + lds.ssq[2] + lds.ssq[3]) / (float)opp->k + kb_->pro_eps);
    uint32_t tg0 = ~0u, tg1 = ~0u, tg2 = ~0u;  // (op << 16 | chunk) held by each activation region
    const auto tag_of = [&](uint32_t rg) { return rg == 0 ? tg0 : rg == 1 ? tg1 : tg2; };
    f32x4 acc[NS] = {};
    uint32_t par = 0;
    for (;;) {
        const AffineOp& op = *opp;
        const uint32_t R = op.k / (WV * kUnitK);
        const uint32_t t0 = (e & 0xffffffu) * TR, n0 = min(t0, op.n - TR);
        const uint32_t c = wave + WV * ri;
        const uint32_t rg = ri % kXR;
        const uint32_t tag = (op.xid << 16) | c;
        u32x4* xpw = lds.xp[wave][rg];
        float* xsw = lds.xs[wave][rg];
        int* xew = lds.xe[wave][rg];
        if (tag_of(rg) != tag) {  // stage this unit's activations (loaded with the unit)
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                u32x4 t = xv[m];
                if constexpr (PRO == STARK_QMM_PROLOGUE_RMS_NORM) t = prologue_norm(t, pv[m], inv);
                if constexpr (PRO == STARK_QMM_PROLOGUE_SILU_GATE) t = prologue_silu(t, pv[m]);
                // the group's exponent: its 8 vectors sit in 8 consecutive lanes
                const int E = group_shift(group_max<8>(bf16x8_exp_max(t)));
                const float se = pow2i(E), so = pow2i(E - 4);
                float f[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f[2 * q] = __uint_as_float(t[q] << 16) * se;
                    f[2 * q + 1] = __uint_as_float(t[q] & 0xffff0000u) * so;
                }
                u32x4 pq;  // (x0,x4)(x1,x5)(x2,x6)(x3,x7), as the codes unpack
                pq[0] = perm(__float_as_uint(f[4]), __float_as_uint(f[0]), 0x07060302u);
                pq[1] = perm(__float_as_uint(f[5]), __float_as_uint(f[1]), 0x07060302u);
                pq[2] = perm(__float_as_uint(f[6]), __float_as_uint(f[2]), 0x07060302u);
                pq[3] = perm(__float_as_uint(f[7]), __float_as_uint(f[3]), 0x07060302u);
                xpw[lane + 64 * m] = pq;
                float sm = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q) sm = dot2_bf16(t[q], 0x3F803F80u, sm);
                sm = group_sum<8>(sm);
                if ((lane & 7) == 0) {
                    xsw[8 * m + (lane >> 3)] = sm;
                    xew[8 * m + (lane >> 3)] = 133 - E;
                }
            }
            tg0 = rg == 0 ? tag : tg0;
            tg1 = rg == 1 ? tag : tg1;
            tg2 = rg == 2 ? tag : tg2;
        }
        {  // plane vectors -> f32 (scale, bias term) pairs at [row][group]
            float sv[8], bv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t hs = (pls[q >> 1] >> (16 * (q & 1))) & 0xffffu;
                const uint32_t hb = (plb[q >> 1] >> (16 * (q & 1))) & 0xffffu;
                const float sc = plane_f32(hs, BF);
                sv[q] = sc;
                bv[q] = BIASED ? plane_f32(hb, BF) : -8.0f * sc;
            }
            float2* pw = (float2*)lds.pl[wave];
            if (op.os == 1) {  // lane = (group, rows 8*part ..)
                const uint32_t g = (lane / NS) & 15, r0 = 8 * (lane % NS);
                if (lane < 16 * NS) {
#pragma unroll
                    for (int q = 0; q < 8; ++q) pw[(r0 + q) * 16 + g] = float2{sv[q], bv[q]};
                }
            } else if (lane < 2 * TR) {  // lane = (row, groups 8*half ..)
                const uint32_t row = (lane >> 1) & (TR - 1), g0 = 8 * (lane & 1);
#pragma unroll
                for (int q = 0; q < 8; ++q) pw[row * 16 + g0 + q] = float2{sv[q], bv[q]};
            }
        }

        // ---- next unit: issue its activation and plane loads now; its code
        // loads refill the ring from step 8 on
        uint32_t ni = i, nr = ri + 1;
        if (nr == R) {
            ni = i + 1;
            nr = 0;
        }
        const bool more = ni < hi;
        const uint32_t ne = more ? entry(ni) : e;
        const uint32_t nc = more ? wave + WV * nr : c;
        const AffineOp& nop = kb_->op[ne >> 24];
        const uint32_t nn0 = tile_row(nop, ne);
        issue_aux(nop, nn0, nc, more && tag_of(nr % kXR) != ((nop.xid << 16) | nc));
        const __amdgpu_buffer_rsrc_t ncr = code_rsrc(nop, nn0);
        const uint32_t nvo = more ? r * (nop.k / 2) + nc * UB + piece : OOB;

        // ---- the unit's NSTEP steps
        f32x4 C0[NS] = {}, C1[NS] = {};
        const u32x4* zero = lds.zero[wave];
#pragma unroll
        for (int u = 0; u < NSTEP; ++u) {
            const int st = u % NS, ks = u / NS, sl = u % 8;
            // unpack this step's codes, then refill the ring slot: the
            // scheduling barrier keeps the refill after the last read of the
            // slot, so the slot keeps its registers across units (a copy of a
            // register with a load in flight would wait for every load)
            u32x4 bq[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t w = ring[sl][t];
                if (SIGNED) w ^= 0x88888888u;
                const uint32_t w8 = w >> 8;
                bq[t][0] = w & 0x000F000Fu;   // (q0, q4)
                bq[t][1] = w & 0x00F000F0u;   // (16 q1, 16 q5)
                bq[t][2] = w8 & 0x000F000Fu;  // (q2, q6)
                bq[t][3] = w8 & 0x00F000F0u;  // (16 q3, 16 q7)
            }
            __builtin_amdgcn_sched_barrier(0);
            if (u + 8 < NSTEP)
                ring[sl] = buf_load<kBufNt>(cr, vo, step_soff(op, u + 8));
            else
                ring[sl] = buf_load<kBufNt>(ncr, nvo, step_soff(nop, u + 8 - NSTEP));
            // A row c16 = (byte half hh, slot r): x of this lane's k block when
            // the block's group (4ks + 2hh + kb/2 of the unit) sits in slot r
            const u32x4* src = r == 2 * ks + (kb >> 1) ? xpw + 32 * ks + 16 * hh + 4 * kb : zero;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                f32x4& cc = (t & 1) ? C1[st] : C0[st];
                cc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, src[t]),
                                                             __builtin_bit_cast(bf16x8, bq[t]), cc, 0, 0, 0);
            }
        }
        cr = ncr;
        vo = nvo;

        // ---- flush: C row 4kb+q of column (hh, r) is slot 4(kb&1)+q of byte
        // half kb>>1, i.e. unit group gb + 4(q>>1) + (q&1) of row r, with
        // gb = 8(kb&1) + 2hh (meaningful where kb>>1 == hh; the other lanes'
        // sums are dropped at the tile end)
        {
            const uint32_t gb = 8 * (kb & 1) + 2 * hh;
            const float2 xa = *(const float2*)&xsw[gb];
            const float2 xb = *(const float2*)&xsw[gb + 4];
            const float xq[4] = {xa.x, xa.y, xb.x, xb.y};
            const int2 ea = *(const int2*)&xew[gb];
            const int2 eb = *(const int2*)&xew[gb + 4];
            const int nq[4] = {ea.x, ea.y, eb.x, eb.y};
            const f32x4* pw = lds.pl[wave];
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                const f32x4 cs = C0[st] + C1[st];
                const uint32_t row = 8 * st + r;
                const f32x4 pa = pw[(row * 16 + gb) / 2], pb = pw[(row * 16 + gb + 4) / 2];  // (s, b) of 2 groups each
                const float sq[4] = {pa[0], pa[2], pb[0], pb[2]}, bq[4] = {pa[1], pa[3], pb[1], pb[3]};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc[st][q] = fmaf(sq[q], ldexp_f32(cs[q], nq[q]), fmaf(bq[q], xq[q], acc[st][q]));
            }
        }

        // ---- tile end: the row sums of the four waves meet in LDS, then the D-ops
        if (ri + 1 == R) {
#pragma unroll
            for (int st = 0; st < NS; ++st) {
                float v = (acc[st][0] + acc[st][1]) + (acc[st][2] + acc[st][3]);
                v = (kb >> 1) == hh ? v : 0.0f;  // lanes whose C rows pair the other byte half hold no row
                v += __shfl_xor(v, 8, 64);
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                if (lane < 8) lds.red[par][wave][8 * st + lane] = v;
                acc[st] = f32x4{0, 0, 0, 0};
            }
            lds_barrier();
            if (tid < (uint32_t)TR) {
                const uint32_t n = n0 + tid;
                if (n >= t0) {  // rows of the previous tile (shifted last tile) are not written again
                    // the waves' sums in fixed order: fours added pairwise, then the fours in turn
                    float o = (lds.red[par][0][tid] + lds.red[par][1][tid]) + (lds.red[par][2][tid] + lds.red[par][3][tid]);
#pragma unroll
                    for (int w = 4; w < WV; w += 4)
                        o += (lds.red[par][w][tid] + lds.red[par][w + 1][tid]) +
                             (lds.red[par][w + 2][tid] + lds.red[par][w + 3][tid]);
                    o *= op.ab_scale;
                    if (op.flags & FLAG_ACCUMULATE) o += load_as_f32(op.d, op.d_dt, n);
                    if (op.bias) o += load_as_f32(op.bias, op.w_dt, n);
                    if (op.flags & FLAG_SOFT_CAP) o = op.soft_cap * tanhf(o / op.soft_cap);
                    store_from_f32(op.d, op.d_dt, n, o);
                }
            }
            par ^= 1;
        }
        if (!more) break;
        i = ni;
        ri = nr;
        e = ne;
        opp = &nop;
    }
}

// Whether a batch of 4-bit ops takes the streaming kernel (one activation
// row, group size 64, K a multiple of 4096, at least one 32-row tile).
bool stream_eligible(const AffineOp* ops, uint32_t count) {
    for (uint32_t i = 0; i < count; ++i)
        if (ops[i].m != 1 || ops[i].group_size != 64 || ops[i].k % (4 * kUnitK) || ops[i].n < (uint32_t)kTR)
            return false;
    return count > 0;
}

template <bool SIGNED, bool BF, bool BIASED>
stark_qmm_status launch_stream_planes(const AffineOp* ops, uint32_t count, hipStream_t stream,
                                      const StreamPrologue* pro = nullptr) {
    std::vector<AffineOp> sorted(ops, ops + count);
    std::stable_sort(sorted.begin(), sorted.end(), [](const AffineOp& a, const AffineOp& b) { return a.k > b.k; });
    AffineBatch batch{};
    uint32_t tiles = 0;
    for (uint32_t i = 0; i < count; ++i) {
        batch.op[i] = sorted[i];
        // ops that read the same activations (q/k/v, gate/up) stage them once
        uint32_t x = i;
        for (uint32_t j = 0; j < i; ++j)
            if (sorted[j].x == sorted[i].x && sorted[j].k == sorted[i].k) {
                x = j;
                break;
            }
        batch.op[i].xid = x;
        tiles += (sorted[i].n + kTR - 1) / kTR;
    }
    batch.count = count;
    batch.total = tiles;
    if (tiles == 0) return STARK_QMM_OK;
    const uint32_t pk = pro ? pro->kind : (uint32_t)STARK_QMM_PROLOGUE_NONE;
    if (pro) {
        batch.pro_data = pro->data;
        batch.pro_eps = pro->eps;
    }
    int dev = 0, cus = 0;
    QMM_HIP_CHECK(hipGetDevice(&dev));
    QMM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    // Twelve waves per workgroup (one unit of a 12288-deep tile each) when the
    // launch has fewer tiles than CUs: its workgroups cannot fill the chip, so
    // each keeps three times the loads in flight instead.
    bool deep = tiles < (uint32_t)cus;
    for (uint32_t i = 0; i < count; ++i) deep = deep && sorted[i].k % (12 * kUnitK) == 0;
    // Otherwise, a launch with fewer 32-row tiles than CUs (a decode step's o
    // product) takes 16-row tiles: twice the workgroups, and each wave's unit
    // is 8 steps, its loads all in flight at once (the same arithmetic per
    // row, so the same bits): 6.7 -> 5.8 us for the Qwen3-8B o product. Not
    // with the RMS-norm prologue, whose every workgroup reads the whole row
    // (the q/k/v launch measured 8.3 -> 9.1 us). Launches of more tiles lose
    // with 16 rows (gate/up 15.3 -> 16.3 us, the headline layer set 5.07 ->
    // 4.47 TB/s).
    const bool half = !deep && tiles < (uint32_t)cus && pk != STARK_QMM_PROLOGUE_RMS_NORM;
    uint32_t tiles16 = 0;
    for (uint32_t i = 0; i < count; ++i) tiles16 += (sorted[i].n + 15) / 16;
    const auto pick = [&](auto wv, auto tr) {
        constexpr int W = decltype(wv)::value, T = decltype(tr)::value;
        return pk == STARK_QMM_PROLOGUE_RMS_NORM    ? qmv_stream<SIGNED, BF, BIASED, STARK_QMM_PROLOGUE_RMS_NORM, W, T>
               : pk == STARK_QMM_PROLOGUE_SILU_GATE ? qmv_stream<SIGNED, BF, BIASED, STARK_QMM_PROLOGUE_SILU_GATE, W, T>
                                                    : qmv_stream<SIGNED, BF, BIASED, STARK_QMM_PROLOGUE_NONE, W, T>;
    };
    using I4 = std::integral_constant<int, 4>;
    auto kern = deep ? pick(std::integral_constant<int, 12>{}, std::integral_constant<int, 32>{})
                     : half ? pick(I4{}, std::integral_constant<int, 16>{}) : pick(I4{}, std::integral_constant<int, 32>{});
    const int block = deep ? 12 * 64 : kWg;
    const uint32_t rows = half ? 16u : (uint32_t)kTR, ntiles = half ? tiles16 : tiles;
    // two workgroups (eight waves) per CU, or one of twelve waves; a multiple of the 8 XCDs
    const uint32_t per_launch = (uint32_t)std::max(8, cus * (deep ? 1 : 2) / 8 * 8);
    const uint32_t grid = std::min(std::min(persistent_grid(kern, block), per_launch), (ntiles + 7) / 8 * 8);
    if (grid == 0) return STARK_QMM_DEVICE_FAILURE;
    Schedule sched;
    const stark_qmm_status st = schedule_for(sorted.data(), count, grid, &sched, stream, rows);
    if (st != STARK_QMM_OK) return st;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(block), 0, stream, batch, sched);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

// One streaming launch per (plane type, correction) class of the batch.
template <bool SIGNED>
stark_qmm_status launch_stream(const AffineOp* ops, uint32_t count, hipStream_t stream,
                               const StreamPrologue* pro = nullptr) {
    std::vector<AffineOp> cls[2][2];
    for (uint32_t i = 0; i < count; ++i)
        cls[ops[i].w_dt == STARK_QMM_BF16][ops[i].corr_kind == STARK_QMM_CORRECTION_BIASES].push_back(ops[i]);
    for (int bf = 0; bf < 2; ++bf)
        for (int bi = 0; bi < 2; ++bi) {
            const std::vector<AffineOp>& v = cls[bf][bi];
            if (v.empty()) continue;
            const uint32_t n = (uint32_t)v.size();
            const stark_qmm_status st =
                bf ? (bi ? launch_stream_planes<SIGNED, true, true>(v.data(), n, stream, pro)
                         : launch_stream_planes<SIGNED, true, false>(v.data(), n, stream, pro))
                   : (bi ? launch_stream_planes<SIGNED, false, true>(v.data(), n, stream, pro)
                         : launch_stream_planes<SIGNED, false, false>(v.data(), n, stream, pro));
            if (st != STARK_QMM_OK) return st;
        }
    return STARK_QMM_OK;
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
    if (grid == 0) return STARK_QMM_DEVICE_FAILURE;
    Schedule sched;
    const stark_qmm_status st = schedule_for(sorted.data(), count, grid, &sched, stream);
    if (st != STARK_QMM_OK) return st;
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
        if constexpr (MP == 1 && MB == 1 && BITS == 4)
            if (stream_eligible(o, n)) return sg ? launch_stream<true>(o, n, st) : launch_stream<false>(o, n, st);
        if constexpr (MP >= 4 && BITS == 4)  // M = 3 .. 16
            if (small_m_eligible(o, n)) return launch_small_m(o, n, sg, st);
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

stark_qmm_status schedule_store(const std::vector<uint32_t>& key, uint32_t grid,
                                const std::function<std::vector<uint32_t>()>& build, mfma::Schedule* out,
                                hipStream_t stream) {
    return store_schedule(key, grid, build, out, stream);
}

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

stark_qmm_status launch_stream_prologue(const AffineOp* ops, uint32_t count, const StreamPrologue& pro,
                                        hipStream_t stream) {
    if (count == 0) return STARK_QMM_OK;
    if (count > (uint32_t)kMaxBatchOps || !stream_eligible(ops, count)) return STARK_QMM_UNSUPPORTED;
    std::vector<AffineOp> sg[2];
    for (uint32_t i = 0; i < count; ++i) {
        const AffineOp& o = ops[i];
        if (!mfma_eligible(o, 4) || o.x != ops[0].x || o.k != ops[0].k) return STARK_QMM_UNSUPPORTED;
        sg[(o.flags & FLAG_SIGNED) != 0].push_back(o);
    }
    for (int s = 0; s < 2; ++s) {
        if (sg[s].empty()) continue;
        const uint32_t n = (uint32_t)sg[s].size();
        const stark_qmm_status st = s ? launch_stream<true>(sg[s].data(), n, stream, &pro)
                                      : launch_stream<false>(sg[s].data(), n, stream, &pro);
        if (st != STARK_QMM_OK) return st;
    }
    return STARK_QMM_OK;
}

}  // namespace qmm
