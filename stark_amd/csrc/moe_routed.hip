// Routed experts (RoutedExperts::encode_scaled,
// crates/stark-engine/src/encodable_block/mlp/routed.rs:154-257) as one device
// pipeline with expert compaction:
//
//   1. route (moe.hip) and, when asked, adjust the routes (fused with 2. in one
//      workgroup for small token counts);
//   2. compaction (one workgroup): a counting sort of the routes by expert,
//      cut into slots of at most 16 routes of one expert, each slot filed in a
//      list by its route count class (1-2 or 3-16). The counting-sort
//      idea follows vendor/lily-core/src/kernels/metal/moe.metal:905-1036;
//   3. grouped up product per class: every slot streams its expert's
//      [value | gate] rows once for all its routes (matrix-core tile with the
//      8 value rows and the matching 8 gate rows of the expert), rounds both to
//      bf16 and applies the gated SiLU in the epilogue (gated_act_mul semantics);
//   4. grouped down product per class: bf16 result per route;
//   5. weighted accumulation over the ranks of each token in rank order, with
//      the reference's rounding switches (moe.rs:109-145).
//
// The numerics per (token, rank) are those of the reference's loop: products
// rounded to bf16 where LinearMatmul writes bf16, the gate on bf16 inputs, and
// accumulation in rank order. Compaction changes only which workgroup computes
// a route; each output value of the matrix-core tile depends on its own
// activation row alone.
#include <cmath>
#include <mutex>

#include "mfma_tile.h"

namespace qmm {

namespace {

using namespace mfma;

constexpr uint32_t kSlotRoutes = 16;  // routes per slot (record capacity)

// Routes per slot of a call: 2 up to 16 tokens (every slot then fits the
// 2-row tile of the small class, so each product is one launch; an expert
// with more routes streams its rows once per slot: measured against 4-route
// slots, 4 tokens 1.51 -> 1.61 TB/s, 16 tokens 1.95 -> 2.15), else 16.
__device__ __host__ inline uint32_t slot_routes(uint32_t rows) {
    return rows <= 16 ? 2u : kSlotRoutes;
}
// Two route-count classes, one launch each: small slots (1-2 routes) and
// large slots (3-16 routes); each launch takes the narrowest tile shape that
// fits the largest slot its class can hold in this call.
constexpr int kClasses = 2;

__device__ __host__ inline uint32_t count_class(uint32_t c) { return c <= 2 ? 0 : 1; }

// Workspace carve-up (byte offsets, 256-aligned).
struct RoutedLayout {
    uint64_t ids, weights, sorted, table, header, act, proj, total;
    uint32_t routes, max_slots;
};

// Slot record: expert, route count, then up to 16 route ids (128 bytes).
constexpr uint32_t kRecWords = 32;

RoutedLayout routed_layout(uint32_t rows, uint32_t model, uint32_t hidden, uint32_t experts, uint32_t active) {
    RoutedLayout L{};
    const uint64_t routes = (uint64_t)rows * active;
    L.routes = (uint32_t)routes;
    const uint32_t sr = slot_routes(rows);
    L.max_slots = (uint32_t)(std::min<uint64_t>(experts, routes) + (routes + sr - 1) / sr);
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) {
        const uint64_t at = off;
        off += (bytes + 255) / 256 * 256;
        return at;
    };
    L.ids = take(4 * routes);
    L.weights = take(4 * routes);
    L.sorted = take(4 * routes);
    L.table = take(4ull * kRecWords * kClasses * L.max_slots);
    L.header = take(4 * 8);
    L.act = take(2 * routes * hidden);
    L.proj = take(2 * routes * model);
    L.total = off;
    return L;
}

// ---- 2. compaction: one workgroup of 1024 threads, one thread per expert id.
// Routes are counting-sorted by expert, then every expert's routes are cut
// into slots of at most 16 and each slot is written as a self-contained record
// into the table of its route-count class. `ids` may be in LDS or global.
struct CompactLds {
    uint32_t cnt[1024], fill[1024], off[1024], wsum[16], ccount[kClasses];
};

__device__ __forceinline__ void compact_routes(const uint32_t* ids, uint32_t routes, uint32_t experts,
                                               uint32_t max_slots, uint32_t slot, uint32_t* sorted, uint32_t* table,
                                               uint32_t* header, CompactLds& s) {
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    s.cnt[t] = 0;
    s.fill[t] = 0;
    if (t < kClasses) s.ccount[t] = 0;
    __syncthreads();
    for (uint32_t r = t; r < routes; r += 1024) {
        uint32_t e = ids[r];
        e = e < experts ? e : 0;  // out-of-range ids read expert 0's rows (MoeGatherRows, moe.rs:87-107)
        atomicAdd(&s.cnt[e], 1u);
    }
    __syncthreads();
    // exclusive scan of the route counts over experts
    const uint32_t c = s.cnt[t];
    uint32_t ic = c;
    for (uint32_t d = 1; d < 64; d <<= 1) {
        const uint32_t u = __shfl_up(ic, d, 64);
        if (lane >= d) ic += u;
    }
    if (lane == 63) s.wsum[wave] = ic;
    __syncthreads();
    uint32_t pc = 0;
    for (uint32_t w = 0; w < wave; ++w) pc += s.wsum[w];
    s.off[t] = pc + ic - c;
    __syncthreads();
    for (uint32_t r = t; r < routes; r += 1024) {
        uint32_t e = ids[r];
        e = e < experts ? e : 0;
        sorted[s.off[e] + atomicAdd(&s.fill[e], 1u)] = r;
    }
    __syncthreads();  // sorted[] complete and visible to the workgroup
    for (uint32_t s0 = 0; s0 < c; s0 += slot) {
        const uint32_t n = min(slot, c - s0), cl = count_class(n);
        uint32_t* rec = table + ((size_t)cl * max_slots + atomicAdd(&s.ccount[cl], 1u)) * kRecWords;
        rec[0] = t;
        rec[1] = n;
        for (uint32_t i = 0; i < n; ++i) rec[2 + i] = sorted[s.off[t] + s0 + i];
    }
    __syncthreads();
    if (t < kClasses) header[t] = s.ccount[t];
}

__global__ __launch_bounds__(1024) void moe_compact(const uint32_t* ids, uint32_t routes, uint32_t experts,
                                                    uint32_t max_slots, uint32_t slot, uint32_t* sorted,
                                                    uint32_t* table, uint32_t* header) {
    __shared__ CompactLds s;
    compact_routes(ids, routes, experts, max_slots, slot, sorted, table, header, s);
}

// ---- 1+2 fused for up to kFusedRoutes routes: route, adjust and compaction in
// one workgroup, every phase spread over all 1024 threads (a single wave64
// retires about one VALU instruction per 4 clocks, so no phase may leave the
// work to a few waves):
//   a. the logits of all rows into LDS (bf16-rounded if asked) as 64-bit keys
//      (order-preserving value bits over the inverted expert id, -0 taken as
//      +0), a per-row finite flag;
//   b. per row (one wave each): max and den = sum exp(x - max) (a wave tree
//      sum, the device expf);
//   c. ranks: expert e of a row lands at rank
//      #{e' : x[e'] > x[e] or (x[e'] == x[e] and e' < e)}, the order of the
//      reference's repeated argmax in which a strictly greater value wins and
//      ties go to the lower id (moe.rs:52-70), i.e. #{e' : key(e') > key(e)}.
//      Eight consecutive lanes count one expert against interleaved eighths
//      of the row (adjacent keys: no LDS bank conflicts) and add by shuffles;
//   d. per row (one wave, lane = rank): score exp(x - max) / den, summed in
//      rank order and renormalised (moe.rs:71-84); then the gains and the
//      stable id sort of MoeAdjustRoutes (moe.rs:147-184), the sort as a rank
//      count over the row's routes; ids and weights to the workspace and LDS;
//   e. compaction.
// Dynamic LDS: rows * E keys. The rank count costs rows * E^2 compares in one
// CU, so larger cases take the multi-workgroup route kernel.
constexpr uint32_t kFusedRoutes = 2048;
constexpr uint32_t kFusedKeys = 4096;
constexpr uint32_t kFusedRows = 512;
constexpr uint64_t kFusedCompares = 65536;

__device__ __forceinline__ uint64_t route_key(float x, uint32_t e) {
    const uint32_t u = __float_as_uint(x + 0.0f);  // -0 -> +0: equal values tie
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (0xffffffffu - e);
}

__device__ __forceinline__ float route_key_value(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}

__device__ __forceinline__ float route_round_bf16(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

__global__ __launch_bounds__(1024) void moe_route_compact(const float* logits, uint32_t rows, uint32_t experts,
                                                          uint32_t active, uint32_t round_weights,
                                                          uint32_t round_logits, const float* gains,
                                                          uint32_t adjust, uint32_t sort_ids, uint32_t max_slots,
                                                          uint32_t* ids, float* weights, uint32_t* sorted,
                                                          uint32_t* table, uint32_t* header) {
    __shared__ CompactLds s;
    __shared__ uint32_t rid[kFusedRoutes];  // ids, then (after d) the compaction input
    __shared__ float rmax[kFusedRows], rden[kFusedRows];
    __shared__ uint32_t rbad[kFusedRows];
    extern __shared__ uint64_t keys[];
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t E = experts, RE = rows * experts;
    // a.
    for (uint32_t r = tid; r < rows; r += 1024) rbad[r] = 0;
    __syncthreads();
    for (uint32_t i = tid; i < RE; i += 1024) {
        float x = logits[i];
        if (round_logits) x = route_round_bf16(x);
        keys[i] = route_key(x, i % E);
        if (!__builtin_isfinite(x)) rbad[i / E] = 1;
    }
    __syncthreads();
    // b.
    for (uint32_t row = wave; row < rows; row += 16) {
        const uint64_t* kr = keys + (size_t)row * E;
        float mx = -INFINITY;
        for (uint32_t e = lane; e < E; e += 64) mx = fmaxf(mx, route_key_value(kr[e]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float den = 0.0f;
        for (uint32_t e = lane; e < E; e += 64) den += expf(route_key_value(kr[e]) - mx);
        den = wave_sum(den);
        if (lane == 0) {
            rmax[row] = mx;
            rden[row] = den;
        }
    }
    // c.
    for (uint32_t it = tid; it < RE * 8; it += 1024) {  // RE * 8 is a multiple of 8: lane groups stay whole
        const uint32_t q = it & 7, re = it >> 3, row = re / E, e = re % E;
        const uint64_t* kr = keys + (size_t)row * E;
        const uint64_t k = kr[e];
        uint32_t rank = 0;
#pragma unroll 4
        for (uint32_t f = q; f < E; f += 8) rank += kr[f] > k ? 1u : 0u;  // lanes of a group: adjacent keys
        rank += __shfl_xor(rank, 1, 64);
        rank += __shfl_xor(rank, 2, 64);
        rank += __shfl_xor(rank, 4, 64);
        if (q == 0 && rank < active) rid[row * active + rank] = e;
    }
    __syncthreads();
    // d.
    for (uint32_t row = wave; row < rows; row += 16) {
        const bool valid = rbad[row] == 0;
        const uint32_t my_id = lane < active ? rid[row * active + lane] : 0u;
        // a row with a non-finite logit may leave ranks unfilled: its ids become 0
        const float my_v = lane < active && my_id < E ? route_key_value(keys[(size_t)row * E + my_id]) : 0.0f;
        const float score = lane < active ? expf(my_v - rmax[row]) / rden[row] : 0.0f;
        float sum = 0.0f;
        for (uint32_t r = 0; r < active; ++r) sum += __shfl(score, r, 64);
        float w = score / sum;
        if (round_weights) w = route_round_bf16(w);
        const uint32_t id = valid ? my_id : 0u;
        w = valid ? w : __builtin_nanf("");
        uint32_t pos = lane;
        if (adjust) {
            w = id < experts ? w * (gains ? gains[id] : 1.0f) : __builtin_nanf("");
            if (sort_ids) {
                pos = 0;
                for (uint32_t r = 0; r < active; ++r) {
                    const uint32_t o = __shfl(id, r, 64);
                    pos += (o < id || (o == id && r < lane)) ? 1u : 0u;
                }
            }
        }
        // every lane has read its rank's id before any lane rewrites the row
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane < active) {
            ids[(size_t)row * active + pos] = id;
            weights[(size_t)row * active + pos] = w;
            rid[row * active + pos] = id;
        }
    }
    __syncthreads();
    // e.
    compact_routes(rid, rows * active, experts, max_slots, slot_routes(rows), sorted, table, header, s);
}

// Launch record of a grouped product, read through the kernarg segment.
struct GroupedLaunch {
    AffineOp op;             // the bank: codes, planes, activation base, k, group, strides
    const uint32_t* table;   // this class's slot records
    const uint32_t* header;  // per-class slot counts
    uint16_t* out;           // up: act [routes][hidden]; down: proj [routes][model]
    uint32_t cls, tiles, active, hidden, model;
};

// Work items (slot, tile) in XCD-aware order. Workgroups are dealt to the 8
// XCDs round-robin (block b on XCD b % 8; a persistent loop with a grid that
// is a multiple of 8 keeps item i on XCD i % 8), and each XCD has its own L2.
// In the group-output plane layout a 128-byte plane line holds one group of
// 64 consecutive bank rows, i.e. TPL tiles (8-row up tiles: 8; 16-row down
// tiles: 4): item i = x + 8 k takes line group L = x + 8 (k / TPL) and its
// tile k % TPL, so the tiles that share a plane line run on one XCD and the
// line is fetched from HBM once. Items past the last line group (padding up
// to padded_items) return false.
__device__ __host__ inline uint32_t line_groups(uint32_t slots, uint32_t tiles, uint32_t tpl) {
    return slots * (tiles / tpl);
}
__device__ __host__ inline uint32_t padded_items(uint32_t slots, uint32_t tiles, uint32_t tpl) {
    return 8 * tpl * ((line_groups(slots, tiles, tpl) + 7) / 8);
}
__device__ __forceinline__ bool xcd_item(uint32_t i, uint32_t slots, uint32_t tiles, uint32_t tpl, uint32_t& slot,
                                         uint32_t& t) {
    const uint32_t lg = tiles / tpl, k = i >> 3;
    const uint32_t L = (i & 7) + 8 * (k / tpl);
    if (L >= slots * lg) return false;
    slot = L / lg;
    t = tpl * (L % lg) + k % tpl;
    return true;
}
// tiles per plane line for a tile height (1 when the tiles do not divide into lines)
__device__ __host__ inline uint32_t line_tiles(uint32_t tiles, uint32_t rows) {
    const uint32_t tpl = 64 / rows;
    return tiles % tpl == 0 ? tpl : 1u;
}

// silu(gate) * value in bf16 steps (gated_act_mul; SiLU as
// src/backends/common/gpu_types/activation_type.rs:35-46)
__device__ __forceinline__ uint16_t gated_silu(float value_f, float gate_f) {
    const float v = bf16_bits_to_f32(f32_to_bf16_bits(value_f));
    const float x = bf16_bits_to_f32(f32_to_bf16_bits(gate_f));
    const float y = x / (1.0f + expf(-1.0f * x));
    const float a = bf16_bits_to_f32(f32_to_bf16_bits(y));
    return f32_to_bf16_bits(v * a);
}

// ---- 3. grouped up product + gated SiLU. Work item = (slot, tile of 8 value rows).
template <int MP, int MB, int GS, bool SIGNED, int P1>
__global__ __launch_bounds__(kWg) void moe_up_mfma(GroupedLaunch launch) {
    (void)launch;
    __shared__ MfmaLds<MP, MB, GS, 4, P1> lds;
    const GroupedLaunch* L = (const GroupedLaunch*)__builtin_amdgcn_kernarg_segment_ptr();
    const uint32_t slots = L->header[L->cls], tpl = line_tiles(L->tiles, 8);
    const uint32_t items = padded_items(slots, L->tiles, tpl);
    const uint32_t H = L->hidden, A = L->active, model = L->model;
    for (uint32_t item = blockIdx.x; item < items; item += gridDim.x) {
        uint32_t sl, t;
        if (!xcd_item(item, slots, L->tiles, tpl, sl, t)) continue;
        const uint32_t* rec = L->table + (size_t)sl * kRecWords;
        const uint32_t e = rec[0], cnt = rec[1];
        const uint32_t nA = e * 2 * H + 8 * t, nB = nA + H;
        const uint32_t* routes = rec + 2;
        mfma_tile<MP, MB, GS, 4, SIGNED, P1>(
            L->op, plane_flags(L->op), nA, nB, cnt, [&](uint32_t m) { return (size_t)(routes[m] / A) * model; }, lds);
        for (uint32_t q = threadIdx.x; q < (uint32_t)MP * MB * 8; q += kWg) {
            const uint32_t m = q / 8, i = q % 8;
            if (m >= cnt) continue;
            const float v = (lds.red[0][m][i] + lds.red[1][m][i]) + (lds.red[2][m][i] + lds.red[3][m][i]);
            const float g = (lds.red[0][m][8 + i] + lds.red[1][m][8 + i]) +
                            (lds.red[2][m][8 + i] + lds.red[3][m][8 + i]);
            L->out[(size_t)routes[m] * H + 8 * t + i] = gated_silu(v, g);
        }
        __syncthreads();  // lds.red is rewritten by the next item
    }
}

// ---- 4. grouped down product. Work item = (slot, tile of 16 output rows).
template <int MP, int MB, int GS, bool SIGNED, int P1>
__global__ __launch_bounds__(kWg) void moe_down_mfma(GroupedLaunch launch) {
    (void)launch;
    __shared__ MfmaLds<MP, MB, GS, 4, P1> lds;
    const GroupedLaunch* L = (const GroupedLaunch*)__builtin_amdgcn_kernarg_segment_ptr();
    const uint32_t slots = L->header[L->cls], tpl = line_tiles(L->tiles, 16);
    const uint32_t items = padded_items(slots, L->tiles, tpl);
    const uint32_t H = L->hidden, model = L->model;
    for (uint32_t item = blockIdx.x; item < items; item += gridDim.x) {
        uint32_t sl, t;
        if (!xcd_item(item, slots, L->tiles, tpl, sl, t)) continue;
        const uint32_t* rec = L->table + (size_t)sl * kRecWords;
        const uint32_t e = rec[0], cnt = rec[1];
        const uint32_t nA = e * model + 16 * t;
        const uint32_t* routes = rec + 2;
        mfma_tile<MP, MB, GS, 4, SIGNED, P1>(
            L->op, plane_flags(L->op), nA, nA + 8, cnt, [&](uint32_t m) { return (size_t)routes[m] * H; }, lds);
        for (uint32_t q = threadIdx.x; q < (uint32_t)MP * MB * kRows; q += kWg) {
            const uint32_t m = q / kRows, r = q % kRows;
            if (m >= cnt) continue;
            const float v = (lds.red[0][m][r] + lds.red[1][m][r]) + (lds.red[2][m][r] + lds.red[3][m][r]);
            L->out[(size_t)routes[m] * model + 16 * t + r] = f32_to_bf16_bits(v);
        }
        __syncthreads();
    }
}

// ---- 1+2+3 fused for one token (rows == 1, up to kOneTokenExperts experts):
// every workgroup routes the token itself -- phases a-d of moe_route_compact
// restricted to one row, in the same operations, so the ids and weights are
// the same bits -- files route r as its own one-route slot r (one token gives
// an expert at most one route, and each route's product depends on its own
// activation row alone, so a slot per route computes what the counting sort's
// slots compute), and then computes its (slot, tile) item of the up product.
// Workgroup 0 also writes the ids, the weights and the class-0 slot table that
// the down product and the rank accumulation read. This takes the separate
// route launch off the one-token chain.
constexpr uint32_t kOneTokenExperts = 256;
constexpr uint64_t kOneTokenWork = 1ull << 20;  // A * H * E bound of the fused path (top-8, H 768, 128 experts: 0.75)

struct RouteOneArgs {
    const float* logits;
    const float* gains;
    uint32_t experts, active, round_weights, round_logits, adjust, sort_ids;
    uint32_t* ids;
    float* weights;
    uint32_t* table;
    uint32_t* header;
};

template <int GS, bool SIGNED, int P1>
__global__ __launch_bounds__(kWg) void moe_route_up_one(GroupedLaunch launch, RouteOneArgs ra) {
    (void)launch;
    __shared__ MfmaLds<1, 1, GS, 4, P1> lds;
    __shared__ uint64_t keys[kOneTokenExperts];
    __shared__ uint32_t rid[32], sid[32];
    __shared__ float rmax, rden;
    __shared__ uint32_t rbad;
    const GroupedLaunch* L = (const GroupedLaunch*)__builtin_amdgcn_kernarg_segment_ptr();
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t E = ra.experts, A = ra.active;
    // a. keys (bf16-rounded logits if asked) and the finite flag
    if (tid == 0) rbad = 0;
    if (tid < 32) rid[tid] = 0;
    __syncthreads();
    for (uint32_t e = tid; e < E; e += kWg) {
        float x = ra.logits[e];
        if (ra.round_logits) x = route_round_bf16(x);
        keys[e] = route_key(x, e);
        if (!__builtin_isfinite(x)) rbad = 1;
    }
    __syncthreads();
    // b. max and den (wave 0, as one row of moe_route_compact)
    if (wave == 0) {
        float mx = -INFINITY;
        for (uint32_t e = lane; e < E; e += 64) mx = fmaxf(mx, route_key_value(keys[e]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
        float den = 0.0f;
        for (uint32_t e = lane; e < E; e += 64) den += expf(route_key_value(keys[e]) - mx);
        den = wave_sum(den);
        if (lane == 0) {
            rmax = mx;
            rden = den;
        }
    }
    // c. ranks: #{e' : key(e') > key(e)}, eight consecutive lanes per expert
    // over interleaved eighths of the keys (as moe_route_compact)
    for (uint32_t it = tid; it < E * 8; it += kWg) {  // lane groups of 8 stay whole
        const uint32_t qq = it & 7, e = it >> 3;
        const uint64_t k = keys[e];
        uint32_t rank = 0;
#pragma unroll 4
        for (uint32_t f = qq; f < E; f += 8) rank += keys[f] > k ? 1u : 0u;
        rank += __shfl_xor(rank, 1, 64);
        rank += __shfl_xor(rank, 2, 64);
        rank += __shfl_xor(rank, 4, 64);
        if (qq == 0 && rank < A) rid[rank] = e;
    }
    __syncthreads();
    // d. weights in rank order, renormalised; gains and the stable id sort
    if (wave == 0) {
        const bool valid = rbad == 0;
        const uint32_t my_id = lane < A ? rid[lane] : 0u;
        const float my_v = lane < A && my_id < E ? route_key_value(keys[my_id]) : 0.0f;
        const float score = lane < A ? expf(my_v - rmax) / rden : 0.0f;
        float sum = 0.0f;
        for (uint32_t r = 0; r < A; ++r) sum += __shfl(score, r, 64);
        float w = score / sum;
        if (ra.round_weights) w = route_round_bf16(w);
        const uint32_t id = valid ? my_id : 0u;
        w = valid ? w : __builtin_nanf("");
        uint32_t pos = lane;
        if (ra.adjust) {
            w = id < E ? w * (ra.gains ? ra.gains[id] : 1.0f) : __builtin_nanf("");
            if (ra.sort_ids) {
                pos = 0;
                for (uint32_t r = 0; r < A; ++r) {
                    const uint32_t o = __shfl(id, r, 64);
                    pos += (o < id || (o == id && r < lane)) ? 1u : 0u;
                }
            }
        }
        if (lane < A) {
            sid[pos] = id;
            if (blockIdx.x == 0) {
                ra.ids[pos] = id;
                ra.weights[pos] = w;
                uint32_t* rec = ra.table + (size_t)pos * kRecWords;
                rec[0] = id < E ? id : 0u;  // out-of-range ids read expert 0's rows (moe.rs:87-107)
                rec[1] = 1;
                rec[2] = pos;
            }
        }
        if (blockIdx.x == 0 && lane < kClasses) ra.header[lane] = lane == 0 ? A : 0u;
    }
    __syncthreads();
    // the item: route (slot) and tile of 8 value rows
    const uint32_t H = L->hidden, model = L->model;
    uint32_t slot, t;
    if (!xcd_item(blockIdx.x, A, L->tiles, line_tiles(L->tiles, 8), slot, t)) return;  // padding block
    const uint32_t e = sid[slot] < E ? sid[slot] : 0u;
    const uint32_t nA = e * 2 * H + 8 * t, nB = nA + H;
    mfma_tile<1, 1, GS, 4, SIGNED, P1>(L->op, plane_flags(L->op), nA, nB, 1, [&](uint32_t) { return (size_t)0; }, lds);
    (void)model;
    if (threadIdx.x < 8) {
        const uint32_t i = threadIdx.x;
        const float v = (lds.red[0][0][i] + lds.red[1][0][i]) + (lds.red[2][0][i] + lds.red[3][0][i]);
        const float g = (lds.red[0][0][8 + i] + lds.red[1][0][8 + i]) + (lds.red[2][0][8 + i] + lds.red[3][0][8 + i]);
        L->out[(size_t)slot * H + 8 * t + i] = gated_silu(v, g);
    }
}

// ---- 5. accumulation over ranks in order (moe.rs:109-145 applied rank 0..k-1).
__global__ void moe_accumulate_ranks(const uint16_t* proj, const float* weights, uint16_t* output, uint32_t model,
                                     uint32_t active, uint32_t round_product, uint32_t round_accumulator) {
    const uint32_t row = blockIdx.y, p = blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= model) return;
    float acc = 0.0f;
    // the operands of 8 ranks are loaded together, then added in rank order
    for (uint32_t r0 = 0; r0 < active; r0 += 8) {
        float pv[8], wv[8];
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t route = row * active + min(r0 + j, active - 1);
            pv[j] = bf16_bits_to_f32(proj[(size_t)route * model + p]);
            wv[j] = weights[route];
        }
#pragma unroll
        for (uint32_t j = 0; j < 8; ++j) {
            const uint32_t rank = r0 + j;
            if (rank >= active) break;
            float product = pv[j] * wv[j];
            if (round_product) product = bf16_bits_to_f32(f32_to_bf16_bits(product));
            float value = (rank == 0 ? 0.0f : acc) + product;
            if (round_accumulator) value = bf16_bits_to_f32(f32_to_bf16_bits(value));
            acc = value;
        }
    }
    output[(size_t)row * model + p] = f32_to_bf16_bits(acc);
}

// ---- 4+5 fused for one token: the down products of the token's routes and
// their accumulation in rank order, one workgroup per 16 output rows and one
// wave per route (rank). The wave stages its route's activation row in LDS
// (loaded before the expert id is known); lane (row r = lane / 4, quarter
// q = lane % 4) loads its quarter of the route's expert row (NL 16-byte
// pieces, whole groups), sums x*q and x per group on v_dot2 (products
// exact) and adds s * sum(x q) + bias_term * sum(x); the quarters meet by two
// shuffles in a fixed order, the route's product is rounded to bf16 as the
// reference's down product writes it, and 16 threads accumulate the routes in
// rank order with the reference's rounding switches (moe.rs:109-145), as
// moe_accumulate_ranks does. This takes the down launch's 8 x (model / 16)
// one-route items and the accumulation launch off the one-token chain.
struct DownAccArgs {
    const uint8_t* codes;    // down bank [E * model, H / 2]
    const uint16_t* scales;  // bf16 planes
    const uint16_t* corr;    // bf16 bias plane, or null (symmetric: bias_term = -8 s)
    uint32_t os, gs;         // plane strides (elements)
    const uint16_t* act;     // [A, H] bf16, rank r at r * H
    const uint32_t* ids;     // [A] expert of each rank
    const float* weights;    // [A]
    uint16_t* out;           // [model] bf16
    uint32_t model, hidden, experts, active, signed_codes, round_product, round_accumulator;
};

template <int NL, int GS>
__global__ __launch_bounds__(512) void moe_down_acc_one(DownAccArgs a) {
    constexpr int KQ = NL * 32;   // k values of a lane's quarter of the row (H / 4)
    constexpr int GPL = KQ / GS;  // whole groups per lane
    constexpr int XV = KQ / 2;    // 16-byte activation vectors of a row (H / 8)
    static_assert(KQ % GS == 0, "a lane's quarter holds whole groups");
    __shared__ float proj[8][16];
    __shared__ float rw[8];
    __shared__ u32x4 xs[8][XV];  // each wave's activation row
    const uint32_t tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    uint32_t one, tile;
    if (!xcd_item(blockIdx.x, 1, a.model / 16, line_tiles(a.model / 16, 16), one, tile)) return;  // padding block
    const uint32_t H = a.hidden, n0 = tile * 16, r = lane >> 2, q = lane & 3;
    // first the loads that need no route: the wave's activation row and the
    // route weights (the codes' addresses wait for the expert id)
    const bool live = w < a.active;
    const u32x4* xg = (const u32x4*)(a.act + (size_t)min(w, a.active - 1) * H);
    u32x4 x0 = live && lane < (uint32_t)XV ? xg[lane] : u32x4{0, 0, 0, 0};
    u32x4 x1 = live && lane + 64 < (uint32_t)XV ? xg[lane + 64] : u32x4{0, 0, 0, 0};
    const float wt = tid < a.active ? a.weights[tid] : 0.0f;
    if (live) {
        uint32_t e = a.ids[w];
        e = e < a.experts ? e : 0u;  // out-of-range ids read expert 0's rows (moe.rs:87-107)
        const size_t row = (size_t)e * a.model + n0 + r;
        const u32x4* cp = (const u32x4*)(a.codes + row * (H / 2) + q * (KQ / 2));
        u32x4 c[NL];
#pragma unroll
        for (int j = 0; j < NL; ++j) c[j] = cp[j];
        float sc[GPL], bi[GPL];
#pragma unroll
        for (int g = 0; g < GPL; ++g) {
            const size_t idx = row * a.os + (size_t)(q * GPL + g) * a.gs;
            sc[g] = bf16_bits_to_f32(a.scales[idx]);
            bi[g] = a.corr ? bf16_bits_to_f32(a.corr[idx]) : -8.0f * sc[g];
        }
        if (lane < (uint32_t)XV) xs[w][lane] = x0;
        if (lane + 64 < (uint32_t)XV) xs[w][lane + 64] = x1;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        const u32x4* xw = xs[w] + q * (KQ / 8);
        const uint32_t flip = a.signed_codes ? 0x88888888u : 0u;
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < GPL; ++g) {
            float sq = 0.0f, sa = 0.0f;
#pragma unroll
            for (int j = g * (GS / 32); j < (g + 1) * (GS / 32); ++j)  // 16-byte pieces of the group
#pragma unroll
                for (int t = 0; t < 4; ++t) {  // 8 codes, k = 32 j + 8 t + i (low nibble first)
                    const uint32_t cw = c[j][t] ^ flip;
                    const uint32_t ev = cw & 0x0F0F0F0Fu, od = (cw >> 4) & 0x0F0F0F0Fu;
                    const u32x4 xv = xw[4 * j + t];  // bf16 pairs (x0, x1) (x2, x3) ..
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float qe = (float)((ev >> (8 * b)) & 255u), qo = (float)((od >> (8 * b)) & 255u);
                        const uint32_t qp = perm(__float_as_uint(qo), __float_as_uint(qe), 0x07060302u);
                        sq = dot2_bf16(xv[b], qp, sq);
                        sa = dot2_bf16(xv[b], 0x3F803F80u, sa);
                    }
                }
            acc = fmaf(sc[g], sq, fmaf(bi[g], sa, acc));
        }
        acc += __shfl_xor(acc, 1, 64);
        acc += __shfl_xor(acc, 2, 64);
        if (q == 0) proj[w][r] = bf16_bits_to_f32(f32_to_bf16_bits(acc));
    }
    if (tid < a.active) rw[tid] = wt;
    __syncthreads();
    if (tid < 16 && n0 + tid < a.model) {
        float acc = 0.0f;
        for (uint32_t rank = 0; rank < a.active; ++rank) {
            float product = proj[rank][tid] * rw[rank];
            if (a.round_product) product = bf16_bits_to_f32(f32_to_bf16_bits(product));
            float value = (rank == 0 ? 0.0f : acc) + product;
            if (a.round_accumulator) value = bf16_bits_to_f32(f32_to_bf16_bits(value));
            acc = value;
        }
        a.out[n0 + tid] = f32_to_bf16_bits(acc);
    }
}

// The fused one-token down kernel for (H, group size), or null when the
// shape is outside it (H / 128 pieces per lane in {2, 4, 6, 8}, whole
// groups per lane).
void* pick_down_acc_one(uint32_t H, uint32_t gs) {
#define QMM_DA(NL)                                                             \
    case NL:                                                                   \
        if (gs == 32) return (void*)&moe_down_acc_one<NL, 32>;                 \
        if (gs == 64 && (NL * 32) % 64 == 0) return (void*)&moe_down_acc_one<NL, (NL * 32) % 64 == 0 ? 64 : 32>; \
        if (gs == 128 && (NL * 32) % 128 == 0) return (void*)&moe_down_acc_one<NL, (NL * 32) % 128 == 0 ? 128 : 32>; \
        return nullptr;
    if (H % 128) return nullptr;
    switch (H / 128) {
        QMM_DA(2)
        QMM_DA(4)
        QMM_DA(6)
        QMM_DA(8)
    default: return nullptr;
    }
#undef QMM_DA
}

#define QMM_GROUPED_KERNEL(NAME)                                  \
    template <int MP, int MB, int GS, bool SG, int P1>            \
    struct NAME##_k {                                             \
        static void* fn() { return (void*)&NAME<MP, MB, GS, SG, P1>; } \
    };
QMM_GROUPED_KERNEL(moe_up_mfma)
QMM_GROUPED_KERNEL(moe_down_mfma)
#undef QMM_GROUPED_KERNEL

// Kernel of one (class tile shape, group size, signedness); group size 32 needs
// 4 slots per activation row, i.e. MP <= 4 (checked by check_bank).
template <template <int, int, int, bool, int> class K, int MP, int MB, int P1>
void* pick(uint32_t gs, bool sg) {
    if (gs == 32) {
        if constexpr (16 / MP >= 4) return sg ? K<MP, MB, 32, true, P1>::fn() : K<MP, MB, 32, false, P1>::fn();
        return nullptr;
    }
    if (gs == 64) return sg ? K<MP, MB, 64, true, P1>::fn() : K<MP, MB, 64, false, P1>::fn();
    return sg ? K<MP, MB, 128, true, P1>::fn() : K<MP, MB, 128, false, P1>::fn();
}

// Kernel for a route-count class, given the largest route count of any slot
// in this call; the one- and two-route shapes take a pass length matched to K
// so that all four waves of a tile get work.
template <template <int, int, int, bool, int> class K>
void* pick_class(int cls, uint32_t max_count, uint32_t gs, bool sg, uint32_t k) {
    const bool short_k = k <= 1024;
    if (cls == 0) {
        if (max_count <= 1) return short_k ? pick<K, 1, 1, 1024>(gs, sg) : pick<K, 1, 1, 2048>(gs, sg);
        return short_k ? pick<K, 2, 1, 1024>(gs, sg) : pick<K, 2, 1, 2048>(gs, sg);
    }
    if (max_count <= 4) return pick<K, 4, 1, 2048>(gs, sg);
    if (max_count <= 8) return pick<K, 8, 1, 2048>(gs, sg);
    return pick<K, 8, 2, 2048>(gs, sg);
}

// The one-token fused kernel of a group size and signedness (the one-route
// tile shape, pass length as pick_class takes for class 0).
void* pick_route_up_one(uint32_t gs, bool sg, uint32_t k) {
#define QMM_RU(G, S, P) (void*)&moe_route_up_one<G, S, P>
    const bool short_k = k <= 1024;
    if (gs == 32) return short_k ? (sg ? QMM_RU(32, true, 1024) : QMM_RU(32, false, 1024))
                                 : (sg ? QMM_RU(32, true, 2048) : QMM_RU(32, false, 2048));
    if (gs == 64) return short_k ? (sg ? QMM_RU(64, true, 1024) : QMM_RU(64, false, 1024))
                                 : (sg ? QMM_RU(64, true, 2048) : QMM_RU(64, false, 2048));
    return short_k ? (sg ? QMM_RU(128, true, 1024) : QMM_RU(128, false, 1024))
                   : (sg ? QMM_RU(128, true, 2048) : QMM_RU(128, false, 2048));
#undef QMM_RU
}

// Largest number of slots a class can hold: an expert receives at most one
// route per token, so it has at most one small slot (the remainder after full
// slots of 16), and a large slot holds at least 3 routes.
uint32_t class_slot_bound(int cls, uint32_t routes, uint32_t experts, uint32_t max_slots) {
    if (cls == 0) return std::min<uint32_t>(std::min<uint32_t>(max_slots, routes), experts);
    return std::min<uint32_t>(max_slots, routes / 3);
}

AffineOp bank_op(const stark_qmm_b& b, uint32_t rows, uint32_t k, const void* x) {
    AffineOp o{};
    o.codes = (const uint8_t*)b.codes;
    o.scales = b.scales;
    o.corr = b.correction_data;
    o.x = x;
    o.n = rows;
    o.k = k;
    o.m = 1;
    if (b.params.layout == STARK_QMM_LAYOUT_OUTPUT_GROUP) {
        o.os = b.params.group_count;
        o.gs = 1;
    } else {
        o.os = 1;
        o.gs = (b.params.row_count + 3u) / 4u * 4u;
    }
    o.group_size = b.group_size;
    o.corr_kind = b.correction;
    o.w_dt = STARK_QMM_BF16;
    o.x_dt = STARK_QMM_BF16;
    o.d_dt = STARK_QMM_BF16;
    o.flags = b.signed_codes ? FLAG_SIGNED : 0u;
    o.ab_scale = 1.0f;
    return o;
}

// Bank accepted by the grouped matrix-core kernels.
stark_qmm_status check_bank(const stark_qmm_b& b, uint64_t rows, uint32_t k, uint32_t max_count) {
    if (!b.codes || !b.scales) return STARK_QMM_INVALID_ARGUMENT;
    if (b.mode != STARK_QMM_MODE_U4) return STARK_QMM_UNSUPPORTED;
    if (b.group_size != 32 && b.group_size != 64 && b.group_size != 128) return STARK_QMM_UNSUPPORTED_GROUP_SIZE;
    if (b.correction == STARK_QMM_CORRECTION_ZERO_POINTS) return STARK_QMM_UNSUPPORTED;
    if (b.correction == STARK_QMM_CORRECTION_BIASES && !b.correction_data) return STARK_QMM_INVALID_ARGUMENT;
    if (b.params.materialize_affine_input_sum) return STARK_QMM_UNSUPPORTED;
    if (b.params.row_count != rows || (uint64_t)b.params.group_count * b.group_size != k)
        return STARK_QMM_UNSUPPORTED_LAYOUT;
    if (rows * k / 2 > b.codes_size) return STARK_QMM_UNSUPPORTED_LAYOUT;
    // the widest class in use must fit a step's groups into its slots (S = 16 / MP)
    const uint32_t mp = max_count <= 1 ? 1 : max_count <= 2 ? 2 : max_count <= 4 ? 4 : 8;
    if (16 / mp < 128 / b.group_size) return STARK_QMM_UNSUPPORTED_GROUP_SIZE;
    if (((uintptr_t)b.codes | (uintptr_t)b.scales | (uintptr_t)b.correction_data) & 15) return STARK_QMM_UNSUPPORTED;
    // group-output planes: the 16-byte metadata loads need 8-row aligned plane rows
    if (b.params.layout == STARK_QMM_LAYOUT_GROUP_OUTPUT && ((rows + 3) / 4 * 4) % 8)
        return STARK_QMM_UNSUPPORTED_LAYOUT;
    return STARK_QMM_OK;
}

}  // namespace

}  // namespace qmm

using namespace qmm;

extern "C" {

uint64_t stark_qmm_routed_experts_workspace_size(uint32_t rows, uint32_t model, uint32_t hidden, uint32_t experts,
                                                 uint32_t active) {
    return routed_layout(rows, model, hidden, experts, active).total;
}

}  // extern "C"

namespace {

// The routed pipeline on a workspace of ws_size bytes at ws (device memory).
stark_qmm_status routed_run(const stark_qmm_routed_args* a, uint8_t* ws, uint64_t ws_size, void* stream_ptr) {
    if (!a || a->struct_size != sizeof(stark_qmm_routed_args)) return STARK_QMM_ABI_MISMATCH;
    const uint32_t R = a->rows, model = a->model, H = a->hidden, E = a->experts, A = a->active;
    // geometry accepted by RoutedExperts::new / encode_scaled (routed.rs:62-73, 162-170)
    if (R == 0 || R > 1024 || E == 0 || E > 1024 || A == 0 || A > 32 || A > E || model == 0 || model > 16384 ||
        H == 0 || H > 131072)
        return STARK_QMM_INVALID_ARGUMENT;
    if (!a->input || !a->router_logits || !a->output || !ws) return STARK_QMM_INVALID_ARGUMENT;
    if (model % 64 || H % 64) return STARK_QMM_UNSUPPORTED_LAYOUT;  // K of both products, 16-row tiles
    if (((uintptr_t)a->input | (uintptr_t)ws) & 15) return STARK_QMM_UNSUPPORTED;
    const RoutedLayout Lw = routed_layout(R, model, H, E, A);
    if (ws_size < Lw.total) return STARK_QMM_WORKSPACE_TOO_SMALL;
    const uint32_t max_count = std::min<uint32_t>(R, slot_routes(R));
    stark_qmm_status st = check_bank(a->up, (uint64_t)E * 2 * H, model, max_count);
    if (st != STARK_QMM_OK) return st;
    st = check_bank(a->down, (uint64_t)E * model, H, max_count);
    if (st != STARK_QMM_OK) return st;
    if (a->up.signed_codes != a->down.signed_codes || a->up.correction != a->down.correction)
        return STARK_QMM_UNSUPPORTED;

    hipStream_t stream = (hipStream_t)stream_ptr;
    uint32_t* ids = (uint32_t*)(ws + Lw.ids);
    float* weights = (float*)(ws + Lw.weights);
    uint32_t* sorted = (uint32_t*)(ws + Lw.sorted);
    uint32_t* table = (uint32_t*)(ws + Lw.table);
    uint32_t* header = (uint32_t*)(ws + Lw.header);
    uint16_t* act = (uint16_t*)(ws + Lw.act);
    uint16_t* proj = (uint16_t*)(ws + Lw.proj);

    // 1. route (+ adjust), as routed.rs:188-209, and 2. compaction
    const bool adjust = a->expert_scales || a->sort_expert_ids;
    const uint32_t sort = a->expert_scales ? a->sort_expert_ids : 1;
    const uint64_t nkeys = (uint64_t)R * E;
    const bool sg = a->up.signed_codes != 0;
    // one token: route, slots and the up product in one launch, while the
    // route that each of its A * H / 8 workgroups repeats (O(E^2) compares)
    // costs less than the separate route launch (measured, one token,
    // separate against fused: model 2048 / hidden 768 / 128 experts 19.4 vs
    // 17.1 us; 256 experts 21.4 vs 22.6; hidden 1536, 128 experts 37.4 vs
    // 38.3; 256 experts 39.3 vs 49.1)
    const bool one = R == 1 && E <= kOneTokenExperts && (uint64_t)A * H * E <= kOneTokenWork;
    if (one) {
        RouteOneArgs ra{a->router_logits, a->expert_scales, E, A, a->round_weights_bf16, a->round_logits_bf16,
                        (uint32_t)adjust, sort, ids, weights, table, header};
        GroupedLaunch g{};
        g.op = bank_op(a->up, E * 2 * H, model, a->input);
        g.header = header;
        g.table = table;
        g.out = act;
        g.tiles = H / 8;
        g.active = A;
        g.hidden = H;
        g.model = model;
        g.cls = 0;
        void* fn = pick_route_up_one(g.op.group_size, sg, model);
        void* argv[] = {&g, &ra};
        const uint32_t blocks = padded_items(A, g.tiles, line_tiles(g.tiles, 8));
        QMM_HIP_CHECK(hipLaunchKernel(fn, dim3(blocks), dim3(kWg), argv, 0, stream));
    } else if (Lw.routes <= kFusedRoutes && R <= kFusedRows && nkeys <= kFusedKeys && nkeys * E <= kFusedCompares) {
        hipLaunchKernelGGL(moe_route_compact, dim3(1), dim3(1024), nkeys * 8, stream, a->router_logits, R, E, A,
                           a->round_weights_bf16, a->round_logits_bf16, a->expert_scales, (uint32_t)adjust, sort,
                           Lw.max_slots, ids, weights, sorted, table, header);
        QMM_HIP_CHECK(hipGetLastError());
    } else {
        st = stark_qmm_moe_route(a->router_logits, ids, weights, R, E, A, a->round_weights_bf16,
                                 a->round_logits_bf16, stream);
        if (st != STARK_QMM_OK) return st;
        if (adjust) st = launch_moe_adjust(ids, weights, a->expert_scales, R, E, A, sort, stream);
        if (st != STARK_QMM_OK) return st;
        hipLaunchKernelGGL(moe_compact, dim3(1), dim3(1024), 0, stream, ids, Lw.routes, E, Lw.max_slots,
                           slot_routes(R), sorted,
                           table, header);
        QMM_HIP_CHECK(hipGetLastError());
    }
    // 3./4. grouped products, one launch per route-count class in use (the
    // one-token path has run the up product already)
    const int top = (int)count_class(max_count);
    // one token: the down products and the rank accumulation in one launch
    void* down_acc = R == 1 && A <= 8 && model % 16 == 0 ? pick_down_acc_one(H, a->down.group_size) : nullptr;
    for (int pass = one ? 1 : 0; pass < (down_acc ? 1 : 2); ++pass) {
        GroupedLaunch g{};
        const bool up = pass == 0;
        g.op = up ? bank_op(a->up, E * 2 * H, model, a->input) : bank_op(a->down, E * model, H, act);
        g.header = header;
        g.out = up ? act : proj;
        g.tiles = up ? H / 8 : model / 16;
        g.active = A;
        g.hidden = H;
        g.model = model;
        for (int c = 0; c <= top; ++c) {
            g.cls = (uint32_t)c;
            g.table = table + (size_t)c * Lw.max_slots * kRecWords;
            const uint64_t items = (uint64_t)class_slot_bound(c, Lw.routes, E, Lw.max_slots) * g.tiles;
            if (items == 0) continue;
            // a multiple of 8 (the items' XCD order), at most 4096
            const uint32_t grid = (uint32_t)std::min<uint64_t>((items + 7) / 8 * 8, 4096);
            void* fn = up ? pick_class<moe_up_mfma_k>(c, max_count, g.op.group_size, sg, model)
                          : pick_class<moe_down_mfma_k>(c, max_count, g.op.group_size, sg, H);
            if (!fn) return STARK_QMM_UNSUPPORTED_GROUP_SIZE;
            void* argv[] = {&g};
            QMM_HIP_CHECK(hipLaunchKernel(fn, dim3(grid), dim3(kWg), argv, 0, stream));
        }
    }
    if (down_acc) {
        const AffineOp d = bank_op(a->down, E * model, H, act);
        DownAccArgs da{(const uint8_t*)a->down.codes,
                       (const uint16_t*)a->down.scales,
                       a->down.correction == STARK_QMM_CORRECTION_BIASES ? (const uint16_t*)a->down.correction_data
                                                                         : nullptr,
                       d.os, d.gs, act, ids, weights, (uint16_t*)a->output, model, H, E, A,
                       a->down.signed_codes ? 1u : 0u, a->round_products_bf16, a->round_accumulator_bf16};
        void* argv[] = {&da};
        const uint32_t blocks = padded_items(1, model / 16, line_tiles(model / 16, 16));
        QMM_HIP_CHECK(hipLaunchKernel(down_acc, dim3(blocks), dim3(64 * A), argv, 0, stream));
        return STARK_QMM_OK;
    }
    // 5. accumulate ranks in order
    hipLaunchKernelGGL(moe_accumulate_ranks, dim3((model + 255) / 256, R), dim3(256), 0, stream, proj, weights,
                       (uint16_t*)a->output, model, A, a->round_products_bf16, a->round_accumulator_bf16);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

// ---- Allocation-free variant: the workspace is a file-scope device array,
// one copy per GPU, held from module load until the process ends. In host
// code `scratch` only names the symbol; its device address comes from
// hipGetSymbolAddress once per device (on the entry point's first call there)
// and is the only form ever passed to a kernel. Nothing in the workspace has
// to start at zero: every route, table and intermediate is written before it
// is read within one call.
constexpr uint64_t kScratchBytes = STARK_QMM_ROUTED_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

uint8_t* scratch_ptr() {
    static std::mutex mu;
    static uint8_t* ptrs[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> g(mu);
    if (!ptrs[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) return nullptr;
        ptrs[dev] = (uint8_t*)p;
    }
    return ptrs[dev];
}

}  // namespace

extern "C" {

stark_qmm_status stark_qmm_routed_experts(const stark_qmm_routed_args* a, void* stream_ptr) {
    if (!a || a->struct_size != sizeof(stark_qmm_routed_args)) return STARK_QMM_ABI_MISMATCH;
    return routed_run(a, (uint8_t*)a->workspace, a->workspace_size, stream_ptr);
}

stark_qmm_status stark_qmm_routed_experts_static(const stark_qmm_routed_args* a, void* stream_ptr) {
    if (!a || a->struct_size != sizeof(stark_qmm_routed_args)) return STARK_QMM_ABI_MISMATCH;
    if (stark_qmm_routed_experts_workspace_size(a->rows, a->model, a->hidden, a->experts, a->active) >
        kScratchBytes)
        return STARK_QMM_WORKSPACE_TOO_SMALL;
    uint8_t* ws = scratch_ptr();
    if (!ws) return STARK_QMM_DEVICE_FAILURE;
    return routed_run(a, ws, kScratchBytes, stream_ptr);
}

}  // extern "C"
