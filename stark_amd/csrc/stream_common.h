// stream_common.h -- pieces shared by the streaming one-row products
// (qmv_stream in qmv_mfma.hip, qmv_chain in qmv_chain.hip): tile geometry,
// the LDS layout of a streaming workgroup, buffer loads, the input prologues
// and the device-resident schedule store.
#pragma once
#include <functional>

#include "mfma_tile.h"

namespace qmm {
namespace mfma {

struct Schedule {
    const uint32_t* begin;  // [grid + 1] offsets into tiles
    const uint32_t* tiles;  // [total tiles]
};

// ---------------------------------------------------------------------------
// Streaming kernel for one activation row of 4-bit codes, group size 64 and
// K % 4096 == 0 (the decode shapes). Same arithmetic as TileEngine -- codes as
// raw bf16 bit patterns, one-hot activation rows per group slot, one f32 flush
// per group -- with a load layout built for HBM streaming:
//  - Split columns. B column c = 8*hh + r of the MFMA holds row r of an 8-row
//    subtile, byte half hh of a 128-byte block: lane r + 8*hh + 16*kb loads the
//    16 bytes at 16*(4*hh + kb) of the block. One load instruction then covers
//    128 contiguous bytes (whole cache lines) of each of 8 rows, and the codes
//    go straight from the load into the MFMA operand with no LDS transpose.
//    A rows 8*hh .. 8*hh+7 are the 8 group slots of byte half hh (x at that
//    half's positions); the C entries that pair one half's activations with
//    the other half's codes are never read.
//  - Tiles of 32 rows (4 subtiles), units of 1024 k. A unit is 16 steps
//    (4 k-blocks of 256 x 4 subtiles, 16 KiB of codes) and one flush period
//    (16 groups per row, 8 per byte half). Wave w takes chunks w, w+4, ... of
//    every tile; the four waves of a workgroup meet once per tile, at an
//    LDS-only barrier. The scale and bias planes of a unit are 16 groups x 32
//    rows: half cache lines in the group-output layout, whose other half is
//    the neighbouring tile's, scheduled on the same XCD.
//  - Loads in flight. A ring of 8 step registers, refilled 8 steps ahead
//    across unit, tile and barrier boundaries (8 KiB per wave in flight). Two
//    workgroups per CU: more bytes in flight only lengthen the queues.
//  - Activations are staged per wave (no barrier) into one of kXR regions,
//    as x * 2^E with a per-group exponent E (group_shift in qmm_common.h),
//    tagged (activation id, chunk), so consecutive tiles of ops that read the
//    same activations (q/k/v, gate/up) reuse them; the plane
//    vectors of a unit are loaded with the unit and pass through a
//    wave-private LDS block at the flush.
constexpr int kXR = 3;         // activation regions per wave
constexpr int kTR = 32;        // tile rows
constexpr int kUnitK = 1024;   // k values per unit (16 groups of 64)
constexpr int kListLds = kWg;  // schedule entries staged in LDS at kernel start (one per thread)

template <int WV>  // waves per workgroup
struct StreamLds {
    u32x4 xp[WV][kXR][kUnitK / 8];  // activation pairs (x0,x4)(x1,x5).. per 8 values; x*2^E, odd values x*2^(E-4)
    float xs[WV][kXR][kUnitK / 64];  // activation sum per group
    int xe[WV][kXR][kUnitK / 64];    // 133 - E per group: the flush's ldexp (activations staged as x * 2^E)
    f32x4 pl[WV][kTR * 8];          // (scale, bias term) of [row][group] of the wave's unit
    float red[2][WV][kTR];           // per-wave row sums, double-buffered by tile parity
    u32x4 zero[WV][4];
    uint32_t list[kListLds];         // the workgroup's first kListLds schedule entries
    float ssq[4];                    // sums of squares of the row by the first four waves (RMS-norm prologue)
};

template <int AUX = 0>
__device__ __forceinline__ u32x4 buf_load(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff = 0) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Input prologues of the streaming kernel, applied to 8 bf16 values of the
// row (t) with the matching 8 values of the prologue operand (w) as they are
// staged; both are elementwise and written in the same operations as the
// decode loop's separate kernels (rms_norm_kernel, silu_mul_kernel), so the
// staged row is bit-identical to the one those write:
//  - RMS norm: bf16(bf16(x * inv) * w), inv = 1 / sqrt(sum(x^2) / K + eps);
//  - SiLU gate: bf16(up * bf16(silu(g))), the activation of GatedActMul's SiLU
//    (crates/stark-engine/src/backends/cpu/kernel/gated_act_mul/gated_act_mul.rs)
//    with the hardware exp2 and reciprocal in place of expf and a division:
//    within one bf16 ulp of it (both round the f32 result to bf16).
// Two f32 values to a bf16 pair (lo, hi), round to nearest even, in one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    const bf16x2_v v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float lo_f32(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float hi_f32(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }

__device__ __forceinline__ u32x4 prologue_norm(u32x4 t, u32x4 w, float inv) {
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t n = bf16_pair(lo_f32(t[q]) * inv, hi_f32(t[q]) * inv);
        o[q] = bf16_pair(lo_f32(n) * lo_f32(w[q]), hi_f32(n) * hi_f32(w[q]));
    }
    return o;
}

// silu(g) = g / (1 + e^-g) with the hardware exp2 and reciprocal
__device__ __forceinline__ float silu_f32(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

__device__ __forceinline__ u32x4 prologue_silu(u32x4 g, u32x4 u) {
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t sg = bf16_pair(silu_f32(lo_f32(g[q])), silu_f32(hi_f32(g[q])));
        o[q] = bf16_pair(lo_f32(u[q]) * lo_f32(sg), hi_f32(u[q]) * hi_f32(sg));
    }
    return o;
}

}  // namespace mfma

// ---- Chained products (qmv_chain.hip). Products of several dependent stages
// run in one persistent launch; a stage's input rows are handed over in
// tagged words (bf16 value in the low half, a 16-bit tag in the high half)
// that the producer writes through to the device-coherent level and the
// consumer polls until every word it needs carries the expected tag.
enum : uint32_t {
    CHAIN_OUT_PLAIN = 0,    // d plain bf16 (ready after the launch)
    CHAIN_OUT_TAGGED = 1,   // d tagged
    CHAIN_OUT_PARTIAL = 2,  // K slice: raw row sums as (part_tag << 32 | f32 bits) into part
    CHAIN_OUT_COMBINE = 3,  // last K slice: adds the nparts earlier slices' sums, then d plain or tagged
};

struct ChainOp {
    const uint8_t* codes;  // first code byte of the slice's K range; rows ldc bytes apart
    const void* scales;    // bf16 planes, offset to the slice's first group
    const void* corr;      // bf16 bias planes, likewise
    const void* x;         // input row of this slice (plain bf16 or tagged words)
    void* d;               // [N] output (plain bf16 or tagged words)
    const void* pro_data;  // RMS-norm weights (plain bf16) or the gate's up row (format of x)
    uint64_t* part;        // PARTIAL: this slice's [N] words; COMBINE: the nparts earlier slices, [nparts][N]
    uint32_t n, k, ldc, os, gs;
    float ab_scale, eps;
    uint32_t pro;          // STARK_QMM_PROLOGUE_*
    uint32_t in_tag;       // 0: x (and a gate's up row) plain, ready at launch; else the tag to wait for
    uint32_t out, out_tag; // CHAIN_OUT_*; tag written to d (0: d plain)
    uint32_t part_tag;     // tag of the K slices' partial words (PARTIAL, COMBINE)
    uint32_t acc_tag;      // accumulate into tagged d: 0 = d ready at launch, else the tag d must carry first
    uint32_t nparts;       // COMBINE: earlier slices
    uint32_t flags;        // FLAG_ACCUMULATE, FLAG_SIGNED
    uint32_t xid;          // ops that read the same row at the same stage share an id (set by the launcher)
    uint32_t order;        // schedule order: ops of a lower order come first in every workgroup's list
};

constexpr int kMaxChainOps = 16;

// Launch a chain of at most kMaxChainOps ops (already split into K slices),
// bf16 planes with biases, M = 1, K a multiple of 4096, N a multiple of 32.
// seq: device word whose low bit flips between calls that reuse the same
// tagged buffers with the same tags (it is xor-ed into bit 15 of every tag);
// may be null. err: device word, set non-zero when a wait gave up.
stark_qmm_status launch_chain(const ChainOp* ops, uint32_t count, const uint32_t* seq, uint32_t* err,
                              hipStream_t stream);

// Device-resident schedule of a launch, built by `build` and uploaded on
// `stream` on first use of `key` (one store per device, shared by every
// persistent kernel of the library; keys of different kernels must differ).
stark_qmm_status schedule_store(const std::vector<uint32_t>& key, uint32_t grid,
                                const std::function<std::vector<uint32_t>()>& build, mfma::Schedule* out,
                                hipStream_t stream);

}  // namespace qmm
