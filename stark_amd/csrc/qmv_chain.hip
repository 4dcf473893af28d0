// Chained one-row products: the dependent products of a decode layer (for
// example o -> gate/up -> down -> the next layer's q/k/v) in ONE persistent
// launch. No counterpart in the reference, whose decoder encodes every
// product (and the norms and gated activation between them) as a dispatch of
// its own (crates/stark-engine/src/encodable_block/transformer_layer.rs); the
// arithmetic of every product is the streaming kernel's (qmv_stream in
// qmv_mfma.hip, MatmulCpuKernel::encode semantics, kernel.rs:168-285), so the
// rows written here are bit-identical to a launch per stage.
//
// Why one launch. Each product launch of a decode step pays a fixed cost
// (dispatch, the first loads' latency, the tail of the slowest workgroup)
// that is a third or more of a 10-56 MB product. The weight streams do not
// depend on the activations, so a persistent workgroup can issue the next
// stage's code loads while the stage it depends on is still being written.
//
// Hand-over without barriers. A stage's input rows are written as tagged
// 32-bit words, bf16 value | tag << 16, with write-through stores (sc1: the
// device-coherent level, past the writer's XCD L2), and read with sc1 loads;
// a consumer re-reads (with a short sleep) until every word it needs carries
// the tag it expects. Each word is its own flag, so there is no counter, no
// fence and no grid barrier; a unit waits only for the rows it reads (the
// down product's unit c only for gate/up rows 1024c.. of its chunk). Tags are
// per (buffer, writer); bit 15 is flipped by the low bit of a caller's
// sequence word between calls that reuse the same tags, so a stale word of
// the previous call never matches.
//
// Deep products are split in K into slices of 4096 (one tile of a slice per
// workgroup, four units); the slices before the last write raw row sums as
// 64-bit (part_tag << 32 | f32) words, and the last slice's tile adds them in slice
// order, ((p0 + p1) + p2), the order in which the one-launch kernel's twelve
// waves add their units' sums, before the D-ops.
//
// Progress. The grid is one resident wave of workgroups (two per CU); every
// workgroup walks its list in stage order, so the lowest unfinished stage
// always has a runnable tile. Every wait is bounded (kSpinLimit re-reads):
// a wave that gives up sets *err and stops waiting for the rest of the
// launch, so a misuse ends in wrong rows and a flag, never a hang.
#include <algorithm>
#include <map>
#include <mutex>

#include "stream_common.h"

namespace qmm {

namespace {

using namespace mfma;

constexpr int kCoh = 16;                // buffer cache policy sc1: device-coherent read / write-through
constexpr uint32_t kSpinLimit = 1u << 16;  // re-reads before a wait gives up (about 0.1 s)


struct ChainBatch {
    ChainOp op[kMaxChainOps];
    uint32_t count;
    const uint32_t* seq;
    uint32_t* err;
};

// 8 tagged words (two vectors) -> 4 bf16 pairs (low half = even element)
__device__ __forceinline__ u32x4 untag(const u32x4& a, const u32x4& b) {
    return u32x4{perm(a[1], a[0], 0x05040100u), perm(a[3], a[2], 0x05040100u), perm(b[1], b[0], 0x05040100u),
                 perm(b[3], b[2], 0x05040100u)};
}

__device__ __forceinline__ bool tags_ok(const u32x4& v, uint32_t tag) {
    return (v[0] >> 16) == tag && (v[1] >> 16) == tag && (v[2] >> 16) == tag && (v[3] >> 16) == tag;
}

// every active lane's predicate holds
__device__ __forceinline__ bool wave_all(bool p) { return __builtin_amdgcn_ballot_w64(!p) == 0; }

template <bool SIGNED>
__global__ __launch_bounds__(kWg) __attribute__((amdgpu_waves_per_eu(2))) void qmv_chain(ChainBatch batch,
                                                                                        Schedule sched) {
    (void)batch;
    constexpr int WV = 4;
    constexpr int RING = 8;  // code loads in flight per wave (steps of 1 KiB; 16 measured no faster)
    constexpr uint32_t UB = kUnitK / 2;
    constexpr uint32_t OOB = 0x80000000u;
    constexpr uint32_t PLANE = 0x7fffffffu;
    __shared__ StreamLds<WV> lds;
    const ChainBatch* kb_ = (const ChainBatch*)__builtin_amdgcn_kernarg_segment_ptr();
    typedef const __attribute__((address_space(4))) uint32_t cu32;
    const uint32_t lo = ((cu32*)sched.begin)[blockIdx.x], hi = ((cu32*)sched.begin)[blockIdx.x + 1];
    if (lo >= hi) return;
    const uint32_t tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t c16 = lane & 15, kb = lane >> 4, hh = c16 >> 3, r = lane & 7;
    const uint32_t piece = 16 * (4 * hh + kb);
    if (lane < 4) lds.zero[wave][lane] = u32x4{0, 0, 0, 0};
    const uint32_t list_v = tid < min(hi - lo, (uint32_t)kListLds) ? sched.tiles[lo + tid] : 0u;
    const auto entry = [&](uint32_t t) {
        return t - lo < (uint32_t)kListLds ? __builtin_amdgcn_readfirstlane(lds.list[t - lo])
                                           : ((cu32*)sched.tiles)[t];
    };
    const auto tile_row = [&](const ChainOp& op, uint32_t e) { return min((e & 0xffffffu) * kTR, op.n - kTR); };
    // tag parity of this call
    const uint32_t flip = kb_->seq ? (__builtin_amdgcn_readfirstlane(*kb_->seq) & 1u) << 15 : 0u;
    bool gave_up = false;  // this wave stopped waiting (wave-uniform)
    const auto give_up = [&] {
        gave_up = true;
        if (lane == 0) __hip_atomic_fetch_or(kb_->err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };

    u32x4 ring[RING];
    u32x4 xv[4], pv[4], pls, plb;
    // Activation (and prologue operand) vectors of unit c: 8 values per lane
    // at c*1024 + 8*lane (+ 512 for the second vector).
    const auto load_x = [&](const ChainOp& op, uint32_t c, bool need_x) {
        const uint32_t e0 = c * kUnitK + lane * 8;
        if (op.in_tag) {
            const __amdgpu_buffer_rsrc_t xr = rsrc(op.x, op.k * 4);
            const uint32_t xo = need_x ? e0 * 4 : OOB;
            xv[0] = buf_load<kCoh>(xr, xo);
            xv[1] = buf_load<kCoh>(xr, xo + 16);
            xv[2] = buf_load<kCoh>(xr, xo + 2048);
            xv[3] = buf_load<kCoh>(xr, xo + 2064);
            if (op.pro == STARK_QMM_PROLOGUE_SILU_GATE) {
                const __amdgpu_buffer_rsrc_t pr = rsrc(op.pro_data, op.k * 4);
                pv[0] = buf_load<kCoh>(pr, xo);
                pv[1] = buf_load<kCoh>(pr, xo + 16);
                pv[2] = buf_load<kCoh>(pr, xo + 2048);
                pv[3] = buf_load<kCoh>(pr, xo + 2064);
            }
        } else {
            const __amdgpu_buffer_rsrc_t xr = rsrc(op.x, op.k * 2);
            const uint32_t xo = need_x ? e0 * 2 : OOB;
            xv[0] = buf_load(xr, xo);
            xv[1] = buf_load(xr, xo + 1024);
            if (op.pro == STARK_QMM_PROLOGUE_SILU_GATE) {
                const __amdgpu_buffer_rsrc_t pr = rsrc(op.pro_data, op.k * 2);
                pv[0] = buf_load(pr, xo);
                pv[1] = buf_load(pr, xo + 1024);
            }
        }
        if (op.pro == STARK_QMM_PROLOGUE_RMS_NORM) {  // norm weights: plain bf16
            const __amdgpu_buffer_rsrc_t pr = rsrc(op.pro_data, op.k * 2);
            const uint32_t po = need_x ? e0 * 2 : OOB;
            pv[0] = buf_load(pr, po);
            pv[1] = buf_load(pr, po + 1024);
        }
    };
    const auto issue_aux = [&](const ChainOp& op, uint32_t n0, uint32_t c, bool need_x) {
        load_x(op, c, need_x);
        const size_t off = op.os == 1 ? (size_t)(c * 16 + ((lane >> 2) & 15)) * op.gs + n0 + 8 * (lane & 3)
                                      : (size_t)(n0 + ((lane >> 1) & 31)) * op.os + c * 16 + 8 * (lane & 1);
        pls = buf_load(rsrc(op.scales, PLANE), (uint32_t)off * 2);
        plb = buf_load(rsrc(op.corr, PLANE), (uint32_t)off * 2);
    };
    const auto code_rsrc = [&](const ChainOp& op, uint32_t n0) {
        return rsrc(op.codes + (size_t)n0 * op.ldc, kTR * op.ldc);
    };
    const auto step_soff = [&](const ChainOp& op, int v) { return (uint32_t)(8 * (v % 4)) * op.ldc + (v / 4) * 128; };

    uint32_t i = lo, ri = 0, e = ((cu32*)sched.tiles)[lo];
    const ChainOp* opp = &kb_->op[e >> 24];
    __amdgpu_buffer_rsrc_t cr;
    uint32_t vo;
    {
        const uint32_t n0 = tile_row(*opp, e);
        issue_aux(*opp, n0, wave, true);
        cr = code_rsrc(*opp, n0);
        vo = r * opp->ldc + wave * UB + piece;
#pragma unroll
        for (int s = 0; s < RING; ++s) ring[s] = buf_load<kBufNt>(cr, vo, step_soff(*opp, s));
    }
    if (tid < (uint32_t)kListLds) lds.list[tid] = list_v;
    lds_barrier();
    float inv = 0.0f;
    uint32_t inv_xid = ~0u;  // row whose RMS factor `inv` holds
    uint32_t tg0 = ~0u, tg1 = ~0u, tg2 = ~0u;
    const auto tag_of = [&](uint32_t rg) { return rg == 0 ? tg0 : rg == 1 ? tg1 : tg2; };
    f32x4 acc[4] = {};
    uint32_t par = 0;
    for (;;) {
        const ChainOp& op = *opp;
        const uint32_t R = op.k / (WV * kUnitK);
        const uint32_t t0 = (e & 0xffffffu) * kTR, n0 = min(t0, op.n - kTR);
        const uint32_t c = wave + WV * ri;
        const uint32_t rg = ri % kXR;
        const uint32_t tag = (op.xid << 16) | c;
        u32x4* xpw = lds.xp[wave][rg];
        float* xsw = lds.xs[wave][rg];
        int* xew = lds.xe[wave][rg];
        if (tag_of(rg) != tag) {
            if (op.in_tag && !gave_up) {  // wait for the unit's rows
                const uint32_t want = op.in_tag ^ flip;
                const bool silu = op.pro == STARK_QMM_PROLOGUE_SILU_GATE;
                const auto ready = [&] {
                    bool ok = tags_ok(xv[0], want) && tags_ok(xv[1], want) && tags_ok(xv[2], want) &&
                              tags_ok(xv[3], want);
                    if (silu)
                        ok = ok && tags_ok(pv[0], want) && tags_ok(pv[1], want) && tags_ok(pv[2], want) &&
                             tags_ok(pv[3], want);
                    return wave_all(ok);
                };
                // While the rows are incomplete, poll one word per producer
                // tile (32 rows) of the chunk -- lanes 0..31 the row, lanes
                // 32..63 a gate's up row -- and reload the chunk once they all
                // carry the tag.
                const uint32_t* probe = (const uint32_t*)(lane < 32 ? op.x : silu ? op.pro_data : op.x) +
                                        c * kUnitK + 32 * (lane & 31) + 31;
                for (uint32_t spins = 0; !gave_up && !ready();) {
                    for (;;) {
                        __builtin_amdgcn_s_sleep(8);
                        const uint32_t w = __hip_atomic_load(probe, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        if (wave_all((w >> 16) == want)) break;
                        if (++spins > kSpinLimit) {
                            give_up();
                            break;
                        }
                    }
                    load_x(op, c, true);
                }
            }
            if (op.pro == STARK_QMM_PROLOGUE_RMS_NORM && inv_xid != op.xid) {
                // RMS factor of the row (K = 4096: one unit per wave, wave w
                // staging chunk w), in the decode loop's RMS-norm kernel order:
                // per lane the vectors 128w + l and 128w + 64 + l of chunk w,
                // the wave sum by xor butterfly, then the four chunks in turn
                float ss = 0.0f;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const u32x4 t = op.in_tag ? untag(xv[2 * h], xv[2 * h + 1]) : xv[h];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float a = __uint_as_float(t[q] << 16), b = __uint_as_float(t[q] & 0xffff0000u);
                        ss = fmaf(a, a, fmaf(b, b, ss));
                    }
                }
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
                if (lane == 0) lds.ssq[wave] = ss;
                lds_barrier();
                inv = 1.0f / sqrtf((lds.ssq[0] + lds.ssq[1] + lds.ssq[2] + lds.ssq[3]) / (float)op.k + op.eps);
                inv_xid = op.xid;
            }
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                u32x4 t = op.in_tag ? untag(xv[2 * m], xv[2 * m + 1]) : xv[m];
                if (op.pro == STARK_QMM_PROLOGUE_RMS_NORM) t = prologue_norm(t, pv[m], inv);
                if (op.pro == STARK_QMM_PROLOGUE_SILU_GATE)
                    t = prologue_silu(t, op.in_tag ? untag(pv[2 * m], pv[2 * m + 1]) : pv[m]);
                const int E = group_shift(group_max<8>(bf16x8_exp_max(t)));
                const float se = pow2i(E), so = pow2i(E - 4);
                float f[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f[2 * q] = __uint_as_float(t[q] << 16) * se;
                    f[2 * q + 1] = __uint_as_float(t[q] & 0xffff0000u) * so;
                }
                u32x4 pq;
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
        {  // plane vectors -> f32 (scale, bias) pairs at [row][group]
            float sv[8], bv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                sv[q] = plane_f32((pls[q >> 1] >> (16 * (q & 1))) & 0xffffu, true);
                bv[q] = plane_f32((plb[q >> 1] >> (16 * (q & 1))) & 0xffffu, true);
            }
            float2* pw = (float2*)lds.pl[wave];
            if (op.os == 1) {
                const uint32_t g = (lane >> 2) & 15, r0 = 8 * (lane & 3);
#pragma unroll
                for (int q = 0; q < 8; ++q) pw[(r0 + q) * 16 + g] = float2{sv[q], bv[q]};
            } else {
                const uint32_t row = (lane >> 1) & 31, g0 = 8 * (lane & 1);
#pragma unroll
                for (int q = 0; q < 8; ++q) pw[row * 16 + g0 + q] = float2{sv[q], bv[q]};
            }
        }

        // ---- next unit: activation and plane loads now, code loads from step 8 on
        uint32_t ni = i, nr = ri + 1;
        if (nr == R) {
            ni = i + 1;
            nr = 0;
        }
        const bool more = ni < hi;
        const uint32_t ne = more ? entry(ni) : e;
        const uint32_t nc = more ? wave + WV * nr : c;
        const ChainOp& nop = kb_->op[ne >> 24];
        const uint32_t nn0 = tile_row(nop, ne);
        issue_aux(nop, nn0, nc, more && tag_of(nr % kXR) != ((nop.xid << 16) | nc));
        const __amdgpu_buffer_rsrc_t ncr = code_rsrc(nop, nn0);
        const uint32_t nvo = more ? r * nop.ldc + nc * UB + piece : OOB;

        f32x4 C0[4] = {}, C1[4] = {};
        const u32x4* zero = lds.zero[wave];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int st = u % 4, ks = u / 4, sl = u % RING;
            u32x4 bq[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint32_t w = ring[sl][t];
                if (SIGNED) w ^= 0x88888888u;
                const uint32_t w8 = w >> 8;
                bq[t][0] = w & 0x000F000Fu;
                bq[t][1] = w & 0x00F000F0u;
                bq[t][2] = w8 & 0x000F000Fu;
                bq[t][3] = w8 & 0x00F000F0u;
            }
            __builtin_amdgcn_sched_barrier(0);
            if (u + RING < 16)
                ring[sl] = buf_load<kBufNt>(cr, vo, step_soff(op, u + RING));
            else
                ring[sl] = buf_load<kBufNt>(ncr, nvo, step_soff(nop, u + RING - 16));
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

        {  // flush (as qmv_stream)
            const uint32_t gb = 8 * (kb & 1) + 2 * hh;
            const float2 xa = *(const float2*)&xsw[gb];
            const float2 xb = *(const float2*)&xsw[gb + 4];
            const float xq[4] = {xa.x, xa.y, xb.x, xb.y};
            const int2 ea = *(const int2*)&xew[gb];
            const int2 eb = *(const int2*)&xew[gb + 4];
            const int nq[4] = {ea.x, ea.y, eb.x, eb.y};
            const f32x4* pw = lds.pl[wave];
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const f32x4 cs = C0[st] + C1[st];
                const uint32_t row = 8 * st + r;
                const f32x4 pa = pw[(row * 16 + gb) / 2], pb = pw[(row * 16 + gb + 4) / 2];
                const float sq[4] = {pa[0], pa[2], pb[0], pb[2]}, bq[4] = {pa[1], pa[3], pb[1], pb[3]};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    acc[st][q] = fmaf(sq[q], ldexp_f32(cs[q], nq[q]), fmaf(bq[q], xq[q], acc[st][q]));
            }
        }

        if (ri + 1 == R) {
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                float v = (acc[st][0] + acc[st][1]) + (acc[st][2] + acc[st][3]);
                v = (kb >> 1) == hh ? v : 0.0f;
                v += __shfl_xor(v, 8, 64);
                v += __shfl_xor(v, 16, 64);
                v += __shfl_xor(v, 32, 64);
                if (lane < 8) lds.red[par][wave][8 * st + lane] = v;
                acc[st] = f32x4{0, 0, 0, 0};
            }
            lds_barrier();
            if (tid < (uint32_t)kTR) {  // wave 0, lanes 0..31: one output row each
                const uint32_t n = n0 + tid;
                const bool own = n >= t0;  // rows of the previous tile (shifted last tile) are not written again
                float o = (lds.red[par][0][tid] + lds.red[par][1][tid]) + (lds.red[par][2][tid] + lds.red[par][3][tid]);
                const uint32_t out_tag = op.out_tag ^ flip, part_tag = op.part_tag ^ flip;
                if (op.out == CHAIN_OUT_PARTIAL) {
                    if (own)
                        __hip_atomic_store(op.part + n, ((uint64_t)part_tag << 32) | __float_as_uint(o),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                } else {
                    if (op.out == CHAIN_OUT_COMBINE) {
                        uint64_t w[8];
                        const uint32_t np = op.nparts;
                        const auto rd = [&] {
                            for (uint32_t j = 0; j < np; ++j)
                                w[j] = __hip_atomic_load(op.part + (size_t)j * op.n + n, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                        };
                        rd();
                        for (uint32_t spins = 0; !gave_up;) {
                            bool ok = true;
                            for (uint32_t j = 0; j < np; ++j) ok = ok && (uint32_t)(w[j] >> 32) == part_tag;
                            if (wave_all(ok)) break;
                            if (++spins > kSpinLimit) {
                                give_up();
                                break;
                            }
                            __builtin_amdgcn_s_sleep(2);
                            rd();
                        }
                        float t = __uint_as_float((uint32_t)w[0]);
                        for (uint32_t j = 1; j < np; ++j) t = t + __uint_as_float((uint32_t)w[j]);
                        o = t + o;
                    }
                    o *= op.ab_scale;
                    if (!op.out_tag) {  // plain bf16 d (ready at launch when accumulated)
                        if (op.flags & FLAG_ACCUMULATE) o += bf16_bits_to_f32(((const uint16_t*)op.d)[n]);
                        if (own) ((uint16_t*)op.d)[n] = f32_to_bf16_bits(o);
                    } else {
                        uint32_t* dw = (uint32_t*)op.d;
                        if (op.flags & FLAG_ACCUMULATE) {
                            uint32_t a = __hip_atomic_load(dw + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            if (op.acc_tag) {
                                const uint32_t want = op.acc_tag ^ flip;
                                for (uint32_t spins = 0; !gave_up;) {
                                    if (wave_all((a >> 16) == want)) break;
                                    if (++spins > kSpinLimit) {
                                        give_up();
                                        break;
                                    }
                                    __builtin_amdgcn_s_sleep(2);
                                    a = __hip_atomic_load(dw + n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                                }
                            }
                            o += bf16_bits_to_f32(a & 0xffffu);
                        }
                        if (own)
                            __hip_atomic_store(dw + n, (uint32_t)f32_to_bf16_bits(o) | (out_tag << 16),
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
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

// Lists for `grid` workgroups: op orders in turn; within one order the
// tiles sharing a group-output plane line (two 32-row tiles) go to one XCD,
// and each tile goes to the least-loaded workgroup of its XCD (load = units
// of every earlier tile), so that a workgroup that finishes a stage early
// takes more of the next.
std::vector<uint32_t> build_chain_schedule(const ChainOp* ops, uint32_t count, uint32_t grid) {
    const uint32_t per_xcd = grid / 8;
    std::vector<std::vector<uint32_t>> lists(grid);
    std::vector<uint64_t> load(grid, 0);
    std::vector<uint32_t> orders;
    for (uint32_t i = 0; i < count; ++i) orders.push_back(ops[i].order);
    std::sort(orders.begin(), orders.end());
    orders.erase(std::unique(orders.begin(), orders.end()), orders.end());
    uint32_t quad = 0;
    for (uint32_t ord : orders) {
        // the ops of one order interleaved by tile pair (gate and up rows of
        // the same chunk come out together, so a later stage that waits for
        // a chunk of both can start while the rest is still being written)
        std::vector<std::vector<std::pair<uint32_t, uint32_t>>> xcd_tiles(8);
        uint32_t most = 0;
        for (uint32_t i = 0; i < count; ++i)
            if (ops[i].order == ord) most = std::max(most, (ops[i].n + kTR - 1) / kTR);
        for (uint32_t t0 = 0; t0 < most; t0 += 2)
            for (uint32_t i = 0; i < count; ++i) {
                if (ops[i].order != ord) continue;
                const uint32_t tiles = (ops[i].n + kTR - 1) / kTR;
                if (t0 >= tiles) continue;
                for (uint32_t t = t0; t < std::min(tiles, t0 + 2); ++t)
                    xcd_tiles[quad % 8].push_back({(i << 24) | t, ops[i].k});
                ++quad;
            }
        for (uint32_t x = 0; x < 8; ++x)
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
    return host;
}

template <class Kern>
uint32_t resident_grid(Kern kern) {
    static std::mutex mu;
    static std::map<std::pair<const void*, int>, uint32_t> cache;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    std::lock_guard<std::mutex> lock(mu);
    const auto key = std::make_pair((const void*)kern, dev);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kWg, 0) != hipSuccess)
        return 0;
    // two workgroups per CU (eight waves), never more than fit at once: every
    // workgroup of the grid must be resident for the hand-over to progress
    const uint32_t grid = per_cu < 1 ? 0u : (uint32_t)(cus * std::min(per_cu, 2) / 8 * 8);
    cache.emplace(key, grid);
    return grid;
}

}  // namespace

stark_qmm_status launch_chain(const ChainOp* ops, uint32_t count, const uint32_t* seq, uint32_t* err,
                              hipStream_t stream) {
    if (count == 0) return STARK_QMM_OK;
    if (count > (uint32_t)kMaxChainOps || !err) return STARK_QMM_UNSUPPORTED;
    ChainBatch batch{};
    bool sg = (ops[0].flags & FLAG_SIGNED) != 0;
    for (uint32_t i = 0; i < count; ++i) {
        if ((ops[i].flags & FLAG_SIGNED) != 0 != sg) return STARK_QMM_UNSUPPORTED;
        batch.op[i] = ops[i];
        // ops of one order that read the same row (and prologue) stage it once
        uint32_t x = i;
        for (uint32_t j = 0; j < i; ++j)
            if (ops[j].order == ops[i].order && ops[j].x == ops[i].x && ops[j].k == ops[i].k &&
                ops[j].in_tag == ops[i].in_tag && ops[j].pro == ops[i].pro && ops[j].pro_data == ops[i].pro_data) {
                x = j;
                break;
            }
        batch.op[i].xid = x;
    }
    batch.count = count;
    batch.seq = seq;
    batch.err = err;
    auto kern = sg ? qmv_chain<true> : qmv_chain<false>;
    const uint32_t grid = resident_grid(kern);
    if (grid == 0) return STARK_QMM_DEVICE_FAILURE;
    std::vector<uint32_t> key{grid, 0xC4A10000u, count};
    for (uint32_t i = 0; i < count; ++i) {
        key.push_back(ops[i].n);
        key.push_back(ops[i].k);
        key.push_back(ops[i].order);
    }
    Schedule sched;
    const stark_qmm_status st =
        schedule_store(key, grid, [&] { return build_chain_schedule(batch.op, count, grid); }, &sched, stream);
    if (st != STARK_QMM_OK) return st;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(kWg), 0, stream, batch, sched);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // namespace qmm

