// Decode-step kernels around the quantized products for the config-4
// end-to-end stand-in: a Qwen3-architecture decoder (pre-norm RMSNorm,
// per-head q/k RMSNorm, rotate-half RoPE, GQA attention over a bf16 KV cache,
// gated SiLU MLP, final norm, greedy argmax). They are not part of the
// quantized matrix-product drop-in (libstark_qmm): the reference's own
// versions live in its model runtime (normalization:
// crates/stark-engine/src/backends/cpu/kernel/normalization/normalization.rs:17-140;
// q/k norm: attention/qkv_norm.rs; KV update: attention/kv_cache_update.rs;
// single-pass attention: attention/attention_single_pass.rs; gated activation:
// gated_act_mul). Storage is bf16, arithmetic f32.
//
// Every position-dependent kernel reads the position from device memory so a
// whole token step can be captured once in a HIP graph and replayed.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>

namespace {

constexpr int kHd = 128;      // head dim
constexpr int kChunk = 64;    // attention positions per partial workgroup
constexpr int kMaxChunks = 1024;  // chunks the reduction takes (capacity <= 65536)

// RoPE frequencies in revolutions per position, theta^(-2i/hd) / (2 pi) for
// the 64 rotation pairs, computed on the host in double and passed by value:
// the angle pos * f is then one f32 product (as pos * inv_freq was), reduced
// exactly to its fraction of a turn, and sine and cosine come from the
// hardware v_sin_f32 / v_cos_f32 on that fraction.
struct RopeTable {
    float f[kHd / 2];
};

__device__ __forceinline__ void rope_sincos(const RopeTable& t, uint32_t i, int32_t pos, float& sn, float& cs) {
    const float turn = __builtin_amdgcn_fractf((float)pos * t.f[i]);
    sn = __builtin_amdgcn_sinf(turn);
    cs = __builtin_amdgcn_cosf(turn);
}

RopeTable rope_table(float theta) {
    RopeTable t;
    for (int i = 0; i < kHd / 2; ++i)
        t.f[i] = (float)(std::pow((double)theta, -2.0 * i / kHd) / (2.0 * 3.14159265358979323846));
    return t;
}

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// f32 -> bf16 round to nearest even on v_cvt_pk_bf16_f32 (the conversion of
// the products' input prologues)
__device__ __forceinline__ uint16_t hw_bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

__device__ __forceinline__ uint16_t to_bf(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Wave reductions on DPP (quad_perm xor 1 and xor 2, half-row and row
// mirrors: every lane of a 16-lane row holds the row's value) and the four
// rows read into scalars, added as (r0 + r1) + (r2 + r3): a chain of VALU
// operations instead of six LDS-pipe shuffles. The RMS norm keeps the xor
// butterfly above, whose order the products' RMS-norm prologue repeats.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_f32(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// out = x * rsqrt(mean(x^2) + eps) * w, one row of n (n % 256 == 0), 256 threads;
// the bf16 roundings on v_cvt_pk_bf16_f32, as the products' RMS-norm prologue.
// Thread t = 64 w + l owns the 8-value vectors 128c + l and 128c + 64 + l of
// the 1024-value chunks c = w, w + 4, ... (chunk-major: the order in which
// the products' RMS-norm prologue sums the row, so that both compute the same
// inverse norm), summed in that order, then the wave sums (xor butterfly) and
// the four waves in order; rows that are not whole chunks take vectors t,
// t + 256, ... instead. Every load of a thread is a 16-byte vector issued
// before the first use (rows up to 8192 stay in registers for the second pass).
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* x, const uint16_t* w, uint16_t* out,
                                                       uint32_t n, float eps) {
    constexpr int kKeep = 4;  // vectors of 8 values kept per thread
    __shared__ float part[4];
    const uint32_t t = threadIdx.x, nv = n / 8;
    const bool chunked = n % 1024 == 0;
    // j-th vector of this thread
    const auto vec = [&](uint32_t j) -> uint32_t {
        return chunked ? 128 * ((t >> 6) + 4 * (j >> 1)) + 64 * (j & 1) + (t & 63) : t + 256 * j;
    };
    const uint4* xv = (const uint4*)x;
    uint4 keep[kKeep], wkeep[kKeep];  // the weights are loaded with x: one memory round trip
#pragma unroll
    for (int j = 0; j < kKeep; ++j) keep[j] = vec(j) < nv ? xv[vec(j)] : uint4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < kKeep; ++j) wkeep[j] = vec(j) < nv ? ((const uint4*)w)[vec(j)] : uint4{0, 0, 0, 0};
    float ss = 0.0f;
    const auto sq = [&](const uint4& u) {
        const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float a = __uint_as_float(wd[e] << 16), b = __uint_as_float(wd[e] & 0xffff0000u);
            ss = fmaf(a, a, fmaf(b, b, ss));
        }
    };
#pragma unroll
    for (int j = 0; j < kKeep; ++j) sq(keep[j]);
    for (uint32_t j = kKeep; vec(j) < nv; ++j) sq(xv[vec(j)]);
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)n + eps);
    const auto emit = [&](uint32_t i, const uint4& u, const uint4& wv) {
        const uint32_t xd[4] = {u.x, u.y, u.z, u.w}, wd[4] = {wv.x, wv.y, wv.z, wv.w};
        uint32_t od[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float a = __uint_as_float(xd[e] << 16), b = __uint_as_float(xd[e] & 0xffff0000u);
            const uint16_t lo = hw_bf(bf(hw_bf(a * inv)) * __uint_as_float(wd[e] << 16));
            const uint16_t hi = hw_bf(bf(hw_bf(b * inv)) * __uint_as_float(wd[e] & 0xffff0000u));
            od[e] = (uint32_t)lo | ((uint32_t)hi << 16);
        }
        ((uint4*)out)[i] = uint4{od[0], od[1], od[2], od[3]};
    };
#pragma unroll
    for (int j = 0; j < kKeep; ++j)
        if (vec(j) < nv) emit(vec(j), keep[j], wkeep[j]);
    for (uint32_t j = kKeep; vec(j) < nv; ++j) emit(vec(j), xv[vec(j)], ((const uint4*)w)[vec(j)]);
}

// Per-head RMSNorm of q and k, rotate-half RoPE at *pos, and the k/v write
// into the cache rows at *pos. Workgroup h < qh: query head h; else key/value
// head h - qh. 64 threads, each owning dims i and i + 64 (a rotation pair).
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                          const uint16_t* qw, const uint16_t* kw, uint16_t* kcache,
                                                          uint16_t* vcache, const int32_t* pos_ptr, uint32_t qh,
                                                          uint32_t kvh, uint32_t cap, RopeTable rope, float eps) {
    const uint32_t h = blockIdx.x, i = threadIdx.x;
    const int32_t pos = *pos_ptr;
    const bool is_q = h < qh;
    const uint16_t* src = is_q ? q + (size_t)h * kHd : k + (size_t)(h - qh) * kHd;
    const uint16_t* w = is_q ? qw : kw;
    const float a = bf(src[i]), b = bf(src[i + 64]);
    const float inv = 1.0f / sqrtf(wave_sum_dpp(a * a + b * b) / (float)kHd + eps);
    const float na = bf(to_bf(bf(to_bf(a * inv)) * bf(w[i])));
    const float nb = bf(to_bf(bf(to_bf(b * inv)) * bf(w[i + 64])));
    float sn, cs;
    rope_sincos(rope, i, pos, sn, cs);
    const uint16_t ra = to_bf(na * cs - nb * sn), rb = to_bf(nb * cs + na * sn);
    if (is_q) {
        q[(size_t)h * kHd + i] = ra;
        q[(size_t)h * kHd + i + 64] = rb;
    } else if ((uint32_t)pos < cap) {  // a full cache takes no more rows
        const uint32_t kv = h - qh;
        const size_t row = ((size_t)kv * cap + (uint32_t)pos) * kHd;
        kcache[row + i] = ra;
        kcache[row + i + 64] = rb;
        vcache[row + i] = v[(size_t)kv * kHd + i];
        vcache[row + i + 64] = v[(size_t)kv * kHd + i + 64];
    }
}

// Flash-decoding partials: workgroup (kv head g, chunk c) scores its GQA
// group's G query heads against positions [c*kChunk, min(len, (c+1)*kChunk)),
// len = *pos + 1, and writes the unnormalised partial output with its max and
// sum. 64*G threads: wave h is query head h of the group. The K and V tiles of
// the chunk (kChunk x 128 bf16 each) are read with 16-byte loads issued
// together into LDS (K rows padded so that the row-per-lane score reads spread
// over the banks); scores, softmax and PV then run from LDS.
template <int G>
__global__ __launch_bounds__(64 * G) void attn_partial_kernel(const uint16_t* q, const uint16_t* kcache,
                                                              const uint16_t* vcache, float* po, float* pml,
                                                              const int32_t* pos_ptr, uint32_t kvh, uint32_t cap,
                                                              uint32_t nchunks, float scale) {
    constexpr int kRowK = kHd / 2 + 4;  // padded K row, in u32 (bf16 pairs)
    constexpr int kVec = kChunk * kHd / 8;  // 16-byte vectors per tile
    __shared__ uint32_t ks[kChunk * kRowK];
    __shared__ uint32_t vs[kChunk * kHd / 2];
    __shared__ float qs[G][kHd];
    __shared__ float ws[G][kChunk];
    const uint32_t g = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63, h = t >> 6;
    const uint32_t len = min((uint32_t)*pos_ptr + 1, cap);
    const uint32_t p0 = c * kChunk;
    if (p0 >= len) return;  // chunk past the context: the reduction skips it
    const uint32_t np = min((uint32_t)kChunk, len - p0);
    {
        constexpr int kPer = (kVec + 64 * G - 1) / (64 * G);
        const uint4* kg = (const uint4*)(kcache + ((size_t)g * cap + p0) * kHd);
        const uint4* vg = (const uint4*)(vcache + ((size_t)g * cap + p0) * kHd);
        uint4 kv[kPer], vv[kPer];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const uint32_t v = t + j * 64 * G;
            const bool ok = v < (uint32_t)kVec && v / (kHd / 8) < np;  // rows past the context read nothing
            kv[j] = ok ? kg[v] : uint4{0, 0, 0, 0};
            vv[j] = ok ? vg[v] : uint4{0, 0, 0, 0};
        }
        const uint32_t qd = lane * 2;
        const uint32_t qw = *(const uint32_t*)(q + ((size_t)(g * G + h)) * kHd + qd);
        qs[h][qd] = __uint_as_float(qw << 16);
        qs[h][qd + 1] = __uint_as_float(qw & 0xffff0000u);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const uint32_t v = t + j * 64 * G;
            if (v < (uint32_t)kVec) {
                const uint32_t row = v / (kHd / 8), col = (v % (kHd / 8)) * 4;
                *(uint4*)&ks[row * kRowK + col] = kv[j];
                *(uint4*)&vs[row * (kHd / 2) + col] = vv[j];
            }
        }
    }
    __syncthreads();
    // scores: lane = position, wave = head
    float s = -INFINITY;
    if (lane < np) {
        const uint32_t* kr = &ks[lane * kRowK];
        float acc = 0.0f;
#pragma unroll 8
        for (int d2 = 0; d2 < kHd / 2; d2 += 2) {
            const uint2 u = *(const uint2*)&kr[d2];
            acc = fmaf(qs[h][2 * d2], __uint_as_float(u.x << 16), acc);
            acc = fmaf(qs[h][2 * d2 + 1], __uint_as_float(u.x & 0xffff0000u), acc);
            acc = fmaf(qs[h][2 * d2 + 2], __uint_as_float(u.y << 16), acc);
            acc = fmaf(qs[h][2 * d2 + 3], __uint_as_float(u.y & 0xffff0000u), acc);
        }
        s = acc * scale;
    }
    const float m = wave_max_dpp(s);
    const float e = lane < np ? __expf(s - m) : 0.0f;
    const float l = wave_sum_dpp(e);
    ws[h][lane] = e;
    __syncthreads();
    // PV: lane = dims 2*lane, 2*lane + 1
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll 8
    for (uint32_t p = 0; p < np; ++p) {
        const uint32_t u = vs[p * (kHd / 2) + lane];
        const float wp = ws[h][p];
        o0 = fmaf(wp, __uint_as_float(u << 16), o0);
        o1 = fmaf(wp, __uint_as_float(u & 0xffff0000u), o1);
    }
    const size_t row = (size_t)(g * G + h) * nchunks + c;
    *(float2*)&po[row * kHd + 2 * lane] = float2{o0, o1};
    if (lane == 0) *(float2*)&pml[row * 2] = float2{m, l};
}

// Combine the chunks of each query head: out = sum_c o_c e^(m_c - m) / sum_c l_c e^(m_c - m).
// The chunk maxima and sums are read in parallel first (the first 128 with
// the first partial outputs, before the position is known); the weighted sum
// of the remaining partial outputs issues its loads eight chunks at a time.
__global__ __launch_bounds__(128) void attn_reduce_kernel(const float* po, const float* pml, uint16_t* out,
                                                          const int32_t* pos_ptr, uint32_t nchunks, uint32_t cap) {
    __shared__ float fs[kMaxChunks];
    __shared__ float red[2];
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    // The first kPre chunks' partial outputs are loaded at once, before the
    // position is known (chunks past it are loaded and not used): one memory
    // round trip for contexts up to kPre * kChunk.
    constexpr uint32_t kPre = 80;
    const float* col = po + (size_t)h * nchunks * kHd + d;
    float pre[kPre];
#pragma unroll
    for (uint32_t j = 0; j < kPre; ++j) pre[j] = j < nchunks ? col[(size_t)j * kHd] : 0.0f;
    // this thread's first chunk statistics, likewise before the position is known
    const float2* ml = (const float2*)pml + (size_t)h * nchunks;
    const float2 ml0 = d < nchunks ? ml[d] : float2{0.0f, 0.0f};
    const uint32_t len = min((uint32_t)*pos_ptr + 1, cap);
    const uint32_t nc = min(nchunks, (len + kChunk - 1) / kChunk);
    float mx = d < nc ? ml0.x : -INFINITY;
    for (uint32_t c = d + 128; c < nc; c += 128) mx = fmaxf(mx, ml[c].x);
    mx = wave_max_dpp(mx);
    if ((d & 63) == 0) red[d >> 6] = mx;
    __syncthreads();
    const float m = fmaxf(red[0], red[1]);
    __syncthreads();
    float l = 0.0f;
    for (uint32_t c = d; c < nc; c += 128) {
        const float2 v = c == d ? ml0 : ml[c];
        const float f = __expf(v.x - m);
        fs[c] = f;
        l = fmaf(v.y, f, l);
    }
    l = wave_sum_dpp(l);
    if ((d & 63) == 0) red[d >> 6] = l;
    __syncthreads();
    l = red[0] + red[1];
    float o = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kPre; ++j)
        if (j < nc) o = fmaf(pre[j], fs[j], o);
    uint32_t c = kPre;
    for (; c + 8 <= nc; c += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = col[(size_t)(c + j) * kHd];
#pragma unroll
        for (int j = 0; j < 8; ++j) o = fmaf(v[j], fs[c + j], o);
    }
    for (; c < nc; ++c) o = fmaf(col[(size_t)c * kHd], fs[c], o);
    out[(size_t)h * kHd + d] = to_bf(o / l);
}

// Per-head RMSNorm + rotate-half RoPE of one head (128 values, lane owns dims
// i and i + 64), the arithmetic of qk_norm_rope_kernel: returns the rotated
// pair rounded to bf16.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

__device__ __forceinline__ void norm_rope_pair(float a, float b, uint16_t wa, uint16_t wb, uint32_t i, int32_t pos,
                                               const RopeTable& rope, float eps, uint16_t& ra, uint16_t& rb) {
    const float inv = 1.0f / sqrtf(wave_sum_dpp(a * a + b * b) / (float)kHd + eps);
    const float na = bf(to_bf(bf(to_bf(a * inv)) * bf(wa)));
    const float nb = bf(to_bf(bf(to_bf(b * inv)) * bf(wb)));
    float sn, cs;
    rope_sincos(rope, i, pos, sn, cs);
    ra = to_bf(na * cs - nb * sn);
    rb = to_bf(nb * cs + na * sn);
}

// Attention of one decode step with the q/k norm + RoPE + KV write folded
// in: workgroup (kv head g, chunk c) of four waves, for the G query heads of
// the group.
//  - Registers, not LDS, hold the chunk's K and V: lane l of wave w owns
//    position p = 16 w + l / 4 and dim quarter d4 = l % 4, and loads that
//    row's 32 K values of the quarter (four 16-byte loads) for the scores of
//    every head of the group (the quarters meet by two shuffles), and the V
//    pairs (2 l, 2 l + 1) of the wave's 16 positions (16 loads of 4 bytes, a
//    whole 256-byte row per load instruction) for PV. Each K and V value is
//    read from memory once per workgroup and from no LDS at all.
//  - Every workgroup normalises and rotates its G query heads itself (wave
//    w takes heads w, w + 4, ..) into LDS; the workgroup whose chunk holds the
//    new position builds that K row (norm + RoPE) and V row in LDS, uses them
//    in place of the cache rows and writes them to the cache.
//  - Scores to LDS, per-head max and sum (wave = head), exp weights to LDS,
//    PV per wave over its 16 positions for every head, the four waves' sums
//    added in order; partial output, max and sum per chunk as
//    attn_partial_kernel (attn_combine_kernel combines the chunks; a
//    cross-workgroup combine inside this launch costs more than the second
//    launch).
template <int G>
__global__ __launch_bounds__(256) void attn_fused_kernel(const uint16_t* q, const uint16_t* knew,
                                                         const uint16_t* vnew, const uint16_t* qw,
                                                         const uint16_t* kw, uint16_t* kcache, uint16_t* vcache,
                                                         float* po, float* pml, const int32_t* pos_ptr, uint32_t kvh,
                                                         uint32_t cap, uint32_t nchunks, float scale, RopeTable rope,
                                                         float eps) {
    __shared__ __attribute__((aligned(16))) uint16_t qs[G][kHd];  // rotated queries, bf16
    __shared__ __attribute__((aligned(16))) uint16_t nk[kHd];     // the new position's K row (rotated), bf16
    __shared__ uint16_t nv[kHd];                                   // and its V row
    __shared__ float sc[G][kChunk];                                // scores, then exp weights
    __shared__ __attribute__((aligned(16))) float ew[kChunk][G];   // exp weights, position-major
    __shared__ float part[4][G][kHd];                              // per-wave PV sums
    const uint32_t g = blockIdx.x, c = blockIdx.y, t = threadIdx.x, lane = t & 63, w = t >> 6;
    const uint32_t p0 = c * kChunk;
    const uint32_t pr = 16 * w + (lane >> 2), d4 = lane & 3;  // this lane's score row and dim quarter
    // K and V of the chunk, loaded before the position is known (rows past the
    // context and the new position's stale row are loaded and not used)
    // Every load that does not need the position goes first: the group's
    // queries, the new K and V rows, the norm weights, then the chunk's K and
    // V (rows past the context and the new position's stale row are loaded
    // and not used). The position's scalar load then shares their round trip.
    constexpr int kQH = (G + 3) / 4;  // query heads per wave
    uint16_t qa[kQH], qb[kQH];
#pragma unroll
    for (int i = 0; i < kQH; ++i) {
        const uint32_t h = min(w + 4 * i, (uint32_t)G - 1);
        qa[i] = q[(size_t)(g * G + h) * kHd + lane];
        qb[i] = q[(size_t)(g * G + h) * kHd + lane + 64];
    }
    const uint16_t qwa = qw[lane], qwb = qw[lane + 64], kwa = kw[lane], kwb = kw[lane + 64];
    const uint16_t kna = knew[(size_t)g * kHd + lane], knb = knew[(size_t)g * kHd + lane + 64];
    const uint16_t vna = vnew[(size_t)g * kHd + lane], vnb = vnew[(size_t)g * kHd + lane + 64];
    uint4 kq[4];
    uint32_t vp[16];
    {
        const size_t base = (size_t)g * cap + p0;
        const uint4* kr = (const uint4*)(kcache + (base + min(pr, cap - 1 - p0)) * kHd + 32 * d4);
#pragma unroll
        for (int i = 0; i < 4; ++i) kq[i] = kr[i];
        const uint32_t* vr = (const uint32_t*)(vcache + base * kHd) + lane;
#pragma unroll
        for (int j = 0; j < 16; ++j) vp[j] = vr[(size_t)min(16 * w + j, cap - 1 - p0) * (kHd / 2)];
    }
    const int32_t pos = *pos_ptr;
    const uint32_t len = min((uint32_t)pos + 1, cap);
    if (p0 >= len) return;  // chunk past the context
    const uint32_t np = min((uint32_t)kChunk, len - p0);
    const bool own_row = (uint32_t)pos < cap && (uint32_t)pos >= p0 && (uint32_t)pos < p0 + kChunk;
#pragma unroll
    for (int i = 0; i < kQH; ++i) {  // query head g*G + w + 4 i: norm + RoPE
        const uint32_t h = w + 4 * i;
        if (h < (uint32_t)G) {
            uint16_t ra, rb;
            norm_rope_pair(bf(qa[i]), bf(qb[i]), qwa, qwb, lane, pos, rope, eps, ra, rb);
            qs[h][lane] = ra;
            qs[h][lane + 64] = rb;
        }
    }
    if (own_row && w == 0) {  // the new position's K (norm + RoPE) and V rows
        uint16_t ra, rb;
        norm_rope_pair(bf(kna), bf(knb), kwa, kwb, lane, pos, rope, eps, ra, rb);
        const uint16_t va = vna, vb = vnb;
        nk[lane] = ra;
        nk[lane + 64] = rb;
        nv[lane] = va;
        nv[lane + 64] = vb;
        const size_t crow = ((size_t)g * cap + (uint32_t)pos) * kHd;
        kcache[crow + lane] = ra;
        kcache[crow + lane + 64] = rb;
        vcache[crow + lane] = va;
        vcache[crow + lane + 64] = vb;
    }
    __syncthreads();
    if (own_row) {
        const uint32_t r = (uint32_t)pos - p0;
        if (pr == r) {
#pragma unroll
            for (int i = 0; i < 4; ++i) kq[i] = ((const uint4*)nk)[4 * d4 + i];
        }
        if (r >= 16 * w && r < 16 * w + 16) {
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (16 * w + j == r) vp[j] = ((const uint32_t*)nv)[lane];
        }
    }
    // scores: the lane's 32 dims for every head, the four quarters added by
    // DPP quad permutes ((d0 + d1) + (d2 + d3) in every lane)
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const uint4* qq = (const uint4*)qs[h] + 4 * d4;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 u = qq[i];
            acc = dot2_bf16(kq[i].x, u.x, acc);
            acc = dot2_bf16(kq[i].y, u.y, acc);
            acc = dot2_bf16(kq[i].z, u.z, acc);
            acc = dot2_bf16(kq[i].w, u.w, acc);
        }
        acc += dpp_f32<0xB1>(acc);  // quad_perm [1, 0, 3, 2]
        acc += dpp_f32<0x4E>(acc);  // quad_perm [2, 3, 0, 1]
        if (d4 == 0) sc[h][pr] = pr < np ? acc * scale : -INFINITY;
    }
    __syncthreads();
    // per head: max, exp weights and their sum (lane = position)
    for (uint32_t h = w; h < (uint32_t)G; h += 4) {
        const float sv = sc[h][lane];
        const float m = wave_max_dpp(sv);
        const float e = lane < np ? __expf(sv - m) : 0.0f;
        const float l = wave_sum_dpp(e);
        ew[lane][h] = e;
        if (lane == 0) *(float2*)&pml[((size_t)(g * G + h) * nchunks + c) * 2] = float2{m, l};
    }
    __syncthreads();
    // PV over the wave's 16 positions for every head: dims 2 lane, 2 lane + 1
    float o0[G], o1[G];
#pragma unroll
    for (int h = 0; h < G; ++h) o0[h] = o1[h] = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t p = 16 * w + j;
        if (p < np) {
            const float va = __uint_as_float(vp[j] << 16), vb = __uint_as_float(vp[j] & 0xffff0000u);
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float e = ew[p][h];
                o0[h] = fmaf(e, va, o0[h]);
                o1[h] = fmaf(e, vb, o1[h]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) *(float2*)&part[w][h][2 * lane] = float2{o0[h], o1[h]};
    __syncthreads();
    for (uint32_t o = t; o < (uint32_t)G * kHd / 2; o += 256) {  // (head, dim pair): waves in order
        const uint32_t h = o / (kHd / 2), dp = 2 * (o % (kHd / 2));
        const float2 a = *(const float2*)&part[0][h][dp], b = *(const float2*)&part[1][h][dp];
        const float2 cc = *(const float2*)&part[2][h][dp], dd = *(const float2*)&part[3][h][dp];
        const size_t prow = (size_t)(g * G + h) * nchunks + c;
        *(float2*)&po[prow * kHd + dp] = float2{(a.x + b.x) + (cc.x + dd.x), (a.y + b.y) + (cc.y + dd.y)};
    }
}

// Combine the chunks of each query head: out = sum_c o_c e^(m_c - m) / sum_c l_c e^(m_c - m).
// Workgroup (head, quarter of the dims), 256 threads: dim 32 quarter + t % 32
// and chunk group t / 32 (chunks t / 32, t / 32 + 8, ..). The partial outputs
// of the first 16 chunks per group and the first 256 chunk statistics are
// loaded before the position is known; each group's weighted sum goes to LDS
// and the eight groups are added in order.
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* po, const float* pml, uint16_t* out,
                                                           const int32_t* pos_ptr, uint32_t nchunks, uint32_t cap) {
    constexpr int kCG = 8, kPre = 16;
    __shared__ float fs[kMaxChunks];
    __shared__ float part[kCG][32];
    __shared__ float red[4];
    const uint32_t h = blockIdx.x, t = threadIdx.x, wv = t >> 6, cg = t >> 5, d = 32 * blockIdx.y + (t & 31);
    const float* col = po + (size_t)h * nchunks * kHd + d;
    float pre[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
        const uint32_t cc = cg + kCG * j;
        pre[j] = cc < nchunks ? col[(size_t)cc * kHd] : 0.0f;
    }
    const float2* ml = (const float2*)pml + (size_t)h * nchunks;
    const float2 ml0 = t < nchunks ? ml[t] : float2{0.0f, 0.0f};
    const uint32_t len = min((uint32_t)*pos_ptr + 1, cap);
    const uint32_t nc = min(nchunks, (len + kChunk - 1) / kChunk);
    float mx = t < nc ? ml0.x : -INFINITY;
    for (uint32_t cc = t + 256; cc < nc; cc += 256) mx = fmaxf(mx, ml[cc].x);
    mx = wave_max_dpp(mx);
    if ((t & 63) == 0) red[wv] = mx;
    __syncthreads();
    const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.0f;
    for (uint32_t cc = t; cc < nc; cc += 256) {
        const float2 v = cc == t ? ml0 : ml[cc];
        const float f = __expf(v.x - m);
        fs[cc] = f;
        l = fmaf(v.y, f, l);
    }
    l = wave_sum_dpp(l);
    if ((t & 63) == 0) red[wv] = l;
    __syncthreads();
    l = (red[0] + red[1]) + (red[2] + red[3]);
    float o = 0.0f;
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
        const uint32_t cc = cg + kCG * j;
        if (cc < nc) o = fmaf(pre[j], fs[cc], o);
    }
    for (uint32_t cc = cg + kCG * kPre; cc < nc; cc += kCG) o = fmaf(col[(size_t)cc * kHd], fs[cc], o);
    part[cg][t & 31] = o;
    __syncthreads();
    if (t < 32) {
        float sum = 0.0f;
#pragma unroll
        for (int gi = 0; gi < kCG; ++gi) sum += part[gi][t];
        out[(size_t)h * kHd + d] = to_bf(sum / l);
    }
}

// a = silu(g) * u in bf16 steps (gated_act_mul semantics), silu(g) = g / (1 +
// e^-g) with the hardware exp2 and reciprocal, each rounding on
// v_cvt_pk_bf16_f32: the operations of the products' SiLU-gate prologue.
__global__ void silu_mul_kernel(const uint16_t* g, const uint16_t* u, uint16_t* out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = bf(g[i]);
    const float s = bf(hw_bf(x * __builtin_amdgcn_rcpf(1.0f + __expf(-x))));
    out[i] = hw_bf(s * bf(u[i]));
}

// Greedy token: index of the largest logit (lowest index on ties), one
// workgroup of 1024 threads; then the next position.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, uint32_t n, int32_t* token,
                                                      int32_t* pos, int32_t* history, uint32_t hist) {
    __shared__ float bv[16];
    __shared__ uint32_t bi[16];
    const uint32_t t = threadIdx.x;
    float best = -INFINITY;
    uint32_t idx = 0xffffffffu;
    // 16-byte loads, eight in flight per thread; a thread sees its indices in
    // increasing order, so the strict > keeps the lowest index of a tie
    const uint32_t n4 = n / 4;
    const float4* l4 = (const float4*)logits;
#pragma unroll 8
    for (uint32_t c = t; c < n4; c += 1024) {
        const float4 v = l4[c];
        const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (e[q] > best) {
                best = e[q];
                idx = 4 * c + q;
            }
    }
    for (uint32_t i = 4 * n4 + t; i < n; i += 1024) {
        const float v = logits[i];
        if (v > best) {
            best = v;
            idx = i;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const uint32_t oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) {
            best = ov;
            idx = oi;
        }
    }
    if ((t & 63) == 0) {
        bv[t >> 6] = best;
        bi[t >> 6] = idx;
    }
    __syncthreads();
    if (t == 0) {
        float b = bv[0];
        uint32_t ix = bi[0];
        for (int w = 1; w < 16; ++w)
            if (bv[w] > b || (bv[w] == b && bi[w] < ix)) {
                b = bv[w];
                ix = bi[w];
            }
        if (ix >= n) ix = 0;  // every logit NaN: keep the token in range
        *token = (int32_t)ix;
        const int32_t p = *pos;
        if ((uint32_t)p < hist) {  // the history holds hist entries; the position stops there
            history[p] = (int32_t)ix;
            *pos = p + 1;
        }
    }
}

// x = embedding row of *token (bf16 table [vocab][n]).
__global__ void embed_kernel(const uint16_t* table, const int32_t* token, uint16_t* x, uint32_t n, uint32_t vocab) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t tok = min((uint32_t)*token, vocab - 1);
    if (i < n) x[i] = table[(size_t)tok * n + i];
}

// Tagged residual row (bf16 | tag << 16 per word, for chained products):
// the embedding row of *token with tag ^ ((*seq & 1) << 15).
__global__ void embed_tagged_kernel(const uint16_t* table, const int32_t* token, uint32_t* x, uint32_t n,
                                    uint32_t vocab, uint32_t tag, const int32_t* seq) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t tok = min((uint32_t)*token, vocab - 1);
    const uint32_t t = (tag ^ (((uint32_t)*seq & 1u) << 15)) << 16;
    if (i < n) x[i] = (uint32_t)table[(size_t)tok * n + i] | t;
}

// out[i] = bf16 value of tagged word x[i]
__global__ void untag_kernel(const uint32_t* x, uint16_t* out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = (uint16_t)(x[i] & 0xffffu);
}

}  // namespace

extern "C" {

int stark_decode_embed_tagged(const void* table, const int32_t* token, void* x, uint32_t n, uint32_t vocab,
                              uint32_t tag, const int32_t* seq, void* stream) {
    if (vocab == 0 || tag == 0 || tag > 0x7fff) return 1;
    hipLaunchKernelGGL(embed_tagged_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)table, token, (uint32_t*)x, n, vocab, tag, seq);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_untag(const void* x, void* out, uint32_t n, void* stream) {
    hipLaunchKernelGGL(untag_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, (const uint32_t*)x,
                       (uint16_t*)out, n);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_rms_norm(const void* x, const void* w, void* out, uint32_t n, float eps, void* stream) {
    if (n % 256) return 1;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x,
                       (const uint16_t*)w, (uint16_t*)out, n, eps);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_qk_norm_rope(void* q, const void* k, const void* v, const void* qw, const void* kw, void* kcache,
                              void* vcache, const int32_t* pos, uint32_t qh, uint32_t kvh, uint32_t cap, float theta,
                              float eps, void* stream) {
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3(qh + kvh), dim3(64), 0, (hipStream_t)stream, (uint16_t*)q,
                       (const uint16_t*)k, (const uint16_t*)v, (const uint16_t*)qw, (const uint16_t*)kw,
                       (uint16_t*)kcache, (uint16_t*)vcache, pos, qh, kvh, cap, rope_table(theta), eps);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

uint32_t stark_decode_attn_chunks(uint32_t cap) { return (cap + kChunk - 1) / kChunk; }

int stark_decode_attention(const void* q, const void* kcache, const void* vcache, float* po, float* pml, void* out,
                           const int32_t* pos, uint32_t qh, uint32_t kvh, uint32_t cap, void* stream) {
    if (kvh == 0 || qh % kvh || cap == 0) return 1;
    const uint32_t nchunks = (cap + kChunk - 1) / kChunk, G = qh / kvh;
    const float scale = 1.0f / sqrtf((float)kHd);
    hipStream_t s = (hipStream_t)stream;
    if (nchunks > (uint32_t)kMaxChunks) return 1;
    const dim3 grid(kvh, nchunks);
#define QMM_ATTN(GG)                                                                                              \
    hipLaunchKernelGGL(attn_partial_kernel<GG>, grid, dim3(64 * GG), 0, s, (const uint16_t*)q, (const uint16_t*)kcache, \
                       (const uint16_t*)vcache, po, pml, pos, kvh, cap, nchunks, scale)
    switch (G) {
    case 1: QMM_ATTN(1); break;
    case 2: QMM_ATTN(2); break;
    case 4: QMM_ATTN(4); break;
    case 8: QMM_ATTN(8); break;
    default: return 1;
    }
#undef QMM_ATTN
    hipLaunchKernelGGL(attn_reduce_kernel, dim3(qh), dim3(kHd), 0, s, po, pml, (uint16_t*)out, pos, nchunks, cap);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_attention_fused(const void* q, const void* k, const void* v, const void* qw, const void* kw,
                                 void* kcache, void* vcache, float* po, float* pml, void* out, const int32_t* pos,
                                 uint32_t qh, uint32_t kvh, uint32_t cap, float theta, float eps, void* stream) {
    if (kvh == 0 || qh % kvh || cap == 0) return 1;
    if ((cap + kChunk - 1) / kChunk > (uint32_t)kMaxChunks) return 1;
    const uint32_t nchunks = (cap + kChunk - 1) / kChunk, G = qh / kvh;
    const float scale = 1.0f / sqrtf((float)kHd);
    const RopeTable rope = rope_table(theta);
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(kvh, nchunks);
#define QMM_ATTN_F(GG)                                                                                          \
    hipLaunchKernelGGL(attn_fused_kernel<GG>, grid, dim3(256), 0, s, (const uint16_t*)q, (const uint16_t*)k, \
                       (const uint16_t*)v, (const uint16_t*)qw, (const uint16_t*)kw, (uint16_t*)kcache,          \
                       (uint16_t*)vcache, po, pml, pos, kvh, cap, nchunks, scale, rope, eps)
    switch (G) {
    case 1: QMM_ATTN_F(1); break;
    case 2: QMM_ATTN_F(2); break;
    case 4: QMM_ATTN_F(4); break;
    case 8: QMM_ATTN_F(8); break;
    default: return 1;
    }
#undef QMM_ATTN_F
    hipLaunchKernelGGL(attn_combine_kernel, dim3(qh, kHd / 32), dim3(256), 0, s, po, pml, (uint16_t*)out, pos, nchunks, cap);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_silu_mul(const void* g, const void* u, void* out, uint32_t n, void* stream) {
    hipLaunchKernelGGL(silu_mul_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)g, (const uint16_t*)u, (uint16_t*)out, n);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_argmax(const float* logits, uint32_t n, int32_t* token, int32_t* pos, int32_t* history,
                        uint32_t hist, void* stream) {
    hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, logits, n, token, pos, history,
                       hist);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

int stark_decode_embed(const void* table, const int32_t* token, void* x, uint32_t n, uint32_t vocab, void* stream) {
    if (vocab == 0) return 1;
    hipLaunchKernelGGL(embed_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       (const uint16_t*)table, token, (uint16_t*)x, n, vocab);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

}  // extern "C"
