// Token sampling after the lm_head (UnifiedSampling,
// crates/stark-engine/src/backends/cpu/kernel/sampling/unified_sampling.rs:14-117;
// noise crates/stark-engine/src/encodable_block/sampling/gumbel.rs):
// non-finite rows give u32::MAX; the bitmask sends masked tokens to -inf; the
// temperature scales (after a uniform shift that puts the maximum at zero when
// scaling would overflow a finite logit); top-k / top-p / min-p keep a prefix
// of the logits sorted by value (ties: lower index first); a seeded row adds
// Gumbel noise -ln(-ln u), u from Philox4x32-10; the result is the argmax
// (ties: lower index), or u32::MAX when no finite logit is left.
//
// One workgroup of 1024 threads per row, in passes over the row (L2-resident):
//  - the prefix kept by the filters has length L, the minimum of top_k, the
//    count of logits at or above max + ln(min_p), and for top-p the first
//    prefix whose mass reaches p. Top-p follows the reference's f32 sums in
//    its order: only terms exp(x - max) of at least 2^-27 can move them, and
//    when at most 4096 logits carry such terms they are sorted in LDS and
//    summed in order on one thread (exact_top_p_prefix). Rows with more
//    significant terms (very flat rows) take a radix descent over the
//    order-preserving key with per-digit mass histograms in 2^-40 fixed
//    point (integer atomics: independent of thread timing), which differs
//    from the sequential f32 sums only where the prefix mass lands within
//    their rounding error of p;
//  - the kept set, the first L logits in (value desc, index asc) order, is
//    located by a second radix select over the key (and over the index among
//    equal keys);
//  - the final pass scores kept logits (+ noise) and takes the argmax.
// Without noise the filters cannot change the argmax (the maximum is always
// kept), so a greedy row is one max/argmax pass.
#include <cmath>

#include "qmm_common.h"

namespace qmm {
namespace {

constexpr int kST = 1024;  // threads per row

struct SampleArgs {
    const void* logits;
    uint32_t* out;
    const uint64_t* seeds;
    const uint32_t* bitmask;
    uint32_t vocab, dt;
    uint32_t has_temperature, has_top_k, has_top_p, has_min_p;
    float temperature, top_p, min_p;
    uint32_t top_k;
};

struct SampleLds {
    unsigned long long hist[256];  // mass (fixed point) or counts per digit
    unsigned long long acc64[2];
    float redf[kST / 64];
    uint32_t redi[kST / 64];
    uint32_t flag;
    uint32_t scal[4];
};

// Philox4x32-10 (Salmon et al., SC'11; the constants are the published ones)
__device__ __forceinline__ uint32_t philox_word(uint32_t offset, uint32_t word, uint64_t seed) {
    uint32_t c0 = offset, c1 = 0, c2 = 0, c3 = 0;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) {
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
    }
    return word == 0 ? c0 : word == 1 ? c1 : word == 2 ? c2 : c3;
}

// gumbel.rs:49-79 (revidx maps a logit to its Philox counter and word)
__device__ __forceinline__ float gumbel(uint64_t seed, uint32_t i, uint32_t vocab) {
    const uint32_t t = i % 1024u, blk = i / 1024u;
    const uint32_t offset = ((vocab + 4095u) / 4096u) * t + blk / 4u;
    uint32_t v = philox_word(offset, blk % 4u, seed) >> 8;
    v = v < 1u ? 1u : v;
    const float u = (float)v * (1.0f / 16777216.0f);
    return -logf(-logf(u));
}

// Top-p in the reference's order: terms of at least 2^-27 (times the maximum's)
// sorted in LDS, at most kExactCap of them.
constexpr int kExactCap = 4096;
constexpr float kSignificant = 0x1p-27f;

struct ExactLds {
    unsigned long long key[kExactCap];  // fkey(x) << 32 | ~index: descending = (value desc, index asc)
    float term[kExactCap];
    float norm;
    uint32_t n, len;
};

// order-preserving key of a non-NaN float (larger float -> larger key)
__device__ __forceinline__ uint32_t fkey(float f) {
    const uint32_t b = __float_as_uint(f + 0.0f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ float logit_at(const SampleArgs& a, size_t row, uint32_t i) {
    return load_as_f32(a.logits, a.dt, row * a.vocab + i);
}

// block reductions (every thread gets the result)
__device__ float block_max(float v, SampleLds& s) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s.redf[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = s.redf[0];
    for (int w = 1; w < kST / 64; ++w) m = fmaxf(m, s.redf[w]);
    return m;
}

__device__ uint32_t block_or(uint32_t v, SampleLds& s) {
    __syncthreads();
    if (threadIdx.x == 0) s.flag = 0;
    __syncthreads();
    if (v) atomicOr(&s.flag, 1u);
    __syncthreads();
    return s.flag;
}

__device__ uint32_t block_min_u32(uint32_t v, SampleLds& s) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = min(v, (uint32_t)__shfl_xor((int)v, o, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) s.redi[threadIdx.x >> 6] = v;
    __syncthreads();
    uint32_t m = s.redi[0];
    for (int w = 1; w < kST / 64; ++w) m = min(m, s.redi[w]);
    return m;
}

__device__ unsigned long long block_sum_u64(unsigned long long v, SampleLds& s) {
    __syncthreads();
    if (threadIdx.x == 0) s.acc64[0] = 0;
    __syncthreads();
    atomicAdd(&s.acc64[0], v);
    __syncthreads();
    return s.acc64[0];
}

__device__ __forceinline__ float fkey_value(uint32_t k) {
    return (k & 0x80000000u) ? __uint_as_float(k & 0x7fffffffu) : __uint_as_float(~k);
}

// Length of the top-p prefix as unified_sampling.rs:85-97 computes it: the
// norm is the f32 sum of exp(x - max) over the logits sorted by value desc
// (index asc), the mass adds exp(x - max) / norm in that order, and the prefix
// ends before the first logit at which the mass has reached p. C is the count
// of significant terms (see the caller); returns V when the mass never
// reaches p.
template <class ValueFn>
__device__ uint32_t exact_top_p_prefix(const SampleArgs& a, ValueFn value, float F, uint32_t C, uint32_t V,
                                       SampleLds& s) {
    __shared__ ExactLds ex;
    const uint32_t tid = threadIdx.x;
    uint32_t N = 1;
    while (N < C) N <<= 1;
    __syncthreads();
    if (tid == 0) ex.n = 0;
    __syncthreads();
    for (uint32_t i = tid; i < V; i += kST) {
        const float x = value(i);
        if (expf(x - F) >= kSignificant)
            ex.key[atomicAdd(&ex.n, 1u)] = ((unsigned long long)fkey(x) << 32) | (0xffffffffu - i);
    }
    for (uint32_t j = C + tid; j < N; j += kST) ex.key[j] = 0;  // below every real key
    __syncthreads();
    // bitonic sort, descending
    for (uint32_t k = 2; k <= N; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i = tid; i < N; i += kST) {
                const uint32_t o = i ^ j;
                if (o > i) {
                    const unsigned long long u = ex.key[i], w = ex.key[o];
                    if ((i & k) == 0 ? u < w : u > w) {
                        ex.key[i] = w;
                        ex.key[o] = u;
                    }
                }
            }
            __syncthreads();
        }
    for (uint32_t r = tid; r < C; r += kST) ex.term[r] = expf(fkey_value((uint32_t)(ex.key[r] >> 32)) - F);
    __syncthreads();
    if (tid == 0) {
        float norm = 0.0f;
        for (uint32_t r = 0; r < C; ++r) norm += ex.term[r];
        ex.norm = norm;
    }
    __syncthreads();
    const float norm = ex.norm;
    for (uint32_t r = tid; r < C; r += kST) ex.term[r] = ex.term[r] / norm;
    __syncthreads();
    if (tid == 0) {
        float mass = 0.0f;
        uint32_t len = V;
        for (uint32_t r = 0; r < C; ++r) {
            if (mass >= a.top_p) {
                len = r;
                break;
            }
            mass += ex.term[r];
        }
        if (len == V && mass >= a.top_p) len = C;
        ex.len = len;
    }
    __syncthreads();
    (void)s;
    return ex.len;
}

__global__ __launch_bounds__(kST) void unified_sampling(SampleArgs a) {
    __shared__ SampleLds s;
    const size_t row = blockIdx.x;
    const uint32_t tid = threadIdx.x, V = a.vocab, words = (V + 31u) / 32u;
    const uint32_t* bm = a.bitmask ? a.bitmask + row * words : nullptr;
    const bool masked_row = bm != nullptr;
    const auto masked = [&](uint32_t i) { return masked_row && ((bm[i / 32] >> (i % 32)) & 1u) == 0; };

    // ---- pass A: finiteness; masked max and the temperature's overflow check
    const float recip = a.has_temperature ? 1.0f / a.temperature : 1.0f;
    uint32_t bad = 0, over = 0;
    float m0 = -INFINITY;
    for (uint32_t i = tid; i < V; i += kST) {
        float x = logit_at(a, row, i);
        if (!__builtin_isfinite(x)) bad = 1;
        if (masked(i)) x = -INFINITY;
        m0 = fmaxf(m0, x);
        if (__builtin_isfinite(x) && !__builtin_isfinite(x * recip)) over = 1;
    }
    if (block_or(bad, s)) {
        if (tid == 0) a.out[row] = 0xffffffffu;
        return;
    }
    const bool center = a.has_temperature && block_or(over, s);
    const float shift = center ? block_max(m0, s) : 0.0f;
    const auto value = [&](uint32_t i) {
        float x = masked(i) ? -INFINITY : logit_at(a, row, i);
        if (a.has_temperature) {
            if (center) x -= shift;
            x *= recip;
        }
        return x;
    };

    // ---- pass B: maximum and its lowest index
    float fmx = -INFINITY;
    for (uint32_t i = tid; i < V; i += kST) fmx = fmaxf(fmx, value(i));
    const float F = block_max(fmx, s);
    if (!a.seeds) {
        uint32_t best = 0xffffffffu;
        for (uint32_t i = tid; i < V; i += kST)
            if (value(i) == F) best = min(best, i);
        best = block_min_u32(best, s);
        if (tid == 0) a.out[row] = __builtin_isfinite(F) ? best : 0xffffffffu;
        return;
    }

    // ---- kept prefix length L (in sorted order)
    uint32_t L = V;
    if (a.has_top_k) L = min(L, a.top_k);
    if (a.has_min_p) {
        const float thr = F + logf(a.min_p);
        unsigned long long c = 0;
        for (uint32_t i = tid; i < V; i += kST) c += value(i) >= thr ? 1u : 0u;
        L = min(L, (uint32_t)block_sum_u64(c, s));
    }
    if (a.has_top_p && L > 1) {
        // Terms exp(x - max) below 2^-27 cannot move the reference's sequential
        // f32 sums: the norm is at least 1 (the maximum's own term), and a
        // running mass m is at least 1 / norm, so such a term (or its quotient
        // by the norm) is below half an ulp of the running value and every
        // later one is smaller still. When the terms at or above 2^-27 fit in
        // LDS, they are sorted (value desc, index asc) and both sums run in the
        // reference's order on one thread, which gives its prefix exactly.
        uint32_t cnt = 0;
        for (uint32_t i = tid; i < V; i += kST) cnt += expf(value(i) - F) >= kSignificant ? 1u : 0u;
        const uint32_t C = (uint32_t)block_sum_u64(cnt, s);
        if (C <= (uint32_t)kExactCap) {
            L = min(L, exact_top_p_prefix(a, value, F, C, V, s));
        } else {
            const double kFix = 1099511627776.0;  // 2^40
            const auto term = [&](float x) { return (unsigned long long)((double)expf(x - F) * kFix); };
            unsigned long long z = 0;
            for (uint32_t i = tid; i < V; i += kST) z += term(value(i));
            const unsigned long long norm = block_sum_u64(z, s);
            const unsigned long long target = (unsigned long long)ceil((double)a.top_p * (double)norm);
            // radix descent: prefix of the key bits fixed so far, and the mass of
            // every logit above the current bucket
            uint32_t prefix = 0, pmask = 0;
            unsigned long long above = 0;
            bool found = false;
            for (int shiftb = 24; shiftb >= 0; shiftb -= 8) {
                __syncthreads();
                if (tid < 256) s.hist[tid] = 0;
                __syncthreads();
                for (uint32_t i = tid; i < V; i += kST) {
                    const float x = value(i);
                    const uint32_t k = fkey(x);
                    if ((k & pmask) == prefix) atomicAdd(&s.hist[(k >> shiftb) & 255u], term(x));
                }
                __syncthreads();
                if (tid == 0) {
                    uint32_t d = 256;
                    unsigned long long acc = above;
                    for (int b = 255; b >= 0; --b) {
                        if (acc + s.hist[b] >= target) {
                            d = (uint32_t)b;
                            break;
                        }
                        acc += s.hist[b];
                    }
                    s.scal[0] = d;
                    s.acc64[1] = acc;
                }
                __syncthreads();
                const uint32_t d = s.scal[0];
                if (d == 256) break;  // the whole row's mass stays below p: every logit is kept
                above = s.acc64[1];
                prefix |= d << shiftb;
                pmask |= 255u << shiftb;
                found = shiftb == 0;
            }
            if (found) {
                // logits with key == prefix all carry the same term t; the prefix
                // ends at the first of them whose addition reaches the target
                const float xk = (prefix & 0x80000000u) ? __uint_as_float(prefix & 0x7fffffffu) : __uint_as_float(~prefix);
                const unsigned long long t = term(xk);
                unsigned long long greater = 0;
                for (uint32_t i = tid; i < V; i += kST) greater += fkey(value(i)) > prefix ? 1u : 0u;
                greater = block_sum_u64(greater, s);
                const unsigned long long need = t ? (target - above + t - 1) / t : 1ull;  // ties up to the crossing one
                L = min(L, (uint32_t)min<unsigned long long>(greater + need, V));
            }
        }
    }
    L = max(L, 1u);

    // ---- the kept set: the L largest keys (ties by lower index), by radix select
    uint32_t kprefix = 0, kmask = 0, rank = L;  // rank: 1-based position wanted within the current bucket
    for (int shiftb = 24; shiftb >= 0; shiftb -= 8) {
        __syncthreads();
        if (tid < 256) s.hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < V; i += kST) {
            const uint32_t k = fkey(value(i));
            if ((k & kmask) == kprefix) atomicAdd(&s.hist[(k >> shiftb) & 255u], 1ull);
        }
        __syncthreads();
        if (tid == 0) {
            uint32_t r = rank, d = 0;
            for (int b = 255; b >= 0; --b) {
                if (s.hist[b] >= r) {
                    d = (uint32_t)b;
                    break;
                }
                r -= (uint32_t)s.hist[b];
            }
            s.scal[0] = d;
            s.scal[1] = r;
        }
        __syncthreads();
        kprefix |= s.scal[0] << shiftb;
        kmask |= 255u << shiftb;
        rank = s.scal[1];
    }
    // among logits with key == kprefix, the first `rank` by index are kept:
    // the rank-th smallest index, by radix select over the index bits
    uint32_t iprefix = 0, imask = 0;
    for (int shiftb = 24; shiftb >= 0; shiftb -= 8) {
        __syncthreads();
        if (tid < 256) s.hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < V; i += kST)
            if (fkey(value(i)) == kprefix && (i & imask) == iprefix) atomicAdd(&s.hist[(i >> shiftb) & 255u], 1ull);
        __syncthreads();
        if (tid == 0) {
            uint32_t r = rank, d = 0;
            for (uint32_t b = 0; b < 256; ++b) {
                if (s.hist[b] >= r) {
                    d = b;
                    break;
                }
                r -= (uint32_t)s.hist[b];
            }
            s.scal[0] = d;
            s.scal[1] = r;
        }
        __syncthreads();
        iprefix |= s.scal[0] << shiftb;
        imask |= 255u << shiftb;
        rank = s.scal[1];
    }

    // ---- scores of the kept logits with noise, argmax (lowest index on ties)
    const uint64_t seed = a.seeds[row];
    float best = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = tid; i < V; i += kST) {
        const float x = value(i);
        const uint32_t k = fkey(x);
        const bool kept = k > kprefix || (k == kprefix && i <= iprefix);
        const float sc = (kept ? x : -INFINITY) + gumbel(seed, i, V);
        if (sc > best) {  // strided ascending: the first maximum of this thread has the lowest index
            best = sc;
            bi = i;
        }
    }
    const float gb = block_max(best, s);
    uint32_t cand = best == gb ? bi : 0xffffffffu;
    cand = block_min_u32(cand, s);
    if (tid == 0) a.out[row] = __builtin_isfinite(gb) ? cand : 0xffffffffu;
}

}  // namespace
}  // namespace qmm

using namespace qmm;

extern "C" {

stark_qmm_status stark_qmm_unified_sampling(const stark_qmm_sampling_args* args, void* stream) {
    if (!args) return STARK_QMM_INVALID_ARGUMENT;
    if (args->struct_size != sizeof(stark_qmm_sampling_args)) return STARK_QMM_ABI_MISMATCH;
    const stark_qmm_sampling_args& x = *args;
    if (x.data_type != STARK_QMM_F32 && x.data_type != STARK_QMM_BF16) return STARK_QMM_UNSUPPORTED_DATA_TYPE;
    // SamplingMethod::validate (src/encodable_block/sampling/mod.rs:73-101)
    if (x.vocab_size == 0 || !x.logits || !x.output) return STARK_QMM_INVALID_ARGUMENT;
    if (x.has_temperature &&
        (!std::isfinite(x.temperature) || x.temperature <= 0.0f || !std::isfinite(1.0f / x.temperature)))
        return STARK_QMM_INVALID_ARGUMENT;
    if (x.has_top_k && (x.top_k == 0 || x.top_k > x.vocab_size)) return STARK_QMM_INVALID_ARGUMENT;
    if (x.has_top_p && (!std::isfinite(x.top_p) || x.top_p <= 0.0f || x.top_p > 1.0f)) return STARK_QMM_INVALID_ARGUMENT;
    if (x.has_min_p && (!std::isfinite(x.min_p) || x.min_p < 0.0f || x.min_p > 1.0f)) return STARK_QMM_INVALID_ARGUMENT;
    if (x.batch_size == 0) return STARK_QMM_OK;
    SampleArgs a{};
    a.logits = x.logits;
    a.out = x.output;
    a.seeds = x.seeds;
    a.bitmask = x.bitmask;
    a.vocab = x.vocab_size;
    a.dt = x.data_type;
    a.has_temperature = x.has_temperature;
    a.temperature = x.temperature;
    a.has_top_k = x.has_top_k;
    a.top_k = x.top_k;
    a.has_top_p = x.has_top_p;
    a.top_p = x.top_p;
    a.has_min_p = x.has_min_p;
    a.min_p = x.min_p;
    hipLaunchKernelGGL(unified_sampling, dim3(x.batch_size), dim3(kST), 0, (hipStream_t)stream, a);
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

}  // extern "C"
