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

namespace {

constexpr int kHd = 128;      // head dim
constexpr int kChunk = 128;   // attention positions per partial workgroup

__device__ __forceinline__ float bf(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

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

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// out = x * rsqrt(mean(x^2) + eps) * w, one row of n (n % 256 == 0), 256 threads.
__global__ __launch_bounds__(256) void rms_norm_kernel(const uint16_t* x, const uint16_t* w, uint16_t* out,
                                                       uint32_t n, float eps) {
    __shared__ float part[4];
    const uint32_t t = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t i = t; i < n; i += 256) {
        const float v = bf(x[i]);
        ss += v * v;
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)n + eps);
    for (uint32_t i = t; i < n; i += 256) out[i] = to_bf(bf(to_bf(bf(x[i]) * inv)) * bf(w[i]));
}

// Per-head RMSNorm of q and k, rotate-half RoPE at *pos, and the k/v write
// into the cache rows at *pos. Workgroup h < qh: query head h; else key/value
// head h - qh. 64 threads, each owning dims i and i + 64 (a rotation pair).
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                          const uint16_t* qw, const uint16_t* kw, uint16_t* kcache,
                                                          uint16_t* vcache, const int32_t* pos_ptr, uint32_t qh,
                                                          uint32_t kvh, uint32_t cap, float theta, float eps) {
    const uint32_t h = blockIdx.x, i = threadIdx.x;
    const int32_t pos = *pos_ptr;
    const bool is_q = h < qh;
    const uint16_t* src = is_q ? q + (size_t)h * kHd : k + (size_t)(h - qh) * kHd;
    const uint16_t* w = is_q ? qw : kw;
    const float a = bf(src[i]), b = bf(src[i + 64]);
    const float inv = 1.0f / sqrtf(wave_sum(a * a + b * b) / (float)kHd + eps);
    const float na = bf(to_bf(bf(to_bf(a * inv)) * bf(w[i])));
    const float nb = bf(to_bf(bf(to_bf(b * inv)) * bf(w[i + 64])));
    // inv_freq_i = theta^(-2i/hd), angle = pos * inv_freq_i
    const float freq = powf(theta, -2.0f * (float)i / (float)kHd);
    float sn, cs;
    sincosf((float)pos * freq, &sn, &cs);
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
// group's query heads against positions [c*kChunk, min(len, (c+1)*kChunk)),
// len = *pos + 1, and writes the unnormalised partial output with its max and
// sum. 256 threads; group size G = qh / kvh <= 8.
template <int G>
__global__ __launch_bounds__(256) void attn_partial_kernel(const uint16_t* q, const uint16_t* kcache,
                                                           const uint16_t* vcache, float* po, float* pml,
                                                           const int32_t* pos_ptr, uint32_t kvh, uint32_t cap,
                                                           uint32_t nchunks, float scale) {
    __shared__ float qs[G][kHd];
    __shared__ float w[G][kChunk];
    __shared__ float red[G][4];
    const uint32_t g = blockIdx.x, c = blockIdx.y, t = threadIdx.x;
    const uint32_t len = min((uint32_t)*pos_ptr + 1, cap);
    const uint32_t p0 = c * kChunk;
    float* out_o = po + ((size_t)(g * G) * nchunks + c) * kHd;
    if (p0 >= len) return;  // chunk past the context: the reduction skips it
    const uint32_t np = min((uint32_t)kChunk, len - p0);
    for (uint32_t e = t; e < G * kHd; e += 256) qs[e / kHd][e % kHd] = bf(q[(size_t)(g * G) * kHd + e]);
    __syncthreads();
    // scores: thread t -> position t / 2, half t % 2 (64 dims)
    {
        const uint32_t p = t >> 1, half = t & 1;
        float s[G];
#pragma unroll
        for (int h = 0; h < G; ++h) s[h] = 0.0f;
        if (p < np) {
            const uint4* kr = (const uint4*)(kcache + ((size_t)g * cap + p0 + p) * kHd + half * 64);
#pragma unroll
            for (int v8 = 0; v8 < 8; ++v8) {
                const uint4 u = kr[v8];
                const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float k0 = __uint_as_float(wd[e] << 16), k1 = __uint_as_float(wd[e] & 0xffff0000u);
                    const uint32_t d = half * 64 + v8 * 8 + 2 * e;
#pragma unroll
                    for (int h = 0; h < G; ++h) s[h] = fmaf(qs[h][d], k0, fmaf(qs[h][d + 1], k1, s[h]));
                }
            }
        }
#pragma unroll
        for (int h = 0; h < G; ++h) {
            s[h] += __shfl_xor(s[h], 1, 64);
            if (half == 0 && p < kChunk) w[h][p] = p < np ? s[h] * scale : -INFINITY;
        }
    }
    __syncthreads();
    // per head: max and exp-sum over the chunk (threads 0..127 hold w[h][t])
    float m[G], l[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float v = t < kChunk ? w[h][t] : -INFINITY;
        v = wave_max(v);
        if ((t & 63) == 0) red[h][t >> 6] = v;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) m[h] = fmaxf(red[h][0], red[h][1]);
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float e = 0.0f;
        if (t < kChunk) {
            e = t < np ? __expf(w[h][t] - m[h]) : 0.0f;
            w[h][t] = e;
        }
        e = wave_sum(e);
        if ((t & 63) == 0) red[h][t >> 6] = e;
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) l[h] = red[h][0] + red[h][1];
    // PV: thread t -> dim t % 128, heads of parity t / 128
    {
        const uint32_t d = t % kHd, hp = t / kHd;
        float o[G / 2 > 0 ? G / 2 : 1];
#pragma unroll
        for (int q2 = 0; q2 < (G > 1 ? G / 2 : 1); ++q2) o[q2] = 0.0f;
        const uint16_t* vr = vcache + ((size_t)g * cap + p0) * kHd + d;
        for (uint32_t p = 0; p < np; ++p) {
            const float vv = bf(vr[(size_t)p * kHd]);
#pragma unroll
            for (int q2 = 0; q2 < (G > 1 ? G / 2 : 1); ++q2) {
                const int h = G > 1 ? 2 * q2 + hp : 0;
                o[q2] = fmaf(w[h][p], vv, o[q2]);
            }
        }
#pragma unroll
        for (int q2 = 0; q2 < (G > 1 ? G / 2 : 1); ++q2) {
            const int h = G > 1 ? 2 * q2 + hp : 0;
            if (G == 1 && hp) continue;
            po[((size_t)(g * G + h) * nchunks + c) * kHd + d] = o[q2];
        }
    }
    if (t < G) {
        pml[((size_t)(g * G + t) * nchunks + c) * 2 + 0] = m[t];
        pml[((size_t)(g * G + t) * nchunks + c) * 2 + 1] = l[t];
    }
    (void)out_o;
}

// Combine the chunks of each query head: out = sum_c o_c e^(m_c - m) / sum_c l_c e^(m_c - m).
__global__ __launch_bounds__(128) void attn_reduce_kernel(const float* po, const float* pml, uint16_t* out,
                                                          const int32_t* pos_ptr, uint32_t nchunks, uint32_t cap) {
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const uint32_t len = min((uint32_t)*pos_ptr + 1, cap);
    const uint32_t nc = min(nchunks, (len + kChunk - 1) / kChunk);
    float m = -INFINITY;
    for (uint32_t c = 0; c < nc; ++c) m = fmaxf(m, pml[((size_t)h * nchunks + c) * 2]);
    float l = 0.0f, o = 0.0f;
    for (uint32_t c = 0; c < nc; ++c) {
        const float f = __expf(pml[((size_t)h * nchunks + c) * 2] - m);
        l = fmaf(pml[((size_t)h * nchunks + c) * 2 + 1], f, l);
        o = fmaf(po[((size_t)h * nchunks + c) * kHd + d], f, o);
    }
    out[(size_t)h * kHd + d] = to_bf(o / l);
}

// a = silu(g) * u in bf16 steps (gated_act_mul semantics).
__global__ void silu_mul_kernel(const uint16_t* g, const uint16_t* u, uint16_t* out, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = bf(g[i]);
    const float s = bf(to_bf(x / (1.0f + __expf(-x))));
    out[i] = to_bf(s * bf(u[i]));
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
    for (uint32_t i = t; i < n; i += 1024) {
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

}  // namespace

extern "C" {

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
                       (uint16_t*)kcache, (uint16_t*)vcache, pos, qh, kvh, cap, theta, eps);
    return hipGetLastError() == hipSuccess ? 0 : 10;
}

uint32_t stark_decode_attn_chunks(uint32_t cap) { return (cap + kChunk - 1) / kChunk; }

int stark_decode_attention(const void* q, const void* kcache, const void* vcache, float* po, float* pml, void* out,
                           const int32_t* pos, uint32_t qh, uint32_t kvh, uint32_t cap, void* stream) {
    if (kvh == 0 || qh % kvh || cap == 0) return 1;
    const uint32_t nchunks = (cap + kChunk - 1) / kChunk, G = qh / kvh;
    const float scale = 1.0f / sqrtf((float)kHd);
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid(kvh, nchunks);
#define QMM_ATTN(GG)                                                                                              \
    hipLaunchKernelGGL(attn_partial_kernel<GG>, grid, dim3(256), 0, s, (const uint16_t*)q, (const uint16_t*)kcache, \
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
