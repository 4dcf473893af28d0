// Activation transforms around the quantized products, on gfx950:
//  - ActivationTransform (crates/stark-engine/src/backends/cpu/kernel/activation_transform/activation_transform.rs:48-156):
//    input RHT (x * factors, then the 32-point Walsh-Hadamard transform),
//    output RHT (transform, then * factors, optional bias), and symmetric int8
//    quantization of the input-RHT result (scale per 32/64/128 values, codes
//    in sequential or grouped-by-nibble order, optional int32 group sums);
//  - GatedActMul (crates/stark-engine/src/backends/cpu/kernel/gated_act_mul/gated_act_mul.rs:17-152):
//    value * activation(gate) in the storage type, optional clipping and SiLU
//    alpha, optional RHT and int8 quantization;
//  - the output-RHT D-op of the products (kernel.rs:287-300), which runs the
//    output transform in place on d and adds the bias after it.
// Work items are one thread each: a 32-value stripe, or a whole scale group
// (up to four stripes) when quantizing; the butterfly runs in registers in
// the reference's order (pairs (l, l|s) for s = 1, 2, .., 16), then the
// scale 1/sqrt(32) as the reference computes it, so every float matches the
// CPU restatement. These are small launches (one row of activations per
// token); the HBM-bound products stay the hot path.
#include "qmm_common.h"

// The reference evaluates `a * b + c` as a rounded product and a rounded sum;
// no contraction into fma here, so the floats match the CPU restatement.
#pragma clang fp contract(off)

namespace qmm {
namespace {

constexpr int kBlock = 32;  // HADAMARD_TRANSFORM_BLOCK_SIZE (gpu_types/hadamard_order.rs:1)

__device__ __forceinline__ float ld(const void* p, uint32_t dt, size_t i) { return load_as_f32(p, dt, i); }
__device__ __forceinline__ void st(void* p, uint32_t dt, size_t i, float v) { store_from_f32(p, dt, i, v); }
__device__ __forceinline__ float rnd(uint32_t dt, float v) {
    return dt == STARK_QMM_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(v)) : v;
}

// activation_transform/mod.rs:28-43
__device__ __forceinline__ void hadamard32(float (&v)[kBlock]) {
#pragma unroll
    for (int s = 1; s < kBlock; s <<= 1)
#pragma unroll
        for (int l = 0; l < kBlock; ++l)
            if ((l & s) == 0) {
                const float a = v[l], b = v[l | s];
                v[l] = a + b;
                v[l | s] = a - b;
            }
    const float scale = 1.0f / __fsqrt_rn((float)kBlock);
#pragma unroll
    for (int l = 0; l < kBlock; ++l) v[l] *= scale;
}

// Int8CodeLayout::index (matmul_a.rs:31-46)
__device__ __forceinline__ uint32_t code_index(bool grouped, uint32_t i) {
    if (!grouped) return i;
    const uint32_t o = i & 7u;
    return i - o + (o & 1u) * 4u + o / 2u;
}

// mod.rs:9-26 on one scale group; writes codes (layout order), the scale and
// the group sums of the sum groups inside it.
template <int SG>
__device__ __forceinline__ void quantize_group(const float (&t)[SG], uint32_t base, bool grouped, uint32_t sum_group,
                                               int8_t* q, float* scale_out, int32_t* sums) {
    float mn = INFINITY, mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < SG; ++i) {
        mn = fminf(mn, t[i]);
        mx = fmaxf(mx, t[i]);
    }
    const float m = fmaxf(fabsf(mn), fabsf(mx));
    const float divisor = (isfinite(m) && m > 0.0f) ? m / 127.0f : 1.0f;
    *scale_out = divisor;
    int32_t sum = 0;
#pragma unroll
    for (int i = 0; i < SG; ++i) {
        float r = roundf(t[i] / divisor);
        const int8_t c = isnan(r) ? (int8_t)0 : (int8_t)fminf(fmaxf(r, -127.0f), 127.0f);
        q[code_index(grouped, base + i)] = c;
        sum += c;
        if (sums && ((uint32_t)(i + 1) % sum_group) == 0) {
            sums[(base + i) / sum_group] = sum;
            sum = 0;
        }
    }
}

struct TransformArgs {
    const void* input;     // T, or NULL (in place: read fp_out)
    void* fp_out;          // T
    const void* bias;      // BiasT or NULL
    int8_t* q_out;
    float* scales_out;
    int32_t* sums_out;
    const int32_t* factors;
    uint32_t batch, count, op, grouped, scale_group, sum_group, t_dt, bias_dt;
};

// ActivationTransform: thread = (row, stripe) for the FP ops, (row, scale group)
// for the quantizing ops (SG values, SG / 32 stripes).
template <int SG>
__global__ __launch_bounds__(256) void activation_transform(TransformArgs a) {
    const uint32_t per_row = a.count / SG;
    const uint32_t item = blockIdx.x * 256 + threadIdx.x;
    if (item >= a.batch * per_row) return;
    const uint32_t row = item / per_row, g = item % per_row;
    const size_t ro = (size_t)row * a.count, k0 = (size_t)g * SG;
    const void* src = a.input ? a.input : a.fp_out;
    const bool input_rht = a.op != 1;
    float t[SG];
#pragma unroll
    for (int s = 0; s < SG / kBlock; ++s) {
        float v[kBlock];
#pragma unroll
        for (int l = 0; l < kBlock; ++l) {
            const float x = ld(src, a.t_dt, ro + k0 + s * kBlock + l);
            v[l] = input_rht ? x * (float)a.factors[k0 + s * kBlock + l] : x;
        }
        hadamard32(v);
#pragma unroll
        for (int l = 0; l < kBlock; ++l)
            t[s * kBlock + l] = input_rht ? v[l] : v[l] * (float)a.factors[k0 + s * kBlock + l];
    }
    if (a.op >= 2) {  // Quantize / QuantizeWithGroupSums
        quantize_group<SG>(t, (uint32_t)k0, a.grouped != 0, a.sum_group, a.q_out + ro,
                           a.scales_out + (size_t)row * per_row + g,
                           a.op == 3 ? a.sums_out + (size_t)row * (a.count / a.sum_group) : nullptr);
        return;
    }
#pragma unroll
    for (int i = 0; i < SG; ++i) {
        float v = t[i];
        if (a.bias) v = rnd(a.t_dt, v) + ld(a.bias, a.bias_dt, k0 + i);
        st(a.fp_out, a.t_dt, ro + k0 + i, v);
    }
}

// ActivationType::activate (gpu_types/activation_type.rs:19-111) on a value
// stored in dt; every bf16 operation of the materialized forms rounds.
__device__ __forceinline__ float activate(uint32_t type, float x, uint32_t dt, bool has_alpha, float alpha) {
    constexpr float K0 = 0.044715f, K1 = 0.7978846f;
    switch (type) {
    case STARK_QMM_ACT_SILU: {
        const float al = has_alpha ? alpha : 1.0f;
        return rnd(dt, x / (1.0f + expf(-al * x)));
    }
    case STARK_QMM_ACT_SILU_MATERIALIZED_SIGMOID: {
        const float e = rnd(dt, expf(fabsf(x)));
        const float lower = rnd(dt, 1.0f / rnd(dt, 1.0f + e));
        const float sig = x < 0.0f ? lower : rnd(dt, 1.0f - lower);
        return rnd(dt, x * sig);
    }
    case STARK_QMM_ACT_GELU_APPROX: {
        const float arg = K1 * (x + K0 * x * x * x);
        return rnd(dt, 0.5f * x * (1.0f + tanhf(arg)));
    }
    case STARK_QMM_ACT_GELU_MATERIALIZED_POLYNOMIAL: {
        const float cubic = rnd(dt, x * x * x);
        const float term = rnd(dt, rnd(dt, K0) * cubic);
        const float inner = rnd(dt, x + term);
        const float arg = rnd(dt, rnd(dt, K1) * inner);
        const float act = rnd(dt, tanhf(arg));
        return rnd(dt, rnd(dt, 0.5f * x) * rnd(dt, 1.0f + act));
    }
    case STARK_QMM_ACT_GELU_EXACT: return rnd(dt, 0.5f * x * (1.0f + erff(x * 0.70710677f)));
    case STARK_QMM_ACT_SOFTPLUS: return x > 20.0f ? x : rnd(dt, logf(1.0f + expf(x)));
    default: return x;  // identity
    }
}

__device__ __forceinline__ float clamp_f(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

struct GatedArgs {
    const void* act;
    const void* value;     // separate value operand, or NULL (interleaved)
    void* fp_out;
    int8_t* q_out;
    float* scales_out;
    int32_t* sums_out;
    const int32_t* factors;  // RHT signs or NULL
    uint32_t gated_dim, batch, value_offset, value_row_stride, act_type, has_alpha;
    float alpha, gate_min, gate_max, value_min, value_max;
    uint32_t clip_gate, clip_value, op, grouped, scale_group, sum_group, t_dt;
};

__device__ __forceinline__ float gated_one(const GatedArgs& a, size_t batch, uint32_t g) {
    size_t act_index;
    float value;
    if (!a.value) {
        const size_t base = batch * 2 * a.gated_dim;
        act_index = base + a.gated_dim + g;
        value = ld(a.act, a.t_dt, base + g);
    } else {
        act_index = batch * a.gated_dim + g;
        value = ld(a.value, a.t_dt, batch * a.value_row_stride + a.value_offset + g);
    }
    float gate = ld(a.act, a.t_dt, act_index);
    if (a.clip_gate) gate = rnd(a.t_dt, clamp_f(gate, a.gate_min, a.gate_max));
    const bool alpha = a.has_alpha && a.act_type == STARK_QMM_ACT_SILU;
    const float activated = activate(a.act_type, gate, a.t_dt, alpha, a.alpha);
    if (a.clip_value) value = rnd(a.t_dt, clamp_f(value, a.value_min, a.value_max));
    return rnd(a.t_dt, value * activated);
}

// GatedActMul: thread = one element (no RHT), one stripe (RHT, FP out) or one
// scale group (RHT + quantize).
template <int SG>
__global__ __launch_bounds__(256) void gated_act_mul(GatedArgs a) {
    const uint32_t per_row = a.factors ? a.gated_dim / SG : a.gated_dim;
    const uint32_t item = blockIdx.x * 256 + threadIdx.x;
    if (item >= a.batch * per_row) return;
    const size_t batch = item / per_row;
    const uint32_t g = item % per_row;
    if (!a.factors) {
        st(a.fp_out, a.t_dt, batch * a.gated_dim + g, gated_one(a, batch, g));
        return;
    }
    const uint32_t k0 = g * SG;
    float t[SG];
#pragma unroll
    for (int s = 0; s < SG / kBlock; ++s) {
        float v[kBlock];
#pragma unroll
        for (int l = 0; l < kBlock; ++l) {
            const uint32_t i = k0 + s * kBlock + l;
            v[l] = gated_one(a, batch, i) * (float)a.factors[i];
        }
        hadamard32(v);
#pragma unroll
        for (int l = 0; l < kBlock; ++l) t[s * kBlock + l] = v[l];
    }
    if (a.op != 0) {
        const uint32_t spr = a.gated_dim / SG;
        quantize_group<SG>(t, k0, a.grouped != 0, a.sum_group, a.q_out + batch * a.gated_dim,
                           a.scales_out + batch * spr + g,
                           a.op == 2 ? a.sums_out + batch * (a.gated_dim / a.sum_group) : nullptr);
        return;
    }
#pragma unroll
    for (int i = 0; i < SG; ++i) st(a.fp_out, a.t_dt, batch * a.gated_dim + k0 + i, t[i]);
}

template <template <int> class K, class Args>
stark_qmm_status launch_by_group(uint32_t sg, uint32_t items, const Args& a, hipStream_t stream) {
    if (items == 0) return STARK_QMM_OK;
    const dim3 grid((items + 255) / 256);
    switch (sg) {
    case 32: hipLaunchKernelGGL(K<32>::fn(), grid, dim3(256), 0, stream, a); break;
    case 64: hipLaunchKernelGGL(K<64>::fn(), grid, dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL(K<128>::fn(), grid, dim3(256), 0, stream, a); break;
    default: return STARK_QMM_INVALID_ARGUMENT;
    }
    QMM_HIP_CHECK(hipGetLastError());
    return STARK_QMM_OK;
}

template <int SG>
struct AT {
    static auto fn() { return activation_transform<SG>; }
};
template <int SG>
struct GA {
    static auto fn() { return gated_act_mul<SG>; }
};

bool float_dt(uint32_t dt) { return dt == STARK_QMM_F32 || dt == STARK_QMM_BF16; }

}  // namespace

stark_qmm_status launch_output_rht(void* d, uint32_t d_dt, const void* bias, uint32_t bias_dt,
                                   const int32_t* factors, uint32_t rows, uint32_t n, hipStream_t stream) {
    TransformArgs a{};
    a.fp_out = d;
    a.bias = bias;
    a.factors = factors;
    a.batch = rows;
    a.count = n;
    a.op = STARK_QMM_TRANSFORM_OUTPUT_RHT;
    a.t_dt = d_dt;
    a.bias_dt = bias_dt;
    return launch_by_group<AT>(32, rows * (n / 32), a, stream);
}

}  // namespace qmm

using namespace qmm;

extern "C" {

stark_qmm_status stark_qmm_activation_transform(const stark_qmm_activation_transform_args* args, void* stream) {
    if (!args || args->struct_size != sizeof(stark_qmm_activation_transform_args)) return STARK_QMM_ABI_MISMATCH;
    const stark_qmm_activation_transform_args& x = *args;
    if (x.op > STARK_QMM_TRANSFORM_QUANTIZE_WITH_GROUP_SUMS || !float_dt(x.data_type) ||
        (x.bias && !float_dt(x.bias_data_type)))
        return STARK_QMM_UNSUPPORTED_DATA_TYPE;
    if (!x.rht_factors || x.element_count % kBlock) return STARK_QMM_INVALID_ARGUMENT;
    const bool quantize = x.op >= STARK_QMM_TRANSFORM_QUANTIZE;
    uint32_t sg = kBlock;
    if (quantize) {
        // ActivationQuantization::new (activation_transform.rs:27-42)
        sg = x.scale_group_size;
        if (!(sg == 32 || sg == 64 || sg == 128) || x.element_count % sg || !x.q_out || !x.scales_out)
            return STARK_QMM_INVALID_ARGUMENT;
        if (x.op == STARK_QMM_TRANSFORM_QUANTIZE_WITH_GROUP_SUMS &&
            (!(x.sum_group_size == 32 || x.sum_group_size == 64 || x.sum_group_size == 128) ||
             x.sum_group_size > sg || !x.group_sums_out))
            return STARK_QMM_INVALID_ARGUMENT;
    } else if (!x.output) {
        return STARK_QMM_INVALID_ARGUMENT;
    }
    TransformArgs a{};
    a.input = x.in_place ? nullptr : x.input;
    if (!x.in_place && !x.input) return STARK_QMM_INVALID_ARGUMENT;
    a.fp_out = x.output;
    a.bias = x.bias;
    a.q_out = x.q_out;
    a.scales_out = x.scales_out;
    a.sums_out = x.group_sums_out;
    a.factors = x.rht_factors;
    a.batch = x.batch_size;
    a.count = x.element_count;
    a.op = x.op;
    a.grouped = x.grouped_by_nibble;
    a.scale_group = sg;
    a.sum_group = x.sum_group_size;
    a.t_dt = x.data_type;
    a.bias_dt = x.bias_data_type;
    return launch_by_group<AT>(sg, x.batch_size * (x.element_count / sg), a, (hipStream_t)stream);
}

stark_qmm_status stark_qmm_gated_act_mul(const stark_qmm_gated_act_mul_args* args, void* stream) {
    if (!args || args->struct_size != sizeof(stark_qmm_gated_act_mul_args)) return STARK_QMM_ABI_MISMATCH;
    const stark_qmm_gated_act_mul_args& x = *args;
    if (!float_dt(x.data_type)) return STARK_QMM_UNSUPPORTED_DATA_TYPE;
    if (x.act_type > STARK_QMM_ACT_GELU_MATERIALIZED_POLYNOMIAL || x.op > STARK_QMM_GATED_QUANTIZE_WITH_GROUP_SUMS ||
        !x.act_operand)
        return STARK_QMM_INVALID_ARGUMENT;
    if (!x.interleaved && !x.value_operand) return STARK_QMM_INVALID_ARGUMENT;
    // gated_act_mul.rs:46-51
    const bool quantize = x.op != STARK_QMM_GATED_FULL_PRECISION;
    if (quantize && !x.hadamard_factors) return STARK_QMM_INVALID_ARGUMENT;  // quantized gate activation requires RHT
    if (x.hadamard_factors && x.gated_dim % kBlock) return STARK_QMM_INVALID_ARGUMENT;
    uint32_t sg = kBlock;
    if (quantize) {
        sg = x.scale_group_size;
        if (!(sg == 32 || sg == 64 || sg == 128) || x.gated_dim % sg || !x.q_out || !x.scales_out)
            return STARK_QMM_INVALID_ARGUMENT;
        if (x.op == STARK_QMM_GATED_QUANTIZE_WITH_GROUP_SUMS &&
            (!(x.sum_group_size == 32 || x.sum_group_size == 64 || x.sum_group_size == 128) ||
             x.sum_group_size > sg || !x.group_sums_out))
            return STARK_QMM_INVALID_ARGUMENT;
    } else if (!x.fp_out) {
        return STARK_QMM_INVALID_ARGUMENT;
    }
    GatedArgs a{};
    a.act = x.act_operand;
    a.value = x.interleaved ? nullptr : x.value_operand;
    a.fp_out = x.fp_out;
    a.q_out = x.q_out;
    a.scales_out = x.scales_out;
    a.sums_out = x.group_sums_out;
    a.factors = x.hadamard_factors;
    a.gated_dim = x.gated_dim;
    a.batch = x.batch_dim;
    a.value_offset = x.value_offset;
    a.value_row_stride = x.value_row_stride;
    a.act_type = x.act_type;
    a.has_alpha = x.has_activation_alpha;
    a.alpha = x.activation_alpha;
    a.clip_gate = x.clip_gate;
    a.gate_min = x.gate_clip_min;
    a.gate_max = x.gate_clip_max;
    a.clip_value = x.clip_value;
    a.value_min = x.value_clip_min;
    a.value_max = x.value_clip_max;
    a.op = x.op;
    a.grouped = x.grouped_by_nibble;
    a.scale_group = sg;
    a.sum_group = x.sum_group_size;
    a.t_dt = x.data_type;
    const uint32_t items = x.batch_dim * (x.hadamard_factors ? x.gated_dim / sg : x.gated_dim);
    return launch_by_group<GA>(sg, items, a, (hipStream_t)stream);
}

}  // extern "C"
