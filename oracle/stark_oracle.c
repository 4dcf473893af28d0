/*
 * stark_oracle.c -- CPU restatement of the reference's quantized-matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the CPU baseline. Nothing in
 * the product library calls into this file.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp -shared).
 * -ffp-contract=off matters: Rust evaluates `acc += a * b` as a rounded product
 * followed by a rounded sum; only explicit `mul_add` calls are fused, and those
 * are written as fmaf() below.
 *
 * Each function names the reference file:line it follows; paths are relative
 * to the reference repository root, `crates/stark-engine/src/` abbreviated as
 * `src/`.
 */
#include "stark_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* half 2.7.1 conversions (Cargo.lock:897-899, used by read_f32/write_f32 at  */
/* src/backends/cpu/kernel/matmul/reference.rs:157-187).                      */
/* ------------------------------------------------------------------------ */

static uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float so_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* Round to nearest, ties to even; NaN keeps its sign and top payload bits and
 * is forced quiet. */
uint16_t so_f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t round_bit = 0x00008000u;
    if ((x & round_bit) != 0 && (x & (3u * round_bit - 1u)) != 0) return (uint16_t)((x >> 16) + 1u);
    return (uint16_t)(x >> 16);
}

float so_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0x1f) return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        if (man == 0) return bits_f32(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* IEEE binary16 round-to-nearest-even, overflow to infinity, gradual underflow. */
uint16_t so_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {
        if (man == 0) return sign | 0x7c00u;
        return sign | 0x7e00u | (uint16_t)(man >> 13);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign; /* rounds to zero (|x| < 2^-25) */
        uint32_t m = man | 0x800000u;
        int shift = 14 - e; /* 14..24 */
        uint32_t half_bit = 1u << (shift - 1);
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        if (rem > half_bit || (rem == half_bit && (q & 1u))) q += 1u;
        return sign | (uint16_t)q;
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u; /* may carry into inf: correct */
    return sign | (uint16_t)q;
}

void so_f32_to_bf16_n(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = so_f32_to_bf16(s[i]); }
void so_bf16_to_f32_n(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = so_bf16_to_f32(s[i]); }
void so_f32_to_f16_n(const float* s, uint16_t* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = so_f32_to_f16(s[i]); }
void so_f16_to_f32_n(const uint16_t* s, float* d, size_t n) { for (size_t i = 0; i < n; ++i) d[i] = so_f16_to_f32(s[i]); }

static float read_f32(const void* base, int dt, size_t index) {
    switch (dt) {
    case SO_F32: return ((const float*)base)[index];
    case SO_F16: return so_f16_to_f32(((const uint16_t*)base)[index]);
    default: return so_bf16_to_f32(((const uint16_t*)base)[index]);
    }
}
static void write_f32(void* base, int dt, size_t index, float v) {
    switch (dt) {
    case SO_F32: ((float*)base)[index] = v; break;
    case SO_F16: ((uint16_t*)base)[index] = so_f32_to_f16(v); break;
    default: ((uint16_t*)base)[index] = so_f32_to_bf16(v); break;
    }
}
static int dt_size(int dt) { return dt == SO_F32 ? 4 : 2; }

/* src/backends/cpu/kernel/matmul/reference.rs:91-104 */
uint8_t so_packed_code(const uint8_t* codes, int bits, size_t index) {
    size_t bit = index * (size_t)bits;
    size_t offset = bit / 8;
    unsigned shift = (unsigned)(bit % 8);
    uint16_t value = codes[offset];
    if (shift + (unsigned)bits > 8) value |= (uint16_t)((uint16_t)codes[offset + 1] << 8);
    return (uint8_t)((value >> shift) & ((1u << bits) - 1u));
}

/* src/backends/common/kernel/matmul/mod.rs:131-156; the group-output rows are
 * padded to a multiple of 4 (QUANT_PARAMS_GROUP_OUTPUT_ALIGNMENT,
 * src/backends/common/gpu_types/matmul.rs:1). */
void so_quant_strides(int layout, uint32_t row_count, uint32_t group_count, uint32_t pd, uint32_t* os, uint32_t* gs) {
    if (layout == SO_LAYOUT_OUTPUT_GROUP) {
        *os = (group_count + pd - 1) / pd * pd;
        *gs = 1;
    } else {
        *os = 1;
        *gs = (row_count + 3u) / 4u * 4u;
    }
}

/* src/backends/cpu/kernel/matmul/reference.rs:109-154 (materialized_affine_dot).
 * bf16 + bf16 in `half` widens, adds in f32 and rounds back to bf16. */
static float materialized_affine_dot(const so_matmul_args* a, const uint16_t* input, size_t row, size_t column,
                                     size_t k, uint32_t os, uint32_t gs) {
    float result = 0.0f;
    for (size_t begin = 0; begin < k; begin += 16) {
        size_t end = begin + 16 < k ? begin + 16 : k;
        float dot = 0.0f, sum = 0.0f;
        for (size_t quad = begin; quad < end; quad += 4) {
            uint16_t values[4] = {0, 0, 0, 0};
            float subtotal = 0.0f;
            for (size_t i = 0; i < 4; ++i) {
                if (quad + i < end) {
                    values[i] = input[row * k + quad + i];
                    uint8_t code = so_packed_code(a->codes, 4, column * k + quad + i);
                    subtotal += so_bf16_to_f32(values[i]) * (float)code;
                }
            }
            dot += subtotal;
            uint16_t s01 = so_f32_to_bf16(so_bf16_to_f32(values[0]) + so_bf16_to_f32(values[1]));
            uint16_t s012 = so_f32_to_bf16(so_bf16_to_f32(s01) + so_bf16_to_f32(values[2]));
            uint16_t s0123 = so_f32_to_bf16(so_bf16_to_f32(s012) + so_bf16_to_f32(values[3]));
            sum += so_bf16_to_f32(s0123);
        }
        size_t md = column * os + (begin / a->group_size) * gs;
        float scale = so_bf16_to_f32(((const uint16_t*)a->scales)[md]);
        float bias = so_bf16_to_f32(((const uint16_t*)a->correction_data)[md]);
        result += scale * dot + bias * sum;
    }
    return result;
}

/* src/backends/common/kernel/matmul/arguments.rs:36-61 */
static int affine_input_sum_policy_ok(const so_matmul_args* a) {
    if (!a->materialize_affine_input_sum) return 1;
    if (a->weights_dt != SO_BF16 || a->input_dt != SO_BF16 || a->output_dt != SO_BF16 || a->bits != 4 ||
        a->correction != SO_CORR_BIASES || a->signed_codes || !a->b_transpose ||
        !(a->group_size == 16 || a->group_size == 32 || a->group_size == 64 || a->group_size == 128) ||
        (a->k % 4) != 0)
        return 0;
    return 1;
}

/* One output of src/backends/cpu/kernel/matmul/kernel.rs:170-282. */
static void matmul_one(const so_matmul_args* a, size_t row, size_t col, int materialize, uint32_t os, uint32_t gs,
                       uint32_t zos, uint32_t zgs) {
    size_t n = a->n, k = a->k;
    const uint8_t* input = (const uint8_t*)a->a + a->a_offset * (size_t)dt_size(a->input_dt);
    size_t b_col = a->gather_indices ? (size_t)a->gather_indices[row * n + col] : col;
    float accumulator = 0.0f;
    if (materialize) accumulator = materialized_affine_dot(a, (const uint16_t*)input, row, b_col, k, os, gs);
    size_t inner_end = materialize ? 0 : k;
    float midpoint = (float)(1u << (a->bits - 1));
    for (size_t inner = 0; inner < inner_end; ++inner) {
        float a_value;
        if (a->a_codes) {  /* kernel.rs:193-205 */
            size_t groups = (k + a->a_scale_group_size - 1) / a->a_scale_group_size;
            size_t code_index = so_int8_code_index(a->a_grouped_by_nibble, inner);
            float q = (float)a->a_codes[row * k + code_index];
            a_value = q * a->a_scales[row * groups + inner / a->a_scale_group_size];
        } else {
            a_value = read_f32(input, a->input_dt, row * k + inner);
        }
        if (!a->codes) {
            size_t ld = a->b_leading_dimension ? a->b_leading_dimension : (a->b_transpose ? k : n);
            size_t index = a->b_transpose ? b_col * ld + inner : inner * ld + b_col;
            accumulator += a_value * read_f32(a->b_values, a->weights_dt, index);
            continue;
        }
        size_t wl = b_col * k + inner;
        uint8_t code = so_packed_code(a->codes, a->bits, wl);
        if (a->signed_codes) code ^= (uint8_t)(1u << (a->bits - 1));
        float q = (float)code;
        size_t g = inner / a->group_size;
        size_t md = b_col * os + g * gs;
        float scale = read_f32(a->scales, a->weights_dt, md);
        float bias_term;
        if (a->correction == SO_CORR_ZERO_POINTS) {
            size_t zi = b_col * zos + g * zgs;
            float zp;
            if (a->bits == 4) {
                uint8_t byte = ((const uint8_t*)a->correction_data)[zi / 2];
                zp = (float)((zi % 2 == 0) ? (byte & 0x0f) : ((byte >> 4) & 0x0f));
            } else {
                zp = (float)((const uint8_t*)a->correction_data)[zi];
            }
            bias_term = -scale * zp;
        } else if (a->correction == SO_CORR_BIASES) {
            bias_term = read_f32(a->correction_data, a->weights_dt, md);
        } else {
            bias_term = -scale * midpoint;
        }
        float b_value = scale * q + bias_term;
        accumulator += a_value * b_value;
    }
    size_t oi = row * n + col;
    float value = a->ab_scale * accumulator;
    if (a->accumulate) value += read_f32(a->d, a->output_dt, oi);
    if (a->bias && !a->rht_factors) value += read_f32(a->bias, a->weights_dt, col);  /* kernel.rs:275 */
    if (a->has_soft_cap) value = a->soft_cap * tanhf(value / a->soft_cap);
    write_f32(a->d, a->output_dt, oi, value);
}

/* kernel.rs:287-300: output RHT in place over d, then the bias add
 * (tensor_add_bias.rs:9-32: f32(d) + f32(bias), rounded to d's type). */
static void matmul_output_rht(const so_matmul_args* a) {
    so_activation_transform(NULL, a->d, NULL, NULL, NULL, NULL, a->rht_factors, a->m, a->n, SO_OUTPUT_RHT, 0, 1, 0,
                            0, a->output_dt, SO_F32);
    if (!a->bias) return;
    for (size_t i = 0; i < (size_t)a->m * a->n; ++i)
        write_f32(a->d, a->output_dt, i, read_f32(a->d, a->output_dt, i) + read_f32(a->bias, a->weights_dt, i % a->n));
}

static int matmul_prepare(const so_matmul_args* a, int* materialize, uint32_t* os, uint32_t* gs, uint32_t* zos,
                          uint32_t* zgs) {
    int dts[3] = {a->weights_dt, a->input_dt, a->output_dt};
    for (int i = 0; i < 3; ++i)
        if (dts[i] != SO_F32 && dts[i] != SO_F16 && dts[i] != SO_BF16) return 2;
    if (a->rht_factors && (a->output_dt == SO_F16 || a->n % 32)) return 4;
    if (a->a_codes) {  /* kernel.rs:130-141 */
        uint32_t g = a->a_scale_group_size;
        if (!(g == 32 || g == 64 || g == 128) || a->k % g || !a->codes || !(a->bits == 4 || a->bits == 8) ||
            !(a->group_size == 32 || a->group_size == 64 || a->group_size == 128))
            return 3;
    }
    if (!a->codes) {
        *materialize = 0;
        *os = *gs = *zos = *zgs = 0;
        return a->materialize_affine_input_sum ? 1 : 0;
    }
    if (!affine_input_sum_policy_ok(a)) return 1;
    /* reference.rs:62-71: the codes buffer must hold ceil(n*k*bits/8) bytes */
    size_t required = ((size_t)a->n * a->k * (size_t)a->bits + 7) / 8;
    if (required > a->codes_size) return 1;
    *materialize = a->m == 1 && a->materialize_affine_input_sum;
    so_quant_strides(a->layout, a->row_count, a->group_count, 1, os, gs);
    uint32_t pd = 8u / (uint32_t)a->bits;
    if (a->correction == SO_CORR_ZERO_POINTS) so_quant_strides(a->layout, a->row_count, a->group_count, pd, zos, zgs);
    else *zos = *zgs = 0;
    return 0;
}

/* src/backends/cpu/kernel/matmul/kernel.rs:58-303 (quantized B, FullPrecision A,
 * D-ops scale/accumulate/bias/soft-cap; output RHT is not restated). */
int so_matmul(const so_matmul_args* a) {
    int materialize;
    uint32_t os, gs, zos, zgs;
    int st = matmul_prepare(a, &materialize, &os, &gs, &zos, &zgs);
    if (st) return st;
    for (size_t row = 0; row < a->m; ++row)
        for (size_t col = 0; col < a->n; ++col) matmul_one(a, row, col, materialize, os, gs, zos, zgs);
    if (a->rht_factors) matmul_output_rht(a);
    return 0;
}

int so_matmul_parallel(const so_matmul_args* a, int threads) {
    int materialize;
    uint32_t os, gs, zos, zgs;
    int st = matmul_prepare(a, &materialize, &os, &gs, &zos, &zgs);
    if (st) return st;
    long total = (long)a->m * (long)a->n;
#pragma omp parallel for schedule(static) num_threads(threads)
    for (long i = 0; i < total; ++i) matmul_one(a, (size_t)(i / a->n), (size_t)(i % a->n), materialize, os, gs, zos, zgs);
    if (a->rht_factors) matmul_output_rht(a);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Activation transforms: src/backends/cpu/kernel/activation_transform/       */
/* ------------------------------------------------------------------------ */

#define SO_HADAMARD_BLOCK 32 /* src/backends/common/gpu_types/hadamard_order.rs:1 */

/* mod.rs:28-43 */
void so_hadamard32(float* v) {
    for (int stride = 1; stride < SO_HADAMARD_BLOCK; stride <<= 1)
        for (int lane = 0; lane < SO_HADAMARD_BLOCK; ++lane)
            if ((lane & stride) == 0) {
                float x = v[lane], y = v[lane | stride];
                v[lane] = x + y;
                v[lane | stride] = x - y;
            }
    const float scale = 1.0f / sqrtf((float)SO_HADAMARD_BLOCK);
    for (int i = 0; i < SO_HADAMARD_BLOCK; ++i) v[i] *= scale;
}

/* mod.rs:9-19: the group's largest magnitude / 127, or 1 when that is zero or
 * not finite (f32::min/max ignore NaN). */
float so_min_max_symmetric_divisor(const float* v, size_t n) {
    float mn = INFINITY, mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) {
        mn = fminf(mn, v[i]);
        mx = fmaxf(mx, v[i]);
    }
    float m = fmaxf(fabsf(mn), fabsf(mx));
    return (isfinite(m) && m > 0.0f) ? m / 127.0f : 1.0f;
}

/* mod.rs:21-26: round half away from zero, clamp to +-127, as i8 (NaN -> 0) */
int8_t so_quantize_symmetric_i8(float value, float divisor) {
    float q = roundf(value / divisor);
    if (isnan(q)) return 0;
    if (q < -127.0f) q = -127.0f;
    if (q > 127.0f) q = 127.0f;
    return (int8_t)q;
}

size_t so_int8_code_index(int grouped, size_t index) {
    if (!grouped) return index;
    size_t offset = index % 8;
    return index - offset + (offset % 2) * 4 + offset / 2;
}

/* activation_transform.rs:14-46 */
static void quantize_transformed_row(const float* t, size_t n, size_t scale_group, size_t sum_group, int8_t* values,
                                     float* scales, int32_t* sums, int grouped) {
    if (sums)
        for (size_t i = 0; i < n / sum_group; ++i) sums[i] = 0;
    for (size_t g = 0; g < n / scale_group; ++g) {
        const float* src = t + g * scale_group;
        float scale = so_min_max_symmetric_divisor(src, scale_group);
        scales[g] = scale;
        for (size_t i = 0; i < scale_group; ++i) {
            int8_t code = so_quantize_symmetric_i8(src[i], scale);
            size_t absolute = g * scale_group + i;
            values[so_int8_code_index(grouped, absolute)] = code;
            if (sums) sums[absolute / sum_group] += code;
        }
    }
}

/* f32::clamp: NaN stays NaN */
static float clamp_f32(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

static float round_to(int dt, float v) { return dt == SO_BF16 ? so_bf16_to_f32(so_f32_to_bf16(v)) : v; }

/* activation_transform.rs:48-156 */
int so_activation_transform(const void* input, void* fp_out, const void* bias, int8_t* q_out, float* scales_out,
                            int32_t* group_sums_out, const int32_t* factors, uint32_t batch_size,
                            uint32_t element_count, int op, int grouped, int in_place, uint32_t scale_group,
                            uint32_t sum_group, int t_dt, int bias_dt) {
    const void* src = in_place ? fp_out : input;
    size_t columns = element_count;
    if (columns % SO_HADAMARD_BLOCK) return 1;
    int input_rht = op != SO_OUTPUT_RHT;
    int quantize = op == SO_QUANTIZE || op == SO_QUANTIZE_WITH_GROUP_SUMS;
    if (quantize && (!scale_group || columns % scale_group ||
                     (op == SO_QUANTIZE_WITH_GROUP_SUMS && (!sum_group || columns % sum_group))))
        return 1;
    float* transformed = (float*)malloc(columns * sizeof(float));
    for (size_t row = 0; row < batch_size; ++row) {
        size_t ro = row * columns;
        for (size_t s0 = 0; s0 < columns; s0 += SO_HADAMARD_BLOCK) {
            float stripe[SO_HADAMARD_BLOCK];
            for (int lane = 0; lane < SO_HADAMARD_BLOCK; ++lane) {
                float value = read_f32(src, t_dt, ro + s0 + lane);
                float factor = (float)factors[s0 + lane];
                stripe[lane] = input_rht ? value * factor : value;
            }
            so_hadamard32(stripe);
            for (int lane = 0; lane < SO_HADAMARD_BLOCK; ++lane) {
                float factor = (float)factors[s0 + lane];
                transformed[s0 + lane] = input_rht ? stripe[lane] : stripe[lane] * factor;
            }
        }
        if (quantize) {
            size_t spr = columns / scale_group;
            quantize_transformed_row(transformed, columns, scale_group,
                                     op == SO_QUANTIZE_WITH_GROUP_SUMS ? sum_group : 0, q_out + ro,
                                     scales_out + row * spr,
                                     op == SO_QUANTIZE_WITH_GROUP_SUMS ? group_sums_out + row * (columns / sum_group)
                                                                       : NULL,
                                     grouped);
        } else {
            for (size_t i = 0; i < columns; ++i) {
                float value = transformed[i];
                if (bias) value = round_to(t_dt, value) + read_f32(bias, bias_dt, i);
                write_f32(fp_out, t_dt, ro + i, value);
            }
        }
    }
    free(transformed);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Activations: src/backends/common/gpu_types/activation_type.rs, in the      */
/* storage type T (half's bf16 arithmetic rounds after every operation).      */
/* ------------------------------------------------------------------------ */

#define GELU_K0 0.044715f   /* activation_type.rs:3 */
#define GELU_K1 0.7978846f  /* activation_type.rs:4 */

float so_activate(int act_type, float x, int dt, int has_alpha, float alpha) {
    switch (act_type) {
    case SO_SILU: { /* activation_silu_alpha :35-42 (alpha 1 for plain SILU) */
        float a = has_alpha ? alpha : 1.0f;
        return round_to(dt, x / (1.0f + expf(-a * x)));
    }
    case SO_SILU_MATERIALIZED_SIGMOID: { /* :48-60 */
        float exponential = round_to(dt, expf(fabsf(x)));
        float lower = round_to(dt, 1.0f / round_to(dt, 1.0f + exponential));
        float sigmoid = x < 0.0f ? lower : round_to(dt, 1.0f - lower);
        return round_to(dt, x * sigmoid);
    }
    case SO_GELU_APPROX: { /* :62-67 */
        float tan_arg = GELU_K1 * (x + GELU_K0 * x * x * x);
        return round_to(dt, 0.5f * x * (1.0f + tanhf(tan_arg)));
    }
    case SO_GELU_MATERIALIZED_POLYNOMIAL: { /* :69-76 */
        float cubic = round_to(dt, x * x * x);
        float term = round_to(dt, round_to(dt, GELU_K0) * cubic);
        float inner = round_to(dt, x + term);
        float argument = round_to(dt, round_to(dt, GELU_K1) * inner);
        float activated = round_to(dt, tanhf(argument));
        return round_to(dt, round_to(dt, 0.5f * x) * round_to(dt, 1.0f + activated));
    }
    case SO_GELU_EXACT: /* :78-82 */
        return round_to(dt, 0.5f * x * (1.0f + erff(x * 0.70710677f)));
    case SO_SOFTPLUS: /* :84-92 */
        if (x > 20.0f) return x;
        return round_to(dt, logf(1.0f + expf(x)));
    default: /* IDENTITY */
        return x;
    }
}

/* gated_act_mul.rs:17-152 */
int so_gated_act_mul(const void* act, const void* value_operand, void* fp_out, int8_t* q_out, float* scales_out,
                     int32_t* sums_out, const int32_t* factors, uint32_t gated_dim, uint32_t batch_dim,
                     uint32_t value_offset, uint32_t value_row_stride, int act_type, int has_alpha, float alpha,
                     int clip_gate, float gate_min, float gate_max, int clip_value, float value_min,
                     float value_max, int op, int grouped, int interleaved, int use_hadamard, uint32_t scale_group,
                     uint32_t sum_group, int dt) {
    int quantize = op == SO_GAM_QUANTIZE || op == SO_GAM_QUANTIZE_WITH_GROUP_SUMS;
    int emit_sums = op == SO_GAM_QUANTIZE_WITH_GROUP_SUMS;
    if (quantize && !use_hadamard) return 1;
    if (quantize && (!scale_group || gated_dim % scale_group)) return 1;
    if (emit_sums && (!sum_group || gated_dim % sum_group)) return 1;
    if (use_hadamard && gated_dim % SO_HADAMARD_BLOCK) return 1;
    float* transformed = use_hadamard ? (float*)malloc((size_t)gated_dim * sizeof(float)) : NULL;
    for (size_t batch = 0; batch < batch_dim; ++batch) {
        for (size_t g = 0; g < gated_dim; ++g) {
            size_t act_index;
            float value;
            if (interleaved) {
                size_t base = batch * 2 * gated_dim;
                act_index = base + gated_dim + g;
                value = read_f32(act, dt, base + g);
            } else {
                act_index = batch * gated_dim + g;
                value = read_f32(value_operand, dt, batch * value_row_stride + value_offset + g);
            }
            float gate = read_f32(act, dt, act_index);
            if (clip_gate) gate = round_to(dt, clamp_f32(gate, gate_min, gate_max));
            float activated = (has_alpha && act_type == SO_SILU) ? so_activate(SO_SILU, gate, dt, 1, alpha)
                                                                 : so_activate(act_type, gate, dt, 0, 1.0f);
            if (clip_value) value = round_to(dt, clamp_f32(value, value_min, value_max));
            float result = round_to(dt, value * activated);
            if (transformed) transformed[g] = result;
            else write_f32(fp_out, dt, batch * gated_dim + g, result);
        }
        if (transformed) {
            for (size_t s0 = 0; s0 < gated_dim; s0 += SO_HADAMARD_BLOCK) {
                float stripe[SO_HADAMARD_BLOCK];
                for (int lane = 0; lane < SO_HADAMARD_BLOCK; ++lane)
                    stripe[lane] = transformed[s0 + lane] * (float)factors[s0 + lane];
                so_hadamard32(stripe);
                memcpy(transformed + s0, stripe, sizeof stripe);
            }
            if (quantize) {
                quantize_transformed_row(transformed, gated_dim, scale_group, emit_sums ? sum_group : 0,
                                         q_out + batch * gated_dim, scales_out + batch * (gated_dim / scale_group),
                                         emit_sums ? sums_out + batch * (gated_dim / sum_group) : NULL, grouped);
            } else {
                for (size_t g = 0; g < gated_dim; ++g) write_f32(fp_out, dt, batch * gated_dim + g, transformed[g]);
            }
        }
    }
    free(transformed);
    return 0;
}

/* src/backends/cpu/kernel/matmul/vision.rs:249-336. `mul_add` is fused (fmaf). */
void so_reference_affine_linear_bf16(const uint16_t* input, const uint8_t* weights, const uint16_t* scales,
                                     const uint16_t* biases, const uint32_t* indices, uint16_t* bf16_output,
                                     float* f32_output, uint32_t m, uint32_t n, uint32_t k, uint32_t bank_rows,
                                     uint32_t bits, uint32_t sos, uint32_t sgs) {
    for (size_t row = 0; row < m; ++row) {
        for (size_t column = 0; column < n; ++column) {
            size_t out_index = row * n + column;
            size_t source_row = indices ? indices[out_index] : column;
            uint16_t result;
            if (source_row >= bank_rows || k % 32 != 0 ||
                (bits != 0 && (!(bits == 4 || bits == 5 || bits == 6 || bits == 8) || k % 64 != 0))) {
                result = 0x7fc0; /* bf16::NAN */
            } else {
                float sums[8][4];
                memset(sums, 0, sizeof sums);
                for (size_t start = 0; start < k; start += 32) {
                    for (int reg = 0; reg < 8; ++reg) {
                        for (int lane = 0; lane < 4; ++lane) {
                            size_t inner = start + (size_t)reg * 4 + (size_t)lane;
                            float value;
                            if (bits == 0) {
                                value = so_bf16_to_f32(((const uint16_t*)weights)[source_row * k + inner]);
                            } else {
                                size_t bit = inner * bits;
                                unsigned shift = (unsigned)(bit % 8);
                                size_t offset = source_row * (k * bits / 8) + bit / 8;
                                uint32_t packed = weights[offset];
                                if (shift + bits > 8) packed |= (uint32_t)weights[offset + 1] << 8;
                                uint32_t code = (packed >> shift) & ((1u << bits) - 1u);
                                size_t group = source_row * sos + inner / 64 * sgs;
                                float v = (float)code * so_bf16_to_f32(scales[group]) + so_bf16_to_f32(biases[group]);
                                value = so_bf16_to_f32(so_f32_to_bf16(v));
                            }
                            float av = so_bf16_to_f32(input[row * k + inner]);
                            sums[reg][lane] = fmaf(av, value, sums[reg][lane]);
                        }
                    }
                }
                for (int offset = 4; offset >= 1; offset /= 2)
                    for (int reg = 0; reg < offset; ++reg)
                        for (int lane = 0; lane < 4; ++lane) sums[reg][lane] += sums[reg + offset][lane];
                result = so_f32_to_bf16((sums[0][0] + sums[0][1]) + (sums[0][2] + sums[0][3]));
            }
            if (f32_output) f32_output[out_index] = so_bf16_to_f32(result);
            if (bf16_output) bf16_output[out_index] = result;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* GGUF blocks: src/engine/hybrid/weights.rs                                  */
/* ------------------------------------------------------------------------ */

/* weights.rs:2565-2584 (subset: the kinds restated by so_decode_block) */
int so_block_layout(uint32_t kind, size_t* elements, size_t* bytes) {
    switch (kind) {
    case 0: *elements = 1; *bytes = 4; return 0;
    case 1: case 30: *elements = 1; *bytes = 2; return 0;
    case 8: *elements = 32; *bytes = 34; return 0;
    case 10: *elements = 256; *bytes = 84; return 0;
    case 11: *elements = 256; *bytes = 110; return 0;
    case 12: *elements = 256; *bytes = 144; return 0;
    case 13: *elements = 256; *bytes = 176; return 0;
    case 14: *elements = 256; *bytes = 210; return 0;
    case 16: *elements = 256; *bytes = 66; return 0;
    case 17: *elements = 256; *bytes = 74; return 0;
    case 18: *elements = 256; *bytes = 98; return 0;
    case 23: *elements = 256; *bytes = 136; return 0;
    default: return 1;
    }
}

static float half_at(const uint8_t* b, size_t at) { return so_f16_to_f32((uint16_t)(b[at] | (b[at + 1] << 8))); }

/* weights.rs:2908-2921 */
void so_scale_min(const uint8_t* s, int index, uint8_t* scale, uint8_t* min) {
    if (index < 4) {
        *scale = s[index] & 63;
        *min = s[index + 4] & 63;
    } else {
        *scale = (uint8_t)((s[index + 4] & 15) | ((s[index - 4] >> 6) << 4));
        *min = (uint8_t)((s[index + 4] >> 4) | ((s[index] >> 6) << 4));
    }
}

/* weights.rs:2923-3012 for kinds 0, 1, 30 (scalars), 8 (Q8_0), 12 (Q4_K), 13 (Q5_K). */
int so_decode_block(uint32_t kind, const uint8_t* bytes, size_t nbytes, float* out, size_t count) {
    size_t be, bb;
    if (so_block_layout(kind, &be, &bb) || nbytes != bb || count != be) return 1;
    switch (kind) {
    case 0: memcpy(out, bytes, 4); return 0;
    case 1: out[0] = half_at(bytes, 0); return 0;
    case 30: out[0] = so_bf16_to_f32((uint16_t)(bytes[0] | (bytes[1] << 8))); return 0;
    case 8: {
        float d = half_at(bytes, 0);
        for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)bytes[2 + i];
        return 0;
    }
    case 12:
    case 13: {
        float d = half_at(bytes, 0);
        float minimum = half_at(bytes, 2);
        const uint8_t* scales = bytes + 4;
        size_t qstart = kind == 13 ? 48 : 16;
        for (int part = 0; part < 4; ++part) {
            for (int half = 0; half < 2; ++half) {
                uint8_t sc, mn;
                so_scale_min(scales, part * 2 + half, &sc, &mn);
                int at = part * 64 + half * 32;
                for (int l = 0; l < 32; ++l) {
                    uint8_t ql = (uint8_t)((bytes[qstart + part * 32 + l] >> (half * 4)) & 15);
                    uint8_t high = (kind == 13 && (bytes[16 + l] & (1u << (part * 2 + half)))) ? 16 : 0;
                    out[at + l] = d * (float)sc * (float)(uint8_t)(ql + high) - minimum * (float)mn;
                }
            }
        }
        return 0;
    }
    default: return 2;
    }
}

/* weights.rs:2533-2550: decode_values for one row, then
 * `values.iter().zip(input).map(|(w, x)| w * x).sum()` (a left fold from -0.0). */
/* decode_block over whole rows of blocks (test helper: the dequantised
 * matrix for tolerance magnitudes); rows are independent, OpenMP over rows. */
int so_decode_rows(uint32_t kind, const uint8_t* bytes, size_t rows, size_t columns, float* output) {
    size_t be, bb;
    if (so_block_layout(kind, &be, &bb) || columns % be) return 1;
    size_t row_bytes = columns / be * bb;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(|:bad)
    for (long r = 0; r < (long)rows; ++r)
        for (size_t b = 0; b < columns / be; ++b)
            bad |= so_decode_block(kind, bytes + (size_t)r * row_bytes + b * bb, bb,
                                   output + (size_t)r * columns + b * be, be);
    return bad ? 2 : 0;
}

int so_hybrid_packed_matvec(uint32_t kind, const uint8_t* bytes, size_t rows, size_t columns, const float* input,
                            float* output) {
    size_t be, bb;
    if (so_block_layout(kind, &be, &bb) || columns % be) return 1;
    size_t row_bytes = columns / be * bb;
    float* values = (float*)malloc(columns * sizeof(float));
    if (!values) return 3;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t b = 0; b < columns / be; ++b)
            if (so_decode_block(kind, bytes + r * row_bytes + b * bb, bb, values + b * be, be)) { free(values); return 2; }
        float s = -0.0f;
        for (size_t c = 0; c < columns; ++c) s += values[c] * input[c];
        output[r] = s;
    }
    free(values);
    return 0;
}

/* weights.rs:1284-1309 affine_row (planes [N, G]), then the same f32 fold. */
int so_hybrid_affine_matvec(const uint8_t* codes, const void* scales, const void* biases, int scale_dt, int bits,
                            size_t group, size_t rows, size_t columns, const float* input, float* output) {
    if (!(bits == 4 || bits == 8) || columns % group) return 1;
    size_t group_count = columns / group;
    size_t packed_row = columns * (size_t)bits / 8;
    for (size_t r = 0; r < rows; ++r) {
        const uint8_t* c = codes + r * packed_row;
        float s = -0.0f;
        for (size_t col = 0; col < columns; ++col) {
            size_t index = r * group_count + col / group;
            float scale = read_f32(scales, scale_dt, index);
            float bias = read_f32(biases, scale_dt, index);
            uint8_t q = (uint8_t)((c[col * bits / 8] >> (col * bits % 8)) & ((1u << bits) - 1u));
            float value = scale * (float)q + bias;
            s += value * input[col];
        }
        output[r] = s;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* MoE: src/backends/cpu/kernel/moe.rs                                        */
/* ------------------------------------------------------------------------ */

/* moe.rs:23-85. f32::max ignores NaN like fmaxf; exp is the platform expf. */
void so_moe_route(const float* logits, uint32_t* ids, float* weights, uint32_t rows, uint32_t experts,
                  uint32_t active, uint32_t round_weights, uint32_t round_logits) {
    float* x = (float*)malloc((experts ? experts : 1) * sizeof(float));
    for (size_t row = 0; row < rows; ++row) {
        const float* src = logits + row * experts;
        int valid = experts >= 1 && experts <= 1024 && active >= 1 && active <= 32 && active <= experts;
        for (size_t e = 0; e < experts; ++e) {
            x[e] = round_logits ? so_bf16_to_f32(so_f32_to_bf16(src[e])) : src[e];
            if (!isfinite(x[e])) valid = 0;
        }
        float maximum = -INFINITY;
        for (size_t e = 0; e < experts; ++e) maximum = fmaxf(maximum, x[e]);
        float denominator = -0.0f;
        for (size_t e = 0; e < experts; ++e) denominator += expf(x[e] - maximum);
        uint32_t* rid = ids + row * active;
        float* rw = weights + row * active;
        float selected_sum = 0.0f;
        for (size_t rank = 0; rank < active; ++rank) {
            float best = -INFINITY;
            uint32_t selected = 0;
            for (size_t e = 0; e < experts; ++e) {
                int used = 0;
                for (size_t p = 0; p < rank; ++p) used |= rid[p] == (uint32_t)e;
                if (!used && x[e] > best) {
                    best = x[e];
                    selected = (uint32_t)e;
                }
            }
            rid[rank] = valid ? selected : 0;
            rw[rank] = expf(best - maximum) / denominator;
            selected_sum += rw[rank];
        }
        for (size_t rank = 0; rank < active; ++rank) {
            rw[rank] /= selected_sum;
            if (round_weights) rw[rank] = so_bf16_to_f32(so_f32_to_bf16(rw[rank]));
            if (!valid) rw[rank] = NAN;
        }
    }
    free(x);
}

/* moe.rs:87-107 */
void so_moe_gather_rows(const uint32_t* ids, uint32_t* indices, uint32_t route_offset, uint32_t rows_per_expert,
                        uint32_t experts, uint32_t length) {
    uint32_t expert = ids[route_offset];
    if (expert >= experts) expert = 0;
    for (uint32_t p = 0; p < length; ++p) indices[p] = expert * rows_per_expert + p;
}

/* moe.rs:109-145 */
void so_moe_accumulate(const uint16_t* input, const float* weights, float* accumulator, uint16_t* output,
                       uint32_t length, uint32_t weight_offset, uint32_t output_offset, uint32_t initialize,
                       uint32_t finalize, uint32_t round_product, uint32_t round_accumulator) {
    float weight = weights[weight_offset];
    for (uint32_t p = 0; p < length; ++p) {
        size_t out = (size_t)output_offset + p;
        float product = so_bf16_to_f32(input[p]) * weight;
        if (round_product) product = so_bf16_to_f32(so_f32_to_bf16(product));
        float value = (initialize ? 0.0f : accumulator[out]) + product;
        if (round_accumulator) value = so_bf16_to_f32(so_f32_to_bf16(value));
        accumulator[out] = value;
        if (finalize) output[out] = so_f32_to_bf16(value);
    }
}

/* moe.rs:147-184 */
void so_moe_adjust_routes(uint32_t* ids, float* weights, const float* scales, uint32_t rows, uint32_t experts,
                          uint32_t active, uint32_t sort_ids) {
    for (size_t row = 0; row < rows; ++row) {
        size_t base = row * active;
        for (size_t r = 0; r < active; ++r) {
            uint32_t id = ids[base + r];
            weights[base + r] = id < experts ? weights[base + r] * scales[id] : NAN;
        }
        if (sort_ids) {
            for (size_t r = 1; r < active; ++r) {
                size_t i = r;
                while (i > 0 && ids[base + i] < ids[base + i - 1]) {
                    uint32_t t = ids[base + i]; ids[base + i] = ids[base + i - 1]; ids[base + i - 1] = t;
                    float w = weights[base + i]; weights[base + i] = weights[base + i - 1]; weights[base + i - 1] = w;
                    --i;
                }
            }
        }
    }
}

/* src/backends/cpu/kernel/gated_act_mul/gated_act_mul.rs (interleaved operand,
 * plain SiLU from src/backends/common/gpu_types/activation_type.rs:35-46).
 * bf16 * bf16 in `half` widens, multiplies in f32 and rounds back. */
void so_gated_silu_bf16(const uint16_t* projected, uint16_t* out, uint32_t hidden, uint32_t batch) {
    for (size_t b = 0; b < batch; ++b) {
        size_t base = b * 2 * (size_t)hidden;
        for (size_t g = 0; g < hidden; ++g) {
            uint16_t value = projected[base + g];
            float x = so_bf16_to_f32(projected[base + hidden + g]);
            float y = x / (1.0f + expf(-1.0f * x));
            uint16_t activated = so_f32_to_bf16(y);
            uint16_t r = so_f32_to_bf16(so_bf16_to_f32(value) * so_bf16_to_f32(activated));
            out[b * hidden + g] = r;
        }
    }
}

/* encodable_block/mlp/routed.rs:154-257 */
int so_routed_experts(const uint16_t* input, const float* logits, const float* expert_scales,
                      const uint8_t* up_codes, const void* up_scales, const void* up_biases,
                      const uint8_t* down_codes, const void* down_scales, const void* down_biases, int layout,
                      int bits, uint32_t group_size, int plane_dt, uint32_t rows, uint32_t model, uint32_t hidden,
                      uint32_t experts, uint32_t active, int round_logits, int round_weights, int round_products,
                      int round_accumulator, int sort_ids, uint16_t* output) {
    const size_t routes = (size_t)rows * active;
    uint32_t* ids = (uint32_t*)malloc(routes * sizeof(uint32_t));
    float* weights = (float*)malloc(routes * sizeof(float));
    float* accumulator = (float*)calloc((size_t)rows * model, sizeof(float));
    uint32_t* up_ids = (uint32_t*)malloc((size_t)2 * hidden * sizeof(uint32_t));
    uint32_t* down_ids = (uint32_t*)malloc((size_t)model * sizeof(uint32_t));
    uint16_t* projected = (uint16_t*)malloc((size_t)2 * hidden * sizeof(uint16_t));
    uint16_t* activated = (uint16_t*)malloc((size_t)hidden * sizeof(uint16_t));
    uint16_t* down_out = (uint16_t*)malloc((size_t)model * sizeof(uint16_t));
    float* unit = (float*)malloc((size_t)experts * sizeof(float));
    int status = 0;
    so_moe_route(logits, ids, weights, rows, experts, active, round_weights, round_logits);
    if (expert_scales) {
        so_moe_adjust_routes(ids, weights, expert_scales, rows, experts, active, sort_ids);
    } else if (sort_ids) {
        for (uint32_t e = 0; e < experts; ++e) unit[e] = 1.0f;
        so_moe_adjust_routes(ids, weights, unit, rows, experts, active, 1);
    }
    so_matmul_args up = {0}, down = {0};
    up.codes = up_codes;
    up.codes_size = (size_t)experts * 2 * hidden * model * (size_t)bits / 8;
    up.scales = up_scales;
    up.correction = up_biases ? SO_CORR_BIASES : SO_CORR_SYMMETRIC;
    up.correction_data = up_biases;
    up.layout = layout;
    up.row_count = experts * 2 * hidden;
    up.group_count = model / group_size;
    up.bits = bits;
    up.group_size = group_size;
    up.b_transpose = 1;
    up.ab_scale = 1.0f;
    up.m = 1;
    up.n = 2 * hidden;
    up.k = model;
    up.weights_dt = plane_dt;
    up.input_dt = SO_BF16;
    up.output_dt = SO_BF16;
    up.gather_indices = up_ids;
    up.d = projected;
    down = up;
    down.codes = down_codes;
    down.codes_size = (size_t)experts * model * hidden * (size_t)bits / 8;
    down.scales = down_scales;
    down.correction = down_biases ? SO_CORR_BIASES : SO_CORR_SYMMETRIC;
    down.correction_data = down_biases;
    down.row_count = experts * model;
    down.group_count = hidden / group_size;
    down.n = model;
    down.k = hidden;
    down.gather_indices = down_ids;
    down.a = activated;
    down.d = down_out;
    for (uint32_t row = 0; row < rows && status == 0; ++row) {
        for (uint32_t rank = 0; rank < active && status == 0; ++rank) {
            const uint32_t route = row * active + rank;
            so_moe_gather_rows(ids, up_ids, route, 2 * hidden, experts, 2 * hidden);
            up.a = input + (size_t)row * model;
            status = so_matmul(&up);
            if (status) break;
            so_gated_silu_bf16(projected, activated, hidden, 1);
            so_moe_gather_rows(ids, down_ids, route, model, experts, model);
            status = so_matmul(&down);
            if (status) break;
            so_moe_accumulate(down_out, weights, accumulator, output, model, route, row * model, rank == 0,
                              rank + 1 == active, round_products, round_accumulator);
        }
    }
    free(ids); free(weights); free(accumulator); free(up_ids); free(down_ids);
    free(projected); free(activated); free(down_out); free(unit);
    return status;
}

/* ------------------------------------------------------------------------ */
/* Test-input generators. Parity is defined on decode of the packed bytes, so */
/* these only need to produce valid encodings.                                */
/* ------------------------------------------------------------------------ */

/* MLX affine: per group scale=(max-min)/(2^bits-1), bias=min, stored as bf16;
 * q = clamp(round((w - bias)/scale)). Codes little-endian, low nibble first. */
void so_quantize_affine(const float* w, size_t rows, size_t cols, int bits, size_t group, int layout,
                        uint8_t* codes, uint16_t* scales, uint16_t* biases) {
    size_t G = cols / group;
    size_t n4 = (rows + 3) / 4 * 4;
    float qmax = (float)((1u << bits) - 1u);
    size_t row_bytes = cols * (size_t)bits / 8;
    memset(codes, 0, rows * row_bytes);
    if (layout == SO_LAYOUT_GROUP_OUTPUT) {
        memset(scales, 0, G * n4 * 2);
        memset(biases, 0, G * n4 * 2);
    }
    for (size_t r = 0; r < rows; ++r) {
        for (size_t g = 0; g < G; ++g) {
            const float* v = w + r * cols + g * group;
            float mn = v[0], mx = v[0];
            for (size_t i = 1; i < group; ++i) { if (v[i] < mn) mn = v[i]; if (v[i] > mx) mx = v[i]; }
            uint16_t sb = so_f32_to_bf16((mx - mn) / qmax);
            uint16_t bb = so_f32_to_bf16(mn);
            float s = so_bf16_to_f32(sb), b = so_bf16_to_f32(bb);
            size_t md = layout == SO_LAYOUT_OUTPUT_GROUP ? r * G + g : g * n4 + r;
            scales[md] = sb;
            biases[md] = bb;
            for (size_t i = 0; i < group; ++i) {
                float qf = s > 0.0f ? rintf((v[i] - b) / s) : 0.0f;
                if (qf < 0.0f) qf = 0.0f;
                if (qf > qmax) qf = qmax;
                unsigned q = (unsigned)qf;
                size_t kk = g * group + i;
                if (bits == 4) codes[r * row_bytes + kk / 2] |= (uint8_t)(q << (4 * (kk % 2)));
                else codes[r * row_bytes + kk] = (uint8_t)q;
            }
        }
    }
}

/* Q8_0: d = amax/127 (stored f16), q = round(x/d) in [-127, 127]. */
void so_quantize_q8_0(const float* w, size_t rows, size_t cols, uint8_t* out) {
    size_t nb = cols / 32;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t b = 0; b < nb; ++b) {
            const float* v = w + r * cols + b * 32;
            uint8_t* o = out + (r * nb + b) * 34;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) if (fabsf(v[i]) > amax) amax = fabsf(v[i]);
            float d = amax / 127.0f;
            uint16_t dh = so_f32_to_f16(d);
            o[0] = (uint8_t)(dh & 0xff);
            o[1] = (uint8_t)(dh >> 8);
            float id = d > 0.0f ? 1.0f / d : 0.0f;
            for (int i = 0; i < 32; ++i) {
                float q = rintf(v[i] * id);
                if (q > 127.0f) q = 127.0f;
                if (q < -127.0f) q = -127.0f;
                o[2 + i] = (uint8_t)(int8_t)q;
            }
        }
    }
}

/* Q4_K: 8 sub-blocks of 32 with 6-bit (scale, min) and f16 d/dmin. A single
 * pass of the min/scale fit ggml's quantize_row_q4_K_ref starts from
 * (scale=(max-min)/15, min=-min clamped at 0), without its iterative refine. */
void so_quantize_q4_k(const float* w, size_t rows, size_t cols, uint8_t* out) {
    size_t nb = cols / 256;
    for (size_t r = 0; r < rows; ++r) {
        for (size_t b = 0; b < nb; ++b) {
            const float* v = w + r * cols + b * 256;
            uint8_t* o = out + (r * nb + b) * 144;
            float scf[8], mnf[8];
            float max_sc = 0.0f, max_mn = 0.0f;
            for (int j = 0; j < 8; ++j) {
                float mn = v[j * 32], mx = v[j * 32];
                for (int l = 1; l < 32; ++l) { float x = v[j * 32 + l]; if (x < mn) mn = x; if (x > mx) mx = x; }
                if (mn > 0.0f) mn = 0.0f;
                scf[j] = (mx - mn) / 15.0f;
                mnf[j] = -mn;
                if (scf[j] > max_sc) max_sc = scf[j];
                if (mnf[j] > max_mn) max_mn = mnf[j];
            }
            uint16_t dh = so_f32_to_f16(max_sc / 63.0f), mh = so_f32_to_f16(max_mn / 63.0f);
            float d = so_f16_to_f32(dh), dmin = so_f16_to_f32(mh);
            uint8_t sc[8], mm[8];
            for (int j = 0; j < 8; ++j) {
                float s = d > 0.0f ? rintf(scf[j] / d) : 0.0f;
                float m = dmin > 0.0f ? rintf(mnf[j] / dmin) : 0.0f;
                sc[j] = (uint8_t)(s > 63.0f ? 63.0f : s);
                mm[j] = (uint8_t)(m > 63.0f ? 63.0f : m);
            }
            o[0] = (uint8_t)(dh & 0xff); o[1] = (uint8_t)(dh >> 8);
            o[2] = (uint8_t)(mh & 0xff); o[3] = (uint8_t)(mh >> 8);
            uint8_t* s = o + 4;
            for (int j = 0; j < 4; ++j) {
                s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
                s[j + 4] = (uint8_t)((mm[j] & 63) | ((mm[j + 4] >> 4) << 6));
                s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mm[j + 4] & 15) << 4));
            }
            uint8_t q[256];
            for (int j = 0; j < 8; ++j) {
                float ds = d * (float)sc[j], dm = dmin * (float)mm[j];
                for (int l = 0; l < 32; ++l) {
                    float qf = ds > 0.0f ? rintf((v[j * 32 + l] + dm) / ds) : 0.0f;
                    if (qf < 0.0f) qf = 0.0f;
                    if (qf > 15.0f) qf = 15.0f;
                    q[j * 32 + l] = (uint8_t)qf;
                }
            }
            for (int part = 0; part < 4; ++part)
                for (int l = 0; l < 32; ++l)
                    o[16 + part * 32 + l] = (uint8_t)(q[part * 64 + l] | (q[part * 64 + 32 + l] << 4));
        }
    }
}

/* ------------------------------------------------------------------------ */
/* UnifiedSampling: src/backends/cpu/kernel/sampling/unified_sampling.rs     */
/* ------------------------------------------------------------------------ */

/* Philox4x32-10 (Salmon et al., SC'11) as src/encodable_block/sampling/gumbel.rs:1-57 */
void so_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c[4] = {ctr_in[0], ctr_in[1], ctr_in[2], ctr_in[3]};
    uint32_t k[2] = {key_in[0], key_in[1]};
    for (int round = 0; round < 10; ++round) {
        if (round) {
            k[0] += 0x9E3779B9u;
            k[1] += 0xBB67AE85u;
        }
        const uint64_t p0 = (uint64_t)0xD2511F53u * c[0], p1 = (uint64_t)0xCD9E8D57u * c[2];
        const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0, hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        const uint32_t n0 = hi1 ^ c[1] ^ k[0], n2 = hi0 ^ c[3] ^ k[1];
        c[0] = n0;
        c[1] = lo1;
        c[2] = n2;
        c[3] = lo0;
    }
    memcpy(out, c, sizeof c);
}

/* gumbel.rs:49-57: uniform in [2^-24, 1 - 2^-24] from the top 24 bits of a word */
float so_unit_interval(uint32_t word) {
    uint32_t v = word >> 8;
    if (v < 1) v = 1;
    return (float)v * (1.0f / 16777216.0f);
}

/* gumbel.rs:59-79: -ln(-ln u) of word `word` of Philox(ctr = (offset, 0, 0, 0), key = seed) */
float so_gumbel(uint64_t seed, uint32_t logit_index, uint32_t vocab) {
    const uint32_t thread_idx = logit_index % 1024u;
    const uint32_t thread_offset = ((vocab + 4096u - 1u) / 4096u) * thread_idx;
    const uint32_t block_idx = logit_index / 1024u;
    const uint32_t offset = thread_offset + block_idx / 4u, word = block_idx % 4u;
    const uint32_t ctr[4] = {offset, 0, 0, 0}, key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t out[4];
    so_philox4x32_10(ctr, key, out);
    return -logf(-logf(so_unit_interval(out[word])));
}

typedef struct {
    float value;
    uint32_t index;
} so_scored;

static int so_scored_desc(const void* a, const void* b) {
    const so_scored* x = (const so_scored*)a;
    const so_scored* y = (const so_scored*)b;
    /* b.1.partial_cmp(&a.1).unwrap_or(Equal).then(a.0.cmp(&b.0)) */
    if (x->value > y->value) return -1;
    if (x->value < y->value) return 1;
    return x->index < y->index ? -1 : (x->index > y->index ? 1 : 0);
}

/* unified_sampling.rs:14-117, one batch row after another. Options are
 * passed as flags plus values; seeds / bitmask may be NULL when unused. */
int so_unified_sampling(const void* logits, int dt, uint32_t* output, const uint64_t* seeds, const uint32_t* bitmask,
                        int has_temperature, float temperature, int has_top_k, uint32_t top_k, int has_top_p,
                        float top_p, int has_min_p, float min_p, uint32_t vocab, uint32_t batch) {
    float* l = (float*)malloc(sizeof(float) * vocab);
    so_scored* sorted = (so_scored*)malloc(sizeof(so_scored) * vocab);
    if (!l || !sorted) {
        free(l);
        free(sorted);
        return 1;
    }
    const uint32_t words = (vocab + 31u) / 32u;
    for (uint32_t b = 0; b < batch; ++b) {
        int bad = 0;
        for (uint32_t i = 0; i < vocab; ++i) {
            l[i] = read_f32(logits, dt, (size_t)b * vocab + i);
            if (!isfinite(l[i])) bad = 1;
        }
        if (bad) {
            output[b] = 0xffffffffu;
            continue;
        }
        if (bitmask)
            for (uint32_t i = 0; i < vocab; ++i)
                if ((bitmask[(size_t)b * words + i / 32] & (1u << (i % 32))) == 0) l[i] = -INFINITY;
        if (has_temperature) {
            const float recip = 1.0f / temperature;
            int center = 0;
            for (uint32_t i = 0; i < vocab; ++i)
                if (isfinite(l[i]) && !isfinite(l[i] * recip)) center = 1;
            float shift = 0.0f;
            if (center) {
                shift = -INFINITY;
                for (uint32_t i = 0; i < vocab; ++i) shift = fmaxf(shift, l[i]);
            }
            for (uint32_t i = 0; i < vocab; ++i) {
                if (center) l[i] -= shift;
                l[i] *= recip;
            }
        }
        if (has_top_k || has_top_p || has_min_p) {
            for (uint32_t i = 0; i < vocab; ++i) sorted[i] = (so_scored){l[i], i};
            qsort(sorted, vocab, sizeof(so_scored), so_scored_desc);
            const float mx = sorted[0].value;
            float norm = 0.0f;
            for (uint32_t i = 0; i < vocab; ++i) norm += expf(sorted[i].value - mx);
            for (uint32_t i = 0; i < vocab; ++i) l[i] = -INFINITY;
            float mass = 0.0f;
            for (uint32_t r = 0; r < vocab; ++r) {
                if ((has_top_k && r >= top_k) || (has_top_p && mass >= top_p) ||
                    (has_min_p && sorted[r].value < mx + logf(min_p)))
                    break;
                l[sorted[r].index] = sorted[r].value;
                mass += expf(sorted[r].value - mx) / norm;
            }
        }
        if (seeds)
            for (uint32_t i = 0; i < vocab; ++i) l[i] += so_gumbel(seeds[b], i, vocab);
        /* max_by(partial_cmp.then(b.0.cmp(&a.0))): the largest value, the lowest index among equals */
        uint32_t best = 0;
        for (uint32_t i = 1; i < vocab; ++i)
            if (l[i] > l[best]) best = i;
        output[b] = isfinite(l[best]) ? best : 0xffffffffu;
    }
    free(l);
    free(sorted);
    return 0;
}
