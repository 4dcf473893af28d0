/*
 * stark_oracle.h -- CPU restatement of the reference's quantized-matmul semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP path
 * and the CPU baseline timed by bench.py. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it. The product library
 * (stark_amd/libstark_qmm.so) never links or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root). Compiled with -ffp-contract=off so that each
 * `a * b + c` rounds twice, as Rust does (Rust never contracts to FMA unless
 * `mul_add` is written, and the restated code marks those places).
 */
#ifndef STARK_ORACLE_H
#define STARK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype ids follow the GGUF kind numbers the hybrid engine uses for planes. */
enum { SO_F32 = 0, SO_F16 = 1, SO_BF16 = 30 };
enum { SO_LAYOUT_OUTPUT_GROUP = 0, SO_LAYOUT_GROUP_OUTPUT = 1 };
enum { SO_CORR_SYMMETRIC = 0, SO_CORR_BIASES = 1, SO_CORR_ZERO_POINTS = 2 };

/* half 2.7.1 conversions (Cargo.lock:897-899). */
float so_bf16_to_f32(uint16_t h);
uint16_t so_f32_to_bf16(float f);
float so_f16_to_f32(uint16_t h);
uint16_t so_f32_to_f16(float f);
void so_f32_to_bf16_n(const float* src, uint16_t* dst, size_t n);
void so_bf16_to_f32_n(const uint16_t* src, float* dst, size_t n);
void so_f32_to_f16_n(const float* src, uint16_t* dst, size_t n);
void so_f16_to_f32_n(const uint16_t* src, float* dst, size_t n);

/* backends/cpu/kernel/matmul/reference.rs:91-104 */
uint8_t so_packed_code(const uint8_t* codes, int bits, size_t index);

/* Plane strides derived as backends/common/kernel/matmul/mod.rs:109-156 does. */
void so_quant_strides(int layout, uint32_t row_count, uint32_t group_count, uint32_t packing_divisor,
                      uint32_t* output_stride, uint32_t* group_stride);

typedef struct so_matmul_args {
    /* A: FullPrecision values (+offset elements) in input_dt */
    const void* a;
    size_t a_offset;
    /* B: full precision when codes == NULL (values in weights_dt, row-major
     * [n, ld] if b_transpose else [k, ld]; ld 0 selects k or n) */
    const void* b_values;
    uint32_t b_leading_dimension;
    /* B: quantized */
    const uint8_t* codes;
    size_t codes_size;
    const void* scales;      /* weights_dt */
    int correction;          /* SO_CORR_* */
    const void* correction_data; /* biases (weights_dt) or zero points (packed u8) */
    int layout;
    uint32_t row_count, group_count;
    int materialize_affine_input_sum;
    int bits;
    uint32_t group_size;
    int signed_codes;
    int b_transpose;
    /* D */
    void* d;
    float ab_scale;
    int accumulate;
    const void* bias;        /* weights_dt, indexed by output column */
    int has_soft_cap;
    float soft_cap;
    const uint32_t* gather_indices; /* [m*n] or NULL */
    uint32_t m, n, k;
    int weights_dt, input_dt, output_dt;
    /* MatmulA::Int8Symmetric (src/backends/common/kernel/matmul/matmul_a.rs:51-61):
     * a_codes non-NULL replaces the FullPrecision A: int8 codes [m, k] in
     * a_code_layout order, f32 scales [m, k / a_scale_group_size] */
    const int8_t* a_codes;
    const float* a_scales;
    uint32_t a_scale_group_size;
    int a_grouped_by_nibble;
    /* MatmulDOps::rht_factors: output RHT then bias (kernel.rs:167, 287-300) */
    const int32_t* rht_factors;
} so_matmul_args;

/* Status: 0 ok, 1 unsupported layout (undersized codes / policy), 2 unsupported
 * dtype, 3 incompatible A (int8 activations with unsupported groups or codes),
 * 4 unsupported D-op (output RHT on an f16 output or a width not a multiple of 32). */
int so_matmul(const so_matmul_args* args);
/* Row-parallel variant (OpenMP over output columns); identical arithmetic per output. */
int so_matmul_parallel(const so_matmul_args* args, int threads);

/* encodable_block/mlp/routed.rs:154-257 (RoutedExperts::encode_scaled): route
 * (moe.rs:24-85), optional adjust (moe.rs:147-184; unit gains when only
 * sort_ids is set, routed.rs:205-208), then per (row, rank) in order: gathered
 * up product [2*hidden] (bf16 out), gated SiLU, gathered down product [model]
 * (bf16 out), accumulate (moe.rs:109-145). Banks are MLX affine with planes in
 * `plane_dt`; biases NULL selects the symmetric correction. Returns so_matmul's
 * status (0 ok). */
int so_routed_experts(const uint16_t* input, const float* logits, const float* expert_scales,
                      const uint8_t* up_codes, const void* up_scales, const void* up_biases,
                      const uint8_t* down_codes, const void* down_scales, const void* down_biases, int layout,
                      int bits, uint32_t group_size, int plane_dt, uint32_t rows, uint32_t model, uint32_t hidden,
                      uint32_t experts, uint32_t active, int round_logits, int round_weights, int round_products,
                      int round_accumulator, int sort_ids, uint16_t* output);

/* ---- activation transforms (src/backends/cpu/kernel/activation_transform/) */
/* mod.rs:28-43: the 32-point Walsh-Hadamard butterfly, then * 1/sqrt(32). */
void so_hadamard32(float* values);
/* mod.rs:9-26 */
float so_min_max_symmetric_divisor(const float* values, size_t count);
int8_t so_quantize_symmetric_i8(float value, float divisor);
/* Int8CodeLayout::index (src/backends/common/kernel/matmul/matmul_a.rs:31-46) */
size_t so_int8_code_index(int grouped_by_nibble, size_t index);
/* ActivationTransformOp (src/backends/common/gpu_types/activation_transform.rs:3-8) */
enum { SO_INPUT_RHT = 0, SO_OUTPUT_RHT = 1, SO_QUANTIZE = 2, SO_QUANTIZE_WITH_GROUP_SUMS = 3 };
/* activation_transform.rs:48-156. T (t_dt) and BiasT (bias_dt) are F32 or
 * BF16; in_place reads fp_out. Returns 0, or 1 for a width not a multiple of 32. */
int so_activation_transform(const void* input, void* fp_out, const void* bias, int8_t* q_out, float* scales_out,
                            int32_t* group_sums_out, const int32_t* rht_factors, uint32_t batch_size,
                            uint32_t element_count, int op, int grouped_by_nibble, int in_place,
                            uint32_t scale_group_size, uint32_t sum_group_size, int t_dt, int bias_dt);
/* ActivationType (src/backends/common/gpu_types/activation_type.rs:8-16) */
enum { SO_SILU = 0, SO_GELU_APPROX = 1, SO_GELU_EXACT = 2, SO_IDENTITY = 3, SO_SOFTPLUS = 4,
       SO_SILU_MATERIALIZED_SIGMOID = 5, SO_GELU_MATERIALIZED_POLYNOMIAL = 6 };
/* ActivationType::activate / activation_silu_alpha (activation_type.rs:19-111)
 * on a value stored in t_dt, result rounded to t_dt. */
float so_activate(int act_type, float x, int t_dt, int has_alpha, float alpha);
/* GatedActMulOp (src/backends/common/gpu_types/gated_act_mul.rs:3-7) */
enum { SO_GAM_FULL_PRECISION = 0, SO_GAM_QUANTIZE = 1, SO_GAM_QUANTIZE_WITH_GROUP_SUMS = 2 };
/* src/backends/cpu/kernel/gated_act_mul/gated_act_mul.rs:17-152. Returns 0, or
 * 1 when the op's preconditions fail (quantize without RHT, widths). */
int so_gated_act_mul(const void* act_operand, const void* value_operand, void* fp_out, int8_t* q_out,
                     float* scales_out, int32_t* group_sums_out, const int32_t* hadamard_factors,
                     uint32_t gated_dim, uint32_t batch_dim, uint32_t value_offset, uint32_t value_row_stride,
                     int act_type, int has_alpha, float alpha, int clip_gate, float gate_min, float gate_max,
                     int clip_value, float value_min, float value_max, int op, int grouped_by_nibble,
                     int interleaved, int use_hadamard, uint32_t scale_group_size, uint32_t sum_group_size,
                     int t_dt);

/* backends/cpu/kernel/matmul/vision.rs:249-336 (BF16-effective reference dot). */
void so_reference_affine_linear_bf16(const uint16_t* input, const uint8_t* weights, const uint16_t* scales,
                                     const uint16_t* biases, const uint32_t* indices, uint16_t* bf16_output,
                                     float* f32_output, uint32_t m, uint32_t n, uint32_t k, uint32_t bank_rows,
                                     uint32_t bits, uint32_t scale_output_stride, uint32_t scale_group_stride);

/* engine/hybrid/weights.rs:2565-2584, 2908-2921, 2923-3012 (kinds 0,1,30,8,12,13). */
int so_block_layout(uint32_t kind, size_t* elements, size_t* bytes);
void so_scale_min(const uint8_t* scales, int index, uint8_t* scale, uint8_t* min);
int so_decode_block(uint32_t kind, const uint8_t* bytes, size_t nbytes, float* output, size_t count);
/* weights.rs:2533-2550: per row decode_values(...) . input, f32 sequential sum. */
int so_decode_rows(uint32_t kind, const uint8_t* bytes, size_t rows, size_t columns, float* output);
int so_hybrid_packed_matvec(uint32_t kind, const uint8_t* bytes, size_t rows, size_t columns, const float* input,
                            float* output);
/* weights.rs:1284-1309 affine_row . input (OutputGroup [N,G] planes). */
int so_hybrid_affine_matvec(const uint8_t* codes, const void* scales, const void* biases, int scale_dt, int bits,
                            size_t group, size_t rows, size_t columns, const float* input, float* output);

/* backends/cpu/kernel/moe.rs */
void so_moe_route(const float* logits, uint32_t* ids, float* weights, uint32_t rows, uint32_t experts,
                  uint32_t active, uint32_t round_weights, uint32_t round_logits);
void so_moe_gather_rows(const uint32_t* ids, uint32_t* indices, uint32_t route_offset, uint32_t rows_per_expert,
                        uint32_t experts, uint32_t length);
void so_moe_accumulate(const uint16_t* input, const float* weights, float* accumulator, uint16_t* output,
                       uint32_t length, uint32_t weight_offset, uint32_t output_offset, uint32_t initialize,
                       uint32_t finalize, uint32_t round_product, uint32_t round_accumulator);
void so_moe_adjust_routes(uint32_t* ids, float* weights, const float* scales, uint32_t rows, uint32_t experts,
                          uint32_t active, uint32_t sort_ids);
/* backends/cpu/kernel/gated_act_mul/gated_act_mul.rs (interleaved, SiLU, bf16):
 * row layout [value(hidden) | gate(hidden)], out = bf16(value * bf16(silu(gate))). */
void so_gated_silu_bf16(const uint16_t* projected, uint16_t* out, uint32_t hidden, uint32_t batch);

/* Test-input generators (not part of the parity contract: parity is defined on decode). */
void so_quantize_affine(const float* w, size_t rows, size_t cols, int bits, size_t group, int layout,
                        uint8_t* codes, uint16_t* scales, uint16_t* biases);
void so_quantize_q8_0(const float* w, size_t rows, size_t cols, uint8_t* out);
void so_quantize_q4_k(const float* w, size_t rows, size_t cols, uint8_t* out);

/* UnifiedSampling (src/backends/cpu/kernel/sampling/unified_sampling.rs) and its noise
 * (src/encodable_block/sampling/gumbel.rs). */
void so_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float so_unit_interval(uint32_t word);
float so_gumbel(uint64_t seed, uint32_t logit_index, uint32_t vocab);
int so_unified_sampling(const void* logits, int dt, uint32_t* output, const uint64_t* seeds, const uint32_t* bitmask,
                        int has_temperature, float temperature, int has_top_k, uint32_t top_k, int has_top_p,
                        float top_p, int has_min_p, float min_p, uint32_t vocab, uint32_t batch);

#ifdef __cplusplus
}
#endif
#endif
