/*
 * stark_qmm.h -- C ABI of the MI355X (gfx950) quantized matrix-product path.
 *
 * This is the drop-in boundary for the reference engine's quantized matmul
 * operators. Every entry point names the reference interface it replaces
 * (paths relative to the reference root, `crates/stark-engine/src/` written
 * as `src/`). Conventions follow the reference's own C bridge
 * (vendor/glm-exl3-bridge/include/stark_glm.h:11-31): a status enum, an ABI
 * version constant, opaque handles, plain pointers and sizes.
 *
 * Memory: all tensor pointers are DEVICE pointers owned by the caller and
 * borrowed for the duration of the (stream-ordered) call. The library never
 * frees caller memory. `stream` is a hipStream_t passed as void* (NULL = the
 * default stream). Work is asynchronous on that stream unless an entry point
 * says otherwise. No entry point allocates device memory or waits for the
 * device on its stream-ordered path, with these documented exceptions:
 * stark_qmm_mapped_many (synchronous, as the reference; one 256-byte status
 * word per device on first use), and the matvec schedule store: the first
 * call on a new shape set enqueues small upload launches on the caller's
 * stream into a fixed 4 MiB device array per GPU (no allocation); when that
 * array is full, an eager call synchronizes the device once and drops the
 * schedules no captured graph references (a capturing call returns
 * STARK_QMM_OUT_OF_MEMORY instead). Calls are capture-safe (hipStreamBeginCapture).
 *
 * Threading: a handle is not reentrant (the reference keeps each kernel object
 * behind a Mutex, src/encodable_block/linear/matmul.rs:42); distinct handles
 * may be used concurrently.
 */
#ifndef STARK_QMM_H
#define STARK_QMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define STARK_QMM_ABI_VERSION 2u

/* The library is built with hidden visibility; only these entry points are exported. */
#if defined(__GNUC__)
#define STARK_QMM_API __attribute__((visibility("default")))
#else
#define STARK_QMM_API
#endif

typedef uint32_t stark_qmm_status;
enum {
    STARK_QMM_OK = 0,
    /* hybrid Error::Invalid (src/engine/hybrid/weight_metal.rs:435-537) and malformed arguments */
    STARK_QMM_INVALID_ARGUMENT = 1,
    STARK_QMM_ABI_MISMATCH = 2,
    /* MatmulError::UnsupportedDataType (src/backends/common/kernel/matmul/error.rs:12) */
    STARK_QMM_UNSUPPORTED_DATA_TYPE = 3,
    /* MatmulError::UnsupportedGroupSize (error.rs:14) */
    STARK_QMM_UNSUPPORTED_GROUP_SIZE = 4,
    /* MatmulError::UnsupportedDOp (error.rs:16-19) */
    STARK_QMM_UNSUPPORTED_D_OP = 5,
    /* MatmulError::UnsupportedLayout (error.rs:20-23), e.g. an undersized codes buffer */
    STARK_QMM_UNSUPPORTED_LAYOUT = 6,
    /* MatmulError::IncompatibleA (error.rs:24-28) */
    STARK_QMM_INCOMPATIBLE_A = 7,
    /* hybrid Error::Unsupported */
    STARK_QMM_UNSUPPORTED = 8,
    STARK_QMM_OUT_OF_MEMORY = 9,
    /* MatmulError::BackendError (error.rs:29-30): a HIP call failed */
    STARK_QMM_DEVICE_FAILURE = 10,
    /* caller workspace smaller than the size query returned */
    STARK_QMM_WORKSPACE_TOO_SMALL = 11,
    /* ParameterLoaderError::KeyNotFound (src/parameters/error.rs:11-12) */
    STARK_QMM_KEY_NOT_FOUND = 12,
    /* ParameterLoaderError::InvalidTensor / InvalidTensorSize (error.rs:19-32) */
    STARK_QMM_INVALID_TENSOR = 13,
    /* ParameterLoaderError::HeaderLoadingError (src/parameters/safetensors_metadata.rs:14-39) */
    STARK_QMM_HEADER_ERROR = 14,
    /* ParameterLoaderError::ArrayLoadingError: the file could not be read (error.rs:15-16) */
    STARK_QMM_IO_ERROR = 15,
    /* WeightMatrixError::UnsupportedConfiguration (src/encodable_block/weight_matrix.rs:22-28) */
    STARK_QMM_UNSUPPORTED_CONFIGURATION = 16
};

/* Data types. The numbers are the GGUF kind ids the hybrid engine already uses
 * for plane dtypes (src/engine/hybrid/weight_metal.rs:486-490). */
enum { STARK_QMM_F32 = 0, STARK_QMM_F16 = 1, STARK_QMM_BF16 = 30 };
/* Integer tensor types of a weight file; the first four are the hybrid
 * engine's private tags (src/engine/hybrid/weights.rs:93-96). */
enum { STARK_QMM_U32 = 101, STARK_QMM_I64 = 102, STARK_QMM_I32 = 103, STARK_QMM_U8 = 104, STARK_QMM_I8 = 105,
       STARK_QMM_U64 = 106 };

/* QuantParamsLayout (src/backends/common/kernel/matmul/mod.rs:19-25). */
enum { STARK_QMM_LAYOUT_OUTPUT_GROUP = 0, /* [N, G] */
       STARK_QMM_LAYOUT_GROUP_OUTPUT = 1  /* [G, round_up_4(N)] */ };

/* QuantizedCorrection (src/backends/common/kernel/matmul/matmul_b.rs:24-29). */
enum { STARK_QMM_CORRECTION_SYMMETRIC = 0, STARK_QMM_CORRECTION_BIASES = 1, STARK_QMM_CORRECTION_ZERO_POINTS = 2 };

/* QuantizationMode (src/backends/common/gpu_types/quantization.rs:9-23). */
enum { STARK_QMM_MODE_U4 = 0, STARK_QMM_MODE_I8 = 1, STARK_QMM_MODE_U8 = 2, STARK_QMM_MODE_U5 = 3,
       STARK_QMM_MODE_U6 = 4, STARK_QMM_MODE_U3 = 5 };

/* Hybrid packed kinds (src/engine/hybrid/weights.rs:2565-2584). */
enum { STARK_QMM_KIND_Q8_0 = 8, STARK_QMM_KIND_Q4_K = 12 };

/* ------------------------------------------------------------------ */
/* Generic engine operator: trait MatmulKernel                         */
/* (src/backends/common/kernel/matmul/kernel.rs:15-79)                 */
/* ------------------------------------------------------------------ */

typedef struct stark_qmm_kernel stark_qmm_kernel;

/* QuantParams (src/backends/common/kernel/matmul/mod.rs:33-41). */
typedef struct stark_qmm_quant_params {
    uint32_t layout;      /* STARK_QMM_LAYOUT_* */
    uint32_t row_count;   /* N of the stored planes */
    uint32_t group_count; /* G = K / group_size */
    uint32_t materialize_affine_input_sum; /* MLXSpec flag (src/config/weight_matrix/mlx_spec.rs:10-12) */
} stark_qmm_quant_params;

/* MatmulB (src/backends/common/kernel/matmul/matmul_b.rs:6-22). `codes == NULL`
 * selects MatmulB::FullPrecision with `values` in the kernel's weights dtype. */
typedef struct stark_qmm_b {
    const void* values;        /* FullPrecision only */
    const void* codes;         /* packed codes, [N, K*bits/8] bytes */
    uint64_t codes_size;       /* bytes available at codes (validated as reference.rs:62-71) */
    const void* scales;        /* weights dtype, plane per params.layout */
    uint32_t correction;       /* STARK_QMM_CORRECTION_* */
    const void* correction_data; /* biases (weights dtype) or packed zero points (u8) */
    stark_qmm_quant_params params;
    uint32_t mode;             /* STARK_QMM_MODE_* */
    uint32_t group_size;
    uint32_t signed_codes;
} stark_qmm_b;

/* MatmulDOps (src/backends/common/kernel/matmul/d_ops.rs:3-9). */
typedef struct stark_qmm_d_ops {
    float ab_scale;           /* 1.0 for none */
    uint32_t accumulate;      /* d = ... + d */
    const void* bias;         /* [N] in the weights dtype, or NULL */
    /* int32 signs [N]: output RHT (32-point Walsh-Hadamard of each 32 outputs
     * of a row, times the signs), applied to d after the product, then the
     * bias (kernel.rs:167, 287-300). F32 / BF16 outputs with N % 32 == 0;
     * otherwise STARK_QMM_UNSUPPORTED_D_OP. */
    const void* rht_factors;
    uint32_t has_soft_cap;
    float soft_cap;
} stark_qmm_d_ops;

/* MatmulArguments (src/backends/common/kernel/matmul/arguments.rs:7-25). */
/* MatmulA (src/backends/common/kernel/matmul/matmul_a.rs:51-61) and
 * Int8CodeLayout (matmul_a.rs:6-9). */
enum { STARK_QMM_A_FULL_PRECISION = 0, STARK_QMM_A_INT8_SYMMETRIC = 1 };
enum { STARK_QMM_CODES_SEQUENTIAL = 0, STARK_QMM_CODES_GROUPED_BY_NIBBLE = 1 };

typedef struct stark_qmm_args {
    uint32_t struct_size;     /* sizeof(stark_qmm_args) */
    const void* a;            /* FullPrecision: values [M, K] in the input dtype; Int8Symmetric: int8 codes [M, K] */
    uint64_t a_offset;        /* element offset into a (FullPrecision) */
    /* MatmulA::Int8Symmetric: codes in a (in a_code_layout order), f32 scales
     * [M, K / a_scale_group_size]; a_group_sums may be NULL. Requires a
     * quantized 4- or 8-bit B with group 32, 64 or 128 and an activation
     * group of 32, 64 or 128 dividing K (kernel.rs:130-141), else
     * STARK_QMM_INCOMPATIBLE_A. */
    uint32_t a_kind;          /* STARK_QMM_A_* */
    const float* a_scales;
    const int32_t* a_group_sums;
    uint32_t a_scale_group_size;
    uint32_t a_code_layout;   /* STARK_QMM_CODES_* */
    stark_qmm_b b;
    uint32_t b_leading_dimension; /* FullPrecision B only; 0 = default */
    uint32_t b_transpose;     /* must be 1 for quantized B (the only layout the path uses) */
    void* d;                  /* [M, N] in the output dtype */
    stark_qmm_d_ops d_ops;
    const uint32_t* gather_indices; /* [M*N] weight row per output, or NULL */
    uint32_t m, n, k;
} stark_qmm_args;

/* Replaces MatmulKernel::new (kernel.rs:18-23; CPU twin
 * src/backends/cpu/kernel/matmul/kernel.rs:31-56): F32/F16/BF16 only. */
STARK_QMM_API stark_qmm_status stark_qmm_create(uint32_t weights_dtype, uint32_t input_dtype, uint32_t output_dtype,
                                  stark_qmm_kernel** out);

/* Replaces MatmulKernel::encode (kernel.rs:51-62; Metal dispatch
 * src/backends/metal/kernel/matmul/mod.rs:551-613). Chooses the GEMV/verify
 * path for M <= 16 and the MFMA dequant-GEMM for larger M. */
STARK_QMM_API stark_qmm_status stark_qmm_encode(stark_qmm_kernel* kernel, const stark_qmm_args* args, void* stream);

/* Independent products with one submission, in the manner of the hybrid
 * engine's Weights::matvec_many (src/engine/hybrid/weights.rs:1323-1388): every
 * args[i] is validated as stark_qmm_encode would, then all eligible GEMV
 * products share one launch per (bits, M class) and the dequant-GEMM products
 * (M > 16) one per (bits, signed codes, correction, plane type). Outputs must
 * not alias inputs or outputs of other entries. */
STARK_QMM_API stark_qmm_status stark_qmm_encode_many(stark_qmm_kernel* kernel, const stark_qmm_args* args, uint32_t count,
                                       void* stream);

/* Input prologue of a batched product. No counterpart in the reference: its
 * decoder runs the RMS norm and the gated activation as kernels of their own
 * ahead of the products that read them. This entry point is for decode loops
 * that want those folded into the products' activation staging, saving one
 * launch and one round trip of the row each:
 *   STARK_QMM_PROLOGUE_RMS_NORM:  a' = bf16(bf16(a * r) * w[k]),
 *       r = 1 / sqrt(sum(a^2) / K + eps), w = data (bf16 [K]);
 *   STARK_QMM_PROLOGUE_SILU_GATE: a' = bf16(up[k] * bf16(a / (1 + exp(-a)))),
 *       up = data (bf16 [K]) -- GatedActMul's SiLU with no alpha or clips.
 * The transformed row is bit-identical to the one the separate kernel writes. */
enum { STARK_QMM_PROLOGUE_NONE = 0, STARK_QMM_PROLOGUE_RMS_NORM = 1, STARK_QMM_PROLOGUE_SILU_GATE = 2 };

typedef struct stark_qmm_prologue {
    uint32_t struct_size;   /* sizeof(stark_qmm_prologue) */
    uint32_t kind;          /* STARK_QMM_PROLOGUE_* */
    const void* data;       /* bf16 [K], 16-byte aligned */
    float eps;              /* RMS norm only */
} stark_qmm_prologue;

/* stark_qmm_encode_many with a prologue on the shared input row: every
 * args[i] is a FullPrecision-A product with the same a (and a_offset) and K,
 * BF16 input, M = 1, 4-bit codes with group 64, K % 4096 == 0, N >= 32, no
 * gather, no output RHT, at most 8 entries; anything else returns
 * STARK_QMM_UNSUPPORTED (so do a kernel in reference-accumulation mode and
 * STARK_QMM_PROLOGUE_NONE). Outputs must not alias the row or data. */
STARK_QMM_API stark_qmm_status stark_qmm_encode_many_prologue(stark_qmm_kernel* kernel, const stark_qmm_args* args,
                                                            uint32_t count, const stark_qmm_prologue* prologue,
                                                            void* stream);

/* Chained products: several dependent stages of one-row products in ONE
 * persistent launch. No counterpart in the reference, whose decoder encodes
 * every product of a layer as a dispatch of its own
 * (crates/stark-engine/src/encodable_block/transformer_layer.rs); this is for
 * decode loops that want a layer's o -> gate/up -> down -> next q/k/v products
 * without a launch boundary (and its fixed cost) between them. Each product
 * computes exactly what stark_qmm_encode_many_prologue computes for it.
 *
 * Rows handed from one stage to a later one are TAGGED: one 32-bit word per
 * element, bf16 value in the low half and a tag (1..0x7fff) in the high half.
 * A product whose in_tag is non-zero reads tagged a (and, with the SiLU-gate
 * prologue, tagged up values) and waits until every word it reads carries
 * in_tag; one whose out_tag is non-zero writes tagged d. Plain rows (tag 0)
 * must be complete before the launch. A stage may read only rows written by
 * earlier stages or before the launch, and every element of a tagged row must
 * be rewritten with another tag between two writes of the same tag: reusing
 * the same tags in consecutive calls needs `seq`, a device word whose low bit
 * differs between the calls (it flips bit 15 of every tag; NULL = no flip).
 *
 * k_slices > 1 splits the product's K into that many slices of 4096 whose row
 * sums meet in the workspace as words tagged part_tag (same rule as the row
 * tags) and are added in slice order (bit-identical to
 * stark_qmm_encode_many_prologue for K = 12288 and 3 slices); d may then be
 * plain or tagged. Requirements: BF16 input/output/planes with biases, M = 1,
 * 4-bit codes, group 64, K % 4096 == 0 (the RMS-norm prologue: K == 4096),
 * N % 32 == 0, no gather, bias, soft cap or RHT; at most 16 tiles lists
 * (products plus extra slices). Otherwise STARK_QMM_UNSUPPORTED.
 *
 * Every wait is bounded: a wait that gives up (about 0.1 s) sets the status
 * word at workspace offset 0 non-zero (the caller clears it) and the rows of
 * that launch are invalid. The launch needs every workgroup resident at once:
 * do not run it concurrently with other kernels on the same device. */
typedef struct stark_qmm_chain_product {
    uint32_t struct_size;         /* sizeof(stark_qmm_chain_product) */
    uint32_t stage;               /* stages run in increasing order */
    const stark_qmm_args* args;   /* the product (a/d tagged as in_tag/out_tag say) */
    uint32_t prologue;            /* STARK_QMM_PROLOGUE_* */
    const void* prologue_data;    /* RMS norm: bf16 weights; SiLU gate: up row, in a's format */
    float eps;
    uint32_t in_tag, out_tag;     /* 0 = plain bf16 row */
    uint32_t acc_tag;             /* tagged d with accumulate: tag d carries before it is read (0: at launch) */
    uint32_t k_slices;            /* 0 or 1: whole K */
    uint32_t part_tag;            /* k_slices > 1: tag of the slices' partial sums (1..0x7fff) */
} stark_qmm_chain_product;

/* Workspace bytes stark_qmm_encode_chain needs for these products. */
STARK_QMM_API stark_qmm_status stark_qmm_chain_workspace_size(const stark_qmm_chain_product* products, uint32_t count,
                                                            uint64_t* bytes);

STARK_QMM_API stark_qmm_status stark_qmm_encode_chain(stark_qmm_kernel* kernel, const stark_qmm_chain_product* products,
                                                    uint32_t count, const uint32_t* seq, void* workspace,
                                                    uint64_t workspace_bytes, void* stream);

/* Replaces MatmulKernel::set_reference_accumulation (kernel.rs:34-37): when
 * enabled, every M uses the GEMV/verify kernels (f32 dequant semantics). */
STARK_QMM_API stark_qmm_status stark_qmm_set_reference_accumulation(stark_qmm_kernel* kernel, uint32_t enabled);

STARK_QMM_API void stark_qmm_destroy(stark_qmm_kernel* kernel);

STARK_QMM_API uint32_t stark_qmm_abi_version(void);
/* Text for a status code; never NULL. */
STARK_QMM_API const char* stark_qmm_status_string(stark_qmm_status status);

/* ------------------------------------------------------------------ */
/* Hybrid engine operator: weight_metal::mapped_many                   */
/* (src/engine/hybrid/weight_metal.rs:376-392, 539-545)                */
/* ------------------------------------------------------------------ */

/* MatrixFormat (weight_metal.rs:376-383). */
enum { STARK_QMM_FORMAT_PACKED = 0, STARK_QMM_FORMAT_AFFINE = 1 };

/* MappedMatrix: one matrix view. Affine planes are [rows, G] (native MLX). */
typedef struct stark_qmm_mapped_matrix {
    const void* codes;
    uint64_t codes_length;  /* bytes */
    const void* scales;     /* affine only */
    const void* biases;     /* affine only */
    uint64_t plane_length;  /* bytes of each plane; 0 for packed */
} stark_qmm_mapped_matrix;

/* MappedOperation (weight_metal.rs:385-392). inputs: [batches, columns] f32
 * where batches = matrix_count, or rows / rows_per_batch when rows_per_batch
 * != 0 (a single matrix). Output: [matrix_count * rows] f32. */
typedef struct stark_qmm_mapped_op {
    const stark_qmm_mapped_matrix* matrices; /* HOST array of matrix views */
    uint32_t matrix_count;
    const float* inputs;    /* device */
    uint64_t input_length;  /* floats */
    uint64_t rows, columns, rows_per_batch;
    uint32_t format;        /* STARK_QMM_FORMAT_* */
    uint32_t packed_kind;   /* STARK_QMM_KIND_* for packed */
    uint32_t scale_dtype;   /* affine: STARK_QMM_F32 / F16 / BF16 */
    uint32_t bits;          /* affine: 4 or 8 */
    uint32_t group;         /* affine: 32, 64 or 128 */
} stark_qmm_mapped_op;

/* Replaces mapped_many (weight_metal.rs:539-545). Thread-safe: concurrent calls on one
 * device serialize on that device's status word. Validates every operation as
 * parameters_for_input does (weight_metal.rs:442-537; at most 64 ops), runs all
 * of them in one launch per format, and -- like the reference -- returns only
 * after the work completes. A non-finite input makes the call return
 * STARK_QMM_INVALID_ARGUMENT (weight_metal.rs:435-440); outputs are then
 * unspecified. outputs[i] is a device pointer with room for
 * matrix_count * rows floats. */
STARK_QMM_API stark_qmm_status stark_qmm_mapped_many(const stark_qmm_mapped_op* ops, uint32_t op_count, float* const* outputs,
                                       void* stream);

/* Asynchronous form of stark_qmm_mapped_many: no host wait. The finite check
 * ORs 1 into *status_word (device u32, caller-zeroed) when any input is not
 * finite. */
STARK_QMM_API stark_qmm_status stark_qmm_mapped_many_async(const stark_qmm_mapped_op* ops, uint32_t op_count,
                                             float* const* outputs, uint32_t* status_word, void* stream);

/* ------------------------------------------------------------------ */
/* MoE kernels (src/backends/cpu/kernel/moe.rs; Metal                   */
/* src/backends/metal/kernel/moe.metal)                                 */
/* ------------------------------------------------------------------ */

/* MoeRoute (moe.rs:23-85, moe.metal:13-50): softmax over experts, repeated
 * argmax top-k (ties to the lowest id), renormalised weights. */
STARK_QMM_API stark_qmm_status stark_qmm_moe_route(const float* logits, uint32_t* ids, float* weights, uint32_t rows,
                                     uint32_t experts, uint32_t active, uint32_t round_weights,
                                     uint32_t round_logits, void* stream);

/* MoeAdjustRoutes (moe.rs:147-184, moe.metal:88-104). */
STARK_QMM_API stark_qmm_status stark_qmm_moe_adjust_routes(uint32_t* ids, float* weights, const float* scales, uint32_t rows,
                                             uint32_t experts, uint32_t active, uint32_t sort_ids, void* stream);

/* MoeGatherRows (moe.rs:87-107, moe.metal:52-63). */
STARK_QMM_API stark_qmm_status stark_qmm_moe_gather_rows(const uint32_t* ids, uint32_t* indices, uint32_t route_offset,
                                           uint32_t rows_per_expert, uint32_t experts, uint32_t length,
                                           void* stream);

/* MoeAccumulate (moe.rs:109-145, moe.metal:65-86). input/output are bf16. */
STARK_QMM_API stark_qmm_status stark_qmm_moe_accumulate(const void* input, const float* weights, float* accumulator,
                                          void* output, uint32_t length, uint32_t weight_offset,
                                          uint32_t output_offset, uint32_t initialize, uint32_t finalize,
                                          uint32_t round_product, uint32_t round_accumulator, void* stream);

/* RoutedExperts::encode_scaled (src/encodable_block/mlp/routed.rs:154-257) as
 * one fused device pipeline: route -> (optional) adjust -> expert-index
 * compaction (counting sort into expert-major slots, after
 * vendor/lily-core/src/kernels/metal/moe.metal:905-1036) -> grouped gate/up
 * matvec with SiLU gating -> grouped down matvec -> weighted accumulation.
 * Banks flatten [experts, rows, cols] (routed.rs:1-5): up [E*2*hidden, model]
 * with rows [value(hidden) | gate(hidden)] per expert, down [E*model, hidden].
 * Both banks are 4-bit affine (group size 32, 64 or 128) with BF16 scale
 * and bias planes, or symmetric; other banks return STARK_QMM_UNSUPPORTED or
 * STARK_QMM_UNSUPPORTED_GROUP_SIZE. The workspace holds the routes, the
 * compaction tables and the intermediate activations; its contents do not
 * survive the call. */
typedef struct stark_qmm_routed_args {
    uint32_t struct_size;
    const void* input;          /* [rows, model] bf16 */
    const float* router_logits; /* [rows, experts] f32 */
    const float* expert_scales; /* [experts] f32 or NULL */
    stark_qmm_b up;             /* bank [experts*2*hidden, model] */
    stark_qmm_b down;           /* bank [experts*model, hidden] */
    void* output;               /* [rows, model] bf16 */
    uint32_t rows, model, hidden, experts, active;
    uint32_t round_logits_bf16, round_weights_bf16, round_products_bf16, round_accumulator_bf16, sort_expert_ids;
    void* workspace;            /* device, >= stark_qmm_routed_experts_workspace_size() bytes */
    uint64_t workspace_size;
} stark_qmm_routed_args;

STARK_QMM_API uint64_t stark_qmm_routed_experts_workspace_size(uint32_t rows, uint32_t model, uint32_t hidden, uint32_t experts,
                                                 uint32_t active);
STARK_QMM_API stark_qmm_status stark_qmm_routed_experts(const stark_qmm_routed_args* args, void* stream);

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): stark_qmm_routed_experts with the workspace taken from a
 * fixed device array inside the library (one per GPU, held until the process
 * ends); args->workspace and args->workspace_size are ignored. Calls whose
 * stark_qmm_routed_experts_workspace_size() exceeds
 * STARK_QMM_ROUTED_STATIC_SCRATCH_BYTES return STARK_QMM_WORKSPACE_TOO_SMALL.
 * Every call on one GPU shares that array: calls that overlap on one GPU
 * (different streams, or threads) race; serialize them. Allocates nothing. */
#define STARK_QMM_ROUTED_STATIC_SCRATCH_BYTES (8ull << 20)
STARK_QMM_API stark_qmm_status stark_qmm_routed_experts_static(const stark_qmm_routed_args* args, void* stream);

/* ------------------------------------------------------------------ */
/* BF16-effective affine reference dot                                 */
/* ------------------------------------------------------------------ */

typedef struct stark_qmm_reference_affine_args {
    uint32_t struct_size;
    const void* input;           /* bf16 [M, K] at input + input_offset */
    uint64_t input_offset;       /* bytes */
    uint64_t input_size;         /* bytes available at input */
    /* FullPrecision (codes == NULL): bf16 values [bank, K], values_size bytes.
     * Quantized: U4/U5/U6/U8 codes, group 64, bf16 scales and biases (correction
     * BIASES), unsigned codes; the bank is codes_size / (K * bits / 8) rows and
     * params must describe exactly that bank. */
    stark_qmm_b weights;
    uint64_t values_size;
    uint64_t scales_size, biases_size; /* bytes */
    uint32_t source_output_width_count; /* non-zero: a fused-source matrix, which keeps its own route */
    const uint32_t* indices;     /* [M*N] bank row per output, or NULL (row = column, N <= bank) */
    uint64_t indices_size;       /* bytes */
    void* output;                /* [M, N] in output_dtype */
    uint32_t output_dtype;       /* BF16, or F32 = the bf16 result widened */
    uint32_t m, n, k;
} stark_qmm_reference_affine_args;

/* Replaces ReferenceAffineBF16Matmul::encode
 * (src/encodable_block/linear/reference_affine.rs:105-280; kernel
 * src/backends/cpu/kernel/matmul/vision.rs:249-336): w = bf16(code * scale +
 * bias), 32 fma partial sums over K in steps of 32 and the fixed 8x4 tree,
 * bit-identical to the reference. Bounds as ReferenceAffinePlan
 * (reference_affine.rs:55-96); a gathered row outside the bank gives NaN. The
 * caller provides the output (the reference allocates it). */
STARK_QMM_API stark_qmm_status stark_qmm_reference_affine_bf16(const stark_qmm_reference_affine_args* args, void* stream);

/* ------------------------------------------------------------------ */
/* Sampling after the lm_head                                          */
/* ------------------------------------------------------------------ */

typedef struct stark_qmm_sampling_args {
    uint32_t struct_size;
    const void* logits;          /* [batch, vocab] in data_type (F32 or BF16) */
    uint32_t data_type;
    uint32_t* output;            /* [batch] token ids; 0xFFFFFFFF: non-finite logits or nothing left */
    const uint64_t* seeds;       /* [batch] Philox keys: stochastic (Gumbel) sampling; NULL: greedy */
    const uint32_t* bitmask;     /* [batch, ceil(vocab / 32)] allowed tokens, or NULL */
    uint32_t has_temperature;
    float temperature;
    uint32_t has_top_k;
    uint32_t top_k;
    uint32_t has_top_p;
    float top_p;
    uint32_t has_min_p;
    float min_p;
    uint32_t vocab_size, batch_size;
} stark_qmm_sampling_args;

/* Replaces Sampling::encode's UnifiedSampling kernel
 * (src/backends/cpu/kernel/sampling/unified_sampling.rs:14-117; noise
 * src/encodable_block/sampling/gumbel.rs): bitmask, temperature, top-k / top-p /
 * min-p prefix of the sorted logits, Gumbel noise from Philox4x32-10, argmax.
 * Options are validated as SamplingMethod::validate (sampling/mod.rs:73-101). */
STARK_QMM_API stark_qmm_status stark_qmm_unified_sampling(const stark_qmm_sampling_args* args, void* stream);

/* ------------------------------------------------------------------ */
/* Activation transforms and gated activations                        */
/* ------------------------------------------------------------------ */

/* ActivationTransformOp (src/backends/common/gpu_types/activation_transform.rs:3-8) */
enum { STARK_QMM_TRANSFORM_INPUT_RHT = 0, STARK_QMM_TRANSFORM_OUTPUT_RHT = 1, STARK_QMM_TRANSFORM_QUANTIZE = 2,
       STARK_QMM_TRANSFORM_QUANTIZE_WITH_GROUP_SUMS = 3 };

typedef struct stark_qmm_activation_transform_args {
    uint32_t struct_size;
    uint32_t op;                 /* STARK_QMM_TRANSFORM_* */
    uint32_t data_type;          /* T: F32 or BF16 */
    uint32_t in_place;           /* read `output` instead of `input` (FP ops) */
    const void* input;           /* [batch, count] T */
    void* output;                /* [batch, count] T (FP ops) */
    const void* bias;            /* [count] in bias_data_type, FP ops, or NULL */
    uint32_t bias_data_type;
    int8_t* q_out;               /* [batch, count] codes (quantizing ops) */
    float* scales_out;           /* [batch, count / scale_group_size] */
    int32_t* group_sums_out;     /* [batch, count / sum_group_size] */
    const int32_t* rht_factors;  /* [count] signs */
    uint32_t batch_size, element_count;
    uint32_t scale_group_size;   /* 32, 64 or 128 (quantizing ops) */
    uint32_t sum_group_size;     /* 32, 64 or 128, <= scale_group_size (with group sums) */
    uint32_t grouped_by_nibble;  /* code order for 4-bit weights (Int8CodeLayout) */
} stark_qmm_activation_transform_args;

/* Replaces ActivationTransform::encode_* (src/backends/common/kernel/activation_transform.rs;
 * CPU twin src/backends/cpu/kernel/activation_transform/activation_transform.rs:48-156):
 * input RHT, output RHT (+ bias), or input RHT then symmetric int8
 * quantization per scale group (optionally with int32 sums per weight group),
 * the activations of the int8 (A8W4 / A8W8) products. */
STARK_QMM_API stark_qmm_status stark_qmm_activation_transform(const stark_qmm_activation_transform_args* args,
                                                             void* stream);

/* ActivationType (src/backends/common/gpu_types/activation_type.rs:8-16) */
enum { STARK_QMM_ACT_SILU = 0, STARK_QMM_ACT_GELU_APPROX = 1, STARK_QMM_ACT_GELU_EXACT = 2,
       STARK_QMM_ACT_IDENTITY = 3, STARK_QMM_ACT_SOFTPLUS = 4, STARK_QMM_ACT_SILU_MATERIALIZED_SIGMOID = 5,
       STARK_QMM_ACT_GELU_MATERIALIZED_POLYNOMIAL = 6 };
/* GatedActMulOp (src/backends/common/gpu_types/gated_act_mul.rs:3-7) */
enum { STARK_QMM_GATED_FULL_PRECISION = 0, STARK_QMM_GATED_QUANTIZE = 1, STARK_QMM_GATED_QUANTIZE_WITH_GROUP_SUMS = 2 };

typedef struct stark_qmm_gated_act_mul_args {
    uint32_t struct_size;
    uint32_t op;                 /* STARK_QMM_GATED_* (quantizing ops need hadamard_factors) */
    uint32_t data_type;          /* T: F32 or BF16 */
    uint32_t act_type;           /* STARK_QMM_ACT_* */
    uint32_t interleaved;        /* act_operand rows [value(gated_dim) | gate(gated_dim)] */
    const void* act_operand;     /* interleaved rows, or gates [batch, gated_dim] */
    const void* value_operand;   /* separate values: row b at b * value_row_stride + value_offset */
    void* fp_out;                /* [batch, gated_dim] T */
    int8_t* q_out;
    float* scales_out;
    int32_t* group_sums_out;
    const int32_t* hadamard_factors; /* [gated_dim] signs, or NULL */
    uint32_t gated_dim, batch_dim, value_offset, value_row_stride;
    uint32_t has_activation_alpha;   /* SiLU with alpha */
    float activation_alpha;
    uint32_t clip_gate;
    float gate_clip_min, gate_clip_max;
    uint32_t clip_value;
    float value_clip_min, value_clip_max;
    uint32_t scale_group_size, sum_group_size, grouped_by_nibble;
} stark_qmm_gated_act_mul_args;

/* Replaces GatedActMul::encode_* (src/backends/common/kernel/gated_act_mul.rs;
 * CPU twin src/backends/cpu/kernel/gated_act_mul/gated_act_mul.rs:17-152):
 * value * activation(gate) in T, with optional clipping, SiLU alpha, RHT and
 * int8 quantization. */
STARK_QMM_API stark_qmm_status stark_qmm_gated_act_mul(const stark_qmm_gated_act_mul_args* args, void* stream);

/* ------------------------------------------------------------------ */
/* Weight files: Stark's converted artifact (model.safetensors) and      */
/* GGUF v3 checkpoints                                                    */
/* ------------------------------------------------------------------ */

/* Detail text of the last failing weight-file call on this thread (never NULL). */
STARK_QMM_API const char* stark_qmm_last_error(void);

typedef struct stark_qmm_file stark_qmm_file;
enum { STARK_QMM_FILE_SAFETENSORS = 0, STARK_QMM_FILE_GGUF = 1 };

typedef struct stark_qmm_tensor_info {
    uint32_t dtype;      /* safetensors: STARK_QMM_F32 .. STARK_QMM_U64; GGUF: the GGML kind (8 = Q8_0, 12 = Q4_K, ...) */
    uint32_t rank;
    uint64_t shape[8];   /* outermost first (GGUF dimensions reversed, as weights.rs:2823 does) */
    uint64_t offset;     /* byte offset of the payload in its file */
    uint64_t size;       /* payload bytes */
    const void* host;    /* read-only mapping of the payload, valid until stark_qmm_file_close */
} stark_qmm_tensor_info;

/* Opens a weight file. A `.safetensors` file is indexed as ParameterLoader::new
 * does (src/parameters/loader.rs:80-127; header read_metadata,
 * src/parameters/safetensors_metadata.rs:113-128). A `.gguf` file, or a
 * directory of `.gguf` split files, is read as the hybrid engine's
 * Weights::open / read_gguf (src/engine/hybrid/weights.rs:815-895, 2770-2865):
 * version 3, alignment, block sizes, overlap and split completeness checked.
 * Files are mapped read-only; nothing is copied until an upload. */
STARK_QMM_API stark_qmm_status stark_qmm_file_open(const char* path, stark_qmm_file** out);
STARK_QMM_API void stark_qmm_file_close(stark_qmm_file* file);
STARK_QMM_API uint32_t stark_qmm_file_kind(const stark_qmm_file* file);
STARK_QMM_API uint64_t stark_qmm_file_tensor_count(const stark_qmm_file* file);
/* Tensor names in sorted order; NULL past the end. */
STARK_QMM_API const char* stark_qmm_file_tensor_name(const stark_qmm_file* file, uint64_t index);
STARK_QMM_API stark_qmm_status stark_qmm_file_tensor(const stark_qmm_file* file, const char* name,
                                                     stark_qmm_tensor_info* info);
/* Metadata value as text (safetensors __metadata__ strings; GGUF values, arrays as [a,b,...]). */
STARK_QMM_API stark_qmm_status stark_qmm_file_metadata(const stark_qmm_file* file, const char* key, const char** value);
/* Copies one tensor's payload to new device memory (hipMalloc; free with
 * stark_qmm_device_free): GGUF block matrices then feed stark_qmm_mapped_many. */
STARK_QMM_API stark_qmm_status stark_qmm_file_upload(const stark_qmm_file* file, const char* name, void** device,
                                                     void* stream);
STARK_QMM_API stark_qmm_status stark_qmm_device_free(void* device);

/* AnyWeightMatrixSpec (src/config/weight_matrix/): FullPrecisionSpec, MLXSpec
 * (mlx_spec.rs:5-13) and IntSpec; Layout OutputInput / InputOutput. */
enum { STARK_QMM_SPEC_FULL_PRECISION = 0, STARK_QMM_SPEC_MLX = 1, STARK_QMM_SPEC_INT = 2 };
enum { STARK_QMM_WEIGHT_OUTPUT_INPUT = 0, STARK_QMM_WEIGHT_INPUT_OUTPUT = 1 };
typedef struct stark_qmm_weight_spec {
    uint32_t struct_size;   /* sizeof(stark_qmm_weight_spec) */
    uint32_t kind;          /* STARK_QMM_SPEC_* */
    uint32_t bits, group_size;
    uint32_t layout;        /* STARK_QMM_WEIGHT_* */
    uint32_t is_symmetric;  /* IntSpec */
    uint32_t materialize_affine_input_sum;  /* MLXSpec */
    /* QuantParams::with_source_output_widths (src/backends/common/kernel/matmul/mod.rs:78-92):
     * consecutive row spans of a fused matrix (q/k/v, gate/up); count 0 = one source */
    uint32_t source_output_widths[4];
    uint32_t source_output_count;
} stark_qmm_weight_spec;

typedef struct stark_qmm_weight_matrix {
    uint32_t struct_size;   /* sizeof(stark_qmm_weight_matrix), set by the caller */
    stark_qmm_b b;          /* ready for stark_qmm_args.b (device pointers owned by this struct) */
    uint32_t rows, columns; /* physical shape */
    uint32_t source_output_widths[4];
    uint32_t source_output_count;
    void* device[3];        /* weights, scales, biases / zero points */
} stark_qmm_weight_matrix;

/* Replaces WeightMatrix::load (src/encodable_block/weight_matrix.rs:114-216)
 * on the artifact's `<prefix>.weights`, `.scales`, `.biases` / `.zero_points`:
 * the same spec checks (parse_spec, :53-96), shapes, dtypes and byte sizes
 * (ParameterLeaf::validate, src/parameters/loader.rs:272-305), then copies
 * the tensors to the device (load time: allocates, and waits for the copy).
 * Output-input matrices get group-output planes [G, roundup4(N)], input-output
 * matrices output-group planes [N, G]. */
STARK_QMM_API stark_qmm_status stark_qmm_weight_matrix_load(const stark_qmm_file* file, const char* prefix,
                                                            const stark_qmm_weight_spec* spec, uint32_t required_layout,
                                                            uint32_t output_dim, uint32_t input_dim, uint32_t data_type,
                                                            stark_qmm_weight_matrix* out, void* stream);
STARK_QMM_API void stark_qmm_weight_matrix_free(stark_qmm_weight_matrix* matrix);

#ifdef __cplusplus
}
#endif
#endif
