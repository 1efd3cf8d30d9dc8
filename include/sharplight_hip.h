/*
 * libsharplight_hip -- C ABI of the Sharplight HIP execution provider (MI355X / gfx950).
 *
 * The managed provider (Sharplight.Hip) binds these entry points with [LibraryImport], the way
 * Sharplight.Metal binds its system frameworks (src/Sharplight.Metal/Interop/MetalFramework.cs:14-18);
 * the Python package sharplight_amd binds the same symbols with ctypes.
 *
 * Conventions
 *  - Every function returns an int status: SLHIP_OK (0) or a negative slhip_status. The message of the
 *    last failure on the calling thread is slhip_last_error(). The managed side turns statuses into
 *    the exceptions the reference's providers throw: SLHIP_ERR_INVALID -> ArgumentException,
 *    SLHIP_ERR_UNSUPPORTED -> NotSupportedException, SLHIP_ERR_INDEX -> ArgumentOutOfRangeException,
 *    SLHIP_ERR_CACHE -> InvalidOperationException, SLHIP_ERR_FORMAT -> InvalidDataException.
 *  - Tensor pointers are device pointers (slhip_malloc). Sizes and strides are in ELEMENTS of the
 *    tensor's own dtype, rows are the leading dims flattened, the normalized/activated axis is last and
 *    dense.
 *  - Op entry points only enqueue work on the given stream (NULL = the device's null stream) and return;
 *    nothing is synchronous except slhip_stream_sync / slhip_event_synchronize / slhip_memcpy_*_sync.
 *  - Ops read inputs and write outputs only; outputs may alias an input of the same shape and layout
 *    (in-place) unless stated otherwise.
 *  - No op entry point allocates device memory. Errors found by a kernel (a gather id outside the
 *    table, a KV-cache row outside the cache) go to a per-device error word, a device variable of the
 *    library, and are reported by the next slhip_stream_sync.
 */
#ifndef SHARPLIGHT_HIP_H
#define SHARPLIGHT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(_WIN32)
#define SLHIP_API __declspec(dllexport)
#else
#define SLHIP_API __attribute__((visibility("default")))
#endif

#define SLHIP_ABI_VERSION 5

typedef enum slhip_status {
    SLHIP_OK = 0,
    SLHIP_ERR_INVALID = -1,     /* bad argument: null pointer, size, stride, dtype combination */
    SLHIP_ERR_UNSUPPORTED = -2, /* valid request this library has no kernel for */
    SLHIP_ERR_HIP = -3,         /* the HIP runtime reported an error */
    SLHIP_ERR_INDEX = -4,       /* a gather index was outside [0, V) (reported by slhip_stream_sync) */
    SLHIP_ERR_NO_DEVICE = -5,   /* no usable device / driver */
    SLHIP_ERR_CACHE = -6,       /* a KV-cache row outside the cache or block table (at slhip_stream_sync) */
    SLHIP_ERR_FORMAT = -7       /* malformed file data: a truncated or inconsistent GGUF file */
} slhip_status;

/* Element types of activations. */
typedef enum slhip_dtype { SLHIP_F32 = 0, SLHIP_F16 = 1, SLHIP_BF16 = 2 } slhip_dtype;

/* Row formats of a gathered table (Sharplight.Tensors.WeightFormat for these formats; the block
 * layouts are ggml's, src/Sharplight.Cpu/Quant.cs:181-216). */
typedef enum slhip_format {
    SLHIP_FMT_F32 = 0,
    SLHIP_FMT_F16 = 1,
    SLHIP_FMT_BF16 = 2,
    SLHIP_FMT_Q8_0 = 3, /* 34-byte blocks: f16 d, int8 q[32]           -> q*d        */
    SLHIP_FMT_Q4_0 = 4, /* 18-byte blocks: f16 d, u8 qs[16] (nibbles)   -> (q-8)*d    */
    SLHIP_FMT_Q4_1 = 5, /* 20-byte blocks: f16 d, f16 m, u8 qs[16]      -> q*d + m    */
    SLHIP_FMT_Q5_0 = 6, /* 22-byte blocks: f16 d, u32 qh, u8 qs[16]     -> (q-16)*d   */
    SLHIP_FMT_Q5_1 = 7, /* 24-byte blocks: f16 d, f16 m, u32 qh, qs[16] -> q*d + m    */
    /* 256-value super-blocks (ggml's K-quants; src/Sharplight.Cpu/Quant.cs:500-624, Quant.KQuants.cs:36-107) */
    SLHIP_FMT_Q2_K = 8,   /* 84 bytes: scales[16], qs[64], f16 d, f16 dmin   -> q*(d*sc) - dmin*m   */
    SLHIP_FMT_Q3_K = 9,   /* 110 bytes: hmask[32], qs[64], scales[12], f16 d -> (q-4h)*(d*(sc-32))  */
    SLHIP_FMT_Q4_K = 10,  /* 144 bytes: f16 d, f16 dmin, scales[12], qs[128] -> fma(q, d*sc, -dmin*m) */
    SLHIP_FMT_Q5_K = 11,  /* 176 bytes: as Q4_K with qh[32] before qs         */
    SLHIP_FMT_Q6_K = 12,  /* 210 bytes: ql[128], qh[64], int8 scales[16], f16 d -> fma(q, s, -32 s)   */
    /* the 4-bit codebook formats (Quant.cs:407-446): value = scale * codebook[nibble] */
    SLHIP_FMT_IQ4_NL = 13, /* 18-byte blocks of 32: f16 d, qs[16]          */
    SLHIP_FMT_IQ4_XS = 14, /* 136 bytes per 256: f16 d, u16 scales_h, scales_l[4], qs[128] */
    /* ternary and 4-bit float formats (Quant.Ternary.cs:27-86, Quant.Fp4.cs:36-80): value = code * scale */
    SLHIP_FMT_TQ1_0 = 15, /* 54 bytes per 256: qs[48] (5 base-3 digits per byte), qh[4], f16 d -> (t-1)*d */
    SLHIP_FMT_TQ2_0 = 16, /* 66 bytes per 256: qs[64] (4 two-bit codes per byte), f16 d -> (q-1)*d         */
    SLHIP_FMT_MXFP4 = 17, /* 17 bytes per 32: E8M0 e, qs[16] (E2M1 nibbles) -> fp4 * 2^(e-128)            */
    SLHIP_FMT_NVFP4 = 18, /* 36 bytes per 64: UE4M3 d[4] (per 16), qs[32] (E2M1 nibbles) -> fp4 * d/2      */
    /* ggml's grid IQ formats (Quant.Iq.cs:113-306), 256 values per block: groups of 8 values index a
     * lattice table, with sign patterns and small scales */
    SLHIP_FMT_IQ2_XXS = 19, /* 66 bytes  */
    SLHIP_FMT_IQ2_XS = 20,  /* 74 bytes  */
    SLHIP_FMT_IQ2_S = 21,   /* 82 bytes  */
    SLHIP_FMT_IQ3_XXS = 22, /* 98 bytes  */
    SLHIP_FMT_IQ3_S = 23,   /* 110 bytes */
    SLHIP_FMT_IQ1_S = 24,   /* 50 bytes  */
    SLHIP_FMT_IQ1_M = 25,   /* 56 bytes  */
    /* The reference's own formats (src/Sharplight.Core/Tensors/DataType.cs:154-244; decoders Quant.cs:656-718,
     * Quant.Grouped.cs, Quant.Absmax.cs, Quant.Fp4.cs:86-107, Quant.Fp8.cs): */
    SLHIP_FMT_Q1_0 = 26,       /* 128 values, 18 bytes: f16 d, u8 bits[16]; bit i of byte j -> value 8j+i = +-d */
    SLHIP_FMT_Q2_0 = 27,       /* 64 values, 18 bytes: f16 d, u8 qs[16]; 2-bit code i of byte j -> (c-1)*d      */
    SLHIP_FMT_Q2_0_G128 = 28,  /* 128 values, 34 bytes: the Q2_0 code with one scale per 128                 */
    SLHIP_FMT_TERN1_G128 = 29, /* 128 values, 28 bytes: base-3 digits in bytes 0..25, f16 d at 26 -> t*d      */
    SLHIP_FMT_NVFP4_GS = 30,   /* 64 values, 40 bytes: f32 g, UE4M3 d[4], qs[32] -> fp4 * (d*g)              */
    SLHIP_FMT_Q4Z_G32 = 31,    /* 32 values, 20 bytes: f16 d, f16 z, nibbles -> (q - z)*d                   */
    SLHIP_FMT_Q4Z_G128 = 32,   /* 128 values, 68 bytes: the same, four 32-value runs                        */
    SLHIP_FMT_Q8Z_G32 = 33,    /* 32 values, 36 bytes: f16 d, f16 z, u8 q[32] -> (q - z)*d                  */
    SLHIP_FMT_Q8Z_G128 = 34,   /* 128 values, 132 bytes                                                     */
    SLHIP_FMT_NF4_B64 = 35,    /* 64 values, 36 bytes: f32 d, nibbles -> NF4[q]*d                           */
    SLHIP_FMT_FP4_B64 = 36,    /* 64 values, 36 bytes: f32 d, nibbles -> FP4[q]*d                           */
    SLHIP_FMT_Q8A_G32 = 37,    /* 32 values, 36 bytes: f32 d, i8 q[32] -> q*d*(1/127)                       */
    SLHIP_FMT_Q2S_G128 = 38,   /* 128 values, 36 bytes: f32 d, u8 qs[32]; byte j: values j, 32+j, 64+j, 96+j */
    SLHIP_FMT_F8E4M3 = 39,     /* OCP E4M3FN bytes                                                          */
    SLHIP_FMT_F8E5M2 = 40,     /* E5M2 bytes (the top byte of an IEEE half)                                 */
    SLHIP_FMT_F8E4M3_B32 = 41, /* 32 values, 36 bytes: f32 d, E4M3 q[32] -> e4m3(q)*d                       */
    SLHIP_FMT_F8E4M3_B128 = 42, /* 128 values, 132 bytes                                                    */
    /* Trellis-coded, 128 values: f16 d, then the path bytes of N steps of V values and K new bits each; step t's
     * 16-bit state hashes to codebook points, value = d * point (src/Sharplight.Core/Tensors/TrellisBlocks.cs) */
    SLHIP_FMT_TRELLIS_V4K8_G128 = 43, /* 34 bytes: V = 4, K = 8 (states from byte pairs)                     */
    SLHIP_FMT_TRELLIS_V4K6_G128 = 44, /* 26 bytes: V = 4, K = 6 (states from a circular bit stream)          */
    SLHIP_FMT_TRELLIS_V4K7_G128 = 45, /* 30 bytes: V = 4, K = 7                                              */
    SLHIP_FMT_TRELLIS_V2K5_G128 = 46, /* 42 bytes: V = 2, K = 5                                              */
    SLHIP_FMT_TRELLIS_V2K6_G128 = 47, /* 50 bytes: V = 2, K = 6                                              */
    SLHIP_FMT_TRELLIS_V2K7_G128 = 48  /* 58 bytes: V = 2, K = 7                                              */
} slhip_format;

/* Row-norm kinds (StandardOps RmsNorm / L2Norm / LayerNorm). */
typedef enum slhip_norm { SLHIP_NORM_RMS = 0, SLHIP_NORM_L2 = 1, SLHIP_NORM_LAYER = 2 } slhip_norm;

/* Gate activations of the gated MLP (MlpActivations.cs:38-40). */
typedef enum slhip_act { SLHIP_ACT_SILU = 0, SLHIP_ACT_GELU_TANH = 1, SLHIP_ACT_GELU_ERF = 2 } slhip_act;

typedef void* slhip_stream; /* a hipStream_t */
typedef void* slhip_event;  /* a hipEvent_t  */

typedef struct slhip_device_props {
    char name[256];        /* marketing name, e.g. "AMD Instinct MI355X" */
    char arch[64];         /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    int64_t total_memory;  /* bytes of device memory */
    int32_t compute_units;
    int32_t wavefront_size;
    int32_t pci_domain, pci_bus, pci_device;
    int32_t clock_khz;
    int64_t l2_bytes;
    int32_t max_threads_per_block;
    int32_t lds_bytes_per_block;
} slhip_device_props;

/* ---- library / errors ------------------------------------------------------------------------- */

/* Message of the last failed call on this thread ("" if none). Never NULL. */
SLHIP_API const char* slhip_last_error(void);
SLHIP_API int slhip_abi_version(void);

/* ---- devices (IExecutionProvider.CheckAvailability / GetDevices, IExecutionProvider.cs:25-40;
 *      DeviceInfo fields, src/Sharplight.Core/Runtime/DeviceInfo.cs:4-50) ------------------------ */

/* Number of visible devices; 0 with SLHIP_OK when the driver loads but reports none, SLHIP_ERR_NO_DEVICE
 * when the runtime cannot start. */
SLHIP_API int slhip_device_count(int* count);
SLHIP_API int slhip_device_props_get(int device, slhip_device_props* props);
/* Makes `device` current for the calling thread (IExecutionProvider.OpenDevice). */
SLHIP_API int slhip_set_device(int device);
SLHIP_API int slhip_get_device(int* device);
/* Free / total bytes of the current device (IComputeDevice.AvailableMemory / GetMemoryInfo). */
SLHIP_API int slhip_mem_info(size_t* free_bytes, size_t* total_bytes);

/* ---- memory (weights, state and activations a compiled segment owns, IComputeDevice.Compile) --- */

SLHIP_API int slhip_malloc(void** ptr, size_t bytes);
SLHIP_API int slhip_free(void* ptr);
SLHIP_API int slhip_host_malloc(void** ptr, size_t bytes); /* pinned host staging buffer */
SLHIP_API int slhip_host_free(void* ptr);
/* Asynchronous copies on `stream` (ICompiledSegment.SetInput / GetOutput stage through these). */
SLHIP_API int slhip_memcpy_h2d(void* dst, const void* src, size_t bytes, slhip_stream stream);
SLHIP_API int slhip_memcpy_d2h(void* dst, const void* src, size_t bytes, slhip_stream stream);
SLHIP_API int slhip_memcpy_d2d(void* dst, const void* src, size_t bytes, slhip_stream stream);
SLHIP_API int slhip_memset(void* dst, int value, size_t bytes, slhip_stream stream);

/* ---- streams and events ---------------------------------------------------------------------- */

SLHIP_API int slhip_stream_create(slhip_stream* stream); /* default priority */
SLHIP_API int slhip_stream_destroy(slhip_stream stream);
/* Waits for the stream, then reports (and clears) a pending gather index error on the current device
 * as SLHIP_ERR_INDEX, like GatherOp's ArgumentOutOfRangeException (src/Sharplight.Cpu/GatherOp.cs:60-63). */
SLHIP_API int slhip_stream_sync(slhip_stream stream);
SLHIP_API int slhip_event_create(slhip_event* event);
SLHIP_API int slhip_event_destroy(slhip_event event);
SLHIP_API int slhip_event_record(slhip_event event, slhip_stream stream);
SLHIP_API int slhip_event_synchronize(slhip_event event);
SLHIP_API int slhip_event_elapsed_ms(float* ms, slhip_event start, slhip_event stop);

/* ---- graphs: record a sequence of launches once, replay it without host work per launch ------------
 * The HIP counterpart of the Vulkan segment's command buffer recorded once per symbol binding and
 * resubmitted every step (src/Sharplight.Vulkan/VulkanSegment.cs:440-457). Capture every op call made on
 * `stream` between begin and end (the op entry points enqueue only kernels: no memset or copy is
 * recorded); replay with slhip_graph_launch on any stream. */
typedef void* slhip_graph; /* an instantiated hipGraphExec_t */
SLHIP_API int slhip_graph_begin(slhip_stream stream);
SLHIP_API int slhip_graph_end(slhip_stream stream, slhip_graph* graph);
SLHIP_API int slhip_graph_launch(slhip_graph graph, slhip_stream stream);
SLHIP_API int slhip_graph_destroy(slhip_graph graph);

/* ---- fused layer ops ------------------------------------------------------------------------- */

/*
 * Row normalization over the last axis, with an optional residual add fused in front.
 *   h = res ? x + res : x                            (f32)
 *   RMS:   y = h * (1/sqrt(sum(h^2)/D + eps)) * w
 *   L2:    y = h * (1/sqrt(sum(h^2) + eps))          (w must be NULL)
 *   LAYER: y = ((h - mean) * (1/sqrt(var + eps))) * w + b
 * w, b: f32 [D] or NULL. x, res, h_out have dtype_in; y has dtype_out. h_out (the updated residual
 * stream) is written only when res is given and h_out is not NULL; the norm reads the unrounded f32 sum.
 * Replaces: RowOp RmsNorm/L2Norm/LayerNorm (src/Sharplight.Cpu/RowOp.cs:63-113) and the Vulkan lowerer's
 * norm kernels, including the Add+RmsNorm unit of FoldNormTails
 * (src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:215-238, GraphLowerer.Elementwise.cs:110-117,
 * GraphLowerer.Transformer.cs:9-34, Kernels/norm.slang:20-47, Kernels/rows.slang:41-138).
 * dtype_in/dtype_out: F32 or BF16 (any combination).
 */
SLHIP_API int slhip_rownorm(int kind, int dtype_in, int dtype_out, const void* x, const void* res, const float* w,
                            const float* b, void* y, void* h_out, int64_t rows, int64_t D, int64_t x_stride,
                            int64_t res_stride, int64_t y_stride, int64_t h_stride, float eps, slhip_stream stream);

/*
 * The GEMM activation copies a row norm can write beside (or instead of) y, from the same f32 values
 * (the "nrm" of the reference's two-pass row norm kernel):
 *   y16: f16 rows (round to nearest even; NaN keeps its payload top bits), row stride y16_stride elements;
 *   yq:  E4M3 activation rows of the fp8 GEMM: per row D codes, then D/128 f32 scales; for each 128-value
 *        group d = amax/448 and code = e4m3(v * (d > 0 ? 1/d : 0)) (quantize_fp8). Row stride yq_stride
 *        bytes >= D + D/32 (the reference's dense rows are exactly that), D a multiple of 128,
 *        4-byte aligned.
 * Either may be NULL.
 * Replaces: the f16 copy outputs and Fp8Output of RowNormKernelSource
 * (src/Sharplight.Shaders/Lowering/RowNormKernelSource.cs:45-57,108-124,282-291; GraphLowerer.HalfCopies.cs:
 * 36-40,106-151; GraphLowerer.Elementwise.cs:150-200), quantize_fp8 (Kernels/gemm_fp8.slang:36-55) and
 * e4m3_code / e4m3_pack4 (Kernels/e4m3.slang:5-38).
 */
typedef struct slhip_norm_copies {
    void* y16;
    int64_t y16_stride;
    void* yq;
    int64_t yq_stride;
} slhip_norm_copies;

/*
 * slhip_rownorm that also writes the copies in `copies` (NULL: none). y may be NULL when a copy is given:
 * the reference's norm skips its f32 rows from prefill sizes when every reader takes the copy
 * (GraphLowerer.Elementwise.cs:184-200).
 */
SLHIP_API int slhip_rownorm_copies(int kind, int dtype_in, int dtype_out, const void* x, const void* res,
                                   const float* w, const float* b, void* y, void* h_out, int64_t rows, int64_t D,
                                   int64_t x_stride, int64_t res_stride, int64_t y_stride, int64_t h_stride,
                                   float eps, const slhip_norm_copies* copies, slhip_stream stream);

/*
 * Decode matvec y = x . W^T and the dual gate/up matvec y = act(x . Wg^T) * (x . Wu^T) for few activation
 * rows (the decode FFN's gate/up projections with the gating epilogue).
 *   x: [T, K] f32 or bf16 (dtype_x), 16-byte aligned, row stride x_stride elements (a multiple of 8);
 *   W, Wg, Wu: N rows of K weights in `fmt`, 16-byte aligned: dense F32/F16/BF16 (K a multiple of 8,
 *   K <= 16384), or the GGUF block formats Q8_0/Q4_0/Q4_1/Q5_0/Q5_1 and Q4_K/Q5_K/Q6_K (K a multiple of
 *   256 and the rows' block images fitting in LDS), or Q2_K / Q3_K (K a multiple of 256); y: [T, N] f32 or bf16
 *   (dtype_y), row stride y_stride.
 *   act: SLHIP_ACT_SILU / GELU_TANH / GELU_ERF, the same forms as slhip_gated_act.
 * Products and sums in f32 (in another order than the CPU provider's, so equal to it within the rounding of
 * a K-term f32 dot product); block formats sum d * sum(x q) + a * sum(x) per block, as the reference's
 * fused Q4_0 dot does (the K-quants per 32-value sub-block: d0 * sum(x q) - m * sum(x); Q6_K
 * s * sum(x (q - 32)) per 16 values). BF16 weights with T >= SLHIP_MATVEC_MFMA_MIN_T (environment, default 3; 0 keeps the
 * VALU kernel) and K a multiple of 64 go to the matrix cores with f32 x split exactly into three bf16 parts:
 * the same products, summed in another order, under the same bound. Q4_K and Q6_K at T = 1 (K a multiple of
 * 4096 for Q4_K, 2048 for Q6_K) go to the integer matrix cores: x represented to 2^(e-28) of its 32-value
 * block's largest power of two, the code sums exact, under the same bound. Q8_0/Q4_0/Q4_1/Q5_0/Q5_1 from
 * SLHIP_MATVEC_MQ_MIN_T tokens (default 3), Q2_K..Q6_K from SLHIP_MATVEC_KQ_MIN_T (default 5), with K a
 * multiple of 1024 (Q6_K: 512), go to the matrix cores as exact bf16 codes (Q4_0 q - 8, Q6_K q - 32) against
 * x in two bf16 parts (|x - h - m| <= 2^-18 |x|), 16 tokens per launch, block scales (and the K-quants'
 * minima, scales per 16 values) applied per block in f32: the same bound.
 * Replaces: MatMulOp's float-row path (src/Sharplight.Cpu/MatMulOp.cs:376-465; fused Q8_0/Q4_0 dots, Quant.cs:738-803)
 * followed by the activation and
 * Mul, i.e. the reference's dual matvec unit (FoldDualMatMuls, src/Sharplight.Shaders/Lowering/
 * GraphLowerer.Fusion.cs:286-353; tests/Sharplight.Vulkan.Tests/FusionTests.cs:59-80).
 */
SLHIP_API int slhip_matvec(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T, int64_t K,
                           const void* w, int64_t N, void* y, int64_t y_stride, slhip_stream stream);
SLHIP_API int slhip_dual_matvec(int act, int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T,
                                int64_t K, const void* w_gate, const void* w_up, int64_t N, void* y, int64_t y_stride,
                                slhip_stream stream);
/* slhip_matvec followed by y += bias (bias [N] f32, NULL for none) in the same launch: the reference's matmul
 * whose only reader adds a constant row vector (FoldMatMulBiases, src/Sharplight.Shaders/Lowering/
 * GraphLowerer.Fusion.cs:355-408; LowerMatMulBias, GraphLowerer.MatMul.cs:205-245: the same f32 sum as the Add). */
SLHIP_API int slhip_matvec_bias(int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride, int64_t T,
                                int64_t K, const void* w, int64_t N, const float* bias, void* y, int64_t y_stride,
                                slhip_stream stream);

/*
 * Integer-dot decode matvec: the reference's few-row MatMul on quantized weights when activations may be
 * quantized (src/Sharplight.Cpu/MatMulOp.cs:144-146,173-213 with IntDot.cs; the Vulkan lowerer's int-dot matvec,
 * src/Sharplight.Shaders/Lowering/GraphLowerer.IntDot.cs:52-117 and Kernels/mmvq.slang). Two steps, so that
 * several matmuls reading the same x share one quantized copy (GraphLowerer.IntDot.cs:119-220):
 *
 * slhip_quantize_q8: x [T, K] f32 or bf16 (row stride x_stride elements, a multiple of 4; x and xq 16-byte
 *   aligned; K a multiple of 32) -> xq, T rows of slhip_q8_row_bytes(K) = 1.5 K bytes each:
 *     int8 q[K], then per 32-value block f32 {d, d * sum(q[0..15]), d * sum(q[16..31]), 0},
 *   with d = amax / 127 and q = (int)(x / d rounded half away from zero through an f32 addition), bit for bit
 *   IntDot.QuantizeBlockScalar (IntDot.cs:92-126; NaN in a block: d NaN, codes 0).
 * slhip_matvec_q8 / slhip_dual_matvec_q8: y [T, N] (f32 or bf16, row stride y_stride) = xq . W^T (+ bias[N] f32,
 *   single form, may be NULL), or act(xq . Wg^T) * (xq . Wu^T). Weights: Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, IQ4_NL,
 *   MXFP4 (K a multiple of 32, rows of an even number of bytes), Q4_K, Q5_K, Q6_K, IQ4_XS (K a multiple of 256)
 *   (IntDot.Supports, IntDot.cs:36-38), 16-byte aligned. Per 16 values the
 *   integer sum s of codes times q is exact; y sums a * d * s + b * gs (w = a * code + b, IntDot.Decode) in f32, in
 *   another order than IntDot.DotScalar, so within f32 accumulation of those terms of the CPU provider's result.
 */
SLHIP_API int64_t slhip_q8_row_bytes(int64_t K);
SLHIP_API int slhip_quantize_q8(int dtype_x, const void* x, int64_t x_stride, int64_t T, int64_t K, void* xq,
                                slhip_stream stream);
SLHIP_API int slhip_matvec_q8(int fmt, int dtype_y, const void* xq, int64_t T, int64_t K, const void* w, int64_t N,
                              void* y, int64_t y_stride, const float* bias, slhip_stream stream);
SLHIP_API int slhip_dual_matvec_q8(int act, int fmt, int dtype_y, const void* xq, int64_t T, int64_t K,
                                   const void* w_gate, const void* w_up, int64_t N, void* y, int64_t y_stride,
                                   slhip_stream stream);
/* The decode FFN's gate/up pair in one call: slhip_quantize_q8 of x into `work` (work_bytes >= T *
 * slhip_q8_row_bytes(K), 16-byte aligned), then slhip_dual_matvec_q8 -- the lowerer's "x->q8" and int-dot
 * launches (GraphLowerer.IntDot.cs:82-117,226-249). SLHIP_ERR_INVALID when the workspace is too small. */
SLHIP_API int slhip_dual_matvec_int8(int act, int fmt, int dtype_x, int dtype_y, const void* x, int64_t x_stride,
                                     int64_t T, int64_t K, const void* w_gate, const void* w_up, int64_t N, void* y,
                                     int64_t y_stride, void* work, int64_t work_bytes, slhip_stream stream);
/* slhip_dual_matvec_int8 without a workspace argument and without allocating: no counterpart in the reference;
 * for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops). The
 * quantized rows go to a static 1 MiB array per device (T * 1.5 K <= 1048576 bytes, else SLHIP_ERR_UNSUPPORTED),
 * which every call on that device shares: calls that overlap on one GPU (several streams, several host threads)
 * race on it. The same kernels and results as slhip_dual_matvec_int8. */
SLHIP_API int slhip_dual_matvec_int8_noalloc(int act, int fmt, int dtype_x, int dtype_y, const void* x,
                                             int64_t x_stride, int64_t T, int64_t K, const void* w_gate,
                                             const void* w_up, int64_t N, void* y, int64_t y_stride,
                                             slhip_stream stream);

/*
 * Gated activation out = act(gate) * up over [rows, cols] (IMlpActivation.ActivateGated,
 * src/Sharplight.Core/Architectures/IMlpActivation.cs:12; CPU: UnaryOp then BinaryOp Mul,
 * src/Sharplight.Cpu/ScalarMath.cs:552-641, BinaryOp.cs:8-103; Vulkan: the fused[Silu,Mul]
 * elementwise unit, GraphLowerer.Fusion.cs:89-142).
 *   SILU:      g / (1 + exp(-g))
 *   GELU_TANH: g / (1 + exp(-u)), u = 2*0.7978845608*(g + 0.044715*g^3)
 *   GELU_ERF:  0.5*g*(1 + erf(g/sqrt(2)))
 * Row strides let gate and up be the two halves of one merged [rows, 2*cols] projection.
 * dtype_in/dtype_out: F32 or BF16.
 */
SLHIP_API int slhip_gated_act(int act, int dtype_in, int dtype_out, const void* gate, const void* up, void* out,
                              int64_t rows, int64_t cols, int64_t gate_stride, int64_t up_stride, int64_t out_stride,
                              slhip_stream stream);

/* Destination rows of KV-cache writes (CacheWrite, src/Sharplight.Core/Graph/StandardOps.cs:310-319):
 * token t of a launch goes to cache row
 *   SLHIP_ROWS_PAST   n_past + t
 *   SLHIP_ROWS_SEQ    slot * (ctx / slots) + position, from sequence rows seq[t] = (slot, position, ., .)
 *   SLHIP_ROWS_PAGED  pages[slot, position / block_size] * block_size + position % block_size
 * as src/Sharplight.Cpu/CacheWriteOp.cs:103-155 and KvPages.cs:28-49 map them. PAST overflow
 * (n_past + T > ctx) is refused at the call; a SEQ/PAGED row outside the cache or block table is skipped
 * and reported as SLHIP_ERR_CACHE by the next slhip_stream_sync (the other rows are written). */
typedef enum slhip_rows_mode { SLHIP_ROWS_PAST = 0, SLHIP_ROWS_SEQ = 1, SLHIP_ROWS_PAGED = 2 } slhip_rows_mode;

typedef struct slhip_cache_rows {
    int32_t mode;
    int32_t reserved;
    int64_t ctx;              /* rows of the cache */
    int64_t n_past;           /* PAST */
    const int32_t* seq;       /* SEQ, PAGED: [T, 4] int32 */
    int64_t slots;            /* SEQ: sequences sharing the cache in equal parts */
    const int32_t* pages;     /* PAGED: block table [page_slots, blocks_per_slot] int32 */
    int64_t page_slots, blocks_per_slot, block_size;
} slhip_cache_rows;

/* One tensor of a rope launch: x and y are [T, heads, D] with the given token/head strides
 * (innermost stride 1). norm_w: f32 [D] per-head RMSNorm weight, used when cfg->norm is set.
 * rows: NULL, or y is a KV cache whose row t' = rows(t) receives token t (y_stride_t is then the cache
 * row stride): the reference lowerer's Rope absorbed into its CacheWrite
 * (src/Sharplight.Shaders/Lowering/GraphLowerer.Fusion.cs:633-648, Kernels/rope.slang:110-147).
 * All tensors of one launch that have rows must describe the same rows. */
typedef struct slhip_rope_tensor {
    const void* x;
    void* y;
    const float* norm_w;
    int64_t heads;
    int64_t x_stride_t, x_stride_h;
    int64_t y_stride_t, y_stride_h;
    const slhip_cache_rows* rows;
} slhip_rope_tensor;

typedef struct slhip_rope_cfg {
    int32_t dims;      /* rotated dims (even, <= D); 0 means D. Dims past it are copied */
    int32_t neox;      /* 1: pairs (i, i + dims/2); 0: "normal"/gptj pairs (2i, 2i+1) */
    float base;        /* theta base */
    float freq_scale;  /* multiplies every inverse frequency */
    float attn_factor; /* multiplies cos and sin */
    int32_t norm;      /* 1: per-head RMSNorm (norm_w, eps) before the rotation */
    float eps;
    int32_t pos_axes;  /* A: positions are int32 [T, A], 1..4 (0 means 1) */
    /* Multi-axis rope (M-RoPE; StandardOps.Rope's sections / interleaved / sections_per_element,
     * src/Sharplight.Core/Graph/StandardOps.cs:182-192; RopeOp.AxisOf, src/Sharplight.Cpu/RopeOp.cs:54-106):
     * pair section i takes position axis
     *   sector = i % (s0+s1+s2+s3); sectioned: 0 below s0, 1 below s0+s1, 2 below s0+s1+s2, else 3;
     *   interleaved: 1 if sector % 3 == 1 and sector < 3*s1, 2 if % 3 == 2 and < 3*s2, 0 if % 3 == 0 and
     *   < 3*s0, else 3;
     * with per_element the elements are sectioned two by two (element e takes pair section e/2), so the two
     * elements of a neox pair may rotate by different axes' angles: y0 = x0*c1 - x1*s1, y1 = x0*s2 + x1*c2.
     * An axis beyond A reads axis 0 when A == 1, else position 0. All of s0..s2 zero: one axis. */
    int32_t sections[4];
    int32_t interleaved;
    int32_t per_element;
} slhip_rope_cfg;

/*
 * Rotary embedding of up to 4 tensors that share positions (q and k of one layer in one launch), with
 * the per-head q/k RMSNorm of Qwen3-style blocks fused in front when cfg->norm is set:
 *   inv_i = base^(-2i/dims) * freq_scale (f64); theta = pos[t] * inv_i (/ ff[i]) (f64);
 *   c = (float)cos(theta) * attn_factor, s = (float)sin(theta) * attn_factor;
 *   y0 = x0*c - x1*s, y1 = x0*s + x1*c.
 * pos: int32 [T, cfg->pos_axes]; ff: f32 [dims/2] frequency divisors or NULL. dtype_in: F32 or BF16; dtype_out: F32, F16
 * (for f16 caches) or BF16.
 * Replaces: RopeOp (src/Sharplight.Cpu/RopeOp.cs:28-183) after RowOp RmsNorm, and the Vulkan rope kernels
 * with the absorbed norm (GraphLowerer.Fusion.cs:618-630, GraphLowerer.Transformer.cs:40, Kernels/rope.slang:5-30,150-195),
 * single-axis and multi-axis.
 */
SLHIP_API int slhip_rope(int dtype_in, int dtype_out, const slhip_rope_tensor* tensors, int n_tensors,
                         const int32_t* pos, const float* ff, int64_t T, int64_t D, const slhip_rope_cfg* cfg,
                         slhip_stream stream);

/*
 * Embedding gather y[i, :] = dequant(table[ids[i], :]) for i < N; table is the [V, row_bytes] image of a
 * [V, D] tensor in `format`. dtype_out: F32 or BF16 (f32 values rounded to nearest even). An id outside
 * [0, V) leaves its output row zero and raises SLHIP_ERR_INDEX at the next slhip_stream_sync.
 * Formats: F32, F16, BF16, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1 (D a multiple of 32), Q2_K..Q6_K, IQ4_XS, TQ1_0
 * and TQ2_0 and the grid IQ formats IQ2_XXS..IQ1_M (D a multiple of 256), IQ4_NL and MXFP4 (32), NVFP4 (64),
 * and the reference's formats Q1_0 .. F8E4M3_B128 and the trellis formats (D a multiple of their block size).
 * Replaces: GatherOp (src/Sharplight.Cpu/GatherOp.cs:22-75) with Quant.Dequantize
 * (src/Sharplight.Cpu/Quant.cs:242-446,500-624; Quant.KQuants.cs:36-107), and the Vulkan gather
 * (GraphLowerer.Transformer.cs:133-179, Kernels/data.slang:4-37).
 */
SLHIP_API int slhip_gather(int format, const void* table, int64_t V, int64_t D, const int32_t* ids, int64_t N,
                           int dtype_out, void* y, int64_t y_stride, slhip_stream stream);

/*
 * KV-cache write (CacheWrite without an absorbed producer; src/Sharplight.Cpu/CacheWriteOp.cs:129-175):
 * token t's `inner` values x[t*x_stride, +inner) go to cache[rows(t)*inner, +inner), converted from
 * dtype_in (F32, BF16) to the cache's dtype (F32, F16 rounding to nearest even as .NET's (Half), BF16).
 */
SLHIP_API int slhip_cache_write(int dtype_in, int dtype_cache, const void* x, int64_t x_stride, int64_t T,
                                int64_t inner, void* cache, const slhip_cache_rows* rows, slhip_stream stream);

/*
 * Element type conversion y = cast(x) of n elements (F32, F16, BF16 in any direction); f32 -> bf16 rounds
 * to nearest even with NaNs quieted (Simd.FloatToBFloat, src/Sharplight.Cpu/Simd.cs:530-540).
 * Replaces the CPU provider's Cast of activations.
 */
SLHIP_API int slhip_convert(int dtype_in, int dtype_out, const void* x, void* y, int64_t n, slhip_stream stream);

/* ---- standalone elementwise ops ------------------------------------------------------------------ */

/* Two-operand ops, in the order of the reference's BinaryKind (src/Sharplight.Cpu/BinaryKind.cs:4);
 * SLHIP_BIN_FMOD is Mod with the attribute fmod=true (C fmod: the sign of the dividend). Comparisons and
 * logic ops give 1.0 / 0.0. */
typedef enum slhip_binary_op {
    SLHIP_BIN_ADD = 0, SLHIP_BIN_SUB, SLHIP_BIN_MUL, SLHIP_BIN_DIV, SLHIP_BIN_MAX, SLHIP_BIN_MIN, SLHIP_BIN_POW,
    SLHIP_BIN_MOD, SLHIP_BIN_PRELU, SLHIP_BIN_EQUAL, SLHIP_BIN_NOT_EQUAL, SLHIP_BIN_LESS, SLHIP_BIN_LESS_EQUAL,
    SLHIP_BIN_GREATER, SLHIP_BIN_GREATER_EQUAL, SLHIP_BIN_AND, SLHIP_BIN_OR, SLHIP_BIN_XOR, SLHIP_BIN_ATAN2,
    SLHIP_BIN_FMOD
} slhip_binary_op;

/* One-operand ops, in the order of the reference's UnaryKind (src/Sharplight.Cpu/UnaryKind.cs:4-6). p0/p1
 * are its two parameters: Scale (scale, bias), Clip (min, max), HardSigmoid (alpha, beta), Elu/Celu/
 * ThresholdedRelu/LeakyRelu (alpha), Selu (alpha, gamma)
 * (CpuCompiledSegment.LowerElementwise.cs:31-39). */
typedef enum slhip_unary_op {
    SLHIP_UN_NEG = 0, SLHIP_UN_EXP, SLHIP_UN_LOG, SLHIP_UN_SQRT, SLHIP_UN_RSQRT, SLHIP_UN_SIGMOID, SLHIP_UN_SILU,
    SLHIP_UN_GELU, SLHIP_UN_GELU_TANH, SLHIP_UN_TANH, SLHIP_UN_SOFTPLUS, SLHIP_UN_RELU, SLHIP_UN_ABS,
    SLHIP_UN_SQUARE, SLHIP_UN_RECIP, SLHIP_UN_SCALE, SLHIP_UN_ERF, SLHIP_UN_HARD_SWISH, SLHIP_UN_HARD_SIGMOID,
    SLHIP_UN_CLIP, SLHIP_UN_SIN, SLHIP_UN_COS, SLHIP_UN_TAN, SLHIP_UN_ASIN, SLHIP_UN_ACOS, SLHIP_UN_ATAN,
    SLHIP_UN_SINH, SLHIP_UN_COSH, SLHIP_UN_ASINH, SLHIP_UN_ACOSH, SLHIP_UN_ATANH, SLHIP_UN_FLOOR, SLHIP_UN_CEIL,
    SLHIP_UN_ROUND, SLHIP_UN_SIGN, SLHIP_UN_SOFTSIGN, SLHIP_UN_MISH, SLHIP_UN_ELU, SLHIP_UN_CELU, SLHIP_UN_SELU,
    SLHIP_UN_LEAKY_RELU, SLHIP_UN_THRESHOLDED_RELU, SLHIP_UN_NOT, SLHIP_UN_IS_NAN, SLHIP_UN_IS_INF
} slhip_unary_op;

/*
 * y = op(a, b) with numpy-style broadcasting, y dense [dims] (rank <= 8). a_strides / b_strides: element
 * strides of a and b aligned to y's rank, 0 along a dim the operand broadcasts (extent 1, or missing in
 * front) -- BinaryOp's Align (src/Sharplight.Cpu/BinaryOp.cs:37-58); NULL means dense [dims].
 * dtype_a: F32, F16 or BF16; dtype_b: dtype_a or F32 (a bias or scale kept in f32); dtype_out: any.
 * Arithmetic in f32 as BinaryOp (BinaryOp.cs:60-357): Max/Min propagate NaN and order -0 below +0; Pow
 * with an exponent that is one value along y's innermost dim takes BinaryOp.Apply's forms for 2, 1, 0.5
 * and 3. y may alias a or b when it has that operand's shape and layout.
 * Replaces: BinaryOp and the Vulkan lowerer's generated elementwise kernels
 * (src/Sharplight.Shaders/Lowering/GraphLowerer.Elementwise.cs:60-200).
 */
SLHIP_API int slhip_binary(int op, int dtype_a, int dtype_b, int dtype_out, const void* a, const int64_t* a_strides,
                           const void* b, const int64_t* b_strides, void* y, const int64_t* dims, int rank,
                           slhip_stream stream);

/*
 * y = op(x) over [rows, cols] with row strides (elements). dtype_in, dtype_out: F32, F16 or BF16.
 * The forms are ScalarMath.Unary's vector forms (src/Sharplight.Cpu/ScalarMath.cs:100-650): Scale and
 * HardSigmoid/HardSwish fused multiply-adds, Gelu with the f64 rational erf (as slhip_gated_act),
 * GeluTanh as v / (1 + exp(-u)), Softplus in f64; exp, tanh, log and the trigonometric functions to
 * within 2 f32 ulp of the correctly rounded value.
 * Replaces: UnaryOp (src/Sharplight.Cpu/UnaryOp.cs:30-75) and the lowerer's lone-activation kernels.
 */
SLHIP_API int slhip_unary(int op, int dtype_in, int dtype_out, const void* x, void* y, int64_t rows, int64_t cols,
                          int64_t x_stride, int64_t y_stride, float p0, float p1, slhip_stream stream);

/*
 * A fused elementwise group (the lowerer's generated elementwise kernel, src/Sharplight.Shaders/Lowering/
 * GraphLowerer.Fusion.cs:88-205), optionally with the row norm before it (FoldNormHeads, :240-284) or after it
 * (FoldNormTails, :211-238), over an output of [rows, cols] (cols a multiple of 4):
 *   registers 0 .. n_inputs-1 are loaded with the inputs, each FULL ([rows, cols]), ROW (one value per
 *   column: [cols]), COL (one value per row: [rows]) or SCALAR (one value); f32 / bf16 / f16, FULL and ROW
 *   inputs 16-byte (f32) or 8-byte aligned; then the ops run in order, op k (kind BINARY: slhip_binary_op of
 *   registers a, b; UNARY: slhip_unary_op of register a with p0, p1) writing register dst in f32, rounded to
 *   `round` (the node's output type); SLHIP_EW_MAX_REGS registers;
 *   each output stores one register ([rows, cols], f32 / bf16 / f16).
 *   head (kind SLHIP_EWN_RMS / SLHIP_EWN_L2, SLHIP_EWN_NONE for none): input register `reg` is replaced by
 *   round(norm(input) * w) (w [cols] f32 or NULL; round to dtype_y) before the ops;
 *   tail: y [rows, cols] (dtype_y) = norm(register reg) * w after the ops; at most one of head and tail.
 * The arithmetic is that of slhip_binary / slhip_unary / slhip_rownorm per node, so the group equals the
 * nodes run one by one. */
#define SLHIP_EW_MAX_INPUTS 8
#define SLHIP_EW_MAX_OPS 16
#define SLHIP_EW_MAX_OUTPUTS 4
#define SLHIP_EW_MAX_REGS 16
typedef enum slhip_ew_input_mode { SLHIP_EWI_FULL = 0, SLHIP_EWI_ROW = 1, SLHIP_EWI_COL = 2, SLHIP_EWI_SCALAR = 3 } slhip_ew_input_mode;
typedef enum slhip_ew_op_kind { SLHIP_EWK_BINARY = 0, SLHIP_EWK_UNARY = 1 } slhip_ew_op_kind;
typedef enum slhip_ew_norm_kind { SLHIP_EWN_NONE = 0, SLHIP_EWN_RMS = 1, SLHIP_EWN_L2 = 2 } slhip_ew_norm_kind;
typedef struct slhip_ew_input {
    const void* data;
    int dtype;
    int mode;
} slhip_ew_input;
typedef struct slhip_ew_op {
    int kind, op;
    int a, b;   /* source registers */
    int dst;    /* destination register */
    int round;  /* SLHIP_F32 (none), SLHIP_BF16 or SLHIP_F16 */
    float p0, p1;
} slhip_ew_op;
typedef struct slhip_ew_output {
    void* data;
    int dtype;
    int reg;
} slhip_ew_output;
typedef struct slhip_ew_norm {
    int kind;     /* slhip_ew_norm_kind */
    int reg;
    const float* w;
    float eps;
    void* y;      /* tail only */
    int dtype_y;
} slhip_ew_norm;
typedef struct slhip_ew_program {
    int n_inputs, n_ops, n_outputs;
    slhip_ew_input inputs[SLHIP_EW_MAX_INPUTS];
    slhip_ew_op ops[SLHIP_EW_MAX_OPS];
    slhip_ew_output outputs[SLHIP_EW_MAX_OUTPUTS];
    slhip_ew_norm head, tail;
} slhip_ew_program;
SLHIP_API int slhip_ew_program_run(const slhip_ew_program* prog, int64_t rows, int64_t cols, slhip_stream stream);

/* ---- provider / compiled segment (IExecutionProvider, IComputeDevice, ICompiledSegment) ----------------
 *
 * A graph segment arrives as text, one declaration per line ('#' starts a comment line):
 *   value <id> <type> <dim> ...       type: a DataType name of the reference (f32 f16 bf16 i32, and the
 *                                     block formats slhip_format lists: q8_0 q4_k iq2_xxs nf4_b64 ...); a dim
 *                                     is a size (at most 2^40; at most 2^46 elements per value without T), or
 *                                     "T", the symbolic token count bound at execute time (at most
 *                                     max_tokens); other symbols are refused
 *   input <id> | weight <id> | output <id> | state <id>    (a state -- a KV cache -- has fixed dims, persists
 *                                     across runs, starts at zero and is zeroed again by reset_state)
 *   node <Op> <in,ids> -> <out,ids> [key=value ...]
 *   option <key>=<value> ...         compile options: reduced_precision=0|1 (CompileOptions.
 *                                     AllowReducedPrecision), int_dot=lowerer|cpu|off (below)
 * with the StandardOps names and attributes of the reference (src/Sharplight.Core/Graph/StandardOps.cs):
 *   the binary ops Add, Sub, Mul, Div, Max, Min, Pow, Mod (fmod), PRelu, the comparisons and logic ops,
 *   Atan2 (numpy broadcasting), the one-operand ops of slhip_unary_op by name, Scale (scale, bias), Clip
 *   (min, max), HardSigmoid (alpha, beta), Elu/Celu/LeakyRelu/ThresholdedRelu (alpha), Selu (alpha, gamma),
 *   RmsNorm (x[, w]; eps), L2Norm (x; eps),
 *   LayerNorm (x[, w[, b]]; eps), Rope (x [T,H,D], pos i32 [T] or [T,A<=4][, ff]; dims, base,
 *   style=neox|normal|gptj, freq_scale, attn_factor, sections=s0,s1,s2,s3, interleaved, sections_per_element),
 *   Gather (table [V, D...], ids i32 [N]), Cast,
 *   CacheWrite (state [ctx, ...], x [T, ...][, rows i32 [T,4][, pages i32 [slots, blocks]]]; offset=<scalar
 *   name, default n_past>, slots, block_size): rows n_past + t, or the multi-sequence / paged rows,
 *   MatMul (x [.., K] f32/bf16, a weight [N, K]; f32_activations): the decode matvec.
 * A MatMul quantizes x to q8 and runs the integer-dot matvec (slhip_quantize_q8 + slhip_matvec_q8, one q8 copy
 * per x and row range shared by the matmuls that read it) unless it carries f32_activations=1 and the
 * compile does not allow reduced precision (GraphLowerer.IntDot.cs:61-62), for the activation row counts of
 * the rule int_dot names: "lowerer" (default; GraphLowerer.IntDot.cs:18-19,52-75): Q8_0 2..16 rows,
 * Q4_K/Q5_K/Q6_K and Q4_0/Q5_0/IQ4_NL/MXFP4 1..8 rows; "cpu" (MatMulOp.cs:104,138-147): every format of
 * IntDot.Supports, 1..31 rows; "off": never. Other row counts take the f32 matvec (IQ4_NL, IQ4_XS and MXFP4
 * have no f32 matvec: such a run fails with SLHIP_ERR_UNSUPPORTED). A MatMul whose product only feeds an Add
 * of a constant f32 [N] weight folds the Add into its launch (FoldMatMulBiases).
 * Compile applies the reference lowerer's fusions (Add+RmsNorm, act+Mul, RmsNorm inside Rope, a Rope whose
 * only consumer is a CacheWrite stored into the cache, q/k ropes in one launch); slhip_segment_launches
 * lists the fused launches, one per line. Segments run on a stream
 * of their own on the device current at compile time. */
typedef void* slhip_segment;

/* IExecutionProvider.CheckAvailability (IExecutionProvider.cs:30): SLHIP_OK when a device is usable, else a
 * status and the reason (no device, no runtime). Never throws; cheap. */
SLHIP_API int slhip_provider_check(char* reason, size_t reason_size);
/* IComputeDevice.Supports(Node) (IComputeDevice.cs:30-31) for node `node_index` of a segment text:
 * *supported = 1, or 0 with the reason (the node then goes to the placement fallback). */
SLHIP_API int slhip_node_supports(const char* segment_ir, int node_index, int* supported, char* reason,
                                  size_t reason_size);
/* IComputeDevice.Compile (IComputeDevice.cs:33-38): allocates every value for max_tokens tokens
 * (CompileOptions.MaxTokens, 0 .. 2^20). SLHIP_ERR_UNSUPPORTED for a node or pattern this provider cannot run. */
SLHIP_API int slhip_segment_compile(const char* segment_ir, int64_t max_tokens, slhip_segment* segment);
/* ICompiledSegment.SetInput (ICompiledSegment.cs:9-10): dense host bytes of an input or weight value. */
SLHIP_API int slhip_segment_set_input(slhip_segment segment, int value, const void* data, size_t bytes);
/* ICompiledSegment.Execute: runs the launches for `tokens` tokens; asynchronous until an output is read.
 * A token count above the compiled bound fails like CpuCompiledSegment.Execute
 * (src/Sharplight.Cpu/CpuCompiledSegment.cs:115-121). */
SLHIP_API int slhip_segment_execute(slhip_segment segment, int64_t tokens);
/* ICompiledSegment.GetOutput: waits for the segment, then copies the output's dense bytes for the last
 * run's token count (the size must match); a state value reads back the whole state. Reports a gather
 * index error as SLHIP_ERR_INDEX and a cache row outside the cache as SLHIP_ERR_CACHE. */
SLHIP_API int slhip_segment_get_output(slhip_segment segment, int value, void* data, size_t bytes);
/* ICompiledSegment.ResetState: every state back to zero (CpuCompiledSegment.ResetState,
 * src/Sharplight.Cpu/CpuCompiledSegment.cs:259-265); and DeviceMemoryBytes. */
SLHIP_API int slhip_segment_reset_state(slhip_segment segment);
/* A runtime scalar of the next runs (RunParameters.Scalars, src/Sharplight.Core/Runtime/RunParameters.cs:12),
 * e.g. n_past for CacheWrite. A CacheWrite whose scalar was never set fails like CacheWriteOp.Run. */
SLHIP_API int slhip_segment_set_scalar(slhip_segment segment, const char* name, int64_t value);
SLHIP_API int slhip_segment_device_bytes(slhip_segment segment, int64_t* bytes);
/* The fused launches of the compiled segment, one label per line (e.g. "fused[Add]+RmsNorm"). */
SLHIP_API int slhip_segment_launches(slhip_segment segment, char* buf, size_t size);
/* The launches a run of `tokens` tokens makes, one per line: the units whose row-count condition holds, each
 * matvec labelled with the path it takes (" int-dot" or " f32"), a quantization as "x->q8". */
SLHIP_API int slhip_segment_launches_at(slhip_segment segment, int64_t tokens, char* buf, size_t size);
/* The launches slhip_segment_compile would create for a segment text, one label per line, decided without
 * touching a device: the lowerer's plan (GraphLowerer.Lower, src/Sharplight.Shaders/Lowering/GraphLowerer.cs:
 * 64-71, without the buffers). Fails as compile would for a node or pattern this provider cannot run. */
SLHIP_API int slhip_segment_plan(const char* segment_ir, char* buf, size_t size);
/* The segment text as the provider read it, in canonical form: value lines by id, then the input, weight,
 * output and state lines by id, then the node lines in order with their attributes sorted by key. No device
 * is touched; malformed text fails as compile would. A buffer too small fails (nothing is truncated). */
SLHIP_API int slhip_segment_describe(const char* segment_ir, char* buf, size_t size);
SLHIP_API int slhip_segment_destroy(slhip_segment segment);

/* ---- GGUF files and weight upload (the on-disk -> device path) --------------------------------
 *
 * A GGUF file (versions 2 and 3) memory-mapped read-only, its header, metadata and tensor table parsed
 * with every read bounds-checked, so a truncated or hostile file fails with SLHIP_ERR_FORMAT instead of
 * reading out of bounds. Replaces GgufFile.Open and its reader (src/Sharplight.Import.Gguf/GgufFile.cs:72-110,
 * GgufReader.cs:1-175); the uploader replaces the Vulkan provider's staged weight upload
 * (src/Sharplight.Vulkan/WeightUploader.cs:6-140). Strings returned by these functions live until
 * slhip_gguf_close; host pointers into the mapping likewise. Parsing touches no device. */

typedef struct slhip_gguf slhip_gguf; /* an open file, or a header prefix */

/* GGUF metadata value types (gguf_metadata_value_type; GgufValueType.cs:4-19). */
typedef enum slhip_gguf_vtype {
    SLHIP_GGUF_UINT8 = 0, SLHIP_GGUF_INT8 = 1, SLHIP_GGUF_UINT16 = 2, SLHIP_GGUF_INT16 = 3,
    SLHIP_GGUF_UINT32 = 4, SLHIP_GGUF_INT32 = 5, SLHIP_GGUF_FLOAT32 = 6, SLHIP_GGUF_BOOL = 7,
    SLHIP_GGUF_STRING = 8, SLHIP_GGUF_ARRAY = 9, SLHIP_GGUF_UINT64 = 10, SLHIP_GGUF_INT64 = 11,
    SLHIP_GGUF_FLOAT64 = 12
} slhip_gguf_vtype;

typedef struct slhip_gguf_info {
    uint32_t version;        /* 2 or 3 (0 for a prefix that is not GGUF) */
    uint32_t alignment;      /* general.alignment, default 32 */
    int64_t n_tensors;       /* entries in the tensor table (0 for a prefix that does not hold it whole) */
    int64_t n_kv;            /* metadata pairs read (a prefix: the pairs it holds whole) */
    int64_t data_offset;     /* absolute offset of the tensor data section (-1 when unknown) */
    int64_t file_length;     /* bytes mapped (a prefix: its length) */
    int32_t has_data;        /* 1: opened from a file, tensor data readable; 0: a header prefix */
    int32_t table_complete;  /* 1 when the whole tensor table was read */
} slhip_gguf_info;

/* One metadata value, a node of the value tree. Scalars: `u` (unsigned and bool), `i` (signed) or `f`
 * (float32 widened exactly, float64). Strings: `data` -> `count` UTF-8 bytes (not NUL-terminated).
 * Arrays: `elem_type` and `count`; numeric and bool elements are `count` packed little-endian values at
 * `data` (unaligned); string and array elements are the nodes first_child .. first_child + count - 1. */
typedef struct slhip_gguf_value {
    uint32_t type;
    uint32_t elem_type;
    int64_t count;
    uint64_t u;
    int64_t i;
    double f;
    const void* data;
    int64_t first_child;
} slhip_gguf_value;

/* A tensor of the table (GgufTensorInfo, GgufTensorInfo.cs:7-79). The element type is the one the file's
 * ggml type id is read as (GgmlTypes.TryGetDataType, GgmlTypes.cs:94-119): the interleaved Q4_0 ids 31-33
 * read as q4_0 rows, the narrow IQ1 ids 64-66 as iq1_s blocks, I2_S (36) as q2s_g128 blocks. */
typedef struct slhip_gguf_tensor {
    const char* name;
    const char* type_name;   /* the reference's DataType name, e.g. "q4_k", "bf16" */
    int32_t ggml_type;       /* the id stored in the file */
    int32_t format;          /* the slhip_format this library's kernels read it as, or -1 */
    int32_t block_size;      /* values per block (1 for plain element types) */
    int32_t block_bytes;
    int32_t n_dims;
    int32_t reserved;
    int64_t ne[8];           /* ggml dimensions, innermost first */
    int64_t relative_offset; /* from the start of the data section */
    int64_t offset;          /* absolute file offset (0 for a prefix) */
    int64_t byte_size;       /* bytes as the element type above */
    int64_t stored_bytes;    /* bytes the file holds for it */
} slhip_gguf_tensor;

/* Opens and maps `path` (GgufFile.Open). SLHIP_ERR_FORMAT: not GGUF, truncated, a tensor beyond the end
 * of the file, a row length that is not a multiple of its type's block size; SLHIP_ERR_UNSUPPORTED: a
 * GGUF version other than 2/3 or an unknown ggml type id; SLHIP_ERR_INVALID: the file cannot be opened. */
SLHIP_API int slhip_gguf_open(const char* path, slhip_gguf** file);
/* Parses the first `length` bytes of a GGUF file (copied; GgufHeaderProbe.ReadMetadata / ReadTensorTable,
 * GgufHeaderProbe.cs:17-135): the pairs it holds whole, and the tensor table when it holds all of it
 * (type ids unknown to this library are kept, with type_name "" and sizes 0). Never fails on content. */
SLHIP_API int slhip_gguf_open_prefix(const void* bytes, size_t length, slhip_gguf** file);
SLHIP_API int slhip_gguf_close(slhip_gguf* file);
SLHIP_API int slhip_gguf_get_info(const slhip_gguf* file, slhip_gguf_info* info);
/* Metadata pair `index` (file order): its key and the node of its value. */
SLHIP_API int slhip_gguf_kv(const slhip_gguf* file, int64_t index, const char** key, int64_t* node);
/* The pair of `key`, -1 when absent (the last one when a key repeats, as the reference's dictionary). */
SLHIP_API int slhip_gguf_find_kv(const slhip_gguf* file, const char* key, int64_t* index);
SLHIP_API int slhip_gguf_get_value(const slhip_gguf* file, int64_t node, slhip_gguf_value* value);
SLHIP_API int slhip_gguf_tensor_info(const slhip_gguf* file, int64_t index, slhip_gguf_tensor* tensor);
/* The tensor named `name`, -1 when absent (GgufFile.FindTensor). */
SLHIP_API int slhip_gguf_find_tensor(const slhip_gguf* file, const char* name, int64_t* index);
/* Describes a ggml type id as the tensor table would (name, block size and bytes, slhip_format);
 * SLHIP_ERR_UNSUPPORTED for an unknown or removed id (GgmlTypes.GetDataType). */
SLHIP_API int slhip_gguf_type(int ggml_type, slhip_gguf_tensor* type);
/* Host read of bytes [offset, offset + bytes) of a tensor as its element type (IWeightSource.Read:
 * GgufWeightSource.cs:9-19, GgufInterleavedQ4_0Source.cs:43-79, GgufI2sSource.cs:39-64): the interleaved
 * Q4_0 rows de-interleaved, I2_S codes with the tensor's scale in front of every block, the narrow IQ1
 * blocks widened to IQ1_S (GgmlNarrowIq1.cs:55-86). SLHIP_ERR_INDEX for a range outside the tensor. */
SLHIP_API int slhip_gguf_read(const slhip_gguf* file, int64_t index, int64_t offset, void* dst, size_t bytes);
/* The tensor's bytes in the mapping when they are its element type's bytes as stored (TryGetPointer),
 * else NULL. */
SLHIP_API int slhip_gguf_tensor_pointer(const slhip_gguf* file, int64_t index, const void** ptr);
/* Uploads a whole tensor, as slhip_gguf_read returns it, to device memory `dst` of at least byte_size
 * bytes, through the staging uploader below (WeightUploader.Upload). */
SLHIP_API int slhip_gguf_upload(const slhip_gguf* file, int64_t index, void* dst, size_t dst_bytes,
                                slhip_stream stream);
/* Copies `bytes` of pageable host memory (a mapped file, say) to device memory through two pinned
 * staging buffers of the current device: host threads fill one while the DMA engine drains the other.
 * Returns once every source byte has been read; the device copies are ordered on `stream` (wait on it
 * before reading dst). Calls on one device serialize on its uploader. Staging size
 * SLHIP_UPLOAD_STAGING_MB (default 64 MiB per buffer), host threads SLHIP_UPLOAD_THREADS (default 8). */
SLHIP_API int slhip_upload(void* dst, const void* src, size_t bytes, slhip_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* SHARPLIGHT_HIP_H */
