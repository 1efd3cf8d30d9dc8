/*
 * CPU oracle for the Sharplight fused layer ops -- TEST INFRASTRUCTURE ONLY.
 *
 * A restatement in plain C of the arithmetic of the reference's CPU execution provider
 * (src/Sharplight.Cpu) for the ops on the fused-layer path. It is the parity checker for the
 * HIP kernels of libsharplight_hip and the timed CPU baseline of bench.py; nothing in the
 * product links it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.
 *
 * Conventions: all activations are f32 (the reference CPU provider has no bf16 activations);
 * the bf16 helpers restate the provider's own f32<->bf16 casts. Every function that touches a
 * row range runs on the calling thread; the *_mt variants split the work the way the
 * reference's CpuParallel.For does (chunks = min(threads*4, total/minChunk)).
 */
#ifndef SL_ORACLE_H
#define SL_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Table formats, numbered like the C ABI's slhip_format (include/sharplight_hip.h). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_Q8_0 = 3, ORC_Q4_0 = 4, ORC_Q4_1 = 5, ORC_Q5_0 = 6, ORC_Q5_1 = 7,
       ORC_Q2_K = 8, ORC_Q3_K = 9, ORC_Q4_K = 10, ORC_Q5_K = 11, ORC_Q6_K = 12, ORC_IQ4_NL = 13, ORC_IQ4_XS = 14,
       ORC_TQ1_0 = 15, ORC_TQ2_0 = 16, ORC_MXFP4 = 17, ORC_NVFP4 = 18, ORC_IQ2_XXS = 19, ORC_IQ2_XS = 20,
       ORC_IQ2_S = 21, ORC_IQ3_XXS = 22, ORC_IQ3_S = 23, ORC_IQ1_S = 24, ORC_IQ1_M = 25,
       /* the reference's own formats */
       ORC_Q1_0 = 26, ORC_Q2_0 = 27, ORC_Q2_0_G128 = 28, ORC_TERN1_G128 = 29, ORC_NVFP4_GS = 30, ORC_Q4Z_G32 = 31,
       ORC_Q4Z_G128 = 32, ORC_Q8Z_G32 = 33, ORC_Q8Z_G128 = 34, ORC_NF4_B64 = 35, ORC_FP4_B64 = 36, ORC_Q8A_G32 = 37,
       ORC_Q2S_G128 = 38, ORC_F8E4M3 = 39, ORC_F8E5M2 = 40, ORC_F8E4M3_B32 = 41, ORC_F8E4M3_B128 = 42,
       /* trellis-coded (TrellisBlocks.cs), 128 values per block */
       ORC_TRELLIS_V4K8 = 43, ORC_TRELLIS_V4K6 = 44, ORC_TRELLIS_V4K7 = 45, ORC_TRELLIS_V2K5 = 46,
       ORC_TRELLIS_V2K6 = 47, ORC_TRELLIS_V2K7 = 48 };
/* E4M3FN / E5M2 byte -> f32 (Quant.E4m3ToFloat, Quant.BuildE5m2) */
float orc_e4m3_value(uint8_t x);
float orc_e5m2_value(uint8_t x);

/* ---- scalar conversions (Simd.cs:518-540, Quant.cs:371-381) ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n);
void orc_bf16_to_f32_n(const uint16_t* x, float* y, int64_t n);
void orc_f16_to_f32_n(const uint16_t* x, float* y, int64_t n);

/* ---- reductions (Simd.cs:274-340) ---- */
float orc_sumsq(const float* a, int64_t n);
float orc_sum(const float* a, int64_t n);

/* ---- row ops (RowOp.cs:37-113); mode 0 = RmsNorm, 1 = L2Norm ---- */
void orc_rmsnorm(const float* x, const float* w, float* y, int64_t rows, int64_t n, float eps, int mode);
void orc_layernorm(const float* x, const float* w, const float* b, float* y, int64_t rows, int64_t n, float eps);

/* ---- elementwise (BinaryOp.cs:8-103, ScalarMath.cs:521-641) ---- */
void orc_add(const float* a, const float* b, float* y, int64_t n);
void orc_mul(const float* a, const float* b, float* y, int64_t n);
/* act: 0 = Silu, 1 = GeluTanh, 2 = Gelu (erf) */
void orc_unary(int act, const float* x, float* y, int64_t n);
/* kind: the reference's UnaryKind number (Neg = 0 ... IsInf = 44); p0/p1 its two parameters */
void orc_unary_kind(int kind, const float* x, float* y, int64_t n, float p0, float p1);
/* kind: BinaryKind number (Add = 0 ... Atan2 = 18), 19 = Mod with fmod; y dense [dims], a/b aligned strides */
void orc_binary(int kind, const float* a, const int64_t* sa, const float* b, const int64_t* sb, float* y,
                const int64_t* dims, int rank);
void orc_align(const int64_t* a_dims, int a_rank, int y_rank, int64_t* strides);
double orc_erf(double x);
float orc_erf_rational(float x);

/* ---- rope (RopeOp.cs:28-183); x,y [T,H,D] dense; pos [T]; ff [dims/2] or NULL ---- */
void orc_rope(const float* x, const int32_t* pos, const float* ff, float* y, int64_t T, int64_t H, int64_t D, int dims,
              int neox, float base, float freq_scale, float attn_factor);

/* Multi-axis rope: pos [T, axes] (axes 1..4), sections[4] (NULL or all of [0..2] zero: one axis),
 * interleaved (Qwen3-VL sectors), per_element (XD-RoPE: element e takes the axis of pair section e/2). */
void orc_rope_multi(const float* x, const int32_t* pos, int axes, const int32_t* sections, int interleaved,
                    int per_element, const float* ff, float* y, int64_t T, int64_t H, int64_t D, int dims, int neox,
                    float base, float freq_scale, float attn_factor);
int orc_rope_axis_of(int i, const int32_t* sections, int interleaved);

/* ---- dequant / gather (Quant.cs:242-405, GatherOp.cs:22-75) ---- */
int64_t orc_row_bytes(int fmt, int64_t d);
int orc_dequant(int fmt, const uint8_t* src, int64_t count, float* dst);
/* Returns 0, or -1 with *bad_index set to the first out-of-range id (the reference throws). */
int orc_gather(int fmt, const uint8_t* table, int64_t V, int64_t D, const int32_t* ids, int64_t N, float* y,
               int64_t* bad_index);

/* ---- KV cache writes (CacheWriteOp.cs, KvPages.cs) ---- */
enum { ORC_ROWS_PAST = 0, ORC_ROWS_SEQ = 1, ORC_ROWS_PAGED = 2 };
uint16_t orc_f32_to_f16(float f);
void orc_f32_to_f16_n(const float* x, uint16_t* y, int64_t n);
/* Cache row of every token (all checked first); 0, or -1 with the reference's message in err. */
int orc_cache_rows(int mode, int64_t T, int64_t ctx, int64_t n_past, const int32_t* seq, int64_t slots,
                   const int32_t* pages, int64_t page_slots, int64_t blocks_per_slot, int64_t block_size,
                   int64_t* rows, char* err, int64_t err_size);
/* x [T, inner] f32 -> cache rows[t] (cache_type ORC_F32 / ORC_F16 / ORC_BF16). */
void orc_cache_write(int cache_type, void* cache, int64_t inner, const float* x, int64_t T, const int64_t* rows);

/* ---- E4M3 activation rows (Kernels/e4m3.slang, Kernels/gemm_fp8.slang quantize_fp8) ---- */
uint8_t orc_e4m3_code(float v);
/* rows of K values (K % 128 == 0) -> rows of K + K/32 bytes: K codes, then K/128 f32 scales */
void orc_quantize_fp8_rows(const float* x, int64_t rows, int64_t K, uint8_t* out);
void orc_quantize_fp8_rows_mt(const float* x, int64_t rows, int64_t K, uint8_t* out);
void orc_f32_to_f16_mt(const float* x, uint16_t* y, int64_t n);

/* ---- Matvec y = x . W^T for few activation rows (MatMulOp's float-row path) ---- */
int orc_matvec(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y);
int orc_matvec_mt(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y);

/* ---- Integer-dot matvec: q8 activations (MatMulOp's IntDot path, IntDot.cs) ----
 * quantized rows: q int8 [rows][K], d f32 [rows][K/32] (block scales), gs f32 [rows][K/16] (d * sum q per 16) */
int orc_q8_quantize(const float* x, int64_t rows, int64_t K, int8_t* q, float* d, float* gs);
/* weight row -> codes u [K], multiplier a and offset b per 16 values (value = a u + b) */
int orc_intdot_decode(int fmt, const uint8_t* row, int64_t K, uint8_t* u, float* a, float* b);
float orc_intdot_dot(const uint8_t* u, const float* a, const float* b, const int8_t* q, const float* d, const float* gs,
                     int64_t K);
int orc_intdot_supported(int fmt);
/* y [T, N] (may be null); yabs [T, N] (may be null): sum |a d s| + |b gs| per output */
int orc_matvec_q8(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y, double* yabs);
int orc_matvec_q8_mt(int fmt, const uint8_t* w, int64_t N, int64_t K, const float* x, int64_t T, float* y);

/* ---- threaded variants for the CPU baseline (CpuParallel.cs:34-78) ---- */
void orc_set_threads(int threads);
int orc_get_threads(void);
void orc_rmsnorm_mt(const float* x, const float* w, float* y, int64_t rows, int64_t n, float eps, int mode);
void orc_layernorm_mt(const float* x, const float* w, const float* b, float* y, int64_t rows, int64_t n, float eps);
void orc_add_mt(const float* a, const float* b, float* y, int64_t n);
void orc_mul_mt(const float* a, const float* b, float* y, int64_t n);
void orc_unary_mt(int act, const float* x, float* y, int64_t n);
void orc_rope_mt(const float* x, const int32_t* pos, const float* ff, float* y, int64_t T, int64_t H, int64_t D, int dims,
                 int neox, float base, float freq_scale, float attn_factor);
void orc_cache_write_mt(int cache_type, void* cache, int64_t inner, const float* x, int64_t T, const int64_t* rows);
int orc_gather_mt(int fmt, const uint8_t* table, int64_t V, int64_t D, const int32_t* ids, int64_t N, float* y,
                  int64_t* bad_index);

#ifdef __cplusplus
}
#endif
#endif
