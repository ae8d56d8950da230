/*
 * glypr_oracle.h — CPU restatement of glypr's CPU Q8_0 path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the correctness oracle and the
 * timed CPU baseline for the HIP backend in glypr_amd/.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker.  The product library (libglypr_hip.so) never links,
 * loads or calls it.
 *
 * Reference: phrozen/glypr v0.3.0 (Rust) on candle-core 0.11.0.  candle is a
 * crates.io dependency (Cargo.lock:258-261) that is not vendored in the
 * reference tree; its Q8_0 arithmetic (k_quants::BlockQ8_0 from_float /
 * to_float / vec_dot_unopt and k_quants::matmul) is restated here from the
 * published GGML Q8_0 definition.  Every function cites the glypr call site
 * it follows.
 *
 * Block format (GGUF Q8_0): 34 bytes = { uint16 f16 scale d; int8 qs[32] },
 * rows of K/32 blocks, row-major [N][K/32].
 *
 * How each function is pinned (tests/test_oracle.py):
 *  - f16 codec: every finite f16 and RNE ties against numpy's float16.
 *  - quantize / dequantize / vec_dot: exact known-answer blocks
 *    (tests/golden/q8_0_kat.json), float64 restatement of the definition,
 *    lossless case (GEMM == numpy float64 X @ W^T exactly).
 *  - matmul / matmul_preq: float64 brute force over the same quantized operands.
 *  - vec_dot_fma / matmul_fma: exact rational brute force of every fused
 *    rounding on small inputs, vec_dot itself for one block (k = 32), and the
 *    float64 brute force within the fused form's error bound.
 *  - rmsnorm: constant-row KAT, float64 formula, 2^k scale invariance.
 *  - tanhf / geglu: double-precision tanh (<= 3 ulp), exact special points.
 *  - embed_gather, pool_normalize: dequantized rows; closed-form KAT and the
 *    reference's long-context generator against float64.
 *  - l2_normalize / cosine: the reference's own known answers (util.rs:258-268),
 *    numpy's sequential float32 accumulate (np.add.accumulate) bit for bit,
 *    zero-norm and clamp special cases, float64 within f32 rounding.
 *  - attention: chunked band == dense masked attention in float64.
 *  - rope_tables: closed form (f32 product, float64 cos/sin).
 *  - encoder_layer / model_forward: an independent float64 statement of the
 *    whole forward at small dimensions, both layer types.
 *  - vector codecs (binary / int8 quantize, hamming, int8 dot, both cosines):
 *    the reference's own known answers (tests/quantization.rs:10-31,
 *    util.rs:273-306), brute-force bit/integer sums, complement and symmetry
 *    invariants, and the float64 cosine within f32 rounding.
 * Parity unpinned (no runnable reference vector exists offline): the exact f32
 * bit pattern of candle's vec_dot accumulation (scalar vec_dot_unopt order is
 * restated; AVX/NEON builds differ in the last bits), pulp's RMSNorm lane order
 * (the AVX2 8-lane order is restated), and the platform tanhf (this file's own
 * tanh replaces it; the substitution is bounded by a test).
 */
#ifndef GLYPR_ORACLE_H
#define GLYPR_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QK8_0 32
#define ORC_BLOCK_BYTES 34

/* ---- f16 codec (half 2.7.1 semantics: round-to-nearest-even) ---- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_array(const float* x, uint16_t* y, int64_t n);
void orc_f16_to_f32_array(const uint16_t* x, float* y, int64_t n);

/* ---- Q8_0 block codec ---- */
/* BlockQ8_0::from_float (activation / weight quantize), k % 32 == 0. */
void orc_q8_0_quantize_row(const float* x, int64_t k, uint8_t* blocks);
/* Quantize m rows of k floats into m*(k/32) blocks. */
void orc_q8_0_quantize_rows(const float* x, int64_t m, int64_t k, uint8_t* blocks);
/* BlockQ8_0::to_float / QTensor::dequantize: y = f32(d) * q (exact). */
void orc_q8_0_dequantize_row(const uint8_t* blocks, int64_t k, float* y);
void orc_q8_0_dequantize_rows(const uint8_t* blocks, int64_t rows, int64_t k, float* y);

/* BlockQ8_0::vec_dot_unopt: sum_b ((float)isum_b * f32(d_w)) * f32(d_x), f32 sequential. */
float orc_q8_0_vec_dot(int64_t k, const uint8_t* wblocks, const uint8_t* xblocks);
/* INT8_FMA (this backend's third variant): sum = fmaf((float)isum_b * d_w, d_x, sum). */
float orc_q8_0_vec_dot_fma(int64_t k, const uint8_t* wblocks, const uint8_t* xblocks);
void orc_q8_0_matmul_fma(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                         float* y, int threads);

/* k_quants::matmul::<BlockQ8_0> as reached from LinearOp::forward (Quantized arm):
 * x f32 [m,k], w Q8_0 [n][k/32], y f32 [m,n].  threads <= 0 -> all cores. */
void orc_q8_0_matmul(const float* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                     float* y, int threads);
/* Same GEMM on pre-quantized activations (xq: m*(k/32) blocks). */
void orc_q8_0_matmul_preq(const uint8_t* xq, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                          float* y, int threads);
/* Float64 brute force over the same quantized operands (checker for the above):
 * y = sum_b I_b * d_w * d_x in double. */
void orc_q8_0_matmul_f64(const uint8_t* xq, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                         double* y);
/* Dequant oracle (CANDLE_DEQUANTIZE_ALL / Metal semantics): double sum of
 * x[m,k] * (f32(d)*q)[n,k]; activations are NOT quantized. */
void orc_q8_0_matmul_dequant_f64(const float* x, int64_t m, int64_t k, const uint8_t* w,
                                 int64_t n, double* y, int threads);

/* ---- RMSNorm (cpu_simd/rmsnorm.rs:6-47) ---- */
/* weight may be NULL (v_norm). eps is the f32 value. */
void orc_rmsnorm_row(const float* x, const float* weight, float eps, float* y, int64_t d);
void orc_rmsnorm(const float* x, const float* weight, float eps, float* y, int64_t rows,
                 int64_t d, int threads);

/* ---- GeGLU (cpu_simd/geglu.rs:6-18) ---- */
float orc_tanhf(float x);
float orc_geglu_scalar(float g, float u);
void orc_geglu(const float* gate, const float* up, float* out, int64_t n, int threads);
/* Same with the platform libm tanhf (glibc), for the tanh-substitution study. */
float orc_geglu_scalar_libm(float g, float u);
void orc_geglu_libm(const float* gate, const float* up, float* out, int64_t n, int threads);

/* ---- Token embedding gather (model.rs:252-255, 507-508) ---- */
/* out[t,:] = dequant(table[ids[t],:]) * scale.  Returns 0, or -1 if an id >= vocab. */
int orc_embed_gather(const uint8_t* table, int64_t vocab, int64_t d, const uint32_t* ids,
                     int64_t n_ids, float scale, float* out);

/* ---- Mean pool + L2 + MRL (model.rs:654-705) ---- */
/* tokens f32 [t,d]; mask (nullable) uint8 [t]; writes out[trunc] (trunc==0 or >=d -> d). */
void orc_pool_normalize(const float* tokens, const uint8_t* mask, int64_t t, int64_t d,
                        int64_t trunc, float* out);
/* l2_normalize (util.rs:22-29): sequential f32 sum of squares, a zero norm
 * returns x unchanged.  cosine_similarity (util.rs:32-41): sequential f32
 * sums, 0 for a zero norm, clamp to [-1, 1]. */
void orc_l2_normalize(const float* x, int64_t n, float* y);
float orc_cosine(const float* a, const float* b, int64_t n);

/* ---- Synthetic inputs (seeded, shared by tests, bench and the CPU baseline) ---- */
/* Output-vector codecs (glypr-core util.rs:52-197). */
int orc_quantize_binary(const float* x, int64_t dim, uint64_t* words);
uint32_t orc_hamming(const uint64_t* a, const uint64_t* b, int64_t words);
float orc_binary_cosine(const uint64_t* a, const uint64_t* b, int64_t words);
void orc_quantize_int8(const float* x, int64_t n, int8_t* q);
int32_t orc_int8_dot(const int8_t* a, const int8_t* b, int64_t n);
float orc_int8_cosine(const int8_t* a, const int8_t* b, int64_t n);

uint64_t orc_splitmix64(uint64_t* state);
void orc_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float stddev);
void orc_fill_uniform_ids(uint32_t* ids, int64_t n, uint64_t seed, uint32_t vocab);
/* GGUF Q8_0 weight [n][k/32]: qs uniform in [-127,127], d = f16(|N(0,sigma)|/127). */
void orc_make_q8_0_weight(uint8_t* blocks, int64_t n, int64_t k, uint64_t seed, float sigma);

/* ---- Backbone (configs 4-5 run without PLE; layer.rs:20-50, ple.rs) ---- */
typedef struct {
  int64_t hidden;       /* 768 */
  int64_t ffn;          /* 1152 */
  int64_t n_heads;      /* 3 */
  int64_t n_kv_heads;   /* 1 */
  int64_t head_dim;     /* 256 */
  int64_t n_layers;     /* 24 */
  int64_t vocab;        /* 262144 */
  int64_t sliding_window; /* 512 */
  float eps;            /* 1e-6 */
  double rope_theta_sliding; /* 10000 */
  double rope_theta_full;    /* 1e6 */
  int64_t ple_dim;      /* hidden_size_per_layer_input; 0 = no PLE (configs 4-5) */
  int64_t out_dim;      /* rows of output.weight; 0 = no embedding projection */
  int64_t full_head_dim;   /* full-attention layers' head_dim (config.rs:149-166); 0 = head_dim */
  int64_t full_n_kv_heads; /* full-attention layers' kv heads (config.rs:151-157); 0 = n_kv_heads */
  const uint8_t* layer_types; /* n_layers entries, nonzero = full attention (the
                               * sliding_window_pattern of config.rs:117-140);
                               * NULL = orc_layer_is_full's default pattern */
} orc_model_config;

/* Per-layer weights, host memory.  Q8_0 tensors are GGUF blocks. */
typedef struct {
  /* head_dim / n_kv of the layer's type (TextConfig::get_head_dim /
   * get_num_kv_heads, config.rs:208-230) */
  const uint8_t* q;     /* [n_heads*head_dim][hidden] */
  const uint8_t* k;     /* [n_kv*head_dim][hidden] */
  const uint8_t* v;     /* [n_kv*head_dim][hidden] */
  const uint8_t* o;     /* [hidden][n_heads*head_dim] */
  const uint8_t* gate;  /* [ffn][hidden] */
  const uint8_t* up;    /* [ffn][hidden] */
  const uint8_t* down;  /* [hidden][ffn] */
  const float* input_norm;     /* [hidden] */
  const float* post_attn_norm; /* [hidden] */
  const float* pre_ffn_norm;   /* [hidden] */
  const float* post_ffn_norm;  /* [hidden] */
  const float* q_norm;         /* [head_dim] */
  const float* k_norm;         /* [head_dim] */
  /* TextPLEBlock (ple.rs:96-145) and the layer scalar; unused when ple_dim 0 */
  const uint8_t* ple_gate;     /* inp_gate [ple_dim][hidden] */
  const uint8_t* ple_proj;     /* proj [hidden][ple_dim] */
  const float* ple_post_norm;  /* post_norm [hidden] */
  const float* layer_scalar;   /* layer_output_scale [1] */
} orc_layer_weights;

/* The default layer_types without a sliding_window_pattern: 0 = sliding,
 * 1 = full, layer i full iff (i+1) % 6 == 0 (config.rs:131-140). */
int orc_layer_is_full(int64_t layer_idx);
/* RoPE tables (rope.rs:14-87): cos/sin f32 [t][head_dim]. */
void orc_rope_tables(int64_t head_dim, double theta, int64_t t, float* cos_t, float* sin_t);
/* One encoder layer in place on hidden [t][hidden].  per_layer_input
 * [t][ple_dim] (this layer's PLE slice) when cfg->ple_dim > 0, else NULL. */
void orc_encoder_layer(const orc_model_config* cfg, const orc_layer_weights* w, int64_t layer_idx,
                       float* hidden, const float* per_layer_input, int64_t t, int threads);
/* Full forward: gather*sqrt(hidden) -> [PLE inputs] -> layers -> final norm
 * -> [embedding projection] -> pool/L2/MRL.  final_norm [hidden];
 * ple_model_proj [n_layers*ple_dim][hidden] and ple_proj_norm [ple_dim] when
 * ple_dim > 0; out_proj [out_dim][hidden] when out_dim > 0 (else NULL).
 * out [trunc or out dim]; hidden_out [t][out dim] (the unpooled token
 * embeddings), out dim = out_dim or hidden. */
int orc_model_forward(const orc_model_config* cfg, const uint8_t* embed_table,
                      const orc_layer_weights* layers, const float* final_norm,
                      const uint8_t* ple_model_proj, const float* ple_proj_norm,
                      const uint8_t* out_proj, const uint32_t* ids, int64_t t, int64_t trunc,
                      float* out, float* hidden_out /* nullable */, int threads);
/* Attention core for one sequence (attention/standard.rs, chunked.rs):
 * q [n_heads][t][hd], k,v [n_kv][t][hd] -> ctx [t][n_heads*hd]; window 0 = full. */
void orc_attention(const float* q, const float* k, const float* v, int64_t n_heads,
                   int64_t n_kv, int64_t t, int64_t hd, int64_t window, float* ctx, int threads);

#ifdef __cplusplus
}
#endif
#endif
