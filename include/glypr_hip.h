/*
 * glypr_hip.h — C ABI of glypr's MI355X (gfx950) Q8_0 backend.
 *
 * A HIP backend beside glypr-core's Metal and CPU-SIMD backends.  The entry
 * points are what a Rust `glypr-hip-sys` crate binds from a `LinearOp::HipQ8_0`
 * arm of linear.rs.  Each declaration names the
 * reference interface it replaces (paths inside phrozen/glypr v0.3.0,
 * crates/glypr-core/src/).
 *
 * Conventions
 *  - Every entry point returns a glypr_status (0 = GLYPR_OK).  On error,
 *    glypr_hip_last_error() returns a thread-local message.
 *  - All arguments are validated on the host before anything is launched, so
 *    every error path is reachable without a GPU.
 *  - Tensors are caller-allocated device buffers, row-major and contiguous,
 *    f32 unless stated.  Q8_0 weights are library-owned opaque handles.
 *  - Launches are asynchronous on `stream` (a hipStream_t; NULL = the null
 *    stream).  A context's workspace is shared by its calls: calls on one
 *    context must be issued from one thread, and all onto one stream (work
 *    queued on a second stream could still read the workspace while a call on
 *    the first one overwrites it).  Use one context per stream.
 *  - Workspace: each weight created on a context sizes the context's activation
 *    workspace for its in_dim at glypr_hip_ctx_reserve's row count (8320 =
 *    glypr's DEFAULT_MAX_SEQ_LEN, lib.rs:47, until changed), so calls within
 *    it allocate nothing and never synchronise.  A call with more rows grows the
 *    workspace first (a device synchronisation, then hipFree / hipMalloc).
 *  - Q8_0 is the GGUF block format: 34 bytes = { f16 d; int8 qs[32] }, rows
 *    of K/32 blocks; K must be a multiple of 32.
 */
#ifndef GLYPR_HIP_H
#define GLYPR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLYPR_HIP_ABI_VERSION 8

typedef enum glypr_status {
  GLYPR_OK = 0,
  GLYPR_ERR_INVALID_ARG = 1, /* null pointer, negative or zero size */
  GLYPR_ERR_SHAPE = 2,       /* K % 32 != 0, dimension mismatch */
  GLYPR_ERR_ALIGNMENT = 3,   /* device pointer not 16-byte aligned */
  GLYPR_ERR_DEVICE = 4,      /* no HIP device, or handle from another device */
  GLYPR_ERR_HIP = 5,         /* HIP runtime error (message has the HIP error) */
  GLYPR_ERR_OOM = 6,         /* device allocation failed */
  GLYPR_ERR_RANGE = 7,       /* token id >= vocab */
  GLYPR_ERR_UNSUPPORTED = 8, /* unknown variant or flag, unsupported file layout */
  GLYPR_ERR_NOT_FOUND = 9,   /* GGUF metadata key or tensor absent */
  GLYPR_ERR_BUSY = 10        /* (ABI >= 7) the no-allocation scratch is in use by a
                                pending call on another stream */
} glypr_status;

/* Numerics of the Q8_0 GEMM.
 * INT8_EXACT: activations quantized per 32-block exactly as candle's
 *   BlockQ8_0::from_float, int8 MFMA block sums, and the scalar vec_dot's
 *   f32 sequence sum += ((float)isum * d_w) * d_x in block order: the output
 *   is bit-identical to glypr's CPU QMatMul path on x86-64.
 * BF16_DEQUANT: weights dequantized in registers to bf16(q*d), activations
 *   rounded to bf16, bf16 MFMA with f32 accumulation (the semantics of
 *   glypr's Metal kernels / CANDLE_DEQUANTIZE_ALL, at bf16 precision).
 * INT8_FMA (ABI >= 7): INT8_EXACT's operands and block sums, with each
 *   block's term added as sum = fma((float)isum * d_w, d_x, sum): one
 *   rounding fewer per block than the vec_dot sequence, so not bit-identical
 *   to it (within 1e-3 relative / 1e-4 absolute; measured to ~1e-6 relative),
 *   and 2 instead of 3 vector ops per output and block, the bound of the
 *   int8 GEMM at large M.  The model driver uses INT8_EXACT unless
 *   glypr_hip_model_set_variant (ABI >= 8) selects INT8_FMA. */
typedef enum glypr_q8_variant {
  GLYPR_Q8_INT8_EXACT = 0,
  GLYPR_Q8_BF16_DEQUANT = 1,
  GLYPR_Q8_INT8_FMA = 2
} glypr_q8_variant;

typedef struct glypr_hip_ctx glypr_hip_ctx; /* per-device context + workspace */
typedef struct glypr_q8w glypr_q8w;         /* Q8_0 weight on one device */
typedef struct glypr_bf16w glypr_bf16w;     /* dense bf16 weight on one device */
typedef void* glypr_stream;                 /* hipStream_t */

/* ---- library / context ------------------------------------------------- */

/* Thread-local description of the last error on this thread ("" if none). */
const char* glypr_hip_last_error(void);
int glypr_hip_abi_version(void);

/* Per-device state: replaces candle's per-device Metal pipeline/library
 * caches keyed by device (metal_kernels/mod.rs:15-114). */
int glypr_hip_ctx_create(int device, glypr_hip_ctx** out);
int glypr_hip_ctx_destroy(glypr_hip_ctx* ctx);

/* Block until `stream` is idle: the read-back synchronisation of
 * encode_single_text (lib.rs:988-989). */
int glypr_hip_sync(glypr_hip_ctx* ctx, glypr_stream stream);

/* Row count the workspace is sized for (the max_seq_len of GlyprEmbedder,
 * lib.rs:47, 267-274, times the batch a caller runs).  Grows the workspace
 * now for the weights created so far; weights created later are sized for
 * it too.  rows <= 0 -> GLYPR_ERR_SHAPE. */
int glypr_hip_ctx_reserve(glypr_hip_ctx* ctx, int64_t rows);

/* ---- Q8_0 weights (LinearOp load path) --------------------------------- */

/* LinearOp::from_gguf_tensor, Q8_0 arm (linear.rs:36-78; the Metal arm keeps
 * the raw bytes [N, K/32*34], linear.rs:55-71).  `gguf_blocks` is host memory
 * holding n*(k/32) GGUF Q8_0 blocks.  The weight is uploaded and repacked once
 * into an int8 plane [n][k] plus an f32 scale plane [n][k/32] (f32 of the f16
 * d, exact).  K % 32 != 0 -> GLYPR_ERR_SHAPE (the caller falls back to its CPU
 * QMatMul exactly as linear.rs:57-60 does for Metal). */
int glypr_hip_q8_0_weight_create(glypr_hip_ctx* ctx, const uint8_t* gguf_blocks, int64_t n,
                                 int64_t k, glypr_q8w** out);

/* LinearOp::try_concat (linear.rs:82-148): concatenate `count` >= 2 weights
 * with equal K along out_dim into one buffer.  If `views` is non-NULL it
 * receives `count` handles that are narrow views of the fused buffer (the
 * zero-copy views of linear.rs:128-137).  Differing K -> GLYPR_ERR_SHAPE
 * (try_concat returns None). */
int glypr_hip_q8_0_weight_concat(glypr_hip_ctx* ctx, const glypr_q8w* const* parts, int count,
                                 glypr_q8w** fused, glypr_q8w** views);

/* Tensor::narrow(0, row0, rows) of a weight: a view sharing the buffer. */
int glypr_hip_q8_0_weight_view(const glypr_q8w* w, int64_t row0, int64_t rows, glypr_q8w** out);

/* Release a handle; the buffer is freed with its last handle. */
int glypr_hip_q8_0_weight_destroy(glypr_q8w* w);

/* (out_dim, in_dim) of a handle: the fields of LinearOp::MetalQ8_0 (linear.rs:10-14). */
int glypr_hip_q8_0_weight_shape(const glypr_q8w* w, int64_t* n, int64_t* k);

/* QTensor::dequantize (model.rs:252-254; BlockQ8_0::to_float): out f32 [n,k],
 * out[r][j] = f32(d) * q, bit-exact. */
int glypr_hip_q8_0_dequantize(glypr_hip_ctx* ctx, const glypr_q8w* w, float* out,
                              glypr_stream stream);

/* ---- dense bf16 weights (LinearOp over an F16/BF16 tensor) ------------ */

/* LinearOp::from_gguf_tensor, dense arm (linear.rs:48-54: F32/F16/BF16
 * tensors become a plain Linear; on Metal the model dtype is BF16,
 * lib.rs:222-229).  `bf16_rows` is host memory, n rows of k bf16 values (the
 * GGUF (out_dim, in_dim) layout).  k % 64 != 0 -> GLYPR_ERR_UNSUPPORTED. */
int glypr_hip_bf16_weight_create(glypr_hip_ctx* ctx, const uint16_t* bf16_rows, int64_t n,
                                 int64_t k, glypr_bf16w** out);
int glypr_hip_bf16_weight_destroy(glypr_bf16w* w);

/* LinearOp::forward (linear.rs:150-172) for a dense bf16 weight: x f32 [m,k]
 * rounded to bf16 (nearest even), y f32 [m,n] = x . w^T on bf16 MFMA with f32
 * accumulation. */
int glypr_hip_bf16_matmul(glypr_hip_ctx* ctx, const glypr_bf16w* w, const float* x, float* y,
                          int64_t m, glypr_stream stream);

/* ---- Q8_0 activations --------------------------------------------------- */

/* BlockQ8_0::from_float as k_quants::matmul applies it to activations
 * (reached from linear.rs:153-162): x f32 [m,k] -> GGUF blocks [m][k/32]
 * (34 B each) in device memory, bit-exact with the CPU path. */
int glypr_hip_q8_0_quantize(glypr_hip_ctx* ctx, const float* x, int64_t m, int64_t k,
                            uint8_t* out_blocks, glypr_stream stream);

/* ---- the hot path ------------------------------------------------------ */

/* LinearOp::forward (linear.rs:150-172) -> QMatMul::forward on CPU, or
 * fused_metal_q8_0_matmul(weight, x, out_dim, in_dim) on Metal
 * (metal_kernels/mod.rs:1271-1394).  x [m,k], y [m,n]. */
int glypr_hip_q8_0_matmul(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x, float* y,
                          int64_t m, int variant, glypr_stream stream);

/* No counterpart in the reference: glypr_hip_q8_0_matmul for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, kernels and bits
 * as glypr_hip_q8_0_matmul, but the activation operand (Q8_0 or bf16 copy of
 * x) lives in a file-scope device array of GLYPR_NOALLOC_SCRATCH_BYTES that
 * each device holds until the process ends; the call allocates nothing.
 * Calls whose operand needs more (INT8_EXACT: m*k + 4*m*k/32 bytes, rounded
 * up to 256 each; BF16_DEQUANT: 2*m*k) fail with GLYPR_ERR_SHAPE.  Every call
 * on a device shares that device's array, across contexts: calls on one
 * stream are ordered, but calls that overlap on one device (other streams,
 * other threads) would race.  (ABI >= 7) The library records an event after
 * each call on a device; a call on another stream while the previous call's
 * event is still pending fails with GLYPR_ERR_BUSY and launches nothing (wait
 * for the earlier stream, or order the streams, and call again).  Calls on a
 * stream under HIP graph capture are not checked and not recorded: their
 * replays must not overlap other calls on the device. */
#define GLYPR_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int glypr_hip_q8_0_matmul_noalloc(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x,
                                  float* y, int64_t m, int variant, glypr_stream stream);

/* RMSNorm::forward (norm.rs:22-63) -> cpu_rmsnorm (cpu_simd/mod.rs:10-32;
 * simd_rmsnorm_row_f32, cpu_simd/rmsnorm.rs:6-47).  weight may be NULL (the
 * weightless v_norm).  x,y [rows,dim]; x == y allowed. */
int glypr_hip_rmsnorm(glypr_hip_ctx* ctx, const float* x, const float* weight, float eps,
                      float* y, int64_t rows, int64_t dim, glypr_stream stream);

/* RMSNorm::forward feeding LinearOp::forward (layer.rs:30-31, 38-39): the
 * RMSNorm prologue fused with activation quantization; the normalised f32
 * tensor is never written.  x [m,k] (k = norm dim), y [m,n]. */
int glypr_hip_rmsnorm_q8_0_matmul(glypr_hip_ctx* ctx, const glypr_q8w* w, const float* x,
                                  const float* norm_weight, float eps, float* y, int64_t m,
                                  int variant, glypr_stream stream);

/* cpu_geglu (cpu_simd/mod.rs:35-47; geglu_scalar_f32, cpu_simd/geglu.rs:6-18):
 * out = gelu_tanh(gate) * up, elementwise over n floats; out may alias. */
int glypr_hip_geglu(glypr_hip_ctx* ctx, const float* gate, const float* up, float* out,
                    int64_t n, glypr_stream stream);

/* MLP::forward (mlp.rs:31-70): gate/up GEMM with the GeGLU applied in its
 * epilogue (and the result quantized there for `down`), then down.
 * gate_up: the try_concat of [gate; up] ([2F, H]); down: [H, F].
 * x [m,H] is the (already normalised) input; y [m,H]. */
int glypr_hip_mlp(glypr_hip_ctx* ctx, const glypr_q8w* gate_up, const glypr_q8w* down,
                  const float* x, float* y, int64_t m, int variant, glypr_stream stream);

/* pre_feedforward_layernorm + MLP::forward (layer.rs:37-39): the same with
 * the RMSNorm prologue fused into the gate/up GEMM's activation quantizer. */
int glypr_hip_rmsnorm_mlp(glypr_hip_ctx* ctx, const glypr_q8w* gate_up, const glypr_q8w* down,
                          const float* x, const float* norm_weight, float eps, float* y,
                          int64_t m, int variant, glypr_stream stream);

/* Embedding::forward + x embed_scale (model.rs:254-255, 507-508): rows of a
 * Q8_0 token table gathered and dequantized directly from the int8 plane,
 * out[t,:] = (f32(d)*q) * scale.  `ids` is host memory (tokenizer output);
 * any id >= vocab -> GLYPR_ERR_RANGE before launch.  out [n_ids, k]. */
int glypr_hip_q8_0_embed_gather(glypr_hip_ctx* ctx, const glypr_q8w* table, const uint32_t* ids,
                                int64_t n_ids, float scale, float* out, glypr_stream stream);

/* pool_and_normalize (model.rs:654-705) with truncate_mrl semantics
 * (util.rs:6-19): mean over valid tokens (mask NULL = all; else host uint8
 * [t]), L2 with the 1e-12 clamp, then MRL truncation to `trunc` dims and
 * renormalisation (trunc 0 or >= d keeps d).  tokens [t,d] -> out [trunc]. */
int glypr_hip_pool_normalize(glypr_hip_ctx* ctx, const float* tokens, const uint8_t* mask,
                             int64_t t, int64_t d, int64_t trunc, float* out,
                             glypr_stream stream);

/* ---- output-vector codecs (serving) --------------------------------------- */

/* quantize_binary (util.rs:52-71): bit i of word i/64 is x[i] > 0 (NaN -> 0).
 * x [n][dim] f32 -> out [n][dim/64] u64.  dim % 64 != 0 -> GLYPR_ERR_SHAPE
 * (the reference's bail). */
int glypr_hip_quantize_binary(glypr_hip_ctx* ctx, const float* x, int64_t n, int64_t dim,
                              uint64_t* out, glypr_stream stream);
/* quantize_int8 (util.rs:128-133): (x * 127).round().clamp(-127, 127) as i8,
 * round half away from zero, NaN -> 0.  x [count] -> out [count]. */
int glypr_hip_quantize_int8(glypr_hip_ctx* ctx, const float* x, int64_t count, int8_t* out,
                            glypr_stream stream);
/* hamming_distance (util.rs:75-109) between every pair: out[i][j] =
 * popcount(a_i XOR b_j) over `words` u64 words.  a [na][words],
 * b [nb][words] -> out [na][nb] u32. */
int glypr_hip_hamming(glypr_hip_ctx* ctx, const uint64_t* a, int64_t na, const uint64_t* b,
                      int64_t nb, int64_t words, uint32_t* out, glypr_stream stream);
/* binary_cosine_similarity (util.rs:112-119) between every pair:
 * cos(PI * (h as f32 / dim as f32)) in f32 with dim = 64 words, evaluated by
 * the host libm's cosf once per h (a table per dim); words 0 -> 1.0.
 * -> out [na][nb] f32. */
int glypr_hip_binary_cosine(glypr_hip_ctx* ctx, const uint64_t* a, int64_t na,
                            const uint64_t* b, int64_t nb, int64_t words, float* out,
                            glypr_stream stream);
/* int8_dot_product (util.rs:137-176) between every pair, exact i32 on int8
 * MFMA.  a [na][dim], b [nb][dim] -> out [na][nb].  dim <= 65536. */
int glypr_hip_int8_dot(glypr_hip_ctx* ctx, const int8_t* a, int64_t na, const int8_t* b,
                       int64_t nb, int64_t dim, int32_t* out, glypr_stream stream);
/* int8_cosine_similarity (util.rs:181-197) between every pair:
 * dot / (sqrt(|a|^2) * sqrt(|b|^2)) in f32, clamped to [-1, 1]; 0 when either
 * squared norm is 0.  -> out [na][nb] f32.  dim <= 65536. */
int glypr_hip_int8_cosine(glypr_hip_ctx* ctx, const int8_t* a, int64_t na, const int8_t* b,
                          int64_t nb, int64_t dim, float* out, glypr_stream stream);

/* ---- attention core ------------------------------------------------------ */

/* SelfAttention::forward between the projections and o_proj
 * (attention/mod.rs:166-273): per-head q_norm / k_norm / weightless v_norm
 * (RMSNorm over head_dim, bit-exact with the CPU path), RoPE with the caller's
 * cos/sin tables (rope.rs:99-106; [t][head_dim] f32 device arrays as
 * RotaryEmbedding::get_cos_sin returns them), repeat_kv, and attention with
 * scale 1.0 and f32 softmax (attention/standard.rs:10-83); window > 0 and
 * t > window applies the sliding band |i - j| <= window (attention/chunked.rs).
 * qkv [t][(n_heads + 2*n_kv_heads) * head_dim] (q | k | v columns, the fused
 * projection's output) -> ctx [t][n_heads * head_dim].  head_dim must be 256. */
int glypr_hip_attention(glypr_hip_ctx* ctx, const float* qkv, const float* q_norm_weight,
                        const float* k_norm_weight, float eps, const float* cos_table,
                        const float* sin_table, int64_t t, int64_t n_heads, int64_t n_kv_heads,
                        int64_t head_dim, int64_t window, float* ctx_out, glypr_stream stream);

/* ---- text backbone (configs 4-5) ---------------------------------------- */

/* EmbeddingGemma layer geometry (TextConfig, config.rs:76-213; BASELINE uses
 * hidden 768, ffn 1152, 3 q heads / 1 kv head, head_dim 256, 24 layers; the
 * released EmbeddingGemma-2 has hidden 512, ffn 2048, 4 q heads, sliding
 * layers 2 kv heads of 256, full layers 1 kv head of 512). */
typedef struct glypr_model_config {
  int64_t hidden;
  int64_t ffn;
  int64_t n_heads;
  int64_t n_kv_heads;
  int64_t head_dim;
  int64_t n_layers;
  int64_t vocab;
  int64_t sliding_window;      /* 512 (config.rs:191) */
  float eps;                   /* rms_norm_eps, 1e-6 */
  double rope_theta_sliding;   /* 10000 (config.rs:171-172) */
  double rope_theta_full;      /* 1e6 (config.rs:173-174) */
  int64_t ple_dim;             /* hidden_size_per_layer_input (config.rs:100-101);
                                * 0 = no Per-Layer-Embedding block (configs 4-5) */
  int64_t out_dim;             /* rows of output.weight, the embedding projection
                                * (model.rs:472-473, 577); 0 = none */
  int64_t full_head_dim;       /* head_dim of the full-attention layers
                                * (attention.key_length, config.rs:149-150,
                                * 158-166); 0 = head_dim */
  int64_t full_n_kv_heads;     /* kv heads of the full-attention layers
                                * (head_count_kv[i], config.rs:151-157); 0 =
                                * n_kv_heads */
  int64_t max_seq_len;         /* longest sequence model_embed accepts
                                * (GlyprEmbedder::max_seq_len, lib.rs:47, 425);
                                * every activation buffer is sized for it at
                                * finalize; 0 = 8320 */
  int64_t max_batch_tokens;    /* padded rows one glypr_hip_model_embed_batch
                                * call may take (each sequence rounded up to 64);
                                * buffers are sized for max(max_seq_len, this) */
  const uint8_t* layer_types;  /* nullable: n_layers entries, nonzero = a
                                * full-attention layer, 0 = sliding (the
                                * layer_types TextConfig builds from
                                * sliding_window_pattern, config.rs:117-140);
                                * read at create, not kept.  NULL = the default
                                * pattern, layer i full iff (i+1) % 6 == 0 */
} glypr_model_config;

typedef struct glypr_model glypr_model;

/* EmbeddingGemma2Model::from_gguf_content (model.rs:244-488): an empty model
 * whose tensors arrive through glypr_hip_model_set_tensor.  Layer i is full
 * attention as cfg->layer_types says, or iff (i+1) % 6 == 0 without it
 * (config.rs:117-140), sliding otherwise.  With
 * ple_dim > 0 (a multiple of 32) every layer ends with the TextPLEBlock and its
 * layer scalar (layer.rs:45-49); with out_dim > 0 the final norm feeds the
 * embedding projection. */
int glypr_hip_model_create(glypr_hip_ctx* ctx, const glypr_model_config* cfg,
                           glypr_model** out);

/* One GGUF tensor by its glypr name (model.rs:252-470): "token_embd.weight",
 * "output_norm.weight", "blk.{i}.{attn_norm, post_attention_norm, ffn_norm,
 * post_ffw_norm, attn_q_norm, attn_k_norm}.weight" (f32, dtype 0) and
 * "blk.{i}.{attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up,
 * ffn_down}.weight" (Q8_0 GGUF blocks, dtype 1, or dense bf16 rows, dtype 2 (the
 * F16/BF16 arm of linear.rs:48-54); all seven projections of every layer share
 * one kind, and dense ones need hidden, ffn % 64 == 0, ple_dim == 0 and
 * out_dim == 0).  With ple_dim > 0 also
 * "per_layer_model_proj.weight" (Q8_0, n_layers*ple_dim x hidden),
 * "per_layer_proj_norm.weight" (f32 [ple_dim]) and per layer "inp_gate"
 * (Q8_0, ple_dim x hidden), "proj" (Q8_0, hidden x ple_dim), "post_norm"
 * (f32 [hidden]) and "layer_output_scale" (f32 [1]); with out_dim > 0
 * "output.weight" (Q8_0, out_dim x hidden).  Host memory; rows x cols is the
 * GGUF (out_dim, in_dim). */
int glypr_hip_model_set_tensor(glypr_model* model, const char* name, const void* data,
                               int64_t rows, int64_t cols, int dtype);

/* Check every tensor is present and build the fused q|k|v and gate|up
 * weights (SelfAttention::new / MLP::new via try_concat). */
int glypr_hip_model_finalize(glypr_model* model);

/* forward (model.rs:498-578) + pool_and_normalize (model.rs:654-705) for one
 * sequence: ids (host, tokenizer output) -> out [trunc, or the embedding
 * width when trunc is 0 or wider] on the device.  hidden (nullable, device
 * [t][width]) receives the unpooled token embeddings: the projection's output,
 * or the final-normed states without one.  The embedding width is out_dim
 * when set, else hidden.  Q8_0 projections run as INT8_EXACT (or INT8_FMA,
 * see glypr_hip_model_set_variant); dense bf16 ones take bf16 activations
 * (nearest even) with f32 accumulation. */
int glypr_hip_model_embed(glypr_model* model, const uint32_t* ids, int64_t t, int64_t trunc,
                          float* out, float* hidden, glypr_stream stream);

/* embed_batch_inner (lib.rs:752-952) for text: n_seqs sequences of lens[i]
 * tokens (ids concatenated, host memory) in one forward pass.  Each sequence's
 * embedding is the one the reference computes from its padded batch (pad
 * keys masked out of attention, pads left out of the mean, model.rs:580-705),
 * which is the sequence's own single-sequence embedding: pooled by the mean
 * (sum times 1/len) when all lengths are equal and by the masked sum divided
 * by the token count when they differ, as the reference (lib.rs:902-941); the
 * pooling sum runs in chunks, so it matches the reference's to rounding
 * (float64 bound 1e-6 of the largest value), not bit for bit.  The sequences sit at
 * 64-aligned row offsets, so every projection runs once over all of their rows
 * and attention and pooling stay within each sequence.  out [n_seqs][trunc,
 * or the embedding width].  Each len must be in [1, max_seq_len] (the
 * preflight of lib.rs:838-845) and the padded total <= max(max_seq_len,
 * max_batch_tokens) (GLYPR_ERR_SHAPE otherwise). */
int glypr_hip_model_embed_batch(glypr_model* model, const uint32_t* ids, const int64_t* lens,
                                int64_t n_seqs, int64_t trunc, float* out, glypr_stream stream);

/* (ABI >= 8) No counterpart in the reference, whose CPU path has one
 * numerics (vec_dot, linear.rs:153-162): the block epilogue of every Q8_0
 * projection of the model's later embed calls, GLYPR_Q8_INT8_EXACT (the
 * default, bit-identical to vec_dot) or GLYPR_Q8_INT8_FMA (one rounding fewer
 * per block, within 1e-3 relative / 1e-4 absolute of it, and 2 instead of 3
 * vector ops per output and block).  For callers that trade bit-identity for
 * throughput within the reference's stated tolerance.  Dense bf16 projections
 * are unaffected.  Any other variant -> GLYPR_ERR_UNSUPPORTED. */
int glypr_hip_model_set_variant(glypr_model* model, int variant);

int glypr_hip_model_destroy(glypr_model* model);

/* ---- GGUF v3 files ------------------------------------------------------ */

/* gguf_file::Content::read as glypr calls it (lib.rs:180-186, model.rs:235):
 * memory-map and parse a GGUF (v2/v3) file.  Header, metadata and tensor table
 * are validated with bounds checks (GLYPR_ERR_SHAPE on a truncated or corrupt
 * file, GLYPR_ERR_UNSUPPORTED on another version).  Host only: no device is
 * touched. */
typedef struct glypr_gguf glypr_gguf;
int glypr_gguf_open(const char* path, glypr_gguf** out);
int glypr_gguf_close(glypr_gguf* g);
int glypr_gguf_version(const glypr_gguf* g, uint32_t* version, uint32_t* alignment);
/* Content::tensor_infos: name, ggml type (0 = F32, 8 = Q8_0, ...), dims ne[0..3]
 * (ne[0] innermost; unused dims are 1), the mapped bytes and their size
 * (nbytes = -1, data = NULL for a ggml type this reader does not size). */
int glypr_gguf_tensor_count(const glypr_gguf* g, int64_t* n);
int glypr_gguf_tensor_info(const glypr_gguf* g, int64_t i, const char** name, int* type,
                           int* n_dims, int64_t* ne, const void** data, int64_t* nbytes);
int glypr_gguf_find_tensor(const glypr_gguf* g, const char* name, int64_t* index);
/* Content::metadata lookups (the get_u32 / get_f64 helpers of config.rs:9-40):
 * integer and bool values as u64, numbers as f64; GLYPR_ERR_NOT_FOUND if the
 * key is absent, GLYPR_ERR_UNSUPPORTED if it has another type. */
int glypr_gguf_get_u64(const glypr_gguf* g, const char* key, uint64_t* out);
int glypr_gguf_get_f64(const glypr_gguf* g, const char* key, double* out);
int glypr_gguf_get_str(const glypr_gguf* g, const char* key, const char** out);
int glypr_gguf_get_array(const glypr_gguf* g, const char* key, int* elem_type, int64_t* len);
int glypr_gguf_get_array_u64(const glypr_gguf* g, const char* key, int64_t i, uint64_t* out);

/* GlyprEmbedder::load_gguf_q8 -> EmbeddingGemma2Model::from_gguf_content
 * (lib.rs:180-186; model.rs:244-488) with TextConfig::from_gguf_metadata
 * (config.rs:79-189): the config from the gemma-embedding2.* keys, then every
 * tensor glypr_hip_model_set_tensor names, then finalize.  A file with
 * "per_layer_model_proj.weight" runs the Per-Layer-Embedding path (ple_dim from
 * gemma-embedding2.embedding_length_per_layer_input), one with
 * "output.weight" the embedding projection.  Layouts the backend does not run
 * (a layer pattern other than 5 sliding + 1 full, per-layer kv heads or head
 * dims, tensors in other ggml types) give GLYPR_ERR_UNSUPPORTED. */
int glypr_hip_model_load_gguf(glypr_hip_ctx* ctx, const char* path, glypr_model** out);

/* ---- per-kernel timing --------------------------------------------------- */

/* Kernel identities for the per-kernel timing below. */
typedef enum glypr_kernel_id {
  GLYPR_K_QUANTIZE = 0,       /* activation quantize (BlockQ8_0::from_float) */
  GLYPR_K_RMSNORM_QUANT = 1,  /* RMSNorm prologue emitting Q8_0 activations */
  GLYPR_K_GEMM_I8 = 2,        /* INT8_EXACT GEMM */
  GLYPR_K_GEMM_I8_GEGLU = 3,  /* INT8_EXACT gate/up GEMM + GeGLU + quantize epilogue */
  GLYPR_K_TO_BF16 = 4,        /* f32 -> bf16 activations */
  GLYPR_K_RMSNORM_BF16 = 5,   /* RMSNorm prologue emitting bf16 activations */
  GLYPR_K_GEMM_BF16 = 6,      /* BF16_DEQUANT GEMM */
  GLYPR_K_GEMM_BF16_GEGLU = 7,/* BF16_DEQUANT gate/up GEMM + GeGLU epilogue */
  GLYPR_K_RMSNORM = 8,
  GLYPR_K_GEGLU = 9,
  GLYPR_K_GATHER = 10,
  GLYPR_K_DEQUANT = 11,
  GLYPR_K_POOL = 12,
  GLYPR_K_QKV_POST = 13,      /* q/k/v norms + RoPE + f16 split */
  GLYPR_K_ATTENTION = 14,     /* flash attention */
  GLYPR_K_RESIDUAL_NORM = 15, /* residual + RMSNorm (+ next prologue) */
  GLYPR_K_VEC_ENCODE = 16,    /* binary / int8 output-vector quantization */
  GLYPR_K_VEC_SEARCH = 17,    /* all-pairs hamming / cosine over encoded vectors */
  GLYPR_K_GEMM_I8_PRO = 18,   /* INT8_EXACT GEMM with the quantize / RMSNorm prologue fused */
  GLYPR_K_GEMM_BF16W = 19,    /* GEMM on dense bf16 weights (+ GeGLU epilogue) */
  GLYPR_K_GEMM_I8_QKV = 20,   /* INT8_EXACT q|k|v GEMM with the q/k/v norms + RoPE epilogue */
  GLYPR_K_COUNT = 21
} glypr_kernel_id;

/* The per-op device timing of forward_profiled (profile.rs:53-56, 63-429),
 * without its host syncs: while enabled, every kernel the context launches is
 * bracketed by HIP events on its own stream.  Enabling clears the totals. */
int glypr_hip_profile_enable(glypr_hip_ctx* ctx, int enable);
/* Wait for the recorded events and return, per glypr_kernel_id, the summed
 * duration in milliseconds and the launch count (arrays of GLYPR_K_COUNT). */
int glypr_hip_profile_read(glypr_hip_ctx* ctx, double* total_ms, int64_t* launches);
/* Static name of a glypr_kernel_id ("" if out of range). */
const char* glypr_hip_kernel_name(int id);

#ifdef __cplusplus
}
#endif
#endif /* GLYPR_HIP_H */
