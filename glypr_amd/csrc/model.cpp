// model.cpp — host-side mirror of glypr's text backbone over the HIP kernels.
//
// Class names follow the reference modules they replace:
//   LinearOp            linear.rs:5-172        (a Q8_0 weight handle + forward)
//   RMSNorm             norm.rs:4-95           (device f32 weight + eps)
//   SelfAttention       attention/mod.rs:33-277
//   MLP                 mlp.rs:6-70
//   EncoderLayer        layer.rs:8-50          (PLE block + layer scalar when ple_dim > 0)
//   TextPLE/TextPLEBlock ple.rs:20-145
//   EmbeddingGemma2Model model.rs:244-705      (gather, PLE inputs, layers, final norm,
//                                               embedding projection, pooling)
// The forward pass runs every projection as an INT8_EXACT Q8_0 GEMM (INT8_FMA
// after glypr_hip_model_set_variant) and fuses what the reference computes in
// separate ops:
//   - each RMSNorm that feeds a projection is the GEMM's quantizing prologue;
//   - forward_residual_add of one sublayer and the next sublayer's input
//     RMSNorm are one kernel (residual_norm);
//   - q/k/v and gate/up are single fused GEMMs (try_concat, linear.rs:82-148);
//   - GeGLU is the gate/up GEMM's epilogue;
//   - the PLE block's geglu(gate, per-layer input) is fused with the Q8_0
//     quantization of the proj GEMM's operand, and its forward_residual_add
//     with the layer scalar feeds the next layer's input norm.
// The GEMMs (INT8_EXACT), norms, GeGLU and residual adds are bit-exact with
// the CPU path; attention (f16 MFMA with split operands, see k_attn.hip) and the chunked
// pooling sum differ from it at f32-rounding level.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <string>
#include <vector>

#include "host_common.hpp"
#include "internal.hpp"

using namespace glypr;

namespace glypr {
namespace host {

struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  int ensure(size_t bytes) {
    if (bytes <= cap) return GLYPR_OK;
    if (p) {
      GLYPR_TRY_HIP(hipDeviceSynchronize(), "buffer growth: hipDeviceSynchronize");
      GLYPR_TRY_HIP(hipFree(p), "buffer growth: hipFree");
      p = nullptr;
      cap = 0;
    }
    size_t c = align_up(bytes, 1 << 16);
    GLYPR_TRY_HIP(hipMalloc(&p, c), "buffer: hipMalloc");
    cap = c;
    return GLYPR_OK;
  }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
  }
  template <typename T>
  T* as() const { return reinterpret_cast<T*>(p); }
};

struct LinearOp {
  glypr_q8w* w = nullptr;     // Q8_0 weight
  glypr_bf16w* wb = nullptr;  // or a dense bf16 weight (F16/BF16 GGUF tensors)
};

struct RMSNorm {
  float* weight = nullptr;  // device, nullptr = weightless
};

struct SelfAttention {
  LinearOp q, k, v, o;
  LinearOp fused_qkv;  // try_concat([q, k, v])
  RMSNorm q_norm, k_norm;
};

struct MLP {
  LinearOp gate, up, down;
  LinearOp fused_gate_up;  // try_concat([gate, up])
};

// TextPLEBlock (ple.rs:96-145) + the layer scalar (layer.rs:16, 45-49).
struct PLEBlock {
  LinearOp gate;        // inp_gate [ple_dim][hidden]
  LinearOp projection;  // proj [hidden][ple_dim]
  RMSNorm norm;         // post_norm [hidden]
  float* layer_scalar = nullptr;  // device, 1 value
};

struct EncoderLayer {
  SelfAttention self_attn;
  MLP mlp;
  RMSNorm input_layernorm, post_attention_layernorm, pre_feedforward_layernorm,
      post_feedforward_layernorm;
  PLEBlock ple_block;
  bool full_attention = false;
  // the layer's attention geometry (TextConfig::get_head_dim /
  // get_num_kv_heads, config.rs:142-169)
  int64_t head_dim = 0, n_kv_heads = 0;
};

}  // namespace host
}  // namespace glypr

using namespace glypr::host;

struct glypr_model {
  glypr_hip_ctx* ctx = nullptr;
  glypr_model_config cfg{};
  LinearOp token_embd;
  std::vector<EncoderLayer> layers;
  RMSNorm norm;  // output_norm
  // TextPLE (ple.rs:20-85): per_layer_model_proj + per_layer_proj_norm
  LinearOp ple_projection;
  RMSNorm ple_norm;
  LinearOp embedding_projection;  // output.weight
  bool finalized = false;
  bool dense = false;  // projections are dense bf16 weights (activations run in bf16)
  // the Q8_0 projections' block epilogue: false = INT8_EXACT (vec_dot's
  // three roundings per block), true = INT8_FMA (glypr_hip_model_set_variant)
  bool fma2 = false;
  // RoPE tables [max_seq_len][head_dim] of the sliding and full layer types
  // (rope_sliding / rope_full, model.rs:278-279).
  DevBuf cos_s, sin_s, cos_f, sin_f;
  int64_t rope_cap = 0;
  // activations
  DevBuf h, xq, dx, qkv, attn_q, attn_k, attn_vt, attn_scratch, cq, dc, proj, hq,
      dh, normed, pooled, ids, ple, ple_gate, tokens, xb, hb;
  // several sequences in one forward: the per-row segment table ({start,
  // length} of the row's sequence, int32 pairs) and {offset, length} per
  // sequence; host staging of both and of the padded ids
  DevBuf seg, seqs;
  std::vector<int32_t> h_seg, h_seqs;
  std::vector<uint32_t> h_ids;
  int64_t cap_t = 0;   // rows every buffer holds: max(max_seq_len, max_batch_tokens), 64-aligned
};

namespace {

inline float* dev_f32(const DevBuf& b) { return b.as<float>(); }

// RotaryEmbedding::new + get_cos_sin (rope.rs:14-87): inv_freq computed in f64
// and cast to f32; positions as f32; freqs = pos * inv_freq in f32;
// emb = cat(freqs, freqs); cos/sin in f32.
void rope_table(int64_t hd, double theta, int64_t t, std::vector<float>& c, std::vector<float>& s) {
  const int64_t half = hd / 2;
  std::vector<float> inv(half);
  for (int64_t i = 0; i < half; i++)
    inv[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)hd));
  c.resize(t * hd);
  s.resize(t * hd);
  for (int64_t p = 0; p < t; p++)
    for (int64_t i = 0; i < hd; i++) {
      float f = (float)p * inv[i % half];
      c[p * hd + i] = cosf(f);
      s[p * hd + i] = sinf(f);
    }
}

int upload_f32(const float* host, int64_t n, float** dev) {
  GLYPR_TRY_HIP(hipMalloc((void**)dev, (size_t)n * sizeof(float)), "norm weight: hipMalloc");
  GLYPR_TRY_HIP(hipMemcpy(*dev, host, (size_t)n * sizeof(float), hipMemcpyHostToDevice),
                "norm weight: upload");
  return GLYPR_OK;
}

int ensure_rope(glypr_model* m, int64_t t) {
  if (t <= m->rope_cap) return GLYPR_OK;
  const int64_t cap = t;
  std::vector<float> c, s;
  const int64_t hds = m->cfg.head_dim, hdf = m->cfg.full_head_dim;
  const size_t bs = (size_t)(cap * hds) * sizeof(float), bf = (size_t)(cap * hdf) * sizeof(float);
  RET_IF(m->cos_s.ensure(bs));
  RET_IF(m->sin_s.ensure(bs));
  RET_IF(m->cos_f.ensure(bf));
  RET_IF(m->sin_f.ensure(bf));
  rope_table(hds, m->cfg.rope_theta_sliding, cap, c, s);
  GLYPR_TRY_HIP(hipMemcpy(m->cos_s.p, c.data(), bs, hipMemcpyHostToDevice), "rope upload");
  GLYPR_TRY_HIP(hipMemcpy(m->sin_s.p, s.data(), bs, hipMemcpyHostToDevice), "rope upload");
  rope_table(hdf, m->cfg.rope_theta_full, cap, c, s);
  GLYPR_TRY_HIP(hipMemcpy(m->cos_f.p, c.data(), bf, hipMemcpyHostToDevice), "rope upload");
  GLYPR_TRY_HIP(hipMemcpy(m->sin_f.p, s.data(), bf, hipMemcpyHostToDevice), "rope upload");
  m->rope_cap = cap;
  return GLYPR_OK;
}

// Attention scratch for the largest case the model can meet: any (longest)
// sequence length up to max_seq_len with any padded row count up to the
// capacity, for each layer geometry (attention_scratch_bound).
size_t model_attention_scratch(const glypr_model* m, int64_t cap) {
  const glypr_model_config& c = m->cfg;
  size_t best = 0;
  for (int full = 0; full < 2; full++) {
    const int64_t hd = full ? c.full_head_dim : c.head_dim;
    const int64_t nkv = full ? c.full_n_kv_heads : c.n_kv_heads;
    const int64_t w = full ? 0 : c.sliding_window;
    const size_t sc = attention_scratch_bound(c.max_seq_len, cap, c.n_heads, nkv, hd, w);
    best = sc > best ? sc : best;
  }
  return best;
}

// Every activation buffer for `t` rows (a 64-aligned capacity).
int ensure_activations(glypr_model* m, int64_t t) {
  if (t <= m->cap_t) return GLYPR_OK;
  const glypr_model_config& c = m->cfg;
  const int64_t tp = attn_padded_len(t);
  // the widest attention geometry over the layers
  int64_t qd = 0, kvd = 0, qkvd = 0;
  for (const EncoderLayer& L : m->layers) {
    const int64_t lq = c.n_heads * L.head_dim, lkv = L.n_kv_heads * L.head_dim;
    qd = lq > qd ? lq : qd;
    kvd = lkv > kvd ? lkv : kvd;
    qkvd = lq + 2 * lkv > qkvd ? lq + 2 * lkv : qkvd;
  }
  const size_t sc = model_attention_scratch(m, tp);
  const int64_t wide = c.hidden > qd ? c.hidden : qd;
  RET_IF(m->h.ensure((size_t)(t * c.hidden) * 4));
  RET_IF(m->xq.ensure((size_t)(t * wide)));
  RET_IF(m->dx.ensure((size_t)(t * (wide / 32)) * 4));
  RET_IF(m->qkv.ensure((size_t)(t * qkvd) * 4));
  RET_IF(m->attn_q.ensure((size_t)(tp * qd) * 2));
  RET_IF(m->attn_k.ensure((size_t)(tp * kvd) * 2));
  RET_IF(m->attn_vt.ensure((size_t)(tp * kvd) * 2));
  RET_IF(m->attn_scratch.ensure(sc * 4));
  RET_IF(m->cq.ensure((size_t)(t * qd)));
  RET_IF(m->dc.ensure((size_t)(t * (qd / 32)) * 4));
  RET_IF(m->proj.ensure((size_t)(t * c.hidden) * 4));
  const int64_t hw = c.ffn > c.ple_dim ? c.ffn : c.ple_dim;   // GeGLU outputs (Q8_0)
  RET_IF(m->hq.ensure((size_t)(t * hw)));
  RET_IF(m->dh.ensure((size_t)(t * (hw / 32)) * 4));
  RET_IF(m->normed.ensure((size_t)(t * c.hidden) * 4));
  const int64_t width = c.out_dim > 0 ? c.out_dim : c.hidden;
  const size_t p1 = pool_scratch_floats(t, width);
  const size_t p2 = pool_segments_scratch_floats(tp, tp / 64, width);
  RET_IF(m->pooled.ensure((p1 > p2 ? p1 : p2) * 4));
  if (c.ple_dim > 0) {
    RET_IF(m->ple.ensure((size_t)(t * c.n_layers * c.ple_dim) * 4));
    RET_IF(m->ple_gate.ensure((size_t)(t * c.ple_dim) * 4));
  }
  if (c.out_dim > 0) RET_IF(m->tokens.ensure((size_t)(t * c.out_dim) * 4));
  if (m->dense) {
    RET_IF(m->xb.ensure((size_t)(t * wide) * 2));
    RET_IF(m->hb.ensure((size_t)(t * c.ffn) * 2));
  }
  RET_IF(m->ids.ensure((size_t)t * 4));
  RET_IF(m->seg.ensure((size_t)tp * 8));
  RET_IF(m->seqs.ensure((size_t)(tp / 64) * 8));
  m->h_seg.reserve((size_t)tp * 2);
  m->h_seqs.reserve((size_t)(tp / 64) * 2);
  m->h_ids.reserve((size_t)tp);
  m->cap_t = t;
  return GLYPR_OK;
}

void free_model(glypr_model* m) {
  auto drop = [](LinearOp& l) {
    if (l.w) glypr_hip_q8_0_weight_destroy(l.w);
    if (l.wb) glypr_hip_bf16_weight_destroy(l.wb);
    l.w = nullptr;
    l.wb = nullptr;
  };
  auto dropn = [](RMSNorm& n) {
    if (n.weight) (void)hipFree(n.weight);
    n.weight = nullptr;
  };
  drop(m->token_embd);
  dropn(m->norm);
  drop(m->ple_projection);
  dropn(m->ple_norm);
  drop(m->embedding_projection);
  for (auto& L : m->layers) {
    drop(L.self_attn.q);
    drop(L.self_attn.k);
    drop(L.self_attn.v);
    drop(L.self_attn.o);
    drop(L.self_attn.fused_qkv);
    dropn(L.self_attn.q_norm);
    dropn(L.self_attn.k_norm);
    drop(L.mlp.gate);
    drop(L.mlp.up);
    drop(L.mlp.down);
    drop(L.mlp.fused_gate_up);
    dropn(L.input_layernorm);
    dropn(L.post_attention_layernorm);
    dropn(L.pre_feedforward_layernorm);
    dropn(L.post_feedforward_layernorm);
    drop(L.ple_block.gate);
    drop(L.ple_block.projection);
    dropn(L.ple_block.norm);
    if (L.ple_block.layer_scalar) (void)hipFree(L.ple_block.layer_scalar);
    L.ple_block.layer_scalar = nullptr;
  }
  for (DevBuf* b : {&m->cos_s, &m->sin_s, &m->cos_f, &m->sin_f, &m->h, &m->xq, &m->dx, &m->qkv,
                    &m->attn_q, &m->attn_k, &m->attn_vt, &m->attn_scratch,
                    &m->cq, &m->dc, &m->proj, &m->hq, &m->dh, &m->normed, &m->pooled, &m->ids,
                    &m->ple, &m->ple_gate, &m->tokens, &m->xb, &m->hb, &m->seg, &m->seqs})
    b->release();
}

// LinearOp::try_concat (linear.rs:82-148) for dense bf16 weights: one
// [sum of rows][k] buffer.
int concat_bf16(glypr_hip_ctx* ctx, const glypr_bf16w* const* parts, int count,
                glypr_bf16w** out) {
  int64_t n = 0;
  const int64_t k = parts[0]->k;
  for (int i = 0; i < count; i++) {
    GLYPR_CHECK(parts[i]->k == k, GLYPR_ERR_SHAPE, "concat of differing in_dim");
    n += parts[i]->n;
  }
  glypr_bf16w* w = new (std::nothrow) glypr_bf16w();
  GLYPR_CHECK(w != nullptr, GLYPR_ERR_OOM, "host allocation failed");
  w->n = n;
  w->k = k;
  w->device = ctx->device;
  hipError_t e = hipMalloc((void**)&w->p, (size_t)(n * k) * 2);
  int64_t off = 0;
  for (int i = 0; i < count && e == hipSuccess; i++) {
    e = hipMemcpy(w->p + off * k, parts[i]->p, (size_t)(parts[i]->n * k) * 2,
                  hipMemcpyDeviceToDevice);
    off += parts[i]->n;
  }
  if (e != hipSuccess) {
    if (w->p) (void)hipFree(w->p);
    delete w;
    return hip_error(e, "bf16 weight concat");
  }
  *out = w;
  return GLYPR_OK;
}

// The attention core shared by glypr_hip_attention and the model forward:
// per-head norms + RoPE, then flash attention writing ctx (f32) and/or the
// o projection's Q8_0 operand (cq, dc).
int attention_core(glypr_hip_ctx* ctx, const float* qkv, const float* qnw, const float* knw,
                   float eps, const float* cos_t, const float* sin_t, int64_t t, int64_t nq,
                   int64_t nkv, int64_t hd, int64_t window, uint16_t* q16, uint16_t* k16,
                   uint16_t* vt16, float* scratch, float* out, int8_t* cq, float* dc,
                   hipStream_t s, uint16_t* cb = nullptr, const int32_t* seg = nullptr,
                   int64_t seg_max = 0) {
  const int64_t tp = attn_padded_len(t);
  LAUNCH(GLYPR_K_QKV_POST, s,
         launch_qkv_post(qkv, t, tp, nq, nkv, hd, qnw, knw, eps, cos_t, sin_t, q16, k16, vt16, s,
                         seg),
         "qkv_post launch");
  LAUNCH(GLYPR_K_ATTENTION, s,
         launch_attention(q16, k16, vt16, scratch, out, cq, dc, t, tp, nq, nkv, hd, window, s, cb,
                          seg, seg_max),
         "attention launch");
  return GLYPR_OK;
}

// The rows of one forward: t rows of one sequence (seg NULL), or several
// sequences at 64-aligned offsets of t padded rows with their segment table.
struct Rows {
  int64_t t;
  const int32_t* seg;
  int64_t seg_max;
  const uint32_t* host_ids = nullptr;   // set: the gather reads the ids from the host
};

// The layers, final norm and pooling with dense bf16 projections (the
// bf16-weight variant of configs 4-5): each GEMM takes bf16 activations
// (nearest even) from the norm kernels and the attention combine, the
// residual stream h stays f32, GeGLU leaves the gate/up GEMM as bf16.
int forward_dense(glypr_model* m, glypr_hip_ctx* ctx, const Rows& rows, float* hidden,
                  float** tokens_out, hipStream_t s) {
  const int64_t t = rows.t;
  const glypr_model_config& c = m->cfg;
  const int64_t H = c.hidden, F = c.ffn, nq = c.n_heads;
  float* h = dev_f32(m->h);
  uint16_t* xb = m->xb.as<uint16_t>();
  uint16_t* hb = m->hb.as<uint16_t>();
  LAUNCH(GLYPR_K_RMSNORM_BF16, s,
         launch_rmsnorm_bf16(h, m->layers[0].input_layernorm.weight, c.eps, t, H, xb, s),
         "rmsnorm_bf16 launch");
  for (size_t li = 0; li < m->layers.size(); li++) {
    EncoderLayer& L = m->layers[li];
    const bool last = li + 1 == m->layers.size();
    const int64_t hd = L.head_dim, nkv = L.n_kv_heads, qd = nq * hd;
    const glypr_bf16w* wqkv = L.self_attn.fused_qkv.wb;
    const float* cos_t = dev_f32(L.full_attention ? m->cos_f : m->cos_s);
    const float* sin_t = dev_f32(L.full_attention ? m->sin_f : m->sin_s);
    const int64_t window = L.full_attention ? 0 : c.sliding_window;
    const int64_t tp = attn_padded_len(t);
    if (gemm_bf16w_qkv_ok(t, tp, H, hd)) {
      // the q|k|v GEMM writes the attention operands itself (no f32 q|k|v);
      // the attention writes its context as the o projection's bf16 operand
      LAUNCH(GLYPR_K_GEMM_BF16W, s,
             launch_gemm_bf16w_qkv(xb, wqkv->p, t, tp, H, nq, nkv, hd, L.self_attn.q_norm.weight,
                                   L.self_attn.k_norm.weight, c.eps, cos_t, sin_t,
                                   m->attn_q.as<uint16_t>(), m->attn_k.as<uint16_t>(),
                                   m->attn_vt.as<uint16_t>(), rows.seg, s),
             "qkv gemm launch");
      LAUNCH(GLYPR_K_ATTENTION, s,
             launch_attention(m->attn_q.as<uint16_t>(), m->attn_k.as<uint16_t>(),
                              m->attn_vt.as<uint16_t>(), dev_f32(m->attn_scratch), nullptr,
                              nullptr, nullptr, t, tp, nq, nkv, hd, window, s, xb, rows.seg,
                              rows.seg_max),
             "attention launch");
    } else {
      LAUNCH(GLYPR_K_GEMM_BF16W, s,
             launch_gemm_bf16w(xb, wqkv->p, dev_f32(m->qkv), t, wqkv->n, H, wqkv->n, s),
             "qkv gemm launch");
      RET_IF(attention_core(ctx, dev_f32(m->qkv), L.self_attn.q_norm.weight,
                            L.self_attn.k_norm.weight, c.eps, cos_t, sin_t, t, nq, nkv, hd,
                            window, m->attn_q.as<uint16_t>(), m->attn_k.as<uint16_t>(),
                            m->attn_vt.as<uint16_t>(), dev_f32(m->attn_scratch), nullptr,
                            nullptr, nullptr, s, xb, rows.seg, rows.seg_max));
    }
    const glypr_bf16w* wo = L.self_attn.o.wb;
    LAUNCH(GLYPR_K_GEMM_BF16W, s,
           launch_gemm_bf16w(xb, wo->p, dev_f32(m->proj), t, H, qd, H, s), "o gemm launch");
    LAUNCH(GLYPR_K_RESIDUAL_NORM, s,
           launch_residual_norm(dev_f32(m->proj), L.post_attention_layernorm.weight, h,
                                L.pre_feedforward_layernorm.weight, c.eps, t, H, nullptr,
                                nullptr, s, nullptr, false, xb),
           "residual_norm launch");
    const glypr_bf16w* wgu = L.mlp.fused_gate_up.wb;
    LAUNCH(GLYPR_K_GEMM_BF16W, s, launch_gemm_bf16w_geglu(xb, wgu->p, hb, t, F, H, s),
           "gate/up GeGLU launch");
    const glypr_bf16w* wd = L.mlp.down.wb;
    LAUNCH(GLYPR_K_GEMM_BF16W, s,
           launch_gemm_bf16w(hb, wd->p, dev_f32(m->proj), t, H, F, H, s), "down gemm launch");
    const float* w_next = last ? nullptr : m->layers[li + 1].input_layernorm.weight;
    LAUNCH(GLYPR_K_RESIDUAL_NORM, s,
           launch_residual_norm(dev_f32(m->proj), L.post_feedforward_layernorm.weight, h, w_next,
                                c.eps, t, H, nullptr, nullptr, s, nullptr, false,
                                last ? nullptr : xb),
           "residual_norm launch");
  }
  float* tokens = hidden ? hidden : dev_f32(m->normed);
  LAUNCH(GLYPR_K_RMSNORM, s, launch_rmsnorm(h, m->norm.weight, c.eps, tokens, t, H, s),
         "final rmsnorm launch");
  *tokens_out = tokens;
  return GLYPR_OK;
}

// forward_embeds (model.rs:498-578) over the rows whose ids are in m->ids:
// gather x embed_scale, the Per-Layer-Embedding inputs, the layers, the final
// norm and the embedding projection.  The token embeddings (width out_dim or
// hidden) are left in *tokens_out (`hidden` when given).
int forward_rows(glypr_model* m, glypr_hip_ctx* ctx, const Rows& rows, float* hidden,
                 float** tokens_out, hipStream_t s) {
  const glypr_model_config& c = m->cfg;
  const int64_t t = rows.t;
  const int64_t H = c.hidden, F = c.ffn, nq = c.n_heads;
  float* h = dev_f32(m->h);
  int8_t* xq = m->xq.as<int8_t>();
  float* dx = dev_f32(m->dx);

  // model.rs:507-508: Embedding::forward, then * embed_scale (f64 sqrt(hidden) as f32)
  const float embed_scale = (float)sqrt((double)H);
  const int64_t P = c.ple_dim, NL = c.n_layers;
  // Without PLE the gather and layer 0's input norm run as one launch (the
  // PLE projection would need xq for its own operand in between).
  const bool gather_norm = P == 0 && !m->dense && gather_norm_ok(t, H);
  if (gather_norm)
    LAUNCH(GLYPR_K_GATHER, s,
           launch_gather_norm(m->token_embd.w->qs(), m->token_embd.w->dw(), H, rows.host_ids,
                              rows.host_ids ? nullptr : m->ids.as<uint32_t>(), t, embed_scale,
                              m->layers[0].input_layernorm.weight, c.eps, h, xq, dx, s),
           "gather + input norm launch");
  else if (rows.host_ids)
    LAUNCH(GLYPR_K_GATHER, s,
           launch_gather_host_ids(m->token_embd.w->qs(), m->token_embd.w->dw(), H, rows.host_ids,
                                  t, embed_scale, h, s),
           "gather launch");
  else
    LAUNCH(GLYPR_K_GATHER, s,
           launch_gather(m->token_embd.w->qs(), m->token_embd.w->dw(), H, m->ids.as<uint32_t>(),
                         t, embed_scale, h, s),
           "gather launch");
  // TextPLE::project_and_norm_per_layer (ple.rs:48-85): per_layer_model_proj of
  // the scaled embeddings, * hidden^-0.5 (f64 powf, applied as candle's f32
  // affine), RMSNorm over ple_dim.  Layer l's input is row t*NL + l of [t*NL][P].
  float* ple = dev_f32(m->ple);
  if (P > 0) {
    LAUNCH(GLYPR_K_QUANTIZE, s, launch_quantize_planar(h, t, H, xq, dx, s), "quantize launch");
    const glypr_q8w* wpl = m->ple_projection.w;
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(xq, dx, wpl->qs(), wpl->dw(), ple, t, NL * P, H, NL * P, s, m->fma2),
           "per-layer projection launch");
    LAUNCH(GLYPR_K_RMSNORM, s, launch_affine(ple, t * NL * P, (float)pow((double)H, -0.5), s),
           "per-layer scale launch");
    LAUNCH(GLYPR_K_RMSNORM, s, launch_rmsnorm(ple, m->ple_norm.weight, c.eps, ple, t * NL, P, s),
           "per-layer norm launch");
  }
  if (m->dense) return forward_dense(m, ctx, rows, hidden, tokens_out, s);
  // layer 0 input_layernorm as the qkv GEMM's prologue
  if (!gather_norm)
    LAUNCH(GLYPR_K_RMSNORM_QUANT, s,
           launch_rmsnorm_quant(h, m->layers[0].input_layernorm.weight, c.eps, t, H, xq, dx, s),
           "rmsnorm_quant launch");
  // model.rs:576-577: the final norm rides on the last layer's residual launch:
  // into xq / dx for the embedding projection, else as f32 token rows
  float* tokens = hidden;
  if (!tokens) tokens = dev_f32(c.out_dim > 0 ? m->tokens : m->normed);
  float* final_f32 = c.out_dim > 0 ? nullptr : tokens;

  for (size_t li = 0; li < m->layers.size(); li++) {
    EncoderLayer& L = m->layers[li];
    const bool last = li + 1 == m->layers.size();
    const int64_t hd = L.head_dim, nkv = L.n_kv_heads, qd = nq * hd;
    // ---- attention block (layer.rs:27-34)
    const glypr_q8w* wqkv = L.self_attn.fused_qkv.w;
    const float* cos_t = dev_f32(L.full_attention ? m->cos_f : m->cos_s);
    const float* sin_t = dev_f32(L.full_attention ? m->sin_f : m->sin_s);
    const int64_t window = L.full_attention ? 0 : c.sliding_window;
    const int64_t tp = attn_padded_len(t);
    if (gemm_i8_qkv_ok(t, tp, H, hd)) {
      // the q|k|v GEMM writes the attention operands itself (no f32 q|k|v)
      LAUNCH(GLYPR_K_GEMM_I8_QKV, s,
             launch_gemm_i8_qkv(xq, dx, wqkv->qs(), wqkv->dw(), t, tp, H, nq, nkv, hd,
                                L.self_attn.q_norm.weight, L.self_attn.k_norm.weight, c.eps,
                                cos_t, sin_t, m->attn_q.as<uint16_t>(), m->attn_k.as<uint16_t>(),
                                m->attn_vt.as<uint16_t>(), rows.seg, s, m->fma2),
             "qkv gemm launch");
      LAUNCH(GLYPR_K_ATTENTION, s,
             launch_attention(m->attn_q.as<uint16_t>(), m->attn_k.as<uint16_t>(),
                              m->attn_vt.as<uint16_t>(), dev_f32(m->attn_scratch), nullptr,
                              m->cq.as<int8_t>(), dev_f32(m->dc), t, tp, nq, nkv, hd, window, s,
                              nullptr, rows.seg, rows.seg_max),
             "attention launch");
    } else {
      LAUNCH(GLYPR_K_GEMM_I8, s,
             launch_gemm_i8(xq, dx, wqkv->qs(), wqkv->dw(), dev_f32(m->qkv), t, wqkv->n, H,
                            wqkv->n, s, m->fma2),
             "qkv gemm launch");
      RET_IF(attention_core(ctx, dev_f32(m->qkv), L.self_attn.q_norm.weight,
                            L.self_attn.k_norm.weight, c.eps, cos_t, sin_t, t, nq, nkv, hd,
                            window, m->attn_q.as<uint16_t>(), m->attn_k.as<uint16_t>(),
                            m->attn_vt.as<uint16_t>(), dev_f32(m->attn_scratch), nullptr,
                            m->cq.as<int8_t>(), dev_f32(m->dc), s, nullptr, rows.seg,
                            rows.seg_max));
    }
    const glypr_q8w* wo = L.self_attn.o.w;
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(m->cq.as<int8_t>(), dev_f32(m->dc), wo->qs(), wo->dw(),
                          dev_f32(m->proj), t, H, qd, H, s, m->fma2),
           "o gemm launch");
    // post_attention_layernorm.forward_residual_add + pre_feedforward_layernorm prologue
    LAUNCH(GLYPR_K_RESIDUAL_NORM, s,
           launch_residual_norm(dev_f32(m->proj), L.post_attention_layernorm.weight, h,
                                L.pre_feedforward_layernorm.weight, c.eps, t, H, xq, dx, s),
           "residual_norm launch");
    // ---- feed-forward block (layer.rs:36-42): gate/up + GeGLU epilogue, down
    const glypr_q8w* wgu = L.mlp.fused_gate_up.w;
    LAUNCH(GLYPR_K_GEMM_I8_GEGLU, s,
           launch_gemm_i8_geglu(xq, dx, wgu->qs(), wgu->dw(), m->hq.as<int8_t>(), dev_f32(m->dh),
                                t, F, H, s, m->fma2),
           "gate/up GeGLU launch");
    const glypr_q8w* wd = L.mlp.down.w;
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(m->hq.as<int8_t>(), dev_f32(m->dh), wd->qs(), wd->dw(),
                          dev_f32(m->proj), t, H, F, H, s, m->fma2),
           "down gemm launch");
    // next layer's input norm, or after the last layer the final norm
    const float* w_next = last ? m->norm.weight : m->layers[li + 1].input_layernorm.weight;
    int8_t* q_next = last && final_f32 ? nullptr : xq;
    float* d_next = last && final_f32 ? nullptr : dx;
    float* y_next = last ? final_f32 : nullptr;
    if (P == 0) {
      // post_feedforward_layernorm.forward_residual_add + next layer's input norm
      LAUNCH(GLYPR_K_RESIDUAL_NORM, s,
             launch_residual_norm(dev_f32(m->proj), L.post_feedforward_layernorm.weight, h,
                                  w_next, c.eps, t, H, q_next, d_next, s, nullptr, false, nullptr,
                                  y_next),
             "residual_norm launch");
      continue;
    }
    // post_feedforward_layernorm.forward_residual_add, then Q8_0 of h itself
    // for the PLE block's inp_gate (no norm in front of it)
    LAUNCH(GLYPR_K_RESIDUAL_NORM, s,
           launch_residual_norm(dev_f32(m->proj), L.post_feedforward_layernorm.weight, h, nullptr,
                                c.eps, t, H, xq, dx, s, nullptr, true),
           "residual_norm launch");
    // ---- TextPLEBlock::forward_with_scalar (ple.rs:118-145)
    const glypr_q8w* wg = L.ple_block.gate.w;
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(xq, dx, wg->qs(), wg->dw(), dev_f32(m->ple_gate), t, P, H, P, s, m->fma2),
           "per-layer gate launch");
    LAUNCH(GLYPR_K_GEGLU, s,
           launch_geglu_quant(dev_f32(m->ple_gate), ple + (int64_t)li * P, NL * P, t, P,
                              m->hq.as<int8_t>(), dev_f32(m->dh), s),
           "per-layer geglu launch");
    const glypr_q8w* wpj = L.ple_block.projection.w;
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(m->hq.as<int8_t>(), dev_f32(m->dh), wpj->qs(), wpj->dw(),
                          dev_f32(m->proj), t, H, P, H, s, m->fma2),
           "per-layer proj launch");
    // post_norm.forward_residual_add(.., layer_scalar) + next layer's input norm
    LAUNCH(GLYPR_K_RESIDUAL_NORM, s,
           launch_residual_norm(dev_f32(m->proj), L.ple_block.norm.weight, h, w_next, c.eps, t, H,
                                q_next, d_next, s, L.ple_block.layer_scalar, false, nullptr,
                                y_next),
           "residual_norm launch");
  }
  // then the embedding projection when present
  if (c.out_dim > 0) {
    const glypr_q8w* we = m->embedding_projection.w;
    LAUNCH(GLYPR_K_GEMM_I8, s,
           launch_gemm_i8(xq, dx, we->qs(), we->dw(), tokens, t, c.out_dim, H, c.out_dim, s,
                          m->fma2),
           "embedding projection launch");
  }
  *tokens_out = tokens;
  return GLYPR_OK;
}

}  // namespace

extern "C" {

int glypr_hip_attention(glypr_hip_ctx* ctx, const float* qkv, const float* q_norm_weight,
                        const float* k_norm_weight, float eps, const float* cos_table,
                        const float* sin_table, int64_t t, int64_t n_heads, int64_t n_kv_heads,
                        int64_t head_dim, int64_t window, float* ctx_out, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(t >= 0 && n_heads > 0 && n_kv_heads > 0 && window >= 0, GLYPR_ERR_SHAPE,
              "invalid attention shape");
  GLYPR_CHECK(n_heads % n_kv_heads == 0, GLYPR_ERR_SHAPE,
              "n_heads %lld not a multiple of n_kv_heads %lld", (long long)n_heads,
              (long long)n_kv_heads);
  GLYPR_CHECK(attention_supported(t, n_heads, n_kv_heads, head_dim, window),
              GLYPR_ERR_UNSUPPORTED,
              "attention geometry not supported: head_dim %lld (256 and 512 are supported), %lld q "
              "heads per kv head (at most 4), t = %lld", (long long)head_dim,
              (long long)(n_heads / n_kv_heads), (long long)t);
  GLYPR_CHECK(t == 0 || (qkv && cos_table && sin_table && ctx_out), GLYPR_ERR_INVALID_ARG,
              "qkv, cos/sin tables or ctx_out is NULL");
  GLYPR_CHECK(aligned16(qkv) && aligned16(ctx_out) && aligned16(cos_table) &&
                  aligned16(sin_table) && aligned16(q_norm_weight) && aligned16(k_norm_weight),
              GLYPR_ERR_ALIGNMENT, "attention buffers must be 16-byte aligned");
  RET_IF(check_ctx(ctx));
  if (t == 0) return GLYPR_OK;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  const int64_t tp = attn_padded_len(t);
  const size_t qb = align_up((size_t)(tp * n_heads * head_dim) * 2, 256);
  const size_t kb = align_up((size_t)(tp * n_kv_heads * head_dim) * 2, 256);
  const size_t sb = attention_scratch_floats(t, n_heads, n_kv_heads, head_dim, window) * 4;
  RET_IF(ensure_ws(ctx, qb + 2 * kb + sb));
  char* base = (char*)ctx->ws;
  uint16_t* q16 = (uint16_t*)base;
  uint16_t* k16 = (uint16_t*)(base + qb);
  uint16_t* vt16 = (uint16_t*)(base + qb + kb);
  float* scratch = (float*)(base + qb + 2 * kb);
  return attention_core(ctx, qkv, q_norm_weight, k_norm_weight, eps, cos_table, sin_table, t,
                        n_heads, n_kv_heads, head_dim, window, q16, k16, vt16, scratch, ctx_out,
                        nullptr, nullptr, (hipStream_t)stream);
}

int glypr_hip_model_create(glypr_hip_ctx* ctx, const glypr_model_config* cfg,
                           glypr_model** out) {
  clear_error();
  GLYPR_CHECK(cfg != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "cfg or out is NULL");
  *out = nullptr;
  GLYPR_CHECK(cfg->hidden > 0 && cfg->ffn > 0 && cfg->n_layers > 0 && cfg->vocab > 0,
              GLYPR_ERR_SHAPE, "model dimensions must be positive");
  GLYPR_CHECK(cfg->hidden % 32 == 0 && cfg->ffn % 32 == 0 && cfg->hidden <= 1024, GLYPR_ERR_SHAPE,
              "hidden (<= 1024) and ffn must be multiples of 32");
  GLYPR_CHECK(cfg->head_dim > 0 && cfg->full_head_dim >= 0 && cfg->full_n_kv_heads >= 0 &&
                  cfg->max_seq_len >= 0 && cfg->sliding_window >= 0,
              GLYPR_ERR_SHAPE, "head_dim must be positive; full_head_dim, full_n_kv_heads, "
              "max_seq_len and sliding_window non-negative");
  GLYPR_CHECK(cfg->n_heads > 0 && cfg->n_kv_heads > 0 && cfg->n_heads % cfg->n_kv_heads == 0,
              GLYPR_ERR_SHAPE, "n_heads must be a positive multiple of n_kv_heads");
  GLYPR_CHECK(cfg->full_n_kv_heads == 0 || cfg->n_heads % cfg->full_n_kv_heads == 0,
              GLYPR_ERR_SHAPE, "n_heads must be a multiple of full_n_kv_heads");
  GLYPR_CHECK(cfg->ple_dim >= 0 && cfg->ple_dim % 32 == 0 && cfg->out_dim >= 0, GLYPR_ERR_SHAPE,
              "ple_dim (%lld) must be a non-negative multiple of 32, out_dim (%lld) >= 0",
              (long long)cfg->ple_dim, (long long)cfg->out_dim);
  glypr_model_config c = *cfg;
  c.layer_types = nullptr;   // read below, not kept
  if (c.full_head_dim == 0) c.full_head_dim = c.head_dim;
  if (c.full_n_kv_heads == 0) c.full_n_kv_heads = c.n_kv_heads;
  if (c.max_seq_len == 0) c.max_seq_len = 8320;   // DEFAULT_MAX_SEQ_LEN, lib.rs:47
  GLYPR_CHECK(c.max_batch_tokens >= 0 && c.max_batch_tokens <= (int64_t(1) << 24),
              GLYPR_ERR_SHAPE, "max_batch_tokens %lld outside [0, 2^24]",
              (long long)c.max_batch_tokens);
  {
    // the attention operands hold max(max_seq_len, max_batch_tokens) rows
    const int64_t rows = c.max_seq_len > c.max_batch_tokens ? c.max_seq_len : c.max_batch_tokens;
    const int64_t hd = c.head_dim > c.full_head_dim ? c.head_dim : c.full_head_dim;
    GLYPR_CHECK(attention_rows_ok(rows, hd), GLYPR_ERR_SHAPE,
                "%lld rows of head_dim %lld exceed the attention kernels' 32-bit offsets "
                "(2 * head_dim * padded rows must stay below 2^31)",
                (long long)rows, (long long)hd);
  }
  // the attention kernels' geometry, checked for both layer types at the
  // longest sequence (shorter ones use fewer key partitions)
  GLYPR_CHECK(attention_supported(c.max_seq_len, c.n_heads, c.n_kv_heads, c.head_dim,
                                  c.sliding_window) &&
                  attention_supported(c.max_seq_len, c.n_heads, c.full_n_kv_heads,
                                      c.full_head_dim, 0),
              GLYPR_ERR_UNSUPPORTED,
              "attention geometry not supported: head_dim %lld / %lld (sliding / full; 256 and "
              "512 are supported), %lld q heads over %lld / %lld kv heads (at most 4 per kv "
              "head)",
              (long long)c.head_dim, (long long)c.full_head_dim, (long long)c.n_heads,
              (long long)c.n_kv_heads, (long long)c.full_n_kv_heads);
  RET_IF(check_ctx(ctx));
  glypr_model* m = new (std::nothrow) glypr_model();
  GLYPR_CHECK(m != nullptr, GLYPR_ERR_OOM, "host allocation failed");
  m->ctx = ctx;
  m->cfg = c;
  m->layers.resize((size_t)c.n_layers);
  for (int64_t i = 0; i < c.n_layers; i++) {
    EncoderLayer& L = m->layers[(size_t)i];
    // layer_types from sliding_window_pattern, or the default 5 sliding +
    // 1 full pattern (config.rs:117-140)
    L.full_attention = cfg->layer_types ? cfg->layer_types[i] != 0 : ((i + 1) % 6) == 0;
    L.head_dim = L.full_attention ? c.full_head_dim : c.head_dim;
    L.n_kv_heads = L.full_attention ? c.full_n_kv_heads : c.n_kv_heads;
  }
  *out = m;
  return GLYPR_OK;
}

int glypr_hip_model_set_tensor(glypr_model* m, const char* name, const void* data, int64_t rows,
                               int64_t cols, int dtype) {
  clear_error();
  GLYPR_CHECK(m != nullptr && name != nullptr && data != nullptr, GLYPR_ERR_INVALID_ARG,
              "model, name or data is NULL");
  GLYPR_CHECK(dtype >= 0 && dtype <= 2, GLYPR_ERR_UNSUPPORTED,
              "dtype %d (0 = f32, 1 = Q8_0, 2 = bf16)", dtype);
  GLYPR_CHECK(!m->finalized, GLYPR_ERR_INVALID_ARG, "model already finalized");
  const glypr_model_config& c = m->cfg;
  DeviceScope ds(m->ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  const std::string n(name);

  auto set_q8 = [&](LinearOp& op, int64_t er, int64_t ec) -> int {
    GLYPR_CHECK(dtype == 1, GLYPR_ERR_UNSUPPORTED, "%s must be Q8_0", name);
    GLYPR_CHECK(rows == er && cols == ec, GLYPR_ERR_SHAPE,
                "%s has shape (%lld, %lld), expected (%lld, %lld)", name, (long long)rows,
                (long long)cols, (long long)er, (long long)ec);
    if (op.w) glypr_hip_q8_0_weight_destroy(op.w);
    op.w = nullptr;
    return glypr_hip_q8_0_weight_create(m->ctx, (const uint8_t*)data, rows, cols, &op.w);
  };
  // a layer projection: Q8_0 blocks (dtype 1) or dense bf16 rows (dtype 2)
  auto set_lin = [&](LinearOp& op, int64_t er, int64_t ec) -> int {
    if (dtype != 2) return set_q8(op, er, ec);
    GLYPR_CHECK(rows == er && cols == ec, GLYPR_ERR_SHAPE,
                "%s has shape (%lld, %lld), expected (%lld, %lld)", name, (long long)rows,
                (long long)cols, (long long)er, (long long)ec);
    if (op.w) glypr_hip_q8_0_weight_destroy(op.w);
    if (op.wb) glypr_hip_bf16_weight_destroy(op.wb);
    op.w = nullptr;
    op.wb = nullptr;
    return glypr_hip_bf16_weight_create(m->ctx, (const uint16_t*)data, rows, cols, &op.wb);
  };
  auto set_norm_raw = [&](float*& dst, int64_t len) -> int {
    GLYPR_CHECK(dtype == 0, GLYPR_ERR_UNSUPPORTED, "%s must be f32", name);
    GLYPR_CHECK(rows * cols == len, GLYPR_ERR_SHAPE, "%s has %lld values, expected %lld", name,
                (long long)(rows * cols), (long long)len);
    if (dst) (void)hipFree(dst);
    dst = nullptr;
    return upload_f32((const float*)data, len, &dst);
  };
  auto set_norm = [&](RMSNorm& nm, int64_t len) -> int { return set_norm_raw(nm.weight, len); };

  if (n == "token_embd.weight") return set_q8(m->token_embd, c.vocab, c.hidden);
  if (n == "output_norm.weight") return set_norm(m->norm, c.hidden);
  if (c.ple_dim > 0 && n == "per_layer_model_proj.weight")
    return set_q8(m->ple_projection, c.n_layers * c.ple_dim, c.hidden);
  if (c.ple_dim > 0 && n == "per_layer_proj_norm.weight") return set_norm(m->ple_norm, c.ple_dim);
  if (c.out_dim > 0 && n == "output.weight")
    return set_q8(m->embedding_projection, c.out_dim, c.hidden);
  int layer = -1, consumed = 0;
  char field[64] = {0};
  if (sscanf(name, "blk.%d.%63[^.].weight%n", &layer, field, &consumed) == 2 &&
      name[consumed] == '\0' && layer >= 0 && layer < c.n_layers) {
    EncoderLayer& L = m->layers[(size_t)layer];
    const std::string f(field);
    const int64_t qd = c.n_heads * L.head_dim, kvd = L.n_kv_heads * L.head_dim;
    if (f == "attn_norm") return set_norm(L.input_layernorm, c.hidden);
    if (f == "post_attention_norm") return set_norm(L.post_attention_layernorm, c.hidden);
    if (f == "ffn_norm") return set_norm(L.pre_feedforward_layernorm, c.hidden);
    if (f == "post_ffw_norm") return set_norm(L.post_feedforward_layernorm, c.hidden);
    if (f == "attn_q_norm") return set_norm(L.self_attn.q_norm, L.head_dim);
    if (f == "attn_k_norm") return set_norm(L.self_attn.k_norm, L.head_dim);
    if (f == "attn_q") return set_lin(L.self_attn.q, qd, c.hidden);
    if (f == "attn_k") return set_lin(L.self_attn.k, kvd, c.hidden);
    if (f == "attn_v") return set_lin(L.self_attn.v, kvd, c.hidden);
    if (f == "attn_output") return set_lin(L.self_attn.o, c.hidden, qd);
    if (f == "ffn_gate") return set_lin(L.mlp.gate, c.ffn, c.hidden);
    if (f == "ffn_up") return set_lin(L.mlp.up, c.ffn, c.hidden);
    if (f == "ffn_down") return set_lin(L.mlp.down, c.hidden, c.ffn);
    if (c.ple_dim > 0) {
      if (f == "inp_gate") return set_q8(L.ple_block.gate, c.ple_dim, c.hidden);
      if (f == "proj") return set_q8(L.ple_block.projection, c.hidden, c.ple_dim);
      if (f == "post_norm") return set_norm(L.ple_block.norm, c.hidden);
      if (f == "layer_output_scale") return set_norm_raw(L.ple_block.layer_scalar, 1);
    }
  }
  return set_error(GLYPR_ERR_INVALID_ARG, "unknown tensor name '%s'", name);
}

int glypr_hip_model_finalize(glypr_model* m) {
  clear_error();
  GLYPR_CHECK(m != nullptr, GLYPR_ERR_INVALID_ARG, "model is NULL");
  if (m->finalized) return GLYPR_OK;
  GLYPR_CHECK(m->token_embd.w && m->norm.weight, GLYPR_ERR_INVALID_ARG,
              "token_embd.weight or output_norm.weight missing");
  GLYPR_CHECK(m->cfg.ple_dim == 0 || (m->ple_projection.w && m->ple_norm.weight),
              GLYPR_ERR_INVALID_ARG, "per_layer_model_proj / per_layer_proj_norm missing");
  GLYPR_CHECK(m->cfg.out_dim == 0 || m->embedding_projection.w, GLYPR_ERR_INVALID_ARG,
              "output.weight missing");
  DeviceScope ds(m->ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  // every layer projection is Q8_0, or every one is dense bf16
  int n_q8 = 0, n_bf = 0;
  for (auto& L : m->layers)
    for (const LinearOp* op : {&L.self_attn.q, &L.self_attn.k, &L.self_attn.v, &L.self_attn.o,
                               &L.mlp.gate, &L.mlp.up, &L.mlp.down}) {
      n_q8 += op->w != nullptr;
      n_bf += op->wb != nullptr;
    }
  GLYPR_CHECK(n_q8 == 0 || n_bf == 0, GLYPR_ERR_UNSUPPORTED,
              "layer projections mix Q8_0 and bf16 weights");
  m->dense = n_bf > 0;
  if (m->dense) {
    GLYPR_CHECK(m->cfg.ple_dim == 0 && m->cfg.out_dim == 0, GLYPR_ERR_UNSUPPORTED,
                "dense bf16 projections are supported without the Per-Layer-Embedding block "
                "and the embedding projection");
    GLYPR_CHECK(m->cfg.hidden % 64 == 0 && m->cfg.ffn % 64 == 0, GLYPR_ERR_UNSUPPORTED,
                "dense bf16 projections need hidden and ffn multiples of 64");
  }
  auto has = [](const LinearOp& op) { return op.w != nullptr || op.wb != nullptr; };
  for (size_t i = 0; i < m->layers.size(); i++) {
    EncoderLayer& L = m->layers[i];
    GLYPR_CHECK(has(L.self_attn.q) && has(L.self_attn.k) && has(L.self_attn.v) &&
                    has(L.self_attn.o) && has(L.mlp.gate) && has(L.mlp.up) && has(L.mlp.down) &&
                    L.self_attn.q_norm.weight && L.self_attn.k_norm.weight &&
                    L.input_layernorm.weight && L.post_attention_layernorm.weight &&
                    L.pre_feedforward_layernorm.weight && L.post_feedforward_layernorm.weight,
                GLYPR_ERR_INVALID_ARG, "layer %zu is missing tensors", i);
    GLYPR_CHECK(m->cfg.ple_dim == 0 ||
                    (L.ple_block.gate.w && L.ple_block.projection.w && L.ple_block.norm.weight &&
                     L.ple_block.layer_scalar),
                GLYPR_ERR_INVALID_ARG, "layer %zu is missing its Per-Layer-Embedding tensors", i);
    if (m->dense) {
      const glypr_bf16w* qkv[3] = {L.self_attn.q.wb, L.self_attn.k.wb, L.self_attn.v.wb};
      RET_IF(concat_bf16(m->ctx, qkv, 3, &L.self_attn.fused_qkv.wb));
      const glypr_bf16w* gu[2] = {L.mlp.gate.wb, L.mlp.up.wb};
      RET_IF(concat_bf16(m->ctx, gu, 2, &L.mlp.fused_gate_up.wb));
      continue;
    }
    const glypr_q8w* qkv[3] = {L.self_attn.q.w, L.self_attn.k.w, L.self_attn.v.w};
    RET_IF(glypr_hip_q8_0_weight_concat(m->ctx, qkv, 3, &L.self_attn.fused_qkv.w, nullptr));
    const glypr_q8w* gu[2] = {L.mlp.gate.w, L.mlp.up.w};
    RET_IF(glypr_hip_q8_0_weight_concat(m->ctx, gu, 2, &L.mlp.fused_gate_up.w, nullptr));
  }
  // every buffer and table the forward uses, at max_seq_len: model_embed
  // allocates nothing
  RET_IF(ensure_rope(m, m->cfg.max_seq_len));
  const int64_t cap = m->cfg.max_batch_tokens > m->cfg.max_seq_len ? m->cfg.max_batch_tokens
                                                                  : m->cfg.max_seq_len;
  RET_IF(ensure_activations(m, attn_padded_len(cap)));
  m->finalized = true;
  return GLYPR_OK;
}

int glypr_hip_model_embed(glypr_model* m, const uint32_t* ids, int64_t t, int64_t trunc,
                          float* out, float* hidden, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m != nullptr, GLYPR_ERR_INVALID_ARG, "model is NULL");
  GLYPR_CHECK(m->finalized, GLYPR_ERR_INVALID_ARG, "call glypr_hip_model_finalize first");
  GLYPR_CHECK(t > 0 && trunc >= 0, GLYPR_ERR_SHAPE, "t = %lld, trunc = %lld", (long long)t,
              (long long)trunc);
  GLYPR_CHECK(ids != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG, "ids or out is NULL");
  GLYPR_CHECK(aligned16(out) && aligned16(hidden), GLYPR_ERR_ALIGNMENT,
              "out and hidden must be 16-byte aligned");
  const glypr_model_config& c = m->cfg;
  // the context-length preflight of encode_single_text (lib.rs:970-976)
  GLYPR_CHECK(t <= c.max_seq_len, GLYPR_ERR_SHAPE,
              "sequence length (%lld tokens) exceeds the maximum context limit (%lld tokens)",
              (long long)t, (long long)c.max_seq_len);
  for (int64_t i = 0; i < t; i++)
    GLYPR_CHECK((int64_t)ids[i] < c.vocab, GLYPR_ERR_RANGE,
                "token id %u at position %lld is out of range for vocab %lld", ids[i],
                (long long)i, (long long)c.vocab);
  glypr_hip_ctx* ctx = m->ctx;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  // buffers and RoPE tables were sized at finalize
  hipStream_t s = (hipStream_t)stream;
  // Up to GATHER_ARG_IDS ids ride in the gather's kernel arguments; longer
  // sequences are uploaded first.
  const bool arg_ids = gather_host_ids_ok(c.hidden, t);
  if (!arg_ids)
    GLYPR_TRY_HIP(hipMemcpyAsync(m->ids.p, ids, (size_t)t * 4, hipMemcpyHostToDevice, s),
                  "ids upload");
  float* tokens = nullptr;
  RET_IF(forward_rows(m, ctx, Rows{t, nullptr, 0, arg_ids ? ids : nullptr}, hidden, &tokens, s));
  const int64_t width = c.out_dim > 0 ? c.out_dim : c.hidden;
  LAUNCH(GLYPR_K_POOL, s,
         launch_pool(tokens, nullptr, t, width, trunc, out, dev_f32(m->pooled), s),
         "pool launch");
  return GLYPR_OK;
}

int glypr_hip_model_embed_batch(glypr_model* m, const uint32_t* ids, const int64_t* lens,
                                int64_t n_seqs, int64_t trunc, float* out, glypr_stream stream) {
  clear_error();
  GLYPR_CHECK(m != nullptr, GLYPR_ERR_INVALID_ARG, "model is NULL");
  GLYPR_CHECK(m->finalized, GLYPR_ERR_INVALID_ARG, "call glypr_hip_model_finalize first");
  GLYPR_CHECK(n_seqs > 0 && trunc >= 0, GLYPR_ERR_SHAPE, "n_seqs = %lld, trunc = %lld",
              (long long)n_seqs, (long long)trunc);
  GLYPR_CHECK(ids != nullptr && lens != nullptr && out != nullptr, GLYPR_ERR_INVALID_ARG,
              "ids, lens or out is NULL");
  GLYPR_CHECK(aligned16(out), GLYPR_ERR_ALIGNMENT, "out must be 16-byte aligned");
  const glypr_model_config& c = m->cfg;
  // embed_batch_inner's preflight per item (lib.rs:838-845), then the layout:
  // sequence i at rows [off_i, off_i + lens[i]), offsets 64-aligned
  int64_t rows = 0, total = 0, longest = 0;
  for (int64_t i = 0; i < n_seqs; i++) {
    GLYPR_CHECK(lens[i] > 0 && lens[i] <= c.max_seq_len, GLYPR_ERR_SHAPE,
                "batch item %lld sequence length (%lld) is outside [1, %lld]", (long long)i,
                (long long)lens[i], (long long)c.max_seq_len);
    rows += attn_padded_len(lens[i]);
    total += lens[i];
    longest = lens[i] > longest ? lens[i] : longest;
  }
  GLYPR_CHECK(rows <= m->cap_t, GLYPR_ERR_SHAPE,
              "batch of %lld sequences takes %lld padded rows; the model holds %lld "
              "(max_batch_tokens)", (long long)n_seqs, (long long)rows, (long long)m->cap_t);
  for (int64_t i = 0; i < total; i++)
    GLYPR_CHECK((int64_t)ids[i] < c.vocab, GLYPR_ERR_RANGE,
                "token id %u at position %lld is out of range for vocab %lld", ids[i],
                (long long)i, (long long)c.vocab);
  glypr_hip_ctx* ctx = m->ctx;
  DeviceScope ds(ctx->device);
  if (ds.err != hipSuccess) return hip_error(ds.err, "hipSetDevice");
  std::lock_guard<std::mutex> lk(ctx->mu);
  hipStream_t s = (hipStream_t)stream;
  // host staging (capacity reserved at finalize): padded ids (padding rows take
  // id 0; they never reach a valid token's attention or its pooled mean),
  // the per-row segment table and the per-sequence {offset, length}
  m->h_ids.assign((size_t)rows, 0u);
  m->h_seg.resize((size_t)rows * 2);
  m->h_seqs.resize((size_t)n_seqs * 2);
  int64_t off = 0, src = 0;
  for (int64_t i = 0; i < n_seqs; i++) {
    const int64_t len = lens[i], span = attn_padded_len(len);
    memcpy(m->h_ids.data() + off, ids + src, (size_t)len * 4);
    for (int64_t r = off; r < off + span; r++) {
      m->h_seg[(size_t)r * 2] = (int32_t)off;
      m->h_seg[(size_t)r * 2 + 1] = (int32_t)len;
    }
    m->h_seqs[(size_t)i * 2] = (int32_t)off;
    m->h_seqs[(size_t)i * 2 + 1] = (int32_t)len;
    off += span;
    src += len;
  }
  // pageable-memory uploads are staged before hipMemcpyAsync returns, so the
  // host vectors may be refilled by the next call
  GLYPR_TRY_HIP(hipMemcpyAsync(m->ids.p, m->h_ids.data(), (size_t)rows * 4,
                               hipMemcpyHostToDevice, s), "ids upload");
  GLYPR_TRY_HIP(hipMemcpyAsync(m->seg.p, m->h_seg.data(), (size_t)rows * 8,
                               hipMemcpyHostToDevice, s), "segment table upload");
  GLYPR_TRY_HIP(hipMemcpyAsync(m->seqs.p, m->h_seqs.data(), (size_t)n_seqs * 8,
                               hipMemcpyHostToDevice, s), "sequence table upload");
  float* tokens = nullptr;
  RET_IF(forward_rows(m, ctx, Rows{rows, m->seg.as<int32_t>(), longest}, nullptr, &tokens, s));
  const int64_t width = c.out_dim > 0 ? c.out_dim : c.hidden;
  // lib.rs:902-941: a batch of equal lengths pools by the plain mean, a mixed
  // one by the masked sum over the token count
  bool mixed = false;
  for (int64_t i = 1; i < n_seqs; i++) mixed = mixed || lens[i] != lens[0];
  LAUNCH(GLYPR_K_POOL, s,
         launch_pool_segments(tokens, rows, m->seg.as<int32_t>(), m->seqs.as<int32_t>(), n_seqs,
                              width, trunc, out, dev_f32(m->pooled), s, mixed),
         "pool launch");
  return GLYPR_OK;
}

int glypr_hip_model_set_variant(glypr_model* m, int variant) {
  clear_error();
  GLYPR_CHECK(m != nullptr, GLYPR_ERR_INVALID_ARG, "model is NULL");
  GLYPR_CHECK(variant == GLYPR_Q8_INT8_EXACT || variant == GLYPR_Q8_INT8_FMA,
              GLYPR_ERR_UNSUPPORTED,
              "the model runs its Q8_0 projections as INT8_EXACT or INT8_FMA, not variant %d",
              variant);
  m->fma2 = variant == GLYPR_Q8_INT8_FMA;
  return GLYPR_OK;
}

int glypr_hip_model_destroy(glypr_model* m) {
  clear_error();
  if (!m) return GLYPR_OK;
  {
    DeviceScope ds(m->ctx->device);
    (void)hipDeviceSynchronize();
    free_model(m);
  }
  delete m;
  return GLYPR_OK;
}

}  // extern "C"
