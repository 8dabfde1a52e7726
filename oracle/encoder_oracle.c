/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for the encoder rows.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this; the product path never does.
 *
 * Restates the reference host path of the imported BERT embedder in plain C,
 * with the reference's precision choices:
 *  - BERTEmbeddingsReference (runtime/backend/tensor_ops.go:1451-1512):
 *    token + position + type summed in f32, LayerNorm statistics in f64;
 *  - denseHF / denseHFRange (runtime/backend/bert_encoder_layer_ops.go:423-495):
 *    x W^T + b with an f64 accumulator started at the bias, HF [out, in] weights;
 *  - bertSelfAttentionContextRange (bert_encoder_layer_ops.go:272-324): per
 *    (batch, query, head), logits q.k * 1/sqrt(hd) in f64 over keys whose mask
 *    is nonzero, max-subtracted exp in f64, context accumulated in f32 as
 *    float32(prob * v); a query with no active key keeps a zero context;
 *  - BERTEncoderLayerReference (bert_encoder_layer_ops.go:80-225): post-LN
 *    residual blocks, erf GELU (exactGELU, :742-744, f32 around an f64 erf);
 *  - layerNormAffine (bert_encoder_layer_ops.go:718-740): f64 mean/variance;
 *  - meanPoolMaskedTensor (tensor_ops.go:1644-1709): f32 sums over active rows
 *    times float32(1/count); count 0 -> zeros;
 *  - normalizeRows (tensor_ops.go:1367-1391): f64 sum of squares, f32 norm,
 *    rows with norm 0 unchanged.
 * Also the tiny embed pipeline of examples/embed.eos (config 1): gather,
 * f32 matmulTensor (tensor_ops.go:1168-1249, f32 accumulate in k order), row
 * L2 normalize.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static void layer_norm_affine(float* x, int rows, int dim, const float* gamma, const float* beta,
                              double eps) {
  for (int r = 0; r < rows; ++r) {
    float* row = x + (size_t)r * dim;
    double mean = 0.0;
    for (int d = 0; d < dim; ++d) mean += (double)row[d];
    mean /= (double)dim;
    double var = 0.0;
    for (int d = 0; d < dim; ++d) {
      const double c = (double)row[d] - mean;
      var += c * c;
    }
    var /= (double)dim;
    const double inv = 1.0 / sqrt(var + eps);
    for (int d = 0; d < dim; ++d)
      row[d] = (float)(((double)row[d] - mean) * inv * (double)gamma[d] + (double)beta[d]);
  }
}

/* out[r][o] = b[o] + sum_c x[r][c] w[o][c] (f64 accumulate); W is [out][in]. */
void dense_hf(const float* x, int rows, int in, const float* w, const float* b, int out,
              float* y) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    for (int o = 0; o < out; ++o) {
      double sum = (double)b[o];
      const float* xr = x + (size_t)r * in;
      const float* wr = w + (size_t)o * in;
      for (int c = 0; c < in; ++c) sum += (double)xr[c] * (double)wr[c];
      y[(size_t)r * out + o] = (float)sum;
    }
  }
}

static inline float exact_gelu(float x) {
  return 0.5f * x * (1.0f + (float)erf((double)x / sqrt(2.0)));
}

void bert_attention(const float* q, const float* k, const float* v, const int32_t* mask,
                    int batch, int tokens, int hidden, int heads, float* ctx) {
  const int hd = hidden / heads;
  const double scale = 1.0 / sqrt((double)hd);
  memset(ctx, 0, sizeof(float) * (size_t)batch * tokens * hidden);
#pragma omp parallel for schedule(dynamic, 16)
  for (long job = 0; job < (long)batch * tokens * heads; ++job) {
    const int head = (int)(job % heads);
    const long qidx = job / heads;
    const int b = (int)(qidx / tokens);
    const int qt = (int)(qidx % tokens);
    const size_t qrow = (size_t)b * tokens + qt;
    double* logits = (double*)malloc(sizeof(double) * (size_t)tokens);
    int active = 0;
    double mx = -INFINITY;
    for (int kt = 0; kt < tokens; ++kt) {
      if (mask[(size_t)b * tokens + kt] == 0) continue;
      active++;
      const size_t krow = (size_t)b * tokens + kt;
      double dot = 0.0;
      for (int d = 0; d < hd; ++d) {
        const int idx = head * hd + d;
        dot += (double)q[qrow * hidden + idx] * (double)k[krow * hidden + idx];
      }
      const double lg = dot * scale;
      logits[kt] = lg;
      if (lg > mx) mx = lg;
    }
    if (active > 0) {
      double sum = 0.0;
      for (int kt = 0; kt < tokens; ++kt) {
        if (mask[(size_t)b * tokens + kt] == 0) continue;
        const double ev = exp(logits[kt] - mx);
        logits[kt] = ev;
        sum += ev;
      }
      for (int kt = 0; kt < tokens; ++kt) {
        if (mask[(size_t)b * tokens + kt] == 0) continue;
        const double p = logits[kt] / sum;
        const size_t vrow = (size_t)b * tokens + kt;
        for (int d = 0; d < hd; ++d) {
          const int idx = head * hd + d;
          ctx[qrow * hidden + idx] += (float)(p * (double)v[vrow * hidden + idx]);
        }
      }
    }
    free(logits);
  }
}

/* One post-LN encoder layer in place on h [batch*tokens][hidden].
 * w: 16 tensors in the reference order (bert_embedder_ops.go:164-178):
 * q_w q_b k_w k_b v_w v_b ao_w ao_b aln_g aln_b i_w i_b o_w o_b oln_g oln_b. */
void bert_layer(float* h, const int32_t* mask, int batch, int tokens, int hidden, int heads,
                int inter, double eps, const float* const* w) {
  const int rows = batch * tokens;
  const size_t rh = (size_t)rows * hidden;
  float* q = (float*)malloc(sizeof(float) * rh);
  float* k = (float*)malloc(sizeof(float) * rh);
  float* v = (float*)malloc(sizeof(float) * rh);
  float* ctx = (float*)malloc(sizeof(float) * rh);
  float* t = (float*)malloc(sizeof(float) * rh);
  float* mid = (float*)malloc(sizeof(float) * (size_t)rows * inter);
  dense_hf(h, rows, hidden, w[0], w[1], hidden, q);
  dense_hf(h, rows, hidden, w[2], w[3], hidden, k);
  dense_hf(h, rows, hidden, w[4], w[5], hidden, v);
  bert_attention(q, k, v, mask, batch, tokens, hidden, heads, ctx);
  dense_hf(ctx, rows, hidden, w[6], w[7], hidden, t);
  for (size_t i = 0; i < rh; ++i) t[i] = t[i] + h[i];
  layer_norm_affine(t, rows, hidden, w[8], w[9], eps);
  dense_hf(t, rows, hidden, w[10], w[11], inter, mid);
  for (size_t i = 0; i < (size_t)rows * inter; ++i) mid[i] = exact_gelu(mid[i]);
  dense_hf(mid, rows, inter, w[12], w[13], hidden, q);
  for (size_t i = 0; i < rh; ++i) h[i] = q[i] + t[i];
  layer_norm_affine(h, rows, hidden, w[14], w[15], eps);
  free(q);
  free(k);
  free(v);
  free(ctx);
  free(t);
  free(mid);
}

void bert_embeddings(const float* tok, int vocab, const float* pos, int npos, const float* typ,
                     int ntype, const float* gamma, const float* beta, const int32_t* ids,
                     const int32_t* type_ids, int batch, int tokens, int hidden, double eps,
                     float* out) {
  (void)vocab;
  (void)npos;
  (void)ntype;
  for (int b = 0; b < batch; ++b) {
    for (int t = 0; t < tokens; ++t) {
      const size_t row = (size_t)b * tokens + t;
      const float* te = tok + (size_t)ids[row] * hidden;
      const float* pe = pos + (size_t)t * hidden;
      const float* ye = typ + (size_t)(type_ids ? type_ids[row] : 0) * hidden;
      for (int d = 0; d < hidden; ++d) out[row * hidden + d] = te[d] + pe[d] + ye[d];
    }
  }
  layer_norm_affine(out, batch * tokens, hidden, gamma, beta, eps);
}

void mean_pool_masked(const float* h, const int32_t* mask, int batch, int tokens, int hidden,
                      float* out) {
  memset(out, 0, sizeof(float) * (size_t)batch * hidden);
  for (int b = 0; b < batch; ++b) {
    int count = 0;
    for (int t = 0; t < tokens; ++t) {
      if (mask[(size_t)b * tokens + t] == 0) continue;
      count++;
      const float* row = h + ((size_t)b * tokens + t) * hidden;
      for (int c = 0; c < hidden; ++c) out[(size_t)b * hidden + c] += row[c];
    }
    if (count == 0) continue;
    const float inv = 1.0f / (float)count;
    for (int c = 0; c < hidden; ++c) out[(size_t)b * hidden + c] *= inv;
  }
}

void normalize_rows(float* x, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    float* row = x + (size_t)r * cols;
    double sum = 0.0;
    for (int c = 0; c < cols; ++c) sum += (double)row[c] * (double)row[c];
    const float norm = (float)sqrt(sum);
    if (norm == 0.0f) continue;
    for (int c = 0; c < cols; ++c) row[c] = row[c] / norm;
  }
}

/* Hidden states after the embeddings and `layers` encoder layers (the state
 * BERTEmbedderReferenceWithPooling pools, bert_embedder_ops.go:155-178):
 * h [batch][tokens][hidden], every position computed (masked ones too). */
void bert_hidden(const float* tok, int vocab, const float* pos, int npos, const float* typ,
                 int ntype, const float* emb_gamma, const float* emb_beta,
                 const float* const* layer_w, int layers, const int32_t* ids,
                 const int32_t* type_ids, const int32_t* mask, int batch, int tokens, int hidden,
                 int heads, int inter, double eps, float* h) {
  bert_embeddings(tok, vocab, pos, npos, typ, ntype, emb_gamma, emb_beta, ids, type_ids, batch,
                  tokens, hidden, eps, h);
  for (int l = 0; l < layers; ++l)
    bert_layer(h, mask, batch, tokens, hidden, heads, inter, eps, layer_w + (size_t)l * 16);
}

/* Full embedder with the step's pooling (bert_embedder_ops.go:179-196):
 * pooling 0 masked_mean (mean over mask != 0 rows, count 0 -> zeros), 1 cls
 * (clsPoolTensor: the row of position 0 whatever the mask), then L2
 * (normalizeRows). out: [batch][hidden]. */
void bert_embed_pool(const float* tok, int vocab, const float* pos, int npos, const float* typ,
                     int ntype, const float* emb_gamma, const float* emb_beta,
                     const float* const* layer_w, int layers, const int32_t* ids,
                     const int32_t* type_ids, const int32_t* mask, int batch, int tokens,
                     int hidden, int heads, int inter, double eps, int pooling, float* out) {
  float* h = (float*)malloc(sizeof(float) * (size_t)batch * tokens * hidden);
  bert_hidden(tok, vocab, pos, npos, typ, ntype, emb_gamma, emb_beta, layer_w, layers, ids,
              type_ids, mask, batch, tokens, hidden, heads, inter, eps, h);
  if (pooling == 1) {
    for (int b = 0; b < batch; ++b)
      memcpy(out + (size_t)b * hidden, h + (size_t)b * tokens * hidden, sizeof(float) * hidden);
  } else {
    mean_pool_masked(h, mask, batch, tokens, hidden, out);
  }
  normalize_rows(out, batch, hidden);
  free(h);
}

/* Full embedder: embeddings, `layers` encoder layers, masked mean pool, L2.
 * layer_w: layers*16 pointers. out: [batch][hidden]. */
void bert_embed(const float* tok, int vocab, const float* pos, int npos, const float* typ,
                int ntype, const float* emb_gamma, const float* emb_beta, const float* const* layer_w,
                int layers, const int32_t* ids, const int32_t* type_ids, const int32_t* mask,
                int batch, int tokens, int hidden, int heads, int inter, double eps, float* out) {
  bert_embed_pool(tok, vocab, pos, npos, typ, ntype, emb_gamma, emb_beta, layer_w, layers, ids,
                  type_ids, mask, batch, tokens, hidden, heads, inter, eps, 0, out);
}

/* Tiny embed (examples/embed.eos): rows = gather(table, ids); y = rows @ proj
 * (f32, k ascending, proj [D][E]); y rows L2-normalized. */
void tiny_embed(const float* table, int vocab, int dim, const float* proj, int edim,
                const int32_t* ids, int n, float* out) {
  (void)vocab;
  for (int i = 0; i < n; ++i) {
    const float* row = table + (size_t)ids[i] * dim;
    for (int e = 0; e < edim; ++e) {
      float acc = 0.0f;
      for (int k = 0; k < dim; ++k) acc += row[k] * proj[(size_t)k * edim + e];
      out[(size_t)i * edim + e] = acc;
    }
  }
  normalize_rows(out, n, edim);
}

/* ------------------------------------------------------------------------
 * Compact transformer embedder (family (a): the shipped default embedder's
 * graph, models/default_embedding.go:419-505), restated step by step in the
 * reference's precisions:
 *  - gather + dequant of q8/q4 token and role rows, summed in f32;
 *  - ropeRows (tensor_ops.go:1936-1965): pairs (c, c+1), theta =
 *    pos / 10000^(c/cols) in f64, cos/sin rounded to f32, f32 rotation,
 *    pos = the row's position inside its padded sequence;
 *  - matmulTensor (tensor_ops.go:1168-1249): [in, out] weights, f32 sum in
 *    k order;
 *  - one head: scaled_attention_scores = (q kT) * float32(1/sqrt(D))
 *    (matmulScale "rsqrt_rhs_rows", tensor_ops.go:1291-1315), then
 *    maskedSoftmaxRowsF32 (tensor_ops.go:1825-1865: f32 max over active
 *    keys, f64 exp and sum, f32 probabilities times float32(1/sum)), then
 *    probs @ v in f32; several heads: compactMultiheadAttentionTensor
 *    (tensor_ops.go:1867-1924) = the BERT f64 attention above;
 *  - layerNormRows (tensor_ops.go:1393-1421): non-affine, f32 mean/variance,
 *    invStd = float32(1/sqrt(f64(var) + 1e-5));
 *  - geluTensor (tensor_ops.go:1926-1934): tanh form, f64 tanh;
 *  - normalizeRows per token, the optional output projection per token,
 *    then meanPoolMaskedTensor.
 * ------------------------------------------------------------------------ */

void rope_rows(float* x, int rows, int seq, int cols) {
  for (int r = 0; r < rows; ++r) {
    const int pos = r % seq;
    for (int c = 0; c + 1 < cols; c += 2) {
      const double theta = (double)pos / pow(10000.0, (double)c / (double)cols);
      const float ct = (float)cos(theta), st = (float)sin(theta);
      const float x0 = x[(size_t)r * cols + c], x1 = x[(size_t)r * cols + c + 1];
      x[(size_t)r * cols + c] = x0 * ct - x1 * st;
      x[(size_t)r * cols + c + 1] = x0 * st + x1 * ct;
    }
  }
}

/* y[r][j] = sum_k x[r][k] w[k][j] (f32, k ascending); W is [in][out]. */
void matmul_f32(const float* x, int rows, int in, const float* w, int out, float* y) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * in;
    for (int j = 0; j < out; ++j) {
      float sum = 0.0f;
      for (int k = 0; k < in; ++k) sum += xr[k] * w[(size_t)k * out + j];
      y[(size_t)r * out + j] = sum;
    }
  }
}

void layer_norm_rows(float* x, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    float* row = x + (size_t)r * cols;
    float mean = 0.0f;
    for (int c = 0; c < cols; ++c) mean += row[c];
    mean /= (float)cols;
    float var = 0.0f;
    for (int c = 0; c < cols; ++c) {
      const float d = row[c] - mean;
      var += d * d;
    }
    var /= (float)cols;
    const float inv = (float)(1.0 / sqrt((double)var + 1e-5));
    for (int c = 0; c < cols; ++c) row[c] = (row[c] - mean) * inv;
  }
}

static inline float tanh_gelu(float x) {
  const float cubic = x * x * x;
  const float inner = 0.7978845608f * (x + 0.044715f * cubic);
  return 0.5f * x * (1.0f + (float)tanh((double)inner));
}

void gelu_tanh_inplace(float* x, long n) {
  for (long i = 0; i < n; ++i) x[i] = tanh_gelu(x[i]);
}

/* Single-head attention of the compact graph on [batch][tokens][dim].
 * scaled != 0: scores times float32(1/sqrt(dim)) (scaled_attention_scores);
 * 0: the plain q kT matmul of a plan's matmul step. A mask of all ones gives
 * softmaxRows (tensor_ops.go:1757-1788: f32 max over every column, f64 exp
 * and sum, f32 probabilities times float32(1/sum)). */
static void compact_single_head_attention_s(const float* q, const float* k, const float* v,
                                            const int32_t* mask, int batch, int tokens, int dim,
                                            int scaled, float* mixed) {
  const float scale = (float)(1.0 / sqrt((double)dim));
#pragma omp parallel for schedule(dynamic, 8)
  for (long job = 0; job < (long)batch * tokens; ++job) {
    const int b = (int)(job / tokens);
    const float* qr = q + (size_t)job * dim;
    const int32_t* mb = mask + (size_t)b * tokens;
    float* p = (float*)malloc(sizeof(float) * (size_t)tokens);
    for (int kt = 0; kt < tokens; ++kt) {
      const float* kr = k + ((size_t)b * tokens + kt) * dim;
      float sum = 0.0f;
      for (int d = 0; d < dim; ++d) sum += qr[d] * kr[d];
      p[kt] = scaled ? sum * scale : sum;
    }
    float mx = -INFINITY;
    int any = 0;
    for (int kt = 0; kt < tokens; ++kt) {
      if (mb[kt] == 0) continue;
      if (!any || p[kt] > mx) mx = p[kt];
      any = 1;
    }
    if (!any) {
      for (int kt = 0; kt < tokens; ++kt) p[kt] = 0.0f;
    } else {
      double s = 0.0;
      for (int kt = 0; kt < tokens; ++kt) {
        if (mb[kt] == 0) {
          p[kt] = 0.0f;
          continue;
        }
        const double ev = exp((double)(p[kt] - mx));
        p[kt] = (float)ev;
        s += ev;
      }
      if (s != 0.0) {
        const float inv = (float)(1.0 / s);
        for (int kt = 0; kt < tokens; ++kt)
          if (mb[kt] != 0) p[kt] *= inv;
      }
    }
    float* out = mixed + (size_t)job * dim;
    for (int d = 0; d < dim; ++d) {
      float sum = 0.0f;
      for (int kt = 0; kt < tokens; ++kt) sum += p[kt] * v[((size_t)b * tokens + kt) * dim + d];
      out[d] = sum;
    }
    free(p);
  }
}

void compact_single_head_attention(const float* q, const float* k, const float* v,
                                   const int32_t* mask, int batch, int tokens, int dim,
                                   float* mixed) {
  compact_single_head_attention_s(q, k, v, mask, batch, tokens, dim, 1, mixed);
}

/* tok [vocab][dim], role [nrole][dim] (dequantized); layer_w: 6 pointers per
 * layer, wq wk wv wo [dim][dim], wup [dim][ffn], wdown [ffn][dim], all
 * [in][out]; wout [dim][odim] or NULL. out: [batch][wout ? odim : dim].
 * flags: 1 = no RoPE; 2 = one head's scores unscaled (a plan's plain q kT
 * matmul); 4 = attention over every position of the padded input
 * (softmaxRows), the mask selecting only the pooled rows. */
void compact_embed_opts(const float* tok, int vocab, const float* role, int nrole,
                        const float* const* layer_w, int layers, const float* wout, int odim,
                        const int32_t* ids, const int32_t* role_ids, const int32_t* mask,
                        int batch, int tokens, int dim, int heads, int ffn, int flags,
                        float* out) {
  (void)vocab;
  (void)nrole;
  const int rows = batch * tokens;
  int32_t* ones = NULL;
  const int32_t* amask = mask;
  if (flags & 4) {
    ones = (int32_t*)malloc(sizeof(int32_t) * (size_t)rows);
    for (int r = 0; r < rows; ++r) ones[r] = 1;
    amask = ones;
  }
  const size_t rd = (size_t)rows * dim;
  float* x = (float*)malloc(sizeof(float) * rd);
  float* q = (float*)malloc(sizeof(float) * rd);
  float* k = (float*)malloc(sizeof(float) * rd);
  float* v = (float*)malloc(sizeof(float) * rd);
  float* mixed = (float*)malloc(sizeof(float) * rd);
  float* t = (float*)malloc(sizeof(float) * rd);
  float* mid = (float*)malloc(sizeof(float) * (size_t)rows * ffn);
  for (int r = 0; r < rows; ++r) {
    const float* te = tok + (size_t)ids[r] * dim;
    const float* re = role + (size_t)(role_ids ? role_ids[r] : 0) * dim;
    for (int c = 0; c < dim; ++c) x[(size_t)r * dim + c] = te[c] + re[c];
  }
  if (!(flags & 1)) rope_rows(x, rows, tokens, dim);
  for (int l = 0; l < layers; ++l) {
    const float* const* w = layer_w + (size_t)l * 6;
    matmul_f32(x, rows, dim, w[0], dim, q);
    matmul_f32(x, rows, dim, w[1], dim, k);
    matmul_f32(x, rows, dim, w[2], dim, v);
    if (heads > 1)
      bert_attention(q, k, v, amask, batch, tokens, dim, heads, mixed);
    else
      compact_single_head_attention_s(q, k, v, amask, batch, tokens, dim, !(flags & 2), mixed);
    matmul_f32(mixed, rows, dim, w[3], dim, t);
    for (size_t i = 0; i < rd; ++i) t[i] = t[i] + x[i];
    layer_norm_rows(t, rows, dim);
    matmul_f32(t, rows, dim, w[4], ffn, mid);
    for (size_t i = 0; i < (size_t)rows * ffn; ++i) mid[i] = tanh_gelu(mid[i]);
    matmul_f32(mid, rows, ffn, w[5], dim, q);
    for (size_t i = 0; i < rd; ++i) x[i] = q[i] + t[i];
    layer_norm_rows(x, rows, dim);
  }
  normalize_rows(x, rows, dim);
  if (wout != NULL) {
    float* y = (float*)malloc(sizeof(float) * (size_t)rows * odim);
    matmul_f32(x, rows, dim, wout, odim, y);
    mean_pool_masked(y, mask, batch, tokens, odim, out);
    free(y);
  } else {
    mean_pool_masked(x, mask, batch, tokens, dim, out);
  }
  free(x);
  free(q);
  free(k);
  free(v);
  free(mixed);
  free(t);
  free(mid);
  free(ones);
}

void compact_embed(const float* tok, int vocab, const float* role, int nrole,
                   const float* const* layer_w, int layers, const float* wout, int odim,
                   const int32_t* ids, const int32_t* role_ids, const int32_t* mask, int batch,
                   int tokens, int dim, int heads, int ffn, float* out) {
  compact_embed_opts(tok, vocab, role, nrole, layer_w, layers, wout, odim, ids, role_ids, mask,
                     batch, tokens, dim, heads, ffn, 0, out);
}
