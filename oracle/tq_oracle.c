/*
 * TEST INFRASTRUCTURE ONLY -- the CPU oracle for TurboQuant scoring.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this; the product path never does.
 *
 * Restates, in plain C:
 *  - topTurboQuantRetrievalScoresWithStats / ...Exhaustive
 *    (runtime/retrieval_turboquant.go:1853-1908): per query, score every
 *    document, keep a size-k heap ordered by retrievalScoreBetter
 *    (runtime/retrieval_eval.go:1153-1187: score desc, then id asc), then the
 *    insertion sort slicesSortRetrievalScores (retrieval_turboquant.go:1910-1916);
 *    k <= 0 or k > n means n (:1854-1856);
 *  - the build-defined PrepareQuery / InnerProductPrepared arithmetic of the
 *    scan (the reference's is inside m31labs.dev/turboquant v0.2.1, not vendored):
 *      q' = R q (f64, fma in k order), Qs = rint(q' * (qmax / max|q'|)),
 *      D = sum_j Qs_j C[code_j] (exact int32),
 *      score = ((float)D * alpha) * norm + 0.0f, alpha = (float)((max|q'|/qmax) * s_c);
 *  - the f64 float estimator norm * <R q, s_c C[code]> the integer path
 *    approximates (checked within the stated tolerance, not bit-exact).
 * Built with -ffp-contract=off so that no multiply-add is fused implicitly.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QMAX_LIMIT (127 * 256 + 127)

/* Code j of a row packed low bits first (coordinate j at bits j * bits ..
 * j * bits + bits - 1; a 3-bit code may straddle two bytes). */
static inline unsigned code_at(const uint8_t* row, int j, int bits) {
  const int bit = j * bits, sh = bit & 7;
  unsigned v = (unsigned)row[bit >> 3] >> sh;
  if (sh + bits > 8) v |= (unsigned)row[(bit >> 3) + 1] << (8 - sh);
  return v & ((1u << bits) - 1u);
}

static inline void code_put(uint8_t* row, int j, int bits, unsigned code) {
  const int bit = j * bits, sh = bit & 7;
  row[bit >> 3] |= (uint8_t)(code << sh);
  if (sh + bits > 8) row[(bit >> 3) + 1] |= (uint8_t)(code >> (8 - sh));
}

int tq_qmax(const int8_t* cb, int levels, int d) {
  int cmax = 0;
  for (int v = 0; v < levels; ++v) {
    const int a = abs((int)cb[v]);
    if (a > cmax) cmax = a;
  }
  if (cmax == 0) return QMAX_LIMIT;
  long long lim = 2147483647LL / ((long long)cmax * d) - 128;
  return (int)(lim < QMAX_LIMIT ? lim : QMAX_LIMIT);
}

/* rot: d x d row-major R (NULL = identity). */
void tq_prepare(const float* q, const float* rot, int d, int qmax, float cb_scale, int16_t* qs,
                float* alpha) {
  double* qr = (double*)malloc(sizeof(double) * (size_t)d);
  double maxabs = 0.0;
  for (int j = 0; j < d; ++j) {
    double acc = 0.0;
    if (rot != NULL) {
      for (int k = 0; k < d; ++k) acc = fma((double)rot[(size_t)j * d + k], (double)q[k], acc);
    } else {
      acc = (double)q[j];
    }
    qr[j] = acc;
    if (fabs(acc) > maxabs) maxabs = fabs(acc);
  }
  const double inv = maxabs > 0.0 ? (double)qmax / maxabs : 0.0;
  for (int j = 0; j < d; ++j) {
    double v = rint(qr[j] * inv);
    if (v > qmax) v = qmax;
    if (v < -qmax) v = -qmax;
    qs[j] = (int16_t)v;
  }
  *alpha = maxabs > 0.0 ? (float)((maxabs / (double)qmax) * (double)cb_scale) : 0.0f;
  free(qr);
}

static inline float tq_score(int32_t dot, float alpha, float norm) {
  const float a = (float)dot * alpha;
  const float s = a * norm;
  return s + 0.0f;
}

/* Exact integer dots of one prepared query against n vectors. */
void tq_dots(const int16_t* qs, int d, const uint8_t* codes, int64_t n, int bits,
             const int8_t* cb, int32_t* out) {
  const int row_bytes = (d * bits + 7) / 8;
  for (int64_t i = 0; i < n; ++i) {
    const uint8_t* row = codes + (size_t)i * row_bytes;
    int64_t acc = 0;
    for (int j = 0; j < d; ++j) acc += (int64_t)qs[j] * cb[code_at(row, j, bits)];
    out[i] = (int32_t)acc;
  }
}

/* Scores of nq raw queries against vectors [begin, begin+count). */
void tq_scores(const float* queries, int nq, const float* rot, int d, int bits, const int8_t* cb,
               float cb_scale, const uint8_t* codes, const float* norms, int64_t begin,
               int64_t count, int32_t* dots_out, float* scores_out) {
  const int qmax = tq_qmax(cb, 1 << bits, d);
  const int row_bytes = (d * bits + 7) / 8;
  int16_t* qs = (int16_t*)malloc(sizeof(int16_t) * (size_t)d);
  int32_t* dots = (int32_t*)malloc(sizeof(int32_t) * (size_t)(count > 0 ? count : 1));
  for (int q = 0; q < nq; ++q) {
    float alpha;
    tq_prepare(queries + (size_t)q * d, rot, d, qmax, cb_scale, qs, &alpha);
    tq_dots(qs, d, codes + (size_t)begin * row_bytes, count, bits, cb, dots);
    for (int64_t i = 0; i < count; ++i) {
      if (dots_out) dots_out[(size_t)q * count + i] = dots[i];
      if (scores_out) scores_out[(size_t)q * count + i] = tq_score(dots[i], alpha, norms[begin + i]);
    }
  }
  free(qs);
  free(dots);
}

/* f64 float estimator norm * sum_j (R q)_j * s_c * C[code_j] (no query rounding). */
void tq_scores_f64(const float* queries, int nq, const float* rot, int d, int bits,
                   const int8_t* cb, float cb_scale, const uint8_t* codes, const float* norms,
                   int64_t n, double* out) {
  const int row_bytes = (d * bits + 7) / 8;
  double* qr = (double*)malloc(sizeof(double) * (size_t)d);
  for (int q = 0; q < nq; ++q) {
    const float* x = queries + (size_t)q * d;
    for (int j = 0; j < d; ++j) {
      double acc = 0.0;
      if (rot) {
        for (int k = 0; k < d; ++k) acc += (double)rot[(size_t)j * d + k] * (double)x[k];
      } else {
        acc = x[j];
      }
      qr[j] = acc;
    }
    for (int64_t i = 0; i < n; ++i) {
      const uint8_t* row = codes + (size_t)i * row_bytes;
      double acc = 0.0;
      for (int j = 0; j < d; ++j) acc += qr[j] * (double)cb_scale * (double)cb[code_at(row, j, bits)];
      out[(size_t)q * n + i] = (double)norms[i] * acc;
    }
  }
  free(qr);
}

/* ---------------------------------------------------------------- heap */

typedef struct {
  int64_t id;
  float score;
} scored_t;

/* retrievalScoreBetter (runtime/retrieval_eval.go:1153-1161) on integer ids. */
static inline int better(scored_t a, scored_t b) {
  if (a.score > b.score) return 1;
  if (a.score < b.score) return 0;
  return a.id < b.id;
}

/* Min-heap on "better": the root is the worst kept element (retrieval_eval.go:1163-1187). */
static void sift_down(scored_t* h, int n, int i) {
  for (;;) {
    int w = i;
    const int l = 2 * i + 1, r = l + 1;
    if (l < n && better(h[w], h[l])) w = l;
    if (r < n && better(h[w], h[r])) w = r;
    if (w == i) return;
    scored_t t = h[i];
    h[i] = h[w];
    h[w] = t;
    i = w;
  }
}

static void sift_up(scored_t* h, int i) {
  while (i > 0) {
    const int p = (i - 1) / 2;
    if (!better(h[p], h[i])) return;
    scored_t t = h[i];
    h[i] = h[p];
    h[p] = t;
    i = p;
  }
}

static void heap_offer(scored_t* h, int* len, int k, scored_t s) {
  if (*len < k) {
    h[*len] = s;
    sift_up(h, *len);
    *len += 1;
    return;
  }
  if (better(s, h[0])) {
    h[0] = s;
    sift_down(h, k, 0);
  }
}

/* slicesSortRetrievalScores (retrieval_turboquant.go:1910-1916). */
static void insertion_sort(scored_t* s, int n) {
  for (int i = 1; i < n; ++i)
    for (int j = i; j > 0 && better(s[j], s[j - 1]); --j) {
      scored_t t = s[j];
      s[j] = s[j - 1];
      s[j - 1] = t;
    }
}

/* Per query: prepare, score every document through a per-query byte lookup
 * table (exact: same int32 dots as tq_dots), heap top-k, sort.
 * ids/scores are [nq][kk] with kk = (k <= 0 || k > n) ? n : k; returns kk. */
int64_t tq_topk(const float* queries, int nq, const float* rot, int d, int bits, const int8_t* cb,
                float cb_scale, const uint8_t* codes, const float* norms, int64_t n, int k,
                int64_t* ids, float* scores) {
  const int64_t kk = (k <= 0 || (int64_t)k > n) ? n : k;
  if (kk == 0) return 0;
  const int qmax = tq_qmax(cb, 1 << bits, d);
  const int row_bytes = (d * bits + 7) / 8;
  const int per = 8 / bits;
  int16_t* qs = (int16_t*)malloc(sizeof(int16_t) * (size_t)d);
  int32_t* lut = (int32_t*)malloc(sizeof(int32_t) * (size_t)row_bytes * 256);
  scored_t* heap = (scored_t*)malloc(sizeof(scored_t) * (size_t)kk);
  for (int q = 0; q < nq; ++q) {
    float alpha;
    tq_prepare(queries + (size_t)q * d, rot, d, qmax, cb_scale, qs, &alpha);
    for (int b = 0; b < row_bytes; ++b) {
      for (int byte = 0; byte < 256; ++byte) {
        int32_t acc = 0;
        for (int e = 0; e < per; ++e) {
          const int j = b * per + e;
          if (j < d) acc += (int32_t)qs[j] * cb[(byte >> (e * bits)) & ((1 << bits) - 1)];
        }
        lut[(size_t)b * 256 + byte] = acc;
      }
    }
    int len = 0;
    for (int64_t i = 0; i < n; ++i) {
      const uint8_t* row = codes + (size_t)i * row_bytes;
      int32_t dot = 0;
      for (int b = 0; b < row_bytes; ++b) dot += lut[(size_t)b * 256 + row[b]];
      scored_t s = {i, tq_score(dot, alpha, norms[i])};
      heap_offer(heap, &len, (int)kk, s);
    }
    insertion_sort(heap, len);
    for (int64_t i = 0; i < kk; ++i) {
      ids[(size_t)q * kk + i] = heap[i].id;
      scores[(size_t)q * kk + i] = heap[i].score;
    }
  }
  free(qs);
  free(lut);
  free(heap);
  return kk;
}

/* Reference top-k over an arbitrary score array (exhaustive heap + sort), used
 * to pin the selection itself on hand-built ties. */
int64_t topk_scores(const float* s, int64_t n, int k, int64_t* ids, float* out) {
  const int64_t kk = (k <= 0 || (int64_t)k > n) ? n : k;
  if (kk == 0) return 0;
  scored_t* heap = (scored_t*)malloc(sizeof(scored_t) * (size_t)kk);
  int len = 0;
  for (int64_t i = 0; i < n; ++i) {
    scored_t e = {i, s[i]};
    heap_offer(heap, &len, (int)kk, e);
  }
  insertion_sort(heap, len);
  for (int64_t i = 0; i < kk; ++i) {
    ids[i] = heap[i].id;
    out[i] = heap[i].score;
  }
  free(heap);
  return kk;
}

/* ------------------------------------------------------------- MaxSim
 * Build-defined late interaction over the same per-pair score as the flat
 * scan: for query token i and document vector v, s_iv = tq score; the token's
 * document score is max_v s_iv (the reference child-max,
 * runtime/retrieval_multivector_turboquant.go:746-783 with "max"
 * aggregation, :785-810), and the document score is the sum over the 32
 * token slots (tokens past tq_tokens are zero vectors and contribute +0) as
 * a pairwise tree: at step o = 1, 2, 4, 8, 16 slot i becomes s_i + s_(i^o);
 * slot 0 is the result. With one token this is exactly the child max. */
void tq_maxsim_scores(const float* queries, int nq, int tq_tokens, const float* rot, int d,
                      int bits, const int8_t* cb, float cb_scale, const uint8_t* codes,
                      const float* norms, int64_t ndocs, int doc_len, float* out) {
  const int qmax = tq_qmax(cb, 1 << bits, d);
  const int row_bytes = (d * bits + 7) / 8;
  int16_t* qs = (int16_t*)malloc(sizeof(int16_t) * (size_t)d * 32);
  float alpha[32];
  int32_t* dots = (int32_t*)malloc(sizeof(int32_t) * (size_t)doc_len);
  float* zero = (float*)calloc((size_t)d, sizeof(float));
  for (int q = 0; q < nq; ++q) {
    for (int t = 0; t < 32; ++t) {
      const float* src = t < tq_tokens ? queries + ((size_t)q * tq_tokens + t) * d : zero;
      tq_prepare(src, rot, d, qmax, cb_scale, qs + (size_t)t * d, &alpha[t]);
    }
    for (int64_t doc = 0; doc < ndocs; ++doc) {
      float slot[32];
      for (int t = 0; t < 32; ++t) {
        tq_dots(qs + (size_t)t * d, d, codes + (size_t)doc * doc_len * row_bytes, doc_len, bits, cb,
                dots);
        float m = -INFINITY;
        for (int v = 0; v < doc_len; ++v) {
          const float s = tq_score(dots[v], alpha[t], norms[doc * doc_len + v]);
          if (s > m) m = s;
        }
        slot[t] = m;
      }
      for (int o = 1; o < 32; o <<= 1) {
        float nxt[32];
        for (int t = 0; t < 32; ++t) nxt[t] = slot[t] + slot[t ^ o];
        memcpy(slot, nxt, sizeof(slot));
      }
      out[(size_t)q * ndocs + doc] = slot[0];
    }
  }
  free(qs);
  free(dots);
  free(zero);
}

/* ------------------------------------------------------ parent aggregation
 * topTurboQuantMultiVectorParentScores (runtime/retrieval_multivector_
 * turboquant.go:746-758) for one query vector at a time, on integer ids:
 * parent p owns the corpus vectors [off[p], off[p+1]) (its children). Per
 * parent, the accumulator's add (:769-783) keeps the count, the best child
 * (higher score, then the lower child id) and the 5 best scores in
 * descending order; aggregateMultiVectorParentScores (:785-810) sums the
 * first min(top_n, kept) of them in f64 in that order, divides, subtracts
 * penalty * log1p(count) when the penalty is nonzero, and rounds to f32;
 * topParentScoresFromMap (:890-908) keeps the best k parents under
 * retrievalScoreBetter. Parents without children never enter the map, so
 * kk = min(k, parents with children) (k <= 0 means all of them). Returns kk;
 * ids/scores/best_child/best_child_score are [nq][kk]. */
int64_t tq_parent_topk(const float* queries, int nq, const float* rot, int d, int bits,
                       const int8_t* cb, float cb_scale, const uint8_t* codes, const float* norms,
                       const int64_t* off, int64_t np, int top_n, double penalty, int k,
                       int64_t* ids, float* scores, int64_t* best_child, float* best_child_score) {
  int64_t live = 0;
  for (int64_t p = 0; p < np; ++p) live += off[p + 1] > off[p] ? 1 : 0;
  const int64_t kk = (k <= 0 || (int64_t)k > live) ? live : k;
  if (kk == 0) return 0;
  const int64_t n = off[np];
  float* s = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  float* pscore = (float*)malloc(sizeof(float) * (size_t)np);
  int64_t* pbest = (int64_t*)malloc(sizeof(int64_t) * (size_t)np);
  scored_t* heap = (scored_t*)malloc(sizeof(scored_t) * (size_t)kk);
  for (int q = 0; q < nq; ++q) {
    tq_scores(queries + (size_t)q * d, 1, rot, d, bits, cb, cb_scale, codes, norms, 0, n, NULL, s);
    int len = 0;
    for (int64_t p = 0; p < np; ++p) {
      const int64_t c0 = off[p], c1 = off[p + 1];
      if (c1 <= c0) continue;
      float top[6];
      int kept = 0;
      int64_t bid = -1;
      float bsc = 0.0f;
      for (int64_t c = c0; c < c1; ++c) {
        const float v = s[c];
        if (bid < 0 || v > bsc || (v == bsc && c < bid)) {
          bid = c;
          bsc = v;
        }
        top[kept++] = v;
        for (int i = kept - 1; i > 0 && top[i] > top[i - 1]; --i) {
          const float t = top[i];
          top[i] = top[i - 1];
          top[i - 1] = t;
        }
        if (kept > 5) kept = 5;
      }
      int avail = top_n;
      if (avail <= 0 || avail > kept) avail = kept;
      double sum = 0.0;
      for (int i = 0; i < avail; ++i) sum += (double)top[i];
      double sc = sum / (double)avail;
      if (penalty != 0.0) sc -= penalty * log1p((double)(c1 - c0));
      pscore[p] = (float)sc;
      pbest[p] = bid;
      scored_t e = {p, (float)sc};
      heap_offer(heap, &len, (int)kk, e);
    }
    insertion_sort(heap, len);
    for (int64_t i = 0; i < kk; ++i) {
      const int64_t p = heap[i].id;
      ids[(size_t)q * kk + i] = p;
      scores[(size_t)q * kk + i] = heap[i].score;
      best_child[(size_t)q * kk + i] = pbest[p];
      best_child_score[(size_t)q * kk + i] = s[pbest[p]];
    }
  }
  free(s);
  free(pscore);
  free(pbest);
  free(heap);
  return kk;
}

/* ------------------------------------------------------------- encode
 * Build-defined corpus encoder of the MSE stage (the reference's quantizer,
 * turboquant.IPQuantizer.Quantize, lives in the un-vendored module and is
 * called at runtime/retrieval_turboquant.go:700,708): for each vector x,
 *   u_j  = sum_k R[j][k] x_k          f64, one fma chain in k order (R = I without rotation)
 *   ss   = sum_k x_k^2                f64 fma chain in k order
 *   nrm  = sqrt(ss) (f64), norm = (float)nrm
 *   code_j = argmin_v |u_j - nrm * c_v|, c_v = (double)s_c * (double)C_v,
 *            ties to the lower v (each product and difference rounded once)
 * and the codes are packed low bits first (coordinate j at bit j * bits). */
void tq_encode(const float* x, int64_t n, const float* rot, int d, int bits, const int8_t* cb,
               float cb_scale, uint8_t* codes, float* norms) {
  const int levels = 1 << bits;
  const int row_bytes = (d * bits + 7) / 8;
  double c[16];
  for (int v = 0; v < levels; ++v) c[v] = (double)cb_scale * (double)cb[v];
  double* u = (double*)malloc(sizeof(double) * (size_t)d);
  double nc[16];
  for (int64_t i = 0; i < n; ++i) {
    const float* xi = x + (size_t)i * d;
    double ss = 0.0;
    for (int k = 0; k < d; ++k) ss = fma((double)xi[k], (double)xi[k], ss);
    for (int j = 0; j < d; ++j) {
      if (rot == NULL) {
        u[j] = (double)xi[j];
        continue;
      }
      double acc = 0.0;
      for (int k = 0; k < d; ++k) acc = fma((double)rot[(size_t)j * d + k], (double)xi[k], acc);
      u[j] = acc;
    }
    const double nrm = sqrt(ss);
    norms[i] = (float)nrm;
    for (int v = 0; v < levels; ++v) nc[v] = nrm * c[v];
    uint8_t* row = codes + (size_t)i * row_bytes;
    memset(row, 0, (size_t)row_bytes);
    for (int j = 0; j < d; ++j) {
      int best = 0;
      double bd = fabs(u[j] - nc[0]);
      for (int v = 1; v < levels; ++v) {
        const double dv = fabs(u[j] - nc[v]);
        if (dv < bd) {
          bd = dv;
          best = v;
        }
      }
      code_put(row, j, bits, (unsigned)best);
    }
  }
  free(u);
}

/* ------------------------------------------------------------- QJL stage
 * Build-defined inner-product layout (IPQuantized{MSE, Signs, ResNorm, Norm},
 * runtime/turboquant_bytes.go:14-25 / turboquant_quantized_vector.go; the
 * quantizer itself is in the un-vendored module, called at
 * runtime/retrieval_turboquant.go:700-711), after the published
 * TurboQuant_prod estimator: the MSE stage of tq_encode, then a 1-bit QJL
 * sketch of the residual in the rotated frame:
 *   r_j    = u_j - nrm * c_code_j                        (f64)
 *   ResNorm = (float)(sqrt(sum_j r_j^2) / nrm)           (fma chain; 0 when nrm = 0)
 *   p_i    = sum_j S[i][j] r_j                           (f64 fma chain, j ascending)
 *   sign bit i = p_i >= 0, packed low bit first ((d + 7) / 8 bytes)
 * Scoring: q' = R q, Qs / alpha as tq_prepare; y = S q' (f64 fma chain),
 * Ys = rint(y * qmax2 / max|y|) with qmax2 = min(32767, (2^31 - 1) / d - 1),
 * gamma = max|y| / qmax2, beta = (float)(gamma * sqrt(pi / 2) / d);
 *   D_mse = sum_j Qs_j C[code_j], D_qjl = sum_i Ys_i (2 bit_i - 1)   (exact int32)
 *   score = ((float)D_mse * alpha + ResNorm * ((float)D_qjl * beta)) * Norm
 * (each product and sum rounded to f32 in that order). */
/* QJL query grid limit: |Ys| <= 127 * 256 + 127 (each value splits into an
 * int8 high and low half, Ys = 256 hi + lo, for the int8 MFMA scan) and
 * d * |Ys| < 2^31. */
int tq_qjl_qmax(int d) {
  const long long lim = 2147483647LL / d - 1;
  return (int)(lim < QMAX_LIMIT ? lim : QMAX_LIMIT);
}

void tq_encode_ip(const float* x, int64_t n, const float* rot, const float* qjl, int d, int bits,
                  const int8_t* cb, float cb_scale, uint8_t* codes, uint8_t* signs,
                  float* resnorms, float* norms) {
  const int levels = 1 << bits;
  const int row_bytes = (d * bits + 7) / 8, sign_bytes = (d + 7) / 8;
  tq_encode(x, n, rot, d, bits, cb, cb_scale, codes, norms);
  double c[16];
  for (int v = 0; v < levels; ++v) c[v] = (double)cb_scale * (double)cb[v];
  double* u = (double*)malloc(sizeof(double) * (size_t)d);
  double* r = (double*)malloc(sizeof(double) * (size_t)d);
  for (int64_t i = 0; i < n; ++i) {
    const float* xi = x + (size_t)i * d;
    double ss = 0.0;
    for (int k = 0; k < d; ++k) ss = fma((double)xi[k], (double)xi[k], ss);
    const double nrm = sqrt(ss);
    for (int j = 0; j < d; ++j) {
      if (rot == NULL) {
        u[j] = (double)xi[j];
        continue;
      }
      double acc = 0.0;
      for (int k = 0; k < d; ++k) acc = fma((double)rot[(size_t)j * d + k], (double)xi[k], acc);
      u[j] = acc;
    }
    const uint8_t* row = codes + (size_t)i * row_bytes;
    double rn = 0.0;
    for (int j = 0; j < d; ++j) {
      const int code = (int)code_at(row, j, bits);
      r[j] = u[j] - nrm * c[code];
      rn = fma(r[j], r[j], rn);
    }
    resnorms[i] = nrm > 0.0 ? (float)(sqrt(rn) / nrm) : 0.0f;
    uint8_t* sg = signs + (size_t)i * sign_bytes;
    memset(sg, 0, (size_t)sign_bytes);
    for (int s = 0; s < d; ++s) {
      double p = 0.0;
      for (int j = 0; j < d; ++j) p = fma((double)qjl[(size_t)s * d + j], r[j], p);
      if (p >= 0.0) sg[s >> 3] |= (uint8_t)(1u << (s & 7));
    }
  }
  free(u);
  free(r);
}

void tq_ip_prepare(const float* q, const float* rot, const float* qjl, int d, int qmax,
                   float cb_scale, int16_t* qs, float* alpha, int16_t* ys, float* beta) {
  tq_prepare(q, rot, d, qmax, cb_scale, qs, alpha);
  double* qr = (double*)malloc(sizeof(double) * (size_t)d);
  for (int j = 0; j < d; ++j) {
    double acc = 0.0;
    if (rot != NULL) {
      for (int k = 0; k < d; ++k) acc = fma((double)rot[(size_t)j * d + k], (double)q[k], acc);
    } else {
      acc = (double)q[j];
    }
    qr[j] = acc;
  }
  double* y = (double*)malloc(sizeof(double) * (size_t)d);
  double maxabs = 0.0;
  for (int s = 0; s < d; ++s) {
    double acc = 0.0;
    for (int j = 0; j < d; ++j) acc = fma((double)qjl[(size_t)s * d + j], qr[j], acc);
    y[s] = acc;
    if (fabs(acc) > maxabs) maxabs = fabs(acc);
  }
  const int qmax2 = tq_qjl_qmax(d);
  const double inv = maxabs > 0.0 ? (double)qmax2 / maxabs : 0.0;
  for (int s = 0; s < d; ++s) {
    double v = rint(y[s] * inv);
    if (v > qmax2) v = qmax2;
    if (v < -qmax2) v = -qmax2;
    ys[s] = (int16_t)v;
  }
  const double half_pi = 1.5707963267948966;
  *beta = maxabs > 0.0 ? (float)((maxabs / (double)qmax2) * sqrt(half_pi) / (double)d) : 0.0f;
  free(qr);
  free(y);
}

void tq_ip_scores(const float* queries, int nq, const float* rot, const float* qjl, int d,
                  int bits, const int8_t* cb, float cb_scale, const uint8_t* codes,
                  const uint8_t* signs, const float* resnorms, const float* norms, int64_t n,
                  float* out) {
  const int levels = 1 << bits;
  const int qmax = tq_qmax(cb, levels, d);
  const int row_bytes = (d * bits + 7) / 8, sign_bytes = (d + 7) / 8;
  int16_t* qs = (int16_t*)malloc(sizeof(int16_t) * (size_t)d);
  int16_t* ys = (int16_t*)malloc(sizeof(int16_t) * (size_t)d);
  for (int q = 0; q < nq; ++q) {
    float alpha, beta;
    tq_ip_prepare(queries + (size_t)q * d, rot, qjl, d, qmax, cb_scale, qs, &alpha, ys, &beta);
    for (int64_t i = 0; i < n; ++i) {
      const uint8_t* row = codes + (size_t)i * row_bytes;
      const uint8_t* sg = signs + (size_t)i * sign_bytes;
      int32_t dm = 0, dq = 0;
      for (int j = 0; j < d; ++j) {
        dm += (int32_t)qs[j] * cb[code_at(row, j, bits)];
        dq += ((sg[j >> 3] >> (j & 7)) & 1) ? (int32_t)ys[j] : -(int32_t)ys[j];
      }
      const float t1 = (float)dm * alpha;
      const float t2 = (float)dq * beta;
      const float t3 = resnorms[i] * t2;
      out[(size_t)q * n + i] = (t1 + t3) * norms[i];
    }
  }
  free(qs);
  free(ys);
}
