/* TEST INFRASTRUCTURE ONLY: CPU restatement of the reference's second retrieval
 * stage (f16 rerank of TurboQuant-overfetched candidates), the checker for
 * eos_tq_f16_sidecar / eos_tq_fp16_rerank. Never linked into the product.
 *
 *   oracle_f32_to_half   float32ToHalf        runtime/mll_export.go:1007-1041
 *   oracle_half_to_f32   halfToFloat32        runtime/weight_file.go:461-483
 *   oracle_fp16_rerank   topFP16RerankScores  runtime/retrieval_turboquant.go:1635-1662
 *                        topFP16RerankRescueScores + sortTurboQuantFP16RankedScores
 *                        + applyTurboQuantFP16RerankRescue  :1671-1786
 * Built with -ffp-contract=off: each product and sum is rounded to f32, as Go
 * compiles `s += a * b` for amd64 at its default GOAMD64=v1 (no fused
 * multiply-add). Ids are vector indices; "ID asc/desc" compares them as
 * integers (the reference's string IDs order the same way when they are
 * fixed-width, e.g. d%03d in its rescue fixtures). */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

uint16_t oracle_f32_to_half(float value) {
  uint32_t bits;
  memcpy(&bits, &value, 4);
  const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
  const int exp = (int)((bits >> 23) & 0xffu) - 127 + 15;
  uint32_t mant = bits & 0x7fffffu;
  if (exp <= 0) {
    if (exp < -10) return sign;
    mant |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - exp);
    uint16_t half = (uint16_t)(mant >> shift);
    if ((mant >> (shift - 1)) & 1u) half++;
    return (uint16_t)(sign | half);
  }
  if (exp >= 0x1f) {
    if (mant == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7c00u | (uint16_t)(mant >> 13));
  }
  uint16_t half_exp = (uint16_t)((uint16_t)exp << 10);
  uint16_t half_mant = (uint16_t)(mant >> 13);
  if (mant & 0x00001000u) {
    half_mant++;
    if (half_mant & 0x0400u) {
      half_mant = 0;
      half_exp = (uint16_t)(half_exp + 0x0400u);
      if (half_exp >= 0x7c00u) half_exp = 0x7c00u;
    }
  }
  return (uint16_t)(sign | half_exp | half_mant);
}

float oracle_half_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t mant = h & 0x03ffu, out;
  if (exp == 0) {
    if (mant == 0) {
      out = sign;
    } else {
      uint32_t exp32 = 127 - 15 + 1;
      while ((mant & 0x0400u) == 0) {
        mant <<= 1;
        exp32--;
      }
      mant &= 0x03ffu;
      out = sign | (exp32 << 23) | (mant << 13);
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (mant << 13);
  } else {
    out = sign | ((exp + 127 - 15) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &out, 4);
  return f;
}

void oracle_f32_to_half_n(const float* x, int64_t n, uint16_t* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_half(x[i]);
}

typedef struct {
  int64_t id;
  float score;
  int rank;          /* first-stage rank, 1-based */
  float compact;     /* first-stage score */
} scored_t;

/* retrievalScoreBetter (runtime/retrieval_eval.go:1153-1161). */
static int better(const scored_t* a, const scored_t* b) {
  if (a->score > b->score) return 1;
  if (a->score < b->score) return 0;
  return a->id < b->id;
}

/* sortTurboQuantFP16RankedScores's less (retrieval_turboquant.go:1699-1718). */
static int cmp_fp16_ranked(const void* pa, const void* pb) {
  const scored_t* a = (const scored_t*)pa;
  const scored_t* b = (const scored_t*)pb;
  if (a->score > b->score) return -1;
  if (a->score < b->score) return 1;
  if (a->rank != b->rank) return a->rank < b->rank ? -1 : 1;
  return a->id > b->id ? -1 : (a->id < b->id ? 1 : 0);
}

/* The rescue pool's less (retrieval_turboquant.go:1732-1751). */
static int cmp_rescue_pool(const void* pa, const void* pb) {
  const scored_t* a = (const scored_t*)pa;
  const scored_t* b = (const scored_t*)pb;
  if (a->compact > b->compact) return -1;
  if (a->compact < b->compact) return 1;
  if (a->rank != b->rank) return a->rank < b->rank ? -1 : 1;
  return a->id > b->id ? -1 : (a->id < b->id ? 1 : 0);
}

enum { RESCUE_TOPK = 100, RESCUE_LO = 100, RESCUE_HI = 120, RESCUE_PROMOTE = 5 };

/* applyTurboQuantFP16RerankRescue over ranked[0..m); writes the reordered
 * list to out (m entries). */
void oracle_apply_rescue(const scored_t* ranked, int m, scored_t* out) {
  if (m < RESCUE_HI || m <= RESCUE_TOPK) {
    memcpy(out, ranked, (size_t)m * sizeof(scored_t));
    return;
  }
  scored_t pool[RESCUE_HI - RESCUE_LO + 1];
  int np = 0;
  for (int i = 0; i < m; ++i) {
    const int rank = i + 1;
    if (rank >= RESCUE_LO && rank <= RESCUE_HI) pool[np++] = ranked[i];
  }
  qsort(pool, (size_t)np, sizeof(scored_t), cmp_rescue_pool);
  if (np > RESCUE_PROMOTE) np = RESCUE_PROMOTE;
  unsigned char* seen = (unsigned char*)calloc((size_t)m, 1);
  int o = 0;
  for (int i = 0; i < RESCUE_TOPK; ++i) {
    int promoted = 0;
    for (int r = 0; r < np; ++r) promoted |= pool[r].id == ranked[i].id;
    if (promoted) continue;
    out[o++] = ranked[i];
    seen[i] = 1;
  }
  for (int r = 0; r < np; ++r) {
    int idx = -1;
    for (int i = 0; i < m; ++i)
      if (ranked[i].id == pool[r].id) idx = i;
    if (seen[idx]) continue;
    out[o++] = ranked[idx];
    seen[idx] = 1;
  }
  for (int i = 0; i < m; ++i) {
    if (seen[i]) continue;
    out[o++] = ranked[i];
    seen[i] = 1;
  }
  free(seen);
}

/* One query. Returns the number of results written (<= kk, the k rule of
 * :1636-1638). */
int oracle_fp16_rerank(const float* query, int d, const uint16_t* rows, int64_t n,
                       const int64_t* cand_ids, const float* cand_scores, int c, int k,
                       int rescue, int64_t* out_ids, float* out_scores) {
  int topk = (k <= 0 || k > c) ? c : k;
  scored_t* ranked = (scored_t*)malloc((size_t)(c > 0 ? c : 1) * sizeof(scored_t));
  int m = 0;
  for (int j = 0; j < c; ++j) {
    const int64_t id = cand_ids[j];
    if (id < 0 || id >= n) continue; /* docs[candidate.ID] missing */
    const uint16_t* vec = rows + (size_t)id * (size_t)d;
    float score = 0.0f;
    for (int i = 0; i < d; ++i) score += query[i] * oracle_half_to_f32(vec[i]);
    ranked[m].id = id;
    ranked[m].score = score;
    ranked[m].rank = j + 1;
    ranked[m].compact = cand_scores[j];
    ++m;
  }
  if (rescue) {
    qsort(ranked, (size_t)m, sizeof(scored_t), cmp_fp16_ranked);
    scored_t* out = (scored_t*)malloc((size_t)(m > 0 ? m : 1) * sizeof(scored_t));
    oracle_apply_rescue(ranked, m, out);
    memcpy(ranked, out, (size_t)m * sizeof(scored_t));
    free(out);
  } else {
    /* slicesSortRetrievalScores: insertion sort by retrievalScoreBetter. */
    for (int i = 1; i < m; ++i)
      for (int j = i; j > 0 && better(&ranked[j], &ranked[j - 1]); --j) {
        scored_t t = ranked[j];
        ranked[j] = ranked[j - 1];
        ranked[j - 1] = t;
      }
  }
  if (topk > m) topk = m;
  for (int i = 0; i < topk; ++i) {
    out_ids[i] = ranked[i].id;
    out_scores[i] = ranked[i].score;
  }
  free(ranked);
  return topk;
}

/* ---------------------------------------------------------------------
 * Dense and reconstruct reranks (topDenseRerankScores,
 * topTurboQuantReconstructRerankScores, topTurboQuantMixedWidthRerankScores,
 * retrieval_turboquant.go:1610-1633, 1788-1846): a score per candidate, the
 * candidates outside [0, n) skipped, then the heap + sort of
 * retrievalScoreBetter (score desc, ID asc; with id_rank, the order of the
 * string IDs). */

/* dotRetrievalVectors (retrieval_eval.go:1189-1199) against f32 rows. */
void oracle_dense_scores(const float* query, int d, const float* rows, int64_t n,
                         const int64_t* cand_ids, int c, float* out) {
  for (int j = 0; j < c; ++j) {
    const int64_t id = cand_ids[j];
    if (id < 0 || id >= n) {
      out[j] = 0.0f;
      continue;
    }
    const float* x = rows + (size_t)id * (size_t)d;
    float s = 0.0f;
    for (int i = 0; i < d; ++i) s += query[i] * x[i];
    out[j] = s;
  }
}

/* Code j of a row in the reference row layout: bits j*bits .. j*bits+bits-1
 * of the row, low bits first (a 3-bit code may straddle two bytes). */
static int tq_code_at(const uint8_t* row, int j, int bits) {
  const int bit = j * bits, byte = bit >> 3, sh = bit & 7;
  unsigned v = (unsigned)row[byte] >> sh;
  if (sh + bits > 8) v |= (unsigned)row[byte + 1] << (8 - sh);
  return (int)(v & ((1u << bits) - 1u));
}

/* The dequantized vector of one code-set entry, this build's contract after
 * the published TurboQuant dequantizers (the reference calls the un-vendored
 * module's Dequantize, runtime/retrieval_turboquant.go:1802,1833):
 *   y_j = (double)codebook[code_j], plus, for an inner-product entry
 *         (signs != NULL), coef * z_j with z_j = the f64 sum over i ascending
 *         of (bit_i ? S[i][j] : -S[i][j]) and coef = (sqrt(pi/2) / d) * ResNorm
 *         (TurboQuant_prod's sqrt(pi/2)/d * |r| * S^T sign(S r), with |r| =
 *         ResNorm * Norm and Norm applied below);
 *   x_k = (float)(Norm * acc_k), acc_k the f64 fma chain over j ascending of
 *         R[j][k] * y_j (the inverse rotation R^T y; identity: acc_k = y_k).
 * rot: R row-major (NULL: identity); sketch: S row-major. */
void oracle_tq_dequantize(int d, const float* rot, const uint8_t* row, int bits, float norm,
                          const float* codebook, const uint8_t* sign_row, float resnorm,
                          const float* sketch, float* out) {
  double* y = (double*)malloc(sizeof(double) * (size_t)d);
  for (int j = 0; j < d; ++j) y[j] = (double)codebook[tq_code_at(row, j, bits)];
  if (sign_row != NULL) {
    const double coef = (1.2533141373155003 / (double)d) * (double)resnorm;
    for (int j = 0; j < d; ++j) {
      double z = 0.0;
      for (int i = 0; i < d; ++i) {
        const double s = (double)sketch[(size_t)i * d + j];
        z = ((sign_row[i >> 3] >> (i & 7)) & 1) ? z + s : z - s;
      }
      y[j] = y[j] + coef * z;
    }
  }
  for (int k = 0; k < d; ++k) {
    double acc;
    if (rot != NULL) {
      acc = 0.0;
      for (int j = 0; j < d; ++j) acc = fma((double)rot[(size_t)j * d + k], y[j], acc);
    } else {
      acc = y[k];
    }
    out[k] = (float)((double)norm * acc);
  }
  free(y);
}

/* Reconstruct / mixed-width rerank scores: each candidate's dequantized
 * vector (above) dotted with the query as dotRetrievalVectors does
 * (runtime/retrieval_eval.go:1189-1199: sum += a[i] * b[i] in f32, i
 * ascending, product and sum rounded separately). signs / resnorms / sketch
 * NULL: an MSE-only code set. Candidates outside [0, n) score 0 (skipped by
 * the order). */
void oracle_recon_scores_ip(const float* query, int d, const float* rot, const uint8_t* codes,
                            int bits, const float* norms, const float* codebook,
                            const uint8_t* signs, const float* resnorms, const float* sketch,
                            int64_t n, const int64_t* cand_ids, int c, float* out) {
  const size_t row_bytes = ((size_t)d * bits + 7) / 8, sign_bytes = ((size_t)d + 7) / 8;
  float* x = (float*)malloc(sizeof(float) * (size_t)d);
  for (int j = 0; j < c; ++j) {
    const int64_t id = cand_ids[j];
    if (id < 0 || id >= n) {
      out[j] = 0.0f;
      continue;
    }
    oracle_tq_dequantize(d, rot, codes + (size_t)id * row_bytes, bits, norms[id], codebook,
                         signs != NULL ? signs + (size_t)id * sign_bytes : NULL,
                         resnorms != NULL ? resnorms[id] : 0.0f, sketch, x);
    float s = 0.0f;
    for (int k = 0; k < d; ++k) s += query[k] * x[k];
    out[j] = s;
  }
  free(x);
}

void oracle_recon_scores(const float* query, int d, const float* rot, const uint8_t* codes,
                         int bits, const float* norms, const float* codebook, int64_t n,
                         const int64_t* cand_ids, int c, float* out) {
  oracle_recon_scores_ip(query, d, rot, codes, bits, norms, codebook, NULL, NULL, NULL, n,
                         cand_ids, c, out);
}

/* Order the scored candidates (insertion sort by score desc, tie key asc:
 * id_rank[id] when given, else id) and keep the first kk; returns the count. */
int oracle_rerank_order(const float* scores, const int64_t* cand_ids, int64_t n, int c, int k,
                        const int64_t* id_rank, int64_t* out_ids, float* out_scores) {
  int topk = (k <= 0 || k > c) ? c : k;
  scored_t* ranked = (scored_t*)malloc((size_t)(c > 0 ? c : 1) * sizeof(scored_t));
  int64_t* key = (int64_t*)malloc((size_t)(c > 0 ? c : 1) * sizeof(int64_t));
  int m = 0;
  for (int j = 0; j < c; ++j) {
    const int64_t id = cand_ids[j];
    if (id < 0 || id >= n) continue;
    ranked[m].id = id;
    ranked[m].score = scores[j];
    key[m] = id_rank != NULL ? id_rank[id] : id;
    ++m;
  }
  for (int i = 1; i < m; ++i)
    for (int j = i; j > 0; --j) {
      const int swap = ranked[j].score > ranked[j - 1].score ||
                       (ranked[j].score == ranked[j - 1].score && key[j] < key[j - 1]);
      if (!swap) break;
      scored_t t = ranked[j];
      ranked[j] = ranked[j - 1];
      ranked[j - 1] = t;
      const int64_t tk = key[j];
      key[j] = key[j - 1];
      key[j - 1] = tk;
    }
  if (topk > m) topk = m;
  for (int i = 0; i < topk; ++i) {
    out_ids[i] = ranked[i].id;
    out_scores[i] = ranked[i].score;
  }
  free(ranked);
  free(key);
  return topk;
}
