/* TEST INFRASTRUCTURE ONLY: CPU restatement of the retrieval plan's score
 * ops (checker of the eos_ret_* kernels; never on a product path).
 *
 * Row scores of one query against n document rows, in the reference's own
 * arithmetic and order (runtime/backend/tensor_ops.go):
 *   dotRows       (:1967-1997)  f32 sum += q[c] * x[c], c ascending
 *   cosineRows    (:1999-2057)  f64 dot and squared norms in c order,
 *                               float32(dot / (sqrt(|q|^2) * sqrt(|x|^2))),
 *                               0 when the denominator is 0
 *   l2DistanceRows (:2059-2089) f64 sum of float64(q[c] - x[c])^2 with the
 *                               difference in f32, float32(sqrt(sum))
 * The top-k that follows is topk_scores (tq_oracle.c): score descending,
 * index ascending, as topKTensor's stable sort (:2124-2193). */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

void ret_score_rows(int op, const float* q, const float* docs, int64_t n, int d, float* out) {
  double qn = 0.0;
  for (int c = 0; c < d; ++c) qn += (double)q[c] * (double)q[c];
  for (int64_t r = 0; r < n; ++r) {
    const float* x = docs + (size_t)r * d;
    if (op == 1) {
      float sum = 0.0f;
      for (int c = 0; c < d; ++c) sum += q[c] * x[c];
      out[r] = sum;
    } else if (op == 2) {
      double dot = 0.0, dn = 0.0;
      for (int c = 0; c < d; ++c) {
        const double qv = (double)q[c], xv = (double)x[c];
        dot += qv * xv;
        dn += xv * xv;
      }
      const double denom = sqrt(qn) * sqrt(dn);
      out[r] = denom == 0.0 ? 0.0f : (float)(dot / denom);
    } else {
      double sum = 0.0;
      for (int c = 0; c < d; ++c) {
        const double diff = (double)(q[c] - x[c]);
        sum += diff * diff;
      }
      out[r] = (float)sqrt(sum);
    }
  }
}
