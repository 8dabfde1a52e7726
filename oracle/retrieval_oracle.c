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
#include <stdlib.h>
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

/* ---------------------------------------------------------------------
 * Hadamard TurboQuant codec (checker of eos_hq_encode / eos_hq_decode):
 * the CUDA kernels' arithmetic (runtime/backends/cuda/native_linux.go:
 * 1812-2004; NVRTC's default contracts normSq += v * v into a fused
 * multiply-add) with the host's 8-bit log norm code (quantizeQNorm /
 * dequantizeQNorm, runtime/backend/image_ops.go:759-780, f64 log and exp,
 * round half away from zero). The FWHT block scale is the correctly rounded
 * float(1 / sqrt(size)). */

static void hq_fwht_blocks(float* v, int channels) {
  int offset = 0, remaining = channels;
  while (remaining > 0) {
    int size = 1;
    while ((size << 1) <= remaining) size <<= 1;
    float* b = v + offset;
    for (int step = 1; step < size; step <<= 1)
      for (int i = 0; i < size; i += step << 1)
        for (int j = i; j < i + step; ++j) {
          const float x = b[j], y = b[j + step];
          b[j] = x + y;
          b[j + step] = x - y;
        }
    if (size > 1) {
      const float scale = (float)(1.0 / sqrt((double)size));
      for (int i = 0; i < size; ++i) b[i] = b[i] * scale;
    }
    offset += size;
    remaining -= size;
  }
}

void hq_fwht(float* v, int channels) { hq_fwht_blocks(v, channels); }

int hq_norm_code(float norm) {
  if (!(norm > 0.0f)) return 0;
  if (isinf(norm)) return 255;
  const double t = (log((double)norm) + 16.0) / 32.0;
  if (t <= 0.0) return 0;
  if (t >= 1.0) return 255;
  return (int)round(t * 255.0);
}

float hq_norm_value(int code) { return (float)exp(-16.0 + ((double)code / 255.0) * 32.0); }

void hq_encode(const float* input, int n, int channels, int hw, const int32_t* perm,
               const float* s1, const float* s2, const float* boundaries, int levels,
               uint8_t* coords, uint8_t* norms) {
  float* work = (float*)malloc(sizeof(float) * (size_t)channels);
  for (int img = 0; img < n; ++img)
    for (int p = 0; p < hw; ++p) {
      const float* x = input + (size_t)img * channels * hw + p;
      float normSq = 0.0f;
      for (int c = 0; c < channels; ++c) normSq = fmaf(x[(size_t)c * hw], x[(size_t)c * hw], normSq);
      const float norm = sqrtf(normSq);
      const float scale = norm > 1.0e-12f ? 1.0f / norm : 1.0f;
      for (int i = 0; i < channels; ++i) work[i] = x[(size_t)perm[i] * hw] * scale * s1[i];
      hq_fwht_blocks(work, channels);
      uint8_t* co = coords + (size_t)img * channels * hw + p;
      for (int i = 0; i < channels; ++i) {
        const float r = work[i] * s2[i];
        int lo = 0, hi = levels - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (boundaries[mid] > r) hi = mid;
          else lo = mid + 1;
        }
        co[(size_t)perm[i] * hw] = (uint8_t)lo;
      }
      norms[(size_t)img * hw + p] = (uint8_t)hq_norm_code(norm);
    }
  free(work);
}

void hq_decode(const uint8_t* coords, const uint8_t* norms, int n, int channels, int hw,
               const int32_t* perm, const float* s1, const float* s2, const float* centroids,
               int levels, float* out) {
  float* work = (float*)malloc(sizeof(float) * (size_t)channels);
  for (int img = 0; img < n; ++img)
    for (int p = 0; p < hw; ++p) {
      const uint8_t* co = coords + (size_t)img * channels * hw + p;
      for (int i = 0; i < channels; ++i) {
        int idx = co[(size_t)perm[i] * hw];
        if (idx >= levels) idx = levels - 1;
        work[i] = centroids[idx] * s2[i];
      }
      hq_fwht_blocks(work, channels);
      const float norm = hq_norm_value(norms[(size_t)img * hw + p]);
      float* o = out + (size_t)img * channels * hw + p;
      for (int i = 0; i < channels; ++i) o[(size_t)perm[i] * hw] = work[i] * s1[i] * norm;
    }
  free(work);
}
