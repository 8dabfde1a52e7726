// Retrieval-plan kernels on gfx950: the row scores of a plan's
// dot / cosine / l2_distance step for every (query, document) pair, and the
// gathers that follow its topk step (candidate ids, document rows).
//
// Each score is computed by one thread in the reference's own arithmetic and
// order, so scores are bit-identical to the host ops (dotRows, cosineRows,
// l2DistanceRows, runtime/backend/tensor_ops.go:1967-2122):
//   dot     f32 sum += q[c] * x[c], c ascending, multiply and add rounded
//           separately
//   cosine  f64 dot and squared norms in c order, f64 sqrt of each norm,
//           dot / (|q| |x|) rounded to f32 (0 when the denominator is 0)
//   l2      f64 sum of (double)(q[c] - x[c])^2 (difference in f32), f64 sqrt
// q4 document values decode as (float)(nibble - 8) * scale in f32
// (decodeTensorEntry, runtime/weight_file.go:333-351). The top-k itself is
// the exact radix selection of the TurboQuant code object (score desc, index
// asc, topKTensor's order, tensor_ops.go:2124-2193).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ret_args.h"

#define EOS_DEV __device__ __forceinline__

namespace {

// Flat element i of the document tensor.
EOS_DEV float doc_value(const RetScoreArgs& a, long long i) {
  if (a.docs_q4 == nullptr) return a.docs[i];
  const int nib = (a.docs_q4[i >> 1] >> ((int)(i & 1) * 4)) & 15;
  return __fmul_rn((float)(nib - 8), a.scale);
}

}  // namespace

// Grid (ceil(n / 256), q); one document row per thread.
extern "C" __global__ __launch_bounds__(kRetThreads) void eos_ret_score(RetScoreArgs a) {
  __shared__ float qs[kRetMaxDim];
  __shared__ double qnorm;
  const int qi = blockIdx.y;
  const int tid = threadIdx.x;
  for (int c = tid; c < a.d; c += kRetThreads) qs[c] = a.queries[(size_t)qi * a.d + c];
  __syncthreads();
  if (a.op == 2 && tid == 0) {
    double s = 0.0;
    for (int c = 0; c < a.d; ++c) {
      const double v = (double)qs[c];
      s = __dadd_rn(s, __dmul_rn(v, v));
    }
    qnorm = s;
  }
  __syncthreads();
  const long long r = (long long)blockIdx.x * kRetThreads + tid;
  if (r >= a.n) return;
  const long long base = ((a.batched ? (long long)qi * a.n : 0ll) + r) * a.d;
  float out;
  if (a.op == 1) {
    float sum = 0.0f;
    if (a.docs_q4 == nullptr && (a.d & 3) == 0) {
      const float4* row = reinterpret_cast<const float4*>(a.docs + base);
      for (int c4 = 0; c4 < a.d / 4; ++c4) {
        const float4 x = row[c4];
        sum = __fadd_rn(sum, __fmul_rn(qs[4 * c4], x.x));
        sum = __fadd_rn(sum, __fmul_rn(qs[4 * c4 + 1], x.y));
        sum = __fadd_rn(sum, __fmul_rn(qs[4 * c4 + 2], x.z));
        sum = __fadd_rn(sum, __fmul_rn(qs[4 * c4 + 3], x.w));
      }
    } else {
      for (int c = 0; c < a.d; ++c) sum = __fadd_rn(sum, __fmul_rn(qs[c], doc_value(a, base + c)));
    }
    out = sum;
  } else if (a.op == 2) {
    double dot = 0.0, dn = 0.0;
    for (int c = 0; c < a.d; ++c) {
      const double q = (double)qs[c];
      const double x = (double)doc_value(a, base + c);
      dot = __dadd_rn(dot, __dmul_rn(q, x));
      dn = __dadd_rn(dn, __dmul_rn(x, x));
    }
    const double denom = __dmul_rn(__dsqrt_rn(qnorm), __dsqrt_rn(dn));
    out = denom == 0.0 ? 0.0f : __double2float_rn(__ddiv_rn(dot, denom));
  } else {
    double sum = 0.0;
    for (int c = 0; c < a.d; ++c) {
      const double diff = (double)__fsub_rn(qs[c], doc_value(a, base + c));
      sum = __dadd_rn(sum, __dmul_rn(diff, diff));
    }
    out = __double2float_rn(__dsqrt_rn(sum));
  }
  // -0 ranks like +0 in the reference's comparisons; the selection keys on
  // bits, so zeros are made +0.
  a.scores[(size_t)qi * a.n + r] = out == 0.0f ? 0.0f : out;
}

// Grid (k, q): one workgroup per selected candidate.
extern "C" __global__ __launch_bounds__(kRetThreads) void eos_ret_gather(RetGatherArgs a) {
  const int j = blockIdx.x, qi = blockIdx.y;
  const long long r = a.sel[(size_t)qi * a.k + j];
  const long long brow = a.batched ? (long long)qi * a.n : 0ll;
  if (threadIdx.x == 0) {
    if (a.top_index != nullptr) a.top_index[(size_t)qi * a.k + j] = (int32_t)r;
    if (a.top_ids != nullptr)
      a.top_ids[(size_t)qi * a.k + j] = a.cand_ids != nullptr ? a.cand_ids[brow + r] : (int64_t)r;
  }
  if (a.top_docs == nullptr) return;
  float* dst = a.top_docs + ((size_t)qi * a.k + j) * a.d;
  const long long base = (brow + r) * a.d;
  for (int c = threadIdx.x; c < a.d; c += kRetThreads) {
    const long long i = base + c;
    float v;
    if (a.docs_q4 == nullptr) {
      v = a.docs[i];
    } else {
      const int nib = (a.docs_q4[i >> 1] >> ((int)(i & 1) * 4)) & 15;
      v = __fmul_rn((float)(nib - 8), a.scale);
    }
    dst[c] = v;
  }
}

// ------------------------------------------------------ Hadamard TurboQuant

// The Hadamard TurboQuant codec of NCHW tensors (turboquant_encode /
// turboquant_decode steps; host runtime/backend/image_ops.go:212-300, CUDA
// runtime/backends/cuda/native_linux.go:1812-2004). One thread per pixel
// vector (consecutive threads read consecutive pixels of a channel, so every
// channel load is coalesced); its working vector lives in an LDS column
// work[i * 64 + thread]. Arithmetic, in f32 unless noted:
//   encode  normSq = fma chain over c ascending; norm = sqrt; scale = 1/norm
//           (1 when norm <= 1e-12); work[i] = x[perm[i]] * scale * signs1[i];
//           normalized FWHT on power-of-two blocks from the front (largest
//           power <= remaining), butterflies (a + b, a - b), block scale
//           float(1/sqrt(size)); coord[perm[i]] = index of the first boundary
//           > work[i] * signs2[i] (levels - 1 when none); norm code = the
//           8-bit log code of quantizeQNorm (image_ops.go:759-775: f64 log,
//           t = (log(norm) + 16) / 32, round half away from zero of t * 255)
//   decode  work[i] = centroids[coord[perm[i]]] * signs2[i]; the same FWHT;
//           out[perm[i]] = work[i] * signs1[i] * norm, norm =
//           float(exp(-16 + code / 255 * 32)) in f64 (dequantizeQNorm, :777-780)
namespace {

EOS_DEV void hq_fwht_blocks(float* work, int channels, int t) {
  int offset = 0, remaining = channels;
  while (remaining > 0) {
    int size = 1;
    while ((size << 1) <= remaining) size <<= 1;
    for (int step = 1; step < size; step <<= 1)
      for (int i = 0; i < size; i += step << 1)
        for (int j = i; j < i + step; ++j) {
          const float a = work[(offset + j) * kHqThreads + t];
          const float b = work[(offset + j + step) * kHqThreads + t];
          work[(offset + j) * kHqThreads + t] = __fadd_rn(a, b);
          work[(offset + j + step) * kHqThreads + t] = __fsub_rn(a, b);
        }
    if (size > 1) {
      const float scale = __double2float_rn(1.0 / __dsqrt_rn((double)size));
      for (int i = 0; i < size; ++i)
        work[(offset + i) * kHqThreads + t] = __fmul_rn(work[(offset + i) * kHqThreads + t], scale);
    }
    offset += size;
    remaining -= size;
  }
}

EOS_DEV int hq_norm_code(float norm) {
  if (!(norm > 0.0f)) return 0;  // <= 0 or NaN
  if (__builtin_isinf(norm)) return 255;
  const double t = (log((double)norm) + 16.0) / 32.0;
  if (t <= 0.0) return 0;
  if (t >= 1.0) return 255;
  return (int)round(t * 255.0);
}

}  // namespace

// Dynamic LDS: channels * 64 floats.
extern "C" __global__ __launch_bounds__(kHqThreads) void eos_hq_encode(HqArgs a) {
  extern __shared__ float work[];
  const int t = threadIdx.x;
  const long long pix = (long long)blockIdx.x * kHqThreads + t;
  if (pix >= a.pixels) return;
  const long long img = pix / a.hw, p = pix % a.hw;
  const float* x = a.input + img * (long long)a.channels * a.hw + p;
  float normSq = 0.0f;
  for (int c = 0; c < a.channels; ++c) {
    const float v = x[(long long)c * a.hw];
    normSq = __fmaf_rn(v, v, normSq);
  }
  const float norm = __fsqrt_rn(normSq);
  const float scale = norm > 1.0e-12f ? __fdiv_rn(1.0f, norm) : 1.0f;
  for (int i = 0; i < a.channels; ++i) {
    const float v = x[(long long)a.perm[i] * a.hw];
    work[i * kHqThreads + t] = __fmul_rn(__fmul_rn(v, scale), a.signs1[i]);
  }
  hq_fwht_blocks(work, a.channels, t);
  uint8_t* coords = a.coords + img * (long long)a.channels * a.hw + p;
  for (int i = 0; i < a.channels; ++i) {
    const float r = __fmul_rn(work[i * kHqThreads + t], a.signs2[i]);
    int lo = 0, hi = a.levels - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (a.boundaries[mid] > r) hi = mid;
      else lo = mid + 1;
    }
    coords[(long long)a.perm[i] * a.hw] = (uint8_t)lo;
  }
  a.norms[pix] = (uint8_t)hq_norm_code(norm);
}

extern "C" __global__ __launch_bounds__(kHqThreads) void eos_hq_decode(HqArgs a) {
  extern __shared__ float work[];
  const int t = threadIdx.x;
  const long long pix = (long long)blockIdx.x * kHqThreads + t;
  if (pix >= a.pixels) return;
  const long long img = pix / a.hw, p = pix % a.hw;
  const uint8_t* coords = a.coords_in + img * (long long)a.channels * a.hw + p;
  for (int i = 0; i < a.channels; ++i) {
    int idx = coords[(long long)a.perm[i] * a.hw];
    idx = idx < a.levels ? idx : a.levels - 1;
    work[i * kHqThreads + t] = __fmul_rn(a.centroids[idx], a.signs2[i]);
  }
  hq_fwht_blocks(work, a.channels, t);
  const double tt = (double)a.norms_in[pix] / 255.0;
  const float norm = __double2float_rn(exp(-16.0 + tt * 32.0));
  float* out = a.out + img * (long long)a.channels * a.hw + p;
  for (int i = 0; i < a.channels; ++i)
    out[(long long)a.perm[i] * a.hw] =
        __fmul_rn(__fmul_rn(work[i * kHqThreads + t], a.signs1[i]), norm);
}
