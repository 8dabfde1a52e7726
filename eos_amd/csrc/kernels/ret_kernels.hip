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
