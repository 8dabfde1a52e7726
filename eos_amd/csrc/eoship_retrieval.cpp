// Retrieval-plan half of the C ABI: row scores of a dot / cosine /
// l2_distance step, the plan's topk and the gathers after it
// (runtime/retrieval.go:51-112 runs these plans; examples/retrieve.eos,
// candidates.eos, packed_candidates.eos, batch_candidates.eos).
//   eos_ret_score       one thread per (query, document row), the reference's
//                       arithmetic and order (bit-identical scores)
//   eos_tq_row_select   exact top-k by (score desc, index asc)
//   eos_ret_gather      selected indices -> candidate ids and document rows
#include <cmath>
#include <cstring>
#include <vector>

#include "eoship_internal.h"
#include "kernels/ret_args.h"
#include "kernels/tq_args.h"

using eoship::set_err;

namespace eoship {

int score_topk_launch(Runtime* rt, const EosHipScoreSpec& s, const float* d_queries, int32_t q,
                      int32_t d, const float* d_docs, const uint8_t* d_docs_q4, int64_t n,
                      const int64_t* d_candidate_ids, float* d_scores, int32_t* d_top_index,
                      int64_t* d_top_ids, float* d_top_scores, float* d_top_docs,
                      const char* what, char** err) {
  if (s.op < EOSHIP_SCORE_DOT || s.op > EOSHIP_SCORE_L2)
    return set_err(err, "%s: op must be EOSHIP_SCORE_DOT, _COSINE or _L2 (got %d)", what, s.op);
  if (q < 0 || d <= 0 || d > kRetMaxDim || n <= 0)
    return set_err(err, "%s: need q >= 0, 1 <= d <= %d and n >= 1 (q %d, d %d, n %lld)", what,
                   kRetMaxDim, q, d, (long long)n);
  if (n > 0x7fffffffll) return set_err(err, "%s: n above 2^31 - 1 rows", what);
  if (s.batched != 0 && s.batched != 1) return set_err(err, "%s: batched must be 0 or 1", what);
  if ((d_docs == nullptr) == (d_docs_q4 == nullptr))
    return set_err(err, "%s: exactly one of f32 and q4 documents is needed", what);
  if (d_docs_q4 != nullptr && (!(s.docs_scale >= 0.f) || std::isinf(s.docs_scale)))
    return set_err(err, "%s: docs_scale must be finite and >= 0", what);
  if (d_queries == nullptr || d_scores == nullptr)
    return set_err(err, "%s: NULL queries or scores", what);
  if (s.k < 0) return set_err(err, "%s: k must be >= 0", what);
  if (s.k == 0 && (d_top_index || d_top_ids || d_top_scores || d_top_docs))
    return set_err(err, "%s: top-k outputs need k >= 1", what);
  if (s.k > 0 && (long long)s.k > n)
    return set_err(err, "%s: topk limit %d out of range for %lld scores", what, s.k, (long long)n);
  if (s.k > 8192) return set_err(err, "%s: k above 8192 is not supported", what);
  if (q == 0) return 0;
  if ((d_docs != nullptr && (reinterpret_cast<uintptr_t>(d_docs) & 15) != 0))
    return set_err(err, "%s: f32 documents must be 16-byte aligned", what);
  RetScoreArgs sa{d_queries, d_docs, d_docs_q4, s.docs_scale, d_scores, (long long)n, d, q,
                  s.batched, s.op};
  const unsigned gx = (unsigned)((n + kRetThreads - 1) / kRetThreads);
  if (rt->launch("eos_ret_score", dim3(gx, (unsigned)q), dim3(kRetThreads), 0, &sa, err,
                 "ret_score") != 0)
    return 1;
  if (s.k == 0) return 0;
  // Selected indices (and the scores when the caller takes none) in the
  // runtime workspace.
  const size_t kq = (size_t)q * (size_t)s.k;
  void* ws = nullptr;
  if (rt->workspace(kq * 8 + (d_top_scores == nullptr ? kq * 4 : 0), &ws, err) != 0) return 1;
  long long* sel = static_cast<long long*>(ws);
  float* sel_scores = d_top_scores != nullptr ? d_top_scores
                                              : reinterpret_cast<float*>(sel + kq);
  TqSelectArgs sel_args;
  std::memset(&sel_args, 0, sizeof(sel_args));
  sel_args.rows = d_scores;
  sel_args.ids = sel;
  sel_args.scores = sel_scores;
  sel_args.n = n;
  sel_args.stride = n;
  sel_args.kk = s.k;
  sel_args.mode = 1;
  sel_args.nrows = q;
  if (rt->launch("eos_tq_row_select", dim3((unsigned)q), dim3(1024), 0, &sel_args, err,
                 "ret_topk") != 0)
    return 1;
  if (d_top_index == nullptr && d_top_ids == nullptr && d_top_docs == nullptr) return 0;
  RetGatherArgs ga{sel, d_candidate_ids, d_docs, d_docs_q4, s.docs_scale, d_top_index, d_top_ids,
                   d_top_docs, (long long)n, d, q, s.k, s.batched};
  return rt->launch("eos_ret_gather", dim3((unsigned)s.k, (unsigned)q), dim3(kRetThreads), 0, &ga,
                    err, "ret_gather");
}

}  // namespace eoship

extern "C" {

int eoship_score_topk_device(EosHipRuntime* rt, const EosHipScoreSpec* spec,
                             const float* d_queries, int32_t q, int32_t d, const void* d_docs,
                             int64_t n, const int64_t* d_candidate_ids, float* d_scores,
                             int32_t* d_top_index, int64_t* d_top_ids, float* d_top_scores,
                             float* d_top_docs, char** err) {
  const char* what = "eoship_score_topk_device";
  if (rt == nullptr || spec == nullptr || d_docs == nullptr)
    return set_err(err, "%s: NULL argument", what);
  if (spec->docs_q4 != 0 && spec->docs_q4 != 1) return set_err(err, "%s: docs_q4 must be 0 or 1", what);
  const float* f = spec->docs_q4 ? nullptr : static_cast<const float*>(d_docs);
  const uint8_t* p = spec->docs_q4 ? static_cast<const uint8_t*>(d_docs) : nullptr;
  return eoship::score_topk_launch(rt, *spec, d_queries, q, d, f, p, n, d_candidate_ids,
                                   d_scores, d_top_index, d_top_ids, d_top_scores, d_top_docs,
                                   what, err);
}

int eoship_retrieval_run_device(EosHipRuntime* rt, EosHipRetrieval* ret, const float* d_queries,
                                int32_t q, int32_t d, const float* d_docs, int64_t n,
                                const int64_t* d_candidate_ids, float* d_scores,
                                int32_t* d_top_index, int64_t* d_top_ids, float* d_top_scores,
                                float* d_top_docs, char** err) {
  const char* what = "eoship_retrieval_run_device";
  if (rt == nullptr || ret == nullptr) return set_err(err, "%s: NULL argument", what);
  if (ret->rt != rt) return set_err(err, "%s: the plan is bound to another runtime", what);
  EosHipScoreSpec s = ret->spec;
  const float* docs = d_docs;
  const uint8_t* docs_q4 = nullptr;
  if (ret->docs_param) {
    if (d_docs != nullptr) return set_err(err, "%s: documents are the bound param; pass NULL", what);
    if (d != ret->dim) return set_err(err, "%s: d %d differs from the bound documents' %d", what, d, ret->dim);
    n = ret->rows;
    docs = ret->docs_f32;
    docs_q4 = ret->docs_q4;
    s.batched = 0;
  } else if (d_docs == nullptr) {
    return set_err(err, "%s: NULL documents", what);
  }
  if (ret->has_ids && d_top_ids != nullptr && d_candidate_ids == nullptr)
    return set_err(err, "%s: the plan gathers candidate ids; pass them", what);
  return eoship::score_topk_launch(rt, s, d_queries, q, d, docs, docs_q4, n,
                                   ret->has_ids ? d_candidate_ids : nullptr, d_scores,
                                   d_top_index, d_top_ids, d_top_scores, d_top_docs, what, err);
}

int eoship_retrieval_release(EosHipRuntime* rt, EosHipRetrieval* ret, char** err) {
  if (ret == nullptr) return 0;
  if (rt == nullptr || ret->rt != rt) return set_err(err, "eoship_retrieval_release: wrong runtime");
  if (rt->sync(err) != 0) return 1;
  if (ret->docs_f32) (void)hipFree(ret->docs_f32);
  if (ret->docs_q4) (void)hipFree(ret->docs_q4);
  delete ret;
  return 0;
}

// ------------------------------------------------ Hadamard TurboQuant codec

int eoship_hadamard_tq_bind(EosHipRuntime* rt, const EosHipHadamardSpec* spec,
                            EosHipHadamardTQ** out, char** err) {
  const char* what = "eoship_hadamard_tq_bind";
  if (rt == nullptr || spec == nullptr || out == nullptr) return set_err(err, "%s: NULL argument", what);
  *out = nullptr;
  const int c = spec->channels, bits = spec->bits;
  if (c < 1 || c > kHqMaxChannels)
    return set_err(err, "%s: channels must be in 1..%d (got %d)", what, kHqMaxChannels, c);
  if (bits != 2 && bits != 4 && bits != 8)
    return set_err(err, "%s: turboquant bits must be 2, 4, or 8", what);
  if (!spec->perm || !spec->signs1 || !spec->signs2 || !spec->centroids || !spec->boundaries)
    return set_err(err, "%s: NULL table", what);
  const int levels = 1 << bits;
  std::vector<char> seen((size_t)c, 0);
  for (int i = 0; i < c; ++i) {
    const int p = spec->perm[i];
    if (p < 0 || p >= c || seen[(size_t)p]) return set_err(err, "%s: perm is not a permutation of 0..%d", what, c - 1);
    seen[(size_t)p] = 1;
    if (!std::isfinite(spec->signs1[i]) || !std::isfinite(spec->signs2[i]))
      return set_err(err, "%s: signs must be finite", what);
  }
  for (int i = 0; i < levels; ++i)
    if (!std::isfinite(spec->centroids[i])) return set_err(err, "%s: centroids must be finite", what);
  for (int i = 0; i + 1 < levels; ++i) {
    if (std::isnan(spec->boundaries[i])) return set_err(err, "%s: NaN boundary", what);
    if (i > 0 && spec->boundaries[i] < spec->boundaries[i - 1])
      return set_err(err, "%s: boundaries must be non-decreasing", what);
  }
  auto* h = new EosHipHadamardTQ();
  h->rt = rt;
  h->channels = c;
  h->levels = levels;
  const size_t tb = (size_t)c * 4 * 3 + (size_t)levels * 4 * 2;
  void* mem = nullptr;
  if (rt->alloc(tb, &mem, err) != 0) {
    delete h;
    return 1;
  }
  h->tables = mem;
  char* p = static_cast<char*>(mem);
  h->perm = reinterpret_cast<int32_t*>(p);
  h->signs1 = reinterpret_cast<float*>(p + (size_t)c * 4);
  h->signs2 = reinterpret_cast<float*>(p + (size_t)c * 8);
  h->centroids = reinterpret_cast<float*>(p + (size_t)c * 12);
  h->boundaries = h->centroids + levels;
  struct Part {
    void* dst;
    const void* src;
    size_t bytes;
  } parts[] = {{h->perm, spec->perm, (size_t)c * 4},
               {h->signs1, spec->signs1, (size_t)c * 4},
               {h->signs2, spec->signs2, (size_t)c * 4},
               {h->centroids, spec->centroids, (size_t)levels * 4},
               {h->boundaries, spec->boundaries, (size_t)(levels - 1) * 4}};
  for (const Part& pt : parts) {
    const hipError_t e = rt->copy_sync(pt.dst, pt.src, pt.bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(mem);
      delete h;
      return eoship::hip_err(err, "hipMemcpy(hadamard tables)", e);
    }
  }
  *out = h;
  return 0;
}

static int hq_launch(EosHipRuntime* rt, EosHipHadamardTQ* h, int32_t n, int32_t height,
                     int32_t width, const char* kernel, HqArgs& a, const char* what, char** err) {
  if (rt == nullptr || h == nullptr) return set_err(err, "%s: NULL argument", what);
  if (h->rt != rt) return set_err(err, "%s: the codec is bound to another runtime", what);
  if (n < 0 || height < 0 || width < 0) return set_err(err, "%s: negative shape", what);
  const long long pixels = (long long)n * height * width;
  if (pixels == 0) return 0;
  if ((long long)height * width > 0x7fffffffll) return set_err(err, "%s: height * width too large", what);
  a.perm = h->perm;
  a.signs1 = h->signs1;
  a.signs2 = h->signs2;
  a.centroids = h->centroids;
  a.boundaries = h->boundaries;
  a.pixels = pixels;
  a.channels = h->channels;
  a.hw = height * width;
  a.levels = h->levels;
  const size_t lds = (size_t)h->channels * kHqThreads * sizeof(float);
  return rt->launch(kernel, dim3((unsigned)((pixels + kHqThreads - 1) / kHqThreads)),
                    dim3(kHqThreads), lds, &a, err, kernel);
}

int eoship_hadamard_tq_encode_device(EosHipRuntime* rt, EosHipHadamardTQ* h, const float* d_input,
                                     int32_t n, int32_t height, int32_t width, uint8_t* d_coords,
                                     uint8_t* d_norm_codes, char** err) {
  const char* what = "eoship_hadamard_tq_encode_device";
  if (d_input == nullptr || d_coords == nullptr || d_norm_codes == nullptr)
    return (long long)n * height * width == 0 ? 0 : set_err(err, "%s: NULL buffer", what);
  HqArgs a;
  std::memset(&a, 0, sizeof(a));
  a.input = d_input;
  a.coords = d_coords;
  a.norms = d_norm_codes;
  return hq_launch(rt, h, n, height, width, "eos_hq_encode", a, what, err);
}

int eoship_hadamard_tq_decode_device(EosHipRuntime* rt, EosHipHadamardTQ* h,
                                     const uint8_t* d_coords, const uint8_t* d_norm_codes,
                                     int32_t n, int32_t height, int32_t width, float* d_out,
                                     char** err) {
  const char* what = "eoship_hadamard_tq_decode_device";
  if (d_coords == nullptr || d_norm_codes == nullptr || d_out == nullptr)
    return (long long)n * height * width == 0 ? 0 : set_err(err, "%s: NULL buffer", what);
  HqArgs a;
  std::memset(&a, 0, sizeof(a));
  a.coords_in = d_coords;
  a.norms_in = d_norm_codes;
  a.out = d_out;
  return hq_launch(rt, h, n, height, width, "eos_hq_decode", a, what, err);
}

int eoship_hadamard_tq_release(EosHipRuntime* rt, EosHipHadamardTQ* h, char** err) {
  if (h == nullptr) return 0;
  if (rt == nullptr || h->rt != rt) return set_err(err, "eoship_hadamard_tq_release: wrong runtime");
  if (rt->sync(err) != 0) return 1;
  (void)hipFree(h->tables);
  delete h;
  return 0;
}

}  // extern "C"
