// Internal declarations shared by the eoship host translation units.
#ifndef EOSHIP_INTERNAL_H
#define EOSHIP_INTERNAL_H

#include <hip/hip_runtime_api.h>

#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "eoship.h"

#define EOSHIP_ABI_VERSION 6

namespace eoship {

constexpr int kTimerSlots = 16;

struct ProfileRecord {
  std::string name;
  hipEvent_t begin;
  hipEvent_t end;
};

int set_err(char** err, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_err(char** err, const char* what, hipError_t e);

struct Runtime {
  int device = 0;
  int compute_units = 0;
  std::string name;
  std::string arch;
  hipStream_t stream = nullptr;
  std::vector<hipModule_t> builtin;  // built-in code objects, searched in order
  std::unordered_map<std::string, hipFunction_t> fns;
  bool profiling = false;
  std::string profile_prefix;  // record only labels starting with this (empty = all)
  std::vector<ProfileRecord> records;
  std::vector<hipEvent_t> event_pool;  // recycled profiling events
  std::map<std::string, std::pair<int64_t, double>> totals;
  // Every recorded launch's duration, per label, in launch order (cleared
  // with the totals).
  std::map<std::string, std::vector<float>> samples;
  hipEvent_t timer[kTimerSlots];

  int function(const char* name, hipFunction_t* out, char** err);
  // Launches builtin kernel `name` whose single by-value argument is *args.
  // `label` names the launch in profiles (defaults to the kernel name).
  int launch(const char* name, dim3 grid, dim3 block, size_t lds, void* args, char** err,
             const char* label = nullptr);
  // Workgroups of `block` threads and `lds` dynamic LDS bytes that one CU
  // holds at once for kernel `name` (its register and LDS use); cached.
  std::unordered_map<std::string, int> occupancy;
  int blocks_per_cu(const char* name, int block, size_t lds, int* out, char** err);
  int alloc(size_t bytes, void** p, char** err);
  // A device workspace owned by the runtime, grown (never shrunk) on demand
  // and reused by later calls on the same stream; freed with the runtime.
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int workspace(size_t bytes, void** p, char** err);
  void release(void* p);
  int sync(char** err);
  int flush_profile(char** err);
  int take_event(hipEvent_t* ev, char** err);

  // Execution accounting (the counters the reference's executor reports per
  // step, runtime/backend/symbolic.go:174-216): kernel launches, bytes
  // copied host -> device and device -> host, host synchronisations.
  int64_t n_launches = 0, n_uploaded = 0, n_downloaded = 0, n_syncs = 0;
  void count_copy(hipMemcpyKind kind, size_t bytes) {
    if (kind == hipMemcpyHostToDevice) n_uploaded += (int64_t)bytes;
    if (kind == hipMemcpyDeviceToHost) n_downloaded += (int64_t)bytes;
  }
  // Copies on the runtime stream, counted.
  hipError_t copy_async(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    count_copy(kind, bytes);
    return hipMemcpyAsync(dst, src, bytes, kind, stream);
  }
  // Blocking copies (bind-time uploads), counted as a copy and a host sync.
  hipError_t copy_sync(void* dst, const void* src, size_t bytes, hipMemcpyKind kind) {
    count_copy(kind, bytes);
    ++n_syncs;
    return hipMemcpy(dst, src, bytes, kind);
  }
};

// Two-stage rerank on a caller-chosen scratch buffer of at least
// q * c * 4 bytes (the candidates' f32 scores between its two kernels).
int tq_fp16_rerank_launch(Runtime* rt, const float* d_queries, int32_t q, int32_t d,
                          const uint16_t* d_rows, int64_t n, const int64_t* d_cand_ids,
                          const float* d_cand_scores, int32_t c, int32_t k, int32_t bit_width,
                          int32_t overfetch, const int64_t* d_id_rank, int64_t* d_ids,
                          float* d_scores, float* scratch, const char* what, char** err);
// Resolves the no-allocation entry points' static scratch on `device` (which
// must be current); called once per runtime creation, failures are reported
// by those entry points.
void noalloc_init(int device);

int tq_fp16_rerank_check(const Runtime* rt, const float* d_queries, int32_t q, int32_t d,
                         const uint16_t* d_rows, int64_t n, const int64_t* d_cand_ids,
                         const float* d_cand_scores, int32_t c, int64_t* d_ids, float* d_scores,
                         const char* what, char** err);

// Row scores of a retrieval plan's score step, its topk and the gathers
// (documents as f32 values or a packed q4 tensor, exactly one non-NULL).
int score_topk_launch(Runtime* rt, const EosHipScoreSpec& s, const float* d_queries, int32_t q,
                      int32_t d, const float* d_docs, const uint8_t* d_docs_q4, int64_t n,
                      const int64_t* d_candidate_ids, float* d_scores, int32_t* d_top_index,
                      int64_t* d_top_ids, float* d_top_scores, float* d_top_docs,
                      const char* what, char** err);

}  // namespace eoship

struct EosHipRuntime : eoship::Runtime {};

// A retrieval plan bound from a package: the score op and topk limit, and
// the documents when the plan reads them from a param (uploaded at bind).
struct EosHipRetrieval {
  EosHipRuntime* rt = nullptr;
  EosHipScoreSpec spec{};
  bool docs_param = false;
  bool has_ids = false;
  int64_t rows = 0;
  int dim = 0;
  float* docs_f32 = nullptr;
  uint8_t* docs_q4 = nullptr;
  EosHipRetrievalPlan plan{};
};

// A bound Hadamard TurboQuant codec: the spec tables on the device.
struct EosHipHadamardTQ {
  EosHipRuntime* rt = nullptr;
  int channels = 0, levels = 0;
  void* tables = nullptr;
  int32_t* perm = nullptr;
  float *signs1 = nullptr, *signs2 = nullptr, *centroids = nullptr, *boundaries = nullptr;
};

#endif  // EOSHIP_INTERNAL_H
