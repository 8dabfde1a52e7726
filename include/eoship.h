/*
 * eoship.h -- C ABI of the MI355X (gfx950) backend for Eos's quantized
 * embedding-inference path.
 *
 * Conventions (mirroring the reference CGo bridge, runtime/backends/cuda/
 * native_linux.go:72-148 and :1378-1392):
 *   - every entry point returns int: 0 = success, nonzero = failure;
 *   - on failure a malloc'd, NUL-terminated message is stored in *err when
 *     err is non-NULL; the caller releases it with eoship_free_cstring;
 *   - no caller pointer is retained after a call returns; host buffers are
 *     copied to device memory owned by the runtime or by a bound object;
 *   - all device work of one runtime is ordered on that runtime's single HIP
 *     stream; calls that return host results synchronise that stream.
 *
 * Kernels are gfx950 code objects built offline (hipcc --genco) and loaded
 * with hipModuleLoadData; there is no run-time compiler.
 */
#ifndef EOSHIP_H
#define EOSHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct EosHipRuntime EosHipRuntime;
typedef struct EosHipModule EosHipModule;
typedef struct EosHipFunction EosHipFunction;
typedef struct EosHipTQ EosHipTQ;

/* ---------------------------------------------------------------- runtime */

/* Replaces eosCudaRuntimeCreate / the EosCudaRuntime struct
 * (runtime/backends/cuda/native_linux.go:150-283,
 *  runtime/backends/cuda/eos_cuda_abi.h:22-38): one device, one stream. */
int eoship_runtime_create(int device, EosHipRuntime** out, char** err);
/* Replaces eosCudaRuntimeDestroy (native_linux.go:150-283). */
int eoship_runtime_destroy(EosHipRuntime* rt, char** err);
/* Releases a message returned through char** err (native_linux.go:1378-1392). */
void eoship_free_cstring(char* s);
/* ABI version of this library; bumped on any signature change. */
int eoship_abi_version(void);
/* Device name, compute units and gfx arch of the runtime's device. */
int eoship_device_info(EosHipRuntime* rt, char* name, size_t name_len, int* compute_units,
                       char* arch, size_t arch_len, char** err);

/* Device memory owned by the caller through the runtime; all copies are
 * ordered on the runtime stream (native_linux.go:3321-3421 upload/download). */
int eoship_malloc(EosHipRuntime* rt, size_t bytes, void** dptr, char** err);
int eoship_free(EosHipRuntime* rt, void* dptr, char** err);
int eoship_h2d(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, char** err);
int eoship_d2h(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, char** err);
int eoship_d2d(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, char** err);
int eoship_sync(EosHipRuntime* rt, char** err);

/* Generic code-object path; replaces the NVRTC compile + cuModuleLoadData +
 * cuLaunchKernel bridge (native_linux.go:500-632, :3548-3563). */
int eoship_module_load(EosHipRuntime* rt, const void* image, size_t bytes, EosHipModule** out,
                       char** err);
int eoship_module_unload(EosHipModule* mod, char** err);
int eoship_function(EosHipModule* mod, const char* name, EosHipFunction** out, char** err);
int eoship_launch(EosHipRuntime* rt, EosHipFunction* fn, const uint32_t grid[3],
                  const uint32_t block[3], uint32_t lds_bytes, void** args, char** err);

/* Per-kernel hipEvent timing, the counterpart of EOS_CUDA_COMPACT_PROFILE_EVENTS
 * (native_linux.go:285-500). When enabled, every launch of a library kernel is
 * bracketed by two events on the runtime stream. */
int eoship_profile_enable(EosHipRuntime* rt, int enabled, char** err);
/* Sums the recorded launches of kernels whose name starts with prefix. */
int eoship_profile_read(EosHipRuntime* rt, const char* prefix, int64_t* launches, double* total_ms,
                        char** err);
int eoship_profile_reset(EosHipRuntime* rt, char** err);
/* Stream-level timer: records an event now; eoship_timer_elapsed gives the
 * milliseconds between two recorded marks (synchronising the second). */
int eoship_timer_mark(EosHipRuntime* rt, int slot, char** err);
int eoship_timer_elapsed(EosHipRuntime* rt, int slot_begin, int slot_end, double* ms, char** err);

/* ------------------------------------------------------------- TurboQuant */

/* Build-defined TurboQuant MSE-stage layout (the BASELINE corpus layout):
 * per vector, dim*bits/8 bytes of codes (coordinate j at bit (j*bits)%8 of byte
 * (j*bits)/8, low bits first, as the q4 packer of runtime/mll_export.go:950-958)
 * plus one f32 Norm. Codebook centroid v is codebook_scale * codebook[v]
 * (int8 grid). Scores estimate <q, x> = Norm * <R q, c[code]>. */
typedef struct {
  int32_t dim;              /* vector dimension d (1..2048) */
  int32_t bits;             /* code width: 2 or 4 */
  float codebook_scale;     /* s_c > 0 */
  const int8_t* codebook;   /* 2^bits int8 centroids (host) */
  const float* rotation;    /* d x d row-major orthogonal R (host); NULL = identity */
} EosHipTQDesc;

typedef struct {
  int64_t candidate_count;  /* vectors x queries considered (CandidateCount) */
  int64_t candidates_kept;  /* candidates that passed the threshold filter */
  int32_t fallback_queries; /* queries resolved by the exhaustive path */
  int32_t batches;          /* query batches of up to 64 */
} EosHipTQStats;

/* Binds a corpus: uploads codes and norms and repacks the codes into the
 * MFMA tile layout. Replaces the per-document turboquant.IPQuantized slice
 * the host loop walks (runtime/retrieval_turboquant.go:704-711). Norms must be
 * finite and >= 0 (runtime/turboquant_quantized_vector.go:25-34). */
int eoship_tq_bind_corpus(EosHipRuntime* rt, const EosHipTQDesc* desc, const uint8_t* codes,
                          const float* norms, int64_t n, EosHipTQ** out, char** err);
int eoship_tq_release(EosHipTQ* tq, char** err);

/* Top-k by inner-product estimate for Q queries (host buffers).
 * Replaces PrepareQuery + topTurboQuantRetrievalScoresWithStats
 * (runtime/retrieval_turboquant.go:1324, :1853-1887): order is score
 * descending then id ascending (runtime/retrieval_eval.go:1153-1161); k <= 0 or
 * k > n means k = n (:1854-1856). ids/scores are [Q][min(k,n)]. */
int eoship_tq_topk(EosHipRuntime* rt, EosHipTQ* tq, const float* queries, int32_t q, int32_t k,
                   int64_t* ids, float* scores, EosHipTQStats* stats, char** err);
/* Same on device-resident buffers (queries [Q][d] f32, ids [Q][kk] i64,
 * scores [Q][kk] f32). */
int eoship_tq_topk_device(EosHipRuntime* rt, EosHipTQ* tq, const float* d_queries, int32_t q,
                          int32_t k, int64_t* d_ids, float* d_scores, EosHipTQStats* stats,
                          char** err);
/* Exhaustive scores and exact integer code dot products for vectors
 * [begin, begin+count) (host outputs [Q][count]; either may be NULL). The
 * counterpart of InnerProductPrepared over a slice of documents
 * (runtime/retrieval_turboquant.go:1874). */
int eoship_tq_scores(EosHipRuntime* rt, EosHipTQ* tq, const float* queries, int32_t q,
                     int64_t begin, int64_t count, int32_t* dots, float* scores, char** err);
/* Prepared query of the scan: int16 rotated-and-rounded query [Q][d] and the
 * f32 score scale alpha [Q] (the device PrepareQuery). */
int eoship_tq_prepare(EosHipRuntime* rt, EosHipTQ* tq, const float* queries, int32_t q,
                      int16_t* qs, float* alpha, char** err);

#ifdef __cplusplus
}
#endif

#endif /* EOSHIP_H */
