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
/* Sets bytes of device memory to the byte value, on the runtime stream. */
int eoship_memset(EosHipRuntime* rt, void* dst, int value, size_t bytes, char** err);
int eoship_sync(EosHipRuntime* rt, char** err);
/* Orders two runtimes on one device: work enqueued on rt after this call
 * starts only after all work enqueued on other so far has finished (an event
 * on other's stream that rt's stream waits for; the host does not wait). No
 * counterpart in the reference, whose runtime has one stream per device; it
 * joins concurrent query batches on separate streams. */
int eoship_runtime_wait(EosHipRuntime* rt, EosHipRuntime* other, char** err);

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
/* Restricts profiling to launches whose label starts with prefix (NULL or ""
 * records every launch), so that a timed loop can bracket one kernel without
 * paying two events for every other launch. */
int eoship_profile_select(EosHipRuntime* rt, const char* prefix, char** err);
/* Sums the recorded launches of kernels whose name starts with prefix. */
int eoship_profile_read(EosHipRuntime* rt, const char* prefix, int64_t* launches, double* total_ms,
                        char** err);
int eoship_profile_reset(EosHipRuntime* rt, char** err);
/* The duration (ms) of each recorded launch whose label starts with prefix
 * (labels in name order, launches in order within a label): up to cap values
 * into ms, the number recorded into *count. For medians of per-launch times
 * (no counterpart in the reference, whose profiler keeps totals only). */
int eoship_profile_samples(EosHipRuntime* rt, const char* prefix, float* ms, int64_t cap,
                           int64_t* count, char** err);
/* Execution accounting of a runtime since its creation or the last reset:
 * the per-step counters the reference's executor reports in
 * StepDispatchResult.Metadata and sums into ExecutionAccounting
 * (runtime/backend/symbolic.go:174-216, backend.go:1376-1401). A caller reads
 * it before and after a call and reports the difference for that call. Every
 * call of this library runs on the device (device_execution = 1, no host
 * fallback: there is no fallback_reason); graph captures and replays are
 * always 0 (the library captures no graphs). uploaded_bytes / downloaded_bytes
 * count the host <-> device copies the library makes (bind-time uploads,
 * the host-API entry points' inputs and outputs, status reads); sync_count
 * the host waits it makes. */
typedef struct {
  int64_t kernel_launches;
  int64_t uploaded_bytes;
  int64_t downloaded_bytes;
  int64_t sync_count;
  int64_t graph_captures;
  int64_t graph_replays;
  int32_t device_execution;
  int32_t reserved;
} EosHipAccounting;
int eoship_accounting_read(EosHipRuntime* rt, EosHipAccounting* out, int32_t reset, char** err);

/* Stream-level timer: records an event now; eoship_timer_elapsed gives the
 * milliseconds between two recorded marks (synchronising the second). */
int eoship_timer_mark(EosHipRuntime* rt, int slot, char** err);
int eoship_timer_elapsed(EosHipRuntime* rt, int slot_begin, int slot_end, double* ms, char** err);

/* ------------------------------------------------------------- TurboQuant */

/* Build-defined TurboQuant MSE-stage layout (the benchmark's c2 layout):
 * per vector, dim*bits/8 bytes of codes (coordinate j at bit (j*bits)%8 of byte
 * (j*bits)/8, low bits first, as the q4 packer of runtime/mll_export.go:950-958)
 * plus one f32 Norm. Codebook centroid v is codebook_scale * codebook[v]
 * (int8 grid). Scores estimate <q, x> = Norm * <R q, c[code]>. */
typedef struct {
  int32_t dim;              /* vector dimension d (1..1024) */
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
 * the host loop walks (runtime/retrieval_turboquant.go:704-711). The Norm
 * policy is validateEosQuantizedVectorNorm's
 * (runtime/turboquant_quantized_vector.go:25-34): Norm > 0 is accepted;
 * Norm == 0 is refused here (a vector that dropped its norm field) and
 * accepted only through eoship_tq_bind_corpus_opts for a vector the caller
 * confirms as a genuine zero vector; negative, NaN and infinite norms are
 * refused. */
int eoship_tq_bind_corpus(EosHipRuntime* rt, const EosHipTQDesc* desc, const uint8_t* codes,
                          const float* norms, int64_t n, EosHipTQ** out, char** err);

typedef struct {
  /* [n] or NULL: nonzero when the caller confirms that vector i was the
   * genuine zero vector, so its Norm == 0 is accepted (zeroVectorAllowed of
   * validateEosQuantizedVectorNorm / newEosQuantizedVector,
   * runtime/turboquant_quantized_vector.go:25-49). */
  const uint8_t* zero_vector_allowed;
  /* [n] or NULL: the position of vector i's string ID among the corpus IDs
   * sorted ascending (Go string order), a permutation of 0..n-1. Equal
   * scores then rank by string ID as retrievalScoreBetter does
   * (runtime/retrieval_eval.go:1153-1161; e.g. "d1" < "d10" < "d2"); results
   * still report vector indices. NULL: IDs order like their indices. A ranked
   * corpus serves flat top-k and eoship_tq_scores; MaxSim documents and
   * parents need index order and refuse it. */
  const int64_t* id_rank;
} EosHipTQBindOptions;

/* eoship_tq_bind_corpus with options (opts may be NULL: no options). */
int eoship_tq_bind_corpus_opts(EosHipRuntime* rt, const EosHipTQDesc* desc, const uint8_t* codes,
                               const float* norms, int64_t n, const EosHipTQBindOptions* opts,
                               EosHipTQ** out, char** err);

/* Stored bytes of one turboquant.IPQuantized vector: (bit_width - 1)-bit MSE
 * codes and one QJL sign bit per coordinate, each packed to whole bytes, plus
 * the Norm and ResNorm f32 fields (turboquantVectorBytes,
 * runtime/turboquant_bytes.go:14-25: 136 B at dim 256, bit width 4). */
int eoship_tq_vector_bytes(int32_t dim, int32_t bit_width, int64_t* bytes, char** err);
/* Bytes of one vector of the MSE-stage layout this library binds:
 * ceil(dim * bits / 8) code bytes plus one f32 Norm (196 B at dim 384, 4 bits). */
int eoship_tq_mse_vector_bytes(int32_t dim, int32_t bits, int64_t* bytes, char** err);
int eoship_tq_release(EosHipTQ* tq, char** err);
/* A second handle on a bound corpus for another runtime (stream) of the same
 * device: it shares the resident corpus arrays and owns its own per-call
 * scratch, so batches on the two streams may run concurrently. Handles may be
 * released in any order; the corpus is freed with the last. Handles are not
 * thread-safe: create and release them from one host thread. No counterpart
 * in the reference (one query loop per corpus); it serves concurrent query
 * batches. */
int eoship_tq_share(EosHipRuntime* rt, EosHipTQ* src, EosHipTQ** out, char** err);

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
/* The same top-k with the exactness check left to the caller, for callers that
 * synchronise once per many calls (also topTurboQuantRetrievalScoresWithStats,
 * runtime/retrieval_turboquant.go:1853-1887). Enqueues no exhaustive fallback;
 * writes d_status[Q] instead: 0 means the query's row is final, nonzero means
 * the filtered pass could not prove it and eoship_tq_topk_repair_device must
 * be called for it (with the same queries and k) before the row is used. */
int eoship_tq_topk_device_deferred(EosHipRuntime* rt, EosHipTQ* tq, const float* d_queries,
                                   int32_t q, int32_t k, int64_t* d_ids, float* d_scores,
                                   int32_t* d_status, char** err);
/* Recomputes, exhaustively and exactly, the rows whose d_status is nonzero
 * (the rest are left as they are). */
int eoship_tq_topk_repair_device(EosHipRuntime* rt, EosHipTQ* tq, const float* d_queries, int32_t q,
                                 int32_t k, int64_t* d_ids, float* d_scores,
                                 const int32_t* d_status, char** err);
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

/* Multivector late interaction (MaxSim) over a bound corpus grouped into
 * documents of doc_len consecutive vectors (doc_len a multiple of 32, corpus
 * size a whole number of documents). A query is tq_tokens (1..32) token
 * vectors; its score for a document is the sum, as a pairwise tree over 32
 * token slots (slot i += slot i^o for o = 1, 2, 4, 8, 16; missing tokens
 * contribute +0), of each token's best per-vector TurboQuant score in the
 * document. With one token this is the reference child-max
 * (runtime/retrieval_multivector_turboquant.go:746-783, 785-810 with "max"
 * aggregation); parents rank by score desc, id asc (:890-908).
 * queries [Q][tq_tokens][d]; ids/scores [Q][min(k, ndocs)]. */
int eoship_tq_maxsim_topk(EosHipRuntime* rt, EosHipTQ* tq, int32_t doc_len, const float* queries,
                          int32_t q, int32_t tq_tokens, int32_t k, int64_t* ids, float* scores,
                          char** err);
int eoship_tq_maxsim_topk_device(EosHipRuntime* rt, EosHipTQ* tq, int32_t doc_len,
                                 const float* d_queries, int32_t q, int32_t tq_tokens, int32_t k,
                                 int64_t* d_ids, float* d_scores, char** err);
/* Exhaustive MaxSim document scores for documents [doc_begin, doc_begin +
 * doc_count) (host output [Q][doc_count]). */
int eoship_tq_maxsim_scores(EosHipRuntime* rt, EosHipTQ* tq, int32_t doc_len, const float* queries,
                            int32_t q, int32_t tq_tokens, int64_t doc_begin, int64_t doc_count,
                            float* scores, char** err);

/* Corpus encoder with a bound corpus's quantizer (rotation, codebook, bits;
 * a corpus bound with n = 0 serves as a pure quantizer): rows of x [n][dim]
 * f32 -> codes [n][ceil(dim*bits/8)] in the reference layout (coordinate j
 * at bit j*bits, low bits first) and norms [n]. The MSE stage of the
 * corpus-side quantizer (turboquant.NewIPWithSeed / IPQuantizer.Quantize,
 * called at runtime/retrieval_turboquant.go:700,708; build-defined
 * arithmetic: u = R x in f64 fma chains, norm = (float)sqrt(sum x^2),
 * code_j = argmin_v |u_j - norm_f64 * s_c C_v|, ties to the lower v). The
 * outputs bind directly with eoship_tq_bind_corpus; the device form takes
 * embeddings already on the device (an encoder's output). */
int eoship_tq_encode(EosHipRuntime* rt, EosHipTQ* tq, const float* x, int64_t n, uint8_t* codes,
                     float* norms, char** err);
int eoship_tq_encode_device(EosHipRuntime* rt, EosHipTQ* tq, const float* d_x, int64_t n,
                            uint8_t* d_codes, float* d_norms, char** err);

/* Parent aggregation over children (one query vector per query): the
 * corpus vectors [offsets[p], offsets[p+1]) are the children of parent p
 * (offsets ascending, offsets[0] = 0, offsets[nparents] = corpus size; a
 * parent may have no children). Replaces topTurboQuantMultiVectorParentScores
 * (runtime/retrieval_multivector_turboquant.go:746-758) with its
 * accumulator and aggregation (:769-810) and topParentScoresFromMap
 * (:890-908), ids being integer parent and child indices. Release the
 * parents before their corpus. */
typedef struct EosHipTQParents EosHipTQParents;
int eoship_tq_parents_bind(EosHipRuntime* rt, EosHipTQ* tq, const int64_t* offsets,
                           int64_t nparents, EosHipTQParents** out, char** err);
int eoship_tq_parents_release(EosHipTQParents* parents, char** err);
/* Per query: every child's TurboQuant score; per parent the mean of its
 * best min(top_n, count) child scores (f64 sum in descending order; top_n 1
 * = "max", 2/3/5 = "top2/3/5-mean", validateTurboQuantMultiVectorAggregation-
 * Config :826-837) minus child_count_penalty * log1p(count) when the penalty
 * is nonzero (>= 0, else an error), rounded to f32; the best min(k,
 * parents with children) parents (k <= 0: all of them) by score desc, parent
 * id asc, each with its best child (highest score, then lowest index) and
 * that child's score. Outputs [q][kk] (host buffers). */
int eoship_tq_parent_topk(EosHipRuntime* rt, EosHipTQParents* parents, const float* queries,
                          int32_t q, int32_t k, int32_t top_n, double child_count_penalty,
                          int64_t* parent_ids, float* scores, int64_t* best_child,
                          float* best_child_score, char** err);
/* Same on device buffers, enqueued on the runtime stream (no wait). */
int eoship_tq_parent_topk_device(EosHipRuntime* rt, EosHipTQParents* parents,
                                 const float* d_queries, int32_t q, int32_t k, int32_t top_n,
                                 double child_count_penalty, int64_t* d_parent_ids,
                                 float* d_scores, int64_t* d_best_child, float* d_best_child_score,
                                 char** err);

/* ------------------------------------------------------------- tiny embed */

typedef struct EosHipEmbed EosHipEmbed;

/* The examples/embed.eos pipeline -- gather(token_embedding f16 [V][D]),
 * @matmul(projection f16 [D][E]), l2_normalize -- with resident weights.
 * Replaces the host gather + cuBLAS matmul + l2_normalize kernel steps that
 * Program.Run executes for it (runtime/backend/tensor_ops.go:938-1166,
 * 1168-1249, 1367-1391; runtime/runtime.go:222). f16 tensors are IEEE
 * binary16 bit patterns. */
int eoship_embed_bind(EosHipRuntime* rt, const uint16_t* table_f16, int32_t vocab, int32_t dim,
                      const uint16_t* proj_f16, int32_t edim, EosHipEmbed** out, char** err);
int eoship_embed_release(EosHipEmbed* emb, char** err);
/* tokens [n] -> out [n][E] f16 (host); token ids outside [0, V) are an error
 * (gatherTensor rejects them, runtime/backend/tensor_ops.go:938-1166). */
int eoship_embed_run(EosHipRuntime* rt, EosHipEmbed* emb, const int32_t* tokens, int32_t n,
                     uint16_t* out_f16, char** err);
int eoship_embed_run_device(EosHipRuntime* rt, EosHipEmbed* emb, const int32_t* d_tokens,
                            int32_t n, uint16_t* d_out_f16, char** err);

/* ---------------------------------------------------------------- encoder */

typedef struct EosHipEncoder EosHipEncoder;

/* BERT-style post-LN encoder (the imported bert_embedder step): the
 * architecture fields of BERTEmbedderReferenceWithPooling
 * (runtime/backend/bert_embedder_ops.go:101-197). */
typedef struct {
  int32_t layers;        /* num_hidden_layers */
  int32_t hidden;        /* MFMA kernels: 128, 256, 384, 512 or 768; else the
                            general-shape f32 kernels: a multiple of 8 up to 1024 */
  int32_t heads;         /* MFMA: hidden / heads in {32, 64, 128, 256};
                            general-shape: hidden / heads <= 64 */
  int32_t intermediate;  /* MFMA: a multiple of 128; general-shape: 1 .. 16384 */
  int32_t vocab;         /* token table rows */
  int32_t max_positions; /* position table rows (>= tokens) */
  int32_t type_vocab;    /* token-type table rows */
  float ln_eps;          /* LayerNorm epsilon (BERT: 1e-12) */
  int32_t gelu;          /* 1 = erf GELU (exactGELU), 2 = tanh GELU */
} EosHipEncoderDesc;

/* One layer's weights (host). Dense weights are int8 codes in HF [out][in]
 * layout with one f32 scale per output channel (dequantized weight =
 * code * scale; one equal scale per tensor reproduces the reference's
 * per-tensor q8 grid, runtime/mll_export.go:897-975). w_qkv stacks the query,
 * key and value projections ([3*hidden][hidden]). */
typedef struct {
  const int8_t* w_qkv; const float* s_qkv; const float* b_qkv;
  const int8_t* w_o;   const float* s_o;   const float* b_o;
  const float* ln1_gamma; const float* ln1_beta;
  const int8_t* w_1;   const float* s_1;   const float* b_1;   /* [intermediate][hidden] */
  const int8_t* w_2;   const float* s_2;   const float* b_2;   /* [hidden][intermediate] */
  const float* ln2_gamma; const float* ln2_beta;
} EosHipEncoderLayer;

/* Uploads embedding tables (f32) and layer weights. Replaces loading the
 * bert_embedder step's weights (runtime/backend/bert_embedder_ops.go:101-197;
 * q8 dequantization at load, runtime/weight_file.go:315-333). */
int eoship_encoder_bind(EosHipRuntime* rt, const EosHipEncoderDesc* desc, const float* tok_emb,
                        const float* pos_emb, const float* type_emb, const float* emb_ln_gamma,
                        const float* emb_ln_beta, const EosHipEncoderLayer* layers,
                        EosHipEncoder** out, char** err);
int eoship_encoder_release(EosHipEncoder* enc, char** err);
/* Embeds a [batch][tokens] batch (host buffers): embeddings, all layers,
 * masked mean pool, L2 normalize -> out [batch][hidden] f32 (an encoder bound
 * with eoship_encoder_bind_compact: out [batch][output_dim]). type_ids may be
 * NULL (all 0). Fails with an error for a token, type or position id outside
 * its table, at any position, masked ones included (the reference checks the
 * whole input, runtime/backend/tensor_ops.go:1484-1492).
 * Replaces Program.Run of a bert_embedder plan / EmbeddingModel.EmbedBatch
 * (runtime/inference.go:57-101; runtime/embedding_model.go:669-761). */
int eoship_encoder_forward(EosHipRuntime* rt, EosHipEncoder* enc, const int32_t* ids,
                           const int32_t* type_ids, const int32_t* mask, int32_t batch,
                           int32_t tokens, float* out, char** err);
/* Same on device buffers; enqueued on the runtime stream (no wait). The id
 * check result is readable with eoship_encoder_status after a sync. */
int eoship_encoder_forward_device(EosHipRuntime* rt, EosHipEncoder* enc, const int32_t* d_ids,
                                  const int32_t* d_type_ids, const int32_t* d_mask, int32_t batch,
                                  int32_t tokens, float* d_out, char** err);
/* 0 when every id of the last forward was in range; synchronises. */
int eoship_encoder_status(EosHipRuntime* rt, EosHipEncoder* enc, int32_t* status, char** err);
/* Selects the BERT family's layer tail at hidden 384, 512 and 768: fused
 * (default: O projection, residual, LayerNorm, FFN and the second LayerNorm
 * as one kernel per row block, the intermediate kept on chip) or the unfused
 * GEMM and LayerNorm launches. Both round at the same points. No counterpart
 * in the reference; for comparing the two paths. */
int eoship_encoder_set_fused_tail(EosHipRuntime* rt, EosHipEncoder* enc, int32_t fused,
                                  char** err);
/* BERT family sentence pooling, the bert_embedder step's "pooling" attribute
 * (runtime/backend/bert_embedder_ops.go:150-152, 183-196): 0 masked_mean
 * (the default: mean over mask != 0 positions, then L2), 1 cls (position 0's
 * hidden state, then L2; position 0 is computed even where the mask clears
 * it, attending to the sequence's active positions, as the reference
 * computes every row). Refused for the compact family. */
int eoship_encoder_set_pooling(EosHipRuntime* rt, EosHipEncoder* enc, int32_t pooling,
                               char** err);
/* Diagnostic of the last forward (synchronises): how many times a wavefront
 * of the attention kernels moved its softmax exponent reference after a
 * sequence's first key block (a score far above every earlier one, as peaked
 * late-maximum attention gives). No counterpart in the reference, whose host
 * softmax subtracts the exact maximum (bert_encoder_layer_ops.go:272-324). */
int eoship_encoder_attention_moves(EosHipRuntime* rt, EosHipEncoder* enc, int64_t* moves,
                                   char** err);

/* Compact transformer embedder (family (a): the graph that
 * compactTransformerSource emits, models/default_embedding.go:419-505, with
 * the DefaultEmbeddingPackageConfig fields of :264-300). */
typedef struct {
  int32_t layers;        /* EncoderRepeats (layers may repeat one set of codes: tied) */
  int32_t model_dim;     /* D: 128, 256, 384, 512 or 768 */
  int32_t heads;         /* AttentionHeads; D / heads in {32, 64, 128, 256} */
  int32_t hidden_dim;    /* FFN width H, positive multiple of 128 */
  int32_t vocab;         /* token_embedding rows */
  int32_t max_sequence;  /* longest accepted tokens (RoPE table rows) */
  int32_t output_dim;    /* O; equal to model_dim when there is no output_projection */
} EosHipCompactDesc;

/* One layer's q8 (or unpacked q4) codes in the reference's [in][out] layout,
 * each tensor with its per-tensor scale (dequantized = code * scale,
 * runtime/weight_file.go:315-350; a scale of 0 means an all-zero tensor). */
typedef struct {
  const int8_t* attn_q; float s_q;       /* [D][D] */
  const int8_t* attn_k; float s_k;       /* [D][D] */
  const int8_t* attn_v; float s_v;       /* [D][D] */
  const int8_t* attn_o; float s_o;       /* [D][D] */
  const int8_t* ffn_up; float s_up;      /* [D][H] */
  const int8_t* ffn_down; float s_down;  /* [H][D] */
} EosHipCompactLayer;

/* Uploads a compact embedder: token_embedding [V][D] and role_embedding
 * [3][D] codes, per-layer weights, and output_projection [D][O] (NULL when
 * output_dim == model_dim). The forward calls above then run its graph:
 * rope(dequant(tok) + dequant(role)), per layer q/k/v = x W, masked
 * attention (one head: scaled_attention_scores + masked_softmax; several:
 * compact_multihead_attention_hN), layernorm(x W_o + x), tanh-GELU FFN,
 * layernorm(ffn + h), then normalize per token, the optional projection and
 * the masked mean (out [batch][output_dim]); their type_ids argument carries
 * the role_ids (0..2). Replaces loading and running that graph through
 * ExecuteSymbolic (runtime/backend/symbolic.go:17-172) or the CUDA compact
 * forward (runtime/backends/cuda/compact_forward_accel_linux.go:106-305). */
int eoship_encoder_bind_compact(EosHipRuntime* rt, const EosHipCompactDesc* desc,
                                const int8_t* token_embedding, float s_token,
                                const int8_t* role_embedding, float s_role,
                                const EosHipCompactLayer* layers, const int8_t* output_projection,
                                float s_output, EosHipEncoder** out, char** err);

/* Graph options of a compact embedder, each 0 or 1. eoship_encoder_bind_compact
 * binds with rope, role and scaled_scores 1 and attend_padding 0 (the
 * compactTransformerSource graph). */
typedef struct {
  int32_t rope;            /* 1: ropeRows after the gather; 0: no rotation */
  int32_t role;            /* 1: token + role_embedding[role id]; 0: token rows only
                            * (role_embedding may then be NULL) */
  int32_t scaled_scores;   /* 1: one head's q kT times 1/sqrt(D) (scaled_attention_scores,
                            * runtime/backend/tensor_ops.go:1291-1315); 0: the plain matmul
                            * q kT of a plan's matmul step (tensor_ops.go:1168-1249).
                            * Several heads always scale by 1/sqrt(D / heads). */
  int32_t attend_padding;  /* 0: each query attends the mask != 0 positions of its
                            * sequence (maskedSoftmaxRowsF32, tensor_ops.go:1825-1865; also
                            * what EmbeddingModel's length-grouped batches give,
                            * runtime/embedding_model.go:689-691, 798-850); 1: every position
                            * of the padded [batch][tokens] input is a key and a query (a
                            * plan whose softmax step is softmaxRows, tensor_ops.go:
                            * 1757-1788), and the mask only selects the pooled rows
                            * (meanPoolMaskedTensor, tensor_ops.go:1644-1709); every id,
                            * padding included, must then be in range, as gatherTensor
                            * requires. */
} EosHipCompactOptions;

/* eoship_encoder_bind_compact with graph options (NULL: its defaults); with
 * role 0, role_embedding may be NULL. Also the binding behind
 * eoship_encoder_bind_mll. */
int eoship_encoder_bind_compact_opts(EosHipRuntime* rt, const EosHipCompactDesc* desc,
                                     const EosHipCompactOptions* opts,
                                     const int8_t* token_embedding, float s_token,
                                     const int8_t* role_embedding, float s_role,
                                     const EosHipCompactLayer* layers,
                                     const int8_t* output_projection, float s_output,
                                     EosHipEncoder** out, char** err);

/* Two-stage retrieval, second stage (the promoted serving profile
 * turboquant_ip_b4_overfetch200_fp16_rerank). eoship_f16_sidecar_device turns
 * f32 document vectors into the f16 rerank rows exactly as the halfByID loop of
 * computeTurboQuantFP16RerankRetrievalQuality does
 * (runtime/retrieval_turboquant.go:1503-1511, float32ToHalf in
 * runtime/mll_export.go:1007-1041: ties round away from zero). */
int eoship_f16_sidecar_device(EosHipRuntime* rt, const float* d_x, int64_t count, uint16_t* d_half,
                              char** err);
/* Reranks each query's first-stage candidates (d_cand_ids/d_cand_scores
 * [Q][c], in first-stage order as eoship_tq_topk_device writes them) by the
 * f16 rows d_rows [n][d]: topFP16RerankScores, or topFP16RerankRescueScores
 * when shouldApplyTurboQuantFP16RerankRescue(bit_width, k, overfetch, c)
 * holds (runtime/retrieval_turboquant.go:1551-1556, :1635-1786). c must be
 * the first stage's output width, min(overfetch, n), and at most 4096 (the
 * reference takes any overfetch; larger c is refused). Scores are sequential
 * f32 sums of f32 products. Equal scores rank by id ascending, or by
 * d_id_rank[id] ([n], the string-ID order of EosHipTQBindOptions::id_rank)
 * when it is not NULL. k <= 0 or k > c means k = c; outputs [Q][kk]; a query
 * with fewer than kk candidates in [0, n) pads its row with id -1 and score 0.
 * Enqueued on the runtime stream; uses a workspace of Q * c * 4 bytes that the
 * runtime allocates on first use and keeps. */
int eoship_tq_fp16_rerank_device(EosHipRuntime* rt, const float* d_queries, int32_t q, int32_t d,
                                 const uint16_t* d_rows, int64_t n, const int64_t* d_cand_ids,
                                 const float* d_cand_scores, int32_t c, int32_t k,
                                 int32_t bit_width, int32_t overfetch, const int64_t* d_id_rank,
                                 int64_t* d_ids, float* d_scores, char** err);
/* The inner-product layout (IPQuantized{MSE, Signs, ResNorm, Norm};
 * byte accounting runtime/turboquant_bytes.go:14-25): the MSE codes of
 * eoship_tq_encode_device plus a 1-bit QJL sketch of the residual. The
 * quantizer is in the un-vendored module (called at runtime/
 * retrieval_turboquant.go:700-711), so this is the build's contract after the
 * published TurboQuant_prod estimator, in f64: r = R x - Norm c[code],
 * ResNorm = |r| / Norm, sign bit i = (S r)_i >= 0 (packed low bit first,
 * (d + 7) / 8 bytes). S is a d x d sketch matrix (Gaussian rows) the caller
 * provides, like R. */
typedef struct {
  int32_t dim;               /* d, 1..1024 */
  int32_t bits;              /* MSE bits: 1, 2, 3 or 4 (bit width - 1) */
  float codebook_scale;      /* c_v = codebook_scale * codebook[v] */
  const int8_t* codebook;    /* host [2^bits] int8 grid */
  const float* rotation_t;   /* device [d][d], rotation_t[k * d + j] = R[j][k]; NULL = I */
  const float* qjl_t;        /* device [d][d], qjl_t[j * d + i] = S[i][j] */
} EosHipTQIPSpec;

/* x [n][d] -> codes [n][(d * bits + 7) / 8], signs [n][(d + 7) / 8],
 * resnorms [n], norms [n]. */
int eoship_tq_ip_encode_device(EosHipRuntime* rt, const EosHipTQIPSpec* spec, const float* d_x,
                               int64_t n, uint8_t* d_codes, uint8_t* d_signs, float* d_resnorms,
                               float* d_norms, char** err);
/* Exhaustive scores [q][n] of the inner-product estimate
 *   ((float)D_mse * alpha + ResNorm * ((float)D_qjl * beta)) * Norm
 * with D_mse = sum_j Qs_j C[code_j] and D_qjl = sum_i Ys_i (2 bit_i - 1)
 * exact int32 over int16 grids of R q and S R q (alpha = s_q s_c, beta =
 * s_y sqrt(pi / 2) / d), then with k > 0 the top k per query by (score
 * desc, index asc) into d_top_ids / d_top_scores [q][min(k, n)]. Uses a
 * workspace of q * (8 d + 8) bytes. */
int eoship_tq_ip_scores_device(EosHipRuntime* rt, const EosHipTQIPSpec* spec,
                               const float* d_queries, int32_t q, const uint8_t* d_codes,
                               const uint8_t* d_signs, const float* d_resnorms,
                               const float* d_norms, int64_t n, float* d_scores, int32_t k,
                               int64_t* d_top_ids, float* d_top_scores, char** err);

/* The promoted profile's first stage (turboquant_ip_b4_overfetch200_fp16_
 * rerank, runtime/retrieval_turboquant.go:1500-1556): an inner-product
 * corpus -- the codes, signs, ResNorms and Norms eoship_tq_ip_encode_device
 * writes, MSE codes of 1, 2 or 3 bits (bit widths 2, 3, 4) -- bound for
 * top-k search. Bind repacks it into a tile layout on the device (the
 * caller's buffers may be freed afterwards; spec->rotation_t and qjl_t must
 * stay valid while the corpus is bound) and applies the Norm policy of
 * validateEosQuantizedVectorNorm (Norm < 0 or non-finite refused, Norm == 0
 * only with opts->zero_vector_allowed; id_rank is not supported). */
typedef struct EosHipTQIP EosHipTQIP;
int eoship_tq_ip_bind_corpus(EosHipRuntime* rt, const EosHipTQIPSpec* spec,
                             const uint8_t* d_codes, const uint8_t* d_signs,
                             const float* d_resnorms, const float* d_norms, int64_t n,
                             const EosHipTQBindOptions* opts, EosHipTQIP** out, char** err);
/* Top k per query of the inner-product estimate (the score
 * eoship_tq_ip_scores_device computes; topTurboQuantRetrievalScoresWithStats
 * over InnerProductPrepared scores, :1853-1887): ids and scores [q][kk],
 * kk = min(k, n) (k <= 0: n, at most 8192), by score descending then index
 * ascending. Exact whatever the data: a sample threshold prunes the scan and
 * a device-gated exhaustive pass repairs any query it leaves short.
 * Enqueued on the runtime stream. */
int eoship_tq_ip_topk_device(EosHipRuntime* rt, EosHipTQIP* ip, const float* d_queries,
                             int32_t q, int32_t k, int64_t* d_ids, float* d_scores, char** err);
int eoship_tq_ip_release(EosHipTQIP* ip, char** err);

/* Second stage over f32 rows [n][d] (topDenseRerankScores,
 * runtime/retrieval_turboquant.go:1610-1633): score = sum += q[i] * row[i] in
 * index order, each product and sum rounded to f32, then (score desc, ID
 * asc) -- the id-rank order when d_id_rank is given -- over the candidates in
 * [0, n); others are skipped. Arguments as eoship_tq_fp16_rerank_device, with
 * no rescue. Uses a workspace of q * c * 4 bytes. */
int eoship_tq_dense_rerank_device(EosHipRuntime* rt, const float* d_queries, int32_t q, int32_t d,
                                  const float* d_rows, int64_t n, const int64_t* d_cand_ids,
                                  int32_t c, int32_t k, const int64_t* d_id_rank, int64_t* d_ids,
                                  float* d_scores, char** err);

/* A TurboQuant code set on the device in the reference row layout: the
 * primary codes or a wider sidecar set with its own codebook; with signs,
 * resnorms and qjl_t an inner-product set (IPQuantized{MSE, Signs, ResNorm,
 * Norm}, runtime/turboquant_bytes.go:14-25, the layout of
 * eoship_tq_ip_encode_device). */
typedef struct {
  int32_t bits;               /* 1, 2, 3, 4 or 8 bits per coordinate */
  int32_t dim;                /* d (1..1024) */
  int64_t n;                  /* vectors */
  const uint8_t* codes;       /* [n][(d * bits + 7) / 8], code j at bits j * bits .. + bits - 1
                               * of the row, low bits first (3-bit codes straddle bytes) */
  const float* norms;         /* [n] */
  const float* codebook;      /* [2^bits] f32 centroid values */
  const float* rotation_t;    /* [d][d], rotation_t[k * d + j] = R[j][k]; NULL = identity */
  const uint8_t* signs;       /* NULL, or [n][(d + 7) / 8] QJL sign bits, low bit first */
  const float* resnorms;      /* [n] with signs: |r| / Norm */
  const float* qjl_t;         /* [d][d] with signs: qjl_t[j * d + i] = S[i][j] */
} EosHipTQCodes;

/* Reconstruct rerank: each candidate scored as dotRetrievalVectors(query,
 * Dequantize(codes)) -- the f32 sum += q[k] * x[k] in index order, each
 * product and sum rounded -- then (score desc, ID asc) as
 * eoship_tq_dense_rerank_device. With the primary codes this replaces
 * topTurboQuantReconstructRerankScores, with a sidecar set (e.g. 8-bit codes)
 * topTurboQuantMixedWidthRerankScores (runtime/retrieval_turboquant.go:
 * 1788-1846). Dequantize is in the un-vendored quantizer module, so the
 * dequantized vector is this build's contract after the published TurboQuant
 * dequantizers, in f64 with one rounding per coordinate: y_j =
 * codebook[code_j] (+ (sqrt(pi/2) / d) * ResNorm * sum_i (bit_i ? S[i][j] :
 * -S[i][j]) for an inner-product set, the TurboQuant_prod QJL term), x_k =
 * (float)(Norm * sum_j R[j][k] y_j) (fma chain, j ascending). Uses a
 * workspace of q * c * (d + 1) * 4 bytes. */
int eoship_tq_reconstruct_rerank_device(EosHipRuntime* rt, const EosHipTQCodes* codes,
                                        const float* d_queries, int32_t q,
                                        const int64_t* d_cand_ids, int32_t c, int32_t k,
                                        const int64_t* d_id_rank, int64_t* d_ids,
                                        float* d_scores, char** err);

/* eoship_tq_fp16_rerank_device without any device allocation: no counterpart
 * in the reference; for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). The scores
 * between its two kernels go to a static device array of 2^20 floats per GPU
 * (4 MiB, held until the process ends), so q * c must be <= 2^20 (larger is
 * refused with an error). Arguments, limits and results are those of
 * eoship_tq_fp16_rerank_device. Every call on one GPU shares that array;
 * calls from several runtimes (streams) on one GPU are ordered by a
 * per-device event chain (each call's stream waits for the previous call's
 * kernels), so they do not overwrite each other's scores. A stream under
 * graph capture is left out of that chain: replays of a captured graph that
 * overlap other calls on the same GPU race. */
int eoship_tq_fp16_rerank_device_noalloc(EosHipRuntime* rt, const float* d_queries, int32_t q,
                                         int32_t d, const uint16_t* d_rows, int64_t n,
                                         const int64_t* d_cand_ids, const float* d_cand_scores,
                                         int32_t c, int32_t k, int32_t bit_width,
                                         int32_t overfetch, const int64_t* d_id_rank,
                                         int64_t* d_ids, float* d_scores, char** err);

/* ------------------------------------------------------------------------
 * MLL packages (the reference's sealed .mll container) and plan binding.
 * ------------------------------------------------------------------------ */

/* A parsed, digest-verified package (the file bytes are copied). */
typedef struct EosHipMll EosHipMll;

/* Storage kinds of a TNSR payload. */
#define EOSHIP_MLL_Q8 1   /* int8 codes, dequantized = code * scale */
#define EOSHIP_MLL_Q4 2   /* offset-binary nibbles, low nibble first: (nibble - 8) * scale */
#define EOSHIP_MLL_F32 3  /* little-endian f32 values (logical f32, or q8/q4 held as values) */
#define EOSHIP_MLL_F16 4  /* little-endian binary16 values */
#define EOSHIP_MLL_I32 5
#define EOSHIP_MLL_I64 6

typedef struct {
  int32_t profile;          /* header profile byte */
  int32_t sections;
  int64_t strings;          /* STRG entries, the implicit "" at index 0 included */
  int64_t tensors;
  int32_t has_metadata;     /* an XMTA section that MLLMetadata.Validate accepts */
  char module_name[128];
  char module_version[64];
} EosHipMllInfo;

typedef struct {
  const char* name;         /* valid while the package is open */
  int32_t kind;             /* EOSHIP_MLL_* */
  int32_t storage_dtype;    /* the TNSR entry's dtype byte */
  int32_t rank;
  int64_t dims[8];
  int64_t elements;
  const uint8_t* data;      /* payload inside the package's copy of the file */
  uint64_t bytes;
  float scale;              /* tensor_scales[name] (0 when absent) */
} EosHipMllTensor;

/* Reads an MLL file image: header, section directory, the BLAKE3 digest of
 * every section body (XKBI, the offline kernel images, is skipped without
 * reading its bytes), STRG, TNSR and the XMTA metadata (version, module name
 * and version, artifact JSON, logical dtypes, finite non-negative
 * tensor_scales). A packed Q8/Q4 tensor without a positive scale must hold
 * only zero codes. Replaces DecodeMLL / ReadFile (artifact/eos/mll.go:
 * 332-360, 404-420) and decodeWeightFileFromMLLReader + decodeTensorEntry
 * (runtime/weight_file.go:248-415). */
int eoship_mll_open(const uint8_t* data, uint64_t bytes, EosHipMll** out, char** err);
void eoship_mll_close(EosHipMll* mll);
int eoship_mll_info(const EosHipMll* mll, EosHipMllInfo* info, char** err);
/* Body of a section by its 4-character tag (XKBI is refused). The pointer
 * stays valid while the package is open. mll.Reader.Section. */
int eoship_mll_section(const EosHipMll* mll, const char* tag, const uint8_t** body,
                       uint64_t* size, char** err);
/* A tensor by name (name != NULL) or by TNSR index. */
int eoship_mll_tensor(const EosHipMll* mll, int64_t index, const char* name,
                      EosHipMllTensor* out, char** err);
/* BLAKE3 (hash mode, 32-byte digest) of a buffer: the section digest. */
int eoship_blake3(const uint8_t* data, uint64_t bytes, uint8_t* digest32, char** err);

#define EOSHIP_PLAN_COMPACT_EMBEDDER 1
#define EOSHIP_PLAN_BERT_EMBEDDER 2

typedef struct {
  int32_t route;            /* EOSHIP_PLAN_* */
  int32_t layers;           /* encoder layers in the plan */
  int32_t distinct_layers;  /* distinct weight sets (tied layers share one) */
  int32_t model_dim, heads, hidden_dim, vocab, max_sequence, output_dim;
  int32_t batched;          /* 1: inputs [B, T]; 0: [T] */
  int32_t steps;            /* plan steps of the entry that were matched */
  EosHipCompactOptions options;  /* the plan's graph options (attend_padding: 1
                                  * for softmaxRows, 0 for masked_softmax) */
  char entry[64], token_input[64], mask_input[64], output_name[64];
  /* BERT family (route EOSHIP_PLAN_BERT_EMBEDDER) only: */
  int32_t pooling;            /* 0 masked_mean, 1 cls */
  int32_t type_vocab;         /* token type table rows */
  int32_t weights_quantized;  /* 1: f32/f16 dense weights, quantized at bind to int8
                               * per output channel (the q8 encoder); 0: q8/q4 payloads
                               * used as stored */
  int32_t reserved;
  double ln_eps;              /* the step's epsilon */
  char type_input[64];        /* token_type_ids input; max_sequence holds the
                               * position table rows */
} EosHipMllPlan;

/* Matches an entry's step list (NULL: the embedding_manifest's batch entry,
 * else the only entry point). An entry holding a bert_embedder step (the
 * pretrained-BERT importer's module, runtime/pretrained_bert_importer.go:
 * 901-1009) classifies as EOSHIP_PLAN_BERT_EMBEDDER when it is that step and
 * its return: attributes read as bertEmbedderConfigFromAttrs reads them
 * (runtime/backend/bert_embedder_ops.go:35-77: num_hidden_layers,
 * num_attention_heads, epsilon, hidden_act "gelu", pooling masked_mean or
 * cls), 8 + 16 L inputs (three i32 [B, T] entry inputs, then f32/f16/q8/q4
 * tensors of the shapes the reference validates), within the fused
 * encoder's shapes. Otherwise it is matched against the family-(a) encoder
 * graph by value flow and kernel op class:
 * gather + dequant of the token table; per layer q/k/v = x W, kT, q kT
 * (optionally scale rsqrt_rhs_rows), softmax or masked_softmax, p v, W_o,
 * binary_add + layernorm, W_up, gelu, W_down, binary_add + layernorm; then
 * normalize and mean_pool(mask) returned. Anything else is reported as "not
 * handled" with the step. In the spirit of classifyCUDAKernel
 * (runtime/backends/cuda/native_linux.go:3783-3803) over the plan that
 * ExecuteSymbolic runs (runtime/backend/symbolic.go:17-172). */
int eoship_mll_classify(const EosHipMll* mll, const char* entry, EosHipMllPlan* plan, char** err);

/* Classifies the entry and binds its weights. BERT route: the fused BERT
 * encoder with the step's heads, epsilon, erf GELU and pooling; q8/q4 dense
 * weights keep their codes and per-tensor scale, f32/f16 dense weights are
 * quantized per output channel (scale max|row| / 127, codes rint(w / scale)),
 * every other tensor is dequantized to f32; run it with
 * eoship_encoder_forward[_device] on ids, types and mask [batch][tokens]
 * (attend_padding must be -1 or 0: BERT attention is masked). Compact route:
 * (int8 codes of packed Q8, Q4 unpacked, per-tensor scales; tied layers
 * share one device copy) the fused compact encoder; run it with
 * eoship_encoder_forward[_device] on tokens and mask [batch][tokens].
 * attend_padding: -1 takes the plan's own
 * softmax semantics (the [B, T] entry run as given, padding included); 0
 * attends each sequence's mask != 0 positions only (EmbeddingModel's batches,
 * which group sequences by length, runtime/embedding_model.go:689-691).
 * plan (optional) receives the classification with the options used. */
int eoship_encoder_bind_mll(EosHipRuntime* rt, const EosHipMll* mll, const char* entry,
                            int32_t attend_padding, EosHipEncoder** out, EosHipMllPlan* plan,
                            char** err);

/* ------------------------------------------------------------------------
 * Retrieval plans: a dot / cosine / l2_distance score step, topk and the
 * gathers of candidate ids, scores and document rows (runtime/retrieval.go:
 * 51-112; examples/retrieve.eos, candidates.eos, packed_candidates.eos).
 * ------------------------------------------------------------------------ */

#define EOSHIP_SCORE_DOT 1     /* dotRows, tensor_ops.go:1967-1997: f32 sum in c order */
#define EOSHIP_SCORE_COSINE 2  /* cosineRows, :1999-2057: f64 dot and norms, f32 result */
#define EOSHIP_SCORE_L2 3      /* l2DistanceRows, :2059-2089: f64 sum of f32 differences */

typedef struct {
  int32_t op;          /* EOSHIP_SCORE_* */
  int32_t k;           /* topk limit (1 <= k <= min(n, 8192)); 0: scores only */
  int32_t docs_q4;     /* 0: documents are f32 values; 1: a packed q4 tensor */
  float docs_scale;    /* q4: value = (nibble - 8) * docs_scale */
  int32_t batched;     /* 1: documents [q][n][d], candidate ids [q][n] (the [Q, D] x
                        * [Q, N, D] score layout); 0: documents [n][d] and ids [n]
                        * shared by every query */
} EosHipScoreSpec;

/* Scores of every (query, document row) into d_scores [q][n] (bit-identical
 * to the host ops), then, with k > 0, the top k rows per query by score
 * descending and row index ascending (topKTensor, tensor_ops.go:2124-2193)
 * and its gathers: d_top_index [q][k] (i32 row indices, as topk returns),
 * d_top_ids [q][k] (candidate ids gathered at those rows; the row index when
 * d_candidate_ids is NULL), d_top_scores [q][k], d_top_docs [q][k][d]
 * (document values as f32). Any top output may be NULL. Queries are f32
 * [q][d] (d <= 4096); k > n is refused as the reference refuses it. Uses
 * the runtime workspace (q * k * 12 bytes). Enqueued on the runtime stream. */
int eoship_score_topk_device(EosHipRuntime* rt, const EosHipScoreSpec* spec,
                             const float* d_queries, int32_t q, int32_t d, const void* d_docs,
                             int64_t n, const int64_t* d_candidate_ids, float* d_scores,
                             int32_t* d_top_index, int64_t* d_top_ids, float* d_top_scores,
                             float* d_top_docs, char** err);

/* Plan outputs, in the entry's return order. */
#define EOSHIP_RET_SCORES 1      /* [n] / [Q, n] scores */
#define EOSHIP_RET_TOP_INDEX 2   /* topk indices (i32) */
#define EOSHIP_RET_TOP_IDS 3     /* gather(candidate_ids, topk) (i64) */
#define EOSHIP_RET_TOP_SCORES 4  /* gather(scores, topk) */
#define EOSHIP_RET_TOP_DOCS 5    /* gather(docs, topk) */
#define EOSHIP_RET_PACK 6        /* pack_candidates(ids, scores, docs) */

typedef struct EosHipRetrieval EosHipRetrieval;

typedef struct {
  int32_t op;               /* EOSHIP_SCORE_* */
  int32_t k;                /* topk limit, 0 when the plan has no topk */
  int32_t batched;          /* 1: queries [Q, D], documents [Q, N, D] */
  int32_t docs_param;       /* 1: documents are a param bound from the package */
  int32_t has_candidate_ids;
  int32_t docs_q4;          /* param documents stored as packed q4 */
  int64_t docs_rows;        /* param documents: N */
  int32_t dim;              /* param documents: D (0 when documents are an input) */
  int32_t n_outputs;
  int32_t outputs[8];       /* EOSHIP_RET_* in return order */
  int32_t steps;
  char entry[64], query_input[64], docs_input[64], ids_input[64];
} EosHipRetrievalPlan;

/* Matches an entry's steps: launch_kernel of op class dot / cosine /
 * l2_distance on (query, documents), optionally topk(k) and gathers of the
 * candidate ids, the scores and the documents at the topk indices, an
 * optional pack_candidates, and the return. Anything else is "not handled". */
int eoship_mll_classify_retrieval(const EosHipMll* mll, const char* entry,
                                  EosHipRetrievalPlan* plan, char** err);
/* Classifies the entry and uploads param documents (packed q4 stays packed). */
int eoship_retrieval_bind_mll(EosHipRuntime* rt, const EosHipMll* mll, const char* entry,
                              EosHipRetrieval** out, EosHipRetrievalPlan* plan, char** err);
/* Runs a bound retrieval plan (see eoship_score_topk_device for the
 * buffers); d_docs are f32 document values, NULL when the plan binds them
 * (n and the width then come from the package). */
int eoship_retrieval_run_device(EosHipRuntime* rt, EosHipRetrieval* ret, const float* d_queries,
                                int32_t q, int32_t d, const float* d_docs, int64_t n,
                                const int64_t* d_candidate_ids, float* d_scores,
                                int32_t* d_top_index, int64_t* d_top_ids, float* d_top_scores,
                                float* d_top_docs, char** err);
int eoship_retrieval_release(EosHipRuntime* rt, EosHipRetrieval* ret, char** err);

/* ------------------------------------------------------------------------
 * Hadamard TurboQuant codec of NCHW tensors (the turboquant_encode /
 * turboquant_decode steps: host runtime/backend/image_ops.go:212-300, 759-790;
 * CUDA runtime/backends/cuda/native_linux.go:1812-2004). Each (n, y, x)
 * pixel's channel vector is rotated by one round of permutation, signs, a
 * normalized fast Walsh-Hadamard transform on power-of-two blocks and
 * signs, quantized to the nearest centroid, and its norm kept as an 8-bit
 * log code over [e^-16, e^16].
 * ------------------------------------------------------------------------ */

/* The tables of one rotation round and its codebook (the quantizer module's
 * Spec() for a seed and one round, which the caller provides). */
typedef struct {
  int32_t channels;          /* C, 1..512 */
  int32_t bits;              /* 2, 4 or 8 */
  const int32_t* perm;       /* [C] a permutation of 0..C-1 */
  const float* signs1;       /* [C] */
  const float* signs2;       /* [C] */
  const float* centroids;    /* [2^bits] */
  const float* boundaries;   /* [2^bits - 1], non-decreasing */
} EosHipHadamardSpec;

typedef struct EosHipHadamardTQ EosHipHadamardTQ;

/* Validates the tables and uploads them (host pointers). */
int eoship_hadamard_tq_bind(EosHipRuntime* rt, const EosHipHadamardSpec* spec,
                            EosHipHadamardTQ** out, char** err);
/* d_input f32 [n][C][height][width] -> d_coords u8 [n][C][height][width]
 * centroid indices and d_norm_codes u8 [n][height][width] (the q_norm code
 * of quantizeQNorm). */
int eoship_hadamard_tq_encode_device(EosHipRuntime* rt, EosHipHadamardTQ* h, const float* d_input,
                                     int32_t n, int32_t height, int32_t width, uint8_t* d_coords,
                                     uint8_t* d_norm_codes, char** err);
/* The inverse: indices above the codebook clamp to its last centroid. */
int eoship_hadamard_tq_decode_device(EosHipRuntime* rt, EosHipHadamardTQ* h,
                                     const uint8_t* d_coords, const uint8_t* d_norm_codes,
                                     int32_t n, int32_t height, int32_t width, float* d_out,
                                     char** err);
int eoship_hadamard_tq_release(EosHipRuntime* rt, EosHipHadamardTQ* h, char** err);

#ifdef __cplusplus
}
#endif

#endif /* EOSHIP_H */
