// Kernel argument blocks of the retrieval-plan code object (row scoring and
// candidate gathers), shared with the host shim.
#ifndef EOSHIP_RET_ARGS_H
#define EOSHIP_RET_ARGS_H

#include <stdint.h>

constexpr int kRetMaxDim = 4096;  // query width the scoring kernel stages in LDS
constexpr int kRetThreads = 256;

// Scores of every (query, document row): op 1 dot, 2 cosine, 3 l2 distance.
// Documents are f32 values or a packed q4 tensor (offset-binary nibbles of
// the flattened tensor, low nibble first, value = (nibble - 8) * scale).
struct RetScoreArgs {
  const float* queries;    // [q][d]
  const float* docs;       // [batched ? q : 1][n][d] values, or NULL
  const uint8_t* docs_q4;  // the same tensor packed, or NULL
  float scale;
  float* scores;           // [q][n]
  long long n;
  int d, q, batched, op;
};

// Top-k gathers: per query, the selected row indices (sel, from the top-k
// selection) index the candidate ids and the document rows.
struct RetGatherArgs {
  const long long* sel;        // [q][k]
  const int64_t* cand_ids;     // [batched ? q : 1][n] or NULL
  const float* docs;
  const uint8_t* docs_q4;
  float scale;
  int32_t* top_index;          // [q][k] or NULL
  int64_t* top_ids;            // [q][k] or NULL
  float* top_docs;             // [q][k][d] or NULL
  long long n;
  int d, q, k, batched;
};

#endif
