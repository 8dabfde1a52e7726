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

// Hadamard TurboQuant codec of NCHW tensors (one vector per (n, y, x) pixel
// over the channels): the spec tables of one rotation round.
constexpr int kHqMaxChannels = 512;
constexpr int kHqThreads = 64;   // pixels per workgroup, one per thread
struct HqArgs {
  const float* input;      // encode: [n][c][h][w]
  const uint8_t* coords_in;  // decode: [n][c][h][w] centroid indices
  const uint8_t* norms_in;   // decode: [n][h][w] 8-bit log norm codes
  uint8_t* coords;         // encode out
  uint8_t* norms;          // encode out
  float* out;              // decode out [n][c][h][w]
  const int32_t* perm;     // [c]
  const float* signs1;     // [c]
  const float* signs2;     // [c]
  const float* centroids;  // [levels]
  const float* boundaries; // [levels - 1]
  long long pixels;        // n * h * w
  int channels, hw, levels;
};

#endif
