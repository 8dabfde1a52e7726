// Kernel argument blocks shared by the gfx950 code objects and the host shim.
// Each kernel takes one of these by value; keep field order and types in sync
// on both sides (this header is the only definition).
#ifndef EOSHIP_TQ_ARGS_H
#define EOSHIP_TQ_ARGS_H

#include <stdint.h>

struct TqPrepArgs {
  const float* queries;  // [q][d]
  const float* rot_t;    // [d][d], rot_t[k*d + j] = R[j][k]; NULL = identity
  int8_t* bfrag;         // [ks][ncb][64][16] query fragments
  float* alpha;          // [32*ncb/2]
  float* tau;            // [32*ncb/2] reset to -inf
  uint32_t* cand_count;  // [32*ncb/2] reset to 0
  int16_t* qs_out;       // optional [q][d]
  double* qrot;          // [32*ncb/2][d] rotated columns (written by eos_tq_rotate)
  float* lonorm;         // optional [32*ncb/2]: ||lo||_2 of the column, rounded up
  int q, d, ks, ncb, qmax;
  float cb_scale;
  // Column -> source row: column c belongs to group c / group (a query of the
  // pass) and slot c % group; slots >= group_live are zero columns. The flat
  // scan uses group = group_live = 1 (column c = query c).
  int group, group_live;
};

struct TqPackArgs {
  const uint8_t* codes;  // [n][row_bytes] reference layout
  uint32_t* packed;      // [ntiles][nload][64][4] dwords
  long long n;
  long long total_dwords;
  int d, bits, row_bytes, ks, nload;
};

struct TqScanArgs {
  const int32_t* packed;   // [ntiles][nload][64][4] dwords
  const float* norms;      // [ntiles*32], zero past n
  const int8_t* bfrag;     // [ks][ncb][64][16]
  const float* alpha;      // [32*nqg]
  const float* tau;        // [32*nqg] filter thresholds
  unsigned long long* cand;               // [32*nqg][cap] rank keys
  uint32_t* cand_count;    // [32*nqg]
  float* out_scores;       // dense/sample output [q][out_stride]
  int32_t* out_dots;       // dense output (optional)
  const int* gate;         // non-NULL: run only if some gate[i] != 0, i < q
  const float* lonorm;     // high-half filter: [32*nqg] ||lo||_2 per column (rounded up)
  const float* tile_cn;    // high-half filter: [ntiles][2] max ||C[codes]||_2 of the tile (rounded up), max Norm
  long long n;             // valid vectors
  long long out_begin;     // dense: vector index of column 0
  long long out_count;     // dense: columns
  long long out_stride;
  long long tile_begin;    // first physical tile
  long long tile_step;     // logical tile j -> tile_begin + j * tile_step
  int ntiles;              // logical tiles in this launch
  int q;                   // live query columns
  int cap;                 // candidate capacity per query
  int mode;                // 0 dense, 1 filter, 2 sample (3: high-half filter, kernels _h)
  uint32_t lut0, lut1, lut2, lut3;
};

struct TqSelectArgs {
  const float* rows;       // [nrows][stride] scores
  const int* status;       // mode 1: rows with status 0 are skipped (NULL = all)
  float* tau;              // mode 0 output [nrows]
  long long* ids;          // mode 1 output [nrows][kk]
  float* scores;           // mode 1 output [nrows][kk]
  long long n;             // elements per row
  long long stride;
  int kk;                  // rank
  int mode;                // 0: tau = score of the kk-th best; 1: sorted top-kk
  int nrows;
  const long long* id_map; // mode 1, optional [n]: element i is reported as id id_map[i]
  // mode 2: each row is split into nchunks equal chunks (grid.y); a chunk's
  // top-kk rank keys go unsorted to keys_out[(row * nchunks + chunk) * kk ..],
  // padded with 0 (below every rank key), and chunk 0 sets counts_out[row] =
  // nchunks * kk (the list length eos_tq_finalize merges).
  int nchunks;
  unsigned long long* keys_out;
  uint32_t* counts_out;
};

struct TqFinalizeArgs {
  const unsigned long long* cand;
  uint32_t* cand_count;   // rewritten with the live (nonzero) entry count
  long long* ids;     // [q][kk]
  float* scores;      // [q][kk]
  int* status;        // [q]: 0 ok, 1 too few candidates, 2 overflow
  int cap, kk, q;
  const long long* id_map;  // optional [n]: corpus position p is reported as id id_map[p]
};

// MaxSim over documents of tiles_per_doc consecutive tiles: per query group
// g (32 token columns) and document, the pairwise-tree sum over the 32 token
// slots of each token's best score in the document.
struct TqMaxsimArgs {
  const int32_t* packed;
  const float* norms;
  const int8_t* bfrag;
  const float* alpha;      // [32 * groups] per token column
  float* out;              // [groups][out_stride]
  long long doc_begin;     // first document
  long long ndocs;         // documents in this launch
  long long out_stride;
  int tiles_per_doc;
  int groups;              // live query groups of the launch (all its passes)
  uint32_t lut0, lut1, lut2, lut3;
  // bfrag holds the fragments of every prepared query, [ks][frag_ncb][64];
  // the launch uses column blocks from frag_cb0 on.
  int frag_ncb, frag_cb0;
  // Pass p = blockIdx.y scores query groups [nqg p, nqg p + nqg) of the
  // launch (alpha, out, tau, gate, lonorm and the doc lists offset by it).
  // Document i of a pass is doc_begin + i * doc_stride (doc_stride 0 = 1),
  // or, with doc_list, doc_list[p * list_cap + i] for i < min(count, cap),
  // count = list_count[p]; in that mode the exact scores leave as rank keys
  // cand[group][i] (0 when below tau[group]) with cand_count[group] = count.
  long long doc_stride;
  const uint32_t* doc_list;
  unsigned long long* cand;
  uint32_t* cand_count;
  const float* tau;        // [groups]
  const int* gate;         // or NULL: a pass runs only if a live group's gate is set
  // High-half bound filter (the _h kernels): documents whose score bound
  // reaches tau of some live group of the pass are appended to
  // list[p * list_cap ..] (count list_count[p], entries past cap dropped).
  const float* lonorm;     // [32 * groups] ||lo||_2 of each column, rounded up
  const float* tile_cn;    // [2 * tiles] largest ||C[codes]||_2 of the tile, largest Norm
  uint32_t* list;
  uint32_t* list_count;
  int list_cap;
};

// Parent (multivector) aggregation over child scores: parent p owns children
// [off[p], off[p+1]) of each score row; out[q][p] = f32(mean of its best
// min(top_n, 5, count) child scores (f64 sum in descending order) -
// penalty * l1p[p]); parents without children get -inf.
struct TqParentArgs {
  const float* scores;      // [qb][stride] child scores
  const long long* off;     // [np + 1]
  const double* l1p;        // [np] log1p(child count)
  float* out;               // [qb][np]
  long long np, stride;
  double penalty;
  int top_n, qb;
};

// Best child of each selected parent: the highest child score, ties to the
// lower child index.
struct TqParentBestArgs {
  const float* scores;        // [qb][stride] child scores
  const long long* off;       // [np + 1]
  const long long* parents;   // [qb][kk] selected parent ids
  long long* best_child;      // [qb][kk]
  float* best_score;          // [qb][kk]
  long long stride;
  int kk, qb;
};

// Exact rescoring of the high-half filter's kept ids, in place: each entry of
// cand[q] (a list that did not overflow) becomes the exact rank key when the
// exact score reaches tau, else 0.
struct TqRescoreArgs {
  const uint8_t* codes;    // [n][16 * rs] reference-layout code rows, zero-padded
  const float* norms;
  const int16_t* qs;       // [q][d] int16 queries
  const float* alpha;
  const float* tau;
  unsigned long long* cand;
  const uint32_t* cand_count;
  long long n;               // corpus vectors (ids >= n are dropped)
  int q, d, rs, cap;         // rs: 16-byte chunks per code row (<= 32)
  uint32_t lut0, lut1, lut2, lut3;
};

// Per tile of 32 vectors, the largest ||C[codes]||_2 (rounded up to f32) and
// the largest Norm.
struct TqTileNormArgs {
  const uint8_t* codes;    // [n][row_bytes] reference layout
  const float* norms;      // [n]
  float* tile_cn;          // [ntiles][2]: {max ||C[codes]||_2, max Norm}
  long long n;
  int d, bits, row_bytes;
  int cb[16];              // codebook grid values
};

// Corpus encoder (MSE stage): rows of x -> reference-layout codes + norms,
// 32 vectors per workgroup (d <= 1024).
struct TqEncodeArgs {
  const float* x;          // [n][d]
  const float* rot_t;      // [d][d], rot_t[k*d + j] = R[j][k]; NULL = identity
  uint8_t* codes;          // [n][row_bytes]
  float* norms;            // [n]
  long long n;
  int d, bits, row_bytes;
  float cb_scale;
  int cb[16];
};

// Inner-product layout (MSE codes + QJL signs + ResNorm + Norm): encode,
// query preparation and exhaustive scores.
struct TqIpArgs {
  const float* x;          // encode: [n][d]
  const float* queries;    // prepare: [q][d]
  const float* rot_t;      // [d][d], rot_t[k*d + j] = R[j][k]; NULL = identity
  const float* qjl_t;      // [d][d], qjl_t[j*d + i] = S[i][j]
  uint8_t* codes;          // [n][row_bytes] (encode out / scores in)
  uint8_t* signs;          // [n][sign_bytes]
  float* resnorms;         // [n]
  float* norms;            // [n]
  int* qs;                 // [q][d] MSE query grid
  int* ys;                 // [q][d] QJL query grid
  float* alpha;            // [q]
  float* beta;             // [q]
  float* scores;           // [q][n]
  long long n;
  int d, bits, row_bytes, sign_bytes, q, qmax, qmax2;
  float cb_scale;
  int cb[16];
};

// f16 rerank sidecar: f32 rows -> the reference's half encoding.
struct TqHalfArgs {
  const float* x;          // [count]
  unsigned short* h;       // [count]
  long long count;
};

// Second stage of two-stage retrieval: exact f16-row rerank of the overfetched
// candidates of each query (eos_tq_rr_dots: one lane per candidate;
// eos_tq_rr_sort: one workgroup per query).
struct TqRerankArgs {
  const float* queries;          // [q][d]
  const unsigned short* rows;    // [n][d] halves
  const long long* cand_ids;     // [q][c] first-stage order (score desc, id asc)
  const float* cand_scores;      // [q][c] first-stage scores
  long long* out_ids;            // [q][kk]
  float* out_scores;             // [q][kk]
  float* dots;                   // [q][c] f32 rerank scores (scratch between the two kernels)
  long long n;
  int d, c, kk, rescue;
  // Optional [n]: the order of id's string ID among the corpus IDs; equal
  // rerank scores then rank by it instead of by the integer id.
  const long long* id_rank;
  const float* rows_f32;         // [n][d] f32 rows (dense rerank) instead of rows
  int vec;                       // rows allow whole 16-byte loads (d % 8 or 4, aligned)
  // 1: rows_f32 holds one row per candidate position ([q][c][d], the
  // reconstruct rerank's dequantized vectors) instead of one per id.
  int rows_by_pos;
};

// Reconstruct rerank: each candidate's dequantized vector into xhat
// [q][c][d] (eos_tq_rr_dequant), then the f32 dots of eos_tq_rr_dots_f32
// (rows by position) and eos_tq_rr_sort.
struct TqReconArgs {
  const float* rot_t;            // [d][d], rot_t[k*d + j] = R[j][k]; NULL = identity
  const unsigned char* codes;    // [n][row_bytes]
  const float* norms;            // [n]
  const float* codebook;         // [2^bits] f32 centroid values
  // Inner-product code sets (NULL otherwise): sign bits [n][(d + 7) / 8],
  // ResNorm [n], and the sketch qjl_t[j*d + i] = S[i][j].
  const unsigned char* signs;
  const float* resnorms;
  const float* qjl_t;
  const long long* cand_ids;     // [q][c]
  float* xhat;                   // [q][c][d]
  long long n;
  int d, c, bits, row_bytes;
};


// Inner-product corpus (IPQuantized rows: MSE codes of 1..3 bits + QJL sign
// bits + ResNorm + Norm) in the scan's tile layout: tile t, chunk c (K-steps
// 2c and 2c + 1), lane (m + 32 g): two dwords per K-step s,
//   L:  bit 8 b + 2 k + e = bit e of the code of fragment byte 4 k + b (e = 0, 1)
//   HS: bit 8 b + k = bit 2 of that code; bit 8 b + 4 + k = its QJL sign bit
// where fragment byte i of K-step s, lane group g is dimension 32 s + 16 g + i
// of vector 32 t + m (dimensions past d, and vectors past n: code 0, sign 0).
struct TqIpPackArgs {
  const uint8_t* codes;    // [n][row_bytes] reference layout, low bits first
  const uint8_t* signs;    // [n][sign_bytes]
  const float* norms;      // [n]
  const float* resnorms;   // [n]
  int32_t* packed;         // [ntiles][ks / 2][64][4] dwords
  float* norms_out;        // [ntiles * 32], zero past n
  float* resnorms_out;     // [ntiles * 32]
  long long n, ntiles;
  int d, ks, bits, row_bytes, sign_bytes;
};

// Inner-product scan: exact D_mse = sum Qs_j C[code_j] and D_qjl = sum Ys_i
// (2 bit_i - 1) on int8 MFMA, score = ((float)D_mse alpha + ResNorm
// ((float)D_qjl beta)) Norm; modes as TqScanArgs (0 dense, 1 keep score >=
// tau, 2 sampled tile maxima).
struct TqIpScanArgs {
  const int32_t* packed;
  const float* norms;      // [ntiles * 32]
  const float* resnorms;   // [ntiles * 32]
  const int8_t* bfrag;     // [ks][4 * nqg][64][16]
  const float* alpha;      // [32 * nqg]
  const float* beta;       // [32 * nqg]
  const int* ysum;         // [32 * nqg]
  const float* tau;        // [32 * nqg]
  unsigned long long* cand;  // [32 * nqg][cap]
  uint32_t* cand_count;    // [32 * nqg]
  float* out_scores;
  const int* gate;
  long long n, out_begin, out_count, out_stride, tile_begin, tile_step;
  int ntiles, q, cap, mode;
  uint32_t lut0, lut1;     // the 8-entry int8 codebook: bytes C[0..3], C[4..7]
  // High-half bound filter (the _h kernels, mode 1): only the MSE and QJL
  // grids' high int8 halves enter the MFMAs; kept rows go to cand as ids
  // (~id) for eos_tq_ip_rescore.
  const float* lonorm;     // [32 * nqg] ||MSE lo||_2 of each column, rounded up
  const int* kq;           // [32 * nqg] 2 sum_i max(QJL lo_i, 0) - sum Ys
  const float* tile_cn;    // [ntiles][4]: max ||C[codes]||_2 (rounded up), -, -, -
};

// Exact rescoring of the inner-product filter's kept ids (eos_tq_ip_rescore):
// entry e of cand[q] (an id ~v) becomes rank_key(score, v) when the exact
// score reaches tau[q], else 0 (finalize skips zeros). Codes and signs are
// read from the scan's tile layout.
struct TqIpRescoreArgs {
  const int32_t* packed;   // [ntiles][ks / 2][64][4]
  const float* norms;      // [ntiles * 32]
  const float* resnorms;   // [ntiles * 32]
  const int8_t* bfrag;     // the scan's query fragments [ks][4 nqg][64][16]
  const float* alpha;
  const float* beta;
  const int* ysum;
  const float* tau;
  unsigned long long* cand;
  const uint32_t* cand_count;
  long long n;
  int q, d, ks, nqg, cap;
  uint32_t lut0, lut1;
};

// Per tile of the inner-product layout: {max ||C[codes]||_2 rounded up, 0, 0,
// 0}; one thread per vector, codes from the reference rows (low bits first,
// a code may straddle two bytes).
struct TqIpTileNormArgs {
  const uint8_t* codes;    // [n][row_bytes]
  float* tile_cn;          // [ntiles][4]
  long long n;
  int d, bits, row_bytes;
  int cb[8];
};

// out[c][j] = sum over k ascending of M[j][k] in[c][k] (one f64 fma chain per
// (c, j)), mt[k * d + j] = M[j][k]; in is f32 (in32) or f64 (in64); mt NULL:
// out = in. Grid (ceil(d / 32), ceil(q / 8)).
struct TqIpMatArgs {
  const float* mt;
  const float* in32;
  const double* in64;
  double* out;
  int q, d;
};

// Per query column c < ncols (the grid): Qs and alpha from qr, Ys and beta
// from y (zero columns past q). qs / ys receive the grids when non-NULL; with
// bfrag the scan's query fragments [ks][4 * nqg][64][16] (per 32-column
// group g: MSE hi, MSE lo, QJL hi, QJL lo), ysum, tau (-inf) and cand_count
// (0) of every column too.
struct TqIpQuantArgs {
  const double* qr;        // [q][d]
  const double* y;         // [q][d]
  int* qs;                 // [q][d] or NULL
  int* ys;                 // [q][d] or NULL
  float* alpha;
  float* beta;
  int8_t* bfrag;           // or NULL
  int* ysum;               // [32 * nqg]
  float* tau;              // [32 * nqg]
  uint32_t* cand_count;    // [32 * nqg]
  int q, d, qmax, qmax2;
  float cb_scale;
  int ks, nqg;
  // bound filter inputs (frag mode, each optional): per column ||MSE lo||_2
  // rounded up and 2 sum max(QJL lo, 0) - sum Ys
  float* lonorm;           // [32 * nqg]
  int* kq;                 // [32 * nqg]
};

#endif  // EOSHIP_TQ_ARGS_H
