// Kernel argument blocks of the encoder code object, shared with the host
// shim. f16 tensors are passed as uint16_t pointers (bit patterns).
#ifndef EOSHIP_ENC_ARGS_H
#define EOSHIP_ENC_ARGS_H

#include <stdint.h>

// Packs the active (mask != 0) positions of a [batch][tokens] mask into rows:
// row r holds sequence row_b[r], position row_t[r]; sequence b owns rows
// [seq_off[b], seq_off[b] + seq_cnt[b]).
struct EncPackArgs {
  const int32_t* mask;   // [batch][tokens]
  int32_t* row_b;        // [batch*tokens]
  int32_t* row_t;        // [batch*tokens]
  int32_t* seq_off;      // [batch]
  int32_t* seq_cnt;      // [batch] active positions (the attention keys)
  int32_t* total;        // [1] active rows
  int batch, tokens;
  int all_active;        // 1: every position is packed, whatever the mask says
  // Rows per sequence that carry a query (seq_cnt, plus one when cls_row is
  // set and position 0 is masked: that position then gets a row of its own
  // after the active ones, computed like any row but never a key, because
  // CLS pooling reads position 0 whatever the mask says).
  int32_t* seq_q;        // [batch]
  int cls_row;
  // Every position's ids are range-checked (as the reference checks the
  // whole [B, T] input, masked positions included): status[0] = 1 on an id
  // outside [0, vocab) or a type outside [0, ntype). ids may be NULL (no check).
  const int32_t* ids;
  const int32_t* type_ids;  // or NULL (all 0)
  int vocab, ntype;
  int32_t* status;
  // Optional [batch]: the sequences ordered by key count, longest first (ties
  // by index), written by eos_enc_pack; attention dispatches its workgroups
  // in this order, so that the longest ones start first.
  int32_t* order;
};

// mode 0 (BERT): token + position + type, then affine LayerNorm.
// mode 1 (compact): token + role, then RoPE with the rotation table `pos`
//   ([npos][hidden] f32: cos, sin of each column pair); gamma/beta unused.
struct EncEmbedArgs {
  const int32_t* ids;       // [batch][tokens]
  const int32_t* type_ids;  // [batch][tokens] or NULL (all 0): type or role ids
  const int32_t* row_b;
  const int32_t* row_t;
  const int32_t* total;
  const float* tok;         // [vocab][hidden]
  const float* pos;         // mode 0: [npos][hidden]; mode 1: rotation table
  const float* typ;         // [ntype][hidden] type or role table
  const float* gamma;
  const float* beta;
  uint16_t* out;            // [rows][hidden] f16
  int32_t* status;          // set to 1 on an out-of-range id
  int tokens, hidden, vocab, npos, ntype;
  float eps;
  int mode;
  int8_t* q8;               // optional int8 copy of out, as for EncLnArgs
  float* qscale;
};

// out[m][n] = epi(scale[n] * sum_k a[m][k] w[n][k] + bias[n]) for m < *rows.
// w holds int8 codes stored as f16 (exact), [n][k] (HF [out, in] layout).
// epi: 0 identity, 1 erf GELU, 2 tanh GELU, 3 + residual[m][n] (residual may
// alias out). Rows past *rows are skipped.
struct EncGemmArgs {
  const uint16_t* a;       // [rows][k] f16
  const uint16_t* w;       // [n][k] f16 codes
  const float* wscale;     // [n]
  const float* bias;       // [n]
  uint16_t* out;           // [rows][n] f16
  const int32_t* rows;     // device row count
  const uint16_t* residual;  // epi 3: [rows][n] f16
  int max_rows, n, k, epi;
  uint16_t* vt;            // optional: columns >= vt_col0 go to vt[col - vt_col0][row]
  int vt_col0, vt_ld;      // (vt rows hold vt_ld entries, the first max_rows rounded up to 8 + 72 padding)
  // int8 kernels (eos_enc_gemm8_*): A as int8 codes with one f32 scale per
  // row (a = a8 * ascale[row]) and W as int8 codes; a and w are unused.
  const int8_t* a8;        // [rows][k]
  const float* ascale;     // [rows]
  const int8_t* w8;        // [n][k]
};

// Fused layer tail of the BERT family for one block of rows: O projection +
// bias + residual, affine LayerNorm, FFN up (W8A8 on int8 MFMA) + bias +
// GELU, FFN down + bias + residual, affine LayerNorm. The same rounding
// points as the unfused kernels (f16 after each residual add, after each
// LayerNorm and after the GELU; int8 codes of the first LayerNorm's f32
// output), with the intermediate kept in LDS. h is read as the residual and
// overwritten with the layer output (rows below *rows), together with its
// int8 codes h8 / scales hs; h1 receives the first LayerNorm's f16 output
// (the FFN's residual).
// Workgroup size of the fused tail kernels (4 down + 4 up wavefronts).
#define EOS_TAIL_THREADS 512
struct EncTailArgs {
  const uint16_t* ctx;     // [rows][hidden] f16 attention context
  uint16_t* h;             // [rows][hidden] f16 layer input -> layer output
  uint16_t* h1;            // [rows][hidden] f16 scratch
  int8_t* h8;              // [rows][hidden] int8 codes of the output
  float* hs;               // [rows] their scales
  // Weights in MFMA fragment order: block (nt, ks) = the 64 lanes' operands
  // of output rows 32 nt .. + 31 at K step ks (f16: 16 K values, 8 per lane
  // half; int8: 32 K values, 16 per lane half), 1 KB per block.
  const uint16_t* w_o;     // [hidden][hidden] codes as f16, fragment order
  const float* s_o;
  const float* b_o;
  const float* g1;
  const float* be1;
  const int8_t* w_1;       // [inter][hidden] int8 codes, fragment order
  const float* s_1;
  const float* b_1;
  const uint16_t* w_2;     // [hidden][inter] codes as f16, fragment order
  const float* s_2;
  const float* b_2;
  const float* g2;
  const float* be2;
  const int32_t* rows;     // device row count
  int max_rows, inter;
  float eps;
  int gelu;                // 1 erf, 2 tanh
  // This launch's rows: block b starts at row0 + b * (its block rows), and
  // rows at or past min(*rows, row_cap) are left to another launch.
  int row0, row_cap;
};

// In-place affine LayerNorm of h [rows][hidden] f16 (hidden % 8 == 0, <= 1024).
struct EncLnArgs {
  uint16_t* h;
  const float* gamma;
  const float* beta;
  const int32_t* rows;
  int max_rows, hidden;
  float eps;
  // Optional (q8 != NULL): each output row also as int8 codes, q8 = rint(y /
  // qscale) with qscale = max|y| / 127 (0 for a zero row), y the f32 result.
  int8_t* q8;              // [rows][hidden]
  float* qscale;           // [rows]
};

// Masked multi-head attention over packed rows: every active row of a
// sequence attends to every active row of the same sequence.
struct EncAttnArgs {
  const uint16_t* qkv;     // [rows][3*hidden] f16: q | k (| v unused), head-major
  const uint16_t* vt;      // [hidden][vt_ld] f16: V transposed (feature-major)
  uint16_t* ctx;           // [rows][hidden] f16
  const int32_t* seq_off;
  const int32_t* seq_cnt;  // keys per sequence
  const int32_t* seq_q;    // query rows per sequence (>= seq_cnt), or NULL (= seq_cnt)
  int batch, heads, hidden, max_len, vt_ld;
  float scale_log2;        // log2(e) / sqrt(head_dim)
  // Optional: counts (per wavefront) the exponent-reference moves after a
  // sequence's first key block, the lazy-rescale path trained models reach.
  int32_t* moves;
  // Optional [batch]: workgroup z serves sequence order[z] (else z).
  const int32_t* order;
};

// General-shape BERT path (hidden widths and head dims the MFMA kernels do
// not take): f32 activations, one launch per operation.
//   eos_enc_gen_embed  token + position + type, affine LayerNorm -> y, h16
//   eos_enc_gen_dense  y[m][n] = epi(sum_k x[m][k] (w[n][k] wscale[n]) + bias[n])
//                      (+ res[m][n]); epi 0 identity, 1 erf GELU, 2 tanh GELU
//   eos_enc_gen_ln     affine LayerNorm of y in place (and h16)
//   eos_enc_gen_attn   softmax(q k^T / sqrt(hd)) v per (sequence, head, query)
// Rows are the packed rows of eos_enc_pack (m < *total).
struct EncGenArgs {
  const int32_t* ids;
  const int32_t* type_ids;  // or NULL
  const int32_t* row_b;
  const int32_t* row_t;
  const int32_t* total;
  const float* tok;         // [vocab][hidden]
  const float* pos;         // [npos][hidden]
  const float* typ;         // [ntype][hidden]
  const float* gamma;
  const float* beta;
  const float* x;           // dense input [rows][k]; attention: qkv [rows][3 hidden]
  float* y;                 // [rows][n] (LN, embed: [rows][hidden]; attention: ctx)
  const float* res;         // dense residual [rows][n] or NULL
  const int8_t* w;          // [n][k] int8 codes
  const float* wscale;      // [n]
  const float* bias;        // [n]
  uint16_t* h16;            // embed / LN: f16 copy of the rows (pooling input) or NULL
  int32_t* status;          // embed: 1 on an out-of-range id
  const int32_t* seq_off;   // attention
  const int32_t* seq_cnt;
  const int32_t* seq_q;     // or NULL
  int n, k, epi;
  int hidden, heads, tokens, vocab, npos, ntype, max_rows;
  float eps;
};

// mode 0: masked mean pool, then L2 normalize -> out [batch][hidden].
// mode 1: L2 normalize every row, masked mean pool, then (proj != NULL)
//   times proj [hidden][odim] -> out [batch][odim] (odim = hidden without).
// Two launches: eos_enc_pool_part (chunk partial sums into part) and
// eos_enc_pool (chunk sums in order, mean, normalize or projection).
constexpr int kPoolChunk = 64;   // rows per partial sum
struct EncPoolArgs {
  const uint16_t* h;       // [rows][hidden] f16
  const int32_t* seq_off;
  const int32_t* seq_cnt;
  float* out;
  const float* proj;       // mode 1 only, [hidden][odim] f32, or NULL
  float* part;             // [batch][nchunk][hidden] f32 partial sums
  int batch, hidden, mode, odim, nchunk;
  // NULL, or the [batch][tokens] mask when every position was packed (row r
  // of a sequence is its position r): only rows whose mask is non-zero are
  // pooled, and the mean divides by their count.
  const int32_t* mask;
  int tokens;
  // mode 0 only: non-NULL selects CLS pooling (position 0's row, then L2
  // normalize): the sequence's first row when position 0 is active, else the
  // query-only row after the active ones (seq_q > seq_cnt).
  const int32_t* cls_seq_q;
  // eos_enc_gen_pool: the f32 rows [rows][hidden] (h is not read).
  const float* h32;
};

// Tiny embed pipeline (examples/embed.eos): gather f16 table rows, multiply by
// an f16 [dim][edim] projection (f32, k ascending), L2-normalize each row,
// f16 out.
struct EmbedTinyArgs {
  const uint16_t* table;   // [vocab][dim] f16
  const uint16_t* proj;    // [dim][edim] f16
  const int32_t* tokens;   // [n]
  uint16_t* out;           // [n][edim] f16
  int32_t* status;         // set to 1 on an out-of-range token
  int n, vocab, dim, edim;
};

#endif  // EOSHIP_ENC_ARGS_H
