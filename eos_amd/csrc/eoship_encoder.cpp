// Encoder half of the eoship C ABI: binds a BERT-style q8 encoder and runs its
// forward pass (the bert_embedder step, runtime/backend/bert_embedder_ops.go:
// 101-197) on the runtime stream:
//   eos_enc_pack        active positions -> contiguous rows per sequence
//   eos_enc_embed       token + position + type, affine LayerNorm
//   per layer:  eos_enc_gemm_t* (QKV) -> eos_enc_attn_hd* -> eos_enc_gemm_t*
//               (O + residual) -> eos_enc_ln -> eos_enc_gemm_t* (FFN up + GELU)
//               -> eos_enc_gemm_t* (FFN down + residual) -> eos_enc_ln
//   eos_enc_pool        masked mean pool + L2 normalize
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "eoship_internal.h"
#include "kernels/enc_args.h"

using eoship::hip_err;
using eoship::set_err;

namespace {

// IEEE binary16 bits of an int8 code (every value in [-128, 127] is exact).
uint16_t int8_to_f16_bits(int8_t x) {
  if (x == 0) return 0;
  const uint16_t sign = x < 0 ? 0x8000 : 0;
  unsigned v = (unsigned)(x < 0 ? -(int)x : (int)x);
  int e = 0;
  while ((v >> (e + 1)) != 0) ++e;
  const unsigned mant = (v << (10 - e)) & 0x3ffu;
  return (uint16_t)(sign | ((unsigned)(e + 15) << 10) | mant);
}

struct DevLayer {
  uint16_t* w_qkv = nullptr;
  float* s_qkv = nullptr;
  float* b_qkv = nullptr;
  uint16_t* w_o = nullptr;
  float* s_o = nullptr;
  float* b_o = nullptr;
  float* g1 = nullptr;
  float* be1 = nullptr;
  uint16_t* w_1 = nullptr;
  float* s_1 = nullptr;
  float* b_1 = nullptr;
  uint16_t* w_2 = nullptr;
  float* s_2 = nullptr;
  float* b_2 = nullptr;
  float* g2 = nullptr;
  float* be2 = nullptr;
  // BERT family: int8 copies of the QKV and FFN-up codes for the W8A8 GEMMs
  // (their inputs are LayerNorm / embedding outputs, which carry int8 rows).
  int8_t* w_qkv8 = nullptr;
  int8_t* w_18 = nullptr;
  // Fused layer tail: the O, FFN-up and FFN-down codes in MFMA fragment order
  // (one 1 KB block per 32 output rows x one K step, lane-major), so that every
  // weight load of a wavefront reads 1 KB contiguously.
  uint16_t* w_of = nullptr;
  int8_t* w_1f = nullptr;
  uint16_t* w_2f = nullptr;
  // General-shape path: int8 codes of the O and FFN-down weights.
  int8_t* w_o8 = nullptr;
  int8_t* w_28 = nullptr;
};

}  // namespace

struct EosHipEncoder {
  EosHipRuntime* rt = nullptr;
  EosHipEncoderDesc desc{};
  // 0: BERT family (affine LN embeddings, pool then normalize); 1: compact
  // family (token + role with RoPE, normalize per row then pool, optional
  // output projection `proj` [hidden][odim] f32).
  int family = 0;
  // BERT family at hidden 384 / 512 / 768: O projection through the second
  // LayerNorm as one kernel per row block (eos_enc_tail_*); otherwise, or
  // when switched off, the unfused GEMM + LayerNorm launches.
  bool fused_tail = true;
  // BERT family at a hidden width or head dim the MFMA kernels do not take
  // (e.g. hidden 16, head dim 4): the f32 eos_enc_gen_* kernels run every
  // layer instead.
  bool general = false;
  // Compact family: attention scores times 1/sqrt(head dim) (else plain q kT),
  // and attention over every position of the padded input with the mask
  // selecting only the pooled rows (else over each sequence's mask != 0
  // positions).
  bool scaled_scores = true;
  bool attend_all = false;
  // BERT family pooling: 0 masked mean (the default), 1 CLS (position 0's
  // row), as bert_embedder's "pooling" attribute (bert_embedder_ops.go:
  // 150-152, 183-196).
  int pooling = 0;
  int odim = 0;
  float* proj = nullptr;
  std::vector<void*> owned;
  float *tok = nullptr, *pos = nullptr, *typ = nullptr, *eg = nullptr, *eb = nullptr;
  std::vector<DevLayer> layers;
  // activations, sized for cap_rows = batch * tokens
  size_t cap_rows = 0;
  int cap_batch = 0;
  uint16_t *h = nullptr, *qkv = nullptr, *ctx = nullptr, *mid = nullptr;
  // int8 copy of h with one scale per row (BERT family: QKV and FFN-up run on
  // int8 MFMA with these as activations)
  int8_t* h8 = nullptr;
  float* hs = nullptr;
  float* pool_part = nullptr;  // [batch][chunks][hidden] pool partial sums
  // General-shape path: f32 hidden rows, the first LayerNorm's output, q|k|v
  // rows, attention output and FFN intermediate.
  float *hf = nullptr, *h1f = nullptr, *qkvf = nullptr, *ctxf = nullptr, *midf = nullptr;
  // V of the QKV projection, feature-major [hidden][vt_ld] (zeroed padding
  // past the rows, so attention may read whole 16-byte key groups)
  uint16_t* vt = nullptr;
  int vt_ld = 0;
  int32_t *row_b = nullptr, *row_t = nullptr, *seq_off = nullptr, *seq_cnt = nullptr;
  int32_t* seq_q = nullptr;  // query rows per sequence (CLS pooling may add one)
  int32_t* seq_order = nullptr;  // sequences by key count, longest first
  int32_t *total = nullptr, *status = nullptr;
  // host-API staging
  void* io = nullptr;
  size_t io_bytes = 0;

  ~EosHipEncoder() {
    for (void* p : owned)
      if (p) hipFree(p);
    void* act[] = {h,     qkv,     ctx,     mid,   h8,    hs,   pool_part, vt, row_b,
                   row_t, seq_off, seq_cnt, seq_q, total, status, io,   hf,        h1f, qkvf,
                   ctxf,  midf,    seq_order};
    for (void* p : act)
      if (p) hipFree(p);
  }

  template <typename T>
  int upload(T** dst, const T* src, size_t count, char** err) {
    void* p = nullptr;
    if (rt->alloc(count * sizeof(T), &p, err) != 0) return 1;
    owned.push_back(p);
    hipError_t e = rt->copy_sync(p, src, count * sizeof(T), hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_err(err, "hipMemcpy(encoder weights)", e);
    *dst = static_cast<T*>(p);
    return 0;
  }

  int upload_codes(uint16_t** dst, const int8_t* src, size_t count, char** err) {
    std::vector<uint16_t> h16(count);
    for (size_t i = 0; i < count; ++i) h16[i] = int8_to_f16_bits(src[i]);
    return upload(dst, h16.data(), count, err);
  }

  // Fragment order of an [n][k] code matrix (n % 32 == 0): block (nt, ks) is
  // the 64 lanes' operands of rows 32 nt .. + 31 at K step ks, lane (l, g)
  // holding row 32 nt + l, K values ks * KS + g * KS / 2 .. + KS / 2 - 1.
  // f16 (KS = 16, 8 halves per lane) for the f16 MFMAs, int8 (KS = 32, 16
  // codes per lane) for the int8 ones.
  int upload_frag16(uint16_t** dst, const int8_t* src, int n, int k, char** err) {
    std::vector<uint16_t> f((size_t)n * k);
    size_t o = 0;
    for (int nt = 0; nt < n / 32; ++nt)
      for (int ks = 0; ks < k / 16; ++ks)
        for (int lane = 0; lane < 64; ++lane)
          for (int e = 0; e < 8; ++e)
            f[o++] = int8_to_f16_bits(src[(size_t)(32 * nt + (lane & 31)) * k + 16 * ks + 8 * (lane >> 5) + e]);
    return upload(dst, f.data(), f.size(), err);
  }
  int upload_frag8(int8_t** dst, const int8_t* src, int n, int k, char** err) {
    std::vector<int8_t> f((size_t)n * k);
    size_t o = 0;
    for (int nt = 0; nt < n / 32; ++nt)
      for (int ks = 0; ks < k / 32; ++ks)
        for (int lane = 0; lane < 64; ++lane)
          for (int e = 0; e < 16; ++e)
            f[o++] = src[(size_t)(32 * nt + (lane & 31)) * k + 32 * ks + 16 * (lane >> 5) + e];
    return upload(dst, f.data(), f.size(), err);
  }

  // Stacks [in][out] code matrices (reference layout) into one [sum out][in]
  // f16 code matrix (the kernels' layout) and its per-output-channel scales.
  int upload_codes_t(uint16_t** dst, float** scale, const int8_t* const* src, const float* s,
                     const int* outs, int parts, int in, char** err) {
    size_t total = 0;
    for (int p = 0; p < parts; ++p) total += (size_t)outs[p];
    std::vector<uint16_t> h16(total * (size_t)in);
    std::vector<float> sc(total);
    size_t o0 = 0;
    for (int p = 0; p < parts; ++p) {
      for (int o = 0; o < outs[p]; ++o) {
        sc[o0 + o] = s[p];
        for (int i = 0; i < in; ++i)
          h16[(o0 + o) * (size_t)in + i] = int8_to_f16_bits(src[p][(size_t)i * outs[p] + o]);
      }
      o0 += (size_t)outs[p];
    }
    return upload(dst, h16.data(), h16.size(), err) || upload(scale, sc.data(), sc.size(), err);
  }

  int out_dim() const { return family == 1 ? odim : desc.hidden; }

  // Packed rows: each sequence starts at a multiple of 8, so a batch needs up
  // to batch * (tokens + 7) rows.
  static size_t row_capacity(int batch, int tokens) { return (size_t)batch * (tokens + 7); }

  int ensure_activations(int batch, int tokens, char** err) {
    const size_t rows = row_capacity(batch, tokens);
    if (rows <= cap_rows && batch <= cap_batch) return 0;
    void* act[] = {h,     qkv,   ctx,     mid,     h8,    hs,     pool_part, vt,  row_b, row_t,
                   seq_off, seq_cnt, seq_q, total, status, hf,  h1f,       qkvf, ctxf, midf,
                   seq_order};
    for (void* p : act)
      if (p) hipFree(p);
    hf = h1f = qkvf = ctxf = midf = nullptr;
    seq_order = nullptr;
    h = qkv = ctx = mid = nullptr;
    h8 = nullptr;
    hs = nullptr;
    pool_part = nullptr;
    vt = nullptr;
    row_b = row_t = seq_off = seq_cnt = seq_q = total = status = nullptr;
    cap_rows = 0;
    cap_batch = 0;
    const size_t H = desc.hidden, F = desc.intermediate;
    if (rt->alloc(rows * H * 2, reinterpret_cast<void**>(&h), err) ||
        rt->alloc(rows * 3 * H * 2, reinterpret_cast<void**>(&qkv), err) ||
        rt->alloc(rows * H * 2, reinterpret_cast<void**>(&ctx), err) ||
        rt->alloc(rows * F * 2, reinterpret_cast<void**>(&mid), err) ||
        rt->alloc(rows * H, reinterpret_cast<void**>(&h8), err) ||
        rt->alloc(rows * 4, reinterpret_cast<void**>(&hs), err) ||
        // chunks of any later shape within the caps: batch' * ceil(tokens' /
        // 256) <= rows / 256 + batch
        rt->alloc((rows / kPoolChunk + (size_t)batch) * H * 4,
                  reinterpret_cast<void**>(&pool_part), err) ||
        rt->alloc(rows * 4, reinterpret_cast<void**>(&row_b), err) ||
        rt->alloc(rows * 4, reinterpret_cast<void**>(&row_t), err) ||
        rt->alloc((size_t)batch * 4, reinterpret_cast<void**>(&seq_off), err) ||
        rt->alloc((size_t)batch * 4, reinterpret_cast<void**>(&seq_cnt), err) ||
        rt->alloc((size_t)batch * 4, reinterpret_cast<void**>(&seq_q), err) ||
        rt->alloc((size_t)batch * 4, reinterpret_cast<void**>(&seq_order), err) ||
        rt->alloc(4, reinterpret_cast<void**>(&total), err) ||
        rt->alloc(8, reinterpret_cast<void**>(&status), err))
      return 1;
    if (general &&
        (rt->alloc(rows * H * 4, reinterpret_cast<void**>(&hf), err) ||
         rt->alloc(rows * H * 4, reinterpret_cast<void**>(&h1f), err) ||
         rt->alloc(rows * 3 * H * 4, reinterpret_cast<void**>(&qkvf), err) ||
         rt->alloc(rows * H * 4, reinterpret_cast<void**>(&ctxf), err) ||
         rt->alloc(rows * F * 4, reinterpret_cast<void**>(&midf), err)))
      return 1;
    // At least 64 zeroed entries past the rows (attention reads whole 64-key
    // blocks); 72, so that the row stride is no multiple of 1 KiB (with +64
    // at c3 it was exactly 65 KiB and the transposed V stores of the QKV
    // GEMM ran 3 % slower).
    vt_ld = (int)((rows + 7) / 8 * 8 + 72);
    if (rt->alloc((size_t)H * vt_ld * 2, reinterpret_cast<void**>(&vt), err)) return 1;
    hipError_t e = hipMemset(vt, 0, (size_t)H * vt_ld * 2);
    if (e != hipSuccess) return hip_err(err, "hipMemset(vt)", e);
    cap_rows = rows;
    cap_batch = batch;
    return 0;
  }

  // The general-shape forward (rows already packed): f32 activations,
  // eos_enc_gen_* per operation, pooled from the f32 rows.
  int forward_general(const int32_t* d_ids, const int32_t* d_types, int batch, int tokens,
                      float* d_out, bool cls, char** err) {
    const int H = desc.hidden, F = desc.intermediate, nh = desc.heads;
    const int max_rows = (int)row_capacity(batch, tokens);
    EncGenArgs g;
    memset(&g, 0, sizeof(g));
    g.ids = d_ids;
    g.type_ids = d_types;
    g.row_b = row_b;
    g.row_t = row_t;
    g.total = total;
    g.status = status;
    g.seq_off = seq_off;
    g.seq_cnt = seq_cnt;
    g.seq_q = seq_q;
    g.hidden = H;
    g.heads = nh;
    g.tokens = tokens;
    g.vocab = desc.vocab;
    g.npos = desc.max_positions;
    g.ntype = desc.type_vocab;
    g.max_rows = max_rows;
    g.eps = desc.ln_eps;
    const unsigned row_blocks = (unsigned)((max_rows + 3) / 4);
    {
      EncGenArgs e = g;
      e.tok = tok;
      e.pos = pos;
      e.typ = typ;
      e.gamma = eg;
      e.beta = eb;
      e.y = hf;
      if (rt->launch("eos_enc_gen_embed", dim3(row_blocks), dim3(256), 0, &e, err) != 0) return 1;
    }
    auto dense = [&](const float* x, float* y, const float* res, const int8_t* w, const float* sc,
                     const float* b, int n, int k, int epi, const char* label) {
      EncGenArgs d = g;
      d.x = x;
      d.y = y;
      d.res = res;
      d.w = w;
      d.wscale = sc;
      d.bias = b;
      d.n = n;
      d.k = k;
      d.epi = epi;
      return rt->launch("eos_enc_gen_dense", dim3((unsigned)((n + 63) / 64), row_blocks), dim3(256),
                        0, &d, err, label);
    };
    auto layer_norm = [&](float* y, const float* gm, const float* bt) {
      EncGenArgs l = g;
      l.y = y;
      l.gamma = gm;
      l.beta = bt;
      return rt->launch("eos_enc_gen_ln", dim3(row_blocks), dim3(256), 0, &l, err, "enc_ln");
    };
    for (const DevLayer& L : layers) {
      EncGenArgs at = g;
      at.x = qkvf;
      at.y = ctxf;
      if (dense(hf, qkvf, nullptr, L.w_qkv8, L.s_qkv, L.b_qkv, 3 * H, H, 0, "enc_gemm_qkv") != 0 ||
          rt->launch("eos_enc_gen_attn", dim3((unsigned)((tokens + 8 + 63) / 64), nh, batch),
                     dim3(64), 0, &at, err, "eos_enc_attn") != 0 ||
          dense(ctxf, h1f, hf, L.w_o8, L.s_o, L.b_o, H, H, 0, "enc_gemm_o") != 0 ||
          layer_norm(h1f, L.g1, L.be1) != 0 ||
          dense(h1f, midf, nullptr, L.w_18, L.s_1, L.b_1, F, H, desc.gelu, "enc_gemm_ffn_up") != 0 ||
          dense(midf, hf, h1f, L.w_28, L.s_2, L.b_2, H, F, 0, "enc_gemm_ffn_down") != 0 ||
          layer_norm(hf, L.g2, L.be2) != 0)
        return 1;
    }
    EncPoolArgs pl;
    memset(&pl, 0, sizeof(pl));
    pl.seq_off = seq_off;
    pl.seq_cnt = seq_cnt;
    pl.out = d_out;
    pl.batch = batch;
    pl.hidden = H;
    pl.cls_seq_q = cls ? seq_q : nullptr;
    pl.h32 = hf;
    return rt->launch("eos_enc_gen_pool", dim3(batch), dim3(1024), 0, &pl, err, "eos_enc_pool");
  }

  int forward(const int32_t* d_ids, const int32_t* d_types, const int32_t* d_mask, int batch,
              int tokens, float* d_out, char** err) {
    if (ensure_activations(batch, tokens, err) != 0) return 1;
    const int H = desc.hidden, F = desc.intermediate, nh = desc.heads, hd = H / nh;
    const int max_rows = (int)row_capacity(batch, tokens);
    // status[0]: an id out of range; status[1]: attention reference moves.
    hipError_t e = hipMemsetAsync(status, 0, 8, rt->stream);
    if (e != hipSuccess) return hip_err(err, "hipMemsetAsync(status)", e);
    const bool cls = family == 0 && pooling == 1;
    EncPackArgs pk{};
    pk.mask = d_mask;
    pk.row_b = row_b;
    pk.row_t = row_t;
    pk.seq_off = seq_off;
    pk.seq_cnt = seq_cnt;
    pk.total = total;
    pk.batch = batch;
    pk.tokens = tokens;
    pk.all_active = attend_all ? 1 : 0;
    pk.seq_q = seq_q;
    pk.cls_row = cls ? 1 : 0;
    pk.ids = d_ids;
    pk.type_ids = d_types;
    pk.vocab = desc.vocab;
    pk.ntype = desc.type_vocab;
    pk.status = status;
    pk.order = seq_order;
    if (rt->launch("eos_enc_count", dim3(batch), dim3(256), 0, &pk, err) != 0 ||
        rt->launch("eos_enc_pack", dim3(batch), dim3(256), 0, &pk, err) != 0)
      return 1;
    if (general) return forward_general(d_ids, d_types, batch, tokens, d_out, cls, err);
    EncEmbedArgs em;
    memset(&em, 0, sizeof(em));
    em.ids = d_ids;
    em.type_ids = d_types;
    em.row_b = row_b;
    em.row_t = row_t;
    em.total = total;
    em.tok = tok;
    em.pos = pos;
    em.typ = typ;
    em.gamma = eg;
    em.beta = eb;
    em.out = h;
    em.status = status;
    em.tokens = tokens;
    em.hidden = H;
    em.vocab = desc.vocab;
    em.npos = desc.max_positions;
    em.ntype = desc.type_vocab;
    em.eps = desc.ln_eps;
    em.mode = family;
    // BERT family: QKV and FFN-up run W8A8, so the embedding and every
    // LayerNorm also write their rows as int8 codes with per-row scales.
    const bool a8 = family == 0;
    em.q8 = a8 ? h8 : nullptr;
    em.qscale = a8 ? hs : nullptr;
    if (rt->launch("eos_enc_embed", dim3((max_rows + 3) / 4), dim3(256), 0, &em, err) != 0) return 1;
    char attn_name[48];
    snprintf(attn_name, sizeof(attn_name), "eos_enc_attn_hd%d", hd);
    // GEMM tiles: 256 x 128 for wide outputs, 128 x 128 for hidden-width ones
    // (more workgroups for the smaller N).
    // W8 != NULL: int8 codes of W; A is then h8 with the row scales hs.
    auto gemm = [&](const uint16_t* A, const uint16_t* W, const int8_t* W8, const float* sc,
                    const float* b, uint16_t* out, const uint16_t* res, int n, int k, int epi,
                    const char* label, uint16_t* vt_out = nullptr) {
      const bool wide = n >= 1024;
      const int bm = wide ? 256 : 128;
      EncGemmArgs g{A, W, sc, b, out, total, res, max_rows, n, k, epi, vt_out, 2 * H, vt_ld,
                    W8 != nullptr ? h8 : nullptr, W8 != nullptr ? hs : nullptr, W8};
      const char* name = W8 != nullptr ? (wide ? "eos_enc_gemm8_t256" : "eos_enc_gemm8_t128")
                                       : (wide ? "eos_enc_gemm_t256" : "eos_enc_gemm_t128");
      // One-dimensional grid: n / 128 column tiles for each row block, row
      // blocks rounded up to a multiple of 8 (the kernel maps workgroups to
      // tiles per XCD; tiles past the rows exit at once).
      const unsigned mblk = (unsigned)(((max_rows + bm - 1) / bm + 7) / 8 * 8);
      return rt->launch(name, dim3((unsigned)(n / 128) * mblk), dim3(256), 0, &g, err, label);
    };
    auto layer_norm = [&](const float* gm, const float* bt) {
      EncLnArgs l{h, gm, bt, total, max_rows, H, desc.ln_eps, a8 ? h8 : nullptr, a8 ? hs : nullptr};
      return rt->launch("eos_enc_ln", dim3((unsigned)((max_rows + 3) / 4)), dim3(256), 0, &l, err,
                        "enc_ln");
    };
    // Fused tail: the largest row block whose LDS fits the hidden width.
    const char* tail_name = nullptr;
    char tail_buf[48];
    int tail_bm = 0;
    if (a8 && fused_tail && (H == 384 || H == 512 || H == 768) && F <= 4 * H) {
      tail_bm = H == 384 ? 96 : H == 512 ? 64 : 32;
      snprintf(tail_buf, sizeof(tail_buf), "eos_enc_tail_r%d_h%d_g%d", tail_bm / 32, H, desc.gelu);
      tail_name = tail_buf;
    }
    for (const DevLayer& L : layers) {
      // Q and K rows into qkv, V feature-major into vt.
      if (gemm(h, L.w_qkv, a8 ? L.w_qkv8 : nullptr, L.s_qkv, L.b_qkv, qkv, nullptr, 3 * H, H, 0,
               "enc_gemm_qkv", vt) != 0)
        return 1;
      const double log2e = 1.4426950408889634;
      EncAttnArgs at{qkv, vt, ctx, seq_off, seq_cnt, seq_q, batch, nh, H, tokens, vt_ld,
                     (float)(scaled_scores ? log2e / std::sqrt((double)hd) : log2e), status + 1,
                     seq_order};
      // Head dim 64 over sequences longer than 512: 12-wavefront workgroups
      // (384 queries each); else 4 (128 queries), which waste fewer
      // wavefronts on short sequences.
      const bool wide = hd == 64 && tokens > 512;
      const int qpw = wide ? 384 : 128;
      if (rt->launch(wide ? "eos_enc_attn_hd64_w12" : attn_name,
                     dim3((tokens + qpw - 1) / qpw, nh, batch), dim3(wide ? 768 : 256), 0, &at,
                     err) != 0)
        return 1;
      if (tail_name != nullptr) {
        EncTailArgs tl{ctx,    h,      mid,    h8,     hs,     L.w_of, L.s_o,    L.b_o,     L.g1,
                       L.be1,  L.w_1f, L.s_1,  L.b_1,  L.w_2f, L.s_2,    L.b_2,     L.g2,
                       L.be2,  total,  max_rows, F,    desc.ln_eps, desc.gelu};
        tl.row0 = 0;
        tl.row_cap = max_rows;
        // One block per CU holds the whole tail (its LDS and registers), so
        // rows past one block per CU would run as a second, partly empty
        // round of full blocks. At hidden 512 (64-row blocks) the first
        // round covers one block per CU and the rows after it go to 32-row
        // blocks, which finish sooner (c4: 23,512 rows, tail 0.65 -> 0.59 ms
        // per forward). The row count is known on the device only: when it
        // ends inside the first round, the second launch's blocks exit.
        const int first = rt->compute_units * tail_bm;
        if (H == 512 && max_rows > first) {
          tl.row_cap = first;
          if (rt->launch(tail_name, dim3((unsigned)rt->compute_units), dim3(EOS_TAIL_THREADS), 0,
                         &tl, err, "enc_tail") != 0)
            return 1;
          char rest[48];
          snprintf(rest, sizeof(rest), "eos_enc_tail_r1_h%d_g%d", H, desc.gelu);
          tl.row0 = first;
          tl.row_cap = max_rows;
          if (rt->launch(rest, dim3((unsigned)((max_rows - first + 31) / 32)),
                         dim3(EOS_TAIL_THREADS), 0, &tl, err, "enc_tail") != 0)
            return 1;
          continue;
        }
        if (rt->launch(tail_name, dim3((unsigned)((max_rows + tail_bm - 1) / tail_bm)),
                       dim3(EOS_TAIL_THREADS),
                       0, &tl, err, "enc_tail") != 0)
          return 1;
        continue;
      }
      if (gemm(ctx, L.w_o, nullptr, L.s_o, L.b_o, h, h, H, H, 3, "enc_gemm_o") != 0 ||
          layer_norm(L.g1, L.be1) != 0 ||
          gemm(h, L.w_1, a8 ? L.w_18 : nullptr, L.s_1, L.b_1, mid, nullptr, F, H, desc.gelu,
               "enc_gemm_ffn_up") != 0 ||
          gemm(mid, L.w_2, nullptr, L.s_2, L.b_2, h, h, H, F, 3, "enc_gemm_ffn_down") != 0 ||
          layer_norm(L.g2, L.be2) != 0)
        return 1;
    }
    const int nchunk = (tokens + kPoolChunk - 1) / kPoolChunk;
    EncPoolArgs pl{h,     seq_off, seq_cnt,   d_out,   proj,
                   pool_part, batch, H,     family,  out_dim(),
                   nchunk, attend_all ? d_mask : nullptr, tokens};
    if (cls) {
      pl.cls_seq_q = seq_q;
    } else if (rt->launch("eos_enc_pool_part", dim3((unsigned)nchunk, (unsigned)batch), dim3(256),
                          0, &pl, err) != 0) {
      return 1;
    }
    return rt->launch("eos_enc_pool", dim3(batch), dim3(1024), 0, &pl, err);
  }
};

// Shapes the general-shape (f32) path takes: hidden a multiple of 8 up to
// 1024, head dims up to 64, any positive FFN width up to 16384.
static bool general_dims(int H, int heads, int F) {
  return H >= 8 && H <= 1024 && H % 8 == 0 && heads > 0 && H % heads == 0 && H / heads <= 64 &&
         F > 0 && F <= 16384;
}

// Shapes the MFMA kernels support: hidden widths 128..768 (embed and LayerNorm
// hold a row in one wavefront; every GEMM N a multiple of the 128-column
// tile), attention head dims 32/64/128/256, FFN widths in multiples of 128.
static int check_dims(int H, int heads, int F, const char* what, char** err) {
  if (H != 128 && H != 256 && H != 384 && H != 512 && H != 768)
    return set_err(err, "%s: hidden must be 128, 256, 384, 512 or 768 (got %d)", what, H);
  if (heads <= 0 || H % heads != 0 ||
      (H / heads != 32 && H / heads != 64 && H / heads != 128 && H / heads != 256))
    return set_err(err, "%s: head dim must be 32, 64, 128 or 256 (hidden %d, heads %d)", what,
                   H, heads);
  if (F <= 0 || F % 128 != 0)
    return set_err(err, "%s: intermediate width must be a positive multiple of 128", what);
  return 0;
}

extern "C" {

int eoship_encoder_bind(EosHipRuntime* rt, const EosHipEncoderDesc* desc, const float* tok_emb,
                        const float* pos_emb, const float* type_emb, const float* emb_ln_gamma,
                        const float* emb_ln_beta, const EosHipEncoderLayer* layers,
                        EosHipEncoder** out, char** err) {
  if (rt == nullptr || desc == nullptr || out == nullptr || tok_emb == nullptr ||
      pos_emb == nullptr || type_emb == nullptr || emb_ln_gamma == nullptr ||
      emb_ln_beta == nullptr || (desc->layers > 0 && layers == nullptr))
    return set_err(err, "eoship_encoder_bind: NULL argument");
  *out = nullptr;
  const int H = desc->hidden, F = desc->intermediate;
  // Shapes outside the MFMA kernels run the general-shape path when it takes
  // them (else the MFMA shapes' error is reported).
  const bool general = check_dims(H, desc->heads, F, "", nullptr) != 0 &&
                       general_dims(H, desc->heads, F);
  if (!general && check_dims(H, desc->heads, F, "eoship_encoder_bind", err) != 0) return 1;
  if (desc->layers < 0 || desc->vocab <= 0 || desc->max_positions <= 0 || desc->type_vocab <= 0)
    return set_err(err, "eoship_encoder_bind: layers/vocab/positions/type_vocab out of range");
  if (!(desc->ln_eps >= 0.f)) return set_err(err, "eoship_encoder_bind: ln_eps must be >= 0");
  if (desc->gelu != 1 && desc->gelu != 2)
    return set_err(err, "eoship_encoder_bind: gelu must be 1 (erf) or 2 (tanh)");
  auto* enc = new EosHipEncoder();
  enc->rt = rt;
  enc->desc = *desc;
  enc->general = general;
  auto fail = [&]() {
    delete enc;
    return 1;
  };
  if (enc->upload(&enc->tok, tok_emb, (size_t)desc->vocab * H, err) ||
      enc->upload(&enc->pos, pos_emb, (size_t)desc->max_positions * H, err) ||
      enc->upload(&enc->typ, type_emb, (size_t)desc->type_vocab * H, err) ||
      enc->upload(&enc->eg, emb_ln_gamma, (size_t)H, err) ||
      enc->upload(&enc->eb, emb_ln_beta, (size_t)H, err))
    return fail();
  for (int l = 0; l < desc->layers; ++l) {
    const EosHipEncoderLayer& s = layers[l];
    const void* req[] = {s.w_qkv, s.s_qkv, s.b_qkv, s.w_o, s.s_o, s.b_o, s.ln1_gamma, s.ln1_beta,
                         s.w_1, s.s_1, s.b_1, s.w_2, s.s_2, s.b_2, s.ln2_gamma, s.ln2_beta};
    for (const void* p : req)
      if (p == nullptr) {
        set_err(err, "eoship_encoder_bind: layer %d has a NULL tensor", l);
        return fail();
      }
    DevLayer d;
    if (enc->upload_codes(&d.w_qkv, s.w_qkv, (size_t)3 * H * H, err) ||
        enc->upload(&d.s_qkv, s.s_qkv, (size_t)3 * H, err) ||
        enc->upload(&d.b_qkv, s.b_qkv, (size_t)3 * H, err) ||
        enc->upload_codes(&d.w_o, s.w_o, (size_t)H * H, err) ||
        enc->upload(&d.s_o, s.s_o, (size_t)H, err) || enc->upload(&d.b_o, s.b_o, (size_t)H, err) ||
        enc->upload(&d.g1, s.ln1_gamma, (size_t)H, err) ||
        enc->upload(&d.be1, s.ln1_beta, (size_t)H, err) ||
        enc->upload_codes(&d.w_1, s.w_1, (size_t)F * H, err) ||
        enc->upload(&d.s_1, s.s_1, (size_t)F, err) || enc->upload(&d.b_1, s.b_1, (size_t)F, err) ||
        enc->upload_codes(&d.w_2, s.w_2, (size_t)H * F, err) ||
        enc->upload(&d.s_2, s.s_2, (size_t)H, err) || enc->upload(&d.b_2, s.b_2, (size_t)H, err) ||
        enc->upload(&d.g2, s.ln2_gamma, (size_t)H, err) ||
        enc->upload(&d.be2, s.ln2_beta, (size_t)H, err) ||
        enc->upload(&d.w_qkv8, s.w_qkv, (size_t)3 * H * H, err) ||
        enc->upload(&d.w_18, s.w_1, (size_t)F * H, err))
      return fail();
    if (general && (enc->upload(&d.w_o8, s.w_o, (size_t)H * H, err) ||
                    enc->upload(&d.w_28, s.w_2, (size_t)H * F, err)))
      return fail();
    if ((H == 384 || H == 512 || H == 768) &&
        (enc->upload_frag16(&d.w_of, s.w_o, H, H, err) ||
         enc->upload_frag8(&d.w_1f, s.w_1, F, H, err) ||
         enc->upload_frag16(&d.w_2f, s.w_2, H, F, err)))
      return fail();
    enc->layers.push_back(d);
  }
  *out = enc;
  return 0;
}

int eoship_encoder_bind_compact(EosHipRuntime* rt, const EosHipCompactDesc* desc,
                                const int8_t* token_embedding, float s_token,
                                const int8_t* role_embedding, float s_role,
                                const EosHipCompactLayer* layers, const int8_t* output_projection,
                                float s_output, EosHipEncoder** out, char** err) {
  if (role_embedding == nullptr) return set_err(err, "eoship_encoder_bind_compact: NULL argument");
  return eoship_encoder_bind_compact_opts(rt, desc, nullptr, token_embedding, s_token,
                                          role_embedding, s_role, layers, output_projection,
                                          s_output, out, err);
}

int eoship_encoder_bind_compact_opts(EosHipRuntime* rt, const EosHipCompactDesc* desc,
                                     const EosHipCompactOptions* opts,
                                     const int8_t* token_embedding, float s_token,
                                     const int8_t* role_embedding, float s_role,
                                     const EosHipCompactLayer* layers,
                                     const int8_t* output_projection, float s_output,
                                     EosHipEncoder** out, char** err) {
  const char* what = "eoship_encoder_bind_compact";
  EosHipCompactOptions o{1, 1, 1, 0};
  if (opts != nullptr) o = *opts;
  auto bit = [](int32_t v) { return v == 0 || v == 1; };
  if (!bit(o.rope) || !bit(o.role) || !bit(o.scaled_scores) || !bit(o.attend_padding))
    return set_err(err, "%s: options must be 0 or 1", what);
  if (rt == nullptr || desc == nullptr || out == nullptr || token_embedding == nullptr ||
      (o.role && role_embedding == nullptr) || (desc->layers > 0 && layers == nullptr))
    return set_err(err, "%s: NULL argument", what);
  *out = nullptr;
  const int D = desc->model_dim, F = desc->hidden_dim, O = desc->output_dim;
  if (check_dims(D, desc->heads, F, what, err) != 0) return 1;
  if (desc->layers < 0 || desc->vocab <= 0 || desc->max_sequence <= 0)
    return set_err(err, "%s: layers/vocab/max_sequence out of range", what);
  if (O <= 0 || O > 8192) return set_err(err, "%s: output_dim must be in 1..8192 (got %d)", what, O);
  if ((O != D) != (output_projection != nullptr))
    return set_err(err, "%s: output_projection must be given exactly when output_dim != model_dim",
                   what);
  auto bad_scale = [](float sc) { return !(sc >= 0.f) || std::isinf(sc); };
  if (bad_scale(s_token) || (o.role && bad_scale(s_role)) ||
      (output_projection && bad_scale(s_output)))
    return set_err(err, "%s: scales must be finite and >= 0", what);
  for (int l = 0; l < desc->layers; ++l) {
    const EosHipCompactLayer& s = layers[l];
    if (!s.attn_q || !s.attn_k || !s.attn_v || !s.attn_o || !s.ffn_up || !s.ffn_down)
      return set_err(err, "%s: layer %d has a NULL tensor", what, l);
    if (bad_scale(s.s_q) || bad_scale(s.s_k) || bad_scale(s.s_v) || bad_scale(s.s_o) ||
        bad_scale(s.s_up) || bad_scale(s.s_down))
      return set_err(err, "%s: layer %d has a negative or non-finite scale", what, l);
  }
  auto* enc = new EosHipEncoder();
  enc->rt = rt;
  enc->family = 1;
  enc->odim = O;
  enc->scaled_scores = o.scaled_scores != 0;
  enc->attend_all = o.attend_padding != 0;
  EosHipEncoderDesc& d = enc->desc;
  d.layers = desc->layers;
  d.hidden = D;
  d.heads = desc->heads;
  d.intermediate = F;
  d.vocab = desc->vocab;
  d.max_positions = desc->max_sequence;
  d.type_vocab = 3;
  d.ln_eps = 1e-5f;
  d.gelu = 2;
  auto fail = [&]() {
    delete enc;
    return 1;
  };
  // Dequantized tables (code * scale in f32, as the reference's q8/q4 decode).
  auto dequant = [](const int8_t* c, float sc, size_t n) {
    std::vector<float> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (float)c[i] * sc;
    return v;
  };
  const std::vector<float> tok = dequant(token_embedding, s_token, (size_t)desc->vocab * D);
  // Without roles the role rows are zeros: token + 0 is the token row exactly.
  const std::vector<float> role = o.role ? dequant(role_embedding, s_role, (size_t)3 * D)
                                         : std::vector<float>((size_t)3 * D, 0.0f);
  // RoPE table: per position, (cos, sin) of theta = pos / 10000^(c / D) for
  // each even column c, computed in f64 and rounded to f32 (ropeRows,
  // runtime/backend/tensor_ops.go:1936-1965). Without RoPE, (1, 0) for every
  // pair: the rotation x0 * 1 - x1 * 0, x0 * 0 + x1 * 1 returns the pair exactly.
  std::vector<float> rope((size_t)desc->max_sequence * D);
  for (int pos = 0; pos < desc->max_sequence; ++pos)
    for (int c = 0; c + 1 < D; c += 2) {
      const double theta = (double)pos / std::pow(10000.0, (double)c / (double)D);
      rope[(size_t)pos * D + c] = o.rope ? (float)std::cos(theta) : 1.0f;
      rope[(size_t)pos * D + c + 1] = o.rope ? (float)std::sin(theta) : 0.0f;
    }
  const std::vector<float> ones((size_t)D, 1.0f);
  const std::vector<float> zeros((size_t)std::max(3 * D, F), 0.0f);
  float *g1 = nullptr, *b0 = nullptr;
  if (enc->upload(&enc->tok, tok.data(), tok.size(), err) ||
      enc->upload(&enc->typ, role.data(), role.size(), err) ||
      enc->upload(&enc->pos, rope.data(), rope.size(), err) ||
      enc->upload(&g1, ones.data(), ones.size(), err) ||
      enc->upload(&b0, zeros.data(), zeros.size(), err))
    return fail();
  enc->eg = g1;
  enc->eb = b0;
  if (output_projection != nullptr) {
    const std::vector<float> pr = dequant(output_projection, s_output, (size_t)D * O);
    if (enc->upload(&enc->proj, pr.data(), pr.size(), err)) return fail();
  }
  for (int l = 0; l < desc->layers; ++l) {
    const EosHipCompactLayer& s = layers[l];
    // Tied layers (the same codes and scales as an earlier layer) share its
    // device copies.
    int tied = -1;
    auto same = [](const EosHipCompactLayer& x, const EosHipCompactLayer& y) {
      return x.attn_q == y.attn_q && x.s_q == y.s_q && x.attn_k == y.attn_k && x.s_k == y.s_k &&
             x.attn_v == y.attn_v && x.s_v == y.s_v && x.attn_o == y.attn_o && x.s_o == y.s_o &&
             x.ffn_up == y.ffn_up && x.s_up == y.s_up && x.ffn_down == y.ffn_down &&
             x.s_down == y.s_down;
    };
    for (int j = 0; j < l && tied < 0; ++j)
      if (same(layers[j], s)) tied = j;
    if (tied >= 0) {
      enc->layers.push_back(enc->layers[(size_t)tied]);
      continue;
    }
    DevLayer dl;
    const int8_t* qkv[] = {s.attn_q, s.attn_k, s.attn_v};
    const float sqkv[] = {s.s_q, s.s_k, s.s_v};
    const int oqkv[] = {D, D, D};
    const int oD[] = {D}, oF[] = {F};
    if (enc->upload_codes_t(&dl.w_qkv, &dl.s_qkv, qkv, sqkv, oqkv, 3, D, err) ||
        enc->upload_codes_t(&dl.w_o, &dl.s_o, &s.attn_o, &s.s_o, oD, 1, D, err) ||
        enc->upload_codes_t(&dl.w_1, &dl.s_1, &s.ffn_up, &s.s_up, oF, 1, D, err) ||
        enc->upload_codes_t(&dl.w_2, &dl.s_2, &s.ffn_down, &s.s_down, oD, 1, F, err))
      return fail();
    dl.b_qkv = dl.b_o = dl.b_1 = dl.b_2 = b0;
    dl.g1 = dl.g2 = g1;
    dl.be1 = dl.be2 = b0;
    enc->layers.push_back(dl);
  }
  *out = enc;
  return 0;
}

int eoship_encoder_release(EosHipEncoder* enc, char** err) {
  (void)err;
  if (enc == nullptr) return 0;
  (void)enc->rt->sync(nullptr);
  delete enc;
  return 0;
}

static int check_shape(EosHipEncoder* enc, int32_t batch, int32_t tokens, const char* what,
                       char** err) {
  if (batch <= 0 || tokens <= 0)
    return set_err(err, "%s: batch and tokens must be positive (got %d, %d)", what, batch, tokens);
  if (tokens > enc->desc.max_positions)
    return set_err(err, "%s: tokens %d exceed the position table (%d rows)", what, tokens,
                   enc->desc.max_positions);
  if ((int64_t)batch * tokens > (int64_t)1 << 30)
    return set_err(err, "%s: batch * tokens too large", what);
  return 0;
}

int eoship_encoder_forward_device(EosHipRuntime* rt, EosHipEncoder* enc, const int32_t* d_ids,
                                  const int32_t* d_type_ids, const int32_t* d_mask, int32_t batch,
                                  int32_t tokens, float* d_out, char** err) {
  if (rt == nullptr || enc == nullptr || d_ids == nullptr || d_mask == nullptr || d_out == nullptr)
    return set_err(err, "eoship_encoder_forward_device: NULL argument");
  if (enc->rt != rt) return set_err(err, "eoship_encoder_forward_device: encoder bound on another runtime");
  if (check_shape(enc, batch, tokens, "eoship_encoder_forward_device", err) != 0) return 1;
  return enc->forward(d_ids, d_type_ids, d_mask, batch, tokens, d_out, err);
}

int eoship_encoder_status(EosHipRuntime* rt, EosHipEncoder* enc, int32_t* status, char** err) {
  if (rt == nullptr || enc == nullptr || status == nullptr)
    return set_err(err, "eoship_encoder_status: NULL argument");
  *status = 0;
  if (enc->status == nullptr) return 0;
  hipError_t e = rt->copy_async(status, enc->status, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_err(err, "hipMemcpyAsync(status)", e);
  return rt->sync(err);
}

int eoship_encoder_set_fused_tail(EosHipRuntime* rt, EosHipEncoder* enc, int32_t fused,
                                   char** err) {
  if (rt == nullptr || enc == nullptr) return set_err(err, "eoship_encoder_set_fused_tail: NULL argument");
  enc->fused_tail = fused != 0;
  return 0;
}

int eoship_encoder_set_pooling(EosHipRuntime* rt, EosHipEncoder* enc, int32_t pooling,
                               char** err) {
  if (rt == nullptr || enc == nullptr) return set_err(err, "eoship_encoder_set_pooling: NULL argument");
  if (pooling != 0 && pooling != 1)
    return set_err(err, "eoship_encoder_set_pooling: pooling must be 0 (masked_mean) or 1 (cls)");
  if (pooling == 1 && enc->family != 0)
    return set_err(err, "eoship_encoder_set_pooling: cls pooling applies to the BERT family only");
  enc->pooling = pooling;
  return 0;
}

int eoship_encoder_attention_moves(EosHipRuntime* rt, EosHipEncoder* enc, int64_t* moves,
                                   char** err) {
  if (rt == nullptr || enc == nullptr || moves == nullptr)
    return set_err(err, "eoship_encoder_attention_moves: NULL argument");
  *moves = 0;
  if (enc->status == nullptr) return 0;
  int32_t v = 0;
  hipError_t e = rt->copy_async(&v, enc->status + 1, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_err(err, "hipMemcpyAsync(moves)", e);
  if (rt->sync(err) != 0) return 1;
  *moves = v;
  return 0;
}

int eoship_encoder_forward(EosHipRuntime* rt, EosHipEncoder* enc, const int32_t* ids,
                           const int32_t* type_ids, const int32_t* mask, int32_t batch,
                           int32_t tokens, float* out, char** err) {
  if (rt == nullptr || enc == nullptr || ids == nullptr || mask == nullptr || out == nullptr)
    return set_err(err, "eoship_encoder_forward: NULL argument");
  if (enc->rt != rt) return set_err(err, "eoship_encoder_forward: encoder bound on another runtime");
  if (check_shape(enc, batch, tokens, "eoship_encoder_forward", err) != 0) return 1;
  const size_t n = (size_t)batch * tokens;
  const size_t need = n * 4 * 3 + (size_t)batch * enc->out_dim() * 4 + 64;
  if (enc->io_bytes < need) {
    if (enc->io) hipFree(enc->io);
    enc->io = nullptr;
    enc->io_bytes = 0;
    if (rt->alloc(need, &enc->io, err) != 0) return 1;
    enc->io_bytes = need;
  }
  int32_t* d_ids = static_cast<int32_t*>(enc->io);
  int32_t* d_types = d_ids + n;
  int32_t* d_mask = d_types + n;
  float* d_out = reinterpret_cast<float*>(d_mask + n);
  hipError_t e = rt->copy_async(d_ids, ids, n * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess && type_ids != nullptr)
    e = rt->copy_async(d_types, type_ids, n * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = rt->copy_async(d_mask, mask, n * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_err(err, "hipMemcpyAsync(encoder inputs)", e);
  if (enc->forward(d_ids, type_ids ? d_types : nullptr, d_mask, batch, tokens, d_out, err) != 0)
    return 1;
  e = rt->copy_async(out, d_out, (size_t)batch * enc->out_dim() * 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_err(err, "hipMemcpyAsync(embeddings)", e);
  int32_t st = 0;
  if (eoship_encoder_status(rt, enc, &st, err) != 0) return 1;
  if (st != 0)
    return set_err(err, "eoship_encoder_forward: input id out of range (token, token type or position)");
  return 0;
}

}  // extern "C"
