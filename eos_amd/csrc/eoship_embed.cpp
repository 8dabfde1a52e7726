// Tiny embed pipeline of examples/embed.eos (gather -> @matmul -> l2_normalize)
// as one device kernel over resident weights; replaces the plan the reference
// executes step by step through ExecuteSymbolic (host gather, cuBLAS matmul,
// l2_normalize kernel; runtime/backend/symbolic.go:17-172).
#include <cstring>

#include "eoship_internal.h"
#include "kernels/enc_args.h"

using eoship::hip_err;
using eoship::set_err;

struct EosHipEmbed {
  EosHipRuntime* rt = nullptr;
  int vocab = 0, dim = 0, edim = 0;
  uint16_t* table = nullptr;
  uint16_t* proj = nullptr;
  int32_t* status = nullptr;
  void* io = nullptr;
  size_t io_bytes = 0;
  ~EosHipEmbed() {
    void* p[] = {table, proj, status, io};
    for (void* x : p)
      if (x) hipFree(x);
  }
  int run(const int32_t* d_tokens, int n, uint16_t* d_out, char** err) {
    hipError_t e = hipMemsetAsync(status, 0, 4, rt->stream);
    if (e != hipSuccess) return hip_err(err, "hipMemsetAsync(status)", e);
    EmbedTinyArgs a{table, proj, d_tokens, d_out, status, n, vocab, dim, edim};
    // 4 tokens per workgroup with the projection in LDS when it fits.
    const size_t lds = (size_t)dim * edim * 2 + ((size_t)dim * 4 + (size_t)4 * edim) * 4;
    if ((edim == 64 || edim == 128 || edim == 256) && dim % 8 == 0 && lds <= 150 * 1024) {
      const char* name = edim == 64 ? "eos_embed_tiny_e64"
                         : edim == 128 ? "eos_embed_tiny_e128" : "eos_embed_tiny_e256";
      return rt->launch(name, dim3((unsigned)((n + 3) / 4)), dim3((unsigned)(4 * edim)), lds, &a,
                        err);
    }
    return rt->launch("eos_embed_tiny", dim3((unsigned)((n + 3) / 4)), dim3(256), 0, &a, err);
  }
};

extern "C" {

int eoship_embed_bind(EosHipRuntime* rt, const uint16_t* table_f16, int32_t vocab, int32_t dim,
                      const uint16_t* proj_f16, int32_t edim, EosHipEmbed** out, char** err) {
  if (rt == nullptr || table_f16 == nullptr || proj_f16 == nullptr || out == nullptr)
    return set_err(err, "eoship_embed_bind: NULL argument");
  *out = nullptr;
  if (vocab <= 0 || dim <= 0 || dim > 1024 || edim <= 0 || edim > 1024)
    return set_err(err, "eoship_embed_bind: need vocab > 0, 0 < dim <= 1024, 0 < edim <= 1024");
  auto* m = new EosHipEmbed();
  m->rt = rt;
  m->vocab = vocab;
  m->dim = dim;
  m->edim = edim;
  const size_t tb = (size_t)vocab * dim * 2, pb = (size_t)dim * edim * 2;
  hipError_t e = hipSuccess;
  if (rt->alloc(tb, reinterpret_cast<void**>(&m->table), err) ||
      rt->alloc(pb, reinterpret_cast<void**>(&m->proj), err) ||
      rt->alloc(4, reinterpret_cast<void**>(&m->status), err)) {
    delete m;
    return 1;
  }
  e = rt->copy_sync(m->table, table_f16, tb, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = rt->copy_sync(m->proj, proj_f16, pb, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    delete m;
    return hip_err(err, "hipMemcpy(embed weights)", e);
  }
  *out = m;
  return 0;
}

int eoship_embed_release(EosHipEmbed* m, char** err) {
  (void)err;
  if (m == nullptr) return 0;
  (void)m->rt->sync(nullptr);
  delete m;
  return 0;
}

int eoship_embed_run_device(EosHipRuntime* rt, EosHipEmbed* m, const int32_t* d_tokens, int32_t n,
                            uint16_t* d_out, char** err) {
  if (rt == nullptr || m == nullptr || (n > 0 && (d_tokens == nullptr || d_out == nullptr)))
    return set_err(err, "eoship_embed_run_device: NULL argument");
  if (m->rt != rt) return set_err(err, "eoship_embed_run_device: bound on another runtime");
  if (n < 0) return set_err(err, "eoship_embed_run_device: negative token count");
  if (n == 0) return 0;
  return m->run(d_tokens, n, d_out, err);
}

int eoship_embed_run(EosHipRuntime* rt, EosHipEmbed* m, const int32_t* tokens, int32_t n,
                     uint16_t* out_f16, char** err) {
  if (rt == nullptr || m == nullptr || (n > 0 && (tokens == nullptr || out_f16 == nullptr)))
    return set_err(err, "eoship_embed_run: NULL argument");
  if (m->rt != rt) return set_err(err, "eoship_embed_run: bound on another runtime");
  if (n < 0) return set_err(err, "eoship_embed_run: negative token count");
  if (n == 0) return 0;
  const size_t need = (size_t)n * 4 + (size_t)n * m->edim * 2 + 64;
  if (m->io_bytes < need) {
    if (m->io) hipFree(m->io);
    m->io = nullptr;
    m->io_bytes = 0;
    if (rt->alloc(need, &m->io, err) != 0) return 1;
    m->io_bytes = need;
  }
  int32_t* dt = static_cast<int32_t*>(m->io);
  uint16_t* dout = reinterpret_cast<uint16_t*>(static_cast<char*>(m->io) + (((size_t)n * 4 + 15) & ~(size_t)15));
  hipError_t e = rt->copy_async(dt, tokens, (size_t)n * 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_err(err, "hipMemcpyAsync(tokens)", e);
  if (m->run(dt, n, dout, err) != 0) return 1;
  int32_t st = 0;
  e = rt->copy_async(out_f16, dout, (size_t)n * m->edim * 2, hipMemcpyDeviceToHost);
  if (e == hipSuccess) e = rt->copy_async(&st, m->status, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_err(err, "hipMemcpyAsync(embeddings)", e);
  if (rt->sync(err) != 0) return 1;
  if (st != 0) return set_err(err, "eoship_embed_run: token id out of range [0, %d)", m->vocab);
  return 0;
}

}  // extern "C"
