// TurboQuant compressed-vector scoring on gfx950 (CDNA4).
//
// Scoring contract (build-defined; the reference's IPQuantizer.InnerProductPrepared
// is in the un-vendored module m31labs.dev/turboquant v0.2.1 and is called from
// runtime/retrieval_turboquant.go:1874):
//   q'   = R q                        f64, fma in k order
//   s_q  = max|q'| / qmax,  Qs = rint(q' * (qmax / max|q'|))  (int16 grid)
//   D    = sum_j Qs_j * C[code_j]     exact int32 (codebook C on an int8 grid)
//   score= ((float)D * alpha) * norm + 0.0f,  alpha = (float)(s_q * s_c)
// Ranking: score descending, then vector id ascending
// (runtime/retrieval_eval.go:1153-1161).
//
// The scan computes D with v_mfma_i32_32x32x32_i8: A = 32 corpus vectors x 32
// dims (codes decoded to int8 codebook values in registers), B = 32 query
// columns x 32 dims, each int16 query split into an int8 high and low half
// (Qs = 256*hi + lo), so one pass over the corpus yields both halves and
// D = 256*D_hi + D_lo exactly.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "tq_args.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned long long u64;

#define EOS_DEV __device__ __forceinline__

namespace {

constexpr int kTile = 32;        // corpus vectors per MFMA row block
constexpr int kScanThreads = 256;
// The corpus scans run one workgroup per CU: eight waves (two per SIMD), or
// twelve (three per SIMD) for the high-half filter up to 16 K-steps, whose
// registers fit the 168 of three waves.
constexpr int scan_threads(bool hi, int ks) { return hi && ks <= 16 ? 768 : 512; }

// Order bits of a score; -0 keys as +0 (the reference compares -0 == +0 and
// then breaks the tie by id or index).
EOS_DEV uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
  u = u == 0x80000000u ? 0u : u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
EOS_DEV float key_score(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
// Composite rank key: larger = better; ties on score resolve to the lower id.
EOS_DEV u64 rank_key(float s, uint32_t id) {
  return ((u64)score_key(s) << 32) | (u64)(~id);
}
EOS_DEV uint32_t rank_id(u64 c) { return ~(uint32_t)(c & 0xffffffffu); }

// Calls f(i, src[i]) for i = threadIdx.x, threadIdx.x + NT, ... < n with U
// loads of each thread in flight before any value is used (a loop whose
// every iteration uses its own load would wait one memory round trip per
// iteration). Indices past n are clamped for the load and skipped for f.
template <int NT, int U, typename T, typename F>
EOS_DEV void for_each_batched(const T* src, long long n, F f) {
  for (long long base = threadIdx.x; base < n; base += (long long)NT * U) {
    T v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * NT;
      v[u] = src[i < n ? i : n - 1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long i = base + (long long)u * NT;
      if (i < n) f(i, v[u]);
    }
  }
}

// Copies the query fragments [KS*NCB*64] into LDS with every load issued
// before the first store.
template <int NT, int COUNT>
EOS_DEV void stage_fragments(v4i* dst, const v4i* src) {
  constexpr int PER = (COUNT + NT - 1) / NT;
  v4i v[PER];
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int i = threadIdx.x + r * NT;
    if (i < COUNT) v[r] = src[i];
  }
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int i = threadIdx.x + r * NT;
    if (i < COUNT) dst[i] = v[r];
  }
}

}  // namespace

// ------------------------------------------------------------------ prepare

namespace {
constexpr int kMaxDim = 1024;

// sqrt(v) rounded up to f32 (v >= 0 an exact integer < 2^53): the f32 result
// squared is exact in f64, so one comparison settles the direction.
EOS_DEV float sqrt_up(long long v) {
  const double dv = (double)v;
  float f = (float)sqrt(dv);
  if ((double)f * (double)f < dv) f = __uint_as_float(__float_as_uint(f) + 1u);
  return f;
}

// Column c of the MFMA query block reads source row (c / group) * group_live
// + c % group when c % group < group_live; other columns are zero.
EOS_DEV int prep_source(const TqPrepArgs& a, int c) {
  const int grp = c / a.group, slot = c - grp * a.group;
  const int src = grp * a.group_live + slot;
  return (slot < a.group_live && src < a.q) ? src : -1;
}

// Quantizes column c of the query block from its rotated (or raw) values:
// max |q'|, Qs = rint(q' qmax / max|q'|) clamped, hi/lo int8 fragments,
// alpha; resets the column's threshold and candidate count. Called by the 32
// lanes of one half-wave (t = lane & 31), values fetched by get(j).
template <int M, typename Get>
EOS_DEV void prep_quantize_column(const TqPrepArgs& a, int c, int t, Get get) {
  // M values per lane: dimensions up to 32 M.
  const int src = prep_source(a, c);
  // All of the lane's values are fetched before any is used, so the loads
  // overlap instead of costing one round trip each.
  // The loads come from clamped positions and the validity test is applied
  // afterwards: a load under a per-lane condition compiles to a branch of its
  // own that waits for its data before the next load is issued. (get is only
  // called with a valid source: the callers pass a get that reads nothing
  // when the block has no query rows.)
  double v[M];
  const int srcc = src >= 0 ? src : 0;
#pragma unroll
  for (int m = 0; m < M; ++m) v[m] = get(srcc, min(t + 32 * m, a.d - 1));
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int j = t + 32 * m;
    v[m] = (src >= 0 && j < a.d) ? v[m] : 0.0;
  }
  double mx = 0.0;
#pragma unroll
  for (int m = 0; m < M; ++m) mx = fmax(mx, fabs(v[m]));
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o));
  const double inv = mx > 0.0 ? (double)a.qmax / mx : 0.0;
  const int cb_hi = 2 * (c >> 5), col = c & 31;
  const int dpad = a.ks * 32;
  int lo2 = 0;  // sum of lo^2 over the lane's coordinates (<= 1024 * 128^2)
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int j = t + 32 * m;
    if (j >= dpad) break;
    int qs = 0;
    if (src >= 0 && j < a.d) {
      double x = rint(v[m] * inv);
      x = fmin(fmax(x, (double)-a.qmax), (double)a.qmax);
      qs = (int)x;
      if (a.qs_out != nullptr) a.qs_out[(size_t)src * a.d + j] = (int16_t)qs;
    }
    const int lo = ((qs + 128) & 255) - 128;
    const int hi = (qs - lo) >> 8;
    lo2 += lo * lo;
    const int s = j >> 5, g = (j >> 4) & 1, i = j & 15;
    const int lane = col + 32 * g;
    a.bfrag[((size_t)(s * a.ncb + cb_hi) * 64 + lane) * 16 + i] = (int8_t)hi;
    a.bfrag[((size_t)(s * a.ncb + cb_hi + 1) * 64 + lane) * 16 + i] = (int8_t)lo;
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) lo2 += __shfl_xor(lo2, o);
  if (t == 0) {
    if (a.lonorm != nullptr) a.lonorm[c] = sqrt_up(lo2);
    a.alpha[c] = mx > 0.0 ? (float)((mx / (double)a.qmax) * (double)a.cb_scale) : 0.0f;
    if (a.tau != nullptr) a.tau[c] = -__builtin_inff();
    if (a.cand_count != nullptr) a.cand_count[c] = 0u;
  }
}

constexpr int kPrepJ = 32;     // rotated coordinates per workgroup
constexpr int kPrepC = 8;      // query columns per workgroup
constexpr int kPrepK = 128;    // rotation rows staged in LDS per chunk

}  // namespace

// Rotation of the query block: workgroup (x, y) computes
// q'[c][j] = sum_k R[j][k] q_src(c)[k] in f64 (one fma chain per (c, j), k
// ascending) for j in [32x, 32x + 32) and the 8 columns [8y, 8y + 8). The
// query rows and the R^T slice are staged in LDS with every load of a stage in
// flight at once. eos_tq_quantize runs next on the same stream: the kernel
// boundary orders the two (a device-scope fence inside one launch costs more
// than the second launch).
extern "C" __global__ __launch_bounds__(256) void eos_tq_rotate(TqPrepArgs a) {
  __shared__ float rs[kPrepK * kPrepJ];
  __shared__ float qsh[kPrepC * kMaxDim];
  const int tid = threadIdx.x;
  const int j0 = blockIdx.x * kPrepJ, c0 = blockIdx.y * kPrepC;
  const int jj = tid & 31, cl = tid >> 5;
  {
    // Every query value of the 8 columns is loaded before any is stored, so
    // the staging costs one memory round trip.
    // Loads from clamped positions, then the validity test (a load under a
    // per-lane condition would be a branch of its own, waiting for its data
    // before the next load). With no query rows nothing is loaded.
    // Two rows of 256 values per column at a time (d <= 512: one pass), so
    // that the staging registers stay few (the kernel then fits beside a
    // running filter scan on a CU).
    constexpr int R = 2;
    for (int r0 = 0; r0 < a.d; r0 += 256 * R) {  // uniform
      float qv[kPrepC][R];
      if (a.q > 0) {
#pragma unroll
        for (int cc = 0; cc < kPrepC; ++cc) {
          const int src = prep_source(a, c0 + cc);
          const float* qrow = a.queries + (size_t)(src >= 0 ? src : 0) * a.d;
#pragma unroll
          for (int r = 0; r < R; ++r) qv[cc][r] = qrow[min(r0 + tid + 256 * r, a.d - 1)];
#pragma unroll
          for (int r = 0; r < R; ++r)
            qv[cc][r] = (src >= 0 && r0 + tid + 256 * r < a.d) ? qv[cc][r] : 0.0f;
        }
      } else {
#pragma unroll
        for (int cc = 0; cc < kPrepC; ++cc)
#pragma unroll
          for (int r = 0; r < R; ++r) qv[cc][r] = 0.0f;
      }
#pragma unroll
      for (int cc = 0; cc < kPrepC; ++cc)
#pragma unroll
        for (int r = 0; r < R; ++r)
          if (r0 + tid + 256 * r < a.d) qsh[cc * kMaxDim + r0 + tid + 256 * r] = qv[cc][r];
    }
  }
  const int j = j0 + jj;
  double acc = 0.0;
  for (int k0 = 0; k0 < a.d; k0 += kPrepK) {
    const int kn = min(kPrepK, a.d - k0);
    float tmp[kPrepK * kPrepJ / 256];
#pragma unroll
    for (int r = 0; r < kPrepK * kPrepJ / 256; ++r)
      tmp[r] = a.rot_t[(size_t)(k0 + min((tid >> 5) + 8 * r, kn - 1)) * a.d + min(j, a.d - 1)];
#pragma unroll
    for (int r = 0; r < kPrepK * kPrepJ / 256; ++r) {
      const int kk = (tid >> 5) + 8 * r;
      tmp[r] = (kk < kn && j < a.d) ? tmp[r] : 0.0f;
    }
    __syncthreads();  // previous chunk consumed; qsh visible
#pragma unroll
    for (int r = 0; r < kPrepK * kPrepJ / 256; ++r) rs[tid + 256 * r] = tmp[r];
    __syncthreads();
    const float* qc = qsh + cl * kMaxDim + k0;
#pragma unroll 16
    for (int kk = 0; kk < kn; ++kk) acc = fma((double)rs[kk * kPrepJ + jj], (double)qc[kk], acc);
  }
  const int c = c0 + cl;
  if (j < a.d) a.qrot[(size_t)c * a.d + j] = acc;
}

// Quantization of the query block, one half-wave per column: from the
// rotated columns eos_tq_rotate wrote, or from the raw queries when the
// corpus has no rotation. M values per lane (d <= 32 M): the _m12 variant
// for d <= 384 holds 12 (it then fits beside a running filter scan on a CU).
namespace {

template <int M>
EOS_DEV void quantize_body(const TqPrepArgs& a) {
  const int c = blockIdx.x * kPrepC + (threadIdx.x >> 5);
  if (a.rot_t != nullptr) {
    prep_quantize_column<M>(a, c, threadIdx.x & 31,
                            [&](int, int jx) { return a.qrot[(size_t)c * a.d + jx]; });
  } else if (a.q > 0) {
    prep_quantize_column<M>(a, c, threadIdx.x & 31, [&](int src, int jx) {
      return (double)a.queries[(size_t)src * a.d + jx];
    });
  } else {
    prep_quantize_column<M>(a, c, threadIdx.x & 31, [&](int, int) { return 0.0; });
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void eos_tq_quantize(TqPrepArgs a) {
  quantize_body<kMaxDim / 32>(a);
}
extern "C" __global__ __launch_bounds__(256) void eos_tq_quantize_m12(TqPrepArgs a) {
  quantize_body<12>(a);
}

// --------------------------------------------------------------------- pack


// Repacks reference-layout codes into the scan's tile layout: tile t, load c,
// lane (m + 32 g), dword wd holds the codes of vector 32 t + m for the MFMA
// fragment bytes the scan decodes from that dword. Fragment byte i of K-step s
// for lane group g is dimension 32 s + 16 g + i.
extern "C" __global__ __launch_bounds__(256) void eos_tq_pack(TqPackArgs a) {
  const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
  if (o >= a.total_dwords) return;
  const int wd = (int)(o & 3);
  const int lane = (int)((o >> 2) & 63);
  const long long tc = o >> 8;
  const int c = (int)(tc % a.nload);
  const long long t = tc / a.nload;
  const int m = lane & 31, g = lane >> 5;
  const long long v = t * kTile + m;
  const int cpb = 8 / a.bits;        // codes per byte
  const int spl = 8 / a.bits;        // K-steps per 16-byte load
  const int dps = a.bits / 2;        // dwords per K-step
  const int h = wd / dps;
  const int fbase = (wd % dps) * cpb;
  const int s = c * spl + h;
  const uint32_t mask = (1u << a.bits) - 1u;
  uint32_t out = 0;
  if (v < a.n && s < a.ks) {
    const uint8_t* row = a.codes + (size_t)v * a.row_bytes;
    for (int b = 0; b < 4; ++b) {
      for (int e = 0; e < cpb; ++e) {
        const int f = fbase + e;
        const int k = 32 * s + 16 * g + 4 * f + b;
        if (k < a.d) {
          const int bit = k * a.bits;
          const uint32_t code = (row[bit >> 3] >> (bit & 7)) & mask;
          out |= code << (8 * b + e * a.bits);
        }
      }
    }
  }
  a.packed[o] = out;
}

// Per tile, the largest ||C[codes_v]||_2 over its vectors (exact integer
// sums of squares, rounded up) and the largest Norm: one thread per vector, a
// half-wave per tile.
extern "C" __global__ __launch_bounds__(256) void eos_tq_tile_cnorm(TqTileNormArgs a) {
  const long long v = (long long)blockIdx.x * 256 + threadIdx.x;
  long long ss = 0;
  if (v < a.n) {
    const uint8_t* row = a.codes + (size_t)v * a.row_bytes;
    const uint32_t mask = (1u << a.bits) - 1u;
    const int per = 32 / a.bits;  // codes per dword
    int k = 0;
    if ((a.row_bytes & 3) == 0) {
      // Whole dwords: 8 (4-bit) or 16 (2-bit) codes per load.
      const uint32_t* rw = reinterpret_cast<const uint32_t*>(row);
      for (int w = 0; w < a.row_bytes / 4; ++w) {
        const uint32_t x = rw[w];
        for (int e = 0; e < per && k < a.d; ++e, ++k) {
          const int c = a.cb[(x >> (e * a.bits)) & mask];
          ss += (long long)(c * c);
        }
      }
    }
    for (; k < a.d; ++k) {
      const int bit = k * a.bits;
      const int c = a.cb[(row[bit >> 3] >> (bit & 7)) & mask];
      ss += (long long)(c * c);
    }
  }
  float nm = v < a.n ? a.norms[v] : 0.0f;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    const long long t = __shfl_xor(ss, o);
    ss = t > ss ? t : ss;
    nm = fmaxf(nm, __shfl_xor(nm, o));
  }
  const long long tile = v >> 5;
  if ((threadIdx.x & 31) == 0 && tile * kTile < a.n) {
    a.tile_cn[2 * tile] = sqrt_up(ss);
    a.tile_cn[2 * tile + 1] = nm;
  }
}

// ----------------------------------------------------------------- encode


// Build-defined MSE-stage encoder, one workgroup per V vectors (d <= DMAX):
//   u_j = sum_k R[j][k] x_k (f64, one fma chain per coordinate, k ascending),
//   ss = sum_k x_k^2 (f64 fma chain), nrm = sqrt(ss), norm = (float)nrm,
//   code_j = argmin_v |u_j - nrm c_v| (ties to the lower v), c_v = s_c C_v
// in f64, each product and difference rounded once (nrm c_v is formed before
// the differences and read back from LDS, so nothing is contracted). The
// vectors are staged in LDS ([k][v], f32); thread t runs the chains of
// coordinates t, t + 256, ... for all V vectors, reading R^T rows
// coalesced. Codes go through LDS and are packed low bits first.
namespace {
template <int kEncV, int DMAX>
EOS_DEV void encode_body(const TqEncodeArgs& a) {
  __shared__ float xs[DMAX * kEncV];
  __shared__ double ncs[kEncV * 16];
  __shared__ uint8_t cs[kEncV * DMAX];
  const int tid = threadIdx.x;
  const long long v0 = (long long)blockIdx.x * kEncV;
  const int nv = (int)min((long long)kEncV, a.n - v0);
  if (nv <= 0) return;
  const int d = a.d, levels = 1 << a.bits;
  // Stage x (rows past n are zero).
  for (int i = tid; i < kEncV * d; i += 256) {
    const int v = i / d, k = i - v * d;
    xs[k * kEncV + v] = v < nv ? a.x[(size_t)(v0 + v) * d + k] : 0.0f;
  }
  __syncthreads();
  if (tid < kEncV) {
    double ss = 0.0;
    for (int k = 0; k < d; ++k) {
      const double xk = (double)xs[k * kEncV + tid];
      ss = fma(xk, xk, ss);
    }
    const double nrm = __builtin_sqrt(ss);
    if (tid < nv) a.norms[v0 + tid] = (float)nrm;
    for (int l = 0; l < levels; ++l) ncs[tid * 16 + l] = nrm * ((double)a.cb_scale * (double)a.cb[l]);
  }
  __syncthreads();
  for (int j = tid; j < d; j += 256) {
    double acc[kEncV];
#pragma unroll
    for (int v = 0; v < kEncV; ++v) acc[v] = 0.0;
    if (a.rot_t != nullptr) {
      for (int k = 0; k < d; ++k) {
        const double r = (double)a.rot_t[(size_t)k * d + j];
        const float4* xr = reinterpret_cast<const float4*>(&xs[k * kEncV]);
#pragma unroll
        for (int q = 0; q < kEncV / 4; ++q) {
          const float4 xv = xr[q];
          acc[4 * q + 0] = fma(r, (double)xv.x, acc[4 * q + 0]);
          acc[4 * q + 1] = fma(r, (double)xv.y, acc[4 * q + 1]);
          acc[4 * q + 2] = fma(r, (double)xv.z, acc[4 * q + 2]);
          acc[4 * q + 3] = fma(r, (double)xv.w, acc[4 * q + 3]);
        }
      }
    } else {
#pragma unroll
      for (int v = 0; v < kEncV; ++v) acc[v] = (double)xs[j * kEncV + v];
    }
#pragma unroll 4
    for (int v = 0; v < kEncV; ++v) {
      const double u = acc[v];
      int best = 0;
      double bd = fabs(u - ncs[v * 16]);
      for (int l = 1; l < levels; ++l) {
        const double dv = fabs(u - ncs[v * 16 + l]);
        if (dv < bd) {
          bd = dv;
          best = l;
        }
      }
      cs[v * DMAX + j] = (uint8_t)best;
    }
  }
  __syncthreads();
  // Pack: byte b of vector v holds codes of coordinates 8b/bits ... (low bits first).
  const int per = 8 / a.bits;
  for (int i = tid; i < nv * a.row_bytes; i += 256) {
    const int v = i / a.row_bytes, b = i - v * a.row_bytes;
    uint32_t byte = 0;
    for (int e = 0; e < per; ++e) {
      const int j = b * per + e;
      if (j < d) byte |= (uint32_t)cs[v * DMAX + j] << (e * a.bits);
    }
    a.codes[(size_t)(v0 + v) * a.row_bytes + b] = (uint8_t)byte;
  }
}
}  // namespace

// 32 vectors per workgroup for d <= 512, 16 for d <= 1024 (LDS).
extern "C" __global__ __launch_bounds__(256) void eos_tq_encode_d512(TqEncodeArgs a) {
  encode_body<32, 512>(a);
}
extern "C" __global__ __launch_bounds__(256) void eos_tq_encode_d1024(TqEncodeArgs a) {
  encode_body<16, 1024>(a);
}

// ------------------------------------------------------- inner-product layout

// Build-defined inner-product layout after the published TurboQuant_prod
// estimator (the quantizer is in the un-vendored module; byte layout of
// runtime/turboquant_bytes.go:14-25): the MSE stage of encode_body, then a
// 1-bit QJL sketch of the residual in the rotated frame, all in f64:
//   r_j = u_j - nrm c_code_j;  ResNorm = (float)(sqrt(sum_j r_j^2) / nrm)
//   sign bit i = (sum_j S[i][j] r_j >= 0), fma chains in j order
// Eight vectors per workgroup (d <= 1024); thread t runs coordinates and
// sketch rows t, t + 256, ... for all eight, reading R^T and S^T coalesced.
constexpr int kIpV = 8;
constexpr int kIpDMax = 1024;
extern "C" __global__ __launch_bounds__(256) void eos_tq_encode_ip(TqIpArgs a) {
  __shared__ float xs[kIpDMax * kIpV];
  __shared__ double rs[kIpV * kIpDMax];
  __shared__ double ncs[kIpV * 16];
  __shared__ uint8_t cs[kIpV * kIpDMax];
  __shared__ uint8_t sb[kIpV * kIpDMax];
  __shared__ double nrms[kIpV];
  const int tid = threadIdx.x;
  const long long v0 = (long long)blockIdx.x * kIpV;
  const int nv = (int)min((long long)kIpV, a.n - v0);
  if (nv <= 0) return;
  const int d = a.d, levels = 1 << a.bits;
  for (int i = tid; i < kIpV * d; i += 256) {
    const int v = i / d, k = i - v * d;
    xs[k * kIpV + v] = v < nv ? a.x[(size_t)(v0 + v) * d + k] : 0.0f;
  }
  __syncthreads();
  if (tid < kIpV) {
    double ss = 0.0;
    for (int k = 0; k < d; ++k) {
      const double xk = (double)xs[k * kIpV + tid];
      ss = fma(xk, xk, ss);
    }
    const double nrm = __builtin_sqrt(ss);
    nrms[tid] = nrm;
    if (tid < nv) a.norms[v0 + tid] = (float)nrm;
    for (int l = 0; l < levels; ++l) ncs[tid * 16 + l] = nrm * ((double)a.cb_scale * (double)a.cb[l]);
  }
  __syncthreads();
  for (int j = tid; j < d; j += 256) {
    double acc[kIpV];
#pragma unroll
    for (int v = 0; v < kIpV; ++v) acc[v] = a.rot_t != nullptr ? 0.0 : (double)xs[j * kIpV + v];
    if (a.rot_t != nullptr) {
      for (int k = 0; k < d; ++k) {
        const double r = (double)a.rot_t[(size_t)k * d + j];
#pragma unroll
        for (int v = 0; v < kIpV; ++v) acc[v] = fma(r, (double)xs[k * kIpV + v], acc[v]);
      }
    }
#pragma unroll
    for (int v = 0; v < kIpV; ++v) {
      const double u = acc[v];
      int best = 0;
      double bd = fabs(u - ncs[v * 16]);
      for (int l = 1; l < levels; ++l) {
        const double dv = fabs(u - ncs[v * 16 + l]);
        if (dv < bd) {
          bd = dv;
          best = l;
        }
      }
      cs[v * kIpDMax + j] = (uint8_t)best;
      rs[v * kIpDMax + j] = u - ncs[v * 16 + best];
    }
  }
  __syncthreads();
  if (tid < nv) {
    double rn = 0.0;
    for (int j = 0; j < d; ++j) rn = fma(rs[tid * kIpDMax + j], rs[tid * kIpDMax + j], rn);
    const double nrm = nrms[tid];
    a.resnorms[v0 + tid] = nrm > 0.0 ? (float)(__builtin_sqrt(rn) / nrm) : 0.0f;
  }
  for (int i = tid; i < d; i += 256) {
    double p[kIpV];
#pragma unroll
    for (int v = 0; v < kIpV; ++v) p[v] = 0.0;
    for (int j = 0; j < d; ++j) {
      const double s = (double)a.qjl_t[(size_t)j * d + i];
#pragma unroll
      for (int v = 0; v < kIpV; ++v) p[v] = fma(s, rs[v * kIpDMax + j], p[v]);
    }
#pragma unroll
    for (int v = 0; v < kIpV; ++v) sb[v * kIpDMax + i] = p[v] >= 0.0 ? 1 : 0;
  }
  __syncthreads();
  // Codes packed low bits first: bit t of a row is bit t % bits of code
  // t / bits (a 3-bit code straddles two bytes where t crosses one).
  for (int i = tid; i < nv * a.row_bytes; i += 256) {
    const int v = i / a.row_bytes, b = i - v * a.row_bytes;
    uint32_t byte = 0;
    for (int e = 0; e < 8; ++e) {
      const int t = 8 * b + e, j = t / a.bits;
      if (j < d) byte |= (((uint32_t)cs[v * kIpDMax + j] >> (t - j * a.bits)) & 1u) << e;
    }
    a.codes[(size_t)(v0 + v) * a.row_bytes + b] = (uint8_t)byte;
  }
  for (int i = tid; i < nv * a.sign_bytes; i += 256) {
    const int v = i / a.sign_bytes, b = i - v * a.sign_bytes;
    uint32_t byte = 0;
    for (int e = 0; e < 8; ++e) {
      const int j = b * 8 + e;
      if (j < d) byte |= (uint32_t)sb[v * kIpDMax + j] << e;
    }
    a.signs[(size_t)(v0 + v) * a.sign_bytes + b] = (uint8_t)byte;
  }
}

// Query preparation of the inner-product layout: q' = R q and y = S q' (f64,
// one fma chain per coordinate in k order), then eos_tq_ip_quant. These are
// the matrix-vector products, workgroup (x, y) computing rows [32 x, 32 x +
// 32) for the 8 columns [8 y, 8 y + 8): the columns staged in LDS as f64 and
// the matrix slice (rows j, all k) in chunks of kPrepK values of k, with
// every load of a stage issued before any is stored (one memory round trip
// per stage; d <= kPrepK takes one stage).
extern "C" __global__ __launch_bounds__(256) void eos_tq_ip_matvec(TqIpMatArgs a) {
  __shared__ double xin[8 * kIpDMax];
  __shared__ float ms[kPrepK * kPrepJ];
  const int tid = threadIdx.x, jj = tid & 31, cl = tid >> 5;
  const int j0 = blockIdx.x * kPrepJ, c0 = blockIdx.y * 8;
  const int d = a.d;
  {
    // Loads from clamped positions first, the validity test afterwards (a
    // load under a per-lane condition waits for its data before the next).
    constexpr int R = kIpDMax / 256;
    double xv[8][R];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const int src = min(c0 + c, a.q - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const size_t o = (size_t)src * d + min(tid + 256 * r, d - 1);
        xv[c][r] = a.in64 != nullptr ? a.in64[o] : (double)a.in32[o];
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (tid + 256 * r < d) xin[c * kIpDMax + tid + 256 * r] = c0 + c < a.q ? xv[c][r] : 0.0;
  }
  const int j = j0 + jj, c = c0 + cl;
  double acc = 0.0;
  if (a.mt == nullptr) {
    __syncthreads();
    acc = j < d ? xin[cl * kIpDMax + j] : 0.0;
  } else {
    for (int k0 = 0; k0 < d; k0 += kPrepK) {
      const int kn = min(kPrepK, d - k0);
      float tmp[kPrepK * kPrepJ / 256];
#pragma unroll
      for (int r = 0; r < kPrepK * kPrepJ / 256; ++r)
        tmp[r] = a.mt[(size_t)(k0 + min(cl + 8 * r, kn - 1)) * d + min(j, d - 1)];
#pragma unroll
      for (int r = 0; r < kPrepK * kPrepJ / 256; ++r)
        tmp[r] = (cl + 8 * r < kn && j < d) ? tmp[r] : 0.0f;
      __syncthreads();  // the previous chunk consumed; xin visible
#pragma unroll
      for (int r = 0; r < kPrepK * kPrepJ / 256; ++r) ms[tid + 256 * r] = tmp[r];
      __syncthreads();
      const double* xc = xin + cl * kIpDMax + k0;
#pragma unroll 16
      for (int kk = 0; kk < kn; ++kk) acc = fma((double)ms[kk * kPrepJ + jj], xc[kk], acc);
    }
  }
  if (c < a.q && j < d) a.out[(size_t)c * d + j] = acc;
}

// Grids and scales of one query column from qr = R q and y = S qr: the MSE
// grid Qs = rint(q' qmax / max|q'|) with alpha = (max|q'| / qmax) s_c (as
// eos_tq_rotate / eos_tq_quantize), the QJL grid Ys = rint(y qmax2 / max|y|)
// and beta = (max|y| / qmax2) sqrt(pi / 2) / d; both clamped to +-qmax.
// One workgroup per column c < ncols (columns past q are zero). The grids go
// to qs / ys when given; with bfrag, also the scan's query fragments (per
// K-step and 32-column group g: blocks 4 g + 0 / + 1 the MSE grid's int8
// high / low halves Qs = 256 hi + lo, blocks 4 g + 2 / + 3 the QJL grid's),
// the sum of Ys over the dimensions (D_qjl = 2 sum_{bit = 1} Ys - sum Ys) and
// the column's filter state reset (tau = -inf, no kept candidates).
extern "C" __global__ __launch_bounds__(256) void eos_tq_ip_quant(TqIpQuantArgs a) {
  __shared__ double red[4];
  __shared__ int ired[12];
  const int c = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int d = a.d;
  const bool live = c < a.q;
  auto block_max = [&](double m) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmax(m, __shfl_xor(m, o));
    if (lane == 0) red[w] = m;
    __syncthreads();
    const double r = fmax(fmax(red[0], red[1]), fmax(red[2], red[3]));
    __syncthreads();
    return r;
  };
  const double* qr = a.qr + (size_t)(live ? c : 0) * d;
  const double* y = a.y + (size_t)(live ? c : 0) * d;
  double m1 = 0.0, m2 = 0.0;
  if (live) {
    for (int j = tid; j < d; j += 256) {
      m1 = fmax(m1, fabs(qr[j]));
      m2 = fmax(m2, fabs(y[j]));
    }
  }
  const double mq = block_max(m1);
  const double my = block_max(m2);
  const double inv = mq > 0.0 ? (double)a.qmax / mq : 0.0;
  const double inv2 = my > 0.0 ? (double)a.qmax2 / my : 0.0;
  const int dpad = a.bfrag != nullptr ? a.ks * 32 : d;
  const int gq = c >> 5, col = c & 31, ncb = 4 * a.nqg;
  int ysum = 0, lo2 = 0, plo = 0;
  for (int j = tid; j < dpad; j += 256) {
    int qv = 0, yv = 0;
    if (live && j < d) {
      double v = rint(qr[j] * inv);
      v = fmin(fmax(v, (double)-a.qmax), (double)a.qmax);
      qv = (int)v;
      double u = rint(y[j] * inv2);
      u = fmin(fmax(u, (double)-a.qmax2), (double)a.qmax2);
      yv = (int)u;
      if (a.qs != nullptr) a.qs[(size_t)c * d + j] = qv;
      if (a.ys != nullptr) a.ys[(size_t)c * d + j] = yv;
    }
    ysum += yv;
    if (a.bfrag != nullptr) {
      const int qlo = ((qv + 128) & 255) - 128, qhi = (qv - qlo) >> 8;
      const int ylo = ((yv + 128) & 255) - 128, yhi = (yv - ylo) >> 8;
      lo2 += qlo * qlo;
      plo += ylo > 0 ? ylo : 0;
      const int s = j >> 5, g = (j >> 4) & 1, i = j & 15;
      int8_t* base = a.bfrag + ((size_t)(s * ncb + 4 * gq) * 64 + col + 32 * g) * 16 + i;
      base[0] = (int8_t)qhi;
      base[64 * 16] = (int8_t)qlo;
      base[2 * 64 * 16] = (int8_t)yhi;
      base[3 * 64 * 16] = (int8_t)ylo;
    }
  }
  if (a.bfrag != nullptr) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      ysum += __shfl_xor(ysum, o);
      lo2 += __shfl_xor(lo2, o);
      plo += __shfl_xor(plo, o);
    }
    if (lane == 0) {
      ired[w] = ysum;
      ired[4 + w] = lo2;
      ired[8 + w] = plo;
    }
    __syncthreads();
  }
  if (tid == 0) {
    if (live) {
      a.alpha[c] = mq > 0.0 ? (float)((mq / (double)a.qmax) * (double)a.cb_scale) : 0.0f;
      const double half_pi = 1.5707963267948966;
      a.beta[c] = my > 0.0 ? (float)((my / (double)a.qmax2) * __builtin_sqrt(half_pi) / (double)d)
                           : 0.0f;
    }
    if (a.bfrag != nullptr) {
      const int ys_all = ired[0] + ired[1] + ired[2] + ired[3];
      a.ysum[c] = ys_all;
      a.tau[c] = -__builtin_inff();
      a.cand_count[c] = 0u;
      if (a.lonorm != nullptr) a.lonorm[c] = sqrt_up((long long)(ired[4] + ired[5] + ired[6] + ired[7]));
      if (a.kq != nullptr) a.kq[c] = 2 * (ired[8] + ired[9] + ired[10] + ired[11]) - ys_all;
    }
  }
}

// Exhaustive scores of the inner-product layout: grid (ceil(n / 256),
// ceil(q / 8)), one vector per thread against 8 queries (their grids in
// LDS), exact int32 dots, then the fixed f32 expression
//   ((float)D_mse * alpha + ResNorm * ((float)D_qjl * beta)) * Norm.
constexpr int kIpQ = 8;
extern "C" __global__ __launch_bounds__(256) void eos_tq_ip_scores(TqIpArgs a) {
  __shared__ int qs[kIpQ * kIpDMax];
  __shared__ int ys[kIpQ * kIpDMax];
  const int tid = threadIdx.x;
  const int q0 = blockIdx.y * kIpQ, nq = min(kIpQ, a.q - q0);
  const int d = a.d;
  for (int i = tid; i < kIpQ * d; i += 256) {
    const int g = i / d, j = i - g * d;
    qs[j * kIpQ + g] = g < nq ? a.qs[(size_t)(q0 + g) * d + j] : 0;
    ys[j * kIpQ + g] = g < nq ? a.ys[(size_t)(q0 + g) * d + j] : 0;
  }
  __syncthreads();
  const long long v = (long long)blockIdx.x * 256 + tid;
  if (v >= a.n) return;
  int dm[kIpQ], dq[kIpQ];
#pragma unroll
  for (int g = 0; g < kIpQ; ++g) dm[g] = dq[g] = 0;
  const uint8_t* row = a.codes + (size_t)v * a.row_bytes;
  const int mask = (1 << a.bits) - 1;
  for (int j = 0; j < d; ++j) {
    const int bit = j * a.bits, sh = bit & 7;
    unsigned cv = (unsigned)row[bit >> 3] >> sh;
    if (sh + a.bits > 8) cv |= (unsigned)row[(bit >> 3) + 1] << (8 - sh);
    const int c = a.cb[cv & (unsigned)mask];
#pragma unroll
    for (int g = 0; g < kIpQ; ++g) dm[g] += qs[j * kIpQ + g] * c;
  }
  const uint8_t* sg = a.signs + (size_t)v * a.sign_bytes;
  for (int j = 0; j < d; ++j) {
    const bool pos = (sg[j >> 3] >> (j & 7)) & 1;
#pragma unroll
    for (int g = 0; g < kIpQ; ++g) dq[g] += pos ? ys[j * kIpQ + g] : -ys[j * kIpQ + g];
  }
  const float rn = a.resnorms[v], nm = a.norms[v];
  for (int g = 0; g < nq; ++g) {
    const float t1 = __fmul_rn((float)dm[g], a.alpha[q0 + g]);
    const float t2 = __fmul_rn((float)dq[g], a.beta[q0 + g]);
    const float t3 = __fmul_rn(rn, t2);
    a.scores[(size_t)(q0 + g) * a.n + v] = __fmul_rn(__fadd_rn(t1, t3), nm);
  }
}

// --------------------------------------------------------------------- scan


namespace {

// 16-entry int8 lookup of four 4-bit codes (one per byte) in four VALU ops:
// two 8-byte v_perm tables, the second indexed with bit 3 flipped; table
// bytes are pre-XORed so that the sign-replicate/zero/0xFF selector results
// of the out-of-range half cancel (tables are solved on the host).
EOS_DEV uint32_t lut16(uint32_t x, uint32_t l0, uint32_t l1, uint32_t l2, uint32_t l3) {
  return __builtin_amdgcn_perm(l1, l0, x) ^ __builtin_amdgcn_perm(l3, l2, x ^ 0x08080808u);
}

template <int BITS>
EOS_DEV v4i decode_step(const v4i& raw, int h, const TqScanArgs& a);

template <>
EOS_DEV v4i decode_step<4>(const v4i& raw, int h, const TqScanArgs& a) {
  const uint32_t w0 = (uint32_t)(h == 0 ? raw.x : raw.z);
  const uint32_t w1 = (uint32_t)(h == 0 ? raw.y : raw.w);
  v4i f;
  f.x = (int)lut16(w0 & 0x0f0f0f0fu, a.lut0, a.lut1, a.lut2, a.lut3);
  f.y = (int)lut16((w0 >> 4) & 0x0f0f0f0fu, a.lut0, a.lut1, a.lut2, a.lut3);
  f.z = (int)lut16(w1 & 0x0f0f0f0fu, a.lut0, a.lut1, a.lut2, a.lut3);
  f.w = (int)lut16((w1 >> 4) & 0x0f0f0f0fu, a.lut0, a.lut1, a.lut2, a.lut3);
  return f;
}

template <>
EOS_DEV v4i decode_step<2>(const v4i& raw, int h, const TqScanArgs& a) {
  const uint32_t w = (uint32_t)(h == 0 ? raw.x : h == 1 ? raw.y : h == 2 ? raw.z : raw.w);
  v4i f;
  f.x = (int)__builtin_amdgcn_perm(0u, a.lut0, w & 0x03030303u);
  f.y = (int)__builtin_amdgcn_perm(0u, a.lut0, (w >> 2) & 0x03030303u);
  f.z = (int)__builtin_amdgcn_perm(0u, a.lut0, (w >> 4) & 0x03030303u);
  f.w = (int)__builtin_amdgcn_perm(0u, a.lut0, (w >> 6) & 0x03030303u);
  return f;
}

// Per-workgroup candidate stage of the filter scan: kept rank keys are
// appended with LDS atomics and flushed to the global list once per query at
// the end, so the scan never waits on a global atomic.
constexpr int kLdsSlots = 16;

// Register budget of the scan's stage ring and accumulators (the rest of the
// 256 registers of two waves per SIMD hold decode temporaries, per-query
// constants, addresses and, without HI, the exact-score epilogue), and the
// deepest ring used.
constexpr int kRingRegsHi = 176;
constexpr int kRingRegsExact = 150;
constexpr int kRingCap = 2;
constexpr int kRingCapHi = 2;

template <int NLOAD>
EOS_DEV void load_tile_codes(v4i (&r)[NLOAD], const v4i* packed, long long tile, int lane) {
  const v4i* src = packed + (size_t)tile * NLOAD * 64 + lane;
#pragma unroll
  for (int c = 0; c < NLOAD; ++c) r[c] = __builtin_nontemporal_load(src + c * 64);
}

EOS_DEV void load_tile_norms(float4 (&n)[4], const float* norms, long long tile, int half) {
#pragma unroll
  for (int i4 = 0; i4 < 4; ++i4)
    n[i4] = *reinterpret_cast<const float4*>(norms + tile * kTile + 8 * i4 + 4 * half);
}

// FILTER = true: keep (score >= tau) rank keys (mode 1). FILTER = false: write
// every score (mode 0 dense slice, mode 2 sampled tiles).
// HI (with FILTER): only the high int8 half of the query enters the MFMAs.
// With Qs = 256 hi + lo, D = 256 D_hi + sum_j lo_j C_j and, by Cauchy-Schwarz,
// |sum_j lo_j C_j| <= ||lo||_2 ||C[codes]||_2 <= L = lonorm * tile_cn (both
// rounded up, the product bumped by 2^-22). Rounding to nearest is monotone,
// so fl(fl(256 D_hi + L) n) >= fl(fl(D) n): every row whose exact score could
// reach tau passes the exact filter's pre-test on this bound. Such rows are
// kept as ids only; eos_tq_rescore computes their exact scores.
template <int BITS, int KS, int NQG, bool FILTER, bool HI = false>
EOS_DEV void tq_scan_body(const TqScanArgs& a) {
  constexpr int NCB = 2 * NQG;
  constexpr int NCBU = HI ? NQG : NCB;  // column blocks the MFMAs use
  constexpr int SPL = 8 / BITS;
  constexpr int NLOAD = (KS + SPL - 1) / SPL;
  constexpr int NQ = 32 * NQG;
  constexpr int NTH = scan_threads(HI, KS);
  __shared__ v4i sb[KS * NCBU * 64];
  __shared__ uint32_t lc_cnt[FILTER ? NQ : 1];
  __shared__ u64 lc_buf[FILTER ? NQ * kLdsSlots : 1];
  __shared__ float4 nstage[NTH / 64][8];
  __shared__ int tile_next;
  if (a.gate != nullptr) {
    // Exhaustive pass of the exact fallback: run only when a query was flagged.
    bool any = false;
    for (int i = 0; i < a.q; ++i) any |= a.gate[i] != 0;
    if (!any) return;
  }
  const int lane = threadIdx.x & 63;
  // Wave-uniform tile indices keep the tile addressing in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int NWV = NTH / 64;
  const int half = lane >> 5;
  const v4i* packed = reinterpret_cast<const v4i*>(a.packed);
  // Per-column constants live in registers for the whole scan: a global load
  // inside the tile loop would make every tile wait for the code prefetch
  // issued ahead of it (loads retire in order).
  float al_r[NQG], ta_r[NQG], lo_r[NQG];
  bool live_r[NQG];
#pragma unroll
  for (int g = 0; g < NQG; ++g) {
    const int qi = g * 32 + (lane & 31);
    live_r[g] = qi < a.q;
    al_r[g] = live_r[g] ? a.alpha[qi] : 0.0f;
    ta_r[g] = (FILTER && live_r[g]) ? a.tau[qi] : __builtin_inff();
    lo_r[g] = (HI && live_r[g]) ? a.lonorm[qi] : 0.0f;
  }
  float pt_r[NQG];  // filled once the first tile loads are issued
  // Software pipeline over a ring of register stages (unrolled so that no
  // stage is ever copied: a copy of a register still being loaded would wait
  // for every load issued before it). A stage holds a tile's codes and one
  // norm per lane (row lane % 32 of its tile); the epilogue redistributes the
  // norms to the accumulator layout through a 128-byte LDS slot of the wave.
  struct Stage {
    v4i raw[NLOAD];
    float nv;
    int t;  // tile index in [0, ntiles); >= the range end: none
  };
  // Codes first, then norms: lanes 0-31 load the tile's norms; with HI, lanes
  // 32 and 33 load its tile_cn pair (code-norm bound, largest Norm).
  auto load_stage = [&](Stage& st, int jj) {
    const long long t = a.tile_begin + (long long)jj * a.tile_step;
    load_tile_codes<NLOAD>(st.raw, packed, t, lane);
    if constexpr (HI)
      st.nv = lane < 32 ? a.norms[t * kTile + lane] : a.tile_cn[2 * t + (lane & 1)];
    else
      st.nv = a.norms[t * kTile + (lane & 31)];
  };
  auto process = [&](const Stage& st, int j) {
    const v4i(&raw)[NLOAD] = st.raw;
    const long long tile = a.tile_begin + (long long)j * a.tile_step;
    // Opaque per-tile LDS offset: keeps the query fragments in LDS rather than
    // letting them be hoisted into registers across the tile loop.
    int boff = lane;
    asm volatile("" : "+v"(boff));
    v16i acc[NCBU];
#pragma unroll
    for (int cb = 0; cb < NCBU; ++cb) acc[cb] = v16i{0};
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
      for (int h = 0; h < SPL; ++h) {
        const int s = c * SPL + h;
        if (s < KS) {
          const v4i af = decode_step<BITS>(raw[c], h, a);
#pragma unroll
          for (int cb = 0; cb < NCBU; ++cb) {
            const v4i bf = sb[(s * NCBU + cb) * 64 + boff];
            acc[cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, acc[cb], 0, 0, 0);
          }
        }
      }
    }
    // Epilogue. Accumulator element i of lane l is row 8(i/4) + 4(l/32) + i%4
    // (a corpus vector of the tile) and column l%32 (a query of the group).
    const long long vbase = tile * kTile;
    // Rows of this tile that are real vectors (the last tile may be partial).
    const long long rem64 = a.n - vbase;
    const int rem = rem64 >= kTile ? kTile : (int)rem64;
    // Row r's norm sits at float r of the wave's slot; lane l needs rows
    // 8 i4 + 4 (l / 32) + {0..3}, i.e. float4 2 i4 + l / 32. LDS operations of
    // one wave complete in order, so no barrier is needed around the slot.
    float nrm[16];
    auto row_norms = [&]() {
      if (lane < 32) reinterpret_cast<float*>(nstage[wave])[lane] = st.nv;
      __builtin_amdgcn_wave_barrier();
      float4 nrm4[4];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) nrm4[i4] = nstage[wave][2 * i4 + half];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        nrm[4 * i4 + 0] = nrm4[i4].x;
        nrm[4 * i4 + 1] = nrm4[i4].y;
        nrm[4 * i4 + 2] = nrm4[i4].z;
        nrm[4 * i4 + 3] = nrm4[i4].w;
      }
    };
    if constexpr (HI) {
      const float cn = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(st.nv), 32));
      const float nmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(st.nv), 33));
      // Tile-level test first: with A = max_i acc_i and N = the tile's
      // largest Norm, fl(fl(256 A + lb) N) >= every row's fl(fl(256 acc_i +
      // lb) n_i) whenever it is >= 0 (rounding is monotone, n_i <= N), and
      // when it is < 0 no row reaches pt > 0; pt = -inf passes every tile.
      // Only lanes that pass evaluate their rows.
      bool pass[NQG];
      bool anyp = false;
#pragma unroll
      for (int g = 0; g < NQG; ++g) {
        int am = acc[g][0];
#pragma unroll
        for (int i = 1; i < 16; ++i) am = max(am, acc[g][i]);
        const float lb = (lo_r[g] * cn) * 1.0000002f;  // >= lonorm * cn exactly
        pass[g] = __builtin_fmaf((float)am, 256.0f, lb) * nmax >= pt_r[g];
        anyp |= pass[g];
      }
      if (__ballot(anyp) == 0ull) return;
      row_norms();
#pragma unroll
      for (int g = 0; g < NQG; ++g) {
        if (!pass[g]) continue;
        const int qi = g * 32 + (lane & 31);
        const float lb = (lo_r[g] * cn) * 1.0000002f;  // >= lonorm * cn exactly
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          // fl(D) * 256 is exact, so one fma gives fl(fl(D) * 256 + lb).
          p[i] = __builtin_fmaf((float)acc[g][i], 256.0f, lb) * nrm[i];
        }
        float m = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, p[i]);
        if (m >= pt_r[g]) {
          // Rare path (about one kept row per wave and group): one LDS atomic
          // per kept row reserves its slot; rows past the stage's capacity go
          // to the global list.
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * half + (i & 3);
            if (r < rem && p[i] >= pt_r[g]) {
              const u64 key = (u64)(~(uint32_t)(vbase + r));  // id only; rescored later
              const uint32_t pos = atomicAdd(&lc_cnt[qi], 1u);
              if (pos < (uint32_t)kLdsSlots) {
                lc_buf[qi * kLdsSlots + pos] = key;
              } else {
                const uint32_t gpos = atomicAdd(&a.cand_count[qi], 1u);
                if ((int)gpos < a.cap) a.cand[(size_t)qi * a.cap + gpos] = key;
              }
            }
          }
        }
      }
      return;
    }
    row_norms();
#pragma unroll
    for (int g = 0; g < NQG; ++g) {
      const int qi = g * 32 + (lane & 31);
      const bool live = live_r[g];
      const float al = al_r[g];
      int dots[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) dots[i] = acc[2 * g][i] * 256 + acc[2 * g + 1][i];
      if constexpr (FILTER) {
        const float ta = ta_r[g];
        // Conservative pre-test: max_i fl(fl(D_i) * norm_i) >= pt_r whenever
        // some exact score of the lane reaches tau (pt_r carries the slack).
        float m = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 16; ++i) m = fmaxf(m, (float)dots[i] * nrm[i]);
        if (m >= pt_r[g]) {
          float sc[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) sc[i] = ((float)dots[i] * al) * nrm[i] + 0.0f;
          // Rare path: count this lane's kept rows, reserve LDS slots with one
          // LDS atomic; keys past the stage's capacity go to the global list.
          uint32_t cnt = 0;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * half + (i & 3);
            cnt += (r < rem && sc[i] >= ta) ? 1u : 0u;
          }
          uint32_t pos = atomicAdd(&lc_cnt[qi], cnt);
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * half + (i & 3);
            if (r < rem && sc[i] >= ta) {
              const u64 key = rank_key(sc[i], (uint32_t)(vbase + r));
              if (pos < (uint32_t)kLdsSlots) {
                lc_buf[qi * kLdsSlots + pos] = key;
              } else {
                const uint32_t gpos = atomicAdd(&a.cand_count[qi], 1u);
                if ((int)gpos < a.cap) a.cand[(size_t)qi * a.cap + gpos] = key;
              }
              ++pos;
            }
          }
        }
      } else if (live) {
        float sc[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) sc[i] = ((float)dots[i] * al) * nrm[i] + 0.0f;
        if (a.mode == 0) {
          float* orow = a.out_scores + (size_t)qi * a.out_stride;
          int32_t* drow = a.out_dots != nullptr ? a.out_dots + (size_t)qi * a.out_stride : nullptr;
          const long long c0 = vbase - a.out_begin;
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * half + (i & 3);
            const long long colx = c0 + r;
            if (r < rem && colx >= 0 && colx < a.out_count) {
              orow[colx] = sc[i];
              if (drow != nullptr) drow[colx] = dots[i];
            }
          }
        } else {
          // Sample mode: the best score of the tile's real rows for this query
          // (lanes l and l^32 hold the two halves of the tile's rows).
          float m = -__builtin_inff();
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int r = 8 * (i >> 2) + 4 * half + (i & 3);
            if (r < rem) m = fmaxf(m, sc[i]);
          }
          m = fmaxf(m, __shfl_xor(m, 32));
          if (half == 0) a.out_scores[(size_t)qi * a.out_stride + j] = m;
        }
      }
    }
  };
  // Work distribution: workgroup b (one per CU) owns the contiguous tile
  // range [rb, re). Its waves take their first R - 1 tiles statically and
  // then claim tiles one at a time from an LDS counter, so the two waves that
  // share a SIMD finish together however the SIMD arbitrates between them
  // (with a fixed share per wave, one of them ran its last quarter alone).
  const int nt = a.ntiles;
  const int rb = (int)((long long)blockIdx.x * nt / gridDim.x);
  const int re = (int)((long long)(blockIdx.x + 1) * nt / gridDim.x);
  // Loads past the range are clamped to its last tile rather than skipped, so
  // every path issues the same loads and each wait covers only the stage it
  // needs (the host launches no more workgroups than tiles).
  auto cl = [&](int jj) { return jj < re ? jj : re - 1; };
  auto claim = [&]() {
    int v = 0;
    if (lane == 0) v = atomicAdd(&tile_next, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };
  // Ring depth R: a stage holds one tile's codes and norms; R - 1 stages are in
  // flight while one is processed. Deeper rings keep more bytes in flight per
  // wave (bandwidth = bytes in flight / latency), as many as fit next to the
  // accumulators in the 256 registers of two waves per SIMD.
  constexpr int kStageRegs = NLOAD * 4 + 1;
  constexpr int kRingFit = ((HI ? kRingRegsHi : kRingRegsExact) - NCBU * 16) / kStageRegs;
  constexpr int kCap = HI ? kRingCapHi : kRingCap;
  constexpr int R = kRingFit > kCap ? kCap : kRingFit < 2 ? 2 : kRingFit;
  Stage st[R];
  // Query fragments (HI: the high-half blocks only, block cb = 2 g of each
  // K-step) are staged in LDS once per workgroup. Loads retire in order, so
  // the fragments are requested before the first tiles whenever their
  // registers fit beside the ring: no wave then waits for R - 1 tiles before
  // it can start. Every wave reaches the barrier.
  constexpr int FCOUNT = KS * NCBU * 64;
  constexpr int FPER = (FCOUNT + NTH - 1) / NTH;
  constexpr bool kFragFirst = FPER * 4 + (R - 1) * kStageRegs <= 200;
  const v4i* fsrc = reinterpret_cast<const v4i*>(a.bfrag);
  auto frag_index = [&](int i) {
    if constexpr (HI) {
      const int stp = i / (NQG * 64), g = (i / 64) % NQG, l = i % 64;
      return (stp * NCB + 2 * g) * 64 + l;
    } else {
      return i;
    }
  };
  // Unconditional (indices are clamped; the host launches no scan without a
  // tile): a branch here would make the wait before the fragment writes cover
  // the tile loads as well.
  auto prologue = [&]() {
#pragma unroll
    for (int p = 0; p < R - 1; ++p) {
      st[p].t = rb + wave + p * NWV;
      load_stage(st[p], cl(st[p].t));
    }
  };
  if constexpr (!kFragFirst) prologue();
  {
    v4i fv[FPER];
#pragma unroll
    for (int r = 0; r < FPER; ++r) {
      const int i = threadIdx.x + r * NTH;
      if (i < FCOUNT) fv[r] = fsrc[frag_index(i)];
    }
    if constexpr (kFragFirst) prologue();
#pragma unroll
    for (int r = 0; r < FPER; ++r) {
      const int i = threadIdx.x + r * NTH;
      if (i < FCOUNT) sb[i] = fv[r];
    }
  }
  if (FILTER && threadIdx.x < NQ) lc_cnt[threadIdx.x] = 0u;
  if (threadIdx.x == 0) tile_next = rb + (R - 1) * NWV;
  __syncthreads();
  // Pre-test thresholds of the filter (computed after the first loads are
  // issued, so their wait covers only the per-query values). For tau > 0 and alpha > 0 a kept score
  // s = fl(fl(fl(D) a) n) >= tau implies D > 0, n > 0 and, with u = 2^-24,
  // p = fl(fl(D) n) >= (tau / a)(1 - u) / (1 + u)^2 > (tau / a)(1 - 2^-16)
  // rounded, which is pt. Other cases test every row exactly (pt = -inf) or
  // none (alpha = 0: every score is 0 < tau).
#pragma unroll
  for (int g = 0; g < NQG; ++g) {
    const float ta = ta_r[g], al = al_r[g];
    float pt = -__builtin_inff();
    if (ta > 0.0f) {
      if (!(al > 0.0f)) {
        pt = __builtin_inff();
      } else {
        pt = (ta / al) * 0.9999847412109375f;
        if (!(pt <= 3.402823466e38f)) pt = -__builtin_inff();
      }
    }
    pt_r[g] = pt;
  }
  if (st[0].t < re) {
    // Phase p of a pass refills the stage processed in phase p - 1 with a
    // newly claimed tile, then processes stage p; stages past the range only
    // load (a wave-uniform branch). A wave's claims increase, so once the next
    // stage to process is past the range every later one is too. The loop has
    // a single exit at its end: exits between phases make the compiler's wait
    // analysis merge every phase at the loop head and wait for all but the
    // newest stage.
    do {
#pragma unroll
      for (int p = 0; p < R; ++p) {
        Stage& nx = st[(p + R - 1) % R];
        nx.t = claim();
        load_stage(nx, cl(nx.t));
        if (st[p].t < re) process(st[p], st[p].t);
      }
    } while (st[0].t < re);
  }
  if constexpr (FILTER) {
    // Flush the stage: one global atomic per query per workgroup.
    __syncthreads();
    if (threadIdx.x < NQ && threadIdx.x < a.q) {
      const int qi = threadIdx.x;
      const uint32_t nk = lc_cnt[qi] < (uint32_t)kLdsSlots ? lc_cnt[qi] : (uint32_t)kLdsSlots;
      if (nk > 0) {
        const uint32_t base = atomicAdd(&a.cand_count[qi], nk);
        for (uint32_t i = 0; i < nk; ++i)
          if ((int)(base + i) < a.cap) a.cand[(size_t)qi * a.cap + base + i] = lc_buf[qi * kLdsSlots + i];
      }
    }
  }
}

}  // namespace

#define EOS_TQ_SCAN(BITS, KS, NQG)                                                        \
  extern "C" __global__ __launch_bounds__(scan_threads(false, KS)) __attribute__((amdgpu_waves_per_eu(2, 8))) \
  void eos_tq_scan_b##BITS##_k##KS##_g##NQG##_f(TqScanArgs a) {                           \
    tq_scan_body<BITS, KS, NQG, true>(a);                                                 \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(scan_threads(false, KS)) __attribute__((amdgpu_waves_per_eu(2, 8))) \
  void eos_tq_scan_b##BITS##_k##KS##_g##NQG##_w(TqScanArgs a) {                           \
    tq_scan_body<BITS, KS, NQG, false>(a);                                                \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(scan_threads(true, KS))                         \
      __attribute__((amdgpu_waves_per_eu(scan_threads(true, KS) / 256, 8)))               \
  void eos_tq_scan_b##BITS##_k##KS##_g##NQG##_h(TqScanArgs a) {                           \
    tq_scan_body<BITS, KS, NQG, true, true>(a);                                           \
  }

#define EOS_TQ_SCAN_KS(BITS, NQG) \
  EOS_TQ_SCAN(BITS, 1, NQG)       \
  EOS_TQ_SCAN(BITS, 2, NQG)       \
  EOS_TQ_SCAN(BITS, 4, NQG)       \
  EOS_TQ_SCAN(BITS, 8, NQG)       \
  EOS_TQ_SCAN(BITS, 12, NQG)      \
  EOS_TQ_SCAN(BITS, 16, NQG)      \
  EOS_TQ_SCAN(BITS, 24, NQG)

EOS_TQ_SCAN_KS(4, 1)
EOS_TQ_SCAN_KS(4, 2)
EOS_TQ_SCAN_KS(2, 1)
EOS_TQ_SCAN_KS(2, 2)
EOS_TQ_SCAN(4, 32, 1)
EOS_TQ_SCAN(2, 32, 1)

// ---------------------------------------------------- inner-product scan

// Repacks an inner-product corpus into the scan's tile layout (TqIpPackArgs):
// one thread per (tile, chunk, lane), 16 bytes each; thread 0 .. 31 of a tile's
// chunk 0 also copy the tile's norms and ResNorms (zero past n).
extern "C" __global__ __launch_bounds__(256) void eos_tq_ip_pack(TqIpPackArgs a) {
  const int nl = a.ks / 2;
  const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
  if (o >= a.ntiles * nl * 64) return;
  const int lane = (int)(o & 63);
  const long long tc = o >> 6;
  const int c = (int)(tc % nl);
  const long long t = tc / nl;
  const int m = lane & 31, g = lane >> 5;
  const long long v = t * 32 + m;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (v < a.n) {
    const uint8_t* row = a.codes + (size_t)v * a.row_bytes;
    const uint8_t* sg = a.signs + (size_t)v * a.sign_bytes;
    for (int h = 0; h < 2; ++h) {
      const int s = 2 * c + h;
      uint32_t L = 0u, HS = 0u;
      for (int i = 0; i < 16; ++i) {
        const int j = 32 * s + 16 * g + i;
        if (j >= a.d) break;
        const int bit = j * a.bits, sh = bit & 7;
        uint32_t code = (uint32_t)row[bit >> 3] >> sh;
        if (sh + a.bits > 8) code |= (uint32_t)row[(bit >> 3) + 1] << (8 - sh);
        code &= (1u << a.bits) - 1u;
        const uint32_t sign = (sg[j >> 3] >> (j & 7)) & 1u;
        const int k = i >> 2, b = i & 3;
        L |= (code & 3u) << (8 * b + 2 * k);
        HS |= ((code >> 2) & 1u) << (8 * b + k);
        HS |= sign << (8 * b + 4 + k);
      }
      w[2 * h] = L;
      w[2 * h + 1] = HS;
    }
  }
  int32_t* dst = a.packed + (size_t)o * 4;
  *reinterpret_cast<v4i*>(dst) = v4i{(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
  if (c == 0 && g == 0) {
    a.norms_out[v] = v < a.n ? a.norms[v] : 0.0f;
    a.resnorms_out[v] = v < a.n ? a.resnorms[v] : 0.0f;
  }
}

namespace {

// 8-entry int8 lookup of the 3-bit codes and 0/1 bytes of the sign bits of
// one K-step (dwords L, HS of the tile layout): af = C[code] per fragment
// byte, sf = the sign bits as bytes.
EOS_DEV void ip_decode(uint32_t L, uint32_t HS, uint32_t lut0, uint32_t lut1, v4i& af, v4i& sf) {
  const uint32_t m2 = 0x03030303u, m1 = 0x01010101u;
  const uint32_t c0 = (L & m2) | ((HS & m1) << 2);
  const uint32_t c1 = ((L >> 2) & m2) | (((HS >> 1) & m1) << 2);
  const uint32_t c2 = ((L >> 4) & m2) | (((HS >> 2) & m1) << 2);
  const uint32_t c3 = ((L >> 6) & m2) | (((HS >> 3) & m1) << 2);
  af.x = (int)__builtin_amdgcn_perm(lut1, lut0, c0);
  af.y = (int)__builtin_amdgcn_perm(lut1, lut0, c1);
  af.z = (int)__builtin_amdgcn_perm(lut1, lut0, c2);
  af.w = (int)__builtin_amdgcn_perm(lut1, lut0, c3);
  sf.x = (int)((HS >> 4) & m1);
  sf.y = (int)((HS >> 5) & m1);
  sf.z = (int)((HS >> 6) & m1);
  sf.w = (int)((HS >> 7) & m1);
}

// HI (mode 1 only): the high-half bound filter. With Qs = 256 hi + lo and
// Ys = 256 yhi + ylo, D_mse <= 256 D_mse,hi + lb (lb = ||lo||_2 times the
// tile's largest ||C[codes]||_2, both rounded up, bumped by 2^-22) and
// D_qjl = 2 sum_{bit=1} Ys - sum Ys <= 512 S_hi + kq (S_hi = sum_{bit=1}
// yhi, kq = 2 sum max(ylo, 0) - sum Ys). The score's f32 expression is
// monotone in both dots (alpha, beta, ResNorm, Norm >= 0; rounding is
// monotone), so evaluated on the bounds it is >= the exact score: every row
// scoring >= tau is kept, as an id for eos_tq_ip_rescore.
template <int KS, int NQG, bool HI>
EOS_DEV void tq_ipscan_body(const TqIpScanArgs& a) {
  constexpr int NCB = 4 * NQG, NQ = 32 * NQG, NTH = 512, NWV = NTH / 64, NLOAD = KS / 2;
  constexpr int UPG = HI ? 2 : 4;  // column blocks per group in the MFMAs
  constexpr int NCBU = UPG * NQG;
  __shared__ v4i sb[KS * NCBU * 64];
  __shared__ uint32_t lc_cnt[NQ];
  __shared__ u64 lc_buf[NQ * kLdsSlots];
  __shared__ float4 nstage[NWV][16];
  __shared__ int tile_next;
  if (a.gate != nullptr) {
    bool any = false;
    for (int i = 0; i < a.q; ++i) any |= a.gate[i] != 0;
    if (!any) return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5;
  const v4i* packed = reinterpret_cast<const v4i*>(a.packed);
  const bool filter = a.mode == 1;
  float al_r[NQG], be_r[NQG], ta_r[NQG], lo_r[NQG];
  int ys_r[NQG];
  bool live_r[NQG];
#pragma unroll
  for (int g = 0; g < NQG; ++g) {
    const int qi = g * 32 + (lane & 31);
    live_r[g] = qi < a.q;
    al_r[g] = live_r[g] ? a.alpha[qi] : 0.0f;
    be_r[g] = live_r[g] ? a.beta[qi] : 0.0f;
    ys_r[g] = live_r[g] ? (HI ? a.kq[qi] : a.ysum[qi]) : 0;
    ta_r[g] = (filter && live_r[g]) ? a.tau[qi] : __builtin_inff();
    lo_r[g] = (HI && live_r[g]) ? a.lonorm[qi] : 0.0f;
  }
  struct Stage {
    v4i raw[NLOAD];
    float nv;  // lanes 0-31: the tile's Norms; lanes 32-63: its ResNorms
    float cn;  // HI: the tile's code-norm bound
    int t;
  };
  auto load_stage = [&](Stage& st, int jj) {
    const long long t = a.tile_begin + (long long)jj * a.tile_step;
    const v4i* src = packed + (size_t)t * NLOAD * 64 + lane;
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) st.raw[c] = __builtin_nontemporal_load(src + c * 64);
    st.nv = lane < 32 ? a.norms[t * kTile + lane] : a.resnorms[t * kTile + (lane & 31)];
    if constexpr (HI) st.cn = a.tile_cn[4 * t];
  };
  auto process = [&](const Stage& st, int j) {
    const long long tile = a.tile_begin + (long long)j * a.tile_step;
    int boff = lane;
    asm volatile("" : "+v"(boff));
    v16i acc[NCBU];
#pragma unroll
    for (int cb = 0; cb < NCBU; ++cb) acc[cb] = v16i{0};
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int s = 2 * c + h;
        v4i af, sf;
        ip_decode((uint32_t)(h == 0 ? st.raw[c].x : st.raw[c].z),
                  (uint32_t)(h == 0 ? st.raw[c].y : st.raw[c].w), a.lut0, a.lut1, af, sf);
#pragma unroll
        for (int g = 0; g < NQG; ++g) {
#pragma unroll
          for (int u = 0; u < UPG; ++u) {
            const v4i bf = sb[(s * NCBU + UPG * g + u) * 64 + boff];
            const bool mse = HI ? u == 0 : u < 2;
            acc[UPG * g + u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(mse ? af : sf, bf,
                                                                    acc[UPG * g + u], 0, 0, 0);
          }
        }
      }
    }
    // Epilogue: accumulator element i of lane l is row 8 (i / 4) + 4 (l / 32)
    // + i % 4 of the tile and query column l % 32 of the group.
    const long long vbase = tile * kTile;
    const long long rem64 = a.n - vbase;
    const int rem = rem64 >= kTile ? kTile : (int)rem64;
    // The tile's Norms and ResNorms go to the wave's LDS slot; each group of
    // four rows reads its values there (no per-row registers held across the
    // epilogue). LDS operations of one wave complete in order.
    reinterpret_cast<float*>(nstage[wave])[lane] = st.nv;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int g = 0; g < NQG; ++g) {
      if (!live_r[g]) continue;
      const int qi = g * 32 + (lane & 31);
      float smax = -__builtin_inff();
      const float lb = HI ? (lo_r[g] * st.cn) * 1.0000002f : 0.0f;  // >= lonorm * cn
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        const float4 n4 = nstage[wave][2 * i4 + half];
        const float4 r4 = nstage[wave][8 + 2 * i4 + half];
        const float nv4[4] = {n4.x, n4.y, n4.z, n4.w};
        const float rv4[4] = {r4.x, r4.y, r4.z, r4.w};
        float sc[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * i4 + e;
          float fdm, fdq;
          if constexpr (HI) {
            fdm = __builtin_fmaf((float)acc[2 * g][i], 256.0f, lb);
            fdq = (float)(acc[2 * g + 1][i] * 512 + ys_r[g]);
          } else {
            fdm = (float)(acc[4 * g][i] * 256 + acc[4 * g + 1][i]);
            fdq = (float)(2 * (acc[4 * g + 2][i] * 256 + acc[4 * g + 3][i]) - ys_r[g]);
          }
          const float t1 = fdm * al_r[g];
          const float t2 = fdq * be_r[g];
          const float t3 = rv4[e] * t2;
          sc[e] = (t1 + t3) * nv4[e];
        }
        const int r0 = 8 * i4 + 4 * half;  // rows r0 .. r0 + 3
        if (a.mode == 1) {
          const float ta = ta_r[g];
          uint32_t cnt = 0;
#pragma unroll
          for (int e = 0; e < 4; ++e) cnt += (r0 + e < rem && sc[e] >= ta) ? 1u : 0u;
          if (cnt != 0u) {
            uint32_t pos = atomicAdd(&lc_cnt[qi], cnt);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if (r0 + e < rem && sc[e] >= ta) {
                const u64 key = HI ? (u64)(~(uint32_t)(vbase + r0 + e))
                                   : rank_key(sc[e], (uint32_t)(vbase + r0 + e));
                if (pos < (uint32_t)kLdsSlots) {
                  lc_buf[qi * kLdsSlots + pos] = key;
                } else {
                  const uint32_t gpos = atomicAdd(&a.cand_count[qi], 1u);
                  if ((int)gpos < a.cap) a.cand[(size_t)qi * a.cap + gpos] = key;
                }
                ++pos;
              }
            }
          }
        } else if (a.mode == 0) {
          float* orow = a.out_scores + (size_t)qi * a.out_stride;
          const long long c0 = vbase - a.out_begin;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const long long colx = c0 + r0 + e;
            if (r0 + e < rem && colx >= 0 && colx < a.out_count) orow[colx] = sc[e];
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (r0 + e < rem) smax = fmaxf(smax, sc[e]);
        }
      }
      if (a.mode == 2) {
        smax = fmaxf(smax, __shfl_xor(smax, 32));
        if (half == 0) a.out_scores[(size_t)qi * a.out_stride + j] = smax;
      }
    }
    __builtin_amdgcn_wave_barrier();
  };
  const int nt = a.ntiles;
  const int rb = (int)((long long)blockIdx.x * nt / gridDim.x);
  const int re = (int)((long long)(blockIdx.x + 1) * nt / gridDim.x);
  auto cl = [&](int jj) { return jj < re ? jj : re - 1; };
  auto claim = [&]() {
    int v = 0;
    if (lane == 0) v = atomicAdd(&tile_next, 1);
    return __builtin_amdgcn_readfirstlane(v);
  };
  constexpr int R = 2;
  Stage st[R];
  {
    // HI stages the high blocks only (block 4 g of the MSE grid, 4 g + 2 of
    // the QJL grid).
    constexpr int FCOUNT = KS * NCBU * 64;
    constexpr int FPER = (FCOUNT + NTH - 1) / NTH;
    const v4i* fsrc = reinterpret_cast<const v4i*>(a.bfrag);
    v4i fv[FPER];
#pragma unroll
    for (int r = 0; r < FPER; ++r) {
      const int i = threadIdx.x + r * NTH;
      const int stp = i / (NCBU * 64), rem = i - stp * (NCBU * 64);
      const int cb = HI ? 4 * ((rem >> 6) >> 1) + 2 * ((rem >> 6) & 1) : (rem >> 6);
      if (i < FCOUNT) fv[r] = fsrc[((size_t)stp * NCB + cb) * 64 + (rem & 63)];
    }
    st[0].t = rb + wave;
    load_stage(st[0], cl(st[0].t));
#pragma unroll
    for (int r = 0; r < FPER; ++r) {
      const int i = threadIdx.x + r * NTH;
      if (i < FCOUNT) sb[i] = fv[r];
    }
  }
  if (threadIdx.x < NQ) lc_cnt[threadIdx.x] = 0u;
  if (threadIdx.x == 0) tile_next = rb + NWV;
  __syncthreads();
  if (st[0].t < re) {
    do {
#pragma unroll
      for (int p = 0; p < R; ++p) {
        Stage& nx = st[(p + R - 1) % R];
        nx.t = claim();
        load_stage(nx, cl(nx.t));
        if (st[p].t < re) process(st[p], st[p].t);
      }
    } while (st[0].t < re);
  }
  if (a.mode == 1) {
    __syncthreads();
    if (threadIdx.x < NQ && threadIdx.x < a.q) {
      const int qi = threadIdx.x;
      const uint32_t nk = lc_cnt[qi] < (uint32_t)kLdsSlots ? lc_cnt[qi] : (uint32_t)kLdsSlots;
      if (nk > 0) {
        const uint32_t base = atomicAdd(&a.cand_count[qi], nk);
        for (uint32_t i = 0; i < nk; ++i)
          if ((int)(base + i) < a.cap) a.cand[(size_t)qi * a.cap + base + i] = lc_buf[qi * kLdsSlots + i];
      }
    }
  }
}

}  // namespace

#define EOS_TQ_IPSCAN(KS, NQG)                                                            \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 8))) \
  void eos_tq_ipscan_k##KS##_g##NQG(TqIpScanArgs a) {                                     \
    tq_ipscan_body<KS, NQG, false>(a);                                                    \
  }                                                                                        \
  extern "C" __global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 8))) \
  void eos_tq_ipscan_k##KS##_g##NQG##_h(TqIpScanArgs a) {                                 \
    tq_ipscan_body<KS, NQG, true>(a);                                                     \
  }
EOS_TQ_IPSCAN(4, 2)
EOS_TQ_IPSCAN(8, 2)
EOS_TQ_IPSCAN(12, 2)
EOS_TQ_IPSCAN(16, 1)
EOS_TQ_IPSCAN(24, 1)
EOS_TQ_IPSCAN(32, 1)
#undef EOS_TQ_IPSCAN

// Exact rescoring of the inner-product filter's kept ids (TqIpRescoreArgs):
// grid (q, y), eight threads per candidate. The workgroup's query fragments
// (the scan's int8 halves of both grids, fragment byte order) are staged in
// LDS; a thread takes the (K step, lane half) units u = sub, sub + 8, ... of
// the vector (16 dimensions each, 8 bytes of the tile layout), decodes them
// as the scan does and accumulates the four int8 dots with v_dot4. The dots
// are exact integers, the score the scan's f32 expression.
extern "C" __global__ __launch_bounds__(256) void eos_tq_ip_rescore(TqIpRescoreArgs a) {
  __shared__ v4i fr[32 * 2 * 4];  // [K step][lane half][MSE hi, MSE lo, QJL hi, QJL lo]
  const int q = blockIdx.x;
  if (q >= a.q) return;
  const int tid = threadIdx.x, sub = tid & 7;
  const uint32_t cnt = a.cand_count[q];
  if (cnt > (uint32_t)a.cap) return;  // overflowed: finalize flags it
  const uint32_t first = blockIdx.y * 32u;
  if (first >= cnt) return;
  const int nl = a.ks / 2, nunits = 2 * a.ks;
  u64* list = a.cand + (size_t)q * a.cap;
  // The first entry is requested together with the fragments (one round
  // trip for both).
  uint32_t lid_next = first + (uint32_t)(tid >> 3) < cnt ? rank_id(list[first + (tid >> 3)]) : 0u;
  {
    const int gq = q >> 5, col = q & 31, ncb = 4 * a.nqg;
    const v4i* bf = reinterpret_cast<const v4i*>(a.bfrag);
    for (int i = tid; i < nunits * 4; i += 256) {
      const int u = i >> 2, blk = i & 3, st = u >> 1, g = u & 1;
      fr[i] = bf[((size_t)st * ncb + 4 * gq + blk) * 64 + col + 32 * g];
    }
  }
  __syncthreads();
  const float al = a.alpha[q], be = a.beta[q], ta = a.tau[q];
  const int ysum = a.ysum[q];
  const uint2* packed = reinterpret_cast<const uint2*>(a.packed);
  for (uint32_t base = first; base < cnt; base += 32u * gridDim.y) {
    // Entries are rewritten in place, so a lane past the end reads no entry
    // (it scores vector 0 and writes nothing); an id outside the corpus is
    // dropped without reading its codes.
    const uint32_t i = base + (uint32_t)(tid >> 3);
    const bool in_list = i < cnt;
    const uint32_t lid = base == first ? lid_next : (in_list ? rank_id(list[i]) : 0u);
    const bool live = in_list && (long long)lid < a.n;
    const uint32_t v = live ? lid : 0u;
    const long long t = v >> 5;
    const int m = (int)(v & 31u);
    const float rn = a.resnorms[v], nv = a.norms[v];
    int dm = 0, sq = 0;
    for (int u = sub; u < nunits; u += 8) {
      const int st = u >> 1, g = u & 1;
      // dwords 2 (st % 2) and + 1 of the lane's 16 bytes of chunk st / 2
      const uint2 w = packed[(((size_t)t * nl + (st >> 1)) * 64 + m + 32 * g) * 2 + (st & 1)];
      v4i af, sf;
      ip_decode(w.x, w.y, a.lut0, a.lut1, af, sf);
      const v4i qh = fr[4 * u], ql = fr[4 * u + 1], yh = fr[4 * u + 2], yl = fr[4 * u + 3];
      int dh = 0, dl = 0, sh = 0, sl = 0;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        dh = __builtin_amdgcn_sdot4(af[k], qh[k], dh, false);
        dl = __builtin_amdgcn_sdot4(af[k], ql[k], dl, false);
        sh = __builtin_amdgcn_sdot4(sf[k], yh[k], sh, false);
        sl = __builtin_amdgcn_sdot4(sf[k], yl[k], sl, false);
      }
      dm += dh * 256 + dl;
      sq += sh * 256 + sl;
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) {
      dm += __shfl_xor(dm, o);
      sq += __shfl_xor(sq, o);
    }
    const int dq = 2 * sq - ysum;
    const float t1 = (float)dm * al;
    const float t2 = (float)dq * be;
    const float t3 = rn * t2;
    const float sc = (t1 + t3) * nv;
    if (in_list && sub == 0) list[i] = (live && sc >= ta) ? rank_key(sc, v) : 0ull;
  }
}

// Per tile of the inner-product layout, the largest ||C[codes]||_2 over its
// vectors (exact integer sums of squares, rounded up): one thread per
// vector, a half-wave per tile.
extern "C" __global__ __launch_bounds__(256) void eos_tq_ip_tile_cnorm(TqIpTileNormArgs a) {
  const long long v = (long long)blockIdx.x * 256 + threadIdx.x;
  long long ss = 0;
  if (v < a.n) {
    const uint8_t* row = a.codes + (size_t)v * a.row_bytes;
    const uint32_t mask = (1u << a.bits) - 1u;
    for (int j = 0; j < a.d; ++j) {
      const int bit = j * a.bits, sh = bit & 7;
      uint32_t code = (uint32_t)row[bit >> 3] >> sh;
      if (sh + a.bits > 8) code |= (uint32_t)row[(bit >> 3) + 1] << (8 - sh);
      const int c = a.cb[code & mask];
      ss += (long long)(c * c);
    }
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    const long long t = __shfl_xor(ss, o);
    ss = t > ss ? t : ss;
  }
  const long long tile = v >> 5;
  if ((threadIdx.x & 31) == 0 && tile * kTile < a.n) {
    a.tile_cn[4 * tile] = sqrt_up(ss);
    a.tile_cn[4 * tile + 1] = 0.0f;
    a.tile_cn[4 * tile + 2] = 0.0f;
    a.tile_cn[4 * tile + 3] = 0.0f;
  }
}

// ----------------------------------------------------------------- rescore

namespace {


// Candidates of query blockIdx.x spread over gridDim.y workgroups, four
// threads per id: thread s of the four decodes chunks s, s + 4, ... of the
// id's code row (reference layout, rs 16-byte chunks). The list entry is read
// first, then the code row, the norm and the query are requested together,
// so the kernel waits two memory round trips. The partial dots are summed
// over the four; the entry is rewritten in place with the exact rank key
// when the exact score ((float)D * alpha) * norm + 0 reaches tau, else with 0
// (below every rank key: finalize skips it). Dimension k of a row is at bit
// k * BITS, low bits first.
template <int BITS>
EOS_DEV void rescore_body(const TqRescoreArgs& a) {
  constexpr int kSlots = 8;                 // chunks per thread: rs <= 32
  constexpr int kDims = 32 * 128 / BITS;    // dims of the longest row
  constexpr int kQPer = kDims / 256;        // query values staged per thread
  __shared__ int qsh[kDims];
  const int q = blockIdx.x;
  if (q >= a.q) return;
  const int tid = threadIdx.x, sub = tid & 3;
  const uint32_t cnt = a.cand_count[q];
  if (cnt > (uint32_t)a.cap) return;  // overflowed: finalize flags it
  const uint32_t first = blockIdx.y * 64u;
  if (first >= cnt) return;
  const int dims = a.rs * 128 / BITS;
  const float al = a.alpha[q], ta = a.tau[q];
  u64* list = a.cand + (size_t)q * a.cap;
  for (uint32_t base = first; base < cnt; base += 64u * gridDim.y) {
    // Entries are rewritten in place, so a lane past the end must not read
    // another entry (it may already be 0): it scores vector 0 and writes
    // nothing. An id outside the corpus is dropped without reading its row.
    const uint32_t i = base + (uint32_t)(tid >> 2);
    const bool in_list = i < cnt;
    const uint32_t lid = in_list ? rank_id(list[i]) : 0u;
    const bool live = in_list && (long long)lid < a.n;
    const uint32_t id = live ? lid : 0u;
    const v4i* row = reinterpret_cast<const v4i*>(a.codes + (size_t)id * a.rs * 16);
    v4i r[kSlots];
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int c = sub + 4 * u;
      r[u] = c < a.rs ? row[c] : v4i{0, 0, 0, 0};
    }
    const float nv = a.norms[id];
    if (base == first) {
      int qv[kQPer];
#pragma unroll
      for (int u = 0; u < kQPer; ++u) {
        const int j = tid + 256 * u;
        qv[u] = (j < dims && j < a.d) ? (int)a.qs[(size_t)q * a.d + j] : 0;
      }
#pragma unroll
      for (int u = 0; u < kQPer; ++u)
        if (tid + 256 * u < dims) qsh[tid + 256 * u] = qv[u];
      __syncthreads();
    }
    int D = 0;
#pragma unroll
    for (int u = 0; u < kSlots; ++u) {
      const int c = sub + 4 * u;
      if (c < a.rs) {
#pragma unroll
        for (int wi = 0; wi < 4; ++wi) {
          const uint32_t w = (uint32_t)r[u][wi];
          const int* qp = &qsh[(16 * c + 4 * wi) * (8 / BITS)];  // first dim of the dword
          if constexpr (BITS == 4) {
            // byte b holds dims 2b (low nibble) and 2b + 1
            const uint32_t ev = lut16(w & 0x0f0f0f0fu, a.lut0, a.lut1, a.lut2, a.lut3);
            const uint32_t od = lut16((w >> 4) & 0x0f0f0f0fu, a.lut0, a.lut1, a.lut2, a.lut3);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
              D += qp[2 * b] * (int)(int8_t)(ev >> (8 * b));
              D += qp[2 * b + 1] * (int)(int8_t)(od >> (8 * b));
            }
          } else {
            // byte b holds dims 4b + e, e = 0..3
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const uint32_t v = __builtin_amdgcn_perm(0u, a.lut0, (w >> (2 * e)) & 0x03030303u);
#pragma unroll
              for (int b = 0; b < 4; ++b) D += qp[4 * b + e] * (int)(int8_t)(v >> (8 * b));
            }
          }
        }
      }
    }
    D += __shfl_xor(D, 1);
    D += __shfl_xor(D, 2);
    const float sc = ((float)D * al) * nv + 0.0f;
    if (in_list && sub == 0) list[i] = (live && sc >= ta) ? rank_key(sc, id) : 0ull;
  }
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void eos_tq_rescore_b4(TqRescoreArgs a) {
  rescore_body<4>(a);
}
extern "C" __global__ __launch_bounds__(256) void eos_tq_rescore_b2(TqRescoreArgs a) {
  rescore_body<2>(a);
}

// ------------------------------------------------------------ row select


namespace {

constexpr int kSelThreads = 1024;
constexpr int kSortCap = 8192;

EOS_DEV void bitonic_sort_desc(u64* list, int npow) {
  for (int k = 2; k <= npow; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < npow; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const u64 x = list[i], y = list[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (x < y) : (x > y)) {
            list[i] = y;
            list[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

}  // namespace

// Exact radix selection of the kk-th best element of a score row by its
// composite rank key (up to 8 passes of 8-bit digits; keys are unique, so
// exactly kk elements are >= the selected key). One workgroup per row, or
// per (row, chunk) in mode 2.
extern "C" __global__ __launch_bounds__(kSelThreads) void eos_tq_row_select(TqSelectArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ u64 sel_prefix;
  __shared__ int sel_rem;
  __shared__ int sel_done;
  __shared__ int list_n;
  __shared__ u64 list[kSortCap];
  const int row = blockIdx.x;
  if (row >= a.nrows) return;
  if (a.mode == 1 && a.status != nullptr && a.status[row] == 0) return;
  const int tid = threadIdx.x;
  if (a.kk <= 0 || a.n <= 0) return;
  // Elements [c0, c0 + n) of the row: the whole row, or one chunk in mode 2.
  long long c0 = 0, n = a.n;
  if (a.mode == 2) {
    const long long per = (a.n + a.nchunks - 1) / a.nchunks;
    c0 = (long long)blockIdx.y * per;
    n = c0 < a.n ? (a.n - c0 < per ? a.n - c0 : per) : 0ll;
    if (blockIdx.y == 0 && tid == 0) a.counts_out[row] = (uint32_t)(a.nchunks * a.kk);
  }
  const float* x = a.rows + (size_t)row * a.stride + c0;
  if (a.mode == 0 && (long long)a.kk > n) {
    if (tid == 0) a.tau[row] = -__builtin_inff();
    return;
  }
  // A chunk of at most kk elements is kept whole (threshold 0).
  const int passes = a.mode == 0 ? 4 : ((long long)a.kk >= n ? 0 : 8);
  if (tid == 0) {
    sel_prefix = 0ull;
    sel_rem = a.kk;
    sel_done = 0;
  }
  __syncthreads();
  for (int p = 0; p < passes && sel_done == 0; ++p) {
    const int shift = 56 - 8 * p;
    for (int b = tid; b < 256; b += kSelThreads) hist[b] = 0u;
    __syncthreads();
    const u64 pfx = sel_prefix;
    const u64 hmask = p == 0 ? 0ull : ~((1ull << (shift + 8)) - 1ull);
    for_each_batched<kSelThreads, 8>(x, n, [&](long long i, float v) {
      const u64 c = rank_key(v, (uint32_t)(c0 + i));
      if (((c ^ pfx) & hmask) == 0ull) atomicAdd(&hist[(c >> shift) & 255u], 1u);
    });
    __syncthreads();
    if (tid == 0) {
      int rem = sel_rem;
      uint32_t cum = 0;
      int digit = 0;
      for (int b = 255; b >= 0; --b) {
        if (cum + hist[b] >= (uint32_t)rem) {
          digit = b;
          rem -= (int)cum;
          break;
        }
        cum += hist[b];
      }
      sel_rem = rem;
      sel_prefix = pfx | ((u64)digit << shift);
      // Selecting a set (modes 1, 2): once every element under the prefix
      // is needed, the keys >= the prefix (lower digits 0) are exactly kk.
      if (a.mode != 0 && hist[digit] == (uint32_t)rem) sel_done = 1;
    }
    __syncthreads();
  }
  const u64 thr = sel_prefix;
  if (a.mode == 0) {
    if (tid == 0) a.tau[row] = key_score((uint32_t)(thr >> 32));
    return;
  }
  // modes 1, 2: gather the (at most) kk elements >= thr.
  int npow = 1;
  while (npow < a.kk) npow <<= 1;
  if (tid == 0) list_n = 0;
  for (int i = tid; i < npow; i += kSelThreads) list[i] = 0ull;
  __syncthreads();
  for_each_batched<kSelThreads, 8>(x, n, [&](long long i, float v) {
    const u64 c = rank_key(v, (uint32_t)(c0 + i));
    if (c >= thr) {
      const int pos = atomicAdd(&list_n, 1);
      if (pos < kSortCap) list[pos] = c;
    }
  });
  __syncthreads();
  if (a.mode == 2) {
    u64* out = a.keys_out + ((size_t)row * a.nchunks + blockIdx.y) * a.kk;
    for (int i = tid; i < a.kk; i += kSelThreads) out[i] = list[i];
    return;
  }
  bitonic_sort_desc(list, npow);
  for (int i = tid; i < a.kk; i += kSelThreads) {
    const u64 c = list[i];
    const uint32_t p = rank_id(c);
    a.ids[(size_t)row * a.kk + i] = a.id_map != nullptr ? a.id_map[p] : (long long)p;
    a.scores[(size_t)row * a.kk + i] = key_score((uint32_t)(c >> 32));
  }
}

// --------------------------------------------------------------- threshold

namespace {

constexpr int kFinThreads = 256;
constexpr int kThrMax = 4096;         // tile maxima per row the threshold accepts
constexpr int kThrThreads = 256;
constexpr int kRankSortMax = 1024;    // finalize orders up to this many by rank counting

// Block-wide exclusive suffix sum: thread t gets the sum of v over threads
// t' > t. `scr` holds NT / 64 words.
template <int NT>
EOS_DEV uint32_t block_suffix_excl(uint32_t v, uint32_t* scr) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t s = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const uint32_t t = (uint32_t)__shfl_down((int)s, o);
    if (lane + o < 64) s += t;
  }
  if constexpr (NT > 64) {
    if (lane == 0) scr[wave] = s;  // wave total
    __syncthreads();
    uint32_t above = 0;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w)
      if (w > wave) above += scr[w];
    __syncthreads();
    return s - v + above;
  } else {
    return s - v;
  }
}

// Block-wide min and max of per-thread values (`scr` holds 2 * NT / 64 words).
template <int NT>
EOS_DEV void block_minmax(uint32_t& vmin, uint32_t& vmax, uint32_t* scr) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    vmin = min(vmin, (uint32_t)__shfl_xor((int)vmin, o));
    vmax = max(vmax, (uint32_t)__shfl_xor((int)vmax, o));
  }
  if constexpr (NT > 64) {
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
      scr[wave] = vmin;
      scr[NT / 64 + wave] = vmax;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) {
      vmin = min(vmin, scr[w]);
      vmax = max(vmax, scr[NT / 64 + w]);
    }
    __syncthreads();
  }
}

// The r-th largest (1-based, with multiplicity) of the 32-bit keys
// key_at(i).second over the members (key_at(i).first) of i in [0, count).
// Bits shared by the members' minimum and maximum are skipped; the remaining
// bits are resolved by radix passes of up to 8 bits over per-wave LDS
// histograms (`hist` holds NT / 64 * 256 words; per-wave copies keep the
// atomics of clustered keys from serialising on one bin). Requires
// 1 <= r <= the member count. On return *rank_in_bin is r's rank among the
// members equal to the result and *bin_count their number. Every thread of
// the block calls it.
template <int NT, typename KeyAt>
EOS_DEV uint32_t block_select_desc(int count, KeyAt key_at, uint32_t r, uint32_t* hist,
                                   uint32_t* scr, uint32_t* rank_in_bin, uint32_t* bin_count) {
  constexpr int NW = NT / 64;
  constexpr int BPT = 256 / NT;  // histogram bins per thread
  const int wave = threadIdx.x >> 6;
  uint32_t kmin = 0xffffffffu, kmax = 0u, nmem = 0u;
  for (int i = threadIdx.x; i < count; i += NT) {
    const auto m = key_at(i);
    if (m.first) {
      kmin = min(kmin, m.second);
      kmax = max(kmax, m.second);
      ++nmem;
    }
  }
  block_minmax<NT>(kmin, kmax, scr + 8);
  if (kmin == kmax) {
    // Every member holds the same key.
    const uint32_t tot = nmem + block_suffix_excl<NT>(nmem, scr + 8);  // thread 0: all members
    if (threadIdx.x == 0) scr[2] = tot;
    __syncthreads();
    *rank_in_bin = r;
    *bin_count = scr[2];
    __syncthreads();
    return kmin;
  }
  int bits = 32 - __clz(kmin ^ kmax);  // bits still to resolve: [bits - 1, 0]
  uint32_t mask = bits >= 32 ? 0u : ~((1u << bits) - 1u);
  uint32_t prefix = kmin & mask, nbin = 0u;
  while (bits > 0) {
    const int w = bits < 8 ? bits : 8;
    const int shift = bits - w;
    const uint32_t dmask = (1u << w) - 1u;
    for (int b = threadIdx.x; b < NW * 256; b += NT) hist[b] = 0u;
    __syncthreads();
    uint32_t* wh = hist + wave * 256;
    for (int i = threadIdx.x; i < count; i += NT) {
      const auto m = key_at(i);
      if (m.first && (m.second & mask) == prefix) atomicAdd(&wh[(m.second >> shift) & dmask], 1u);
    }
    __syncthreads();
    uint32_t h[BPT], tot = 0;
#pragma unroll
    for (int k = 0; k < BPT; ++k) {
      uint32_t c = 0;
#pragma unroll
      for (int v = 0; v < NW; ++v) c += hist[v * 256 + threadIdx.x * BPT + k];
      h[k] = c;
      tot += c;
    }
    // Members in bins above this thread's, then walk its bins downwards.
    uint32_t above = block_suffix_excl<NT>(tot, scr + 8);
#pragma unroll
    for (int k = BPT - 1; k >= 0; --k) {
      if (above < r && above + h[k] >= r) {
        scr[0] = (uint32_t)(threadIdx.x * BPT + k);
        scr[1] = r - above;
        scr[2] = h[k];
      }
      above += h[k];
    }
    __syncthreads();
    const uint32_t digit = scr[0];
    r = scr[1];
    nbin = scr[2];
    __syncthreads();
    prefix |= digit << shift;
    mask |= dmask << shift;
    bits = shift;
  }
  *rank_in_bin = r;
  *bin_count = nbin;
  return prefix;
}

struct KeyPair {
  bool first;
  uint32_t second;
};

}  // namespace

// Per query: tau = the r-th best of the sampled tiles' best scores (radix
// selection on the order-preserving key; one wavefront per query). The r-th
// best tile maximum is <= the r-th best sampled score, and any tau <= the true
// k-th best score is valid: the finalize kernel proves the kept set after the
// fact.
extern "C" __global__ __launch_bounds__(kThrThreads) void eos_tq_threshold(TqSelectArgs a) {
  __shared__ uint32_t keys[kThrMax];
  __shared__ uint32_t hist[kThrThreads / 64 * 256];
  __shared__ uint32_t scr[16];
  const int row = blockIdx.x;
  if (row >= a.nrows) return;
  const int tid = threadIdx.x;
  if ((long long)a.kk > a.n || a.kk <= 0 || a.n > kThrMax) {
    if (tid == 0) a.tau[row] = -__builtin_inff();
    return;
  }
  const int n = (int)a.n;
  const float* x = a.rows + (size_t)row * a.stride;
  for_each_batched<kThrThreads, 8>(x, n, [&](long long i, float v) { keys[i] = score_key(v); });
  __syncthreads();
  uint32_t rib, nb;
  const uint32_t k = block_select_desc<kThrThreads>(
      n, [&](int i) { return KeyPair{true, keys[i]}; }, (uint32_t)a.kk, hist, scr, &rib, &nb);
  if (tid == 0) a.tau[row] = k < 0x00800000u ? -__builtin_inff() : key_score(k);
}

// --------------------------------------------------------------- finalize

// Orders each query's kept candidates (score desc, id asc) and emits the first
// kk. A radix selection on the 32-bit score key finds the kk-th best score K;
// if K is tied across the cut, a second selection over the tied candidates'
// low words (~id) picks the lowest ids. Rank keys are unique, so exactly kk
// candidates are >= the resulting composite threshold; they are ordered by
// rank counting (or a bitonic sort when kk is large). A query whose kept set
// is smaller than kk or overflowed is flagged (status 1 / 2) for the
// exhaustive path; status 0 means its output row is final.
namespace {

// SEL: capacity of the selected set (kSortCap, or kRankSortMax for k <= 1024:
// 76 KB of LDS instead of 140, so that it runs beside a filter scan on the
// same CU when batches are in flight on several streams).
template <int SEL>
EOS_DEV void finalize_body(const TqFinalizeArgs& a) {
  __shared__ u64 cbuf[kSortCap];
  __shared__ u64 sel[SEL];
  __shared__ uint32_t hist[kFinThreads / 64 * 256];
  __shared__ uint32_t scr[16];
  __shared__ uint32_t sel_n;
  const int row = blockIdx.x;
  if (row >= a.q) return;
  const int tid = threadIdx.x;
  const uint32_t cnt = a.cand_count[row];
  if (cnt > (uint32_t)a.cap || cnt > (uint32_t)kSortCap) {
    if (tid == 0) a.status[row] = 2;
    return;
  }
  if (cnt < (uint32_t)a.kk || a.kk <= 0) {
    if (tid == 0) a.status[row] = a.kk <= 0 ? 0 : 1;
    return;
  }
  const int n = (int)cnt;
  const u64* src = a.cand + (size_t)row * a.cap;
  // Entries equal to 0 were dropped by the rescoring (below every rank key);
  // the row is final only if at least kk entries remain.
  uint32_t live = 0;
  for_each_batched<kFinThreads, 8>(src, n, [&](long long i, u64 v) {
    cbuf[i] = v;
    live += v != 0ull ? 1u : 0u;
  });
  if (tid == 0) sel_n = 0u;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) live += (uint32_t)__shfl_xor((int)live, o);
  if ((tid & 63) == 0) scr[tid >> 6] = live;
  __syncthreads();
  live = 0;
#pragma unroll
  for (int w = 0; w < kFinThreads / 64; ++w) live += scr[w];
  __syncthreads();  // scr is reused by the selection
  if (tid == 0) a.cand_count[row] = live;
  if (live < (uint32_t)a.kk) {
    if (tid == 0) a.status[row] = 1;
    return;
  }
  const uint32_t kk = (uint32_t)a.kk;
  uint32_t need, ne;
  const uint32_t K = block_select_desc<kFinThreads>(
      n, [&](int i) { return KeyPair{true, (uint32_t)(cbuf[i] >> 32)}; }, kk, hist, scr, &need, &ne);
  u64 thr = (u64)K << 32;
  if (ne > need) {
    // Tie at the cut: of the ne candidates scoring K keep the `need` with the
    // lowest ids, i.e. the largest low words (~id).
    uint32_t r2, n2;
    const uint32_t L = block_select_desc<kFinThreads>(
        n,
        [&](int i) {
          const u64 c = cbuf[i];
          return KeyPair{(uint32_t)(c >> 32) == K, (uint32_t)c};
        },
        need, hist, scr, &r2, &n2);
    thr |= L;
  }
  for (int i = tid; i < n; i += kFinThreads) {
    const u64 c = cbuf[i];
    if (c >= thr) {
      const uint32_t pos = atomicAdd(&sel_n, 1u);
      if (pos < kk) sel[pos] = c;
    }
  }
  __syncthreads();
  if (kk <= (uint32_t)kRankSortMax) {
    for (uint32_t i = tid; i < kk; i += kFinThreads) {
      const u64 x = sel[i];
      uint32_t rank = 0;
#pragma unroll 8
      for (uint32_t j = 0; j < kk; ++j) rank += sel[j] > x ? 1u : 0u;
      const uint32_t p = rank_id(x);
      a.ids[(size_t)row * kk + rank] = a.id_map != nullptr ? a.id_map[p] : (long long)p;
      a.scores[(size_t)row * kk + rank] = key_score((uint32_t)(x >> 32));
    }
  } else {
    int npow = 1;
    while (npow < (int)kk) npow <<= 1;
    for (int i = (int)kk + tid; i < npow; i += kFinThreads) sel[i] = 0ull;
    __syncthreads();
    bitonic_sort_desc(sel, npow);
    for (uint32_t i = tid; i < kk; i += kFinThreads) {
      const u64 x = sel[i];
      const uint32_t p = rank_id(x);
      a.ids[(size_t)row * kk + i] = a.id_map != nullptr ? a.id_map[p] : (long long)p;
      a.scores[(size_t)row * kk + i] = key_score((uint32_t)(x >> 32));
    }
  }
  if (tid == 0) a.status[row] = 0;
}

}  // namespace

extern "C" __global__ __launch_bounds__(kFinThreads) void eos_tq_finalize(TqFinalizeArgs a) {
  finalize_body<kSortCap>(a);
}
extern "C" __global__ __launch_bounds__(kFinThreads) void eos_tq_finalize_k1024(TqFinalizeArgs a) {
  finalize_body<kRankSortMax>(a);
}

// ------------------------------------------------------------------ maxsim

namespace {

// Token maxima of one query group over a tile's 16 rows of the lane: the
// exact score ((float)(256 hi + lo) * alpha) * norm of each (row, token).
EOS_DEV void maxsim_epilogue(float& mx, const v16i& hi, const v16i& lo, float al,
                             const float (&nrm)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int dot = hi[i] * 256 + lo[i];
    mx = fmaxf(mx, ((float)dot * al) * nrm[i]);
  }
}

// High-half bound of the same maxima: with Qs = 256 hi + lo and |sum_j lo_j
// C_j| <= lb (lonorm times the tile's largest ||C[codes]||_2, both rounded
// up, the product bumped by 2^-22), x = fl(256 D_hi + lb) >= fl(D) (rounding
// is monotone), and my = max_i fl(x_i n_i). For alpha, n_i >= 0 every exact
// score fl(fl(fl(D_i) alpha) n_i) is at most max(my, 0) alpha (1 + 2^-21),
// which the caller applies once per token.
EOS_DEV void maxsim_bound(float& my, const v16i& hi, float lb, const float (&nrm)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) my = fmaxf(my, __builtin_fmaf((float)hi[i], 256.0f, lb) * nrm[i]);
}

// Register stages of the MaxSim tile ring: as many as fit beside the
// accumulators in the 168 registers of three waves per SIMD.
template <bool HI>
constexpr int maxsim_ring(int nload) {
  const int stage = 4 * nload + 1;
  const int r = (HI ? 30 : 22) / stage;
  return r < 2 ? 2 : r > 8 ? 8 : r;
}

template <int CTRL>
EOS_DEV float ms_dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// v of lane l ^ 16 / l ^ 32 through a permlane swap of v with itself (the
// builtin's two results are copied out before the bit casts).
EOS_DEV float ms_other16(float v, bool upper) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  return __builtin_bit_cast(float, upper ? r0 : r1);
}
EOS_DEV void ms_halves(float v, float& lo, float& hi) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  lo = __builtin_bit_cast(float, r0);
  hi = __builtin_bit_cast(float, r1);
}
// The token sum of a document score: the butterfly v + v[l ^ o] for o = 1,
// 2, 4, 8, 16 over the 32 token lanes, by DPP and one permlane swap instead
// of LDS permutes. The values are the butterfly's: after the quad steps all
// four lanes of a quad hold the same sum, so the half-row mirror (lane 7 - i
// of each 8) reads the value lane i ^ 4 holds, and likewise the row mirror
// for i ^ 8; each add is commutative.
EOS_DEV float ms_token_sum(float v, int lane) {
  v = v + ms_dpp<0xb1>(v);   // quad_perm [1, 0, 3, 2]: lane ^ 1
  v = v + ms_dpp<0x4e>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2
  v = v + ms_dpp<0x141>(v);  // row_half_mirror
  v = v + ms_dpp<0x140>(v);  // row_mirror
  const bool odd_row = (lane & 16) != 0;
  const float o = ms_other16(v, odd_row);
  return odd_row ? o + v : v + o;
}

// MaxSim of documents against NQG query groups (32 token columns each) per
// pass; HI: the high-half bound filter (half the MFMAs) that lists the
// documents whose score bound reaches some group's tau.
template <int BITS, int KS, int NQG, bool HI>
EOS_DEV void tq_maxsim_body(const TqMaxsimArgs& a) {
  constexpr int NCB = 2 * NQG;
  constexpr int NCBU = HI ? NQG : NCB;  // column blocks staged and used
  constexpr int SPL = 8 / BITS;
  constexpr int NLOAD = (KS + SPL - 1) / SPL;
  constexpr int NWV = kScanThreads / 64;
  __shared__ v4i sb[KS * NCBU * 64];
  __shared__ float4 nstage[NWV][8];
  const int goff = blockIdx.y * NQG;          // first query group of this pass
  const int gl = min(NQG, a.groups - goff);   // its live groups
  if (gl <= 0) return;
  if (a.gate != nullptr) {
    bool any = false;
    for (int g = 0; g < gl; ++g) any |= a.gate[goff + g] != 0;
    if (!any) return;
  }
  const uint32_t* dlist = a.doc_list != nullptr ? a.doc_list + (size_t)blockIdx.y * a.list_cap : nullptr;
  long long ndocs = a.ndocs;
  if (dlist != nullptr) {
    const uint32_t c = a.list_count[blockIdx.y];
    ndocs = c < (uint32_t)a.list_cap ? (long long)c : (long long)a.list_cap;
    if (blockIdx.x == 0 && threadIdx.x < (unsigned)gl) a.cand_count[goff + threadIdx.x] = c;
  }
  {
    // The pass's column blocks of each K step (HI: the high blocks only;
    // fragments laid out [ks][frag_ncb][64] for all queries prepared).
    constexpr int COUNT = KS * NCBU * 64;
    constexpr int PER = (COUNT + kScanThreads - 1) / kScanThreads;
    const v4i* src = reinterpret_cast<const v4i*>(a.bfrag);
    const int cb0 = a.frag_cb0 + 2 * goff;
    v4i v[PER];
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int i = threadIdx.x + r * kScanThreads;
      const int s = i / (NCBU * 64), rem = i - s * (NCBU * 64);
      const int cb = HI ? 2 * (rem >> 6) : (rem >> 6), l = rem & 63;
      if (i < COUNT) v[r] = src[((size_t)s * a.frag_ncb + cb0 + cb) * 64 + l];
    }
#pragma unroll
    for (int r = 0; r < PER; ++r) {
      const int i = threadIdx.x + r * kScanThreads;
      if (i < COUNT) sb[i] = v[r];
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  // Wave-uniform document and tile indices live in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const long long nw = (long long)gridDim.x * NWV;
  const int half = lane >> 5;
  const int tpd = a.tiles_per_doc;
  // Wave w scores documents w, w + nw, ... (no barrier follows).
  const long long doc0 = (long long)blockIdx.x * NWV + wave;
  if (doc0 >= ndocs) return;
  const long long last_doc = doc0 + (ndocs - 1 - doc0) / nw * nw;
  const long long dstride = a.doc_stride > 0 ? a.doc_stride : 1;
  const v4i* packed = reinterpret_cast<const v4i*>(a.packed);
  TqScanArgs la;  // lookup tables for decode_step
  la.lut0 = a.lut0;
  la.lut1 = a.lut1;
  la.lut2 = a.lut2;
  la.lut3 = a.lut3;
  float al[NQG], lo_r[NQG], ta_r[NQG];
#pragma unroll
  for (int g = 0; g < NQG; ++g) {
    const int gg = min(goff + g, a.groups - 1);
    al[g] = a.alpha[gg * 32 + (lane & 31)];
    lo_r[g] = HI ? a.lonorm[gg * 32 + (lane & 31)] : 0.0f;
    ta_r[g] = (HI || dlist != nullptr) ? a.tau[gg] : 0.0f;
  }
  // The wave's tiles form one stream of (document, tile) steps through a
  // ring of register stages that are never copied (a copy of a register
  // still being loaded would wait for every load issued before it). Every
  // phase issues the same loads (past the wave's last step they repeat its
  // last tile), so each wait covers exactly the stages it needs. A stage
  // holds the tile's codes and one value per lane: the norm of row lane % 32
  // (lanes 0-31; all lanes without HI) and, with HI, the tile's code-norm
  // bound and largest Norm (lanes 32 + even / odd); and its document id.
  // Tile indices advance by increments; a listed document's id comes from a
  // register that holds the ids of the wave's next 64 documents (lane j:
  // document j), refilled after every 64, so no load waits on an id.
  struct Stage {
    v4i raw[NLOAD];
    float nv;
    long long id;
  };
  const long long wave_docs = (last_doc - doc0) / nw + 1;
  const long long nsteps = wave_docs * tpd;
  long long ld_k = 0;       // step of the next load
  int ld_t = 0;             // its tile within the document
  long long ld_j = 0;       // its document within the wave's sequence
  uint32_t idreg = 0;
  auto fill_ids = [&](long long j0) {
    const long long jj = j0 + lane;
    idreg = (dlist != nullptr && jj < wave_docs) ? dlist[doc0 + jj * nw] : 0u;
  };
  if (dlist != nullptr) fill_ids(0);
  long long ld_id = dlist != nullptr
                        ? (long long)__builtin_amdgcn_readfirstlane((int)idreg)
                        : a.doc_begin + doc0 * dstride;
  const long long id_step = nw * dstride;
  auto load_next = [&](Stage& st) {
    const long long tile = ld_id * tpd + ld_t;
    st.id = ld_id;
    load_tile_codes<NLOAD>(st.raw, packed, tile, lane);
    if constexpr (HI)
      st.nv = lane < 32 ? a.norms[tile * kTile + lane] : a.tile_cn[2 * tile + (lane & 1)];
    else
      st.nv = a.norms[tile * kTile + (lane & 31)];
    if (ld_k + 1 < nsteps) {
      ++ld_k;
      if (++ld_t == tpd) {
        ld_t = 0;
        ++ld_j;
        if (dlist != nullptr) {
          if ((ld_j & 63) == 0) fill_ids(ld_j);
          ld_id = (long long)(uint32_t)__builtin_amdgcn_readlane((int)idreg, (int)(ld_j & 63));
        } else {
          ld_id += id_step;
        }
      }
    }
  };
  long long doc = doc0;
  int t = 0;
  float mx[NQG];
  auto process = [&](const Stage& st) {
    if (t == 0) {
#pragma unroll
      for (int g = 0; g < NQG; ++g) mx[g] = -__builtin_inff();
    }
    int boff = lane;
    asm volatile("" : "+v"(boff));
    float lb[NQG];
    if constexpr (HI) {
      const float cn = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(st.nv), 32));
#pragma unroll
      for (int g = 0; g < NQG; ++g) lb[g] = (lo_r[g] * cn) * 1.0000002f;  // >= lonorm * cn
    }
    // Row r's norm sits at float r of the wave's slot; lane l needs rows
    // 8 i4 + 4 (l / 32) + {0..3}. LDS operations of one wave complete in
    // order, so no barrier is needed around the slot.
    if (lane < 32) reinterpret_cast<float*>(nstage[wave])[lane] = st.nv;
    __builtin_amdgcn_wave_barrier();
    float nrm[16];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const float4 v = nstage[wave][2 * i4 + half];
      nrm[4 * i4 + 0] = v.x;
      nrm[4 * i4 + 1] = v.y;
      nrm[4 * i4 + 2] = v.z;
      nrm[4 * i4 + 3] = v.w;
    }
    __builtin_amdgcn_wave_barrier();
    // The score's "+ 0.0f" (-0 -> +0) commutes with the maximum (fmaxf
    // treats the zeros as equal), so it is applied once to the token max.
    v16i acc[NCB];
    auto epi = [&](int g) {
      if constexpr (HI)
        maxsim_bound(mx[g], acc[g], lb[g], nrm);
      else
        maxsim_epilogue(mx[g], acc[2 * g], acc[2 * g + 1], al[g], nrm);
    };
    if constexpr (KS <= 8) {
      // Short K: every step's code fragment is decoded once up front, then
      // the query groups run one after another; group g's MFMAs are followed
      // by the epilogue of group g - 1, which does not depend on them (and
      // only two query fragments are live at a time).
      v4i af[KS];
#pragma unroll
      for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
        for (int h = 0; h < SPL; ++h) {
          const int s = c * SPL + h;
          if (s < KS) af[s] = decode_step<BITS>(st.raw[c], h, la);
        }
      }
#pragma unroll
      for (int g = 0; g <= NQG; ++g) {
        if (g < NQG) {
          if constexpr (HI) {
            acc[g] = v16i{0};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
              const v4i bh = sb[(s * NCBU + g) * 64 + boff];
              acc[g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[s], bh, acc[g], 0, 0, 0);
            }
          } else {
            acc[2 * g] = v16i{0};
            acc[2 * g + 1] = v16i{0};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
              const v4i bh = sb[(s * NCBU + 2 * g) * 64 + boff];
              const v4i bl = sb[(s * NCBU + 2 * g + 1) * 64 + boff];
              acc[2 * g] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[s], bh, acc[2 * g], 0, 0, 0);
              acc[2 * g + 1] =
                  __builtin_amdgcn_mfma_i32_32x32x32_i8(af[s], bl, acc[2 * g + 1], 0, 0, 0);
            }
          }
        }
        if (g > 0) epi(g - 1);
      }
    } else {
      // Long K: steps outer, each step's code fragment decoded once and its
      // query fragments read together before its MFMAs.
#pragma unroll
      for (int cb = 0; cb < NCBU; ++cb) acc[cb] = v16i{0};
#pragma unroll
      for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
        for (int h = 0; h < SPL; ++h) {
          const int s = c * SPL + h;
          if (s < KS) {
            v4i bf[NCBU];
#pragma unroll
            for (int cb = 0; cb < NCBU; ++cb) bf[cb] = sb[(s * NCBU + cb) * 64 + boff];
            const v4i af = decode_step<BITS>(st.raw[c], h, la);
#pragma unroll
            for (int cb = 0; cb < NCBU; ++cb)
              acc[cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[cb], acc[cb], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int g = 0; g < NQG; ++g) epi(g);
    }
    if (t == tpd - 1) {
      bool keep = false;
#pragma unroll
      for (int g = 0; g < NQG; ++g) {
        float m0, m1;
        ms_halves(mx[g], m0, m1);
        float v = fmaxf(m0, m1);  // token max over the document
        if constexpr (HI) v = (fmaxf(v, 0.0f) * al[g]) * 1.000001f;  // >= every exact token max
        v = ms_token_sum(v + 0.0f, lane);
        if constexpr (HI) {
          // tau <= 0 (or NaN) cannot prune: every document is listed.
          keep |= g < gl && (v >= ta_r[g] || !(ta_r[g] > 0.0f));
        } else if (dlist != nullptr) {
          if (lane == 0 && g < gl)
            a.cand[(size_t)(goff + g) * a.list_cap + doc] =
                v >= ta_r[g] ? rank_key(v, (uint32_t)st.id) : 0ull;
        } else {
          if (lane == 0 && g < gl) a.out[(size_t)(goff + g) * a.out_stride + doc] = v;
        }
      }
      if constexpr (HI) {
        if (lane == 0 && keep) {
          const uint32_t pos = atomicAdd(&a.list_count[blockIdx.y], 1u);
          if (pos < (uint32_t)a.list_cap)
            a.list[(size_t)blockIdx.y * a.list_cap + pos] = (uint32_t)st.id;
        }
      }
    }
    if (++t == tpd) {
      t = 0;
      doc += nw;
    }
  };
  // Ring of R register stages: R - 1 tiles in flight while one is
  // processed (a tile is 16 bytes of codes and one norm per lane, so one
  // tile ahead kept too few bytes in flight to cover the memory latency).
  // Phase p refills the stage processed in phase p - 1, then processes stage
  // p; the loop has a single exit at its end (exits between phases make the
  // compiler's wait analysis merge the phases at the loop head and wait for
  // the newest stage too).
  constexpr int R = maxsim_ring<HI>(NLOAD);
  Stage st[R];
#pragma unroll
  for (int p = 0; p < R - 1; ++p) load_next(st[p]);
  do {
#pragma unroll
    for (int p = 0; p < R; ++p) {
      load_next(st[(p + R - 1) % R]);
      if (doc <= last_doc) process(st[p]);
    }
  } while (doc <= last_doc);
}

}  // namespace

// A budget of three waves per SIMD (<= 168 VGPRs) keeps the accumulators in
// ordinary VGPRs (the epilogue reads them directly instead of copying each
// element out of the accumulation registers) and lets a third wave's VALU
// fill the gaps of the other two.
#define EOS_TQ_MAXSIM(BITS, KS, NQG)                                                        \
  extern "C" __global__ __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(3))) \
  void eos_tq_maxsim_b##BITS##_k##KS##_g##NQG(TqMaxsimArgs a) {                              \
    tq_maxsim_body<BITS, KS, NQG, false>(a);                                                \
  }                                                                                          \
  extern "C" __global__ __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(3))) \
  void eos_tq_maxsim_b##BITS##_k##KS##_g##NQG##_h(TqMaxsimArgs a) {                          \
    tq_maxsim_body<BITS, KS, NQG, true>(a);                                                 \
  }

EOS_TQ_MAXSIM(2, 1, 4)
EOS_TQ_MAXSIM(2, 2, 4)
EOS_TQ_MAXSIM(2, 4, 4)
EOS_TQ_MAXSIM(2, 8, 4)
EOS_TQ_MAXSIM(2, 12, 2)
EOS_TQ_MAXSIM(2, 16, 2)
EOS_TQ_MAXSIM(2, 24, 2)
EOS_TQ_MAXSIM(2, 32, 1)
EOS_TQ_MAXSIM(4, 1, 4)
EOS_TQ_MAXSIM(4, 2, 4)
EOS_TQ_MAXSIM(4, 4, 4)
EOS_TQ_MAXSIM(4, 8, 4)
EOS_TQ_MAXSIM(4, 12, 2)
EOS_TQ_MAXSIM(4, 16, 2)
EOS_TQ_MAXSIM(4, 24, 2)
EOS_TQ_MAXSIM(4, 32, 1)

// ------------------------------------------------------- parent aggregation

// One wavefront per (query, parent): each lane keeps the 5 best of the child
// scores it reads (sorted descending in registers, 8 loads in flight), then
// the wave pops the best min(top_n, count) values in descending order --
// the order aggregateMultiVectorParentScores sums the accumulator's list in
// (runtime/retrieval_multivector_turboquant.go:769-810) -- and forms the
// parent score in f64 with explicitly rounded operations.
extern "C" __global__ __launch_bounds__(256) void eos_tq_parent_agg(TqParentArgs a) {
  const int lane = threadIdx.x & 63;
  const long long p = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int q = blockIdx.y;
  if (p >= a.np || q >= a.qb) return;
  const long long c0 = a.off[p], c1 = a.off[p + 1];
  const long long cnt = c1 - c0;
  float* out = a.out + (size_t)q * a.np + p;
  if (cnt <= 0) {
    if (lane == 0) *out = -__builtin_inff();
    return;
  }
  const float* row = a.scores + (size_t)q * a.stride;
  float t[5];
#pragma unroll
  for (int i = 0; i < 5; ++i) t[i] = -__builtin_inff();
  constexpr int U = 8;
  for (long long base = c0 + lane; base < c1; base += 64LL * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long c = base + 64LL * u;
      v[u] = row[c < c1 ? c : c1 - 1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + 64LL * u < c1) {
        float x = v[u];
#pragma unroll
        for (int i = 0; i < 5; ++i) {
          const float hi = fmaxf(x, t[i]), lo = fminf(x, t[i]);
          t[i] = hi;
          x = lo;
        }
      }
    }
  }
  const int avail = (a.top_n <= 0 || (long long)a.top_n > cnt || a.top_n > 5)
                        ? (int)(cnt < 5 ? cnt : 5)
                        : a.top_n;
  double sum = 0.0;
  for (int r = 0; r < avail; ++r) {
    float m = t[0];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    const unsigned long long owners = __ballot(t[0] == m);
    if (lane == __builtin_ctzll(owners)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) t[i] = t[i + 1];
      t[4] = -__builtin_inff();
    }
    sum = __dadd_rn(sum, (double)m);
  }
  double sc = __ddiv_rn(sum, (double)avail);
  if (a.penalty != 0.0) sc = __dsub_rn(sc, __dmul_rn(a.penalty, a.l1p[p]));
  if (lane == 0) *out = (float)sc;
}

// One wavefront per (query, selected parent): argmax over its children,
// ties to the lower child index (the accumulator's best child, :769-776).
extern "C" __global__ __launch_bounds__(256) void eos_tq_parent_best(TqParentBestArgs a) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int q = blockIdx.y;
  if (i >= a.kk || q >= a.qb) return;
  const long long p = a.parents[(size_t)q * a.kk + i];
  const long long c0 = a.off[p], c1 = a.off[p + 1];
  const float* row = a.scores + (size_t)q * a.stride;
  float bv = -__builtin_inff();
  long long bi = c1;
  constexpr int U = 8;
  for (long long base = c0 + lane; base < c1; base += 64LL * U) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long c = base + 64LL * u;
      v[u] = row[c < c1 ? c : c1 - 1];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const long long c = base + 64LL * u;
      if (c < c1 && (v[u] > bv || (v[u] == bv && c < bi))) {
        bv = v[u];
        bi = c;
      }
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o);
    const long long oi = __shfl_xor(bi, o);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    a.best_child[(size_t)q * a.kk + i] = bi;
    a.best_score[(size_t)q * a.kk + i] = bv;
  }
}

// ------------------------------------------------- two-stage retrieval (f16)
// f32 -> half exactly as float32ToHalf (runtime/mll_export.go:1007-1041):
// ties round away from zero (bit 12 of the f32 mantissa, not to even), and a
// finite value at or above 2^16 with a nonzero mantissa keeps its top mantissa
// bits under the all-ones exponent (a NaN pattern).
__device__ inline unsigned short ref_f32_to_half(float v) {
  const unsigned bits = __float_as_uint(v);
  const unsigned sign = (bits >> 16) & 0x8000u;
  const int e = (int)((bits >> 23) & 0xffu) - 127 + 15;
  unsigned mant = bits & 0x7fffffu;
  if (e <= 0) {
    if (e < -10) return (unsigned short)sign;
    mant |= 0x800000u;
    const unsigned shift = (unsigned)(14 - e);
    unsigned half = mant >> shift;
    if ((mant >> (shift - 1)) & 1u) half++;
    return (unsigned short)(sign | half);
  }
  if (e >= 0x1f) return (unsigned short)(sign | 0x7c00u | (mant == 0 ? 0u : (mant >> 13)));
  unsigned hexp = (unsigned)e << 10, hmant = mant >> 13;
  if (mant & 0x1000u) {
    hmant++;
    if (hmant & 0x400u) {
      hmant = 0;
      hexp += 0x400u;
      if (hexp >= 0x7c00u) hexp = 0x7c00u;
    }
  }
  return (unsigned short)(sign | hexp | hmant);
}

// halfToFloat32 (runtime/weight_file.go:461-483); a subnormal half is m * 2^-24
// exactly.
__device__ inline float ref_half_to_f32(unsigned h) {
  const unsigned sign = (h & 0x8000u) << 16;
  const unsigned e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0) return __uint_as_float(sign | __float_as_uint((float)m * 5.9604644775390625e-8f));
  if (e == 31) return __uint_as_float(sign | 0x7f800000u | (m << 13));
  return __uint_as_float(sign | ((e + 112u) << 23) | (m << 13));
}

extern "C" __global__ __launch_bounds__(256) void eos_tq_f16_sidecar(TqHalfArgs a) {
  const long long stride = (long long)gridDim.x * blockDim.x;
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.count; i += stride)
    a.h[i] = ref_f32_to_half(a.x[i]);
}

constexpr int kRrThreads = 256;
constexpr int kRrMaxCand = 4096;
constexpr int kRrMaxDim = 4096;
constexpr int kRrMaxDqDim = 1024;  // reconstruct rerank: dimensions it dequantizes
constexpr int kRescueTopK = 100, kRescueLo = 100, kRescueHi = 120, kRescuePromote = 5;

// Order key of a score for a descending sort (-0 and +0 compare equal, as Go's
// float comparisons do).
__device__ inline unsigned rr_desc(float s) {
  unsigned u = __float_as_uint(s);
  if (u == 0x80000000u) u = 0;
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ~u;
}

// First rerank kernels, one wavefront per 64 candidates of a query (grid:
// candidate blocks x queries). The candidates' rows are staged through LDS
// 128 columns at a time with coalesced 16-byte loads (consecutive lanes read
// consecutive bytes of one row), then each lane sums its own candidate in
// index order, each product and sum rounded to f32 (no fused multiply-add):
//   f16 rows   scoreValue += query[i] * halfToFloat32(half)
//              (topFP16RerankScores, runtime/retrieval_turboquant.go:1646-1649)
//   f32 rows   sum += a[i] * b[i] (dotRetrievalVectors, runtime/retrieval_eval.go:
//              1189-1199, as topDenseRerankScores calls it, :1610-1633)
// halfToFloat32 is exact for every finite half and for the infinities, where
// it equals the hardware conversion; a NaN row element gives a NaN score
// either way (NaN payloads are outside the ranking contract). The f32 score
// of candidate j of query qi goes to a.dots[qi * c + j]; candidates whose id
// is outside [0, n) have no row and are left unscored (the sort kernel skips
// them).
constexpr int kRrCand = 64;
constexpr int kRrChunk = 128;

template <bool F32>
EOS_DEV void rr_dots_staged(const TqRerankArgs& a) {
#pragma clang fp contract(off)
  using Elem = typename std::conditional<F32, float, unsigned short>::type;
  constexpr int EPV = 16 / (int)sizeof(Elem);  // elements per 16-byte load
  constexpr int LD = kRrChunk + EPV;           // row pitch in LDS (one 16-byte pad)
  constexpr int CPR = kRrChunk / EPV;          // 16-byte loads per staged row
  __shared__ float qv[kRrMaxDim];
  __shared__ __attribute__((aligned(16))) Elem tile[kRrCand * LD];
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const int qi = blockIdx.y, lane = threadIdx.x;
  const int j = blockIdx.x * kRrCand + lane;
  for (int i = lane; i < a.d; i += kRrCand) qv[i] = a.queries[(size_t)qi * a.d + i];
  const long long myid = j < a.c ? a.cand_ids[(size_t)qi * a.c + j] : -1ll;
  const bool valid = myid >= 0 && myid < a.n;
  // Row of this candidate: its id, or its position (rows_by_pos); -1: none.
  const long long myrow = !valid ? -1ll : (a.rows_by_pos ? (long long)qi * a.c + j : myid);
  const Elem* rows = F32 ? reinterpret_cast<const Elem*>(a.rows_f32)
                         : reinterpret_cast<const Elem*>(a.rows);
  float s = 0.0f;
  for (int c0 = 0; c0 < a.d; c0 += kRrChunk) {
    const int cols = min(kRrChunk, a.d - c0);
    if (a.vec) {
      // d % EPV == 0 and 16-byte aligned rows: whole 16-byte loads.
      v4u buf[kRrCand * CPR / 64];
#pragma unroll
      for (int u = 0; u < kRrCand * CPR / 64; ++u) {
        const int t = lane + 64 * u, r = t / CPR, cc = t % CPR;
        const long long id = __shfl(myrow, r);
        buf[u] = (id >= 0 && cc * EPV < cols)
                     ? __builtin_nontemporal_load(reinterpret_cast<const v4u*>(
                           rows + (size_t)id * a.d + c0 + cc * EPV))
                     : v4u{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < kRrCand * CPR / 64; ++u) {
        const int t = lane + 64 * u, r = t / CPR, cc = t % CPR;
        *reinterpret_cast<v4u*>(&tile[r * LD + cc * EPV]) = buf[u];
      }
    } else {
      for (int t = lane; t < kRrCand * kRrChunk; t += 64) {
        const int r = t / kRrChunk, cc = t % kRrChunk;
        const long long id = __shfl(myrow, r);
        tile[r * LD + cc] = (id >= 0 && cc < cols) ? rows[(size_t)id * a.d + c0 + cc] : (Elem)0;
      }
    }
    __syncthreads();
    if (valid) {
      const Elem* row = &tile[lane * LD];
      for (int i = 0; i < cols; ++i) {
        float x;
        if constexpr (F32) {
          x = row[i];
        } else {
          x = (float)__builtin_bit_cast(_Float16, row[i]);
        }
        const float p = qv[c0 + i] * x;
        s = s + p;
      }
    }
    __syncthreads();
  }
  if (valid) a.dots[(size_t)qi * a.c + j] = s;
}

extern "C" __global__ __launch_bounds__(64) void eos_tq_rr_dots(TqRerankArgs a) {
  rr_dots_staged<false>(a);
}
extern "C" __global__ __launch_bounds__(64) void eos_tq_rr_dots_f32(TqRerankArgs a) {
  rr_dots_staged<true>(a);
}

// Reconstruct rerank (topTurboQuantReconstructRerankScores and, on a sidecar
// code set, topTurboQuantMixedWidthRerankScores, runtime/retrieval_turboquant.
// go:1788-1846): the reference scores dotRetrievalVectors(query,
// q.Dequantize(codes)). The dequantizer is in the un-vendored quantizer
// module; this build's contract follows the published TurboQuant dequantizers
// in f64 with one rounding per coordinate:
//   y_j = (double)codebook[code_j]
//         (+ coef * z_j for an inner-product set: z_j = sum over i ascending of
//          (bit_i ? S[i][j] : -S[i][j]), coef = (sqrt(pi/2) / d) * ResNorm)
//   x_k = (float)(Norm * acc_k), acc_k = fma chain over j ascending of
//         R[j][k] * y_j (identity: y_k)
// eos_tq_rr_dequant writes x for 8 candidates per workgroup into xhat; the
// f32 index-order dots (eos_tq_rr_dots_f32 over rows by position) follow.
// Codes are the reference row layout: code j at bits j*bits .. + bits - 1,
// low bits first (3-bit codes may straddle two bytes).
constexpr int kRrDqCand = 8;

EOS_DEV int rr_code_at(const unsigned char* row, int j, int bits) {
  const int bit = j * bits, byte = bit >> 3, sh = bit & 7;
  unsigned v = (unsigned)row[byte] >> sh;
  if (sh + bits > 8) v |= (unsigned)row[byte + 1] << (8 - sh);
  return (int)(v & ((1u << bits) - 1u));
}

extern "C" __global__ __launch_bounds__(256) void eos_tq_rr_dequant(TqReconArgs a) {
  __shared__ double y[kRrDqCand][kRrMaxDqDim];
  __shared__ unsigned char sg[kRrDqCand][kRrMaxDqDim / 8];
  __shared__ long long ids[kRrDqCand];
  __shared__ double coef[kRrDqCand];
  const int qi = blockIdx.y, tid = threadIdx.x;
  const int j0 = blockIdx.x * kRrDqCand;
  if (tid < kRrDqCand) {
    const int j = j0 + tid;
    const long long id = j < a.c ? a.cand_ids[(size_t)qi * a.c + j] : -1ll;
    ids[tid] = (id >= 0 && id < a.n) ? id : -1ll;
    coef[tid] = (a.signs != nullptr && ids[tid] >= 0)
                    ? __dmul_rn(__ddiv_rn(1.2533141373155003, (double)a.d),
                                (double)a.resnorms[ids[tid]])
                    : 0.0;
  }
  __syncthreads();
  // y = codebook values of each candidate's codes (zeros for no candidate).
  for (int t = tid; t < kRrDqCand * a.d; t += 256) {
    const int cc = t / a.d, j = t % a.d;
    const long long id = ids[cc];
    y[cc][j] = id >= 0 ? (double)a.codebook[rr_code_at(a.codes + (size_t)id * a.row_bytes, j, a.bits)]
                       : 0.0;
  }
  if (a.signs != nullptr) {
    const int sb = (a.d + 7) / 8;
    for (int t = tid; t < kRrDqCand * sb; t += 256) {
      const int cc = t / sb, b = t % sb;
      sg[cc][b] = ids[cc] >= 0 ? a.signs[(size_t)ids[cc] * sb + b] : (unsigned char)0;
    }
    __syncthreads();
    // z_j = S^T sign: thread j streams row j of qjl_t (S[i][j], i ascending).
    for (int j = tid; j < a.d; j += 256) {
      const float* srow = a.qjl_t + (size_t)j * a.d;
      double z[kRrDqCand];
#pragma unroll
      for (int cc = 0; cc < kRrDqCand; ++cc) z[cc] = 0.0;
      for (int i = 0; i < a.d; ++i) {
        const double v = (double)srow[i];
#pragma unroll
        for (int cc = 0; cc < kRrDqCand; ++cc)
          z[cc] = ((sg[cc][i >> 3] >> (i & 7)) & 1) ? __dadd_rn(z[cc], v) : __dsub_rn(z[cc], v);
      }
#pragma unroll
      for (int cc = 0; cc < kRrDqCand; ++cc) y[cc][j] = __dadd_rn(y[cc][j], __dmul_rn(coef[cc], z[cc]));
    }
  }
  __syncthreads();
  // x_k = Norm * (R^T y)_k: thread k streams row k of rot_t (R[j][k], j ascending).
  for (int k = tid; k < a.d; k += 256) {
    double acc[kRrDqCand];
#pragma unroll
    for (int cc = 0; cc < kRrDqCand; ++cc) acc[cc] = a.rot_t != nullptr ? 0.0 : y[cc][k];
    if (a.rot_t != nullptr) {
      const float* rrow = a.rot_t + (size_t)k * a.d;
      for (int j = 0; j < a.d; ++j) {
        const double r = (double)rrow[j];
#pragma unroll
        for (int cc = 0; cc < kRrDqCand; ++cc) acc[cc] = __fma_rn(r, y[cc][j], acc[cc]);
      }
    }
#pragma unroll
    for (int cc = 0; cc < kRrDqCand; ++cc) {
      const long long id = ids[cc];
      if (id >= 0)
        a.xhat[((size_t)qi * a.c + j0 + cc) * a.d + k] =
            __double2float_rn(__dmul_rn((double)a.norms[id], acc[cc]));
    }
  }
}

// Second rerank kernel, one workgroup per query: sorts the candidates in LDS by
// (score desc, id asc) -- the heap + insertion sort of topFP16RerankScores
// (runtime/retrieval_turboquant.go:1635-1662) -- or, with rescue, by (score
// desc, first-stage rank asc) (sortTurboQuantFP16RankedScores, :1698-1719;
// ranks are distinct, so its id tie-break never decides) and then applies
// applyTurboQuantFP16RerankRescue (:1721-1786). Candidates whose id is outside
// [0, n) have no row and are skipped (`if !ok { continue }`).
extern "C" __global__ __launch_bounds__(kRrThreads) void eos_tq_rr_sort(TqRerankArgs a) {
  __shared__ unsigned long long key[kRrMaxCand];
  __shared__ int pos[kRrMaxCand];
  __shared__ int outpos[kRrMaxCand];
  __shared__ unsigned char seen[kRrMaxCand];
  __shared__ unsigned long long pool_key[kRescueHi - kRescueLo + 1];
  __shared__ int valid_n;
  const int qi = blockIdx.x, tid = threadIdx.x;
  const long long* cid = a.cand_ids + (size_t)qi * a.c;
  const float* fscore = a.dots + (size_t)qi * a.c;
  if (tid == 0) valid_n = 0;
  int P = 1;
  while (P < a.c) P <<= 1;
  __syncthreads();
  int my_valid = 0;
  for (int j = tid; j < P; j += kRrThreads) {
    unsigned long long k = ~0ull;
    if (j < a.c) {
      const long long id = cid[j];
      seen[j] = 0;
      if (id >= 0 && id < a.n) {
        const float s = fscore[j];
        const unsigned tie = a.rescue            ? (unsigned)(j + 1)
                             : a.id_rank != nullptr ? (unsigned)a.id_rank[id]
                                                    : (unsigned)id;
        k = ((unsigned long long)rr_desc(s) << 32) | tie;
        ++my_valid;
      }
    }
    key[j] = k;
    pos[j] = j;
  }
  if (my_valid) atomicAdd(&valid_n, my_valid);
  for (int size = 2; size <= P; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      __syncthreads();
      for (int t = tid; t < (P >> 1); t += kRrThreads) {
        const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
        const bool asc = (lo & size) == 0;
        const unsigned long long kl = key[lo], kh = key[hi];
        if ((kl > kh) == asc) {
          key[lo] = kh;
          key[hi] = kl;
          const int pl = pos[lo];
          pos[lo] = pos[hi];
          pos[hi] = pl;
        }
      }
    }
  }
  __syncthreads();
  const int m = valid_n;
  const int nout = a.kk < m ? a.kk : m;
  if (a.rescue && m >= kRescueHi && m > kRescueTopK) {
    // The pool is ranks kRescueLo..kRescueHi (1-based), so ranks below
    // kRescueLo are never promoted and keep their places.
    constexpr int pool = kRescueHi - kRescueLo + 1;
    if (tid < pool) {
      const int p = pos[kRescueLo - 1 + tid];
      pool_key[tid] = ((unsigned long long)rr_desc(a.cand_scores[(size_t)qi * a.c + p]) << 32) |
                      (unsigned)(p + 1);
    }
    for (int i = tid; i < kRescueLo - 1 && i < nout; i += kRrThreads) {
      outpos[i] = pos[i];
      seen[pos[i]] = 1;
    }
    __syncthreads();
    if (tid == 0) {
      // Pool order: first-stage score desc, first-stage rank asc; the first
      // kRescuePromote are promoted.
      int promoted[kRescuePromote];
      unsigned long long taken = 0;
      for (int r = 0; r < kRescuePromote; ++r) {
        int best = -1;
        unsigned long long bk = ~0ull;
        for (int i = 0; i < pool; ++i) {
          if (taken >> i & 1ull) continue;
          const unsigned long long ck = pool_key[i];
          if (best < 0 || ck < bk) { best = i; bk = ck; }
        }
        taken |= 1ull << best;
        promoted[r] = pos[kRescueLo - 1 + best];
      }
      int o = nout < kRescueLo - 1 ? nout : kRescueLo - 1;
      for (int i = kRescueLo - 1; i < kRescueTopK && o < nout; ++i) {
        const int p = pos[i];
        bool pr = false;
        for (int r = 0; r < kRescuePromote; ++r) pr |= promoted[r] == p;
        if (pr) continue;
        outpos[o++] = p;
        seen[p] = 1;
      }
      for (int r = 0; r < kRescuePromote && o < nout; ++r) {
        if (seen[promoted[r]]) continue;
        outpos[o++] = promoted[r];
        seen[promoted[r]] = 1;
      }
      for (int i = kRescueLo - 1; i < m && o < nout; ++i) {
        if (seen[pos[i]]) continue;
        outpos[o++] = pos[i];
        seen[pos[i]] = 1;
      }
    }
  } else {
    for (int i = tid; i < nout; i += kRrThreads) outpos[i] = pos[i];
  }
  __syncthreads();
  for (int i = tid; i < a.kk; i += kRrThreads) {
    long long id = -1;
    float s = 0.0f;
    if (i < nout) {
      const int p = outpos[i];
      id = cid[p];
      s = fscore[p];
    }
    a.out_ids[(size_t)qi * a.kk + i] = id;
    a.out_scores[(size_t)qi * a.kk + i] = s;
  }
}
