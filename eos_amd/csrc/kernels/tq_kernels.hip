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

#include "tq_args.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef unsigned long long u64;

#define EOS_DEV __device__ __forceinline__

namespace {

constexpr int kTile = 32;        // corpus vectors per MFMA row block
constexpr int kScanThreads = 256;

EOS_DEV uint32_t score_key(float s) {
  uint32_t u = __float_as_uint(s);
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

}  // namespace

// ------------------------------------------------------------------ prepare


// One workgroup per query column (padded to a multiple of 32 queries).
extern "C" __global__ __launch_bounds__(256) void eos_tq_prepare(TqPrepArgs a) {
  __shared__ double sq[2048];
  __shared__ double red[256];
  const int qi = blockIdx.x;
  const int tid = threadIdx.x;
  const bool live = qi < a.q;
  const int dpad = a.ks * 32;
  for (int j = tid; j < a.d; j += 256) sq[j] = live ? (double)a.queries[(size_t)qi * a.d + j] : 0.0;
  __syncthreads();
  double qr[8];
  double mx = 0.0;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int j = tid + 256 * r;
    double acc = 0.0;
    if (j < a.d) {
      if (a.rot_t != nullptr) {
        for (int k = 0; k < a.d; ++k) acc = fma((double)a.rot_t[(size_t)k * a.d + j], sq[k], acc);
      } else {
        acc = sq[j];
      }
    }
    qr[r] = acc;
    mx = fmax(mx, fabs(acc));
  }
  red[tid] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (tid < s) red[tid] = fmax(red[tid], red[tid + s]);
    __syncthreads();
  }
  const double maxabs = red[0];
  const double inv = maxabs > 0.0 ? (double)a.qmax / maxabs : 0.0;
  const int cb_hi = 2 * (qi >> 5);
  const int col = qi & 31;
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const int j = tid + 256 * r;
    if (j >= dpad) continue;
    int qs = 0;
    if (j < a.d) {
      double v = rint(qr[r] * inv);
      v = fmin(fmax(v, (double)-a.qmax), (double)a.qmax);
      qs = (int)v;
      if (live && a.qs_out != nullptr) a.qs_out[(size_t)qi * a.d + j] = (int16_t)qs;
    }
    const int lo = ((qs + 128) & 255) - 128;
    const int hi = (qs - lo) >> 8;
    const int s = j >> 5, g = (j >> 4) & 1, i = j & 15;
    const int lane = col + 32 * g;
    a.bfrag[((size_t)(s * a.ncb + cb_hi) * 64 + lane) * 16 + i] = (int8_t)hi;
    a.bfrag[((size_t)(s * a.ncb + cb_hi + 1) * 64 + lane) * 16 + i] = (int8_t)lo;
  }
  if (tid == 0) {
    a.alpha[qi] = maxabs > 0.0 ? (float)((maxabs / (double)a.qmax) * (double)a.cb_scale) : 0.0f;
    a.tau[qi] = -__builtin_inff();
    a.cand_count[qi] = 0u;
  }
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

template <int BITS, int KS, int NQG>
EOS_DEV void tq_scan_body(const TqScanArgs& a) {
  constexpr int NCB = 2 * NQG;
  constexpr int SPL = 8 / BITS;
  constexpr int NLOAD = (KS + SPL - 1) / SPL;
  __shared__ v4i sb[KS * NCB * 64];
  {
    const v4i* src = reinterpret_cast<const v4i*>(a.bfrag);
    for (int i = threadIdx.x; i < KS * NCB * 64; i += kScanThreads) sb[i] = src[i];
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = gridDim.x * (kScanThreads / 64);
  const int half = lane >> 5;
  for (int j = blockIdx.x * (kScanThreads / 64) + wave; j < a.ntiles; j += nw) {
    const long long tile = a.tile_begin + (long long)j * a.tile_step;
    const v4i* src = reinterpret_cast<const v4i*>(a.packed) + (size_t)tile * NLOAD * 64 + lane;
    v4i raw[NLOAD];
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) raw[c] = __builtin_nontemporal_load(src + c * 64);
    v16i acc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[cb] = v16i{0};
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
      for (int h = 0; h < SPL; ++h) {
        const int s = c * SPL + h;
        if (s < KS) {
          const v4i af = decode_step<BITS>(raw[c], h, a);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            const v4i bf = sb[(s * NCB + cb) * 64 + lane];
            acc[cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, acc[cb], 0, 0, 0);
          }
        }
      }
    }
    // Epilogue. Accumulator element i of lane l is row 8(i/4) + 4(l/32) + i%4
    // (a corpus vector of the tile) and column l%32 (a query of the group).
    const long long vbase = tile * kTile;
    float nrm[16];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      const float4 n4 = *reinterpret_cast<const float4*>(a.norms + vbase + 8 * i4 + 4 * half);
      nrm[4 * i4 + 0] = n4.x;
      nrm[4 * i4 + 1] = n4.y;
      nrm[4 * i4 + 2] = n4.z;
      nrm[4 * i4 + 3] = n4.w;
    }
#pragma unroll
    for (int g = 0; g < NQG; ++g) {
      const int qi = g * 32 + (lane & 31);
      if (qi >= a.q) continue;
      const float al = a.alpha[qi];
      const float ta = a.mode == 1 ? a.tau[qi] : 0.0f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int r = 8 * (i >> 2) + 4 * half + (i & 3);
        const long long v = vbase + r;
        const int dot = acc[2 * g][i] * 256 + acc[2 * g + 1][i];
        const float score = ((float)dot * al) * nrm[i] + 0.0f;
        if (a.mode == 1) {
          if (v < a.n && score >= ta) {
            const uint32_t pos = atomicAdd(&a.cand_count[qi], 1u);
            if ((int)pos < a.cap) a.cand[(size_t)qi * a.cap + pos] = rank_key(score, (uint32_t)v);
          }
        } else if (a.mode == 0) {
          const long long colx = v - a.out_begin;
          if (v < a.n && colx >= 0 && colx < a.out_count) {
            a.out_scores[(size_t)qi * a.out_stride + colx] = score;
            if (a.out_dots != nullptr) a.out_dots[(size_t)qi * a.out_stride + colx] = dot;
          }
        } else {
          const long long colx = (long long)j * kTile + r;
          a.out_scores[(size_t)qi * a.out_stride + colx] = v < a.n ? score : -__builtin_inff();
        }
      }
    }
  }
}

}  // namespace

#define EOS_TQ_SCAN(BITS, KS, NQG)                                                        \
  extern "C" __global__ __launch_bounds__(kScanThreads) void eos_tq_scan_b##BITS##_k##KS##_g##NQG( \
      TqScanArgs a) {                                                                     \
    tq_scan_body<BITS, KS, NQG>(a);                                                       \
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
// composite rank key (8 passes of 8-bit digits; keys are unique, so exactly
// kk elements are >= the selected key). One workgroup per row.
extern "C" __global__ __launch_bounds__(kSelThreads) void eos_tq_row_select(TqSelectArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ u64 sel_prefix;
  __shared__ int sel_rem;
  __shared__ int list_n;
  __shared__ u64 list[kSortCap];
  const int row = blockIdx.x;
  if (row >= a.nrows) return;
  if (a.mode == 1 && a.status != nullptr && a.status[row] == 0) return;
  const float* x = a.rows + (size_t)row * a.stride;
  const int tid = threadIdx.x;
  if (a.kk <= 0 || a.n <= 0) return;
  if (a.mode == 0 && (long long)a.kk > a.n) {
    if (tid == 0) a.tau[row] = -__builtin_inff();
    return;
  }
  const int passes = a.mode == 0 ? 4 : 8;
  if (tid == 0) {
    sel_prefix = 0ull;
    sel_rem = a.kk;
  }
  for (int p = 0; p < passes; ++p) {
    const int shift = 56 - 8 * p;
    for (int b = tid; b < 256; b += kSelThreads) hist[b] = 0u;
    __syncthreads();
    const u64 pfx = sel_prefix;
    const u64 hmask = p == 0 ? 0ull : ~((1ull << (shift + 8)) - 1ull);
    for (long long i = tid; i < a.n; i += kSelThreads) {
      const u64 c = rank_key(x[i], (uint32_t)i);
      if (((c ^ pfx) & hmask) == 0ull) atomicAdd(&hist[(c >> shift) & 255u], 1u);
    }
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
    }
    __syncthreads();
  }
  const u64 thr = sel_prefix;
  if (a.mode == 0) {
    if (tid == 0) a.tau[row] = key_score((uint32_t)(thr >> 32));
    return;
  }
  // mode 1: gather the kk elements >= thr and sort them.
  int npow = 1;
  while (npow < a.kk) npow <<= 1;
  if (tid == 0) list_n = 0;
  for (int i = tid; i < npow; i += kSelThreads) list[i] = 0ull;
  __syncthreads();
  for (long long i = tid; i < a.n; i += kSelThreads) {
    const u64 c = rank_key(x[i], (uint32_t)i);
    if (c >= thr) {
      const int pos = atomicAdd(&list_n, 1);
      if (pos < kSortCap) list[pos] = c;
    }
  }
  __syncthreads();
  bitonic_sort_desc(list, npow);
  for (int i = tid; i < a.kk; i += kSelThreads) {
    const u64 c = list[i];
    a.ids[(size_t)row * a.kk + i] = (long long)rank_id(c);
    a.scores[(size_t)row * a.kk + i] = key_score((uint32_t)(c >> 32));
  }
}

// --------------------------------------------------------------- finalize


// Sorts each query's filtered candidates (score desc, id asc) and emits the
// first kk. A query whose candidate set cannot be proven to hold its top-kk is
// flagged for the exhaustive path.
extern "C" __global__ __launch_bounds__(kSelThreads) void eos_tq_finalize(TqFinalizeArgs a) {
  __shared__ u64 list[kSortCap];
  const int row = blockIdx.x;
  if (row >= a.q) return;
  const uint32_t cnt = a.cand_count[row];
  if (cnt > (uint32_t)a.cap || cnt > (uint32_t)kSortCap) {
    if (threadIdx.x == 0) a.status[row] = 2;
    return;
  }
  if (cnt < (uint32_t)a.kk) {
    if (threadIdx.x == 0) a.status[row] = 1;
    return;
  }
  int npow = 1;
  while (npow < (int)cnt) npow <<= 1;
  for (int i = threadIdx.x; i < npow; i += blockDim.x)
    list[i] = i < (int)cnt ? a.cand[(size_t)row * a.cap + i] : 0ull;
  __syncthreads();
  bitonic_sort_desc(list, npow);
  for (int i = threadIdx.x; i < a.kk; i += blockDim.x) {
    const u64 c = list[i];
    a.ids[(size_t)row * a.kk + i] = (long long)rank_id(c);
    a.scores[(size_t)row * a.kk + i] = key_score((uint32_t)(c >> 32));
  }
  if (threadIdx.x == 0) a.status[row] = 0;
}
