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

namespace {
constexpr int kRotJ = 64;    // rotated coordinates per workgroup
constexpr int kRotQ = 4;     // queries per workgroup
constexpr int kRotK = 128;   // rotation rows staged per LDS chunk
constexpr int kMaxDim = 1024;
}  // namespace

// q'[q][j] = sum_k R[j][k] q[k] in f64: one fma chain per (q, j), k ascending.
// Workgroup (x, y) computes j in [64x, 64x + 64) for queries [4y, 4y + 4);
// R^T streams through LDS 128 rows of k at a time (all loads of a chunk are
// issued before any is consumed).
extern "C" __global__ __launch_bounds__(256) void eos_tq_rotate(TqPrepArgs a) {
  __shared__ float rs[kRotK * kRotJ];
  __shared__ double qsh[kRotQ * kMaxDim];
  const int tid = threadIdx.x;
  const int j0 = blockIdx.x * kRotJ, q0 = blockIdx.y * kRotQ;
  const int jj = tid & 63, ql = tid >> 6;
  for (int i = tid; i < kRotQ * a.d; i += 256) {
    const int qq = i / a.d, k = i - qq * a.d;
    const int qi = q0 + qq;
    qsh[qq * kMaxDim + k] = qi < a.q ? (double)a.queries[(size_t)qi * a.d + k] : 0.0;
  }
  double acc = 0.0;
  for (int k0 = 0; k0 < a.d; k0 += kRotK) {
    const int kn = min(kRotK, a.d - k0);
    float tmp[kRotK * kRotJ / 256];
#pragma unroll
    for (int r = 0; r < kRotK * kRotJ / 256; ++r) {
      const int i = tid + 256 * r;
      const int kk = i >> 6, jc = i & 63;
      tmp[r] = (kk < kn && j0 + jc < a.d) ? a.rot_t[(size_t)(k0 + kk) * a.d + j0 + jc] : 0.0f;
    }
    __syncthreads();  // previous chunk consumed; qsh visible
#pragma unroll
    for (int r = 0; r < kRotK * kRotJ / 256; ++r) rs[tid + 256 * r] = tmp[r];
    __syncthreads();
    if (kn == kRotK) {
#pragma unroll 16
      for (int kk = 0; kk < kRotK; ++kk)
        acc = fma((double)rs[kk * kRotJ + jj], qsh[ql * kMaxDim + k0 + kk], acc);
    } else {
      for (int kk = 0; kk < kn; ++kk)
        acc = fma((double)rs[kk * kRotJ + jj], qsh[ql * kMaxDim + k0 + kk], acc);
    }
  }
  const int j = j0 + jj, qi = q0 + ql;
  if (j < a.d && qi < a.q) a.qrot[(size_t)qi * a.d + j] = acc;
}

// One workgroup per query column (padded to a multiple of 32 queries):
// max |q'|, int16 rounding, hi/lo fragments, alpha; resets the query's
// threshold and candidate count for the scan that follows.
extern "C" __global__ __launch_bounds__(256) void eos_tq_quantize(TqPrepArgs a) {
  __shared__ double red[256];
  const int qi = blockIdx.x;  // column
  const int tid = threadIdx.x;
  const int grp = qi / a.group, slot = qi - grp * a.group;
  const int src = grp * a.group_live + slot;  // source row
  const bool live = src < a.q && slot < a.group_live;
  const int dpad = a.ks * 32;
  double qr[kMaxDim / 256];
  double mx = 0.0;
#pragma unroll
  for (int r = 0; r < kMaxDim / 256; ++r) {
    const int j = tid + 256 * r;
    double v = 0.0;
    if (live && j < a.d)
      v = a.rot_t != nullptr ? a.qrot[(size_t)src * a.d + j] : (double)a.queries[(size_t)src * a.d + j];
    qr[r] = v;
    mx = fmax(mx, fabs(v));
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
  for (int r = 0; r < kMaxDim / 256; ++r) {
    const int j = tid + 256 * r;
    if (j >= dpad) continue;
    int qs = 0;
    if (j < a.d) {
      double v = rint(qr[r] * inv);
      v = fmin(fmax(v, (double)-a.qmax), (double)a.qmax);
      qs = (int)v;
      if (live && a.qs_out != nullptr) a.qs_out[(size_t)src * a.d + j] = (int16_t)qs;
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

// Per-workgroup candidate stage of the filter scan: kept rank keys are
// appended with LDS atomics and flushed to the global list once per query at
// the end, so the scan never waits on a global atomic.
constexpr int kLdsSlots = 16;

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
template <int BITS, int KS, int NQG, bool FILTER>
EOS_DEV void tq_scan_body(const TqScanArgs& a) {
  constexpr int NCB = 2 * NQG;
  constexpr int SPL = 8 / BITS;
  constexpr int NLOAD = (KS + SPL - 1) / SPL;
  constexpr int NQ = 32 * NQG;
  __shared__ v4i sb[KS * NCB * 64];
  __shared__ uint32_t lc_cnt[FILTER ? NQ : 1];
  __shared__ u64 lc_buf[FILTER ? NQ * kLdsSlots : 1];
  if (a.gate != nullptr) {
    // Exhaustive pass of the exact fallback: run only when a query was flagged.
    bool any = false;
    for (int i = 0; i < a.q; ++i) any |= a.gate[i] != 0;
    if (!any) return;
  }
  {
    const v4i* src = reinterpret_cast<const v4i*>(a.bfrag);
    for (int i = threadIdx.x; i < KS * NCB * 64; i += kScanThreads) sb[i] = src[i];
    if (FILTER && threadIdx.x < NQ) lc_cnt[threadIdx.x] = 0u;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nw = gridDim.x * (kScanThreads / 64);
  const int half = lane >> 5;
  const v4i* packed = reinterpret_cast<const v4i*>(a.packed);
  // Software pipeline: codes are in flight two tiles ahead and norms one tile
  // ahead of the tile being decoded, multiplied and filtered.
  int j = blockIdx.x * (kScanThreads / 64) + wave;
  v4i raw0[NLOAD], raw1[NLOAD];
  float4 nrm0[4];
  if (j < a.ntiles) {
    const long long t0 = a.tile_begin + (long long)j * a.tile_step;
    load_tile_codes<NLOAD>(raw0, packed, t0, lane);
    load_tile_norms(nrm0, a.norms, t0, half);
  }
  if (j + nw < a.ntiles) load_tile_codes<NLOAD>(raw1, packed, a.tile_begin + (long long)(j + nw) * a.tile_step, lane);
  for (; j < a.ntiles; j += nw) {
    const long long tile = a.tile_begin + (long long)j * a.tile_step;
    v4i raw2[NLOAD];
    float4 nrm1[4];
    if (j + 2 * nw < a.ntiles)
      load_tile_codes<NLOAD>(raw2, packed, a.tile_begin + (long long)(j + 2 * nw) * a.tile_step, lane);
    if (j + nw < a.ntiles)
      load_tile_norms(nrm1, a.norms, a.tile_begin + (long long)(j + nw) * a.tile_step, half);
    // Opaque per-tile LDS offset: keeps the query fragments in LDS rather than
    // letting them be hoisted into registers across the tile loop.
    int boff = lane;
    asm volatile("" : "+v"(boff));
    v16i acc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[cb] = v16i{0};
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
      for (int h = 0; h < SPL; ++h) {
        const int s = c * SPL + h;
        if (s < KS) {
          const v4i af = decode_step<BITS>(raw0[c], h, a);
#pragma unroll
          for (int cb = 0; cb < NCB; ++cb) {
            const v4i bf = sb[(s * NCB + cb) * 64 + boff];
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
      nrm[4 * i4 + 0] = nrm0[i4].x;
      nrm[4 * i4 + 1] = nrm0[i4].y;
      nrm[4 * i4 + 2] = nrm0[i4].z;
      nrm[4 * i4 + 3] = nrm0[i4].w;
    }
    // Rows of this tile that are real vectors (the last tile may be partial).
    const long long rem64 = a.n - vbase;
    const int rem = rem64 >= kTile ? kTile : (int)rem64;
#pragma unroll
    for (int g = 0; g < NQG; ++g) {
      const int qi = g * 32 + (lane & 31);
      const bool live = qi < a.q;
      const float al = live ? a.alpha[qi] : 0.0f;
      float sc[16];
      int dots[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        dots[i] = acc[2 * g][i] * 256 + acc[2 * g + 1][i];
        sc[i] = ((float)dots[i] * al) * nrm[i] + 0.0f;
      }
      if constexpr (FILTER) {
        const float ta = live ? a.tau[qi] : __builtin_inff();
        bool hit = false;
#pragma unroll
        for (int i = 0; i < 16; ++i) hit |= sc[i] >= ta;
        if (hit) {
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
#pragma unroll
    for (int c = 0; c < NLOAD; ++c) {
      raw0[c] = raw1[c];
      raw1[c] = raw2[c];
    }
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) nrm0[i4] = nrm1[i4];
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
  extern "C" __global__ __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) \
  void eos_tq_scan_b##BITS##_k##KS##_g##NQG##_f(TqScanArgs a) {                           \
    tq_scan_body<BITS, KS, NQG, true>(a);                                                 \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(kScanThreads) __attribute__((amdgpu_waves_per_eu(2, 8))) \
  void eos_tq_scan_b##BITS##_k##KS##_g##NQG##_w(TqScanArgs a) {                           \
    tq_scan_body<BITS, KS, NQG, false>(a);                                                \
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

// --------------------------------------------------------------- threshold

namespace {

constexpr int kThrPer = 16;            // tile maxima held per lane (<= 1024 per row)
constexpr int kFinThreads = 256;
constexpr int kFinPer = kSortCap / kFinThreads;

// Block-wide sum of per-wave counts (each wave passes a uniform value). The
// two slot sets alternate, so one barrier per call suffices: a set is
// rewritten only after a later barrier that every reader of it has passed.
template <int NT>
EOS_DEV uint32_t block_sum(uint32_t wave_count, uint32_t* slots, int& parity) {
  uint32_t* set = slots + parity * (NT / 64);
  if ((threadIdx.x & 63) == 0) set[threadIdx.x >> 6] = wave_count;
  __syncthreads();
  uint32_t t = 0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) t += set[i];
  parity ^= 1;
  return t;
}

EOS_DEV void wave_minmax(uint32_t& vmin, uint32_t& vmax) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    vmin = min(vmin, (uint32_t)__shfl_xor((int)vmin, o));
    vmax = max(vmax, (uint32_t)__shfl_xor((int)vmax, o));
  }
}

// Block-wide min and max of per-thread values.
template <int NT>
EOS_DEV void block_minmax(uint32_t& vmin, uint32_t& vmax, uint32_t* smin, uint32_t* smax) {
  wave_minmax(vmin, vmax);
  if ((threadIdx.x & 63) == 0) {
    smin[threadIdx.x >> 6] = vmin;
    smax[threadIdx.x >> 6] = vmax;
  }
  __syncthreads();
  vmin = 0xffffffffu;
  vmax = 0u;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    vmin = min(vmin, smin[i]);
    vmax = max(vmax, smax[i]);
  }
  __syncthreads();
}

}  // namespace

// Per query: tau = the r-th best of the sampled tiles' best scores, by
// bisection on the order-preserving key (one wavefront per query, the row in
// registers, counts by ballots; no barriers). The r-th best tile maximum is
// <= the r-th best sampled score, and any tau <= the true k-th best score is
// valid: the finalize kernel proves the kept set after the fact.
extern "C" __global__ __launch_bounds__(64) void eos_tq_threshold(TqSelectArgs a) {
  const int row = blockIdx.x;
  if (row >= a.nrows) return;
  const int lane = threadIdx.x;
  if ((long long)a.kk > a.n || a.kk <= 0 || a.n > 64LL * kThrPer) {
    if (lane == 0) a.tau[row] = -__builtin_inff();
    return;
  }
  const float* x = a.rows + (size_t)row * a.stride;
  uint32_t key[kThrPer];
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int v = 0; v < kThrPer; ++v) {
    const long long i = lane + 64LL * v;
    key[v] = i < a.n ? score_key(x[i]) : 0u;
    if (i < a.n) {
      kmin = min(kmin, key[v]);
      kmax = max(kmax, key[v]);
    }
  }
  wave_minmax(kmin, kmax);
  uint32_t lo = kmin, hi = kmax;
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1) + 1u;
    uint32_t c = 0;
#pragma unroll
    for (int v = 0; v < kThrPer; ++v) c += (uint32_t)__popcll(__ballot(key[v] >= mid));
    if (c >= (uint32_t)a.kk) lo = mid;
    else hi = mid - 1u;
  }
  if (lane == 0) a.tau[row] = lo < 0x00800000u ? -__builtin_inff() : key_score(lo);
}

// --------------------------------------------------------------- finalize

// Orders each query's kept candidates (score desc, id asc) and emits the first
// kk. Bisection on the 32-bit score key (over the kept range) finds the kk-th
// best score K; if K is tied across the cut, a second bisection over the tied
// ids picks the lowest ones. Rank keys are unique, so exactly kk candidates
// are >= the resulting composite threshold; each one's output slot is its
// count of better selected candidates. A query whose kept set is smaller than
// kk or overflowed is flagged (status 1 / 2) for the exhaustive path; status 0
// means its output row is final.
extern "C" __global__ __launch_bounds__(kFinThreads) void eos_tq_finalize(TqFinalizeArgs a) {
  __shared__ uint32_t slots[2 * (kFinThreads / 64)];
  int parity = 0;
  __shared__ uint32_t smin[kFinThreads / 64], smax[kFinThreads / 64];
  __shared__ u64 sel[kSortCap];
  __shared__ uint32_t sel_n;
  const int row = blockIdx.x;
  if (row >= a.q) return;
  const int tid = threadIdx.x;
  const uint32_t cnt = a.cand_count[row];
  if (cnt > (uint32_t)a.cap || cnt > (uint32_t)kSortCap) {
    if (tid == 0) a.status[row] = 2;
    return;
  }
  if (cnt < (uint32_t)a.kk) {
    if (tid == 0) a.status[row] = 1;
    return;
  }
  const int nv = (int)((cnt + kFinThreads - 1) / kFinThreads);
  u64 c[kFinPer];
  uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
  for (int v = 0; v < kFinPer; ++v) {
    const uint32_t i = tid + v * kFinThreads;
    c[v] = (v < nv && i < cnt) ? a.cand[(size_t)row * a.cap + i] : 0ull;
    if (c[v] != 0ull) {
      kmin = min(kmin, (uint32_t)(c[v] >> 32));
      kmax = max(kmax, (uint32_t)(c[v] >> 32));
    }
  }
  block_minmax<kFinThreads>(kmin, kmax, smin, smax);
  // K = the kk-th best score key.
  uint32_t lo = kmin, hi = kmax;
  while (lo < hi) {
    const uint32_t mid = lo + ((hi - lo) >> 1) + 1u;
    uint32_t n = 0;
#pragma unroll
    for (int v = 0; v < kFinPer; ++v)
      if (v < nv) n += (uint32_t)__popcll(__ballot(c[v] != 0ull && (uint32_t)(c[v] >> 32) >= mid));
    if (block_sum<kFinThreads>(n, slots, parity) >= (uint32_t)a.kk) lo = mid;
    else hi = mid - 1u;
  }
  const uint32_t K = lo;
  uint32_t ng = 0, ne = 0;
#pragma unroll
  for (int v = 0; v < kFinPer; ++v) {
    if (v < nv) {
      const uint32_t k = (uint32_t)(c[v] >> 32);
      ng += (uint32_t)__popcll(__ballot(c[v] != 0ull && k > K));
      ne += (uint32_t)__popcll(__ballot(c[v] != 0ull && k == K));
    }
  }
  ng = block_sum<kFinThreads>(ng, slots, parity);
  ne = block_sum<kFinThreads>(ne, slots, parity);
  u64 thr = (u64)K << 32;
  if (ng + ne > (uint32_t)a.kk) {
    // Tie at the cut: keep the (kk - ng) tied candidates with the lowest ids,
    // i.e. the largest low words (~id).
    const uint32_t need = (uint32_t)a.kk - ng;
    uint32_t l = 0u, h = 0xffffffffu;
    while (l < h) {
      const uint32_t mid = l + ((h - l) >> 1) + 1u;
      uint32_t n = 0;
#pragma unroll
      for (int v = 0; v < kFinPer; ++v)
        if (v < nv)
          n += (uint32_t)__popcll(__ballot(c[v] != 0ull && (uint32_t)(c[v] >> 32) == K &&
                                           (uint32_t)c[v] >= mid));
      if (block_sum<kFinThreads>(n, slots, parity) >= need) l = mid;
      else h = mid - 1u;
    }
    thr |= l;
  }
  if (tid == 0) sel_n = 0u;
  __syncthreads();
#pragma unroll
  for (int v = 0; v < kFinPer; ++v) {
    if (v < nv && c[v] != 0ull && c[v] >= thr) {
      const uint32_t pos = atomicAdd(&sel_n, 1u);
      if (pos < (uint32_t)kSortCap) sel[pos] = c[v];
    }
  }
  __syncthreads();
  for (int i = tid; i < a.kk; i += kFinThreads) {
    const u64 x = sel[i];
    int rank = 0;
#pragma unroll 8
    for (int j = 0; j < a.kk; ++j) rank += sel[j] > x ? 1 : 0;
    a.ids[(size_t)row * a.kk + rank] = (long long)rank_id(x);
    a.scores[(size_t)row * a.kk + rank] = key_score((uint32_t)(x >> 32));
  }
  if (tid == 0) a.status[row] = 0;
}

// ------------------------------------------------------------------ maxsim

namespace {

template <int BITS, int KS, int NQG>
EOS_DEV void tq_maxsim_body(const TqMaxsimArgs& a) {
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
  const v4i* packed = reinterpret_cast<const v4i*>(a.packed);
  TqScanArgs la;  // lookup tables for decode_step
  la.lut0 = a.lut0;
  la.lut1 = a.lut1;
  la.lut2 = a.lut2;
  la.lut3 = a.lut3;
  float al[NQG];
#pragma unroll
  for (int g = 0; g < NQG; ++g) al[g] = a.alpha[g * 32 + (lane & 31)];
  for (long long doc = blockIdx.x * (kScanThreads / 64) + wave; doc < a.ndocs; doc += nw) {
    float mx[NQG];
#pragma unroll
    for (int g = 0; g < NQG; ++g) mx[g] = -__builtin_inff();
    const long long t0 = (a.doc_begin + doc) * a.tiles_per_doc;
    v4i raw[NLOAD];
    float4 nrm4[4];
    load_tile_codes<NLOAD>(raw, packed, t0, lane);
    load_tile_norms(nrm4, a.norms, t0, half);
    for (int t = 0; t < a.tiles_per_doc; ++t) {
      v4i nraw[NLOAD];
      float4 nnrm4[4];
      if (t + 1 < a.tiles_per_doc) {
        load_tile_codes<NLOAD>(nraw, packed, t0 + t + 1, lane);
        load_tile_norms(nnrm4, a.norms, t0 + t + 1, half);
      }
      int boff = lane;
      asm volatile("" : "+v"(boff));
      v16i acc[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) acc[cb] = v16i{0};
#pragma unroll
      for (int c = 0; c < NLOAD; ++c) {
#pragma unroll
        for (int h = 0; h < SPL; ++h) {
          const int s = c * SPL + h;
          if (s < KS) {
            const v4i af = decode_step<BITS>(raw[c], h, la);
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
              const v4i bf = sb[(s * NCB + cb) * 64 + boff];
              acc[cb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf, acc[cb], 0, 0, 0);
            }
          }
        }
      }
      float nrm[16];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        nrm[4 * i4 + 0] = nrm4[i4].x;
        nrm[4 * i4 + 1] = nrm4[i4].y;
        nrm[4 * i4 + 2] = nrm4[i4].z;
        nrm[4 * i4 + 3] = nrm4[i4].w;
      }
#pragma unroll
      for (int g = 0; g < NQG; ++g) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int dot = acc[2 * g][i] * 256 + acc[2 * g + 1][i];
          mx[g] = fmaxf(mx[g], ((float)dot * al[g]) * nrm[i] + 0.0f);
        }
      }
#pragma unroll
      for (int c = 0; c < NLOAD; ++c) raw[c] = nraw[c];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) nrm4[i4] = nnrm4[i4];
    }
#pragma unroll
    for (int g = 0; g < NQG; ++g) {
      float v = fmaxf(mx[g], __shfl_xor(mx[g], 32));  // token max over the document
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) v = v + __shfl_xor(v, o);
      if (lane == 0 && g < a.groups) a.out[(size_t)g * a.out_stride + doc] = v;
    }
  }
}

}  // namespace

#define EOS_TQ_MAXSIM(BITS, KS, NQG)                                                        \
  extern "C" __global__ __launch_bounds__(kScanThreads) void eos_tq_maxsim_b##BITS##_k##KS##_g##NQG( \
      TqMaxsimArgs a) {                                                                     \
    tq_maxsim_body<BITS, KS, NQG>(a);                                                       \
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
