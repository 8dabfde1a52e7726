// q8 BERT-style encoder forward on gfx950 (CDNA4).
//
// Semantics follow the reference host path of the imported BERT embedder
// (runtime/backend/bert_embedder_ops.go:101-197): embeddings + affine LN
// (tensor_ops.go:1451-1512), per layer QKV -> masked attention -> O proj ->
// residual + LN -> FFN (erf GELU) -> residual + LN
// (bert_encoder_layer_ops.go:80-225), masked mean pool then L2 normalize.
//
// The compact transformer family (models/default_embedding.go:419-505) runs
// on the same kernels: embed mode 1 (token + role, RoPE), non-affine LN
// (gamma 1, beta 0, eps 1e-5), tanh GELU, bias-free GEMMs, pool mode 1.
//
// Layout: only active (mask != 0) positions are computed, packed into rows
// [0, total); a sequence's rows are contiguous. Activations are f16, every
// GEMM accumulates in f32 on v_mfma_f32_32x32x16_f16, weights are int8 codes
// (stored as exact f16) with a per-output-channel f32 scale applied in the
// epilogue together with the bias, the activation or the residual + LN.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "enc_args.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#define EOS_DEV __device__ __forceinline__

namespace {

EOS_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
EOS_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

EOS_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Sum over the wavefront without LDS or scalar round trips: DPP adds within
// each row of 16 lanes (quad swaps, then half-row and row mirrors, so every
// lane of a row holds the row's sum), then v_permlane16_swap (lane l gets
// lane l ^ 16's value) and v_permlane32_swap (lane l ^ 32's) with an add
// each. Every lane ends with (r0 + r1) + (r2 + r3) of the row sums r_i (each
// add is commutative, so every lane computes the same value); a different
// summation order from wave_sum.
template <int CTRL>
EOS_DEV float dpp_shuffled(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
// v (lane l) and v (lane l ^ 16) / (lane l ^ 32): the two results of a swap
// of v with itself (odd rows against even rows, or the upper 32 lanes
// against the lower 32; a is the even row's / lower half's value, b the
// other's). The elements are copied out of the builtin's two-element vector
// before the bit casts: __builtin_bit_cast applied to an element r[1]
// directly compiles to element 0.
EOS_DEV void swapped16(float v, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
EOS_DEV void swapped32(float v, float& a, float& b) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const unsigned r0 = r[0], r1 = r[1];
  a = __builtin_bit_cast(float, r0);
  b = __builtin_bit_cast(float, r1);
}
EOS_DEV float wave_sum_dpp(float v) {
  v += dpp_shuffled<0xb1>(v);   // quad_perm [1, 0, 3, 2]
  v += dpp_shuffled<0x4e>(v);   // quad_perm [2, 3, 0, 1]
  v += dpp_shuffled<0x141>(v);  // row_half_mirror
  v += dpp_shuffled<0x140>(v);  // row_mirror
  float a, b;
  swapped16(v, a, b);  // rows {0, 1} and {2, 3}: a is the even row's sum
  v = a + b;
  swapped32(v, a, b);  // a holds r0 + r1, b holds r2 + r3
  return a + b;
}

// Maximum over the wavefront, the same pattern as wave_sum_dpp.
EOS_DEV float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_shuffled<0xb1>(v));
  v = fmaxf(v, dpp_shuffled<0x4e>(v));
  v = fmaxf(v, dpp_shuffled<0x141>(v));
  v = fmaxf(v, dpp_shuffled<0x140>(v));
  float a, b;
  swapped16(v, a, b);
  v = fmaxf(a, b);
  swapped32(v, a, b);
  return fmaxf(a, b);
}

// Maximum over the wavefront of non-negative values (|y|, or 0): for
// non-negative floats the order of the bit patterns as unsigned integers is
// the order of the values, so the steps are integer maxima (one DPP
// instruction each, no NaN canonicalization).
template <int CTRL>
EOS_DEV uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
EOS_DEV float wave_max_nonneg(float f) {
  uint32_t v = __builtin_bit_cast(uint32_t, f);
  v = max(v, dpp_u32<0xb1>(v));
  v = max(v, dpp_u32<0x4e>(v));
  v = max(v, dpp_u32<0x141>(v));
  v = max(v, dpp_u32<0x140>(v));
  const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  const unsigned a16 = r16[0], b16 = r16[1];
  v = max(a16, b16);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  const unsigned a32 = r32[0], b32 = r32[1];
  return __builtin_bit_cast(float, max(a32, b32));
}

// Symmetric per-row int8 quantization: scale = max|y| / 127 (0 for a zero
// row), code = rint(y * 127 / max|y|), |code| <= 127.
EOS_DEV float q8_inv(float amax) { return amax > 0.0f ? 127.0f / amax : 0.0f; }
EOS_DEV int8_t q8_code(float y, float inv) {
  return (int8_t)fminf(fmaxf(rintf(y * inv), -127.0f), 127.0f);
}

// erf(z) by Abramowitz & Stegun, Handbook of Mathematical Functions, 7.1.26
// (|error| <= 1.5e-7): one reciprocal, one exp2 and a degree-5 polynomial,
// branch-free (the library erff evaluates two polynomials in divergent
// branches). The GELU output is rounded to f16, far coarser than either.
EOS_DEV float erf_as(float z) {
  const float a = fabsf(z);
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(0.3275911f, a, 1.0f));
  float p = __builtin_fmaf(1.061405429f, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.254829592f);
  p *= t;
  const float e = __builtin_amdgcn_exp2f(-(a * a) * 1.4426950408889634f);  // exp(-a^2)
  return __builtin_copysignf(1.0f - p * e, z);
}

// tanh(u) = 1 - 2 / (exp(2u) + 1): one exp2 and one reciprocal; saturates to
// +-1 (exp2 -> inf or 0), absolute error ~1e-7.
EOS_DEV float tanh_exp(float u) {
  const float e = __builtin_amdgcn_exp2f(2.8853900817779268f * u);  // exp(2u)
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f);
}

EOS_DEV float gelu(float x, int kind) {
  if (kind == 1) return 0.5f * x * (1.0f + erf_as(x * 0.70710678118654752f));
  const float u = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanh_exp(u));
}

// erf GELU x Phi(x) for the GEMM and layer-tail epilogues as x sigma(z),
// z = x (a + b x^2 + c x^4) with x clamped to [-10, 10] inside z: a minimax
// fit of Phi(x) = sigma(z) whose f32 evaluation stays within 7.9e-5 of the
// exact GELU for every x (checked against erf over [-30, 30]; at |x| >= 10
// the result is x sigma(+-35), within 1e-14 of the GELU). The constants carry
// the -log2(e) factor, so sigma(z) = 1 / (1 + exp2(t)) with t = -z log2(e):
// 7 VALU instructions and 2 transcendental ones per value (the
// Abramowitz & Stegun form of erf took 11 and 2). The 7.9e-5 is below half
// an f16 ulp of every output >= 0.16 in magnitude and small beside the int8
// quantization of the layer's other GEMM inputs.
EOS_DEV float gelu_erf_fast(float x) {
  const float xc = __builtin_amdgcn_fmed3f(x, -10.0f, 10.0f);
  const float x2 = xc * xc;
  float p = __builtin_fmaf(x2, 7.714337719e-04f, -1.050610005e-01f);
  p = __builtin_fmaf(p, x2, -2.303318177e+00f);
  const float e = __builtin_amdgcn_exp2f(p * xc);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

}  // namespace

// ------------------------------------------------------------------- pack

namespace {

// Block-wide exclusive prefix sum of one int per thread (256 threads);
// *total receives the sum over the block. `scr` holds 4 ints.
EOS_DEV int block_exclusive_scan256(int v, int* scr, int* total) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
  if (lane == 63) scr[w] = inc;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    before += i < w ? scr[i] : 0;
    all += scr[i];
  }
  __syncthreads();
  *total = all;
  return before + inc - v;
}

}  // namespace

// Active positions per sequence: one workgroup per sequence, mask values
// read 8 per thread at a time so the loads overlap.
extern "C" __global__ __launch_bounds__(256) void eos_enc_count(EncPackArgs a) {
  __shared__ int scr[4];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int32_t* m = a.mask + (size_t)b * a.tokens;
  const int32_t* ids = a.ids != nullptr ? a.ids + (size_t)b * a.tokens : nullptr;
  const int32_t* tys = a.type_ids != nullptr ? a.type_ids + (size_t)b * a.tokens : nullptr;
  // 16 mask words (and ids, types) per thread requested at a time, from
  // clamped positions (a load under a per-lane condition becomes a branch of
  // its own and waits for its data before the next one is issued).
  int mine = 0;
  bool bad = false;
  for (int b0 = 0; b0 < a.tokens; b0 += 256 * 16) {  // b0: uniform
    const int base = b0 + tid;
    int v[16], iv[16], tv[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int t = min(base + 256 * u, a.tokens - 1);
      if (b0 + 256 * u < a.tokens) {
        v[u] = a.all_active ? 1 : m[t];
        iv[u] = ids != nullptr ? ids[t] : 0;
        tv[u] = tys != nullptr ? tys[t] : 0;
      }
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      if (base + 256 * u < a.tokens) {
        mine += v[u] != 0 ? 1 : 0;
        bad = bad || iv[u] < 0 || iv[u] >= a.vocab || tv[u] < 0 || tv[u] >= a.ntype;
      }
    }
  }
  if (bad && ids != nullptr) *a.status = 1;
  int total = 0;
  (void)block_exclusive_scan256(mine, scr, &total);
  if (tid == 0) {
    a.seq_cnt[b] = total;
    if (a.seq_q != nullptr)
      a.seq_q[b] = total + ((a.cls_row && !a.all_active && m[0] == 0) ? 1 : 0);
  }
}

// One workgroup per sequence: rows of sequence b start at the sum of the
// earlier sequences' counts, each rounded up to a multiple of 8 (so every
// sequence starts 16-byte aligned in feature-major copies); its positions
// are compacted in increasing order, and the rows up to the next multiple
// of 8 are pad rows (position -1). Thread i owns the contiguous positions
// [i * per, (i + 1) * per). The last workgroup writes the row total.
extern "C" __global__ __launch_bounds__(256) void eos_enc_pack(EncPackArgs a) {
  __shared__ int scr[4];
  const int b = blockIdx.x;
  const int tid = threadIdx.x;
  // Rows of a sequence: its query rows (the active positions, plus the
  // query-only CLS row when there is one), rounded up to a multiple of 8.
  const int32_t* qrows = a.seq_q != nullptr ? a.seq_q : a.seq_cnt;
  int before = 0;
  for (int i = tid; i < b; i += 256) before += (qrows[i] + 7) & ~7;
  int seq_base = 0;
  (void)block_exclusive_scan256(before, scr, &seq_base);
  const int32_t* m = a.mask + (size_t)b * a.tokens;
  const int per = (a.tokens + 255) / 256;
  const int t0 = tid * per;
  // The thread's positions in chunks of mask words (8 when a thread has at
  // most 8, else 32), each chunk requested at once; with a single chunk the
  // words stay in registers for the second pass instead of being read
  // again. per is uniform, so every thread takes the same instance.
  int seq_cnt = 0;
  auto pack_body = [&](auto chunk) {
    constexpr int kChunk = decltype(chunk)::value;
    int v[kChunk];
    auto load = [&](int k0) {
      // Clamped positions, then the validity test (see eos_enc_count).
      if (!a.all_active) {
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
          if (k0 + u < per) v[u] = m[min(t0 + k0 + u, a.tokens - 1)];  // uniform test
      }
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        const int t = t0 + k0 + u;
        const bool in = k0 + u < per && t < a.tokens;
        v[u] = in && (a.all_active || v[u] != 0) ? 1 : 0;
      }
    };
    int mine = 0;
    for (int k0 = 0; k0 < per; k0 += kChunk) {
      load(k0);
#pragma unroll
      for (int u = 0; u < kChunk; ++u) mine += v[u] != 0 ? 1 : 0;
    }
    int r = seq_base + block_exclusive_scan256(mine, scr, &seq_cnt);
    for (int k0 = 0; k0 < per; k0 += kChunk) {
      if (per > kChunk) load(k0);
#pragma unroll
      for (int u = 0; u < kChunk; ++u) {
        if (v[u] != 0) {
          a.row_b[r] = b;
          a.row_t[r] = t0 + k0 + u;
          ++r;
        }
      }
    }
  };
  if (per <= 8)
    pack_body(std::integral_constant<int, 8>{});
  else
    pack_body(std::integral_constant<int, 32>{});
  // The query-only row of position 0 (CLS pooling with position 0 masked).
  const int extra = a.seq_q != nullptr ? a.seq_q[b] - seq_cnt : 0;
  if (extra != 0 && tid == 0) {
    a.row_b[seq_base + seq_cnt] = b;
    a.row_t[seq_base + seq_cnt] = 0;
  }
  const int used = seq_cnt + extra;
  const int padded = (used + 7) & ~7;
  if (tid < padded - used) {
    a.row_b[seq_base + used + tid] = b;
    a.row_t[seq_base + used + tid] = -1;
  }
  if (tid == 0) {
    a.seq_off[b] = seq_base;
    if (b == a.batch - 1) *a.total = seq_base + padded;
  }
  if (a.order != nullptr) {
    // Rank of this sequence by key count, longest first, ties by index: an
    // attention workgroup's time grows with its keys, so the long
    // sequences' workgroups are dispatched first and the short ones fill
    // the end.
    const int mc = a.seq_cnt[b];
    int ahead = 0;
    for (int i = tid; i < a.batch; i += 256) {
      const int c = a.seq_cnt[i];
      ahead += (c > mc || (c == mc && i < b)) ? 1 : 0;
    }
    int rank = 0;
    (void)block_exclusive_scan256(ahead, scr, &rank);
    if (tid == 0) a.order[rank] = b;
  }
}

// -------------------------------------------------------------- embedding

// One wavefront per active row: token + position + type in f32 (that order),
// then affine LayerNorm (two-pass statistics), f16 out.
extern "C" __global__ __launch_bounds__(256) void eos_enc_embed(EncEmbedArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= *a.total) return;
  const int b = a.row_b[row], t = a.row_t[row];
  if (t < 0) {
    // Pad row (sequence alignment): zeros, never pooled or attended to.
    for (int c = lane; c < a.hidden; c += 64) a.out[(size_t)row * a.hidden + c] = 0;
    if (a.q8 != nullptr) {
      for (int c = lane; c < a.hidden / 16; c += 64)
        *reinterpret_cast<uint4*>(a.q8 + (size_t)row * a.hidden + 16 * c) = make_uint4(0, 0, 0, 0);
      if (lane == 0) a.qscale[row] = 0.0f;
    }
    return;
  }
  int id = a.ids[(size_t)b * a.tokens + t];
  int ty = a.type_ids ? a.type_ids[(size_t)b * a.tokens + t] : 0;
  const int pos = t;
  if (id < 0 || id >= a.vocab || ty < 0 || ty >= a.ntype || pos >= a.npos) {
    if (lane == 0) *a.status = 1;
    id = id < 0 || id >= a.vocab ? 0 : id;
    ty = ty < 0 || ty >= a.ntype ? 0 : ty;
  }
  const int p = pos < a.npos ? pos : a.npos - 1;
  if (a.mode == 1) {
    // Compact family: lane owns column pairs (2i, 2i + 1), i = lane + 64 j;
    // x = tok + role in f32, then the pair is rotated by the position's
    // (cos, sin) as ropeRows does: (x0 c - x1 s, x0 s + x1 c).
    const float2* te = reinterpret_cast<const float2*>(a.tok + (size_t)id * a.hidden);
    const float2* re = reinterpret_cast<const float2*>(a.typ + (size_t)ty * a.hidden);
    const float2* rt = reinterpret_cast<const float2*>(a.pos + (size_t)p * a.hidden);
    const int pairs = a.hidden >> 1;
    float2 tv[8], rv[8], cs[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = min(lane + 64 * j, pairs - 1);
      tv[j] = te[i];
      rv[j] = re[i];
      cs[j] = rt[i];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int i = lane + 64 * j;
      if (i < pairs) {
        const float x0 = tv[j].x + rv[j].x, x1 = tv[j].y + rv[j].y;
        const float y0 = __fsub_rn(__fmul_rn(x0, cs[j].x), __fmul_rn(x1, cs[j].y));
        const float y1 = __fadd_rn(__fmul_rn(x0, cs[j].y), __fmul_rn(x1, cs[j].x));
        const uint32_t packed = (uint32_t)f2h(y0) | ((uint32_t)f2h(y1) << 16);
        *reinterpret_cast<uint32_t*>(a.out + (size_t)row * a.hidden + 2 * i) = packed;
      }
    }
    return;
  }
  constexpr int kMaxPer = 12;  // hidden <= 768
  // Every table value is loaded from a clamped column before any is used,
  // then the validity test applies (loads under a per-lane condition compile
  // to a branch each and wait for their data one after another); likewise
  // gamma and beta.
  float tv[kMaxPer], pv[kMaxPer], yv[kMaxPer], gv[kMaxPer], bv[kMaxPer];
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    const int c = min(lane + 64 * j, a.hidden - 1);
    tv[j] = a.tok[(size_t)id * a.hidden + c];
    pv[j] = a.pos[(size_t)p * a.hidden + c];
    yv[j] = a.typ[(size_t)ty * a.hidden + c];
    gv[j] = a.gamma[c];
    bv[j] = a.beta[c];
  }
  float v[kMaxPer];
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    const int c = lane + 64 * j;
    v[j] = 0.f;
    if (c < a.hidden) {
      v[j] = tv[j] + pv[j] + yv[j];
      s += v[j];
    }
  }
  const float mean = wave_sum_dpp(s) / (float)a.hidden;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    const int c = lane + 64 * j;
    if (c < a.hidden) q += (v[j] - mean) * (v[j] - mean);
  }
  const float inv = 1.0f / sqrtf(wave_sum_dpp(q) / (float)a.hidden + a.eps);
  // The f16 outputs are kept (not the f32 values, which would stay live
  // across the row maximum and cost occupancy); the int8 codes are taken
  // from them, with the row maximum of the f32 values as the scale.
  _Float16 y16[kMaxPer];
  float amax = 0.0f;
#pragma unroll
  for (int j = 0; j < kMaxPer; ++j) {
    const int c = lane + 64 * j;
    y16[j] = (_Float16)0.0f;
    if (c < a.hidden) {
      const float y = (v[j] - mean) * inv * gv[j] + bv[j];
      y16[j] = (_Float16)y;
      a.out[(size_t)row * a.hidden + c] = __builtin_bit_cast(uint16_t, y16[j]);
      amax = fmaxf(amax, fabsf(y));
    }
  }
  if (a.q8 != nullptr) {
    // The codes are staged in this wavefront's LDS row and written with
    // 16-byte stores. One wavefront writes and reads its own row: LDS
    // operations of a wavefront complete in order.
    __shared__ __attribute__((aligned(16))) int8_t qrow[4][1024];
    int8_t* qr = qrow[threadIdx.x >> 6];
    amax = wave_max_dpp(amax);
    const float qi = q8_inv(amax);
#pragma unroll
    for (int j = 0; j < kMaxPer; ++j) {
      const int c = lane + 64 * j;
      if (c < a.hidden) qr[c] = q8_code((float)y16[j], qi);
    }
    __builtin_amdgcn_wave_barrier();
    for (int c = lane; c < a.hidden / 16; c += 64)
      *reinterpret_cast<uint4*>(a.q8 + (size_t)row * a.hidden + 16 * c) =
          *reinterpret_cast<const uint4*>(qr + 16 * c);
    if (lane == 0) a.qscale[row] = amax / 127.0f;
  }
}

// ------------------------------------------------------------------- GEMM

namespace {
constexpr int kBK = 32;  // K chunk: 32 halves = one 64-byte segment of each operand row

// Stage layout: BM rows of A then BN rows of W, 64 bytes (four 16-byte slots)
// per row, no padding. Chunk c of row r sits in slot c ^ ((r >> 2) & 3): the 16
// rows that a quarter-wavefront's 16-byte fragment reads touch cover all 64
// banks once, and each load instruction still fills 1 KB of LDS contiguously.
EOS_DEV int swz(int r, int c) { return c ^ ((r >> 2) & 3); }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
EOS_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{}).
template <typename F, int... I>
EOS_DEV void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
EOS_DEV void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// LDS byte address of a pointer into a __shared__ array.
typedef __attribute__((address_space(3))) const uint16_t lds_u16;
EOS_DEV uint32_t lds_addr(const uint16_t* p) { return (uint32_t)(uintptr_t)(lds_u16*)p; }

// 16-byte LDS read at addr + OFF. Issued as inline assembly: the compiler's
// wait analysis treats every compiler-visible LDS read as possibly reading
// memory an outstanding direct-to-LDS load writes and waits for all of them
// (vmcnt(0)), which would drain the load pipeline at each step. Completion
// is awaited with lgkm_wait below; stage contents with wait_vmcnt + barrier.
template <int OFF>
EOS_DEV v8h lds_read16(uint32_t addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset range");
  v8h r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

// s_waitcnt lgkmcnt(0) that the fragments pass through, so no consumer of
// them can be scheduled above the wait.
template <int N>
EOS_DEV void lgkm_wait(v8h (&f)[N]) {
  static_assert(N <= 6, "fragment count");
  if constexpr (N == 2)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]));
  else if constexpr (N == 3)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]));
  else if constexpr (N == 4)
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
  else if constexpr (N == 6)
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]));
  else
    static_assert(N == 2 || N == 3 || N == 4 || N == 6, "fragment count");
}

// Workgroup tile (64 WM) x (64 WN) over 4 wavefronts in a 2 x 2 grid, each
// wavefront (32 WM) x (32 WN) = WM x WN MFMA 32x32 blocks. K advances in
// chunks of 32 through NS LDS stages filled by direct global -> LDS loads
// (16 bytes per lane, no staging registers): chunk kc + NS - 1 is requested
// while chunk kc is computed, so each load has NS - 1 chunks of MFMAs to
// land. Per chunk a wavefront issues WM + WN loads (16 rows each) and waits
// with vmcnt((NS - 2)(WM + WN)), i.e. for everything but the newer chunks,
// then one barrier makes the whole stage visible.
// Epilogue: v = scale[n] * acc + bias[n]; mode 1 erf GELU, 2 tanh GELU,
// 3 + residual[m][n] (out may alias residual: each element is read and
// written by the same lane).
// TR = false: W is the MFMA's first operand, a lane's results lie along an
// output row (row-major out). TR = true (columns from vt_col0 on, when vt is
// given): A first, a lane's results lie along an output column, stored
// transposed into vt[col - vt_col0][row].
template <int WM, int WN, int NS, bool TR, bool I8>
EOS_DEV void gemm_tile(const EncGemmArgs& a, int m0, int n0, int rows, uint16_t* st, float* lsc,
                       float* lbi, float* lrs) {
  constexpr int BM = 64 * WM, BN = 64 * WN, ST = (BM + BN) * kBK;  // halves per stage
  constexpr int ESZ = I8 ? 1 : 2;  // operand bytes: a 64-byte chunk is 32 halves or 64 int8
  constexpr int NLD = WM + WN;  // 16-row loads per wavefront per chunk
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int g = lane >> 5, l32 = lane & 31;
  // Load u of this wavefront fills stage rows 16 (wave + 4u) .. + 15 (A rows
  // for u < WM, W rows after): lane i writes slot i % 4 of row
  // 16 (wave + 4u) + i / 4 and so reads chunk swz(row, i % 4) of that row.
  // Rows past the matrix are clamped to its last row (computed, never stored).
  const char* const abytes = I8 ? (const char*)a.a8 : (const char*)a.a;
  const char* const wbytes = I8 ? (const char*)a.w8 : (const char*)a.w;
  const size_t rowb = (size_t)a.k * ESZ;
  const char* src[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = 16 * (wave + 4 * u) + (lane >> 2);
    const int c = swz(r, lane & 3);
    if (u < WM)
      src[u] = abytes + (size_t)min(m0 + r, a.max_rows - 1) * rowb + c * 16;
    else
      src[u] = wbytes + (size_t)(n0 + r - BM) * rowb + c * 16;
  }
  const int nk = (int)(rowb / 64);
  // Chunks past the end are clamped to the last one (loaded, never computed).
  auto issue = [&](uint16_t* st, int kc) {
    const int k0 = min(kc, nk - 1) * 64;
#pragma unroll
    for (int u = 0; u < NLD; ++u)
      __builtin_amdgcn_global_load_lds(src[u] + k0, st + 16 * 32 * (wave + 4 * u), 16, 0, 0);
  };
  // Fragment of lane (l32, g) at K step s: row base + l32, chunk 2s + g (base
  // is a multiple of 32, so the swizzle depends on l32 only). Byte addresses
  // of this lane's first A and B fragments in stage 0, per K step.
  const uint32_t st_b = lds_addr(st);
  uint32_t abase[2], bbase[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int fo = l32 * kBK + swz(l32, 2 * s + g) * 8;
    abase[s] = st_b + 2 * (wm * 32 * WM * kBK + fo);
    bbase[s] = st_b + 2 * ((BM + wn * 32 * WN) * kBK + fo);
  }
  using Acc = std::conditional_t<I8, v16i, v16f>;
  Acc acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = Acc{0};
  // Fragments of K step S of stage STG (read, then awaited).
  auto frags = [&](auto stg_c, auto s_c, v8h (&f)[WM + WN]) {
    constexpr int STG = decltype(stg_c)::value, S = decltype(s_c)::value;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      constexpr int kStage = 2 * STG * ST;
      f[i] = lds_read16<kStage>(abase[S] + 2 * i * 32 * kBK);
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) f[WM + j] = lds_read16<2 * STG * ST>(bbase[S] + 2 * j * 32 * kBK);
  };
  auto mma = [&](v8h (&f)[WM + WN]) {
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        // int8: 32 K values (16 bytes) per lane, the same bytes of the stage
        // as 16 halves, so addressing and layout are shared.
        const v8h& x = TR ? f[i] : f[WM + j];
        const v8h& y = TR ? f[WM + j] : f[i];
        if constexpr (I8)
          acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(v4i, x),
                                                            __builtin_bit_cast(v4i, y), acc[i][j],
                                                            0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, acc[i][j], 0, 0, 0);
      }
  };
  auto compute = [&](auto stg_c) {
    v8h f0[WM + WN], f1[WM + WN];
    frags(stg_c, std::integral_constant<int, 0>{}, f0);
    lgkm_wait(f0);
    frags(stg_c, std::integral_constant<int, 1>{}, f1);
    mma(f0);
    lgkm_wait(f1);
    mma(f1);
  };
  // The tile's column scales and biases (and int8 row scales) are loaded
  // before the first chunks are requested and stored to LDS behind them, so
  // the epilogue reads them from LDS (the loop's barriers publish them).
  const bool ep_c = tid < BN, ep_r = I8 && tid < BM;
  const float v_sc = ep_c ? a.wscale[n0 + tid] : 0.0f;
  const float v_bi = ep_c ? a.bias[n0 + tid] : 0.0f;
  const float v_rs = ep_r ? a.ascale[min(m0 + tid, a.max_rows - 1)] : 1.0f;
  // Chunks 0 .. NS - 2 are requested up front; at the step of chunk c the
  // stage of chunk c - 1 (read at the step before, ordered by this step's
  // barrier) receives chunk c + NS - 1, so NS - 1 chunks are in flight.
#pragma unroll
  for (int c = 0; c < NS - 1; ++c) issue(st + c * ST, c);
  if (ep_c) {
    lsc[tid] = v_sc;
    lbi[tid] = v_bi;
  }
  if (ep_r) lrs[tid] = v_rs;
  // NS chunks per pass, one stage each, stage indices static (the fragment
  // reads address stages by immediate offsets); one back-edge and no exit in
  // the body. The barrier is the bare s_barrier: a fenced one
  // (__syncthreads) must wait for every outstanding direct-to-LDS load,
  // including the chunks just requested, and vmcnt has already made this
  // wavefront's part of the stage land.
  int kc = 0;
  do {
    static_for<NS>([&](auto sc) {
      constexpr int S = decltype(sc)::value;
      wait_vmcnt<(NS - 2) * NLD>();
      __builtin_amdgcn_s_barrier();
      issue(st + ((S + NS - 1) % NS) * ST, kc + S + NS - 1);
      if (S == 0 || kc + S < nk) compute(sc);
    });
    kc += NS;
  } while (kc < nk);
  // No LDS write may land after the workgroup exits.
  wait_vmcnt<0>();
  // Epilogue through LDS (every mode but the residual one): each lane writes
  // its results into the tile in the ring's memory, then whole output rows
  // (or, transposed, whole V^T row segments) go out as 16-byte stores, 16
  // consecutive lanes per 256-byte row segment. Writing the MFMA layout
  // directly scattered every store instruction over 32 rows.
  if (TR || a.epi != 3) {
    __syncthreads();  // every wavefront's last fragment reads are done
    uint16_t* const tile = st;
    constexpr int TS = TR ? BM + 8 : BN + 8;  // halves per tile row (V^T: per column)
    static_assert((TR ? BN * TS : BM * TS) <= NS * ST, "the output tile fits the ring");
    if constexpr (TR) {
      // Element e of lane (l32, g) is row 8(e/4) + 4g + e%4 of the block and
      // column l32: 4 consecutive rows of one column, one 8-byte LDS store.
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int cl = wn * 32 * WN + j * 32 + l32;
        const float sc = lsc[cl], bi = lbi[cl];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int rl = wm * 32 * WM + i * 32 + 8 * q + 4 * g;
            v4h o;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
              if constexpr (I8)
                o[t] = (_Float16)__builtin_fmaf((float)acc[i][j][4 * q + t], sc * lrs[rl + t], bi);
              else
                o[t] = (_Float16)__builtin_fmaf(acc[i][j][4 * q + t], sc, bi);
            }
            *reinterpret_cast<v4h*>(&tile[cl * TS + rl]) = o;
          }
        }
      }
    } else {
      // Element e of lane (l32, g) is row l32 and columns 8(e/4) + 4g ..
      // + 3: one 8-byte LDS store per group of 4.
      auto stage = [&](auto epi_c) {
        constexpr int EPI = decltype(epi_c)::value;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
          const int rl = wm * 32 * WM + i * 32 + l32;
          const float rs = I8 ? lrs[rl] : 1.0f;
#pragma unroll
          for (int j = 0; j < WN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int cl = wn * 32 * WN + j * 32 + 8 * q + 4 * g;
              float4 sc = *reinterpret_cast<const float4*>(lsc + cl);
              const float4 bi = *reinterpret_cast<const float4*>(lbi + cl);
              if constexpr (I8) sc = make_float4(sc.x * rs, sc.y * rs, sc.z * rs, sc.w * rs);
              float v[4] = {__builtin_fmaf((float)acc[i][j][4 * q], sc.x, bi.x),
                            __builtin_fmaf((float)acc[i][j][4 * q + 1], sc.y, bi.y),
                            __builtin_fmaf((float)acc[i][j][4 * q + 2], sc.z, bi.z),
                            __builtin_fmaf((float)acc[i][j][4 * q + 3], sc.w, bi.w)};
              if constexpr (EPI == 1) {
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] = gelu_erf_fast(v[t]);
              } else if constexpr (EPI == 2) {
#pragma unroll
                for (int t = 0; t < 4; ++t) v[t] = gelu(v[t], 2);
              }
              v4h o;
#pragma unroll
              for (int t = 0; t < 4; ++t) o[t] = (_Float16)v[t];
              *reinterpret_cast<v4h*>(&tile[rl * TS + cl]) = o;
            }
          }
        }
      };
      switch (a.epi) {
        case 1: stage(std::integral_constant<int, 1>{}); break;
        case 2: stage(std::integral_constant<int, 2>{}); break;
        default: stage(std::integral_constant<int, 0>{}); break;
      }
    }
    __syncthreads();
    if constexpr (TR) {
      // V^T row (feature) m0 .. m0 + BM - 1 of each of the BN columns, 8 rows
      // per lane; groups start below rows (a multiple of 8), so none passes it.
      constexpr int R8 = BM / 8;
#pragma unroll
      for (int u = 0; u < BN * R8 / 256; ++u) {
        const int idx = tid + 256 * u;
        const int cl = idx / R8, r8 = idx % R8;
        const int row = m0 + 8 * r8;
        if (row < rows)
          *reinterpret_cast<v4i*>(a.vt + (size_t)(n0 + cl - a.vt_col0) * a.vt_ld + row) =
              *reinterpret_cast<const v4i*>(&tile[cl * TS + 8 * r8]);
      }
    } else {
      constexpr int C8 = BN / 8;
#pragma unroll
      for (int u = 0; u < BM * C8 / 256; ++u) {
        const int idx = tid + 256 * u;
        const int rl = idx / C8, c8 = idx % C8;
        const int row = m0 + rl;
        if (row < rows)
          *reinterpret_cast<v4i*>(a.out + (size_t)row * a.n + n0 + 8 * c8) =
              *reinterpret_cast<const v4i*>(&tile[rl * TS + 8 * c8]);
      }
    }
    return;
  }
  // With W as the first operand, element e of lane (l32, g) is output row
  // l32 of the block and column 8(e/4) + 4g + e%4: each group of 4
  // elements is 4 consecutive columns of one row, written as one 8-byte
  // store (and the residual read as one 8-byte load).
  // One straight-line epilogue per mode (the mode is uniform).
  auto epilogue = [&](auto epi_c) {
    constexpr int EPI = decltype(epi_c)::value;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int row = m0 + wm * 32 * WM + i * 32 + l32;
      if (row >= rows) continue;
      uint16_t* orow = a.out + (size_t)row * a.n;
      const uint16_t* rrow = EPI == 3 ? a.residual + (size_t)row * a.n : nullptr;
      const float rs = I8 ? a.ascale[row] : 1.0f;  // int8: the row's activation scale
#pragma unroll
      for (int j = 0; j < WN; ++j) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int col = n0 + wn * 32 * WN + j * 32 + 8 * q + 4 * g;
          float4 sc = *reinterpret_cast<const float4*>(a.wscale + col);
          const float4 bi = *reinterpret_cast<const float4*>(a.bias + col);
          if constexpr (I8) sc = make_float4(sc.x * rs, sc.y * rs, sc.z * rs, sc.w * rs);
          float v[4] = {__builtin_fmaf((float)acc[i][j][4 * q], sc.x, bi.x),
                        __builtin_fmaf((float)acc[i][j][4 * q + 1], sc.y, bi.y),
                        __builtin_fmaf((float)acc[i][j][4 * q + 2], sc.z, bi.z),
                        __builtin_fmaf((float)acc[i][j][4 * q + 3], sc.w, bi.w)};
          if constexpr (EPI == 3) {
            const v4h r = *reinterpret_cast<const v4h*>(rrow + col);
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] += (float)r[t];
          } else if constexpr (EPI == 1) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = gelu_erf_fast(v[t]);
          } else if constexpr (EPI == 2) {
#pragma unroll
            for (int t = 0; t < 4; ++t) v[t] = gelu(v[t], 2);
          }
          v4h o;
#pragma unroll
          for (int t = 0; t < 4; ++t) o[t] = (_Float16)v[t];
          *reinterpret_cast<v4h*>(orow + col) = o;
        }
      }
    }
  };
  epilogue(std::integral_constant<int, 3>{});  // the residual epilogue (a.epi == 3)
}

template <int WM, int WN, int NS, bool I8 = false>
EOS_DEV void gemm_body(const EncGemmArgs& a) {
  constexpr int BM = 64 * WM, BN = 64 * WN, ST = (BM + BN) * kBK;
  __shared__ __attribute__((aligned(16))) uint16_t st[NS * ST];
  __shared__ __attribute__((aligned(16))) float lsc[BN], lbi[BN], lrs[BM];
  const int rows = *a.rows;
  // XCD-aware tile order: workgroup w runs on XCD w % 8 (round-robin
  // dispatch), so XCD x takes row blocks x, x + 8, ... and walks all column
  // tiles of a row block back to back: the block's A rows are fetched into
  // that XCD's L2 once instead of once per column tile.
  const int ntn = a.n / BN;
  const int w = blockIdx.x, xcd = w & 7, l = w >> 3;
  const int mb = xcd + 8 * (l / ntn), nb = l % ntn;
  const int m0 = mb * BM, n0 = nb * BN;
  if (m0 >= rows) return;
  if (a.vt != nullptr && n0 >= a.vt_col0)
    gemm_tile<WM, WN, NS, true, I8>(a, m0, n0, rows, st, lsc, lbi, lrs);
  else
    gemm_tile<WM, WN, NS, false, I8>(a, m0, n0, rows, st, lsc, lbi, lrs);
}

}  // namespace

extern "C" __global__ __launch_bounds__(256) void eos_enc_gemm_t128(EncGemmArgs a) {
  gemm_body<2, 2, 3>(a);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void eos_enc_gemm_t256(EncGemmArgs a) {
  gemm_body<4, 2, 3>(a);
}
// W8A8 variant: int8 activation codes with per-row scales (written by the
// LayerNorm / embedding kernels) times int8 weight codes on
// v_mfma_i32_32x32x32_i8 (exact int32 sums), scaled by weight scale x row
// scale in the epilogue.
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
void eos_enc_gemm8_t256(EncGemmArgs a) {
  gemm_body<4, 2, 3, true>(a);
}
extern "C" __global__ __launch_bounds__(256) void eos_enc_gemm8_t128(EncGemmArgs a) {
  gemm_body<2, 2, 3, true>(a);
}

// ------------------------------------------------------------ LayerNorm

namespace {

// gamma / beta of the column pairs 2 lane + 128 t (t < H / 128) of a row.
template <int H>
struct LnParams {
  float2 g[H / 128], b[H / 128];
};
template <int H>
EOS_DEV void ln_params(const float* gamma, const float* beta, int lane, LnParams<H>& p) {
#pragma unroll
  for (int t = 0; t < H / 128; ++t) {
    p.g[t] = *reinterpret_cast<const float2*>(gamma + 2 * lane + 128 * t);
    p.b[t] = *reinterpret_cast<const float2*>(beta + 2 * lane + 128 * t);
  }
}

// One wavefront: affine LayerNorm of NR f16 rows y[r] (LDS or global memory;
// yout[r] may alias y[r]), processed together so that their wavefront
// reductions overlap. Every lane holds the column pairs 2 lane + 128 t.
// Two-pass mean / variance in f32 (wavefront sums by DPP), then
// out = (x - mean) * (rsq(var + eps) * gamma) + beta as one fma, rounded to
// f16 into yout[r]. With q8 (given for every row or for none), also the
// int8 codes rint(out * 127 / max|out|) of the f32 result (|code| <= 127
// since the reciprocal is within 1 ulp) and the scale max|out| / 127 (0 for
// a zero row) into *qscale[r].
template <int H, int NR>
EOS_DEV void ln_rows(const uint16_t* const (&y)[NR], const LnParams<H>& p, float eps, int lane,
                     uint16_t* const (&yout)[NR], int8_t* const (&q8)[NR],
                     float* const (&qscale)[NR]) {
  constexpr int P = H / 128;
  float x[NR][P][2];
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int t = 0; t < P; ++t) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(y[r] + 2 * lane + 128 * t);
      x[r][t][0] = h2f((uint16_t)(w & 0xffffu));
      x[r][t][1] = h2f((uint16_t)(w >> 16));
    }
  float mean[NR], inv[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < P; ++t) s += x[r][t][0] + x[r][t][1];
    mean[r] = wave_sum_dpp(s) * (1.0f / (float)H);
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    float q = 0.f;
#pragma unroll
    for (int t = 0; t < P; ++t)
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        x[r][t][e] -= mean[r];
        q = __builtin_fmaf(x[r][t][e], x[r][t][e], q);
      }
    inv[r] = __builtin_amdgcn_rsqf(wave_sum_dpp(q) * (1.0f / (float)H) + eps);
  }
  float amax[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    amax[r] = 0.0f;
#pragma unroll
    for (int t = 0; t < P; ++t) {
      x[r][t][0] = __builtin_fmaf(x[r][t][0], inv[r] * p.g[t].x, p.b[t].x);
      x[r][t][1] = __builtin_fmaf(x[r][t][1], inv[r] * p.g[t].y, p.b[t].y);
      amax[r] = fmaxf(amax[r], fmaxf(fabsf(x[r][t][0]), fabsf(x[r][t][1])));
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const h2 hv = {(_Float16)x[r][t][0], (_Float16)x[r][t][1]};
      *reinterpret_cast<uint32_t*>(yout[r] + 2 * lane + 128 * t) = __builtin_bit_cast(uint32_t, hv);
    }
  }
  // int8 codes: callers give q8 for every row or for none. The rows'
  // maxima are reduced together, then every code is stored, then lane 0
  // writes the scales in one branch (per-row reductions and lane-0 branches
  // in turn made the rows wait on each other).
  if (q8[0] == nullptr) return;
  float am[NR], qi[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) am[r] = wave_max_nonneg(amax[r]);
#pragma unroll
  for (int r = 0; r < NR; ++r) qi[r] = am[r] > 0.0f ? 127.0f * __builtin_amdgcn_rcpf(am[r]) : 0.0f;
  // code = rint(out * qi) by one fma: 1.5 * 2^23 + v rounds v to the
  // nearest integer (ties to even) in the low mantissa bits, whose low byte
  // is the code in two's complement for |v| < 2^22; v_perm packs the low
  // bytes of two such values.
#pragma unroll
  for (int r = 0; r < NR; ++r)
#pragma unroll
    for (int t = 0; t < P; ++t) {
      const float f0 = __builtin_fmaf(x[r][t][0], qi[r], 12582912.0f);
      const float f1 = __builtin_fmaf(x[r][t][1], qi[r], 12582912.0f);
      const uint32_t pk =
          __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x0c0c0400u);
      *reinterpret_cast<uint16_t*>(q8[r] + 2 * lane + 128 * t) = (uint16_t)pk;
    }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < NR; ++r) *qscale[r] = am[r] * (1.0f / 127.0f);
  }
}

template <int H>
EOS_DEV void ln_global_row(const EncLnArgs& a, int row, int lane) {
  LnParams<H> p;
  ln_params<H>(a.gamma, a.beta, lane, p);
  uint16_t* rp = a.h + (size_t)row * H;
  const uint16_t* const yin[1] = {rp};
  uint16_t* const yout[1] = {rp};
  int8_t* const q8[1] = {a.q8 != nullptr ? a.q8 + (size_t)row * H : nullptr};
  float* const qs[1] = {a.qscale != nullptr ? a.qscale + row : nullptr};
  ln_rows<H, 1>(yin, p, a.eps, lane, yout, q8, qs);
}

}  // namespace

// In-place affine LayerNorm of rows [0, *rows) of h [rows][hidden] (f16,
// hidden 128 / 256 / 384 / 512 / 768), one wavefront per row (ln_row).
extern "C" __global__ __launch_bounds__(256) void eos_enc_ln(EncLnArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= *a.rows) return;
  switch (a.hidden) {
    case 128: ln_global_row<128>(a, row, lane); break;
    case 256: ln_global_row<256>(a, row, lane); break;
    case 384: ln_global_row<384>(a, row, lane); break;
    case 512: ln_global_row<512>(a, row, lane); break;
    default: ln_global_row<768>(a, row, lane); break;
  }
}

// ------------------------------------------------------- fused layer tail

namespace {

constexpr int kTailFC = 128;  // FFN intermediate columns per chunk

// Block of BM = 32 RT rows, 8 wavefronts (two per SIMD). Every MFMA takes a
// weight fragment (32 output features, read from global memory in fragment
// order, 1 KB per wavefront load) as its first operand and an activation
// fragment (32 rows, from LDS) as its second, so a lane's results are
// 4-feature groups of one row.
//  - "down" wavefronts 0..3: wavefront d owns output features
//    [d H / 4, (d + 1) H / 4) (CT = H / 128 column tiles) of the O and
//    FFN-down projections over all RT row tiles;
//  - "up" wavefronts 4..7: wavefront u owns features [32 u, 32 u + 32) of
//    each 128-wide FFN-up chunk and computes its bias + GELU.
// The FFN is a two-stage pipeline over the chunks: while the down wavefronts
// multiply chunk c out of one LDS buffer, the up wavefronts fill the other
// with chunk c + 1, so one SIMD's MFMAs overlap the other wavefront's GELU.
// LayerNorms use all 8 wavefronts.
//
// LDS: region A holds the context rows (O projection), then the O output
// (first LayerNorm), then the two GELU chunk buffers, then the FFN output
// (second LayerNorm); region B the int8 codes of the first LayerNorm's
// output and their row scales. Row strides are padded by 16 bytes.
template <int RT, int H>
struct TailLds {
  static constexpr int BM = 32 * RT;
  static constexpr int XS = H + 8;           // halves per X / Y row
  static constexpr int QS = H + 16;          // bytes per Q8 row
  static constexpr int MS = kTailFC + 8;     // halves per GELU-chunk row
  static constexpr int FMAX = 4 * H;         // FFN widths up to 4 H
  static_assert(2 * BM * MS <= BM * XS, "two GELU chunks must fit in region A");
  uint16_t A[BM * XS];
  int8_t Q8[BM * QS];
  float rsc[BM];
  // per-feature scales and biases: O (s, b), FFN-down (s, b), FFN-up (s, b)
  float so[H], bo[H], s2[H], b2[H], s1[FMAX], b1[FMAX];
  // the two LayerNorms' gamma and beta
  float lg1[H], lb1[H], lg2[H], lb2[H];
};

// O projection of row tiles [I0, I0 + N) of the block (context rows in X)
// for the features [nb, nb + H / 4): acc[i][j] += Wo rows (nb + 32 j ..) x
// context rows (32 (I0 + i) ..), weight fragments (fragment order, 1 KB per
// load) PF K steps ahead in a ring whose first PF entries the caller primed.
template <int H, int N, int I0, int PF, int XS>
EOS_DEV void tail_o_proj(const char* wbase, uint32_t loff, const uint16_t* X, int l32, int g,
                         v8h (&wq)[PF][H / 128], v16f (&acc)[N][H / 128]) {
  constexpr int CT = H / 128, KSO = H / 16;
  auto wfrag = [&](int j, int ks) {
    return *reinterpret_cast<const v8h*>(wbase + (uint32_t)(j * KSO + ks) * 1024u + loff);
  };
#pragma unroll 1
  for (int ks0 = 0; ks0 < KSO; ks0 += PF) {
#pragma unroll
    for (int p = 0; p < PF; ++p) {
      const int ks = ks0 + p;
      v8h af[CT], bf[N];
#pragma unroll
      for (int j = 0; j < CT; ++j) af[j] = wq[p][j];
      if (ks + PF < KSO) {
#pragma unroll
        for (int j = 0; j < CT; ++j) wq[p][j] = wfrag(j, ks + PF);
      }
#pragma unroll
      for (int i = 0; i < N; ++i)
        bf[i] = *reinterpret_cast<const v8h*>(&X[(32 * (I0 + i) + l32) * XS + 16 * ks + 8 * g]);
#pragma unroll
      for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j], bf[i], acc[i][j], 0, 0, 0);
    }
  }
}

// Epilogue of row tiles [I0, I0 + N) for the features [nb, nb + H / 4), as
// the unfused residual GEMM: v = acc * s + b (one fma), v += residual,
// rounded to f16. The residual rows are in X; each element is read and
// rewritten by one lane.
template <int H, int N, int I0, int XS>
EOS_DEV void tail_epilogue(uint16_t* X, const float* sc_l, const float* bi_l, int nb, int l32,
                           int g, const v16f (&acc)[N][H / 128]) {
  constexpr int CT = H / 128;
#pragma unroll
  for (int j = 0; j < CT; ++j) {
    v4h r[N][4];
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        r[i][q] = *reinterpret_cast<const v4h*>(
            &X[(32 * (I0 + i) + l32) * XS + nb + 32 * j + 8 * q + 4 * g]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int n = nb + 32 * j + 8 * q + 4 * g;
      const float4 sc = *reinterpret_cast<const float4*>(sc_l + n);
      const float4 bi = *reinterpret_cast<const float4*>(bi_l + n);
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int m = 32 * (I0 + i) + l32;
        float v[4] = {__builtin_fmaf(acc[i][j][4 * q], sc.x, bi.x),
                      __builtin_fmaf(acc[i][j][4 * q + 1], sc.y, bi.y),
                      __builtin_fmaf(acc[i][j][4 * q + 2], sc.z, bi.z),
                      __builtin_fmaf(acc[i][j][4 * q + 3], sc.w, bi.w)};
        v4h o;
#pragma unroll
        for (int t = 0; t < 4; ++t) o[t] = (_Float16)(v[t] + (float)r[i][q][t]);
        *reinterpret_cast<v4h*>(&X[m * XS + n]) = o;
      }
    }
  }
}

// Rows m = wave + 8 k of the block through the LayerNorm, four at a time.
template <int RT, int H, typename RowFn>
EOS_DEV void tail_layer_norm(int wave, int lane, const float* gamma, const float* beta, float eps,
                             RowFn&& row_ptrs) {
  constexpr int BM = 32 * RT, NR = BM / 8 >= 4 ? 4 : BM / 8;
  static_assert((BM / 8) % NR == 0, "rows per wavefront");
  LnParams<H> p;
  ln_params<H>(gamma, beta, lane, p);
#pragma unroll 1
  for (int k0 = 0; k0 < BM / 8; k0 += NR) {
    const uint16_t* yin[NR];
    uint16_t* yout[NR];
    int8_t* q8[NR];
    float* qs[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) row_ptrs(wave + 8 * (k0 + r), yin[r], yout[r], q8[r], qs[r]);
    ln_rows<H, NR>(yin, p, eps, lane, yout, q8, qs);
  }
}

// The down and up wavefronts run separate code paths (so that neither path's
// registers are live in the other) that meet at the same sequence of
// NC + 8 workgroup barriers.
template <int RT, int H, int GELU>
EOS_DEV void tail_body(const EncTailArgs& a, TailLds<RT, H>& lds) {
  using L = TailLds<RT, H>;
  constexpr int BM = L::BM, CT = H / 128, XS = L::XS, QS = L::QS, MS = L::MS;
  constexpr int KSO = H / 16, KS1 = H / 32, KS2C = kTailFC / 16, PF = 4;
  uint16_t* const X = lds.A;  // context rows, then O output / FFN output rows
  int8_t* const Q8 = lds.Q8;
  float* const rsc = lds.rsc;
  uint16_t* const Mbuf0 = X;
  uint16_t* const Mbuf1 = X + BM * MS;

  const int rows = min(*a.rows, a.row_cap);
  const int m0 = a.row0 + (int)blockIdx.x * BM;
  if (m0 >= rows) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, l32 = lane & 31;
  const int role = wave & 3;
  const int F = a.inter, NC = F / kTailFC;

  // O projection row tiles: [0, RTD) on the down wavefronts, [RTD, RT) on
  // the up wavefronts (same features).
  constexpr int RTU = RT / 2, RTD = RT - RTU;
  const int nb = role * (H / 4);  // O / FFN-down features of this wavefront pair
  const char* const wo_base = reinterpret_cast<const char*>(a.w_o) + (size_t)(nb / 32) * KSO * 1024;
  auto prime_wo = [&](v8h (&wqo)[PF][CT]) {
#pragma unroll
    for (int p = 0; p < PF; ++p)
#pragma unroll
      for (int j = 0; j < CT; ++j)
        wqo[p][j] = *reinterpret_cast<const v8h*>(wo_base + (uint32_t)(j * KSO + p) * 1024u +
                                                  (uint32_t)lane * 16u);
  };

  // context rows -> X (rows past the matrix clamped; never stored), all
  // loads issued before any store; scales, biases and LayerNorm parameters
  // -> LDS
  static_assert(EOS_TAIL_THREADS == 512, "4 down + 4 up wavefronts");
  {
    constexpr int PER = BM * (H / 8) / EOS_TAIL_THREADS;
    static_assert(BM * (H / 8) % EOS_TAIL_THREADS == 0, "staging split");
    v4i st[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = tid + EOS_TAIL_THREADS * u;
      const int r = i / (H / 8), c = i % (H / 8);
      st[u] = *reinterpret_cast<const v4i*>(a.ctx + (size_t)min(m0 + r, a.max_rows - 1) * H + 8 * c);
    }
    // H / 4 float4 of each O / FFN-down vector (H / 4 <= 512 threads), F / 4
    // of each FFN-up vector (F <= 4 H: at most 2 per thread)
    const float4 zero4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const bool hv = tid < H / 4;
    const bool f0 = tid < F / 4, f1 = tid + EOS_TAIL_THREADS < F / 4;
    const float4 v0 = hv ? reinterpret_cast<const float4*>(a.s_o)[tid] : zero4;
    const float4 v1 = hv ? reinterpret_cast<const float4*>(a.b_o)[tid] : zero4;
    const float4 v2 = hv ? reinterpret_cast<const float4*>(a.s_2)[tid] : zero4;
    const float4 v3 = hv ? reinterpret_cast<const float4*>(a.b_2)[tid] : zero4;
    const float4 s1a = f0 ? reinterpret_cast<const float4*>(a.s_1)[tid] : zero4;
    const float4 b1a = f0 ? reinterpret_cast<const float4*>(a.b_1)[tid] : zero4;
    const float4 s1b = f1 ? reinterpret_cast<const float4*>(a.s_1)[tid + EOS_TAIL_THREADS] : zero4;
    const float4 b1b = f1 ? reinterpret_cast<const float4*>(a.b_1)[tid + EOS_TAIL_THREADS] : zero4;
    const float4 l0 = hv ? reinterpret_cast<const float4*>(a.g1)[tid] : zero4;
    const float4 l1 = hv ? reinterpret_cast<const float4*>(a.be1)[tid] : zero4;
    const float4 l2 = hv ? reinterpret_cast<const float4*>(a.g2)[tid] : zero4;
    const float4 l3 = hv ? reinterpret_cast<const float4*>(a.be2)[tid] : zero4;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int i = tid + EOS_TAIL_THREADS * u;
      const int r = i / (H / 8), c = i % (H / 8);
      *reinterpret_cast<v4i*>(&X[r * XS + 8 * c]) = st[u];
    }
    if (hv) {
      reinterpret_cast<float4*>(lds.so)[tid] = v0;
      reinterpret_cast<float4*>(lds.bo)[tid] = v1;
      reinterpret_cast<float4*>(lds.s2)[tid] = v2;
      reinterpret_cast<float4*>(lds.b2)[tid] = v3;
      reinterpret_cast<float4*>(lds.lg1)[tid] = l0;
      reinterpret_cast<float4*>(lds.lb1)[tid] = l1;
      reinterpret_cast<float4*>(lds.lg2)[tid] = l2;
      reinterpret_cast<float4*>(lds.lb2)[tid] = l3;
    }
    if (f0) {
      reinterpret_cast<float4*>(lds.s1)[tid] = s1a;
      reinterpret_cast<float4*>(lds.b1)[tid] = b1a;
    }
    if (f1) {
      reinterpret_cast<float4*>(lds.s1)[tid + EOS_TAIL_THREADS] = s1b;
      reinterpret_cast<float4*>(lds.b1)[tid + EOS_TAIL_THREADS] = b1b;
    }
  }
  __syncthreads();  // barrier 1

  // First LayerNorm (all wavefronts): f16 -> h1 (global scratch), int8
  // codes -> Q8, scales -> rsc. Rows past the matrix are normalized too
  // (stored only to h1, which has room for them).
  auto layer_norm1 = [&]() {
    tail_layer_norm<RT, H>(wave, lane, lds.lg1, lds.lb1, a.eps,
                           [&](int m, const uint16_t*& yin, uint16_t*& yout, int8_t*& q8, float*& qs) {
                             yin = &X[m * XS];
                             yout = a.h1 + (size_t)min(m0 + m, a.max_rows - 1) * H;
                             q8 = Q8 + m * QS;
                             qs = &rsc[m];
                           });
  };
  // Second LayerNorm (all wavefronts) -> the layer output rows; rows past
  // the matrix go to the clamped last row with the values that row has.
  auto layer_norm2 = [&]() {
    tail_layer_norm<RT, H>(wave, lane, lds.lg2, lds.lb2, a.eps,
                           [&](int m, const uint16_t*& yin, uint16_t*& yout, int8_t*& q8, float*& qs) {
                             const int gr = m0 + m < rows ? m0 + m : m0;  // m0 < rows
                             const bool live = m0 + m < rows;
                             yin = &X[(live ? m : 0) * XS];
                             yout = a.h + (size_t)gr * H;
                             q8 = a.h8 + (size_t)gr * H;
                             qs = a.hs + gr;
                           });
  };

  if (wave < 4) {
    // ================= down wavefront: features [nb, nb + H / 4)
    const uint32_t loff = (uint32_t)lane * 16u;
    // O projection of row tiles [0, RTD) (the up wavefronts take the rest).
    {
      v16f acco[RTD][CT];
#pragma unroll
      for (int i = 0; i < RTD; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j) acco[i][j] = v16f{0};
      v8h wqo[PF][CT];
      prime_wo(wqo);
      // The down wavefront has RTD of the RT row tiles (the up wavefront on
      // its SIMD the rest): it paces the O projection, so it runs it at a
      // raised wave priority.
      __builtin_amdgcn_s_setprio(2);
      tail_o_proj<H, RTD, 0, PF, XS>(wo_base, loff, X, l32, g, wqo, acco);
      __builtin_amdgcn_s_setprio(0);
      __syncthreads();  // barrier 2: every context read done
      __syncthreads();  // barrier 3: the residual rows are in X
      tail_epilogue<H, RTD, 0, XS>(X, lds.so, lds.bo, nb, l32, g, acco);
    }
    v16f acc[RT][CT];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < CT; ++j) acc[i][j] = v16f{0};
    // W2 fragments PF K steps ahead, the ring running on across chunks
    // (primed here, so the first ones land during the first LayerNorm).
    const int KS2 = F / 16;
    const char* const w2base = reinterpret_cast<const char*>(a.w_2) + (size_t)(nb / 32) * KS2 * 1024;
    auto w2frag = [&](int j, int ks) {
      return *reinterpret_cast<const v8h*>(w2base + (uint32_t)(j * KS2 + ks) * 1024u + loff);
    };
    static_assert(KS2C % PF == 0, "the W2 ring slot of a K step is its index within the chunk");
    v8h wq[PF][CT];
#pragma unroll
    for (int p = 0; p < PF; ++p)
#pragma unroll
      for (int j = 0; j < CT; ++j) wq[p][j] = w2frag(j, p);
    __syncthreads();  // barrier 4
    layer_norm1();
    __syncthreads();  // barrier 5: X free, it now holds the two GELU chunk buffers
    __syncthreads();  // barrier 6: chunk 0 written by the up wavefronts
#pragma unroll 1
    for (int c = 0; c < NC; ++c) {
      // acc[i][j] += W2 rows (nb + 32 j ..)[chunk c] x the chunk's rows
      const uint16_t* M = (c & 1) ? Mbuf1 : Mbuf0;
      const int ks0 = c * KS2C;
#pragma unroll
      for (int kk = 0; kk < KS2C; ++kk) {
        v8h af[CT], bf[RT];
#pragma unroll
        for (int j = 0; j < CT; ++j) af[j] = wq[kk % PF][j];
        if (ks0 + kk + PF < KS2) {
#pragma unroll
          for (int j = 0; j < CT; ++j) wq[kk % PF][j] = w2frag(j, ks0 + kk + PF);
        }
#pragma unroll
        for (int i = 0; i < RT; ++i)
          bf[i] = *reinterpret_cast<const v8h*>(&M[(32 * i + l32) * MS + 16 * kk + 8 * g]);
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int j = 0; j < CT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[j], bf[i], acc[i][j], 0, 0, 0);
      }
      __syncthreads();  // barriers 7 .. NC + 6: chunk c consumed, chunk c + 1 written
    }
    __syncthreads();  // barrier NC + 7: the first LayerNorm's output rows are in X
    tail_epilogue<H, RT, 0, XS>(X, lds.s2, lds.b2, nb, l32, g, acc);
    __syncthreads();  // barrier NC + 8
    layer_norm2();
  } else {
    // ================= up wavefront: features [32 role, + 32) of each chunk
    // W1 fragments of chunk c, requested a chunk ahead.
    v4i w1f[KS1];
    auto load_w1 = [&](int c) {
      const char* base = reinterpret_cast<const char*>(a.w_1) +
                         (size_t)(c * (kTailFC / 32) + role) * KS1 * 1024;
      const uint32_t loff = (uint32_t)lane * 16u;
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks)
        w1f[ks] = *reinterpret_cast<const v4i*>(base + (uint32_t)ks * 1024u + loff);
    };
    // The up wavefront paces the chunk pipeline (its MFMAs, then the GELU of
    // their results, while the down wavefront on the same SIMD has the
    // chunk before). It runs each chunk at a raised wave priority, so that
    // its MFMAs issue ahead of the down wavefront's and the down
    // wavefront's MFMAs fill the time of the GELU instead (c3 tail chunk
    // loop 103k -> 85k cycles per block).
    auto up_chunk = [&](int c) {
      const int c0 = c * kTailFC;
      v16i up[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) up[i] = v16i{0};
      __builtin_amdgcn_s_setprio(2);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < KS1; ++ks) {
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const v4i bf = *reinterpret_cast<const v4i*>(Q8 + (32 * i + l32) * QS + 32 * ks + 16 * g);
          up[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w1f[ks], bf, up[i], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (c + 1 < NC) load_w1(c + 1);  // lands behind the GELU and the barrier
      // bias + GELU: v = (float)acc * (s * rs) + b (one fma)
      uint16_t* M = (c & 1) ? Mbuf1 : Mbuf0;
      float rs[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) rs[i] = rsc[32 * i + l32];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = 32 * role + 8 * q + 4 * g;  // within the chunk
        const float4 sc = *reinterpret_cast<const float4*>(lds.s1 + c0 + n);
        const float4 bi = *reinterpret_cast<const float4*>(lds.b1 + c0 + n);
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const int m = 32 * i + l32;
          float v[4] = {__builtin_fmaf((float)up[i][4 * q], sc.x * rs[i], bi.x),
                        __builtin_fmaf((float)up[i][4 * q + 1], sc.y * rs[i], bi.y),
                        __builtin_fmaf((float)up[i][4 * q + 2], sc.z * rs[i], bi.z),
                        __builtin_fmaf((float)up[i][4 * q + 3], sc.w * rs[i], bi.w)};
          v4h o;
#pragma unroll
          for (int t = 0; t < 4; ++t)
            o[t] = (_Float16)(GELU == 1 ? gelu_erf_fast(v[t]) : gelu(v[t], 2));
          *reinterpret_cast<v4h*>(&M[m * MS + n]) = o;
        }
      }
      __builtin_amdgcn_s_setprio(0);
    };
    // Residual rows for the down wavefronts' epilogues, requested while they
    // compute (the O projection; the last FFN chunk) and then copied into X.
    constexpr int RPER = BM * (H / 8) / 256;
    static_assert(BM * (H / 8) % 256 == 0, "residual split");
    const int ut = tid - 256;
    v4i res[RPER];
    auto load_rows = [&](const uint16_t* src) {
#pragma unroll
      for (int u = 0; u < RPER; ++u) {
        const int i = ut + 256 * u;
        const int r = i / (H / 8), c = i % (H / 8);
        res[u] = *reinterpret_cast<const v4i*>(src + (size_t)min(m0 + r, a.max_rows - 1) * H + 8 * c);
      }
    };
    auto store_rows = [&]() {
#pragma unroll
      for (int u = 0; u < RPER; ++u) {
        const int i = ut + 256 * u;
        const int r = i / (H / 8), c = i % (H / 8);
        *reinterpret_cast<v4i*>(&X[r * XS + 8 * c]) = res[u];
      }
    };
    load_rows(a.h);
    if constexpr (RTU > 0) {
      v16f acco[RTU][CT];
#pragma unroll
      for (int i = 0; i < RTU; ++i)
#pragma unroll
        for (int j = 0; j < CT; ++j) acco[i][j] = v16f{0};
      v8h wqo[PF][CT];
      prime_wo(wqo);
      tail_o_proj<H, RTU, RTD, PF, XS>(wo_base, (uint32_t)lane * 16u, X, l32, g, wqo, acco);
      __syncthreads();  // barrier 2: every context read done
      store_rows();
      __syncthreads();  // barrier 3
      tail_epilogue<H, RTU, RTD, XS>(X, lds.so, lds.bo, nb, l32, g, acco);
    } else {
      __syncthreads();  // barrier 2: every context read done
      store_rows();
      __syncthreads();  // barrier 3
    }
    load_w1(0);  // lands during the first LayerNorm
    __syncthreads();  // barrier 4
    layer_norm1();
    __syncthreads();  // barrier 5
    up_chunk(0);
    __syncthreads();  // barrier 6
#pragma unroll 1
    for (int c = 0; c + 1 < NC; ++c) {
      up_chunk(c + 1);
      __syncthreads();  // barriers 7 .. NC + 5
    }
    load_rows(a.h1);  // written by the first LayerNorm before barrier 5
    __syncthreads();  // barrier NC + 6: the last chunk consumed
    store_rows();
    __syncthreads();  // barrier NC + 7
    __syncthreads();  // barrier NC + 8
    layer_norm2();
  }
}

}  // namespace

#define EOS_TAIL_KERNEL(RT, H, G)                                                       \
  extern "C" __global__ __launch_bounds__(EOS_TAIL_THREADS) void                          \
      eos_enc_tail_r##RT##_h##H##_g##G(                                                    \
      EncTailArgs a) {                                                                     \
    __shared__ __attribute__((aligned(16))) TailLds<RT, H> lds;                           \
    tail_body<RT, H, G>(a, lds);                                                         \
  }
EOS_TAIL_KERNEL(3, 384, 1)
EOS_TAIL_KERNEL(3, 384, 2)
EOS_TAIL_KERNEL(2, 512, 1)
EOS_TAIL_KERNEL(2, 512, 2)
EOS_TAIL_KERNEL(1, 512, 1)
EOS_TAIL_KERNEL(1, 512, 2)
EOS_TAIL_KERNEL(1, 768, 1)
EOS_TAIL_KERNEL(1, 768, 2)
#undef EOS_TAIL_KERNEL

// --------------------------------------------------------------- attention

// Flash-style attention in transposed form: each wavefront owns 32 queries of
// one (sequence, head); per block of 32 keys it computes S^T = K Q^T (keys x
// queries, so each lane owns one query column and its softmax state), masks
// keys past the sequence, updates the running max / sum in f32 (exp2 domain),
// and accumulates O^T += V^T P^T on MFMA. P^T is fed straight from the S^T
// registers: the K order of that MFMA is the row order the S^T accumulator
// already has, and the V^T fragment is gathered in the same order.
template <int HD, int KB, bool FOLD = false, int NW = 4>
EOS_DEV void attn_body(const EncAttnArgs& a) {
  static_assert(KB == 32 || KB == 64, "keys per block");
  constexpr int KC = KB / 8;             // 8-key chunks of a V^T row per block
  constexpr int NT = KB / 32;            // 32-key S^T tiles per block
  constexpr int QW = 32;                 // queries per wavefront
  constexpr int NCH = KB * HD / 8;       // 8-half chunks of K (and of V^T) per block
  constexpr int NTHR = 64 * NW;          // threads (NW wavefronts of 32 queries)
  constexpr int CPT = (NCH + NTHR - 1) / NTHR; // chunks per thread
  __shared__ __attribute__((aligned(16))) uint16_t ks[2][KB * (HD + 8)];
  __shared__ __attribute__((aligned(16))) uint16_t vt[2][HD * (KB + 8)];
  // Per-wavefront output staging (head dims up to 64): the K buffers when
  // they are large enough (free once the key loop is done), else its own.
  constexpr bool kStageInK = 2 * KB * (HD + 8) >= NW * 32 * (HD + 8);
  __shared__ __attribute__((aligned(16)))
  uint16_t ostage[(HD <= 64 && !kStageInK) ? NW * 32 * (HD + 8) : 8];
  const int b = a.order != nullptr ? a.order[blockIdx.z] : blockIdx.z, h = blockIdx.y;
  const int cnt = a.seq_cnt[b];                          // keys
  const int qcnt = a.seq_q != nullptr ? a.seq_q[b] : cnt;  // query rows (>= cnt)
  const int q0 = blockIdx.x * (NW * QW);
  if (q0 >= qcnt) return;
  const int off = a.seq_off[b];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, l32 = lane & 31;
  const int ld = 3 * a.hidden;
  const int qi = q0 + wave * QW + l32;           // this lane's query (column)
  const bool qlive = qi < qcnt;
  const bool wlive = q0 + wave * QW < qcnt;      // wave-uniform
  // Q^T fragments (B operand): lane (query l32, group g) holds q[16s + 8g .. +7].
  // Q is pre-scaled by log2(e) / sqrt(hd) (in f32, rounded once to f16), so
  // the scores come out in the exp2 domain.
  v8h qf[HD / 16];
  {
    const uint16_t* qrow = a.qkv + (size_t)(off + (qlive ? qi : 0)) * ld + h * HD;
#pragma unroll
    for (int s = 0; s < HD / 16; ++s) {
      const v8h raw = *reinterpret_cast<const v8h*>(qrow + s * 16 + g * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[s][e] = (_Float16)((float)raw[e] * a.scale_log2);
    }
  }
  v16f o[HD / 32];
#pragma unroll
  for (int t = 0; t < HD / 32; ++t) o[t] = v16f{0};
  float mrun = -__builtin_inff(), lrun = 0.f;
  // FOLD: the exponent reference enters the S MFMAs as their accumulator
  // input (negm = -mrun in every element, 0 before the first block), so the
  // scores come out already shifted and the common path subtracts nothing;
  // sref is the reference they carry.
  v16f negm = v16f{0};
  float sref = 0.f;
  // K [key][HD] and V^T [HD][key] of a 32-key block are staged in LDS from
  // registers; the next block's rows are requested before the current
  // block's MFMAs (double-buffered, one barrier per block).
  // V^T comes from the feature-major copy the QKV GEMM wrote: chunk idx of a
  // block is feature d = idx / KC, keys 8 (idx % KC) .. + 7 (16 bytes). Keys
  // past the sequence (probability 0) read its pad rows, the next sequence or
  // vt's zeroed tail: all finite, since every row the GEMMs read was written
  // in this forward (pad rows of ctx included, below), and 0 * finite = 0.
  v4i kreg[CPT], vreg[CPT];
  auto kv_load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int idx = tid + NTHR * u;
      if (idx < NCH) {
        const int kr = idx / (HD / 8), c = (idx % (HD / 8)) * 8;
        // Clamped to the sequence's rows (row 0 when it has no key: then the
        // block is never multiplied, and row 0 is its query-only row).
        const int key = max(min(k0 + kr, cnt - 1), 0);
        kreg[u] = *reinterpret_cast<const v4i*>(a.qkv + (size_t)(off + key) * ld + a.hidden +
                                                h * HD + c);
        const int d = idx / KC, k8 = (idx % KC) * 8;
        vreg[u] = *reinterpret_cast<const v4i*>(a.vt + (size_t)(h * HD + d) * a.vt_ld + off + k0 + k8);
      }
    }
  };
  auto kv_store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < CPT; ++u) {
      const int idx = tid + NTHR * u;
      if (idx < NCH) {
        const int kr = idx / (HD / 8), c = (idx % (HD / 8)) * 8;
        *reinterpret_cast<v4i*>(&ks[buf][kr * (HD + 8) + c]) = kreg[u];
        // Key k = 16 st + 8 hh + 4 gg + j is stored at 16 st + 8 gg + 4 hh + j,
        // so the 8 keys a lane's P fragment covers are 16 contiguous bytes:
        // the two 4-key halves of this chunk go to positions 8 and 4 apart.
        const int d = idx / KC, k8 = (idx % KC) * 8;
        const int p0 = (k8 & ~15) | ((k8 & 8) >> 1);  // keys k8 .. k8 + 3
        uint16_t* vrow = &vt[buf][d * (KB + 8)];
        const v4i v = vreg[u];
        *reinterpret_cast<uint2*>(vrow + p0) = make_uint2((uint32_t)v.x, (uint32_t)v.y);
        *reinterpret_cast<uint2*>(vrow + p0 + 8) = make_uint2((uint32_t)v.z, (uint32_t)v.w);
      }
    }
  };
  kv_load(0);
  kv_store(0);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < cnt; k0 += KB, buf ^= 1) {
    const bool more = k0 + KB < cnt;
    if (more) kv_load(k0 + KB);
    // A wavefront whose 32 queries all lie past the sequence only helps stage
    // K and V (its outputs are the zero pad rows).
    if (wlive) {
    // S^T, NT tiles of 32 keys x 32 queries
    v16f s[NT];
#pragma unroll
    for (int hh = 0; hh < NT; ++hh) {
#pragma unroll
      for (int st = 0; st < HD / 16; ++st) {
        const v8h kf = *reinterpret_cast<const v8h*>(
            &ks[buf][(32 * hh + l32) * (HD + 8) + st * 16 + g * 8]);
        s[hh] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
            kf, qf[st], st == 0 ? (FOLD ? negm : v16f{0}) : s[hh], 0, 0, 0);
      }
    }
    // element e of tile hh is key k0 + 32 hh + 8(e/4) + 4g + e%4; only the
    // last block of the sequence has keys past its end (masked to -inf).
    if (k0 + KB > cnt) {
#pragma unroll
      for (int hh = 0; hh < NT; ++hh)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int key = k0 + 32 * hh + 8 * (e >> 2) + 4 * g + (e & 3);
          s[hh][e] = key < cnt ? s[hh][e] : -__builtin_inff();
        }
    }
    // Lazy rescaling: the exponentials are taken against a per-query reference
    // mrun that moves only when needed, and o, lrun are rescaled only then (the
    // quotient o / lrun is the same for any reference). A block is accepted
    // when every lane's sum of its 16 NT p stays <= kSafe, so every p fits f16 and
    // no f32 sum can overflow; otherwise (the first block, where mrun = -inf
    // gives inf or NaN, or a score above mrun + 12) the reference of that
    // query moves to the block's maximum, o and lrun are rescaled and the p
    // recomputed. With the first block's maximum as reference later blocks
    // almost never move it, where an exact running maximum grows in a large
    // share of the blocks of a long sequence, and the common path needs no
    // maximum at all. The two lanes of a query (g = 0, 1) hold different keys
    // and move their reference together; lrun is each lane's own partial sum
    // (both are rescaled alike), added at the end.
    constexpr float kSafe = 4096.0f;
    float psum;
    v8h pf[2 * NT];
    auto exps = [&](float shift) {
      psum = 0.f;
#pragma unroll
      for (int hh = 0; hh < NT; ++hh)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          // v_exp_f32 directly: masked keys give exp2(-inf) = 0.
          const float p = __builtin_amdgcn_exp2f(FOLD ? s[hh][e] : s[hh][e] - shift);
          pf[2 * hh + (e >> 3)][e & 7] = (_Float16)p;
        }
      // The row sum is taken over the f16 p the PV MFMAs multiply, two per
      // v_dot2_f32_f16 against (1, 1) with f32 accumulation: half the
      // instructions of adding the f32 p, and the weights of o / lrun sum to
      // one exactly as rounded. A p past the f16 range gives inf (NaN stays
      // NaN), which fails the kSafe test below like the f32 sum would.
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
      for (int j = 0; j < 2 * NT; ++j)
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const h2 pp = {pf[j][e], pf[j][e + 1]};
          psum = __builtin_amdgcn_fdot2(pp, ones, psum, false);
        }
    };
    exps(mrun);
    // FOLD: the first block always moves the reference (its scores carry
    // none yet).
    const bool over = !(psum <= kSafe) || (FOLD && mrun == -__builtin_inff());
    if (__ballot(over) != 0ull) {
      if (a.moves != nullptr && k0 > 0 && lane == 0) atomicAdd(a.moves, 1);
      float mloc = -__builtin_inff();
#pragma unroll
      for (int hh = 0; hh < NT; ++hh)
#pragma unroll
        for (int e = 0; e < 16; ++e) mloc = fmaxf(mloc, s[hh][e]);
      if (FOLD) mloc += sref;  // the block's raw maximum (or -inf)
      const float mpair = fmaxf(mloc, __shfl_xor(mloc, 32));
      // Both shuffles run with every lane active: a shuffle inside the
      // short-circuit of `over || ...` would run only in the lanes that are
      // not over and read 0 from the disabled partner, so a pair where only
      // one lane overflows would move one lane and not the other.
      const int over_pair = (over ? 1 : 0) | __shfl_xor(over ? 1 : 0, 32);
      const bool pover = over_pair != 0;
      const float mnew = pover ? fmaxf(mpair, mrun) : mrun;
      // v_exp_f32 directly: the argument is <= 0 or -inf (exp2 -> 0).
      const float corr = __builtin_amdgcn_exp2f(mrun - mnew);
      lrun *= corr;
#pragma unroll
      for (int t = 0; t < HD / 32; ++t) {
#pragma unroll
        for (int e = 0; e < 16; ++e) o[t][e] *= corr;
      }
      mrun = mnew;
      if constexpr (FOLD) {
        // Re-reference this block's scores to mnew, and the next blocks'.
        const float d = mnew == -__builtin_inff() ? 0.f : mnew - sref;
#pragma unroll
        for (int hh = 0; hh < NT; ++hh)
#pragma unroll
          for (int e = 0; e < 16; ++e) s[hh][e] -= d;
        sref += d;
#pragma unroll
        for (int e = 0; e < 16; ++e) negm[e] = -sref;
      }
      exps(mrun);  // now every score - mrun <= 0 for the moved queries
    }
    lrun += psum;
    // O^T += V^T P^T. K step st covers the keys this lane's P holds for
    // tile st / 2, e in [8 (st % 2), + 8): keys 16 st + {4g..4g+3} and
    // 16 st + 8 + {4g..4g+3} of the block.
#pragma unroll
    for (int t = 0; t < HD / 32; ++t) {
      const int d = t * 32 + l32;
#pragma unroll
      for (int st = 0; st < 2 * NT; ++st) {
        const v8h vf = *reinterpret_cast<const v8h*>(&vt[buf][d * (KB + 8) + 16 * st + 8 * g]);
        o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[st], o[t], 0, 0, 0);
      }
    }
    }  // wlive
    // The other buffer was last read before the previous barrier.
    if (more) kv_store(buf ^ 1);
    __syncthreads();
  }
  const float lsum = lrun + __shfl_xor(lrun, 32);  // before any lane leaves
  if constexpr (HD <= 64) {
    // The wavefront's 32 output rows go through LDS and leave as whole row
    // segments (HD halves each) in 16-byte stores; rows of the sequence's
    // 8-row slot past its end get zeros (no kernel writes them otherwise,
    // and a NaN left there by a freed buffer would reach the next layer's V
    // rows past the sequence). Storing the MFMA layout directly scattered
    // each store over 32 rows.
    constexpr int OS = HD + 8;  // halves per staged row
    uint16_t* const os = (kStageInK ? &ks[0][0] : ostage) + wave * 32 * OS;
    const float inv = (qlive && lsum > 0.f) ? 1.0f / lsum : 0.f;
#pragma unroll
    for (int t = 0; t < HD / 32; ++t) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v4h v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (_Float16)(o[t][4 * q + j] * inv);
        *reinterpret_cast<v4h*>(&os[l32 * OS + t * 32 + 8 * q + 4 * g]) = v;
      }
    }
    __builtin_amdgcn_wave_barrier();
    constexpr int LPR = HD / 8;       // lanes per row (16 bytes each)
    constexpr int RPI = 64 / LPR;     // rows per store instruction
    const int slot = (qcnt + 7) & ~7;  // the sequence's rows, pad rows included
#pragma unroll
    for (int r0 = 0; r0 < 32; r0 += RPI) {
      const int r = r0 + lane / LPR, c = (lane % LPR) * 8;
      const int qr = q0 + wave * QW + r;
      if (qr < slot)
        *reinterpret_cast<v4i*>(a.ctx + (size_t)(off + qr) * a.hidden + h * HD + c) =
            *reinterpret_cast<const v4i*>(&os[r * OS + c]);
    }
    return;
  }
  if (!qlive) {
    // Pad rows of the sequence's 8-row slot get zeros: no kernel writes them
    // otherwise, and the memory may hold anything a freed buffer left (a NaN
    // there would reach the next layer's V rows past the sequence).
    if (qi < ((qcnt + 7) & ~7)) {
      uint16_t* prow = a.ctx + (size_t)(off + qi) * a.hidden + h * HD;
#pragma unroll
      for (int t = 0; t < HD / 32; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<v4h*>(prow + t * 32 + 8 * q + 4 * g) = v4h{0, 0, 0, 0};
    }
    return;
  }
  const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
  uint16_t* orow = a.ctx + (size_t)(off + qi) * a.hidden + h * HD;
  // Elements 4q .. 4q + 3 are the 4 consecutive features 8q + 4g .. + 3: one
  // 8-byte store each.
#pragma unroll
  for (int t = 0; t < HD / 32; ++t) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v4h v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = (_Float16)(o[t][4 * q + j] * inv);
      *reinterpret_cast<v4h*>(orow + t * 32 + 8 * q + 4 * g) = v;
    }
  }
}

// A register budget of at most 256 VGPRs (here: at least 3 or 2 waves per
// SIMD) makes the compiler use the MFMA forms that accumulate in ordinary
// VGPRs. With the 512-register budget of one wave per SIMD it picks the
// accumulation-register forms and copies S and O between the two register
// files in every key block (about 110 extra VALU moves per block at hd 64).
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void eos_enc_attn_hd32(EncAttnArgs a) {
  attn_body<32, 32, true>(a);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void eos_enc_attn_hd64(EncAttnArgs a) {
  attn_body<64, 64, true>(a);
}
// Head dim 64 over long sequences: twelve wavefronts (384 queries) per
// workgroup, one workgroup per CU, so each K/V block is staged once per CU
// for 384 queries instead of once per 128 (three 4-wavefront workgroups):
// the loads and the wait for them were 60 % of a block's time (per-wavefront
// phase timestamps), bound by the L1 misses a CU keeps in flight.
extern "C" __global__ __launch_bounds__(768) __attribute__((amdgpu_waves_per_eu(3)))
void eos_enc_attn_hd64_w12(EncAttnArgs a) {
  attn_body<64, 64, true, 12>(a);
}
extern "C" __global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void eos_enc_attn_hd128(EncAttnArgs a) {
  attn_body<128, 32>(a);
}
// Head dim 256 (the single-head compact graphs at D = 256): the O^T
// accumulator alone is 128 registers and the Q^T fragments 64, so this one
// keeps the one-wave-per-SIMD budget.
extern "C" __global__ __launch_bounds__(256) void eos_enc_attn_hd256(EncAttnArgs a) {
  attn_body<256, 32>(a);
}

// ------------------------------------------------------------------- pool

// Partial sums of the masked mean pool: workgroup (c, b) sums rows
// [64 c, 64 c + 64) of sequence b (mode 1 normalizes each row first:
// x / ||x||, rows of norm 0 kept) into part[b][c][hidden] (f32). Each lane
// covers 8 consecutive columns per 16-byte load (hidden <= 1024: up to two
// 512-column segments); wavefront w sums rows w, w + 4, ... with 8 rows'
// loads in flight, and the 4 wavefront sums are added in wavefront order.
extern "C" __global__ __launch_bounds__(256) void eos_enc_pool_part(EncPoolArgs a) {
  constexpr int kRows = 8;
  __shared__ float wsum[4][1024];
  const int c = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int off = a.seq_off[b], cnt = a.seq_cnt[b];
  const int r_begin = c * kPoolChunk;
  if (r_begin >= cnt && c > 0) return;
  const int r_end = min(r_begin + kPoolChunk, cnt);
  float s[2][8];
#pragma unroll
  for (int gg = 0; gg < 2; ++gg)
#pragma unroll
    for (int e = 0; e < 8; ++e) s[gg][e] = 0.f;
  for (int r0 = r_begin + w * kRows; r0 < r_end; r0 += 4 * kRows) {
    v4i v[kRows][2];
    // Loads from clamped columns, zeroed afterwards (see eos_enc_embed).
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      const int r = min(r0 + u, r_end - 1);
      const uint16_t* row = a.h + (size_t)(off + r) * a.hidden;
#pragma unroll
      for (int gg = 0; gg < 2; ++gg)
        v[u][gg] = *reinterpret_cast<const v4i*>(row + min(gg * 512 + lane * 8, a.hidden - 8));
    }
#pragma unroll
    for (int u = 0; u < kRows; ++u)
#pragma unroll
      for (int gg = 0; gg < 2; ++gg)
        if (gg * 512 + lane * 8 >= a.hidden) v[u][gg] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int u = 0; u < kRows; ++u) {
      float x[2][8];
      float q = 0.f;
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const v8h hv = __builtin_bit_cast(v8h, v[u][gg]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          x[gg][e] = (float)hv[e];
          q += x[gg][e] * x[gg][e];
        }
      }
      float scale = 1.0f;
      if (a.mode == 1) {
        const float norm = sqrtf(wave_sum(q));
        scale = norm > 0.f ? norm : 1.0f;
      }
      if (r0 + u < r_end && (a.mask == nullptr || a.mask[(size_t)b * a.tokens + r0 + u] != 0)) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg)
#pragma unroll
          for (int e = 0; e < 8; ++e) s[gg][e] += a.mode == 1 ? x[gg][e] / scale : x[gg][e];
      }
    }
  }
#pragma unroll
  for (int gg = 0; gg < 2; ++gg) {
    const int col = gg * 512 + lane * 8;
    if (col < a.hidden) {
#pragma unroll
      for (int e = 0; e < 8; ++e) wsum[w][col + e] = s[gg][e];
    }
  }
  __syncthreads();
  float* dst = a.part + ((size_t)b * a.nchunk + c) * a.hidden;
  for (int col = tid; col < a.hidden; col += 256)
    dst[col] = ((wsum[0][col] + wsum[1][col]) + wsum[2][col]) + wsum[3][col];
}

// Pool finalize, one workgroup per sequence: the chunk partials added in
// chunk order, times 1/count (count 0 -> zeros). mode 0 (BERT,
// bert_embedder_ops.go:179-192): then L2 normalize (norm 0 kept). mode 1
// (compact family, models/default_embedding.go:496-505): the rows were
// normalized before pooling; then the optional output projection
// (pool(X) P equals pool(X P) up to f32 rounding, at 1/count of the work).
extern "C" __global__ __launch_bounds__(1024) void eos_enc_pool(EncPoolArgs a) {
  __shared__ float pooled[1024];
  __shared__ float red[16];
  const int b = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  __shared__ int mcount[16];
  const int cnt = a.seq_cnt[b];
  const int nc = cnt > 0 ? (cnt + kPoolChunk - 1) / kPoolChunk : 0;
  // Pooled rows: all of the sequence's rows, or those whose mask is set.
  int pooled_rows = cnt;
  if (a.mask != nullptr) {
    // Eight mask words per thread requested at a time (one memory round trip
    // per 8192 tokens instead of one per 1024).
    int mine = 0;
    for (int t0 = tid; t0 < a.tokens; t0 += 8 * 1024) {
      int mv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) mv[i] = a.mask[(size_t)b * a.tokens + min(t0 + 1024 * i, a.tokens - 1)];
#pragma unroll
      for (int i = 0; i < 8; ++i) mine += (t0 + 1024 * i < a.tokens && mv[i] != 0) ? 1 : 0;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mine += __shfl_xor(mine, o);
    if (lane == 0) mcount[w] = mine;
    __syncthreads();
    pooled_rows = 0;
    for (int i = 0; i < 16; ++i) pooled_rows += mcount[i];
  }
  float v = 0.f;
  if (a.cls_seq_q != nullptr) {
    // CLS pooling (clsPoolTensor, bert_embedder_ops.go:183-196): position
    // 0's row, then the L2 normalization below.
    const int row = a.seq_off[b] + (a.cls_seq_q[b] > cnt ? cnt : 0);
    if (tid < a.hidden) v = (float)__builtin_bit_cast(_Float16, a.h[(size_t)row * a.hidden + tid]);
  } else if (tid < a.hidden) {
    // Up to 32 chunk partials requested at a time, then added in chunk order
    // (the same sum as one load and add per chunk, without a memory round
    // trip per chunk).
    const float* src = a.part + (size_t)b * a.nchunk * a.hidden + tid;
    for (int c0 = 0; c0 < nc; c0 += 32) {
      const int m = min(32, nc - c0);
      float pv[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) pv[i] = src[(size_t)(c0 + min(i, m - 1)) * a.hidden];
#pragma unroll
      for (int i = 0; i < 32; ++i)
        if (i < m) v += pv[i];
    }
    v = pooled_rows > 0 ? v * (1.0f / (float)pooled_rows) : 0.f;
  }
  if (a.mode == 1) {
    if (a.proj == nullptr) {
      if (tid < a.hidden) a.out[(size_t)b * a.hidden + tid] = v;
      return;
    }
    if (tid < a.hidden) pooled[tid] = v;
    __syncthreads();
    for (int o = tid; o < a.odim; o += 1024) {
      float acc = 0.f;
      for (int d = 0; d < a.hidden; ++d) acc += pooled[d] * a.proj[(size_t)d * a.odim + o];
      a.out[(size_t)b * a.odim + o] = acc;
    }
    return;
  }
  const float ss = wave_sum(tid < a.hidden ? v * v : 0.f);
  if (lane == 0) red[w] = ss;
  __syncthreads();
  float tot = 0.f;
  for (int i = 0; i < 16; ++i) tot += red[i];
  const float norm = sqrtf(tot);
  if (tid < a.hidden) a.out[(size_t)b * a.hidden + tid] = norm > 0.f ? v / norm : v;
}

// ------------------------------------------------------------- tiny embed

// The same pipeline for kTinyTok tokens per workgroup when edim is 64, 128
// or 256 and the projection fits LDS: the f16 projection is staged once per
// workgroup (16-byte loads, several in flight per thread), the gathered rows
// are held transposed (xs[k][token]) in f32, and each of the kTinyTok * edim
// threads runs the k-ascending chain of one (token, output) pair (the
// reference's order: one product, then one sum, per k); two or more
// wavefronts per SIMD hide the LDS latency of the chains. The f64 sum of squares uses fma(v, v, ss): v * v of an f32 value is
// exact in f64, so this is the reference's multiply-then-add bit for bit.
// Dynamic LDS: dim * edim halves + dim * kTinyTok + kTinyTok * edim floats.
constexpr int kTinyTok = 4;
template <int EDIM>
EOS_DEV void embed_tiny_lds(const EmbedTinyArgs& a) {
  constexpr int NT = kTinyTok * EDIM;  // threads
  extern __shared__ __attribute__((aligned(16))) unsigned char tiny_lds[];
  uint16_t* pw = reinterpret_cast<uint16_t*>(tiny_lds);
  float* xs = reinterpret_cast<float*>(tiny_lds + (size_t)a.dim * a.edim * 2);
  float* ys = xs + (size_t)a.dim * kTinyTok;
  __shared__ float nrm[kTinyTok];
  __shared__ int toks[kTinyTok];
  const int tid = threadIdx.x;
  const int t0 = blockIdx.x * kTinyTok;
  if (tid < kTinyTok) {
    int tok = t0 + tid < a.n ? a.tokens[t0 + tid] : -1;
    if (t0 + tid < a.n && (tok < 0 || tok >= a.vocab)) {
      *a.status = 1;
      tok = 0;
    }
    toks[tid] = tok;
  }
  // projection: [dim][edim] halves, 8 per 16-byte load, 8 loads of each
  // thread in flight before any is stored (a load-store-load loop would wait
  // one memory latency per load)
  const int nvec = a.dim * a.edim / 8;
  for (int base = tid; base < nvec; base += NT * 8) {
    v4i buf[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + NT * u;
      buf[u] = i < nvec ? reinterpret_cast<const v4i*>(a.proj)[i] : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = base + NT * u;
      if (i < nvec) reinterpret_cast<v4i*>(pw)[i] = buf[u];
    }
  }
  __syncthreads();
  // the rows, 8 halves per 16-byte load (dim % 8 == 0), stored transposed
  const int cpr = a.dim / 8, nch = kTinyTok * cpr;
  for (int i = tid; i < nch; i += NT) {
    const int t = i / cpr, c = i - t * cpr;
    const int tok = toks[t];
    const v4i raw = tok >= 0 ? *reinterpret_cast<const v4i*>(a.table + (size_t)tok * a.dim + 8 * c)
                             : v4i{0, 0, 0, 0};
    const v8h h = __builtin_bit_cast(v8h, raw);
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[(8 * c + e) * kTinyTok + t] = (float)h[e];
  }
  __syncthreads();
  {
    const int e = tid % EDIM, t = tid / EDIM;
    float acc = 0.0f;
#pragma unroll 8
    for (int k = 0; k < a.dim; ++k) {
      const float p = xs[k * kTinyTok + t] * h2f(pw[k * EDIM + e]);
      acc = acc + p;
    }
    ys[t * EDIM + e] = acc;
  }
  __syncthreads();
  if (tid < kTinyTok) {
    double ss = 0.0;
#pragma unroll 8
    for (int c = 0; c < EDIM; ++c) {
      const double v = (double)ys[tid * EDIM + c];
      ss = __builtin_fma(v, v, ss);
    }
    nrm[tid] = (float)sqrt(ss);
  }
  __syncthreads();
  for (int i = tid; i < kTinyTok * EDIM; i += NT) {
    const int t = i / EDIM, c = i - t * EDIM;
    if (t0 + t >= a.n) continue;
    const float v = ys[i], nv = nrm[t];
    a.out[(size_t)(t0 + t) * EDIM + c] = f2h(nv == 0.0f ? v : v / nv);
  }
}

extern "C" __global__ __launch_bounds__(kTinyTok * 64) void eos_embed_tiny_e64(EmbedTinyArgs a) {
  embed_tiny_lds<64>(a);
}
extern "C" __global__ __launch_bounds__(kTinyTok * 128) void eos_embed_tiny_e128(EmbedTinyArgs a) {
  embed_tiny_lds<128>(a);
}
extern "C" __global__ __launch_bounds__(kTinyTok * 256) void eos_embed_tiny_e256(EmbedTinyArgs a) {
  embed_tiny_lds<256>(a);
}

// examples/embed.eos on one wavefront per token: gather (tensor_ops.go:
// 938-1166), f32 matmul with k ascending and separate multiply / add
// (matmulTensor, tensor_ops.go:1168-1249), then normalizeRows
// (tensor_ops.go:1367-1391): f64 sum of squares in column order, f32 norm,
// rows of norm 0 unchanged; stored as f16.
extern "C" __global__ __launch_bounds__(256) void eos_embed_tiny(EmbedTinyArgs a) {
  __shared__ float xs[4][1024];
  __shared__ float ys[4][1024];
  __shared__ float nrm[4];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + w;
  const bool live = row < a.n;
  int tok = live ? a.tokens[row] : 0;
  if (tok < 0 || tok >= a.vocab) {
    if (lane == 0) *a.status = 1;
    tok = 0;
  }
  for (int k = lane; k < a.dim; k += 64) xs[w][k] = h2f(a.table[(size_t)tok * a.dim + k]);
  __syncthreads();
  for (int e = lane; e < a.edim; e += 64) {
    float acc = 0.0f;
    for (int k = 0; k < a.dim; ++k) {
      const float p = xs[w][k] * h2f(a.proj[(size_t)k * a.edim + e]);
      acc = acc + p;
    }
    ys[w][e] = acc;
  }
  __syncthreads();
  if (lane == 0) {
    double ss = 0.0;
    for (int e = 0; e < a.edim; ++e) {
      const double v = (double)ys[w][e];
      ss = ss + v * v;
    }
    nrm[w] = (float)sqrt(ss);
  }
  __syncthreads();
  if (!live) return;
  const float nv = nrm[w];
  for (int e = lane; e < a.edim; e += 64) {
    const float v = ys[w][e];
    a.out[(size_t)row * a.edim + e] = f2h(nv == 0.0f ? v : v / nv);
  }
}

// ---------------------------------------------------------- general shapes

// BERT-family layers at shapes the MFMA kernels do not take (hidden widths
// other than 128..768 in steps of 128, head dims other than 32..256: the
// reference's own golden fixture has hidden 16 and head dim 4). f32
// activations; the sums follow the reference's host path: f64 accumulation
// from the bias in k order for the dense layers (denseHF), f64 mean and
// variance for the LayerNorms (layerNormAffine), f64 logits, maximum, exp and
// sum for the softmax, f32 sums over a sequence's rows in order for the mean
// pool, f64 sum of squares for the L2 norm. Dense weights are the int8 codes
// times their per-channel scale, as on the MFMA path.

namespace {

// Mean and 1 / sqrt(var + eps) (f64) of v[0..n) spread over a wavefront:
// lane l holds v[l + 64 j], j < J.
template <int J>
EOS_DEV void gen_row_stats(const float (&v)[J], int n, int lane, float eps, double* mean,
                           double* inv) {
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (lane + 64 * j < n) s += (double)v[j];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
  const double m = s / (double)n;
  double q = 0.0;
#pragma unroll
  for (int j = 0; j < J; ++j)
    if (lane + 64 * j < n) {
      const double c = (double)v[j] - m;
      q += c * c;
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
  *mean = m;
  *inv = 1.0 / sqrt(q / (double)n + (double)eps);
}

constexpr int kGenMaxHidden = 1024;
constexpr int kGenMaxHeadDim = 64;

}  // namespace

// One wavefront per packed row: token + position + type in f32, then the
// affine LayerNorm; pad rows (position -1) get zeros.
extern "C" __global__ __launch_bounds__(256) void eos_enc_gen_embed(EncGenArgs a) {
  constexpr int J = kGenMaxHidden / 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= *a.total) return;
  const int H = a.hidden;
  float* yr = a.y + (size_t)row * H;
  const int b = a.row_b[row], t = a.row_t[row];
  if (t < 0) {
    for (int c = lane; c < H; c += 64) {
      yr[c] = 0.0f;
      if (a.h16 != nullptr) a.h16[(size_t)row * H + c] = 0;
    }
    return;
  }
  int id = a.ids[(size_t)b * a.tokens + t];
  int ty = a.type_ids != nullptr ? a.type_ids[(size_t)b * a.tokens + t] : 0;
  if (id < 0 || id >= a.vocab || ty < 0 || ty >= a.ntype || t >= a.npos) {
    if (lane == 0) *a.status = 1;
    id = id < 0 || id >= a.vocab ? 0 : id;
    ty = ty < 0 || ty >= a.ntype ? 0 : ty;
  }
  const int p = t < a.npos ? t : a.npos - 1;
  float v[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    v[j] = c < H ? (a.tok[(size_t)id * H + c] + a.pos[(size_t)p * H + c]) + a.typ[(size_t)ty * H + c]
                 : 0.0f;
  }
  double mean, inv;
  gen_row_stats<J>(v, H, lane, a.eps, &mean, &inv);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    if (c < H) {
      const float o = (float)(((double)v[j] - mean) * inv * (double)a.gamma[c] + (double)a.beta[c]);
      yr[c] = o;
      if (a.h16 != nullptr) a.h16[(size_t)row * H + c] = f2h(o);
    }
  }
}

// Thread (row, column): 64 columns x 4 rows per workgroup.
extern "C" __global__ __launch_bounds__(256) void eos_enc_gen_dense(EncGenArgs a) {
  const int col = blockIdx.x * 64 + (threadIdx.x & 63);
  const int row = blockIdx.y * 4 + (threadIdx.x >> 6);
  if (row >= *a.total || col >= a.n) return;
  const float* xr = a.x + (size_t)row * a.k;
  const int8_t* wr = a.w + (size_t)col * a.k;
  const float sc = a.wscale[col];
  double sum = (double)a.bias[col];
  for (int k = 0; k < a.k; ++k) sum += (double)xr[k] * (double)((float)wr[k] * sc);
  float o = (float)sum;
  if (a.epi == 1) {
    o = 0.5f * o * (1.0f + (float)erf((double)o / sqrt(2.0)));
  } else if (a.epi == 2) {
    const float inner = 0.7978845608f * (o + 0.044715f * (o * o * o));
    o = 0.5f * o * (1.0f + (float)tanh((double)inner));
  }
  if (a.res != nullptr) o = o + a.res[(size_t)row * a.n + col];
  a.y[(size_t)row * a.n + col] = o;
}

// One wavefront per row, in place; f16 copy into h16 when given.
extern "C" __global__ __launch_bounds__(256) void eos_enc_gen_ln(EncGenArgs a) {
  constexpr int J = kGenMaxHidden / 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= *a.total) return;
  const int H = a.hidden;
  float* yr = a.y + (size_t)row * H;
  float v[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    v[j] = c < H ? yr[c] : 0.0f;
  }
  double mean, inv;
  gen_row_stats<J>(v, H, lane, a.eps, &mean, &inv);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    if (c < H) {
      const float o = (float)(((double)v[j] - mean) * inv * (double)a.gamma[c] + (double)a.beta[c]);
      yr[c] = o;
      if (a.h16 != nullptr) a.h16[(size_t)row * H + c] = f2h(o);
    }
  }
}

// Thread (query row, head) of sequence blockIdx.z: keys are the sequence's
// active rows, in order; queries its rows up to seq_q (the CLS row included).
// Rows of the sequence's 8-row slot past its queries get zeros.
extern "C" __global__ __launch_bounds__(64) void eos_enc_gen_attn(EncGenArgs a) {
  const int b = blockIdx.z, h = blockIdx.y;
  const int i = blockIdx.x * 64 + threadIdx.x;
  const int cnt = a.seq_cnt[b];
  const int qcnt = a.seq_q != nullptr ? a.seq_q[b] : cnt;
  const int slot = (qcnt + 7) & ~7;
  if (i >= slot) return;
  const int off = a.seq_off[b];
  const int H = a.hidden, hd = H / a.heads;
  float* out = a.y + (size_t)(off + i) * H + h * hd;
  if (i >= qcnt || cnt == 0) {
    for (int d = 0; d < hd; ++d) out[d] = 0.0f;
    return;
  }
  const int ld = 3 * H;
  float q[kGenMaxHeadDim];
  const float* qr = a.x + (size_t)(off + i) * ld + h * hd;
#pragma unroll
  for (int d = 0; d < kGenMaxHeadDim; ++d) q[d] = d < hd ? qr[d] : 0.0f;
  const double scale = 1.0 / sqrt((double)hd);
  auto logit = [&](int j) {
    const float* kr = a.x + (size_t)(off + j) * ld + H + h * hd;
    double dot = 0.0;
#pragma unroll
    for (int d = 0; d < kGenMaxHeadDim; ++d)
      if (d < hd) dot += (double)q[d] * (double)kr[d];
    return dot * scale;
  };
  double mx = -INFINITY;
  for (int j = 0; j < cnt; ++j) mx = fmax(mx, logit(j));
  double sum = 0.0;
  for (int j = 0; j < cnt; ++j) sum += exp(logit(j) - mx);
  float acc[kGenMaxHeadDim];
#pragma unroll
  for (int d = 0; d < kGenMaxHeadDim; ++d) acc[d] = 0.0f;
  for (int j = 0; j < cnt; ++j) {
    const double p = exp(logit(j) - mx) / sum;
    const float* vr = a.x + (size_t)(off + j) * ld + 2 * H + h * hd;
#pragma unroll
    for (int d = 0; d < kGenMaxHeadDim; ++d)
      if (d < hd) acc[d] += (float)(p * (double)vr[d]);
  }
  for (int d = 0; d < hd; ++d) out[d] = acc[d];
}

// One workgroup per sequence, thread c per feature: mean pool (f32 sums over
// the sequence's active rows in order, times float32(1 / count); count 0 ->
// zeros) or CLS (position 0's row), then L2 normalize (f64 sum of squares,
// f32 norm, a zero row unchanged).
extern "C" __global__ __launch_bounds__(1024) void eos_enc_gen_pool(EncPoolArgs a) {
  __shared__ double red[16];
  const int b = blockIdx.x, c = threadIdx.x, lane = c & 63, w = c >> 6;
  const int off = a.seq_off[b], cnt = a.seq_cnt[b];
  float v = 0.0f;
  if (c < a.hidden) {
    if (a.cls_seq_q != nullptr) {
      const int row = off + (a.cls_seq_q[b] > cnt ? cnt : 0);
      v = a.h32[(size_t)row * a.hidden + c];
    } else if (cnt > 0) {
      float s = 0.0f;
      for (int r = 0; r < cnt; ++r) s = s + a.h32[(size_t)(off + r) * a.hidden + c];
      v = s * (1.0f / (float)cnt);
    }
  }
  double q = (double)v * (double)v;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o);
  if (lane == 0) red[w] = q;
  __syncthreads();
  double ss = 0.0;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) ss += red[i];
  const float nrm = (float)sqrt(ss);
  if (c < a.hidden) a.out[(size_t)b * a.hidden + c] = nrm > 0.0f ? v / nrm : v;
}
