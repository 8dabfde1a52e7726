// Measurement kernels for bench.py; the library never launches them. They
// give the matrix-core rate and the shader clock that a stream of independent
// MFMAs reaches on given operand bytes: the clock falls under the power drawn
// by full-range operands, so the rate reachable on real data sits below the
// published dense peak, which assumes the top clock.
//
// Each wave keeps eight accumulators and sixteen operand fragments (its slot
// of `operands`: eight A fragments, then eight B fragments); every iteration
// issues 64 MFMAs, A fragment j against B fragment c into accumulator c, so
// the operands change from one MFMA to the next without any VALU work
// between them. A and B never name the same register: an MFMA that reads one
// register as both operands issues measurably slower.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kProbeSlots = 64;
constexpr int kProbeFrags = 8;  // per operand side

struct MfmaProbeArgs {
  const v4i* operands;         // [kProbeSlots][2 * kProbeFrags][64 lanes]
  int32_t* sink;               // [blocks * 256]: keeps the accumulators live
  unsigned long long* clocks;  // [waves][2]: shader-clock ticks, 100 MHz ticks
  int iters;
};

template <bool F16>
__device__ void probe_body(const MfmaProbeArgs& a) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const v4i* src = a.operands + (size_t)(wave % kProbeSlots) * 2 * kProbeFrags * 64 + lane;
  v4i x[kProbeFrags], y[kProbeFrags];
#pragma unroll
  for (int j = 0; j < kProbeFrags; ++j) {
    x[j] = src[j * 64];
    y[j] = src[(kProbeFrags + j) * 64];
  }
  using Acc = typename std::conditional<F16, v16f, v16i>::type;
  Acc acc[kProbeFrags];
#pragma unroll
  for (int c = 0; c < kProbeFrags; ++c) acc[c] = Acc{0};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  const unsigned long long r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < a.iters; ++it) {
#pragma unroll
    for (int j = 0; j < kProbeFrags; ++j) {
#pragma unroll
      for (int c = 0; c < kProbeFrags; ++c) {
        if constexpr (F16)
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, x[j]),
                                                          __builtin_bit_cast(v8h, y[c]), acc[c],
                                                          0, 0, 0);
        else
          acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(x[j], y[c], acc[c], 0, 0, 0);
      }
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  const unsigned long long r1 = __builtin_amdgcn_s_memrealtime();
  int32_t s = 0;
#pragma unroll
  for (int c = 0; c < kProbeFrags; ++c) s += (int32_t)acc[c][0] + (int32_t)acc[c][15];
  a.sink[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (lane == 0) {
    a.clocks[2 * wave] = t1 - t0;
    a.clocks[2 * wave + 1] = r1 - r0;
  }
}

}  // namespace

// 64 v_mfma_i32_32x32x32_i8 (2 x 32^3 int8 ops each) per wave per iteration.
extern "C" __global__ __launch_bounds__(256) void eos_probe_mfma_i8(MfmaProbeArgs a) {
  probe_body<false>(a);
}

// 64 v_mfma_f32_32x32x16_f16 (2 x 32 x 32 x 16 flops each) per wave per iteration.
extern "C" __global__ __launch_bounds__(256) void eos_probe_mfma_f16(MfmaProbeArgs a) {
  probe_body<true>(a);
}

// Read-only HBM stream: every thread reads 16-byte words at a grid stride,
// U loads in flight at a time, and folds them into one word that it writes
// once (so the loads are kept). The bytes read per launch are `words` x 16;
// writes are one word per thread. This is the achievable rate of a scan that
// only reads, the bound a corpus scan is held to beside the copy's.
struct ReadProbeArgs {
  const v4i* src;
  v4i* sink;                   // [grid threads]
  long long words;             // 16-byte words to read
};

extern "C" __global__ __launch_bounds__(256) void eos_probe_read_stream(ReadProbeArgs a) {
  constexpr int U = 8;
  const long long stride = (long long)gridDim.x * blockDim.x;
  long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  v4i acc = v4i{0, 0, 0, 0};
  for (; i + (U - 1) * stride < a.words; i += U * stride) {
    v4i v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(a.src + i + u * stride);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  for (; i < a.words; i += stride) acc ^= a.src[i];
  a.sink[(long long)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}
