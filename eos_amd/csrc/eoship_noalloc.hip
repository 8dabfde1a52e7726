// Entry points that allocate no device memory, for callers that cannot call
// hipMalloc (code under HIP graph capture, tight serving loops, harnesses that
// forbid allocation). Their scratch memory is one file-scope device array per
// GPU, resolved once per device when a runtime is created on it.
//
// Host code here never passes `scratch` itself to a kernel or copy: on the
// host that name is only a stand-in for the symbol. The per-device address
// from hipGetSymbolAddress is what kernels receive.
//
// Calls on one GPU share its array. They are ordered by a per-device event
// chain: each call's stream waits for the event the previous call recorded
// after its last kernel, then records it again after its own (under one
// mutex, so the chain follows the order of the calls). Calls from several
// runtimes (streams) therefore run one after another on the device instead
// of overwriting each other's scores; nothing is allocated for it. A stream
// under graph capture is left out of the chain (the capturing caller orders
// its graph's replays).
//
// Compiled by hipcc as a host translation unit with a device variable (no
// kernels); the kernels it launches are in the built-in code objects.
#include <hip/hip_runtime.h>

#include <mutex>

#include "eoship_internal.h"

namespace {

// f32 scores between the two rerank kernels: q * c <= kNoAllocRerankFloats
// (4 MiB per GPU, held until the process ends).
constexpr size_t kNoAllocRerankFloats = size_t(1) << 20;
static __device__ __align__(256) float scratch[kNoAllocRerankFloats];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
float* g_ptr[kMaxDevices] = {};
hipError_t g_status[kMaxDevices] = {};
bool g_done[kMaxDevices] = {};
// Completion of the last call on each device (created at set-up; a wait on
// an event never recorded returns at once).
hipEvent_t g_last[kMaxDevices] = {};

}  // namespace

namespace eoship {

// Resolves this device's copy of `scratch` (the device must be current).
// Runs once per device; a failure is kept and reported by the entry points,
// not by runtime creation.
void noalloc_init(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_done[device]) return;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e == hipSuccess) e = hipEventCreateWithFlags(&g_last[device], hipEventDisableTiming);
  g_status[device] = e;
  g_ptr[device] = e == hipSuccess ? static_cast<float*>(p) : nullptr;
  g_done[device] = true;
}

// Runs launch(ptr) with this device's scratch, ordered after the previous
// call on the device (see the event chain above), with g_mu held.
template <typename F>
static int noalloc_run(const Runtime* rt, const char* what, char** err, F launch) {
  const int dev = rt->device;
  if (dev < 0 || dev >= kMaxDevices)
    return set_err(err, "%s: device %d beyond the %d this library tracks", what, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_done[dev]) return set_err(err, "%s: scratch of device %d not resolved", what, dev);
  if (g_status[dev] != hipSuccess)
    return hip_err(err, "hipGetSymbolAddress(scratch) / hipEventCreate", g_status[dev]);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(rt->stream, &cap);
  if (e != hipSuccess) return hip_err(err, "hipStreamIsCapturing", e);
  const bool chained = cap == hipStreamCaptureStatusNone;
  if (chained) {
    e = hipStreamWaitEvent(rt->stream, g_last[dev], 0);
    if (e != hipSuccess) return hip_err(err, "hipStreamWaitEvent(scratch chain)", e);
  }
  const int rc = launch(g_ptr[dev]);
  if (chained) {
    // Recorded whatever launch() returned: a later call must not wait on a
    // stream position before kernels this call did launch.
    e = hipEventRecord(g_last[dev], rt->stream);
    if (e != hipSuccess && rc == 0) return hip_err(err, "hipEventRecord(scratch chain)", e);
  }
  return rc;
}

}  // namespace eoship

extern "C" {

int eoship_tq_fp16_rerank_device_noalloc(EosHipRuntime* rt, const float* d_queries, int32_t q,
                                         int32_t d, const uint16_t* d_rows, int64_t n,
                                         const int64_t* d_cand_ids, const float* d_cand_scores,
                                         int32_t c, int32_t k, int32_t bit_width,
                                         int32_t overfetch, const int64_t* d_id_rank,
                                         int64_t* d_ids, float* d_scores, char** err) {
  const char* what = "eoship_tq_fp16_rerank_device_noalloc";
  if (eoship::tq_fp16_rerank_check(rt, d_queries, q, d, d_rows, n, d_cand_ids, d_cand_scores, c,
                                   d_ids, d_scores, what, err) != 0)
    return 1;
  if (q == 0 || c == 0) return 0;
  if ((size_t)q * (size_t)c > kNoAllocRerankFloats)
    return eoship::set_err(err, "%s: q * c = %lld exceeds the %zu candidates of the static scratch",
                           what, (long long)q * c, kNoAllocRerankFloats);
  // Every valid candidate's score is written by the first kernel before the
  // second reads it, so nothing is cleared between calls.
  return eoship::noalloc_run(rt, what, err, [&](float* ptr) {
    return eoship::tq_fp16_rerank_launch(rt, d_queries, q, d, d_rows, n, d_cand_ids,
                                         d_cand_scores, c, k, bit_width, overfetch, d_id_rank,
                                         d_ids, d_scores, ptr, what, err);
  });
}

}  // extern "C"
