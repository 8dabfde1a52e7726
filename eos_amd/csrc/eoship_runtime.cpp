// Runtime half of the eoship C ABI: device/stream ownership, memory, code
// objects, launches and hipEvent profiling. Mirrors the reference CGo bridge's
// shape (runtime/backends/cuda/native_linux.go:72-632, eos_cuda_abi.h:22-38)
// on HIP: one stream per runtime, int return codes, malloc'd error strings.
#include "eoship_internal.h"

// HIP's launch with dispatch-recorded start/stop events (a C entry point of
// libamdhip64; its header also holds templates only hipcc compiles).
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>

extern "C" {
// Code objects built offline for gfx950 and linked in by eoship_blobs.S.
extern const unsigned char eoship_tq_co_begin[];
extern const unsigned char eoship_tq_co_end[];
extern const unsigned char eoship_enc_co_begin[];
extern const unsigned char eoship_enc_co_end[];
extern const unsigned char eoship_ret_co_begin[];
extern const unsigned char eoship_ret_co_end[];
}

namespace eoship {

int set_err(char** err, const char* fmt, ...) {
  if (err != nullptr) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    const size_t n = strlen(buf) + 1;
    char* out = static_cast<char*>(malloc(n));
    if (out != nullptr) memcpy(out, buf, n);
    *err = out;
  }
  return 1;
}

int hip_err(char** err, const char* what, hipError_t e) {
  return set_err(err, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

int Runtime::function(const char* name, hipFunction_t* out, char** err) {
  auto it = fns.find(name);
  if (it != fns.end()) {
    *out = it->second;
    return 0;
  }
  hipFunction_t f = nullptr;
  hipError_t e = hipErrorNotFound;
  for (hipModule_t m : builtin) {
    e = hipModuleGetFunction(&f, m, name);
    if (e == hipSuccess) break;
  }
  if (e != hipSuccess) return hip_err(err, name, e);
  fns.emplace(name, f);
  *out = f;
  return 0;
}

int Runtime::launch(const char* name, dim3 grid, dim3 block, size_t lds, void* args,
                    char** err, const char* label) {
  hipFunction_t f = nullptr;
  if (function(name, &f, err) != 0) return 1;
  void* params[1] = {args};
  const char* tag = label ? label : name;
  const bool rec = profiling && (profile_prefix.empty() ||
                                 strncmp(tag, profile_prefix.c_str(), profile_prefix.size()) == 0);
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipError_t e;
  if (rec) {
    if (take_event(&e0, err) != 0 || take_event(&e1, err) != 0) return 1;
    // The dispatch itself records the two events at the kernel's start and
    // end, so a profiled duration excludes the gaps around the launch.
    e = hipExtModuleLaunchKernel(f, grid.x * block.x, grid.y * block.y, grid.z * block.z, block.x,
                                 block.y, block.z, lds, stream, params, nullptr, e0, e1, 0);
  } else {
    e = hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                              static_cast<unsigned>(lds), stream, params, nullptr);
  }
  if (e != hipSuccess) {
    if (e0) event_pool.push_back(e0);
    if (e1) event_pool.push_back(e1);
    return hip_err(err, name, e);
  }
  if (rec) records.push_back(ProfileRecord{tag, e0, e1});
  ++n_launches;
  return 0;
}

int Runtime::blocks_per_cu(const char* name, int block, size_t lds, int* out, char** err) {
  const auto it = occupancy.find(name);
  if (it != occupancy.end()) {
    *out = it->second;
    return 0;
  }
  hipFunction_t f = nullptr;
  if (function(name, &f, err) != 0) return 1;
  int n = 0;
  const hipError_t e = hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, block, lds);
  if (e != hipSuccess) return hip_err(err, "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor", e);
  if (n < 1) n = 1;
  occupancy.emplace(name, n);
  *out = n;
  return 0;
}

int Runtime::take_event(hipEvent_t* ev, char** err) {
  if (!event_pool.empty()) {
    *ev = event_pool.back();
    event_pool.pop_back();
    return 0;
  }
  hipError_t e = hipEventCreate(ev);
  if (e != hipSuccess) return hip_err(err, "hipEventCreate", e);
  return 0;
}

int Runtime::alloc(size_t bytes, void** p, char** err) {
  *p = nullptr;
  if (bytes == 0) return 0;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return hip_err(err, "hipMalloc", e);
  return 0;
}

int Runtime::workspace(size_t bytes, void** p, char** err) {
  if (bytes > ws_bytes) {
    if (ws != nullptr) {
      // Earlier launches on this stream may still read the old block.
      if (sync(err) != 0) return 1;
      hipFree(ws);
      ws = nullptr;
      ws_bytes = 0;
    }
    if (alloc(bytes, &ws, err) != 0) return 1;
    ws_bytes = bytes;
  }
  *p = ws;
  return 0;
}

void Runtime::release(void* p) {
  if (p != nullptr) hipFree(p);
}

int Runtime::sync(char** err) {
  ++n_syncs;
  hipError_t e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_err(err, "hipStreamSynchronize", e);
  return 0;
}

int Runtime::flush_profile(char** err) {
  if (records.empty()) return 0;
  if (sync(err) != 0) return 1;
  for (auto& r : records) {
    float ms = 0.f;
    hipEventElapsedTime(&ms, r.begin, r.end);
    auto& acc = totals[r.name];
    acc.first += 1;
    acc.second += ms;
    samples[r.name].push_back(ms);
    event_pool.push_back(r.begin);
    event_pool.push_back(r.end);
  }
  records.clear();
  return 0;
}

}  // namespace eoship

using eoship::hip_err;
using eoship::set_err;

struct EosHipModule {
  hipModule_t module;
};
struct EosHipFunction {
  hipFunction_t function;
  std::string name;
};

extern "C" {

int eoship_abi_version(void) { return EOSHIP_ABI_VERSION; }

void eoship_free_cstring(char* s) { free(s); }

int eoship_runtime_create(int device, EosHipRuntime** out, char** err) {
  if (out == nullptr) return set_err(err, "eoship_runtime_create: out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_err(err, "hipGetDeviceCount", e);
  if (device < 0 || device >= count)
    return set_err(err, "eoship_runtime_create: device %d out of range (%d devices)", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_err(err, "hipSetDevice", e);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_err(err, "hipGetDeviceProperties", e);
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return set_err(err, "eoship: device %d is %s; this library is built for gfx950 only", device,
                   prop.gcnArchName);
  auto* rt = new EosHipRuntime();
  rt->device = device;
  rt->compute_units = prop.multiProcessorCount;
  rt->name = prop.name;
  rt->arch = prop.gcnArchName;
  e = hipStreamCreateWithFlags(&rt->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete rt;
    return hip_err(err, "hipStreamCreateWithFlags", e);
  }
  const unsigned char* images[3][2] = {{eoship_tq_co_begin, eoship_tq_co_end},
                                       {eoship_enc_co_begin, eoship_enc_co_end},
                                       {eoship_ret_co_begin, eoship_ret_co_end}};
  for (auto& im : images) {
    hipModule_t m = nullptr;
    e = im[1] > im[0] ? hipModuleLoadData(&m, im[0]) : hipErrorInvalidImage;
    if (e != hipSuccess) {
      for (hipModule_t mm : rt->builtin) hipModuleUnload(mm);
      hipStreamDestroy(rt->stream);
      delete rt;
      return hip_err(err, "hipModuleLoadData(built-in gfx950 code object)", e);
    }
    rt->builtin.push_back(m);
  }
  for (auto& ev : rt->timer) ev = nullptr;
  eoship::noalloc_init(device);
  *out = rt;
  return 0;
}

int eoship_runtime_destroy(EosHipRuntime* rt, char** err) {
  if (rt == nullptr) return 0;
  hipSetDevice(rt->device);
  hipStreamSynchronize(rt->stream);
  for (auto& r : rt->records) {
    hipEventDestroy(r.begin);
    hipEventDestroy(r.end);
  }
  for (hipEvent_t ev : rt->event_pool) hipEventDestroy(ev);
  for (auto& ev : rt->timer)
    if (ev) hipEventDestroy(ev);
  for (hipModule_t m : rt->builtin) hipModuleUnload(m);
  if (rt->ws != nullptr) hipFree(rt->ws);
  hipError_t e = hipStreamDestroy(rt->stream);
  delete rt;
  if (e != hipSuccess) return hip_err(err, "hipStreamDestroy", e);
  return 0;
}

int eoship_device_info(EosHipRuntime* rt, char* name, size_t name_len, int* compute_units,
                       char* arch, size_t arch_len, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_device_info: runtime is NULL");
  if (name && name_len) snprintf(name, name_len, "%s", rt->name.c_str());
  if (arch && arch_len) snprintf(arch, arch_len, "%s", rt->arch.c_str());
  if (compute_units) *compute_units = rt->compute_units;
  return 0;
}

int eoship_malloc(EosHipRuntime* rt, size_t bytes, void** dptr, char** err) {
  if (rt == nullptr || dptr == nullptr) return set_err(err, "eoship_malloc: NULL argument");
  return rt->alloc(bytes, dptr, err);
}

int eoship_free(EosHipRuntime* rt, void* dptr, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_free: runtime is NULL");
  if (dptr == nullptr) return 0;
  hipError_t e = hipFree(dptr);
  if (e != hipSuccess) return hip_err(err, "hipFree", e);
  return 0;
}

static int copy(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
                const char* what, char** err) {
  if (rt == nullptr) return set_err(err, "%s: runtime is NULL", what);
  if (bytes == 0) return 0;
  if (dst == nullptr || src == nullptr) return set_err(err, "%s: NULL buffer", what);
  hipError_t e = rt->copy_async(dst, src, bytes, kind);
  if (e != hipSuccess) return hip_err(err, what, e);
  if (kind != hipMemcpyDeviceToDevice) return rt->sync(err);
  return 0;
}

int eoship_h2d(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, char** err) {
  return copy(rt, dst, src, bytes, hipMemcpyHostToDevice, "eoship_h2d", err);
}
int eoship_d2h(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, char** err) {
  return copy(rt, dst, src, bytes, hipMemcpyDeviceToHost, "eoship_d2h", err);
}
int eoship_d2d(EosHipRuntime* rt, void* dst, const void* src, size_t bytes, char** err) {
  return copy(rt, dst, src, bytes, hipMemcpyDeviceToDevice, "eoship_d2d", err);
}

int eoship_memset(EosHipRuntime* rt, void* dst, int value, size_t bytes, char** err) {
  if (rt == nullptr || (dst == nullptr && bytes != 0))
    return set_err(err, "eoship_memset: NULL argument");
  if (bytes == 0) return 0;
  const hipError_t e = hipMemsetAsync(dst, value, bytes, rt->stream);
  if (e != hipSuccess) return hip_err(err, "eoship_memset", e);
  return 0;
}

int eoship_sync(EosHipRuntime* rt, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_sync: runtime is NULL");
  return rt->sync(err);
}

int eoship_runtime_wait(EosHipRuntime* rt, EosHipRuntime* other, char** err) {
  if (rt == nullptr || other == nullptr) return set_err(err, "eoship_runtime_wait: NULL runtime");
  if (rt == other) return 0;
  if (rt->device != other->device)
    return set_err(err, "eoship_runtime_wait: runtimes are on devices %d and %d", rt->device,
                   other->device);
  hipEvent_t ev = nullptr;
  hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
  if (e != hipSuccess) return hip_err(err, "hipEventCreateWithFlags", e);
  e = hipEventRecord(ev, other->stream);
  if (e == hipSuccess) e = hipStreamWaitEvent(rt->stream, ev, 0);
  // Destroying a recorded event is deferred by the runtime until it completes.
  hipEventDestroy(ev);
  if (e != hipSuccess) return hip_err(err, "eoship_runtime_wait", e);
  return 0;
}

int eoship_module_load(EosHipRuntime* rt, const void* image, size_t bytes, EosHipModule** out,
                       char** err) {
  if (rt == nullptr || image == nullptr || out == nullptr || bytes == 0)
    return set_err(err, "eoship_module_load: NULL or empty argument");
  hipModule_t m = nullptr;
  hipError_t e = hipModuleLoadData(&m, image);
  if (e != hipSuccess) return hip_err(err, "hipModuleLoadData", e);
  *out = new EosHipModule{m};
  return 0;
}

int eoship_module_unload(EosHipModule* mod, char** err) {
  if (mod == nullptr) return 0;
  hipError_t e = hipModuleUnload(mod->module);
  delete mod;
  if (e != hipSuccess) return hip_err(err, "hipModuleUnload", e);
  return 0;
}

int eoship_function(EosHipModule* mod, const char* name, EosHipFunction** out, char** err) {
  if (mod == nullptr || name == nullptr || out == nullptr)
    return set_err(err, "eoship_function: NULL argument");
  hipFunction_t f = nullptr;
  hipError_t e = hipModuleGetFunction(&f, mod->module, name);
  if (e != hipSuccess) return hip_err(err, name, e);
  *out = new EosHipFunction{f, name};
  return 0;
}

int eoship_launch(EosHipRuntime* rt, EosHipFunction* fn, const uint32_t grid[3],
                  const uint32_t block[3], uint32_t lds_bytes, void** args, char** err) {
  if (rt == nullptr || fn == nullptr || grid == nullptr || block == nullptr)
    return set_err(err, "eoship_launch: NULL argument");
  hipError_t e = hipModuleLaunchKernel(fn->function, grid[0], grid[1], grid[2], block[0], block[1],
                                       block[2], lds_bytes, rt->stream, args, nullptr);
  if (e != hipSuccess) return hip_err(err, fn->name.c_str(), e);
  return 0;
}

int eoship_profile_enable(EosHipRuntime* rt, int enabled, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_profile_enable: runtime is NULL");
  if (!enabled && rt->flush_profile(err) != 0) return 1;
  rt->profiling = enabled != 0;
  return 0;
}

int eoship_profile_select(EosHipRuntime* rt, const char* prefix, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_profile_select: runtime is NULL");
  rt->profile_prefix = prefix ? prefix : "";
  return 0;
}

int eoship_profile_read(EosHipRuntime* rt, const char* prefix, int64_t* launches, double* total_ms,
                        char** err) {
  if (rt == nullptr) return set_err(err, "eoship_profile_read: runtime is NULL");
  if (rt->flush_profile(err) != 0) return 1;
  int64_t n = 0;
  double ms = 0.0;
  const size_t plen = prefix ? strlen(prefix) : 0;
  for (auto& kv : rt->totals) {
    if (plen == 0 || kv.first.compare(0, plen, prefix) == 0) {
      n += kv.second.first;
      ms += kv.second.second;
    }
  }
  if (launches) *launches = n;
  if (total_ms) *total_ms = ms;
  return 0;
}

int eoship_profile_reset(EosHipRuntime* rt, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_profile_reset: runtime is NULL");
  if (rt->flush_profile(err) != 0) return 1;
  rt->totals.clear();
  rt->samples.clear();
  return 0;
}

int eoship_accounting_read(EosHipRuntime* rt, EosHipAccounting* out, int32_t reset, char** err) {
  if (rt == nullptr || out == nullptr) return set_err(err, "eoship_accounting_read: NULL argument");
  memset(out, 0, sizeof(*out));
  out->kernel_launches = rt->n_launches;
  out->uploaded_bytes = rt->n_uploaded;
  out->downloaded_bytes = rt->n_downloaded;
  out->sync_count = rt->n_syncs;
  out->device_execution = 1;
  if (reset) rt->n_launches = rt->n_uploaded = rt->n_downloaded = rt->n_syncs = 0;
  return 0;
}

int eoship_profile_samples(EosHipRuntime* rt, const char* prefix, float* ms, int64_t cap,
                           int64_t* count, char** err) {
  if (rt == nullptr || count == nullptr || (cap > 0 && ms == nullptr))
    return set_err(err, "eoship_profile_samples: NULL argument");
  if (rt->flush_profile(err) != 0) return 1;
  const size_t plen = prefix ? strlen(prefix) : 0;
  int64_t n = 0;
  for (auto& kv : rt->samples) {
    if (plen != 0 && kv.first.compare(0, plen, prefix) != 0) continue;
    for (float v : kv.second) {
      if (n < cap) ms[n] = v;
      ++n;
    }
  }
  *count = n;
  return 0;
}

int eoship_timer_mark(EosHipRuntime* rt, int slot, char** err) {
  if (rt == nullptr) return set_err(err, "eoship_timer_mark: runtime is NULL");
  if (slot < 0 || slot >= eoship::kTimerSlots) return set_err(err, "eoship_timer_mark: bad slot %d", slot);
  if (rt->timer[slot] == nullptr) {
    hipError_t e = hipEventCreate(&rt->timer[slot]);
    if (e != hipSuccess) return hip_err(err, "hipEventCreate", e);
  }
  hipError_t e = hipEventRecord(rt->timer[slot], rt->stream);
  if (e != hipSuccess) return hip_err(err, "hipEventRecord", e);
  return 0;
}

int eoship_timer_elapsed(EosHipRuntime* rt, int slot_begin, int slot_end, double* ms, char** err) {
  if (rt == nullptr || ms == nullptr) return set_err(err, "eoship_timer_elapsed: NULL argument");
  if (slot_begin < 0 || slot_begin >= eoship::kTimerSlots || slot_end < 0 ||
      slot_end >= eoship::kTimerSlots || !rt->timer[slot_begin] || !rt->timer[slot_end])
    return set_err(err, "eoship_timer_elapsed: slot not recorded");
  hipError_t e = hipEventSynchronize(rt->timer[slot_end]);
  if (e != hipSuccess) return hip_err(err, "hipEventSynchronize", e);
  float f = 0.f;
  e = hipEventElapsedTime(&f, rt->timer[slot_begin], rt->timer[slot_end]);
  if (e != hipSuccess) return hip_err(err, "hipEventElapsedTime", e);
  *ms = f;
  return 0;
}

}  // extern "C"
