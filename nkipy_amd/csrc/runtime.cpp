// libnkipy_hip.so -- thin C-ABI runtime over HIP for the NKIPy MI355X backend.
//
// Replaces the Spike C++ runtime (spike/src/spike.cpp, model.cpp, tensor.cpp,
// nrt_wrapper.cpp) of the reference.  Declarations and per-function contracts
// are in include/nkipy_hip.h.
//
// Design:
//   * one process-wide runtime (device + one non-blocking stream at the
//     default priority), created by nkh_init and torn down by nkh_shutdown;
//   * a registry of live allocations keyed by base address, so host-side
//     copies are bounds-checked and use-after-free is an error, not a fault
//     (the reference guards the same way: spike/src/tensor.cpp:61-77);
//   * a registry of loaded modules, unloaded at shutdown;
//   * thread-local last-error text.

#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>

#include "../../include/nkipy_hip.h"
#include "runtime_internal.h"

namespace {

thread_local std::string g_last_error;

struct Runtime {
  bool initialized = false;
  int device = -1;
  hipStream_t stream = nullptr;
  std::map<uintptr_t, size_t> allocations;  // base -> bytes
  std::set<hipModule_t> modules;
  std::set<hipEvent_t> events;
  std::set<hipGraphExec_t> graphs;
};

Runtime g_rt;
std::mutex g_mu;

int set_error(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

int hip_error(hipError_t e, const char *what) {
  std::string msg = std::string("HIP error ") + hipGetErrorName(e) + " (" +
                    std::to_string(static_cast<int>(e)) + ") in " + what +
                    ": " + hipGetErrorString(e);
  return set_error(NKH_ERR_HIP, msg);
}

#define NKH_HIP(call, what)                         \
  do {                                              \
    hipError_t _e = (call);                         \
    if (_e != hipSuccess) return hip_error(_e, what); \
  } while (0)

int require_init() {
  if (!g_rt.initialized)
    return set_error(NKH_ERR_NOT_INIT,
                     "runtime is not initialized (call nkh_init first)");
  return NKH_OK;
}

// Finds the live allocation containing [p, p+n).  Caller holds g_mu.
int check_range(const void *p, size_t n, const char *what) {
  uintptr_t a = reinterpret_cast<uintptr_t>(p);
  auto it = g_rt.allocations.upper_bound(a);
  if (it == g_rt.allocations.begin())
    return set_error(NKH_ERR_FREED, std::string(what) +
                                        ": pointer is not inside a live device "
                                        "allocation (freed or never allocated)");
  --it;
  uintptr_t base = it->first;
  size_t size = it->second;
  if (a >= base + size)
    return set_error(NKH_ERR_FREED, std::string(what) +
                                        ": pointer is not inside a live device "
                                        "allocation (freed or never allocated)");
  size_t offset = a - base;
  if (n > size - offset) {
    char buf[256];
    std::snprintf(buf, sizeof(buf),
                  "%s exceeds the allocation bound: allocation size %zu bytes; "
                  "offset %zu bytes; access size %zu bytes",
                  what, size, offset, n);
    return set_error(NKH_ERR_BOUNDS, buf);
  }
  return NKH_OK;
}

// roctx, opened on first use (the library is part of the ROCm profiler SDK;
// without it profiler ranges are no-ops)
struct Roctx {
  std::once_flag once;
  int (*push)(const char *) = nullptr;
  int (*pop)() = nullptr;
};
Roctx g_roctx;
thread_local int g_range_depth = 0;

void open_roctx() {
  std::call_once(g_roctx.once, [] {
    const char *names[] = {"librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so",
                           "libroctx64.so.4", "libroctx64.so"};
    for (const char *n : names) {
      void *h = dlopen(n, RTLD_NOW | RTLD_LOCAL);
      if (!h) continue;
      auto push = reinterpret_cast<int (*)(const char *)>(dlsym(h, "roctxRangePushA"));
      auto pop = reinterpret_cast<int (*)()>(dlsym(h, "roctxRangePop"));
      if (push && pop) {
        g_roctx.push = push;
        g_roctx.pop = pop;
        return;
      }
      dlclose(h);
    }
  });
}

}  // namespace

namespace nkh_internal {

int set_error(int code, const std::string &msg) { return ::set_error(code, msg); }

int hip_error(hipError_t e, const char *what) { return ::hip_error(e, what); }

int with_stream(const std::function<int(hipStream_t, int)> &fn) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  return fn(g_rt.stream, g_rt.device);
}

}  // namespace nkh_internal

extern "C" {

const char *nkh_last_error(void) { return g_last_error.c_str(); }

int nkh_init(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_rt.initialized)
    return set_error(NKH_ERR_ALREADY_INIT,
                     "runtime already initialized; call nkh_shutdown first");
  int count = 0;
  NKH_HIP(hipGetDeviceCount(&count), "hipGetDeviceCount");
  if (device < 0 || device >= count)
    return set_error(NKH_ERR_INVALID, "device index " + std::to_string(device) +
                                          " out of range (visible devices: " +
                                          std::to_string(count) + ")");
  NKH_HIP(hipSetDevice(device), "hipSetDevice");
  hipStream_t s = nullptr;
  NKH_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
          "hipStreamCreateWithFlags");
  int rc = nkh_internal::device_setup(device);
  if (rc) {
    hipStreamDestroy(s);
    return rc;
  }
  g_rt.device = device;
  g_rt.stream = s;
  g_rt.initialized = true;
  g_last_error.clear();
  return NKH_OK;
}

int nkh_shutdown(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_rt.initialized) return NKH_OK;
  int rc = NKH_OK;
  hipError_t e = hipStreamSynchronize(g_rt.stream);
  if (e != hipSuccess) rc = hip_error(e, "hipStreamSynchronize(shutdown)");
  for (auto &kv : g_rt.allocations) hipFree(reinterpret_cast<void *>(kv.first));
  g_rt.allocations.clear();
  for (auto m : g_rt.modules) hipModuleUnload(m);
  g_rt.modules.clear();
  for (auto ev : g_rt.events) hipEventDestroy(ev);
  g_rt.events.clear();
  for (auto g : g_rt.graphs) hipGraphExecDestroy(g);
  g_rt.graphs.clear();
  hipStreamDestroy(g_rt.stream);
  g_rt.stream = nullptr;
  g_rt.device = -1;
  g_rt.initialized = false;
  return rc;
}

int nkh_is_initialized(int *flag) {
  if (!flag) return set_error(NKH_ERR_INVALID, "flag is null");
  std::lock_guard<std::mutex> lk(g_mu);
  *flag = g_rt.initialized ? 1 : 0;
  return NKH_OK;
}

int nkh_device_count(int *count) {
  if (!count) return set_error(NKH_ERR_INVALID, "count is null");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return NKH_OK;
  }
  if (e != hipSuccess) return hip_error(e, "hipGetDeviceCount");
  *count = n;
  return NKH_OK;
}

int nkh_device_info(int *cu_count, int *clock_khz, int *mem_clock_khz,
                    int *mem_bus_bits, int *l2_bytes, char *arch_name,
                    size_t arch_name_len) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipDeviceProp_t p;
  NKH_HIP(hipGetDeviceProperties(&p, g_rt.device), "hipGetDeviceProperties");
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (clock_khz) *clock_khz = p.clockRate;
  if (mem_clock_khz) *mem_clock_khz = p.memoryClockRate;
  if (mem_bus_bits) *mem_bus_bits = p.memoryBusWidth;
  if (l2_bytes) *l2_bytes = p.l2CacheSize;
  if (arch_name && arch_name_len) {
    std::strncpy(arch_name, p.gcnArchName, arch_name_len - 1);
    arch_name[arch_name_len - 1] = '\0';
  }
  return NKH_OK;
}

int nkh_malloc(size_t bytes, void **ptr) {
  if (!ptr) return set_error(NKH_ERR_INVALID, "ptr is null");
  if (bytes == 0) return set_error(NKH_ERR_INVALID, "allocation of 0 bytes");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  void *p = nullptr;
  NKH_HIP(hipMalloc(&p, bytes), "hipMalloc");
  g_rt.allocations[reinterpret_cast<uintptr_t>(p)] = bytes;
  *ptr = p;
  return NKH_OK;
}

int nkh_free(void *ptr) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  auto it = g_rt.allocations.find(reinterpret_cast<uintptr_t>(ptr));
  if (it == g_rt.allocations.end())
    return set_error(NKH_ERR_FREED,
                     "nkh_free: pointer is not the base of a live allocation "
                     "(double free or foreign pointer)");
  // Launches queued on the runtime stream may still read the buffer.
  NKH_HIP(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize(free)");
  NKH_HIP(hipFree(ptr), "hipFree");
  g_rt.allocations.erase(it);
  return NKH_OK;
}

int nkh_alloc_size(const void *ptr, size_t *bytes) {
  if (!bytes) return set_error(NKH_ERR_INVALID, "bytes is null");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  auto it = g_rt.allocations.find(reinterpret_cast<uintptr_t>(ptr));
  if (it == g_rt.allocations.end())
    return set_error(NKH_ERR_FREED, "nkh_alloc_size: not a live allocation");
  *bytes = it->second;
  return NKH_OK;
}

int nkh_memcpy_h2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return NKH_OK;
  if (!src) return set_error(NKH_ERR_INVALID, "host source is null");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  rc = check_range(dst, bytes, "host-to-device write");
  if (rc) return rc;
  NKH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_rt.stream),
          "hipMemcpyAsync(H2D)");
  NKH_HIP(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize(H2D)");
  return NKH_OK;
}

int nkh_memcpy_d2h(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return NKH_OK;
  if (!dst) return set_error(NKH_ERR_INVALID, "host destination is null");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  rc = check_range(src, bytes, "device-to-host read");
  if (rc) return rc;
  NKH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_rt.stream),
          "hipMemcpyAsync(D2H)");
  NKH_HIP(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize(D2H)");
  return NKH_OK;
}

int nkh_memcpy_d2d(void *dst, const void *src, size_t bytes) {
  if (bytes == 0) return NKH_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  rc = check_range(src, bytes, "device-to-device read");
  if (rc) return rc;
  rc = check_range(dst, bytes, "device-to-device write");
  if (rc) return rc;
  NKH_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_rt.stream),
          "hipMemcpyAsync(D2D)");
  return NKH_OK;
}

int nkh_memset(void *ptr, int value, size_t bytes) {
  if (bytes == 0) return NKH_OK;
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  rc = check_range(ptr, bytes, "memset");
  if (rc) return rc;
  NKH_HIP(hipMemsetAsync(ptr, value, bytes, g_rt.stream), "hipMemsetAsync");
  return NKH_OK;
}

int nkh_module_load(const char *hsaco_path, void **module) {
  if (!hsaco_path || !module)
    return set_error(NKH_ERR_INVALID, "null path or module pointer");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  FILE *f = std::fopen(hsaco_path, "rb");
  if (!f)
    return set_error(NKH_ERR_INVALID,
                     std::string("code object not found: ") + hsaco_path);
  std::fclose(f);
  hipModule_t m = nullptr;
  hipError_t e = hipModuleLoad(&m, hsaco_path);
  if (e != hipSuccess)
    return hip_error(e, (std::string("hipModuleLoad(") + hsaco_path + ")").c_str());
  g_rt.modules.insert(m);
  *module = reinterpret_cast<void *>(m);
  return NKH_OK;
}

int nkh_module_unload(void *module) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipModule_t m = reinterpret_cast<hipModule_t>(module);
  auto it = g_rt.modules.find(m);
  if (it == g_rt.modules.end())
    return set_error(NKH_ERR_FREED, "module is not loaded");
  NKH_HIP(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize(unload)");
  NKH_HIP(hipModuleUnload(m), "hipModuleUnload");
  g_rt.modules.erase(it);
  return NKH_OK;
}

int nkh_get_function(void *module, const char *symbol, void **function) {
  if (!symbol || !function)
    return set_error(NKH_ERR_INVALID, "null symbol or function pointer");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipModule_t m = reinterpret_cast<hipModule_t>(module);
  if (g_rt.modules.find(m) == g_rt.modules.end())
    return set_error(NKH_ERR_FREED, "module is not loaded");
  hipFunction_t fn = nullptr;
  hipError_t e = hipModuleGetFunction(&fn, m, symbol);
  if (e != hipSuccess)
    return hip_error(e, (std::string("hipModuleGetFunction(") + symbol + ")").c_str());
  *function = reinterpret_cast<void *>(fn);
  return NKH_OK;
}

static int launch_locked(void *function, unsigned gx, unsigned gy, unsigned gz,
                         unsigned bx, unsigned by, unsigned bz,
                         unsigned shared_bytes, const void *kernarg,
                         size_t kernarg_bytes) {
  if (!function) return set_error(NKH_ERR_INVALID, "function is null");
  if (gx == 0 || gy == 0 || gz == 0 || bx == 0 || by == 0 || bz == 0)
    return set_error(NKH_ERR_INVALID, "zero grid or block dimension");
  if (bx * by * bz > 1024)
    return set_error(NKH_ERR_INVALID, "block has more than 1024 threads");
  size_t size = kernarg_bytes;
  void *config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, const_cast<void *>(kernarg),
                    HIP_LAUNCH_PARAM_BUFFER_SIZE, &size, HIP_LAUNCH_PARAM_END};
  hipError_t e = hipModuleLaunchKernel(reinterpret_cast<hipFunction_t>(function),
                                       gx, gy, gz, bx, by, bz, shared_bytes,
                                       g_rt.stream, nullptr, config);
  if (e != hipSuccess) return hip_error(e, "hipModuleLaunchKernel");
  return NKH_OK;
}

int nkh_launch(void *function, unsigned gx, unsigned gy, unsigned gz,
               unsigned bx, unsigned by, unsigned bz, unsigned shared_bytes,
               const void *kernarg, size_t kernarg_bytes) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  return launch_locked(function, gx, gy, gz, bx, by, bz, shared_bytes, kernarg,
                       kernarg_bytes);
}

int nkh_profile_range_push(const char *name, int *available) {
  if (!name) return set_error(NKH_ERR_INVALID, "range name is null");
  open_roctx();
  if (available) *available = g_roctx.push != nullptr;
  if (g_roctx.push) g_roctx.push(name);
  ++g_range_depth;
  return NKH_OK;
}

int nkh_profile_range_pop(void) {
  if (g_range_depth <= 0)
    return set_error(NKH_ERR_INVALID, "profiler range pop without a push");
  --g_range_depth;
  if (g_roctx.pop) g_roctx.pop();
  return NKH_OK;
}

int nkh_launch_batch(int count, void *const *functions, const unsigned *grids,
                     const unsigned *blocks, const unsigned *shared,
                     const uint8_t *kernargs, const size_t *kernarg_offsets,
                     const size_t *kernarg_sizes) {
  if (count < 0) return set_error(NKH_ERR_INVALID, "negative launch count");
  if (count == 0) return NKH_OK;
  if (!functions || !grids || !blocks || !shared || !kernargs ||
      !kernarg_offsets || !kernarg_sizes)
    return set_error(NKH_ERR_INVALID, "null array in nkh_launch_batch");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  for (int i = 0; i < count; ++i) {
    rc = launch_locked(functions[i], grids[3 * i], grids[3 * i + 1],
                       grids[3 * i + 2], blocks[3 * i], blocks[3 * i + 1],
                       blocks[3 * i + 2], shared[i],
                       kernargs + kernarg_offsets[i], kernarg_sizes[i]);
    if (rc) {
      g_last_error = "launch " + std::to_string(i) + " of batch: " + g_last_error;
      return rc;
    }
  }
  return NKH_OK;
}

int nkh_graph_create(int count, void *const *functions, const unsigned *grids,
                     const unsigned *blocks, const unsigned *shared,
                     const uint8_t *kernargs, const size_t *kernarg_offsets,
                     const size_t *kernarg_sizes, void **graph) {
  if (!graph) return set_error(NKH_ERR_INVALID, "graph output pointer is null");
  *graph = nullptr;
  if (count <= 0) return set_error(NKH_ERR_INVALID, "a graph needs at least one launch");
  if (!functions || !grids || !blocks || !shared || !kernargs ||
      !kernarg_offsets || !kernarg_sizes)
    return set_error(NKH_ERR_INVALID, "null array in nkh_graph_create");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  // Capture records the launches (kernel nodes with their argument blocks
  // copied) on the runtime stream; nothing runs until nkh_graph_launch.
  NKH_HIP(hipStreamBeginCapture(g_rt.stream, hipStreamCaptureModeThreadLocal),
          "hipStreamBeginCapture");
  for (int i = 0; i < count && !rc; ++i) {
    rc = launch_locked(functions[i], grids[3 * i], grids[3 * i + 1],
                       grids[3 * i + 2], blocks[3 * i], blocks[3 * i + 1],
                       blocks[3 * i + 2], shared[i],
                       kernargs + kernarg_offsets[i], kernarg_sizes[i]);
    if (rc) g_last_error = "launch " + std::to_string(i) + " of graph: " + g_last_error;
  }
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(g_rt.stream, &g);
  if (rc) {
    if (g) hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return hip_error(e, "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (e != hipSuccess) return hip_error(e, "hipGraphInstantiate");
  g_rt.graphs.insert(exec);
  *graph = exec;
  return NKH_OK;
}

int nkh_graph_launch(void *graph) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  auto it = g_rt.graphs.find(reinterpret_cast<hipGraphExec_t>(graph));
  if (it == g_rt.graphs.end())
    return set_error(NKH_ERR_INVALID, "not a live graph of this runtime");
  NKH_HIP(hipGraphLaunch(*it, g_rt.stream), "hipGraphLaunch");
  return NKH_OK;
}

int nkh_graph_destroy(void *graph) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  auto it = g_rt.graphs.find(reinterpret_cast<hipGraphExec_t>(graph));
  if (it == g_rt.graphs.end())
    return set_error(NKH_ERR_INVALID, "not a live graph of this runtime");
  // a replay still queued keeps its own reference: the stream is drained
  // first so that the executable is not released under it
  NKH_HIP(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize");
  hipGraphExec_t g = *it;
  g_rt.graphs.erase(it);
  NKH_HIP(hipGraphExecDestroy(g), "hipGraphExecDestroy");
  return NKH_OK;
}

int nkh_sync(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  NKH_HIP(hipStreamSynchronize(g_rt.stream), "hipStreamSynchronize");
  return NKH_OK;
}

int nkh_time_launch(void *function, unsigned gx, unsigned gy, unsigned gz,
                    unsigned bx, unsigned by, unsigned bz,
                    unsigned shared_bytes, const void *kernarg,
                    size_t kernarg_bytes, int warmup, int iters,
                    float *ms_out) {
  if (!ms_out) return set_error(NKH_ERR_INVALID, "ms_out is null");
  if (iters <= 0 || warmup < 0)
    return set_error(NKH_ERR_INVALID, "iters must be > 0 and warmup >= 0");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  for (int i = 0; i < warmup; ++i) {
    rc = launch_locked(function, gx, gy, gz, bx, by, bz, shared_bytes, kernarg,
                       kernarg_bytes);
    if (rc) return rc;
  }
  hipEvent_t a, b;
  NKH_HIP(hipEventCreate(&a), "hipEventCreate");
  hipError_t e = hipEventCreate(&b);
  if (e != hipSuccess) {
    hipEventDestroy(a);
    return hip_error(e, "hipEventCreate");
  }
  e = hipEventRecord(a, g_rt.stream);
  for (int i = 0; e == hipSuccess && i < iters; ++i) {
    rc = launch_locked(function, gx, gy, gz, bx, by, bz, shared_bytes, kernarg,
                       kernarg_bytes);
    if (rc) break;
  }
  if (e == hipSuccess && rc == NKH_OK) e = hipEventRecord(b, g_rt.stream);
  if (e == hipSuccess && rc == NKH_OK) e = hipEventSynchronize(b);
  float ms = 0.f;
  if (e == hipSuccess && rc == NKH_OK) e = hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  if (rc) return rc;
  if (e != hipSuccess) return hip_error(e, "event timing");
  *ms_out = ms / static_cast<float>(iters);
  return NKH_OK;
}

int nkh_event_create(void **event) {
  if (!event) return set_error(NKH_ERR_INVALID, "event is null");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipEvent_t ev;
  NKH_HIP(hipEventCreate(&ev), "hipEventCreate");
  g_rt.events.insert(ev);
  *event = reinterpret_cast<void *>(ev);
  return NKH_OK;
}

int nkh_event_destroy(void *event) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipEvent_t ev = reinterpret_cast<hipEvent_t>(event);
  auto it = g_rt.events.find(ev);
  if (it == g_rt.events.end())
    return set_error(NKH_ERR_FREED, "event is not live");
  NKH_HIP(hipEventDestroy(ev), "hipEventDestroy");
  g_rt.events.erase(it);
  return NKH_OK;
}

int nkh_event_record(void *event) {
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipEvent_t ev = reinterpret_cast<hipEvent_t>(event);
  if (g_rt.events.find(ev) == g_rt.events.end())
    return set_error(NKH_ERR_FREED, "event is not live");
  NKH_HIP(hipEventRecord(ev, g_rt.stream), "hipEventRecord");
  return NKH_OK;
}

int nkh_event_elapsed_ms(void *start, void *stop, float *ms_out) {
  if (!ms_out) return set_error(NKH_ERR_INVALID, "ms_out is null");
  std::lock_guard<std::mutex> lk(g_mu);
  int rc = require_init();
  if (rc) return rc;
  hipEvent_t a = reinterpret_cast<hipEvent_t>(start);
  hipEvent_t b = reinterpret_cast<hipEvent_t>(stop);
  if (g_rt.events.find(a) == g_rt.events.end() ||
      g_rt.events.find(b) == g_rt.events.end())
    return set_error(NKH_ERR_FREED, "event is not live");
  NKH_HIP(hipEventSynchronize(b), "hipEventSynchronize");
  NKH_HIP(hipEventElapsedTime(ms_out, a, b), "hipEventElapsedTime");
  return NKH_OK;
}

}  // extern "C"
