// Runtime plumbing of libtm_hip.so: HIP symbol resolution, embedded code
// objects, error state, and the generic module loader / launcher exported as
// tm_module_* / tm_launch (the replacement of MetalUtils.load_binary and
// MetalUtils.launch, triton_metal/backend/driver.py:114-227).
#include "runtime.h"

#include <dlfcn.h>
#include <link.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <vector>

// Code objects embedded by embed.S (generated at build time): for each
// module NAME the symbols tm_co_NAME_start / tm_co_NAME_end.
#include "modules.inc"  // defines TM_MODULE_LIST(X): X(name) per module

#define TM_DECLARE_CO(name) \
  extern "C" const char tm_co_##name##_start[]; \
  extern "C" const char tm_co_##name##_end[];
TM_MODULE_LIST(TM_DECLARE_CO)
#undef TM_DECLARE_CO

namespace tmhip {
namespace {

thread_local std::string g_err;

struct CodeObject {
  const char* name;
  const char* start;
  const char* end;
};

const CodeObject kModules[] = {
#define TM_CO_ENTRY(name) {#name, tm_co_##name##_start, tm_co_##name##_end},
    TM_MODULE_LIST(TM_CO_ENTRY)
#undef TM_CO_ENTRY
};
constexpr int kNumModules = sizeof(kModules) / sizeof(kModules[0]);

std::mutex g_mu;
HipApi g_api;
bool g_api_ok = false;
bool g_api_tried = false;
hipModule_t g_mods[kMaxDevices][kNumModules];
bool g_mods_loaded[kMaxDevices];

// Find an already-loaded libamdhip64 in this process.
int find_loaded_cb(struct dl_phdr_info* info, size_t, void* data) {
  const char* n = info->dlpi_name;
  if (n && strstr(n, "libamdhip64.so")) {
    *(std::string*)data = n;
    return 1;
  }
  return 0;
}

void* open_runtime() {
  const char* names[] = {"libamdhip64.so", "libamdhip64.so.7", "libamdhip64.so.6"};
  for (const char* n : names)
    if (void* h = dlopen(n, RTLD_NOW | RTLD_NOLOAD)) return h;
  std::string path;
  dl_iterate_phdr(find_loaded_cb, &path);
  if (!path.empty())
    if (void* h = dlopen(path.c_str(), RTLD_NOW | RTLD_NOLOAD)) return h;
  if (const char* env = getenv("TM_HIP_RUNTIME"))
    if (void* h = dlopen(env, RTLD_NOW | RTLD_GLOBAL)) return h;
  for (const char* n : names)
    if (void* h = dlopen(n, RTLD_NOW | RTLD_GLOBAL)) return h;
  return nullptr;
}

template <class F> bool sym(void* h, F& out, const char* name) {
  out = (F)dlsym(h, name);
  return out != nullptr;
}

bool resolve_api() {
  void* h = open_runtime();
  if (!h) {
    fail(TM_ERR_NO_RUNTIME, "no HIP runtime (libamdhip64.so) could be loaded: %s", dlerror());
    return false;
  }
  bool ok = true;
  ok &= sym(h, g_api.GetDevice, "hipGetDevice");
  ok &= sym(h, g_api.GetDeviceCount, "hipGetDeviceCount");
  ok &= sym(h, g_api.DeviceGetAttribute, "hipDeviceGetAttribute");
  ok &= sym(h, g_api.GetDeviceProperties, "hipGetDevicePropertiesR0600");
  ok &= sym(h, g_api.ModuleLoadData, "hipModuleLoadData");
  ok &= sym(h, g_api.ModuleUnload, "hipModuleUnload");
  ok &= sym(h, g_api.ModuleGetFunction, "hipModuleGetFunction");
  ok &= sym(h, g_api.ModuleGetGlobal, "hipModuleGetGlobal");
  ok &= sym(h, g_api.FuncGetAttribute, "hipFuncGetAttribute");
  ok &= sym(h, g_api.ModuleLaunchKernel, "hipModuleLaunchKernel");
  ok &= sym(h, g_api.StreamSynchronize, "hipStreamSynchronize");
  ok &= sym(h, g_api.GetErrorString, "hipGetErrorString");
  ok &= sym(h, g_api.GetLastError, "hipGetLastError");
  if (!ok) {
    fail(TM_ERR_NO_RUNTIME, "HIP runtime lacks a required entry point");
    return false;
  }
  return true;
}

// Load every embedded module on `dev` (caller holds g_mu).
int load_modules_locked(int dev) {
  if (g_mods_loaded[dev]) return 0;
  for (int i = 0; i < kNumModules; ++i) {
    hipModule_t m = nullptr;
    hipError_t e = g_api.ModuleLoadData(&m, kModules[i].start);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) g_api.ModuleUnload(g_mods[dev][j]);
      return fail(TM_ERR_LOAD, "loading code object '%s' on device %d failed: %s",
                  kModules[i].name, dev, g_api.GetErrorString(e));
    }
    g_mods[dev][i] = m;
  }
  g_mods_loaded[dev] = true;
  return 0;
}

}  // namespace

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  const char* s = (g_api_ok && g_api.GetErrorString) ? g_api.GetErrorString(e) : "?";
  fail((int)e, "%s: HIP error %d (%s)", what, (int)e, s);
  return (int)e;
}

void clear_error() { g_err.clear(); }

const HipApi* api() {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_api_tried) {
    g_api_tried = true;
    g_api_ok = resolve_api();
  }
  return g_api_ok ? &g_api : nullptr;
}

int current_device(int* dev) {
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  hipError_t e = a->GetDevice(dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (*dev < 0 || *dev >= kMaxDevices) return fail(TM_ERR_UNSUPPORTED, "device %d", *dev);
  return 0;
}

int max_dynamic_lds() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (current_device(&dev)) return 65536;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int attr = 0;
  if (g_api.DeviceGetAttribute(&attr, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) !=
          hipSuccess ||
      attr <= 0) {
    g_api.GetLastError();
    attr = 65536;
  }
  cache[dev].store(attr, std::memory_order_relaxed);
  return attr;
}

int cu_count() {
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (current_device(&dev)) return 256;
  int v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int attr = 0;
  if (g_api.DeviceGetAttribute(&attr, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      attr <= 0) {
    g_api.GetLastError();
    attr = 256;
  }
  cache[dev].store(attr, std::memory_order_relaxed);
  return attr;
}

int Kernel::get(hipFunction_t* out) {
  int dev = 0;
  int rc = current_device(&dev);
  if (rc) return rc;
  hipFunction_t f = fn_[dev].load(std::memory_order_acquire);
  if (f) {
    *out = f;
    return 0;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  rc = load_modules_locked(dev);
  if (rc) return rc;
  for (int i = 0; i < kNumModules; ++i) {
    hipFunction_t g = nullptr;
    hipError_t e = g_api.ModuleGetFunction(&g, g_mods[dev][i], name_);
    if (e != hipSuccess) {
      // an expected miss in this module: do not leave it as the runtime's
      // sticky last error for the caller's next HIP call
      g_api.GetLastError();
      continue;
    }
    if (g) {
      fn_[dev].store(g, std::memory_order_release);
      *out = g;
      return 0;
    }
  }
  return fail(TM_ERR_NOT_FOUND, "kernel '%s' not found in the embedded code objects", name_);
}

int DeviceGlobal::get(void** ptr, size_t* bytes) {
  int dev = 0;
  int rc = current_device(&dev);
  if (rc) return rc;
  void* a = addr_[dev].load(std::memory_order_acquire);
  if (a) {
    *ptr = a;
    if (bytes) *bytes = bytes_[dev];
    return 0;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  rc = load_modules_locked(dev);
  if (rc) return rc;
  for (int i = 0; i < kNumModules; ++i) {
    hipDeviceptr_t d = nullptr;
    size_t n = 0;
    hipError_t e = g_api.ModuleGetGlobal(&d, &n, g_mods[dev][i], name_);
    if (e != hipSuccess || !d) {
      g_api.GetLastError();  // an expected miss in this module
      continue;
    }
    bytes_[dev] = n;
    addr_[dev].store((void*)d, std::memory_order_release);
    *ptr = (void*)d;
    if (bytes) *bytes = n;
    return 0;
  }
  return fail(TM_ERR_NOT_FOUND, "device global '%s' not found in the embedded code objects",
              name_);
}

}  // namespace tmhip

using namespace tmhip;

extern "C" {

int tm_init(void) { return api() ? 0 : TM_ERR_NO_RUNTIME; }

const char* tm_last_error(void) { return g_err.c_str(); }

const char* tm_version(void) { return "tm_hip 0.1 (gfx950)"; }

int tm_num_builtin_modules(void) { return kNumModules; }

int tm_builtin_get_function(const char* name, tm_function_t* out) {
  if (!name || !out) return fail(TM_ERR_INVALID_ARG, "tm_builtin_get_function: null argument");
  if (!api()) return TM_ERR_NO_RUNTIME;
  clear_error();
  static std::mutex mu;
  static std::map<std::string, Kernel*> table;
  Kernel* k;
  {
    std::lock_guard<std::mutex> lk(mu);
    auto it = table.find(name);
    if (it == table.end()) it = table.emplace(name, new Kernel(strdup(name))).first;
    k = it->second;
  }
  hipFunction_t f = nullptr;
  const int rc = k->get(&f);
  if (rc) return rc;
  *out = (tm_function_t)f;
  return 0;
}

const char* tm_builtin_module_name(int i) {
  return (i >= 0 && i < kNumModules) ? kModules[i].name : nullptr;
}

int tm_device_info(int device, char* arch, size_t arch_len, int* cu_count,
                   int* max_shared_per_block, int* l2_bytes) {
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  int n = 0;
  hipError_t e = a->GetDeviceCount(&n);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (device < 0 || device >= n) return fail(TM_ERR_INVALID_ARG, "device %d of %d", device, n);
  hipDeviceProp_t p;
  memset(&p, 0, sizeof p);
  e = a->GetDeviceProperties(&p, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (arch && arch_len) {
    strncpy(arch, p.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = 0;
  }
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (max_shared_per_block) *max_shared_per_block = (int)p.sharedMemPerBlock;
  if (l2_bytes) *l2_bytes = p.l2CacheSize;
  return 0;
}

int tm_module_load(const void* image, size_t nbytes, tm_module_t* out) {
  if (!image || nbytes < 64 || !out) return fail(TM_ERR_INVALID_ARG, "tm_module_load: bad image");
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  hipModule_t m = nullptr;
  hipError_t e = a->ModuleLoadData(&m, image);
  if (e != hipSuccess) {
    a->GetLastError();
    fail(TM_ERR_LOAD, "hipModuleLoadData failed: %s", a->GetErrorString(e));
    return TM_ERR_LOAD;
  }
  *out = (tm_module_t)m;
  return 0;
}

int tm_module_unload(tm_module_t module) {
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  if (!module) return fail(TM_ERR_INVALID_ARG, "tm_module_unload: null module");
  hipError_t e = a->ModuleUnload((hipModule_t)module);
  return e == hipSuccess ? 0 : hip_fail(e, "hipModuleUnload");
}

int tm_module_get_function(tm_module_t module, const char* name, tm_function_t* out,
                           int* n_regs, int* n_spills, int* max_threads, int* shared_bytes) {
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  if (!module || !name || !out) return fail(TM_ERR_INVALID_ARG, "tm_module_get_function");
  hipFunction_t f = nullptr;
  hipError_t e = a->ModuleGetFunction(&f, (hipModule_t)module, name);
  if (e != hipSuccess || !f) {
    a->GetLastError();
    return fail(TM_ERR_NOT_FOUND, "kernel '%s' not found in module", name);
  }
  int v = 0;
  if (n_regs) *n_regs = a->FuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_NUM_REGS, f) == hipSuccess ? v : 0;
  if (n_spills)
    *n_spills = a->FuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, f) == hipSuccess ? v : 0;
  if (max_threads)
    *max_threads =
        a->FuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f) == hipSuccess ? v : 0;
  if (shared_bytes)
    *shared_bytes =
        a->FuncGetAttribute(&v, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f) == hipSuccess ? v : 0;
  *out = (tm_function_t)f;
  return 0;
}

int tm_launch(tm_function_t fn, unsigned gx, unsigned gy, unsigned gz, unsigned bx, unsigned by,
              unsigned bz, unsigned shared_bytes, void* stream, void** args) {
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  if (!fn) return fail(TM_ERR_INVALID_ARG, "tm_launch: null function");
  if (!gx || !gy || !gz || !bx || !by || !bz || (size_t)bx * by * bz > 1024)
    return fail(TM_ERR_INVALID_ARG, "tm_launch: invalid grid (%u,%u,%u) / block (%u,%u,%u)", gx,
                gy, gz, bx, by, bz);
  hipError_t e = a->ModuleLaunchKernel((hipFunction_t)fn, gx, gy, gz, bx, by, bz, shared_bytes,
                                       (hipStream_t)stream, args, nullptr);
  return e == hipSuccess ? 0 : hip_fail(e, "hipModuleLaunchKernel");
}

int tm_synchronize(void* stream) {
  const HipApi* a = api();
  if (!a) return TM_ERR_NO_RUNTIME;
  hipError_t e = a->StreamSynchronize((hipStream_t)stream);
  return e == hipSuccess ? 0 : hip_fail(e, "hipStreamSynchronize");
}

}  // extern "C"
