// Host-side runtime of libtm_hip.so: HIP entry points resolved from the HIP
// runtime already present in the process, per-device code-object cache,
// thread-local error state and a typed launch helper.
#pragma once
#include <hip/hip_runtime_api.h>

#include <atomic>
#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>

#include "tm_hip.h"

namespace tmhip {

// HIP runtime entry points (resolved with dlsym; the library never links
// libamdhip64 so that it shares the caller's runtime instead of loading a
// second copy).
struct HipApi {
  hipError_t (*GetDevice)(int*);
  hipError_t (*GetDeviceCount)(int*);
  hipError_t (*DeviceGetAttribute)(int*, hipDeviceAttribute_t, int);
  hipError_t (*GetDeviceProperties)(hipDeviceProp_t*, int);
  hipError_t (*ModuleLoadData)(hipModule_t*, const void*);
  hipError_t (*ModuleUnload)(hipModule_t);
  hipError_t (*ModuleGetFunction)(hipFunction_t*, hipModule_t, const char*);
  hipError_t (*ModuleGetGlobal)(hipDeviceptr_t*, size_t*, hipModule_t, const char*);
  hipError_t (*FuncGetAttribute)(int*, hipFunction_attribute, hipFunction_t);
  hipError_t (*ModuleLaunchKernel)(hipFunction_t, unsigned, unsigned, unsigned, unsigned,
                                   unsigned, unsigned, unsigned, hipStream_t, void**, void**);
  hipError_t (*StreamSynchronize)(hipStream_t);
  const char* (*GetErrorString)(hipError_t);
  hipError_t (*GetLastError)(void);
};

// Returns nullptr (and sets the error) when no runtime can be resolved.
const HipApi* api();

// Error helpers: set the thread-local message and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int hip_fail(hipError_t e, const char* what);
void clear_error();

constexpr int kMaxDevices = 64;

// A kernel in one of the embedded code objects, resolved lazily per device.
class Kernel {
 public:
  explicit Kernel(const char* name) : name_(name) {
    for (auto& f : fn_) f.store(nullptr, std::memory_order_relaxed);
  }
  // Resolve for the current device; returns 0 or an error code.
  int get(hipFunction_t* out);
  const char* name() const { return name_; }

 private:
  const char* name_;
  std::atomic<hipFunction_t> fn_[kMaxDevices];
};

// A __device__ global of one of the embedded code objects: its address on
// each device, resolved once per device (with that device current) through
// hipModuleGetGlobal on the module loaded there, the module-API counterpart
// of hipGetSymbolAddress.  Host code holds only the returned device address.
class DeviceGlobal {
 public:
  explicit DeviceGlobal(const char* name) : name_(name) {
    for (auto& a : addr_) a.store(nullptr, std::memory_order_relaxed);
  }
  // Address and size on the current device; returns 0 or an error code.
  int get(void** ptr, size_t* bytes);

 private:
  const char* name_;
  std::atomic<void*> addr_[kMaxDevices];
  size_t bytes_[kMaxDevices] = {};
};

int current_device(int* dev);
// Largest dynamic LDS allocation per workgroup on the current device (bytes).
int max_dynamic_lds();
// Compute units of the current device (256 if the query fails).
int cu_count();
// The kernel of this name (created on first use, kept for the process).
Kernel& kernel_named(const std::string& name);

// Launch helper: args are passed by value and forwarded as kernelParams.
template <class... Args>
int launch(Kernel& k, dim3 grid, dim3 block, unsigned shared, void* stream, Args... args) {
  hipFunction_t f = nullptr;
  int rc = k.get(&f);
  if (rc) return rc;
  void* params[] = {(void*)&args..., nullptr};
  hipError_t e = api()->ModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                           shared, (hipStream_t)stream, params, nullptr);
  if (e != hipSuccess) return hip_fail(e, k.name());
  return 0;
}

// tm_dot's implementation (ops_dot.cpp), shared with tm_matmul's FP8 path.
int dot_impl(const char* op, const void* A, const void* B, void* C, const void* Z, const void* W,
             int batch, int M, int N, int K, int L, const long long* strides, int epilogue,
             int in_dtype, int out_dtype, int z_dtype, int w_dtype, void* stream);
// The fp32-MFMA dense kernel (ops_gemm.cpp), shared with tm_dot's fp32 path:
// C[M, N] = A[M, K] @ B (B [K, N], or [N, K] with bt), rows ldx apart.
int dense_f32(const float* A, const float* B, void* C, int M, int N, int K, int lda, int ldb,
              int ldc, bool bt, int out_dtype, void* stream);
// The 16-bit MFMA dense kernels (ops_gemm.cpp), shared with tm_dot: launches
// and sets *used when the dense selection picks an MFMA tile kernel for this
// call, else launches nothing and clears *used.
int dense_mfma(const void* A, const void* B, void* C, int M, int N, int K, int lda, int ldb,
               int ldc, bool bt, int in_dtype, int out_dtype, void* stream, bool* used);

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool is_half(int dt) { return dt == TM_DT_F16 || dt == TM_DT_BF16; }
inline bool is_float(int dt) { return dt == TM_DT_F32 || dt == TM_DT_F16 || dt == TM_DT_BF16; }

}  // namespace tmhip
