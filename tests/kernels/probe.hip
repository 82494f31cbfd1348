// Test-only kernels: exercise the generic code-object loader (tm_module_load /
// tm_launch) and check the MFMA operand/result lane layouts that the library's
// kernels assume.  Built by __graft_entry__.build() into probe.hsaco.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));

extern "C" __global__ void probe_axpy(float* y, const float* x, float a, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a * x[i] + y[i];
}

// One wave.  A = identity (A[i][k] = i == k), B[k][j] = 100 k + j, so the
// result D[i][j] = 100 i + j reveals which (i, j) each accumulator holds when
// the assumed input layout is right.
//   16x16x32: A lane l holds A[l%16][8(l/16)+e], B lane l holds B[8(l/16)+e][l%16]
// out[l * 4 + e] = D element e of lane l.
extern "C" __global__ void probe_mfma16_layout(float* out) {
  int l = threadIdx.x;
  h8_t a, b;
  for (int e = 0; e < 8; ++e) {
    int k = 8 * (l / 16) + e;
    a[e] = (_Float16)((l % 16) == k ? 1.0f : 0.0f);
    b[e] = (_Float16)(float)(100 * k + (l % 16));
  }
  f4_t c = {0.f, 0.f, 0.f, 0.f};
  c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  for (int e = 0; e < 4; ++e) out[l * 4 + e] = c[e];
}

//   32x32x16: A lane l holds A[l%32][8(l/32)+e], B lane l holds B[8(l/32)+e][l%32]
// out[l * 16 + e] = D element e of lane l.
extern "C" __global__ void probe_mfma32_layout(float* out) {
  int l = threadIdx.x;
  h8_t a, b;
  for (int e = 0; e < 8; ++e) {
    int k = 8 * (l / 32) + e;
    a[e] = (_Float16)((l % 32) == k ? 1.0f : 0.0f);
    b[e] = (_Float16)(float)(100 * k + (l % 32));
  }
  f16_t c = {};
  c = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  for (int e = 0; e < 16; ++e) out[l * 16 + e] = c[e];
}

// 16x16x4 fp32: A lane l holds A[l%16][l/16], B lane l holds B[l/16][l%16].
// A[i][k] = (k == i%4) * (1 + i/4), B[k][j] = 100 k + j, so
// D[i][j] = (1 + i/4) * (100 (i%4) + j).  out[l * 4 + e] = D element e of lane l.
extern "C" __global__ void probe_mfma16x4_f32_layout(float* out) {
  int l = threadIdx.x;
  int i = l % 16, k = l / 16;
  float a = (k == i % 4) ? (float)(1 + i / 4) : 0.0f;
  float b = (float)(100 * k + (l % 16));
  f4_t c = {0.f, 0.f, 0.f, 0.f};
  c = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  for (int e = 0; e < 4; ++e) out[l * 4 + e] = c[e];
}
