// Calibration program for rocprofv3's HBM counters. A profile of the verify
// step converts FETCH_SIZE / WRITE_SIZE (KiB per dispatch) into bytes by the
// ratio these two kernels of known size give on the same GPU:
//   k_cal_read  streams 64 MiB (every byte read once, nothing written)
//   k_cal_copy  copies 64 MiB into a second buffer (64 MiB read, 64 MiB written)
// so fetch factor = 64 MiB / FETCH_SIZE(k_cal_read) and
// write factor = 64 MiB / WRITE_SIZE(k_cal_copy).
#include <hip/hip_runtime.h>

#include <cstdio>

#define CAL_CHECK(x)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      fprintf(stderr, "hbm_cal: %s at line %d\n", hipGetErrorString(e_), __LINE__);    \
      return 1;                                                                        \
    }                                                                                  \
  } while (0)

__global__ __launch_bounds__(256) void k_cal_read(const float4* __restrict__ p, size_t n4, float* out) {
  float acc = 0.f;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) {
    const float4 v = p[i];
    acc += v.x + v.y + v.z + v.w;
  }
  if (acc == 1234.5f) out[blockIdx.x] = acc;  // never true for the zeroed input; keeps the loads
}

__global__ __launch_bounds__(256) void k_cal_copy(const float4* __restrict__ p, float4* __restrict__ q, size_t n4) {
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) q[i] = p[i];
}

int main() {
  const size_t bytes = (size_t)64 << 20, n4 = bytes / sizeof(float4);
  const unsigned blocks = 2048;
  float4 *a = nullptr, *b = nullptr;
  float* out = nullptr;
  CAL_CHECK(hipMalloc(&a, bytes));
  CAL_CHECK(hipMalloc(&b, bytes));
  CAL_CHECK(hipMalloc(&out, blocks * sizeof(float)));
  CAL_CHECK(hipMemset(a, 0, bytes));
  CAL_CHECK(hipDeviceSynchronize());
  for (int i = 0; i < 3; ++i) {
    hipLaunchKernelGGL(k_cal_read, dim3(blocks), dim3(256), 0, 0, a, n4, out);
    hipLaunchKernelGGL(k_cal_copy, dim3(blocks), dim3(256), 0, 0, a, b, n4);
  }
  CAL_CHECK(hipGetLastError());
  CAL_CHECK(hipDeviceSynchronize());
  CAL_CHECK(hipFree(a));
  CAL_CHECK(hipFree(b));
  CAL_CHECK(hipFree(out));
  printf("hbm_cal: 3 x (64 MiB read, 64 MiB copy)\n");
  return 0;
}
