// Test-only kernels: run the wave64 DPP primitives of c4s_device.hpp on given
// inputs so tests/test_gpu_primitives.py can check them against the host.
// One workgroup of 64 threads per case; every access is within the case's
// 64-element arrays.
#include <hip/hip_runtime.h>

#include "../../mlx-confucius4-tts_amd/csrc/c4s_chain.hpp"

using namespace c4s;

__global__ __launch_bounds__(64) void k_selftest(const uint32_t* u_in, const double* d_in,
                                                 const float* f_in, uint32_t* u_scan,
                                                 double* d_scan, float* f_max, double* d_sum) {
  const int l = threadIdx.x;
  u_scan[l] = wave_scan_u32(u_in[l]);
  d_scan[l] = wave_scan_f64(d_in[l]);
  f_max[l] = wave_max_dpp(f_in[l]);
  d_sum[l] = wave_sum_dpp(d_in[l]);
}

extern "C" int c4s_selftest_wave(const uint32_t* u_in, const double* d_in, const float* f_in,
                                 uint32_t* u_scan, double* d_scan, float* f_max, double* d_sum) {
  hipLaunchKernelGGL(k_selftest, dim3(1), dim3(64), 0, nullptr, u_in, d_in, f_in, u_scan, d_scan,
                     f_max, d_sum);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

__global__ __launch_bounds__(64) void k_selftest2(const uint32_t* u_in, const uint64_t* q_in,
                                                  uint32_t* u_next, uint32_t* u_max,
                                                  uint64_t* q_max) {
  const int l = threadIdx.x;
  u_next[l] = wave_next_u32(u_in[l], 0xdeadbeefu);
  u_max[l] = wave_max_u32_dpp(u_in[l]);
  q_max[l] = wave_max_u64_dpp(q_in[l]);
}

extern "C" int c4s_selftest_wave2(const uint32_t* u_in, const uint64_t* q_in, uint32_t* u_next,
                                  uint32_t* u_max, uint64_t* q_max) {
  hipLaunchKernelGGL(k_selftest2, dim3(1), dim3(64), 0, nullptr, u_in, q_in, u_next, u_max, q_max);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// lane_draw on n_cases sets of 64 lanes (kept flag, id, id-order slot, mass)
// with one uniform each; writes the token and the exact-replay flag per case.
__global__ __launch_bounds__(64) void k_selftest_draw(const uint8_t* kept, const int* id,
                                                      const int* slot, const double* e,
                                                      const double* u, int V, int* out) {
  const int c = blockIdx.x, l = threadIdx.x;
  const int i = 64 * c + l;
  uint32_t ex = 0;
  const int tok = lane_draw(kept[i] != 0, id[i], slot[i], e[i], u[c], V, ex);
  if (l == 0) { out[2 * c] = tok; out[2 * c + 1] = (int)ex; }
}

extern "C" int c4s_selftest_draw(const uint8_t* kept, const int* id, const int* slot, const double* e,
                                 const double* u, int V, int n_cases, int* out) {
  if (n_cases <= 0) return 1;
  hipLaunchKernelGGL(k_selftest_draw, dim3(n_cases), dim3(64), 0, nullptr, kept, id, slot, e, u, V, out);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
