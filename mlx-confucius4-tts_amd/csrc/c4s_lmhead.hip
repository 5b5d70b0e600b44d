// LM head ahead of the sampler: final LayerNorm + semantic_head linear
// (src/t2s/text2semantic.cpp:118-121 -> src/nn/nn.cpp:73-83 and :11-16).
//
// k_layernorm_bf16: one workgroup per hidden row; fp32 mean and biased
//   variance, y = (x - mean) / sqrt(var + eps) * gamma + beta, rounded to bf16
//   (the matrix engine's input type). Rows past M (up to the 64-row tile) are
//   written as zeros so the GEMM never reads undefined data.
// k_lmhead_gemm: logits[m][n] = sum_k h[m][k] * W[n][k] + bias[n] with
//   v_mfma_f32_16x16x32_bf16. A workgroup owns a 64-row x 32-column tile; its
//   four waves split K round-robin in steps of 32 and their fp32 partials are
//   summed through LDS in a fixed order, so results are run-to-run stable.
//   Every operand fragment is one 16-byte load straight from HBM/L2 (W rows
//   are K-contiguous), W is read exactly once.
// k_hbm_probe: streaming copy / read kernels for the achievable-bandwidth line.

#include <hip/hip_runtime.h>

#include "c4s_device.hpp"
#include "c4s_internal.h"

namespace c4s {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kLnThreads = 256;
constexpr int kGemmThreads = 256;
constexpr int kTileM = 64;
constexpr int kTileN = 32;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ float block_sum_f32_256(float v, float* red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  const float r = ((red[0] + red[1]) + red[2]) + red[3];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kLnThreads) void k_layernorm_bf16(LmHeadArgs a) {
  __shared__ float red[kLnThreads / kWave];
  const int m = blockIdx.x;
  const int D = a.D;
  uint16_t* out = a.hnorm + (int64_t)m * D;
  if (m >= a.M) {
    for (int d = threadIdx.x; d < D; d += kLnThreads) out[d] = 0;
    return;
  }
  const uint16_t* x = a.hidden + (int64_t)m * D;
  float s = 0.0f;
  for (int d = threadIdx.x; d < D; d += kLnThreads) s += bf16_to_f32(x[d]);
  const float mean = block_sum_f32_256(s, red) / (float)D;
  float v = 0.0f;
  for (int d = threadIdx.x; d < D; d += kLnThreads) {
    const float c = bf16_to_f32(x[d]) - mean;
    v += c * c;
  }
  const float var = block_sum_f32_256(v, red) / (float)D;
  const float denom = sqrtf(var + a.eps);
  for (int d = threadIdx.x; d < D; d += kLnThreads) {
    const float y = (bf16_to_f32(x[d]) - mean) / denom * a.gamma[d] + a.beta[d];
    out[d] = f32_to_bf16_rne(y);
  }
}

__global__ __launch_bounds__(kGemmThreads) void k_lmhead_gemm(LmHeadArgs a) {
  __shared__ float red[kGemmThreads / kWave][kTileM][kTileN + 1];
  const int n0 = blockIdx.x * kTileN;
  const int m0 = blockIdx.y * kTileM;
  const int D = a.D, V = a.V;
  const int w = wave_id(), l = lane_id();
  const int r = l & 15, g = l >> 4;
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint16_t* wrow0 = a.weight + (int64_t)min(n0 + r, V - 1) * D + 8 * g;
  const uint16_t* wrow1 = a.weight + (int64_t)min(n0 + 16 + r, V - 1) * D + 8 * g;
  const uint16_t* hrow = a.hnorm + (int64_t)(m0 + r) * D + 8 * g;
  const int ksteps = D / 32;
  for (int ks = w; ks < ksteps; ks += kGemmThreads / kWave) {
    const int k0 = ks * 32;
    const bf16x8 b0 = *reinterpret_cast<const bf16x8*>(wrow0 + k0);
    const bf16x8 b1 = *reinterpret_cast<const bf16x8*>(wrow1 + k0);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const bf16x8 am = *reinterpret_cast<const bf16x8*>(hrow + (int64_t)mt * 16 * D + k0);
      acc[mt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, b0, acc[mt][0], 0, 0, 0);
      acc[mt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, b1, acc[mt][1], 0, 0, 0);
    }
  }
  // 16x16 accumulator layout: lane l holds rows 4*(l/16)+i, column l%16.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[w][mt * 16 + 4 * g + i][nt * 16 + r] = acc[mt][nt][i];
  __syncthreads();
  for (int o = threadIdx.x; o < kTileM * kTileN; o += kGemmThreads) {
    const int row = o / kTileN, col = o % kTileN;
    const int n = n0 + col, m = m0 + row;
    if (n < V && m < a.M) {
      const float s = ((red[0][row][col] + red[1][row][col]) + red[2][row][col]) + red[3][row][col];
      a.logits[(int64_t)m * a.ld_out + n] = s + a.bias[n];
    }
  }
}

__global__ __launch_bounds__(256) void k_hbm_copy(const float4* src, float4* dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void k_hbm_read(const float4* src, float* dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  float acc = 0.0f;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float4 v = src[i];
    acc += (v.x + v.y) + (v.z + v.w);
  }
  if (acc == 1234.5f) dst[0] = acc;   // keeps the loads live; practically never stores
}

}  // namespace

hipError_t launch_layernorm_bf16(const LmHeadArgs& a, hipStream_t s) {
  const int rows = (a.M + kTileM - 1) / kTileM * kTileM;
  hipLaunchKernelGGL(k_layernorm_bf16, dim3(rows), dim3(kLnThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_lmhead_gemm(const LmHeadArgs& a, hipStream_t s) {
  const dim3 grid((a.V + kTileN - 1) / kTileN, (a.M + kTileM - 1) / kTileM);
  hipLaunchKernelGGL(k_lmhead_gemm, grid, dim3(kGemmThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_hbm_probe(const void* src, void* dst, int64_t bytes, int mode, hipStream_t s) {
  const int64_t n = bytes / 16;
  if (n <= 0) return hipSuccess;
  const int blocks = 256 * 8;
  if (mode == 0)
    hipLaunchKernelGGL(k_hbm_copy, dim3(blocks), dim3(256), 0, s, static_cast<const float4*>(src),
                       static_cast<float4*>(dst), n);
  else
    hipLaunchKernelGGL(k_hbm_read, dim3(blocks), dim3(256), 0, s, static_cast<const float4*>(src),
                       static_cast<float*>(dst), n);
  return hipGetLastError();
}

}  // namespace c4s
