// LM head ahead of the sampler: final LayerNorm + semantic_head linear
// (src/t2s/text2semantic.cpp:118-121 -> src/nn/nn.cpp:73-83 and :11-16) in one
// kernel, k_lmhead_fused, for weights in bf16, fp32 (the reference's own
// dtype: its .npy weights load as float32, include/c4tts/npy.h:202-206) or
// 8-bit affine groups (the quantized_matmul layout the reference uses for its
// projections, src/t2s/gpt2.cpp:49-62: w = scale * q + bias per group of
// `group` consecutive input elements).
// k_hbm_probe: streaming copy / read kernels for the achievable-bandwidth line.

#include <hip/hip_runtime.h>

#include "c4s_device.hpp"
#include "c4s_internal.h"

namespace c4s {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

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

// ---- LayerNorm folded into the GEMM (one kernel) -------------------------------------
//
// With y = (x - mu) * inv * gamma + beta (nn.cpp:73-83, inv = 1/sqrt(var + eps),
// biased variance) the head's output W y + b (nn.cpp:11-16) is
//   logits[m][n] = inv_m * (G[m][n] - mu_m * c[n]) + d[n] + b[n],
//   G[m][n] = sum_k W[n][k] gamma_k x[m][k],  c[n] = sum_k W[n][k] gamma_k,
//   d[n] = sum_k W[n][k] beta_k,  mu_m and var_m from sum_k x and sum_k x^2.
// So one pass reads W and x once and needs the statistics only in the
// epilogue. The MFMA operands are bf16: gamma_k x[m][k] (fp32) and gamma, beta
// enter as a hi + lo pair of bf16 (two MFMAs), which keeps them to about
// 2^-17 relative, so the logits follow the reference's fp32 LayerNorm + linear
// instead of a bf16-rounded activation. c and d come from a fifth row block
// whose rows 0 and 1 are gamma and beta.
//
// Weights: bf16 enter the MFMA as they are. fp32 weights are split into hi + lo
// bf16 as well; the products hi*hi + lo*hi + hi*lo (three MFMAs) leave out only
// lo*lo, about 2^-16 of 2^-8 relative. 8-bit codes are exact in bf16; a group
// of `group` inputs (SPU = group / 32 k-steps) accumulates sum q * a in a
// partial tile P and sum a in Q (an MFMA against ones), and the group adds
// scale[n] * P + bias[n] * Q to the tile.
//
// A workgroup owns 32 columns (vocabulary entries) and 64 rows; its four waves
// split K round-robin in units of SPU steps of 32 and issue every weight load
// of up to kSteps steps before the first MFMA; the waves' partial sums meet in
// LDS in a fixed order, so results are run-to-run stable.
constexpr int kFuseThreads = 256;
constexpr int kFuseWaves = kFuseThreads / kWave;

// v = hi + lo as two bf16 (round to nearest even), packed: the low halfword
// holds the first of a pair.
__device__ __forceinline__ void split2(float v0, float v1, uint32_t& hi, uint32_t& lo) {
  const uint16_t h0 = f32_to_bf16_rne(v0), h1 = f32_to_bf16_rne(v1);
  const uint16_t l0 = f32_to_bf16_rne(v0 - bf16_to_f32(h0)), l1 = f32_to_bf16_rne(v1 - bf16_to_f32(h1));
  hi = (uint32_t)h0 | ((uint32_t)h1 << 16);
  lo = (uint32_t)l0 | ((uint32_t)l1 << 16);
}

// Eight bf16 of x (one 16-byte fragment) times gamma: the hi and lo fragments
// of the products, and the sums of x and x^2 (zeros when the row is absent).
__device__ __forceinline__ void scaled_split(uint4 xq, float4 ga, float4 gb, bool in, uint4& hi, uint4& lo,
                                             float& s1, float& s2) {
  const uint32_t xw[4] = {xq.x, xq.y, xq.z, xq.w};
  const float gm[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
  uint32_t h[4], o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float x0 = in ? __uint_as_float(xw[q] << 16) : 0.0f;
    const float x1 = in ? __uint_as_float(xw[q] & 0xFFFF0000u) : 0.0f;
    s1 += x0;
    s1 += x1;
    s2 += x0 * x0;
    s2 += x1 * x1;
    split2(x0 * gm[2 * q], x1 * gm[2 * q + 1], h[q], o[q]);
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ void split_vec(float4 va, float4 vb, uint4& hi, uint4& lo) {
  split2(va.x, va.y, hi.x, lo.x);
  split2(va.z, va.w, hi.y, lo.y);
  split2(vb.x, vb.y, hi.z, lo.z);
  split2(vb.z, vb.w, hi.w, lo.w);
}

// Eight 8-bit codes as bf16 (exact: integers below 256 have at most 8
// significant bits).
__device__ __forceinline__ uint4 codes_bf16(uint2 q) {
  uint32_t o[4];
  const uint32_t wd[2] = {q.x, q.y};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t v = wd[i >> 1] >> (16 * (i & 1));
    const uint32_t lo = __float_as_uint((float)(v & 0xFFu)) >> 16;
    const uint32_t hi = __float_as_uint((float)((v >> 8) & 0xFFu)) >> 16;
    o[i] = lo | (hi << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// One lane's raw weight fragment: 8 consecutive k of one column.
template <int WK> struct WRaw;
template <> struct WRaw<kLmW_BF16> {
  uint4 v;
  __device__ void load(const void* w, int64_t off) { v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + off); }
};
template <> struct WRaw<kLmW_F32> {
  float4 a, b;
  __device__ void load(const void* w, int64_t off) {
    const float* p = static_cast<const float*>(w) + off;
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
};
template <> struct WRaw<kLmW_Q8> {
  uint2 v;
  __device__ void load(const void* w, int64_t off) { v = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(w) + off); }
};

// c += a * w for one 16x16x32 block: a as hi + lo, w as the raw fragment.
template <int WK>
__device__ __forceinline__ f32x4 mac(uint4 ah, uint4 al, const WRaw<WK>& w, f32x4 c) {
  if constexpr (WK == kLmW_F32) {
    uint4 wh, wl;
    split_vec(w.a, w.b, wh, wl);
    c = mfma_bf16(ah, wh, c);
    c = mfma_bf16(al, wh, c);
    return mfma_bf16(ah, wl, c);
  } else {
    uint4 b;
    if constexpr (WK == kLmW_Q8) b = codes_bf16(w.v); else b = w.v;
    c = mfma_bf16(ah, b, c);
    return mfma_bf16(al, b, c);
  }
}

// WK: weight kind; SPU: k-steps of 32 per scale group (1 unless 8-bit).
template <int WK, int SPU>
__global__ __launch_bounds__(kFuseThreads) void k_lmhead_fused(LmHeadArgs a) {
  constexpr int kSteps = WK == kLmW_F32 ? 4 : 8;   // weight k-steps a wave keeps in flight (registers)
  constexpr int kUnits = kSteps / SPU;
  constexpr bool kQ = WK == kLmW_Q8;
  __shared__ float red[kFuseWaves][kTileM + 2][kTileN + 1];
  __shared__ float st1[kFuseWaves][kTileM], st2[kFuseWaves][kTileM];
  const int n0 = blockIdx.x * kTileN;
  const int m0 = blockIdx.y * kTileM;
  const int D = a.D, V = a.V, M = a.M;
  const int w = wave_id(), l = lane_id();
  const int r = l & 15, g = l >> 4;
  // acc[0..3][nt]: row blocks of x; acc[4][nt]: rows 0 (gamma) and 1 (beta)
  f32x4 acc[5][2];
#pragma unroll
  for (int i = 0; i < 5; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float s1[4] = {0.f, 0.f, 0.f, 0.f}, s2[4] = {0.f, 0.f, 0.f, 0.f};
  const int col[2] = {min(n0 + r, V - 1), min(n0 + 16 + r, V - 1)};
  const int64_t woff[2] = {(int64_t)col[0] * D + 8 * g, (int64_t)col[1] * D + 8 * g};
  const uint16_t* xrow[4];
  bool xin[4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int m = m0 + mt * 16 + r;
    xin[mt] = m < M;
    xrow[mt] = a.hidden + (int64_t)min(m, M - 1) * D + 8 * g;
  }
  const int ngroups = D / (32 * SPU);
  const int mine = (ngroups - w + kFuseWaves - 1) / kFuseWaves;   // this wave's units: w, w + 4, ...
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  for (int base = 0; base < mine; base += kUnits) {
    // every weight fragment of these units in flight first
    WRaw<WK> wr[kUnits][SPU][2];
    float qs[kUnits][2], qb[kUnits][2];
#pragma unroll
    for (int i = 0; i < kUnits; ++i) {
      const int u = w + kFuseWaves * min(base + i, mine - 1);   // past the end: a repeated unit, not used
#pragma unroll
      for (int j = 0; j < SPU; ++j)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) wr[i][j][nt].load(a.weight, woff[nt] + (u * SPU + j) * 32);
      if constexpr (kQ) {
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
          qs[i][nt] = a.wscale[(int64_t)col[nt] * ngroups + u];
          qb[i][nt] = a.wbias[(int64_t)col[nt] * ngroups + u];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kUnits; ++i) {
      if (base + i < mine) {
        const int u = w + kFuseWaves * (base + i);
        f32x4 P[5][2], Q[5];
        if constexpr (kQ) {
#pragma unroll
          for (int mt = 0; mt < 5; ++mt) {
            Q[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
            P[mt][0] = P[mt][1] = Q[mt];
          }
        }
#pragma unroll
        for (int j = 0; j < SPU; ++j) {
          const int k0 = (u * SPU + j) * 32;
          const int kk = k0 + 8 * g;
          const float4 ga = *reinterpret_cast<const float4*>(a.gamma + kk);
          const float4 gb = *reinterpret_cast<const float4*>(a.gamma + kk + 4);
#pragma unroll
          for (int mt = 0; mt < 5; ++mt) {
            uint4 ah, al;
            if (mt < 4) {
              scaled_split(*reinterpret_cast<const uint4*>(xrow[mt] + k0), ga, gb, xin[mt], ah, al, s1[mt], s2[mt]);
            } else {
              ah = make_uint4(0u, 0u, 0u, 0u);
              al = ah;
              if (r == 0) {
                split_vec(ga, gb, ah, al);
              } else if (r == 1) {
                split_vec(*reinterpret_cast<const float4*>(a.beta + kk),
                          *reinterpret_cast<const float4*>(a.beta + kk + 4), ah, al);
              }
            }
            if constexpr (kQ) {
              P[mt][0] = mac<WK>(ah, al, wr[i][j][0], P[mt][0]);
              P[mt][1] = mac<WK>(ah, al, wr[i][j][1], P[mt][1]);
              Q[mt] = mfma_bf16(ah, ones, Q[mt]);
              Q[mt] = mfma_bf16(al, ones, Q[mt]);
            } else {
              acc[mt][0] = mac<WK>(ah, al, wr[i][j][0], acc[mt][0]);
              acc[mt][1] = mac<WK>(ah, al, wr[i][j][1], acc[mt][1]);
            }
          }
        }
        if constexpr (kQ) {
#pragma unroll
          for (int mt = 0; mt < 5; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
              for (int e = 0; e < 4; ++e) acc[mt][nt][e] += qs[i][nt] * P[mt][nt][e] + qb[i][nt] * Q[mt][e];
        }
      }
    }
  }
  // row statistics: the four lanes of a row (g = 0..3) hold its k sub-ranges
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    s1[mt] += __shfl_xor(s1[mt], 16, kWave);
    s1[mt] += __shfl_xor(s1[mt], 32, kWave);
    s2[mt] += __shfl_xor(s2[mt], 16, kWave);
    s2[mt] += __shfl_xor(s2[mt], 32, kWave);
    if (g == 0) { st1[w][mt * 16 + r] = s1[mt]; st2[w][mt * 16 + r] = s2[mt]; }
  }
  // 16x16 accumulator layout: lane l holds rows 4*(l/16)+i, column l%16.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[w][mt * 16 + 4 * g + i][nt * 16 + r] = acc[mt][nt][i];
  if (g == 0) {   // rows 0 (c) and 1 (d) of the fifth block
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      red[w][kTileM][nt * 16 + r] = acc[4][nt][0];
      red[w][kTileM + 1][nt * 16 + r] = acc[4][nt][1];
    }
  }
  __syncthreads();
  const double invD = 1.0 / (double)D;
  for (int o = threadIdx.x; o < kTileM * kTileN; o += kFuseThreads) {
    const int row = o / kTileN, cl = o % kTileN;
    const int n = n0 + cl, m = m0 + row;
    if (n < V && m < M) {
      double G = 0.0, cc = 0.0, dd = 0.0, S1 = 0.0, S2 = 0.0;
#pragma unroll
      for (int i = 0; i < kFuseWaves; ++i) {
        G += (double)red[i][row][cl];
        cc += (double)red[i][kTileM][cl];
        dd += (double)red[i][kTileM + 1][cl];
        S1 += (double)st1[i][row];
        S2 += (double)st2[i][row];
      }
      const double mu = S1 * invD;
      const double var = fmax(S2 * invD - mu * mu, 0.0);
      const double inv = 1.0 / sqrt(var + (double)a.eps);
      a.logits[(int64_t)m * a.ld_out + n] = (float)(inv * (G - mu * cc) + dd + (double)a.bias[n]);
    }
  }
}

// HBM probes: each workgroup streams one contiguous span with four independent
// 16-byte non-temporal loads per thread in flight.
constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;

__global__ __launch_bounds__(kProbeThreads) void k_hbm_copy(const f32x4* src, f32x4* dst, int64_t n) {
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(n, b0 + per);
  int64_t i = b0 + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * kProbeThreads < b1; i += kProbeUnroll * kProbeThreads) {
    f32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) __builtin_nontemporal_store(v[u], dst + i + u * kProbeThreads);
  }
  for (; i < b1; i += kProbeThreads) dst[i] = src[i];
}

__global__ __launch_bounds__(kProbeThreads) void k_hbm_read(const f32x4* src, float* dst, int64_t n) {
  const int64_t per = (n + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per, b1 = min(n, b0 + per);
  float acc = 0.0f;
  int64_t i = b0 + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * kProbeThreads < b1; i += kProbeUnroll * kProbeThreads) {
    f32x4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * kProbeThreads);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
  }
  for (; i < b1; i += kProbeThreads) {
    const f32x4 v = src[i];
    acc += (v[0] + v[1]) + (v[2] + v[3]);
  }
  if (acc == 1234.5f) dst[0] = acc;   // keeps the loads live; practically never stores
}

}  // namespace

template <int WK, int SPU>
static hipError_t launch_fused(const LmHeadArgs& a, hipStream_t s) {
  const dim3 grid((a.V + kTileN - 1) / kTileN, (a.M + kTileM - 1) / kTileM);
  hipLaunchKernelGGL((k_lmhead_fused<WK, SPU>), grid, dim3(kFuseThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_lmhead_fused(const LmHeadArgs& a, hipStream_t s) {
  switch (a.wkind) {
    case kLmW_BF16: return launch_fused<kLmW_BF16, 1>(a, s);
    case kLmW_F32: return launch_fused<kLmW_F32, 1>(a, s);
    case kLmW_Q8:
      if (a.group == 32) return launch_fused<kLmW_Q8, 1>(a, s);
      if (a.group == 64) return launch_fused<kLmW_Q8, 2>(a, s);
      if (a.group == 128) return launch_fused<kLmW_Q8, 4>(a, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_hbm_probe(const void* src, void* dst, int64_t bytes, int mode, hipStream_t s) {
  const int64_t n = bytes / 16;
  if (n <= 0) return hipSuccess;
  const int blocks = 256 * 8;
  if (mode == 0)
    hipLaunchKernelGGL(k_hbm_copy, dim3(blocks), dim3(kProbeThreads), 0, s, static_cast<const f32x4*>(src),
                       static_cast<f32x4*>(dst), n);
  else
    hipLaunchKernelGGL(k_hbm_read, dim3(blocks), dim3(kProbeThreads), 0, s, static_cast<const f32x4*>(src),
                       static_cast<float*>(dst), n);
  return hipGetLastError();
}

}  // namespace c4s
