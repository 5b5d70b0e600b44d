// LM head ahead of the sampler: final LayerNorm + semantic_head linear
// (src/t2s/text2semantic.cpp:118-121 -> src/nn/nn.cpp:73-83 and :11-16) in one
// kernel, k_lmhead, for weights in bf16, fp32 (the reference's own dtype: its
// .npy weights load as float32, include/c4tts/npy.h:202-206) or 8-bit affine
// groups (the quantized_matmul layout the reference uses for its projections,
// src/t2s/gpt2.cpp:49-62: w = scale * q + bias per group of `group`
// consecutive input elements).
// k_hbm_probe: streaming copy / read kernels for the achievable-bandwidth line.

#include <hip/hip_runtime.h>

#include "c4s_device.hpp"
#include "c4s_internal.h"

namespace c4s {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileM = 64;
constexpr int kTileN = 32;

// ---- LayerNorm folded into the GEMM (one kernel) -------------------------------------
//
// With y = (x - mu) * inv * gamma + beta (nn.cpp:73-83, inv = 1/sqrt(var + eps),
// biased variance) the head's output W y + b (nn.cpp:11-16) is
//   logits[m][n] = inv_m * (G[m][n] - mu_m * c[n]) + d[n] + b[n],
//   G[m][n] = sum_k (W[n][k] gamma_k) x[m][k],  c[n] = sum_k W[n][k] gamma_k,
//   d[n] = sum_k W[n][k] beta_k,  mu_m and var_m from sum_k x and sum_k x^2.
// One pass reads W and x once and needs the statistics only in the epilogue.
//
// x is bf16, so it enters the matrix engine as it is. gamma goes to the weight
// side: each lane forms W[n][k] gamma_k in fp32 for its eight k and splits it
// into hi + lo bf16 (two MFMAs; the pair keeps about 2^-17 relative), adding c
// and d in fp32 on the way; every weight element is converted once on the whole
// chip. fp32 weights take the same path; 8-bit codes q are converted to fp32,
// each step's partial tiles P = sum (q gamma) x and Q = sum gamma x (gamma
// against every column) enter the tile as scale[n] P + bias[n] Q. The row
// statistics come from the matrix engine too: sum_k x against a block of ones,
// sum_k x^2 as the diagonal of the 16x16 Gram block x x^T (bf16 products are
// exact in fp32).
//
// A workgroup owns 32 columns (vocabulary entries) and 64 rows. K goes in
// chunks of eight steps of 32 (256 inputs): the workgroup stages the chunk's
// rows of x in LDS with 16-byte loads that cover whole cache lines (32 KB, two
// buffers), and wave w takes the chunk's steps w and w + 4. The first two
// chunks' loads are issued before the weights (loads complete in issue order,
// so the first chunk does not wait behind the weight window); each later
// chunk's loads are issued two chunks ahead, ahead of that chunk's weights. gamma and beta of the chunk are
// staged with it (a step that loaded them itself would wait, in issue order,
// for the next chunk's rows). Each wave keeps the weights of its next kWin
// chunks in flight. Reading x straight
// from global memory in MFMA fragment order instead (16 rows, 64 bytes each,
// per load) stalled the L1 on tag conflicts and cost three times as long. The
// waves' partial sums meet in LDS (over the staging buffers) in a fixed order,
// so results are run-to-run stable. At most 256 registers a wave and 66 KB of
// LDS: two workgroups fit on a CU, so a grid of a few more tiles than CUs
// (V = 8194: 257) does not take a second round.
constexpr int kLmThreads = 256;
constexpr int kLmWaves = kLmThreads / kWave;
constexpr int kWaveSteps = 2;                                     // steps a wave takes per chunk
constexpr int kChunkK = kLmWaves * kWaveSteps * 32;               // inputs per chunk
constexpr int kXPitch = kChunkK * 2 + 16;                         // bytes per staged row (+16: conflict-free reads)
constexpr int kXLoads = kTileM * kChunkK * 2 / 16 / kLmThreads;   // 16-byte loads per thread per chunk
constexpr int kRowPieces = kChunkK / 8;                           // 16-byte pieces per staged row
constexpr size_t kXBytes = (size_t)kTileM * kXPitch;
constexpr int kRedPitch = kTileM + 4;                             // floats per column of a partial tile (+4: conflict-free)
constexpr size_t kRedBytes = (size_t)kLmWaves * kTileN * kRedPitch * 4;
static_assert(kRedBytes <= 2 * kXBytes, "the partial sums fit over the staging buffers");

// Two floats to two bf16, round to nearest even (v_cvt_pk_bf16_f32); the
// low halfword holds the first.
__device__ __forceinline__ uint32_t pack_bf16(float v0, float v1) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2{v0, v1}), bf16x2));
}

// v = hi + lo as two bf16 each, packed: lo rounds the exact residual v - hi.
__device__ __forceinline__ void split2(float v0, float v1, uint32_t& hi, uint32_t& lo) {
  hi = pack_bf16(v0, v1);
  lo = pack_bf16(v0 - __uint_as_float(hi << 16), v1 - __uint_as_float(hi & 0xFFFF0000u));
}

__device__ __forceinline__ void split8(const float (&v)[8], uint4& hi, uint4& lo) {
  split2(v[0], v[1], hi.x, lo.x);
  split2(v[2], v[3], hi.y, lo.y);
  split2(v[4], v[5], hi.z, lo.z);
  split2(v[6], v[7], hi.w, lo.w);
}

__device__ __forceinline__ f32x4 mfma_bf16(uint4 a, uint4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                 0, 0, 0);
}

// One lane's raw weight fragment (8 consecutive k of one column) and its
// values as fp32: the weight (bf16, fp32) or the code (8-bit).
template <int WK> struct WRaw;
template <> struct WRaw<kLmW_BF16> {
  uint4 v;
  __device__ void load(const void* w, int64_t off) { v = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(w) + off); }
  __device__ uint4 bf16() const { return v; }
  __device__ void get(float (&o)[8]) const {
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(q[i] << 16);
      o[2 * i + 1] = __uint_as_float(q[i] & 0xFFFF0000u);
    }
  }
};
template <> struct WRaw<kLmW_F32> {
  float4 a, b;
  __device__ void load(const void* w, int64_t off) {
    const float* p = static_cast<const float*>(w) + off;
    a = *reinterpret_cast<const float4*>(p);
    b = *reinterpret_cast<const float4*>(p + 4);
  }
  __device__ void get(float (&o)[8]) const {
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
};
template <> struct WRaw<kLmW_Q8> {
  uint2 v;
  __device__ void load(const void* w, int64_t off) { v = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(w) + off); }
  __device__ void get(float (&o)[8]) const {
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (float)(((i < 4 ? v.x : v.y) >> (8 * (i & 3))) & 0xFFu);
  }
  // the codes as bf16 (exact: integers below 256 have at most 8 significant bits)
  __device__ uint4 bf16() const {
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t q = (i < 2 ? v.x : v.y) >> (16 * (i & 1));
      o[i] = pack_bf16((float)(q & 0xFFu), (float)((q >> 8) & 0xFFu));
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// WK: weight kind; SPU: k-steps of 32 per scale group (1 unless 8-bit).
template <int WK, int SPU>
__global__ __launch_bounds__(kLmThreads) __attribute__((amdgpu_waves_per_eu(2))) void k_lmhead(LmHeadArgs a) {
  constexpr bool kQ = WK == kLmW_Q8;
  constexpr bool kCdMfma = WK != kLmW_F32;   // c and d on the matrix engine (the weights are bf16-exact)
  // chunks whose weights a wave keeps in flight (kWaveSteps steps each). Loads
  // complete in issue order, so a chunk's rows of x, issued two chunks ahead,
  // wait behind every weight load issued before them: a window of two chunks
  // (refilled per chunk) instead of the whole of K for bf16 weights took
  // 64 x 1280 x 8194 from 15.7 to 13.8 us.
  constexpr int kWin = WK == kLmW_F32 ? 2 : (WK == kLmW_Q8 ? (SPU > 1 ? 2 : 3) : 2);
  __shared__ __align__(16) unsigned char xs[2 * kXBytes];
  __shared__ __align__(16) float gbs[2][2][kChunkK];   // by buffer: gamma, beta of the chunk
  // by buffer: gamma hi, gamma lo, beta hi, beta lo as bf16 (rows 0-3 of an MFMA
  // block whose product with the raw weights gives c and d; bf16 / 8-bit only)
  __shared__ __align__(16) uint16_t cda[kCdMfma ? 2 : 1][4][kChunkK];
  __shared__ float st1[kLmWaves][kTileM], st2[kLmWaves][kTileM];
  __shared__ float scd[kLmWaves][2][kTileN];
  __shared__ float rmu[kTileM], rinv[kTileM], ccol[kTileN], dcol[kTileN];
  float (*red)[kTileN][kRedPitch] = reinterpret_cast<float (*)[kTileN][kRedPitch]>(xs);   // [wave][column][row]
  const int n0 = blockIdx.x * kTileN;
  const int m0 = blockIdx.y * kTileM;
  const int D = a.D, V = a.V, M = a.M;
  const int t = threadIdx.x, w = wave_id(), l = lane_id();
  const int r = l & 15, g = l >> 4;
  const int nsteps = D / 32, nchunks = (nsteps + kLmWaves * kWaveSteps - 1) / (kLmWaves * kWaveSteps);
  // per row block: the two column blocks, then the ones and the Gram products
  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float cp[2] = {0.f, 0.f}, dp[2] = {0.f, 0.f};   // fp32 weights: this lane's parts of c and d
  f32x4 acd[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};   // the c / d block by column block
  const int col[2] = {min(n0 + r, V - 1), min(n0 + 16 + r, V - 1)};
  const bool live1 = n0 + 16 < V;   // the second column block holds a column (uniform)
  const int64_t woff[2] = {(int64_t)col[0] * D + 8 * g, (int64_t)col[1] * D + 8 * g};
  const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
  // staging: piece j of this thread is row (kLmThreads / kRowPieces) j + t / kRowPieces,
  // 16-byte column t % kRowPieces
  constexpr int kRowsPerLoad = kLmThreads / kRowPieces;
  static_assert(kRowsPerLoad * kXLoads == kTileM, "staging layout");
  const int tr = t / kRowPieces, tc = (t % kRowPieces) * 8;
  // chunk ch's piece j of this thread (past D, a partial last chunk: an
  // in-bounds piece that is not used)
  auto x_piece = [&](int ch, int j) {
    const int k = ch * kChunkK + tc;
    return *reinterpret_cast<const uint4*>(a.hidden + (int64_t)min(m0 + kRowsPerLoad * j + tr, M - 1) * D +
                                           (k < D ? k : 0));
  };
  auto x_lds = [&](int buf, int j) {
    return reinterpret_cast<uint4*>(&xs[buf * kXBytes + (kRowsPerLoad * j + tr) * kXPitch + tc * 2]);
  };
  // gamma (threads 0 .. 63) and beta (64 .. 127): four floats of the chunk each
  constexpr int kGbPieces = kChunkK / 4;
  const bool gb_t = t < 2 * kGbPieces;
  const int gb_a = t / kGbPieces, gb_o = (t % kGbPieces) * 4;
  auto gb_piece = [&](int ch) {
    const int k = ch * kChunkK + gb_o;
    return *reinterpret_cast<const float4*>((gb_a ? a.beta : a.gamma) + (k < D ? k : 0));
  };
  auto gb_store = [&](int buf, float4 v) {
    *reinterpret_cast<float4*>(&gbs[buf][gb_a][gb_o]) = v;
    if constexpr (kCdMfma) {
      uint32_t h0, l0, h1, l1;
      split2(v.x, v.y, h0, l0);
      split2(v.z, v.w, h1, l1);
      *reinterpret_cast<uint2*>(&cda[buf][2 * gb_a][gb_o]) = make_uint2(h0, h1);
      *reinterpret_cast<uint2*>(&cda[buf][2 * gb_a + 1][gb_o]) = make_uint2(l0, l1);
    }
  };
  // the first two chunks' rows, then the weight window (slot i: the steps of chunk i)
  uint4 xv[kXLoads];
  float4 gv = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < kXLoads; ++j) *x_lds(0, j) = x_piece(0, j);
  if (gb_t) gb_store(0, gb_piece(0));
#pragma unroll
  for (int j = 0; j < kXLoads; ++j) xv[j] = x_piece(min(1, nchunks - 1), j);
  if (gb_t) gv = gb_piece(min(1, nchunks - 1));
  WRaw<WK> wr[kWin][kWaveSteps][2];
  float qs[kQ ? kWin : 1][kWaveSteps][2], qb[kQ ? kWin : 1][kWaveSteps][2];   // 8-bit: scale and offset
  auto w_load = [&](int i, int ch) {
#pragma unroll
    for (int h = 0; h < kWaveSteps; ++h) {
      const int step = min(ch * kLmWaves * kWaveSteps + h * kLmWaves + w, nsteps - 1);   // past the end: unused
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        if (nt == 1 && !live1) continue;
        wr[i][h][nt].load(a.weight, woff[nt] + step * 32);
        if constexpr (kQ) {
          const int64_t q = (int64_t)col[nt] * (nsteps / SPU) + step / SPU;
          qs[i][h][nt] = a.wscale[q];
          qb[i][h][nt] = a.wbias[q];
        }
      }
    }
  };
#pragma unroll
  for (int i = 0; i < kWin; ++i) w_load(i, i);
  __syncthreads();
  for (int base = 0; base < nchunks; base += kWin) {
#pragma unroll
    for (int i = 0; i < kWin; ++i) {
      const int ch = base + i;
      if (ch < nchunks) {   // uniform over the workgroup
        // the next chunk into the other buffer (last read before the previous
        // barrier), then the chunk after it in flight
        if (ch + 1 < nchunks) {
#pragma unroll
          for (int j = 0; j < kXLoads; ++j) *x_lds((ch + 1) & 1, j) = xv[j];
          if (gb_t) gb_store((ch + 1) & 1, gv);
        }
#pragma unroll
        for (int j = 0; j < kXLoads; ++j) xv[j] = x_piece(min(ch + 2, nchunks - 1), j);
        if (gb_t) gv = gb_piece(min(ch + 2, nchunks - 1));
#pragma unroll
        for (int h = 0; h < kWaveSteps; ++h) {
          const int step = ch * kLmWaves * kWaveSteps + h * kLmWaves + w;
          if (step < nsteps) {
            const int kc = (h * kLmWaves + w) * 32 + 8 * g;   // this lane's k within the chunk
            const float* gl_ = gbs[ch & 1][0] + kc;
            const float* bl_ = gbs[ch & 1][1] + kc;
            const float4 ga = *reinterpret_cast<const float4*>(gl_), gb = *reinterpret_cast<const float4*>(gl_ + 4);
            const float4 ba = *reinterpret_cast<const float4*>(bl_), bb = *reinterpret_cast<const float4*>(bl_ + 4);
            const float gm[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
            const float bt[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
            uint4 bh[2], bl[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
              if (nt == 1 && !live1) continue;
              float wv[8], wg[8];
              wr[i][h][nt].get(wv);
              float c1 = 0.f, d1 = 0.f;
#pragma unroll
              for (int e = 0; e < 8; ++e) {
                wg[e] = wv[e] * gm[e];
                if constexpr (!kCdMfma) {
                  c1 += wg[e];
                  d1 = __builtin_fmaf(wv[e], bt[e], d1);
                }
              }
              split8(wg, bh[nt], bl[nt]);
              if constexpr (!kCdMfma) {
                cp[nt] += c1;
                dp[nt] += d1;
              }
            }
            uint4 gh, gl;
            float qsc[2] = {0.f, 0.f}, qbi[2] = {0.f, 0.f};
            if constexpr (kQ) {
              split8(gm, gh, gl);
#pragma unroll
              for (int nt = 0; nt < 2; ++nt) {
                qsc[nt] = qs[i][h][nt];
                qbi[nt] = qb[i][h][nt];
              }
            }
            if constexpr (kCdMfma) {
              // c and d: rows 0-3 (gamma hi, lo, beta hi, lo) against the raw weights
              uint4 cdf = make_uint4(0u, 0u, 0u, 0u);
              if (r < 4) cdf = *reinterpret_cast<const uint4*>(&cda[ch & 1][r][kc]);
              if constexpr (kQ) {
                f32x4 Q = mfma_bf16(cdf, ones, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                  const f32x4 P = mfma_bf16(cdf, wr[i][h][nt].bf16(), f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                  for (int e = 0; e < 4; ++e) acd[nt][e] = __builtin_fmaf(qsc[nt], P[e], __builtin_fmaf(qbi[nt], Q[e], acd[nt][e]));
                }
              } else {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                  if (nt == 0 || live1) acd[nt] = mfma_bf16(cdf, wr[i][h][nt].bf16(), acd[nt]);
              }
            }
            const unsigned char* xb = &xs[(ch & 1) * kXBytes + kc * 2];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) {
              const uint4 xa = *reinterpret_cast<const uint4*>(xb + (mt * 16 + r) * kXPitch);
              if constexpr (kQ) {
                f32x4 P0 = f32x4{0.f, 0.f, 0.f, 0.f}, P1 = P0, Q = P0;
                P0 = mfma_bf16(xa, bh[0], P0);
                P0 = mfma_bf16(xa, bl[0], P0);
                P1 = mfma_bf16(xa, bh[1], P1);
                P1 = mfma_bf16(xa, bl[1], P1);
                Q = mfma_bf16(xa, gh, Q);
                Q = mfma_bf16(xa, gl, Q);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  acc[mt][0][e] = __builtin_fmaf(qsc[0], P0[e], __builtin_fmaf(qbi[0], Q[e], acc[mt][0][e]));
                  acc[mt][1][e] = __builtin_fmaf(qsc[1], P1[e], __builtin_fmaf(qbi[1], Q[e], acc[mt][1][e]));
                }
              } else {
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                  if (nt == 1 && !live1) continue;
                  acc[mt][nt] = mfma_bf16(xa, bh[nt], acc[mt][nt]);
                  acc[mt][nt] = mfma_bf16(xa, bl[nt], acc[mt][nt]);
                }
              }
              acc[mt][2] = mfma_bf16(xa, ones, acc[mt][2]);
              acc[mt][3] = mfma_bf16(xa, xa, acc[mt][3]);
            }
          }
        }
        // refill this slot with the steps kWin chunks later
        if (ch + kWin < nchunks) w_load(i, ch + kWin);
        __syncthreads();
      }
    }
  }
  // (the last barrier: every wave is done with the staging buffers)
  // 16x16 accumulator layout: lane l holds rows 4*(l/16)+i, column l%16.
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)   // rows 4g .. 4g + 3 of column r: one 16-byte store
      *reinterpret_cast<f32x4*>(&red[w][nt * 16 + r][mt * 16 + 4 * g]) = acc[mt][nt];
    if (r == 0)   // every column of the ones product holds the row sums
#pragma unroll
      for (int i = 0; i < 4; ++i) st1[w][mt * 16 + 4 * g + i] = acc[mt][2][i];
    if ((r >> 2) == g) {   // the Gram diagonal: row r at column r
      const int i = r & 3;
      const float dg = i == 0 ? acc[mt][3][0] : (i == 1 ? acc[mt][3][1] : (i == 2 ? acc[mt][3][2] : acc[mt][3][3]));
      st2[w][mt * 16 + r] = dg;
    }
  }
  // c and d of this wave's steps
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float cc, dd;
    if constexpr (kCdMfma) {   // lanes 0-15 hold rows 0-3 (gamma hi, lo, beta hi, lo) at column r
      cc = acd[nt][0] + acd[nt][1];
      dd = acd[nt][2] + acd[nt][3];
    } else {                   // the four lanes of a column (g = 0..3) hold its k sub-ranges
      cc = cp[nt];
      dd = dp[nt];
      cc += __shfl_xor(cc, 16, kWave);
      cc += __shfl_xor(cc, 32, kWave);
      dd += __shfl_xor(dd, 16, kWave);
      dd += __shfl_xor(dd, 32, kWave);
    }
    if (g == 0) {
      scd[w][0][nt * 16 + r] = cc;
      scd[w][1][nt * 16 + r] = dd;
    }
  }
  __syncthreads();
  // per row: mean and 1/sqrt(var + eps); per column: c and d + bias
  if (t < kTileM) {
    double S1 = 0.0, S2 = 0.0;
#pragma unroll
    for (int i = 0; i < kLmWaves; ++i) {
      S1 += (double)st1[i][t];
      S2 += (double)st2[i][t];
    }
    const double invD = 1.0 / (double)D;
    const double mu = S1 * invD;
    rmu[t] = (float)mu;
    rinv[t] = (float)(1.0 / sqrt(fmax(S2 * invD - mu * mu, 0.0) + (double)a.eps));
  } else if (t < kTileM + kTileN) {
    const int cl = t - kTileM;
    double cc = 0.0, dd = 0.0;
#pragma unroll
    for (int i = 0; i < kLmWaves; ++i) {
      cc += (double)scd[i][0][cl];
      dd += (double)scd[i][1][cl];
    }
    ccol[cl] = (float)cc;
    dcol[cl] = (float)(dd + (double)a.bias[min(n0 + cl, V - 1)]);
  }
  __syncthreads();
  for (int o = t; o < kTileM * kTileN; o += kLmThreads) {
    const int row = o / kTileN, cl = o % kTileN;
    const int n = n0 + cl, m = m0 + row;
    if (n < V && m < M) {
      float G = 0.0f;
#pragma unroll
      for (int i = 0; i < kLmWaves; ++i) G += red[i][cl][row];
      a.logits[(int64_t)m * a.ld_out + n] = __builtin_fmaf(rinv[row], __builtin_fmaf(-rmu[row], ccol[cl], G), dcol[cl]);
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
static hipError_t launch_k(const LmHeadArgs& a, hipStream_t s) {
  const dim3 grid((a.V + kTileN - 1) / kTileN, (a.M + kTileM - 1) / kTileM);
  hipLaunchKernelGGL((k_lmhead<WK, SPU>), grid, dim3(kLmThreads), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_lmhead(const LmHeadArgs& a, hipStream_t s) {
  switch (a.wkind) {
    case kLmW_BF16: return launch_k<kLmW_BF16, 1>(a, s);
    case kLmW_F32: return launch_k<kLmW_F32, 1>(a, s);
    case kLmW_Q8:
      if (a.group == 32) return launch_k<kLmW_Q8, 1>(a, s);
      if (a.group == 64) return launch_k<kLmW_Q8, 2>(a, s);
      if (a.group == 128) return launch_k<kLmW_Q8, 4>(a, s);
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
