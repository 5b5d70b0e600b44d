// Launch descriptors shared by the HIP kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace c4s {

// Per-row processor selection (kernel side of the public C4S_* mode bits).
enum : uint32_t {
  kPenalty = 1u << 0,
  kTemperature = 1u << 1,
  kTopK = 1u << 2,
  kTopP = 1u << 3,
  kArgmax = 1u << 4,
  kDraw = 1u << 5,
  kCustom = 1u << 8,
};

// Rows at or below this vocabulary size are staged whole in LDS (one
// workgroup per row); larger rows are streamed from HBM in several passes.
constexpr int kLdsVocabMax = 12288;
constexpr int kMaxVocab = 1 << 20;
constexpr int kThreads = 1024;

// Per-row statistics written when the caller asks for them (4 words per row).
enum : int {
  kStatPath = 0,        // bit0 sampled, bit1 top-k applied, bit2 top-p applied, bit3 greedy
  kStatTopPExact = 1,   // 1 if the nucleus cut needed the exact sequential pass
  kStatDrawExact = 2,   // 1 if the draw needed the exact sequential pass
  kStatKept = 3,        // number of ids surviving the chain (before the draw)
};

struct RowsArgs {
  const void* logits;
  int64_t ld;
  int dtype;  // 0 f32, 1 bf16
  int n_rows;
  int vocab;
  const int32_t* hist_ids;
  const int64_t* hist_off;
  const float* temp;
  const int32_t* top_k;
  const float* top_p;
  const float* pen;
  const int32_t* min_keep;
  const uint8_t* do_sample;
  const uint8_t* row_active;
  uint64_t* rng;
  int32_t* out_tok;
  float* out_masked;
  uint32_t* stats;
  uint32_t mode;        // kCustom | processor bits, or 0 for the reference chain
  uint32_t* sort_ws;    // large-vocab exact pass: per-row key buffer
  int64_t sort_ws_stride;
  uint32_t* hist_bits;  // per-row history set kept across steps, or null
  int stop_token;       // with hist_bits: the token that does not join it
};

struct StreamArgs {
  const float* logits;   // [n_steps][n_rows] rows of ld floats
  int64_t ld;
  int64_t step_stride;   // elements between steps
  int n_steps;
  int n_rows;
  int vocab;
  const int32_t* hist_ids;
  const int64_t* hist_off;
  const float* temp;
  const int32_t* top_k;
  const float* top_p;
  const float* pen;
  const uint8_t* do_sample;
  int stop_token;
  uint64_t* rng;
  int32_t* out_tok;      // [n_steps][n_rows]
  uint32_t* stats;       // optional [n_rows][4], accumulated over steps
  // The speculative chains' bounded waits: polls before a wait gives up, and
  // the word (host-visible) a chain that gave up sets to a nonzero value.
  int spin_max;
  uint32_t* status;
};
// Values of StreamArgs::status (bits).
constexpr uint32_t kStatusWaitExpired = 1u;   // a checking wave's bounded wait gave up
constexpr uint32_t kStatusDrawnOverflow = 2u; // more drawn ids than the speculative chain keeps
constexpr int kSpinMaxDefault = 1 << 22;      // about 0.3 s of polls

// Two-phase stream (scan, then chain). The scan writes one summary per
// (step, row); its layout is fixed here so that host code can size the
// workspace.
constexpr int kListSmall = 128;     // greedy and top-k rows
constexpr int kListLarge = 512;     // full-vocabulary nucleus rows
constexpr int kCandCap = 1024;      // candidates the scan may sort
constexpr int kChunkIds = 64;       // ids per mass chunk
constexpr int kMaxChunks = kLdsVocabMax / kChunkIds + 1;
constexpr int kSumHdrBytes = 64;
// 1024 words: every thread of a 256-thread workgroup loads four words of a
// summary unconditionally (no select on in-flight loads), all inside the stride.
constexpr size_t kSumStride = 8192;
static_assert((size_t)kSumHdrBytes + 12 * (size_t)kListLarge + 8 * (size_t)kMaxChunks <= kSumStride,
              "summary layout fits the stride");
constexpr int kStateWords = 8 + 400;  // done, stats[4], pad, new-id bitmap

struct StreamWs {
  unsigned char* sum;      // [steps in chunk][n_rows] summaries of kSumStride bytes
  uint32_t* state;         // [n_rows][kStateWords] carried across kernels and chunks
  int s_begin, s_end;      // steps of this chunk
  int steps_per_group;     // scan: steps per workgroup
  uint32_t* sortbuf;       // exact steps of the pipelined row chain: per-row key buffer
  int64_t sort_stride;     // words per row
  int nseg;                // pipelined row chain: step segments of a row without penalty
  uint64_t* segres;        // [n_rows][nseg][4] segment results (status and stop step, RNG, statistics)
};

// LM head weight kinds (values of c4s_head.wdtype).
enum : int { kLmW_BF16 = 0, kLmW_F32 = 1, kLmW_Q8 = 2 };

struct LmHeadArgs {
  const uint16_t* hidden;  // [M][D] bf16
  const float* gamma;
  const float* beta;
  float eps;
  const void* weight;      // [V][D] bf16, f32 or 8-bit codes (wkind)
  const float* wscale;     // 8-bit: [V][D / group] scales
  const float* wbias;      // 8-bit: [V][D / group] offsets
  int wkind, group;
  const float* bias;       // [V]
  float* logits;           // [M][V] f32 (row stride ld_out)
  int64_t ld_out;
  int M, D, V;
};

// Static device scratch of the no-allocation entry point (per device).
constexpr size_t kNoAllocBytes = (size_t)8 << 20;
// This device's address of that scratch (the current device).
hipError_t noalloc_scratch(void** ptr);

size_t rows_lds_bytes(int vocab);
size_t rows_global_lds_bytes(int vocab);
size_t stream_lds_bytes(int vocab, int unused);

hipError_t launch_rows(const RowsArgs& a, hipStream_t s);
hipError_t launch_hist_bits_init(const int32_t* ids, const int64_t* off, int n_rows, int V, uint32_t* bits,
                                 hipStream_t s);
hipError_t launch_stream(const StreamArgs& a, hipStream_t s);
hipError_t launch_stream_scan(const StreamArgs& a, const StreamWs& w, hipStream_t s);
size_t stream_list_lds_bytes(int vocab);  // candidate-list chain: a row for its exact steps
hipError_t launch_stream_list(const StreamArgs& a, const StreamWs& w, hipStream_t s);
hipError_t launch_stream_rowp(const StreamArgs& a, const StreamWs& w, hipStream_t s);
hipError_t launch_stream_segfix(const StreamArgs& a, const StreamWs& w, hipStream_t s);
hipError_t launch_stream_spec(const StreamArgs& a, const StreamWs& w, hipStream_t s);
hipError_t launch_stream_lspec(const StreamArgs& a, const StreamWs& w, hipStream_t s);
hipError_t launch_stream_chain(const StreamArgs& a, const StreamWs& w, hipStream_t s);
size_t stream_chain_lds_bytes(int vocab);
size_t stream_rowp_lds_bytes(int vocab);  // 0 when the pipelined row chain does not fit
size_t stream_spec_lds_bytes(int vocab);  // dynamic LDS of the speculative row chain (0: no layout for vocab)
size_t stream_lspec_lds_bytes(int vocab); // dynamic LDS of the speculative list chain (0: no layout for vocab)
int stream_spec_max_steps();             // steps a call may have for it
hipError_t launch_lmhead(const LmHeadArgs& a, hipStream_t s);
hipError_t launch_hbm_probe(const void* src, void* dst, int64_t bytes, int mode, hipStream_t s);

}  // namespace c4s
