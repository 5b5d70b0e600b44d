// C ABI of libc4s_sampling.so (declarations and contracts in include/c4s_sampling.h).
//
// Host side only: argument validation, per-context workspace, dispatch to the
// gfx950 kernels. There is no CPU fallback: a missing device or a failed launch
// is reported as an error.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/c4s_sampling.h"
#include "c4s_internal.h"

struct c4s_ctx {
  int device = 0;
  std::string err;
  hipStream_t host_stream = nullptr;  // used by the synchronous host helpers
  void* ws = nullptr;                 // large-vocab exact-pass key buffers
  size_t ws_bytes = 0;
  void* logits_ws = nullptr;          // LM head + sample: logits when the caller gives none
  size_t logits_bytes = 0;
  // host-helper staging: pinned host memory that the device maps
  void* hstage = nullptr;
  size_t hstage_bytes = 0;
  // two-phase stream: summaries of one chunk of steps, per-row carried state
  void* sum_ws = nullptr;
  size_t sum_bytes = 0;
  void* state_ws = nullptr;
  size_t state_bytes = 0;
  // second stream: the two fast chain kernels run side by side
  hipStream_t side = nullptr;
  // third stream: the scan of the next chunk of steps beside the chain of this one
  hipStream_t scan_s = nullptr;
  hipEvent_t ev_start = nullptr;
  // by summary buffer: its scan done, its list chain done, its full-vocabulary chain done
  hipEvent_t ev_scan[3] = {nullptr, nullptr, nullptr}, ev_chain[3] = {nullptr, nullptr, nullptr};
  hipEvent_t ev_side[3] = {nullptr, nullptr, nullptr};
  // Overlapped stream: the scan and the chains on disjoint sets of CUs (half
  // of every 32 CUs for the chains), created at first use.
  int n_cus = 0;
  bool cu_split_tried = false;
  hipStream_t scan_m = nullptr, chain_m = nullptr, side_m = nullptr;
  hipEvent_t ev_done = nullptr;
  // step segments of the pipelined row chain (rows without penalty)
  void* segres = nullptr;
  size_t segres_bytes = 0;
  // Set once a call on a capturing stream used a workspace: from then on a
  // workspace that grows is retired (freed at c4s_destroy) instead of freed,
  // because a captured graph may still write the old buffer when replayed.
  bool graph_used = false;
  std::vector<void*> retired;
  // this device's address of the no-allocation entry point's static scratch
  // (null when the runtime could not give it)
  void* noalloc = nullptr;
  // The speculative chains' give-up report: a word of pinned host memory that
  // the kernels write through its device address, and the polls a bounded
  // wait makes before it gives up.
  volatile uint32_t* status_host = nullptr;
  uint32_t* status_dev = nullptr;
  int spin_max = c4s::kSpinMaxDefault;
};

namespace {

constexpr int kStreamVocabMax = c4s::kLdsVocabMax;
constexpr size_t kLdsLimit = 160 * 1024;
constexpr size_t kChainStaticLds = 38 * 1024;      // chain kernels' static LDS (upper bound)
constexpr size_t kRowPStaticLds = 40 * 1024;       // pipelined row chain's static LDS (upper bound)
constexpr size_t kSpecStaticLds = 12 * 1024;       // speculative row chain's static LDS (upper bound)
constexpr size_t kSumBudget = (size_t)512 << 20;   // stream summaries per chunk of steps
constexpr int kScanStepsPerGroup = 8;
// Chunks of the overlapped stream: the first is short (its scan is not
// hidden), each next one 6/5 times longer (its scan, on its share of the CUs, must end
// before the chain of the previous one: the scan takes about 2.9 us a step
// there, the row chain 3.55), up to kOverlapChunk steps.
constexpr int kOverlapFirst = 64;
constexpr int kOverlapChunk = 256;
// Summary buffers of the overlapped stream: the scans depend on nothing but
// the inputs, so with three buffers a scan waits only for the chains of the
// chunk three back and runs ahead of the chains instead of in step with them.
constexpr int kOverlapBufs = 3;
constexpr int kOverlapStepsPerGroup = 1;   // one step a scan workgroup: the shortest chunk ends on time
// Of every 32 CUs, the chains' shares in the overlapped stream: the
// full-vocabulary chain (a workgroup holds a whole CU's LDS) and the list
// chain (two workgroups a CU); the scans take the rest.
constexpr int kRowCusPer32 = 4;
constexpr int kListCusPer32 = 4;
constexpr int kMaxSegments = 8;   // step segments per row without penalty

int fail(c4s_ctx* ctx, int code, const std::string& msg) {
  if (ctx) ctx->err = msg;
  return code;
}

int hip_fail(c4s_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, C4S_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

struct DeviceGuard {
  int prev = -1;
  hipError_t err = hipSuccess;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) err = hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

bool is_capturing(hipStream_t s) {
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone;
}

// Workspace of at least `need` bytes for a call queued on `s`. A workspace
// never grows while `s` is being captured into a graph (allocation is not
// allowed there): a first call of the same shape outside the capture sizes it.
int ensure(c4s_ctx* ctx, void** buf, size_t* have, size_t need, const char* what, hipStream_t s) {
  const bool cap = is_capturing(s);
  if (need <= *have) {
    if (cap) ctx->graph_used = true;
    return C4S_OK;
  }
  if (cap)
    return fail(ctx, C4S_EINVAL, std::string(what) +
                                     ": the workspace would grow during graph capture; make one call of "
                                     "this shape (or larger) outside the capture first");
  if (*buf) {
    if (ctx->graph_used) {   // a graph may still use it: keep it until c4s_destroy
      ctx->retired.push_back(*buf);
      *buf = nullptr;
      *have = 0;
    } else {
      hipError_t e = hipFree(*buf);
      *buf = nullptr;
      *have = 0;
      if (e != hipSuccess) return hip_fail(ctx, e, what);
    }
  }
  hipError_t e = hipMalloc(buf, need);
  if (e != hipSuccess) {
    *buf = nullptr;
    return e == hipErrorOutOfMemory ? fail(ctx, C4S_ENOMEM, std::string(what) + ": out of memory")
                                    : hip_fail(ctx, e, what);
  }
  *have = need;
  return C4S_OK;
}

size_t pow2_at_least(size_t n) {
  size_t p = 1;
  while (p < n) p <<= 1;
  return p;
}

// logits_given: false when the logits are a buffer the call provides later
// (the LM head entry points without a caller's logits buffer).
int validate_rows(c4s_ctx* ctx, const c4s_rows* r, bool logits_given = true) {
  if (!r) return fail(ctx, C4S_EINVAL, "rows descriptor is NULL");
  if (r->n_rows < 0) return fail(ctx, C4S_EINVAL, "n_rows < 0");
  if (r->n_rows == 0) return C4S_OK;
  if (r->vocab < 1 || r->vocab > c4s::kMaxVocab) return fail(ctx, C4S_EINVAL, "vocab out of range");
  if (r->ld < r->vocab) return fail(ctx, C4S_EINVAL, "ld < vocab");
  if (r->dtype != C4S_DTYPE_F32 && r->dtype != C4S_DTYPE_BF16)
    return fail(ctx, C4S_EINVAL, "unknown dtype");
  if ((logits_given && !r->logits) || !r->out_token) return fail(ctx, C4S_EINVAL, "logits/out_token is NULL");
  const uint32_t m = r->mode;
  const bool custom = (m & C4S_MODE_CUSTOM) != 0;
  const uint32_t known = C4S_P_PENALTY | C4S_P_TEMPERATURE | C4S_P_TOP_K | C4S_P_TOP_P |
                         C4S_T_ARGMAX | C4S_T_DRAW | C4S_MODE_CUSTOM;
  if (m & ~known) return fail(ctx, C4S_EINVAL, "unknown mode bits");
  if (!custom && m != C4S_MODE_CHAIN) return fail(ctx, C4S_EINVAL, "processor bits need C4S_MODE_CUSTOM");
  if (custom && (m & C4S_T_ARGMAX) && (m & C4S_T_DRAW))
    return fail(ctx, C4S_EINVAL, "argmax and draw are exclusive");
  const bool pen = !custom || (m & C4S_P_PENALTY);
  if (pen && (!r->rep_penalty || (!r->hist_offsets && !r->hist_bits)))
    return fail(ctx, C4S_EINVAL, "penalty needs rep_penalty and hist_offsets or hist_bits");
  if (pen && !r->hist_ids) {
    // allowed only when every history is empty; the kernel never reads ids then
  }
  if ((!custom || (m & C4S_P_TEMPERATURE)) && !r->temperature)
    return fail(ctx, C4S_EINVAL, "temperature is NULL");
  if ((!custom || (m & C4S_P_TOP_K)) && !r->top_k) return fail(ctx, C4S_EINVAL, "top_k is NULL");
  if ((!custom || (m & C4S_P_TOP_P)) && !r->top_p) return fail(ctx, C4S_EINVAL, "top_p is NULL");
  const bool draws = !custom || (m & C4S_T_DRAW);
  if (draws && !r->rng_state) return fail(ctx, C4S_EINVAL, "rng_state is NULL");
  return C4S_OK;
}

c4s::RowsArgs to_args(const c4s_rows* r) {
  c4s::RowsArgs a{};
  a.logits = r->logits;
  a.ld = r->ld;
  a.dtype = r->dtype;
  a.n_rows = r->n_rows;
  a.vocab = r->vocab;
  a.hist_ids = r->hist_ids;
  a.hist_off = r->hist_offsets;
  a.temp = r->temperature;
  a.top_k = r->top_k;
  a.top_p = r->top_p;
  a.pen = r->rep_penalty;
  a.min_keep = r->min_keep;
  a.do_sample = r->do_sample;
  a.row_active = r->row_active;
  a.rng = r->rng_state;
  a.out_tok = r->out_token;
  a.out_masked = r->out_masked;
  a.stats = r->out_stats;
  a.mode = r->mode;
  a.hist_bits = r->hist_bits;
  a.stop_token = r->stop_token;
  return a;
}

// The sort workspace of vocabularies the step cannot stage in LDS.
int rows_workspace(c4s_ctx* ctx, const c4s_rows* r, hipStream_t s) {
  if (r->vocab <= c4s::kLdsVocabMax) return C4S_OK;
  const size_t per_row = pow2_at_least((size_t)r->vocab) * sizeof(uint32_t);
  return ensure(ctx, &ctx->ws, &ctx->ws_bytes, per_row * (size_t)r->n_rows, "sort workspace", s);
}

int launch_rows_checked(c4s_ctx* ctx, const c4s_rows* r, hipStream_t s) {
  c4s::RowsArgs a = to_args(r);
  if (r->vocab > c4s::kLdsVocabMax) {
    const size_t per_row = pow2_at_least((size_t)r->vocab) * sizeof(uint32_t);
    int rc = rows_workspace(ctx, r, s);
    if (rc) return rc;
    a.sort_ws = static_cast<uint32_t*>(ctx->ws);
    a.sort_ws_stride = (int64_t)(per_row / sizeof(uint32_t));
  }
  hipError_t e = c4s::launch_rows(a, s);
  if (e != hipSuccess) return hip_fail(ctx, e, "sample_rows launch");
  return C4S_OK;
}

}  // namespace

extern "C" {

const char* c4s_version(void) { return "c4s-sampling 0.1 gfx950"; }

int c4s_create(int device, c4s_ctx** out) {
  if (!out) return C4S_EINVAL;
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return C4S_EHIP;
  if (device < 0 || device >= n) return C4S_EINVAL;
  c4s_ctx* ctx = new c4s_ctx();
  ctx->device = device;
  DeviceGuard g(device);
  if (g.err != hipSuccess) { delete ctx; return C4S_EHIP; }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) { delete ctx; return C4S_EHIP; }
  ctx->n_cus = prop.multiProcessorCount;
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    // The code objects are built for gfx950 only.
    delete ctx;
    return C4S_EINVAL;
  }
  // The stream's status word (C4S_ETIMEOUT reports), host memory the device writes.
  void* sh = nullptr;
  if (hipHostMalloc(&sh, 64, hipHostMallocMapped) != hipSuccess) { delete ctx; return C4S_ENOMEM; }
  ctx->status_host = static_cast<volatile uint32_t*>(sh);
  *ctx->status_host = 0u;
  void* sd = nullptr;
  if (hipHostGetDevicePointer(&sd, sh, 0) != hipSuccess) {
    (void)hipHostFree(sh);
    delete ctx;
    return C4S_EHIP;
  }
  ctx->status_dev = static_cast<uint32_t*>(sd);
  // The static scratch of c4s_lmhead_sample_noalloc: its address on this
  // device, asked for once, with the device current.
  if (c4s::noalloc_scratch(&ctx->noalloc) != hipSuccess) {
    ctx->noalloc = nullptr;
    (void)hipGetLastError();
  }
  if (hipStreamCreateWithFlags(&ctx->host_stream, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->side, hipStreamNonBlocking) != hipSuccess ||
      hipStreamCreateWithFlags(&ctx->scan_s, hipStreamNonBlocking) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_start, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_scan[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_scan[1], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_scan[2], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_chain[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_chain[1], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_chain[2], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_side[0], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_side[1], hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_side[2], hipEventDisableTiming) != hipSuccess) {
    c4s_destroy(ctx);
    return C4S_EHIP;
  }
  *out = ctx;
  return C4S_OK;
}

int c4s_destroy(c4s_ctx* ctx) {
  if (!ctx) return C4S_OK;
  DeviceGuard g(ctx->device);
  if (ctx->host_stream) (void)hipStreamSynchronize(ctx->host_stream);
  if (ctx->side) (void)hipStreamSynchronize(ctx->side);
  if (ctx->scan_s) (void)hipStreamSynchronize(ctx->scan_s);
  for (hipStream_t st : {ctx->scan_m, ctx->chain_m, ctx->side_m})
    if (st) (void)hipStreamSynchronize(st);
  for (void* p : {ctx->ws, ctx->logits_ws, ctx->sum_ws, ctx->state_ws, ctx->segres})
    if (p) (void)hipFree(p);
  for (void* p : ctx->retired) (void)hipFree(p);
  if (ctx->host_stream) (void)hipStreamDestroy(ctx->host_stream);
  if (ctx->side) (void)hipStreamDestroy(ctx->side);
  if (ctx->scan_s) (void)hipStreamDestroy(ctx->scan_s);
  for (hipStream_t st : {ctx->scan_m, ctx->chain_m, ctx->side_m})
    if (st) (void)hipStreamDestroy(st);
  for (hipEvent_t ev : {ctx->ev_start, ctx->ev_scan[0], ctx->ev_scan[1], ctx->ev_scan[2],
                        ctx->ev_chain[0], ctx->ev_chain[1], ctx->ev_chain[2], ctx->ev_done, ctx->ev_side[0],
                        ctx->ev_side[1], ctx->ev_side[2]})
    if (ev) (void)hipEventDestroy(ev);
  if (ctx->status_host) (void)hipHostFree(const_cast<uint32_t*>(ctx->status_host));
  if (ctx->hstage) (void)hipHostFree(ctx->hstage);
  delete ctx;
  return C4S_OK;
}

namespace {
// The status word of the stream calls that have ended, cleared: C4S_OK, or
// C4S_ETIMEOUT with the reason in the context's error text.
int take_status(c4s_ctx* ctx) {
  const uint32_t s = *ctx->status_host;
  if (!s) return C4S_OK;
  *ctx->status_host = 0u;
  return fail(ctx, C4S_ETIMEOUT,
              (s & c4s::kStatusWaitExpired)
                  ? "sample_stream: a speculative chain's bounded wait gave up; that call's tokens are -1 from the "
                    "step where it stopped and its RNG states stop there"
                  : "sample_stream: a speculative chain kept more drawn ids than it holds; that call's tokens are -1 "
                    "from the step where it stopped");
}
}  // namespace

int c4s_stream_status(c4s_ctx* ctx, void* stream) {
  if (!ctx) return C4S_EINVAL;
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(ctx, e, "stream_status synchronize");
  return take_status(ctx);
}

int c4s_set_wait_limit(c4s_ctx* ctx, int32_t polls) {
  if (!ctx) return C4S_EINVAL;
  ctx->spin_max = polls > 0 ? polls : c4s::kSpinMaxDefault;
  return C4S_OK;
}

const char* c4s_last_error(const c4s_ctx* ctx) { return ctx ? ctx->err.c_str() : "no context"; }

int c4s_sample_rows(c4s_ctx* ctx, const c4s_rows* rows, void* stream) {
  if (!ctx) return C4S_EINVAL;
  int rc = validate_rows(ctx, rows);
  if (rc || rows->n_rows == 0) return rc;
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  return launch_rows_checked(ctx, rows, static_cast<hipStream_t>(stream));
}

// Streams of the overlapped stream, created once, on disjoint CU sets: the
// full-vocabulary chain (side_m), the list chain (chain_m) and the scans
// (scan_m). Mask bit c is CU c, and CU c sits on XCD c % 8. Within an XCD the
// CUs go to the sets in bit-reversed order of their index (mod 32), so that
// each set spreads evenly over the XCD's blocks of CUs. False when the device
// or the runtime cannot split.
static int cu_set(int cu) {   // 0: full-vocabulary chain, 1: list chain, 2: scan
  const uint32_t k = (uint32_t)(cu / 8) & 31u;
  const int rev = (int)(((k & 1u) << 4) | ((k & 2u) << 2) | (k & 4u) | ((k & 8u) >> 2) | ((k & 16u) >> 4));
  return rev < kRowCusPer32 ? 0 : (rev < kRowCusPer32 + kListCusPer32 ? 1 : 2);
}
static int cus_in_set(const c4s_ctx* ctx, int set) {
  int c = 0;
  for (int cu = 0; cu < ctx->n_cus; ++cu) c += cu_set(cu) == set ? 1 : 0;
  return c;
}
static int row_cus(const c4s_ctx* ctx) { return cus_in_set(ctx, 0); }
static int list_cus(const c4s_ctx* ctx) { return cus_in_set(ctx, 1); }
static bool cu_split(c4s_ctx* ctx) {
  if (ctx->chain_m) return true;
  if (ctx->cu_split_tried) return false;
  ctx->cu_split_tried = true;
  const int n = ctx->n_cus;
  if (n < 64 || n % 32 != 0) return false;
  const size_t nw = (size_t)n / 32;
  std::vector<uint32_t> row_mask(nw, 0u), list_mask(nw, 0u), scan_mask(nw, 0u);
  for (int cu = 0; cu < n; ++cu) {
    const int set = cu_set(cu);
    std::vector<uint32_t>& m = set == 0 ? row_mask : (set == 1 ? list_mask : scan_mask);
    m[(size_t)cu / 32] |= 1u << (cu % 32);
  }
  if (hipExtStreamCreateWithCUMask(&ctx->scan_m, (uint32_t)nw, scan_mask.data()) != hipSuccess ||
      hipExtStreamCreateWithCUMask(&ctx->chain_m, (uint32_t)nw, list_mask.data()) != hipSuccess ||
      hipExtStreamCreateWithCUMask(&ctx->side_m, (uint32_t)nw, row_mask.data()) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->ev_done, hipEventDisableTiming) != hipSuccess) {
    for (hipStream_t* st : {&ctx->scan_m, &ctx->chain_m, &ctx->side_m})
      if (*st) { (void)hipStreamDestroy(*st); *st = nullptr; }
    (void)hipGetLastError();
    return false;
  }
  return true;
}

int c4s_hist_bits_init(c4s_ctx* ctx, const int32_t* hist_ids, const int64_t* hist_offsets, int32_t n_rows,
                       int32_t vocab, uint32_t* hist_bits, void* stream) {
  if (!ctx) return C4S_EINVAL;
  if (n_rows < 0) return fail(ctx, C4S_EINVAL, "n_rows < 0");
  if (n_rows == 0) return C4S_OK;
  if (vocab < 1 || vocab > c4s::kMaxVocab) return fail(ctx, C4S_EINVAL, "vocab out of range");
  if (!hist_bits || !hist_offsets) return fail(ctx, C4S_EINVAL, "hist_bits/hist_offsets is NULL");
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  const hipError_t e = c4s::launch_hist_bits_init(hist_ids, hist_offsets, n_rows, vocab, hist_bits,
                                                  static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(ctx, e, "hist_bits_init launch");
  return C4S_OK;
}

int c4s_sample_stream(c4s_ctx* ctx, const c4s_stream* st, void* stream) {
  if (!ctx) return C4S_EINVAL;
  if (!st) return fail(ctx, C4S_EINVAL, "stream descriptor is NULL");
  if (st->n_rows < 0 || st->n_steps < 0) return fail(ctx, C4S_EINVAL, "negative size");
  if (st->n_rows == 0 || st->n_steps == 0) return C4S_OK;
  if (st->vocab < 1 || st->vocab > kStreamVocabMax)
    return fail(ctx, C4S_EINVAL, "stream needs 1 <= vocab <= 12288");
  if (st->ld < st->vocab) return fail(ctx, C4S_EINVAL, "ld < vocab");
  if (!st->logits || !st->hist_offsets || !st->temperature || !st->top_k || !st->top_p ||
      !st->rep_penalty || !st->rng_state || !st->out_tokens)
    return fail(ctx, C4S_EINVAL, "stream: required pointer is NULL");
  c4s::StreamArgs a{};
  a.logits = st->logits;
  a.ld = st->ld;
  a.step_stride = st->step_stride;
  a.n_steps = st->n_steps;
  a.n_rows = st->n_rows;
  a.vocab = st->vocab;
  a.hist_ids = st->hist_ids;
  a.hist_off = st->hist_offsets;
  a.temp = st->temperature;
  a.top_k = st->top_k;
  a.top_p = st->top_p;
  a.pen = st->rep_penalty;
  a.do_sample = st->do_sample;
  a.stop_token = st->stop_token;
  a.rng = st->rng_state;
  a.out_tok = st->out_tokens;
  a.stats = st->out_stats;
  a.spin_max = ctx->spin_max;
  a.status = ctx->status_dev;
  if (st->flags & ~(uint32_t)(C4S_STREAM_SEQUENTIAL | C4S_STREAM_NO_SPECULATION))
    return fail(ctx, C4S_EINVAL, "stream: unknown flags");
  if (c4s::stream_lds_bytes(a.vocab, 0) + 4096 > kLdsLimit)
    return fail(ctx, C4S_EINVAL, "stream: row state exceeds LDS");
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  const hipStream_t hs = static_cast<hipStream_t>(stream);
  // The stream call waits on the host for the previous call and may grow its
  // workspaces, so it is not capturable: a graph would also keep pointers to
  // summary buffers that the next eager call reuses.
  if (is_capturing(hs)) return fail(ctx, C4S_EINVAL, "sample_stream: not allowed while the stream is captured");
  // A call of this context that has ended gave up: report it before queuing.
  if (const int rs = take_status(ctx)) return rs;
  // The two-phase stream needs the pipelined full-vocabulary chain (three
  // rows and summaries in LDS, V <= 8232); larger vocabularies, and callers
  // that ask for it, take the single-kernel stream.
  const bool two_phase = !(st->flags & C4S_STREAM_SEQUENTIAL) &&
                         c4s::stream_chain_lds_bytes(a.vocab) + kChainStaticLds <= kLdsLimit &&
                         c4s::stream_rowp_lds_bytes(a.vocab) + kRowPStaticLds <= kLdsLimit;
  if (!two_phase) {
    hipError_t e = c4s::launch_stream(a, hs);
    if (e != hipSuccess) return hip_fail(ctx, e, "sample_stream launch");
    return C4S_OK;
  }
  // Steps go in chunks; the chain carries its per-row state from chunk to
  // chunk. Overlapped (rows at most the chains' CUs, steps for four
  // chunks or more): the scans of later chunks run on their own CUs beside the
  // chains, summaries rotate through kOverlapBufs buffers and a scan waits for
  // the chains that last read its buffer; the first chunk's scan, which nothing
  // hides, runs on every CU. Otherwise the whole stream is one chunk where the
  // budget allows (else two buffers), each phase on every CU.
  const size_t per_step = (size_t)a.n_rows * c4s::kSumStride;
  const bool overlap = a.n_rows <= row_cus(ctx) + list_cus(ctx) && a.n_steps >= 4 * kOverlapFirst &&
                       (size_t)kOverlapChunk * kOverlapBufs * per_step <= kSumBudget && cu_split(ctx);
  size_t chunk_sz = std::min<size_t>((size_t)a.n_steps, kSumBudget / per_step);
  if (overlap) chunk_sz = std::min<size_t>((size_t)a.n_steps, kOverlapChunk);
  else if (chunk_sz < (size_t)a.n_steps) chunk_sz = std::min(chunk_sz, kSumBudget / 2 / per_step);   // two buffers
  const int chunk = (int)std::max<size_t>(1, chunk_sz);   // the longest chunk
  const size_t chunk_bytes = per_step * (size_t)chunk;
  const int n_bufs = chunk >= a.n_steps ? 1 : overlap ? kOverlapBufs : 2;
  int rc = ensure(ctx, &ctx->sum_ws, &ctx->sum_bytes, (size_t)n_bufs * chunk_bytes, "stream summaries", hs);
  if (rc) return rc;
  rc = ensure(ctx, &ctx->state_ws, &ctx->state_bytes, (size_t)a.n_rows * c4s::kStateWords * 4, "stream state", hs);
  if (rc) return rc;
  // The chains' exact steps sort in a per-row global key buffer.
  const size_t sort_row = pow2_at_least((size_t)a.vocab) * sizeof(uint32_t);
  rc = ensure(ctx, &ctx->ws, &ctx->ws_bytes, sort_row * (size_t)a.n_rows, "sort workspace", hs);
  if (rc) return rc;
  // Rows without penalty split their steps into segments, one workgroup each,
  // over the CUs the chains have (every workgroup of the pipelined chain
  // holds a CU's LDS).
  const int nseg = std::max(2, std::min(kMaxSegments, (overlap ? row_cus(ctx) : ctx->n_cus) / std::max(1, a.n_rows)));
  rc = ensure(ctx, &ctx->segres, &ctx->segres_bytes, (size_t)a.n_rows * nseg * 4 * sizeof(uint64_t),
              "segment results", hs);
  if (rc) return rc;
  // Full-vocabulary rows: the speculative chain (several steps decided at
  // once, each checked in order) when a call's drawn ids fit its lists, else
  // the pipelined chain with step segments for rows without penalty.
  // (a layout size of 0: the vocabulary has no layout, nothing fits)
  const size_t spec_lds = c4s::stream_spec_lds_bytes(a.vocab), lspec_lds = c4s::stream_lspec_lds_bytes(a.vocab);
  const bool spec = !(st->flags & C4S_STREAM_NO_SPECULATION) && a.n_steps <= c4s::stream_spec_max_steps() &&
                    spec_lds > 0 && spec_lds + kSpecStaticLds <= kLdsLimit;
  // Greedy and top-k rows likewise: the speculative list chain, else one wave a row.
  const bool spec_list = !(st->flags & C4S_STREAM_NO_SPECULATION) && a.n_steps <= c4s::stream_spec_max_steps() &&
                         lspec_lds > 0 && lspec_lds + kSpecStaticLds <= kLdsLimit;
  auto launch_row_chain = [&](const c4s::StreamWs& w, hipStream_t on) {
    if (spec) return c4s::launch_stream_spec(a, w, on);
    hipError_t e = c4s::launch_stream_rowp(a, w, on);
    return e == hipSuccess ? c4s::launch_stream_segfix(a, w, on) : e;
  };
  const hipStream_t chain_on = overlap ? ctx->chain_m : hs;
  const hipStream_t side_on = overlap ? ctx->side_m : ctx->side;
  // One overlapped call in flight per context: the host waits for the
  // previous one to end before it queues this one. A call's packets queued
  // behind the running one (its first scan's wait at the head of a queue)
  // slowed the running call's kernels by about 7% (dispatches of the short
  // kernels 5 -> 32 us); queuing takes about 1.5 ms of the 4 ms call, so the
  // first scan still starts within tens of microseconds.
  if (overlap) {
    const hipError_t ew = hipEventSynchronize(ctx->ev_done);
    if (ew != hipSuccess) return hip_fail(ctx, ew, "sample_stream previous call");
    if (const int rs = take_status(ctx)) return rs;   // the previous call has ended now
  }
  hipError_t e0 = hipEventRecord(ctx->ev_start, hs);   // inputs and the previous call's chain
  if (e0 == hipSuccess) e0 = hipStreamWaitEvent(ctx->scan_s, ctx->ev_start, 0);
  if (e0 == hipSuccess && overlap) e0 = hipStreamWaitEvent(chain_on, ctx->ev_start, 0);
  if (e0 != hipSuccess) return hip_fail(ctx, e0, "sample_stream scan stream");
  int last_side = -1;   // buffer of the last chunk whose full-vocabulary chain ran on the side stream
  for (int s0 = 0, ci = 0, len = overlap ? kOverlapFirst : chunk; s0 < a.n_steps;
       s0 += len, ++ci, len = std::min(chunk, overlap ? len + len / 5 : chunk)) {
    const int buf = ci % n_bufs;
    const hipStream_t scan_on = (overlap && ci > 0) ? ctx->scan_m : ctx->scan_s;
    c4s::StreamWs w{};
    w.sum = static_cast<unsigned char*>(ctx->sum_ws) + (size_t)buf * chunk_bytes;
    w.state = static_cast<uint32_t*>(ctx->state_ws);
    w.s_begin = s0;
    w.s_end = std::min(a.n_steps, s0 + len);
    w.steps_per_group = overlap ? kOverlapStepsPerGroup : kScanStepsPerGroup;
    w.sortbuf = static_cast<uint32_t*>(ctx->ws);
    w.sort_stride = (int64_t)(sort_row / sizeof(uint32_t));
    w.nseg = nseg;
    w.segres = static_cast<uint64_t*>(ctx->segres);
    hipError_t e = hipSuccess;
    if (overlap && ci == 1 && (e = hipStreamWaitEvent(scan_on, ctx->ev_scan[0], 0)) != hipSuccess)
      return hip_fail(ctx, e, "sample_stream scan order");
    if (ci >= n_bufs && ((e = hipStreamWaitEvent(scan_on, ctx->ev_chain[buf], 0)) != hipSuccess ||
                    (e = hipStreamWaitEvent(scan_on, ctx->ev_side[buf], 0)) != hipSuccess))
      return hip_fail(ctx, e, "sample_stream buffer reuse");
    e = c4s::launch_stream_scan(a, w, scan_on);
    if (e != hipSuccess) return hip_fail(ctx, e, "sample_stream scan launch");
    if ((e = hipEventRecord(ctx->ev_scan[buf], scan_on)) != hipSuccess ||
        (e = hipStreamWaitEvent(chain_on, ctx->ev_scan[buf], 0)) != hipSuccess)
      return hip_fail(ctx, e, "sample_stream scan order");
    // Both fast chains run their exact steps themselves: the full-vocabulary
    // chain on the side stream, the list chain and then the finisher
    // (exact-mode rows only) here, each after the scan.
    if ((e = hipStreamWaitEvent(side_on, ctx->ev_scan[buf], 0)) != hipSuccess ||
        (e = launch_row_chain(w, side_on)) != hipSuccess ||
        (e = hipEventRecord(ctx->ev_side[buf], side_on)) != hipSuccess)
      return hip_fail(ctx, e, "sample_stream row-chain launch");
    if ((e = (spec_list ? c4s::launch_stream_lspec(a, w, chain_on) : c4s::launch_stream_list(a, w, chain_on))) !=
            hipSuccess ||
        (e = c4s::launch_stream_chain(a, w, chain_on)) != hipSuccess ||
        (e = hipEventRecord(ctx->ev_chain[buf], chain_on)) != hipSuccess)
      return hip_fail(ctx, e, "sample_stream chain launch");
    last_side = buf;
  }
  if (last_side >= 0) {   // the last full-vocabulary chain ahead of what follows on chain_on
    hipError_t e = hipStreamWaitEvent(chain_on, ctx->ev_side[last_side], 0);
    if (e != hipSuccess) return hip_fail(ctx, e, "sample_stream join");
  }
  if (overlap) {   // the caller's stream continues after the last chain
    hipError_t e = hipEventRecord(ctx->ev_done, chain_on);
    if (e == hipSuccess) e = hipStreamWaitEvent(hs, ctx->ev_done, 0);
    if (e != hipSuccess) return hip_fail(ctx, e, "sample_stream join caller");
  }
  return C4S_OK;
}

static int lmhead_check(c4s_ctx* ctx, const c4s_head* h) {
  if (!h->hidden || !h->gamma || !h->beta || !h->weight || !h->bias)
    return fail(ctx, C4S_EINVAL, "lmhead: required pointer is NULL");
  if (h->M < 1 || h->D < 32 || h->V < 1 || (h->D % 32) != 0)
    return fail(ctx, C4S_EINVAL, "lmhead: needs M >= 1, V >= 1, D a positive multiple of 32");
  if (h->wdtype != C4S_W_BF16 && h->wdtype != C4S_W_F32 && h->wdtype != C4S_W_Q8)
    return fail(ctx, C4S_EINVAL, "lmhead: unknown weight dtype");
  if (h->wdtype == C4S_W_Q8) {
    if (!h->wscale || !h->wbias) return fail(ctx, C4S_EINVAL, "lmhead: 8-bit weights need wscale and wbias");
    if ((h->group != 32 && h->group != 64 && h->group != 128) || h->D % h->group != 0)
      return fail(ctx, C4S_EINVAL, "lmhead: group must be 32, 64 or 128 and divide D");
  }
  const uintptr_t al16 = reinterpret_cast<uintptr_t>(h->hidden) | reinterpret_cast<uintptr_t>(h->gamma) |
                         reinterpret_cast<uintptr_t>(h->beta) |
                         (h->wdtype == C4S_W_Q8 ? 0 : reinterpret_cast<uintptr_t>(h->weight));
  if ((al16 & 15u) || (reinterpret_cast<uintptr_t>(h->weight) & 7u))
    return fail(ctx, C4S_EINVAL, "lmhead: hidden, gamma, beta and weight must be 16-byte aligned (8-bit weight: 8)");
  return C4S_OK;
}

// The LM head into `logits` (row stride ld_out): one kernel, no workspace.
static int lmhead_launch(c4s_ctx* ctx, const c4s_head* h, float* logits, int64_t ld_out, hipStream_t s) {
  if (!logits) return fail(ctx, C4S_EINVAL, "lmhead: logits is NULL");
  if (ld_out < h->V) return fail(ctx, C4S_EINVAL, "lmhead: ld_out < V");
  c4s::LmHeadArgs a{};
  a.hidden = h->hidden;
  a.gamma = h->gamma;
  a.beta = h->beta;
  a.eps = h->eps;
  a.weight = h->weight;
  a.wkind = h->wdtype;
  a.group = h->group;
  a.wscale = h->wscale;
  a.wbias = h->wbias;
  a.bias = h->bias;
  a.logits = logits;
  a.ld_out = ld_out;
  a.M = h->M;
  a.D = h->D;
  a.V = h->V;
  hipError_t e = c4s::launch_lmhead(a, s);
  if (e != hipSuccess) return hip_fail(ctx, e, "lmhead launch");
  return C4S_OK;
}

static int lmhead_impl(c4s_ctx* ctx, const c4s_head* h, float* logits, int64_t ld_out, hipStream_t s) {
  int rc = lmhead_check(ctx, h);
  if (rc) return rc;
  return lmhead_launch(ctx, h, logits, ld_out, s);
}

int c4s_lmhead(c4s_ctx* ctx, const c4s_head* head, void* stream) {
  if (!ctx) return C4S_EINVAL;
  if (!head) return fail(ctx, C4S_EINVAL, "lmhead descriptor is NULL");
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  return lmhead_impl(ctx, head, head->logits, head->ld_out, static_cast<hipStream_t>(stream));
}

namespace {
// The rows of the sampler behind the LM head: logits, stride, dtype, row count
// and vocabulary come from the head.
c4s_rows head_rows(const c4s_rows& rows, const c4s_head* head, float* logits, int64_t ld) {
  c4s_rows r = rows;
  r.logits = logits;
  r.ld = ld;
  r.dtype = C4S_DTYPE_F32;
  r.n_rows = head->M;
  r.vocab = head->V;
  return r;
}
}  // namespace

// Both descriptors are checked, and every workspace sized, before anything is
// queued: a call that fails queues nothing.
int c4s_lmhead_sample(c4s_ctx* ctx, const c4s_head* head, const c4s_rows* rows, void* stream) {
  if (!ctx) return C4S_EINVAL;
  if (!head || !rows) return fail(ctx, C4S_EINVAL, "descriptor is NULL");
  int rc = lmhead_check(ctx, head);
  if (rc) return rc;
  c4s_rows r = head_rows(*rows, head, head->logits, head->logits ? head->ld_out : head->V);
  rc = validate_rows(ctx, &r, head->logits != nullptr);
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* logits = head->logits;
  if (!logits) {
    rc = ensure(ctx, &ctx->logits_ws, &ctx->logits_bytes,
                (size_t)std::max(head->M, 1) * (size_t)std::max(head->V, 1) * 4, "logits workspace", s);
    if (rc) return rc;
    logits = static_cast<float*>(ctx->logits_ws);
    r.logits = logits;
  }
  rc = rows_workspace(ctx, &r, s);
  if (rc) return rc;
  rc = lmhead_launch(ctx, head, logits, r.ld, s);
  if (rc) return rc;
  return launch_rows_checked(ctx, &r, s);
}

int c4s_lmhead_sample_noalloc(c4s_ctx* ctx, const c4s_head* head, const c4s_rows* rows, void* stream) {
  if (!ctx) return C4S_EINVAL;
  if (!head || !rows) return fail(ctx, C4S_EINVAL, "descriptor is NULL");
  if (!ctx->noalloc) return fail(ctx, C4S_EHIP, "lmhead_sample_noalloc: the static scratch has no address on this device");
  int rc = lmhead_check(ctx, head);
  if (rc) return rc;
  // One AR step at a vocabulary the sampler stages in LDS needs no sampler
  // workspace; larger vocabularies need the context's sort buffers.
  if (head->V > c4s::kLdsVocabMax)
    return fail(ctx, C4S_EINVAL, "lmhead_sample_noalloc: vocab above 12288 needs a workspace");
  const size_t lbytes = head->logits ? 0 : (size_t)head->M * (size_t)head->V * 4;
  if (lbytes > c4s::kNoAllocBytes)
    return fail(ctx, C4S_EINVAL, "lmhead_sample_noalloc: M x V x 4 logits (no logits buffer given) exceed the "
                                 "8 MiB static scratch");
  unsigned char* base = static_cast<unsigned char*>(ctx->noalloc);
  float* logits = head->logits ? head->logits : reinterpret_cast<float*>(base);
  const int64_t ld = head->logits ? head->ld_out : head->V;
  c4s_rows r = head_rows(*rows, head, logits, ld);
  rc = validate_rows(ctx, &r);   // before anything writes the caller's logits or the shared scratch
  if (rc) return rc;
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = lmhead_launch(ctx, head, logits, ld, s);
  if (rc) return rc;
  return launch_rows_checked(ctx, &r, s);
}

uint64_t c4s_seed_single(uint64_t seed) { return seed ? seed : 0x9E3779B97F4A7C15ull; }

void c4s_seed_batch(uint64_t seed, int32_t n, uint64_t* out) {
  if (!out) return;
  const uint64_t base = c4s_seed_single(seed);
  for (int32_t b = 0; b < n; ++b) out[b] = base + static_cast<uint64_t>(b) * 0x100000001b3ull;
}

// ---- synchronous single-row helpers -----------------------------------------------

namespace {

struct Stage {
  float* logits;
  int32_t* ids;
  int64_t* off;
  float* fparams;   // temp, top_p, penalty
  int32_t* iparams; // top_k, min_keep
  uint64_t* rng;
  int32_t* tok;
};

// The staging layout of one single-row call from `base` (device or host
// address); returns its size in bytes (through tok).
size_t stage_at(char* base, int32_t n, int64_t n_ids, Stage* st) {
  auto al = [](size_t b) { return (b + 255) & ~size_t(255); };
  const size_t b_logits = al((size_t)n * 4), b_ids = al((size_t)std::max<int64_t>(n_ids, 1) * 4);
  char* p = base;
  st->logits = reinterpret_cast<float*>(p); p += b_logits;
  st->ids = reinterpret_cast<int32_t*>(p); p += b_ids;
  st->off = reinterpret_cast<int64_t*>(p); p += al(16);
  st->fparams = reinterpret_cast<float*>(p); p += al(12);
  st->iparams = reinterpret_cast<int32_t*>(p); p += al(8);
  st->rng = reinterpret_cast<uint64_t*>(p); p += al(8);
  st->tok = reinterpret_cast<int32_t*>(p);
  return (size_t)(p - base) + 4;
}

// The pinned host staging area, at least `need` bytes.
int ensure_host_stage(c4s_ctx* ctx, size_t need) {
  if (need <= ctx->hstage_bytes) return C4S_OK;
  if (ctx->hstage) {
    hipError_t e = hipHostFree(ctx->hstage);
    ctx->hstage = nullptr;
    ctx->hstage_bytes = 0;
    if (e != hipSuccess) return hip_fail(ctx, e, "host staging");
  }
  hipError_t e = hipHostMalloc(&ctx->hstage, need, hipHostMallocDefault);
  if (e != hipSuccess) {
    ctx->hstage = nullptr;
    return e == hipErrorOutOfMemory ? fail(ctx, C4S_ENOMEM, "host staging: out of pinned memory")
                                    : hip_fail(ctx, e, "host staging");
  }
  ctx->hstage_bytes = need;
  return C4S_OK;
}

// One synchronous single-row call: the row, the history and the parameters
// gathered into pinned host memory, which the step reads and writes in place
// (the device maps it), then the results copied out after the step.
int host_call(c4s_ctx* ctx, float* logits, int32_t n, const int32_t* ids, int64_t n_ids,
              float temp, int32_t k, float p, float pen, int32_t min_keep, uint64_t* rng,
              uint32_t mode, bool write_back, int32_t* tok_out) {
  if (!ctx) return C4S_EINVAL;
  if (n < 0 || n_ids < 0) return fail(ctx, C4S_EINVAL, "negative size");
  if (n > c4s::kMaxVocab) return fail(ctx, C4S_EINVAL, "row too long");
  if (n > 0 && !logits) return fail(ctx, C4S_EINVAL, "logits is NULL");
  if (n_ids > 0 && !ids) return fail(ctx, C4S_EINVAL, "ids is NULL");
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  Stage hs, ds;
  int rc = ensure_host_stage(ctx, stage_at(nullptr, n, n_ids, &hs));
  if (rc) return rc;
  void* dev = nullptr;
  hipError_t e = hipHostGetDevicePointer(&dev, ctx->hstage, 0);
  if (e != hipSuccess) return hip_fail(ctx, e, "host staging: device address");
  stage_at(static_cast<char*>(ctx->hstage), n, n_ids, &hs);
  stage_at(static_cast<char*>(dev), n, n_ids, &ds);
  hipStream_t s = ctx->host_stream;
  const int64_t off[2] = {0, n_ids};
  const float fp[3] = {temp, p, pen};
  const int32_t ip[2] = {k, min_keep};
  if (n > 0) std::memcpy(hs.logits, logits, (size_t)n * 4);
  if (n_ids > 0) std::memcpy(hs.ids, ids, (size_t)n_ids * 4);
  std::memcpy(hs.off, off, sizeof(off));
  std::memcpy(hs.fparams, fp, sizeof(fp));
  std::memcpy(hs.iparams, ip, sizeof(ip));
  if (rng) std::memcpy(hs.rng, rng, 8);
  c4s_rows r{};
  r.logits = ds.logits;
  r.ld = n;
  r.dtype = C4S_DTYPE_F32;
  r.n_rows = 1;
  r.vocab = n;
  r.hist_ids = ds.ids;
  r.hist_offsets = ds.off;
  r.temperature = ds.fparams;
  r.top_p = ds.fparams + 1;
  r.rep_penalty = ds.fparams + 2;
  r.top_k = ds.iparams;
  r.min_keep = ds.iparams + 1;
  r.rng_state = ds.rng;
  r.out_token = ds.tok;
  r.out_masked = write_back ? ds.logits : nullptr;
  r.mode = mode;
  rc = validate_rows(ctx, &r);
  if (rc) return rc;
  rc = launch_rows_checked(ctx, &r, s);
  if (rc) return rc;
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(ctx, e, "single-row call");
  if (write_back && n > 0) std::memcpy(logits, hs.logits, (size_t)n * 4);
  if (rng) std::memcpy(rng, hs.rng, 8);
  if (tok_out) std::memcpy(tok_out, hs.tok, 4);
  return C4S_OK;
}

}  // namespace

int c4s_host_temperature(c4s_ctx* ctx, float* logits, int32_t n, float temp) {
  if (ctx && n == 0) return C4S_OK;
  return host_call(ctx, logits, n, nullptr, 0, temp, 0, 1.0f, 1.0f, 1, nullptr,
                   C4S_MODE_CUSTOM | C4S_P_TEMPERATURE, true, nullptr);
}

int c4s_host_repetition_penalty(c4s_ctx* ctx, float* logits, int32_t n, const int32_t* ids,
                                int64_t n_ids, float penalty) {
  if (ctx && n == 0) return C4S_OK;
  return host_call(ctx, logits, n, ids, n_ids, 1.0f, 0, 1.0f, penalty, 1, nullptr,
                   C4S_MODE_CUSTOM | C4S_P_PENALTY, true, nullptr);
}

int c4s_host_top_k(c4s_ctx* ctx, float* logits, int32_t n, int32_t k) {
  if (ctx && n == 0) return C4S_OK;
  return host_call(ctx, logits, n, nullptr, 0, 1.0f, k, 1.0f, 1.0f, 1, nullptr,
                   C4S_MODE_CUSTOM | C4S_P_TOP_K, true, nullptr);
}

int c4s_host_top_p(c4s_ctx* ctx, float* logits, int32_t n, float p, int32_t min_keep) {
  if (ctx && n == 0) return C4S_OK;  // the reference dereferences an empty max_element
  return host_call(ctx, logits, n, nullptr, 0, 1.0f, 0, p, 1.0f, min_keep, nullptr,
                   C4S_MODE_CUSTOM | C4S_P_TOP_P, true, nullptr);
}

int c4s_host_argmax(c4s_ctx* ctx, const float* logits, int32_t n, int32_t* out) {
  if (!out) return fail(ctx, C4S_EINVAL, "out is NULL");
  if (ctx && n == 0) { *out = 0; return C4S_OK; }   // max_element(empty) - begin == 0
  return host_call(ctx, const_cast<float*>(logits), n, nullptr, 0, 1.0f, 0, 1.0f, 1.0f, 1,
                   nullptr, C4S_MODE_CUSTOM | C4S_T_ARGMAX, false, out);
}

int c4s_host_draw(c4s_ctx* ctx, const float* logits, int32_t n, uint64_t* rng, int32_t* out) {
  if (!out || !rng) return fail(ctx, C4S_EINVAL, "out/rng is NULL");
  if (ctx && n == 0) return fail(ctx, C4S_EINVAL, "draw over an empty row");
  return host_call(ctx, const_cast<float*>(logits), n, nullptr, 0, 1.0f, 0, 1.0f, 1.0f, 1, rng,
                   C4S_MODE_CUSTOM | C4S_T_DRAW, false, out);
}

int c4s_hbm_probe(c4s_ctx* ctx, const void* src, void* dst, int64_t bytes, int32_t mode,
                  void* stream) {
  if (!ctx) return C4S_EINVAL;
  if (!src || !dst || bytes < 0 || (bytes % 16) != 0 || (mode != 0 && mode != 1))
    return fail(ctx, C4S_EINVAL, "hbm_probe: bad arguments");
  DeviceGuard g(ctx->device);
  if (g.err != hipSuccess) return hip_fail(ctx, g.err, "hipSetDevice");
  hipError_t e = c4s::launch_hbm_probe(src, dst, bytes, mode, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(ctx, e, "hbm_probe launch");
  return C4S_OK;
}

}  // extern "C"
