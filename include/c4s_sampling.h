/* c4s_sampling.h -- C ABI of the MI355X (gfx950) token-sampling library for
 * the c4tts Text2Semantic AR loop (libc4s_sampling.so).
 *
 * Plain C: pointers, sizes, status codes. No HIP or torch types appear in the
 * signatures; a HIP stream is passed as `void*` (NULL = the default stream).
 *
 * Reference interfaces replaced (paths in the c4tts tree):
 *   include/c4tts/t2s.h:82-89          c4::t2s::sampling::{temperature,
 *                                      repetition_penalty, top_k, top_p, argmax}
 *   src/t2s/sampling.cpp:14-76         their bodies
 *   src/t2s/text2semantic.cpp:142-166  per-step processor chain + xorshift64
 *                                      inverse-CDF draw (single stream)
 *   src/t2s/text2semantic.cpp:303-337  the same, per row of generate_batch
 *   src/t2s/text2semantic.cpp:109, :292-294   RNG seeding
 *   src/t2s/text2semantic.cpp:118-121, :283-286  LM head (final_norm +
 *                                      semantic_head), src/nn/nn.cpp:11-16, :73-83
 *
 * Conventions
 *   - Every function returns C4S_OK (0) or an error code; no exceptions cross
 *     the ABI. Degenerate sampling parameters keep the reference's no-op
 *     meaning (temperature 1 or <= 0, penalty 1, top_k <= 0 or >= vocab,
 *     out-of-range history ids) and are not errors.
 *   - Device entry points are asynchronous on the given stream; the caller
 *     owns every input/output buffer (device memory); the context owns its
 *     workspace. A context is not thread-safe: use one per host thread.
 *   - Workspaces grow on first use (hipMalloc, which synchronises the device).
 *     c4s_sample_rows with vocab <= 12288 uses none. While the stream is being
 *     captured into a graph a workspace never grows (C4S_EINVAL): make one call
 *     of the same shape outside the capture first. Once a captured call used a
 *     workspace, a later growth keeps the old buffer alive until c4s_destroy.
 *   - Input contract: logits are finite or -inf (no +inf/NaN), temperature is
 *     1, <= 0, or keeps logits/temperature finite.
 *   - top_p tie order: when the nucleus cut falls inside a group of equal
 *     values, the lower token ids of that group survive. (The reference's
 *     unstable std::sort leaves this choice to the host's sort permutation.)
 */
#ifndef C4S_SAMPLING_H
#define C4S_SAMPLING_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  C4S_OK = 0,
  C4S_EINVAL = 1, /* null pointer, bad size/dtype/mode, unsupported shape */
  C4S_EHIP = 2,   /* a HIP call failed; see c4s_last_error */
  C4S_ENOMEM = 3,
  C4S_ETIMEOUT = 4 /* a c4s_sample_stream call of this context gave up a row (see c4s_stream_status) */
};

enum { C4S_DTYPE_F32 = 0, C4S_DTYPE_BF16 = 1 };
/* LM head weight storage: bf16; fp32 (the reference's .npy weights load as
 * float32, include/c4tts/npy.h:202-206); 8-bit affine groups along the input
 * dimension, codes 0..255 as bytes (the quantized_matmul layout of
 * src/t2s/gpt2.cpp:49-62 at 8 bits). */
enum { C4S_W_BF16 = 0, C4S_W_F32 = 1, C4S_W_Q8 = 2 };

/* Processor selection (c4s_rows.mode).
 * C4S_MODE_CHAIN runs the reference chain per row (text2semantic.cpp:142-166):
 *   repetition penalty, then do_sample[b] ? temperature -> top_k -> top_p ->
 *   draw : argmax.
 * C4S_MODE_CUSTOM | C4S_P_* | (C4S_T_ARGMAX or C4S_T_DRAW or neither) runs only
 *   the listed processors, in chain order, on every row (this is what backs the
 *   single-processor legacy functions). */
enum {
  C4S_MODE_CHAIN = 0,
  C4S_P_PENALTY = 1u << 0,
  C4S_P_TEMPERATURE = 1u << 1,
  C4S_P_TOP_K = 1u << 2,
  C4S_P_TOP_P = 1u << 3,
  C4S_T_ARGMAX = 1u << 4,
  C4S_T_DRAW = 1u << 5,
  C4S_MODE_CUSTOM = 1u << 8
};

/* Per-row statistics (c4s_rows.out_stats, 4 words per row). */
enum {
  C4S_STAT_PATH = 0,       /* bit0 drawn, bit1 top-k applied, bit2 top-p applied, bit3 greedy,
                              bit4 decided without the multi-pass chain, bit5 decided on a candidate
                              list, bit6 (vocab above 12288) the row read once; c4s_stream.out_stats:
                              or-ed over the steps, and bit30 when the row's
                              speculative chain gave up (see c4s_stream_status) */
  C4S_STAT_TOPP_EXACT = 1, /* nucleus cut fell inside the error bound -> exact pass ran */
  C4S_STAT_DRAW_EXACT = 2, /* draw fell inside the error bound -> exact pass ran */
  C4S_STAT_KEPT = 3        /* ids left with nonzero weight before the draw */
};

typedef struct c4s_ctx c4s_ctx;

/* One AR step over a batch of rows (device pointers).
 * Replaces the per-row body of text2semantic.cpp:303-337 (and :142-166 for one
 * row); the logits stay on the device and only tokens are produced. */
typedef struct c4s_rows {
  const void* logits;           /* [n_rows][ld] f32 or bf16 */
  int64_t ld;                   /* row stride in elements, >= vocab */
  int32_t dtype;                /* C4S_DTYPE_* */
  int32_t n_rows;
  int32_t vocab;                /* 1 .. 1048576 */
  const int32_t* hist_ids;      /* CSR history (generated ids), may be NULL if no penalty */
  const int64_t* hist_offsets;  /* [n_rows+1] */
  const float* temperature;     /* [n_rows] */
  const int32_t* top_k;         /* [n_rows] */
  const float* top_p;           /* [n_rows] */
  const float* rep_penalty;     /* [n_rows] */
  const int32_t* min_keep;      /* [n_rows] or NULL (= 1, the reference default) */
  const uint8_t* do_sample;     /* [n_rows] or NULL (= all sample) */
  const uint8_t* row_active;    /* [n_rows] or NULL; inactive rows: token -1, RNG untouched */
  uint64_t* rng_state;          /* [n_rows] xorshift64 state, advanced once per drawn row */
  int32_t* out_token;           /* [n_rows] */
  float* out_masked;            /* [n_rows][vocab] or NULL: row state before argmax/draw */
  uint32_t* out_stats;          /* [n_rows][4] or NULL */
  uint32_t mode;                /* C4S_MODE_CHAIN or C4S_MODE_CUSTOM | ... */
  /* The AR loop's history gen[b] kept on the device across steps, as a set:
   * [n_rows][(vocab + 31) / 32] bit words or NULL. When set it is the penalty's
   * history in place of hist_ids/hist_offsets (sampling.cpp:22 applies each
   * distinct id once, so the set is the history), and after the step every
   * active row's token joins it unless it equals stop_token
   * (text2semantic.cpp:333-334). Fill it once with c4s_hist_bits_init. */
  uint32_t* hist_bits;
  int32_t stop_token;           /* with hist_bits: the token that does not join (-1: none) */
} c4s_rows;

/* Many AR steps of a batch whose logits are already known (synthetic or
 * replayed streams): row b's history starts from its CSR ids and grows by each
 * token it samples that is not stop_token; a row that samples stop_token is
 * done (later steps report -1, RNG frozen), as generate_batch does
 * (text2semantic.cpp:333-334). Requires vocab <= 12288 (row staged in LDS). */
typedef struct c4s_stream {
  const float* logits;          /* step s, row b at logits + s*step_stride + b*ld */
  int64_t ld;
  int64_t step_stride;
  int32_t n_steps;
  int32_t n_rows;
  int32_t vocab;
  int32_t stop_token;           /* < 0: never stop */
  const int32_t* hist_ids;
  const int64_t* hist_offsets;
  const float* temperature;
  const int32_t* top_k;
  const float* top_p;
  const float* rep_penalty;
  const uint8_t* do_sample;     /* or NULL */
  uint64_t* rng_state;
  int32_t* out_tokens;          /* [n_steps][n_rows] */
  uint32_t* out_stats;          /* [n_rows][4] (summed over steps) or NULL */
  uint32_t flags;               /* C4S_STREAM_* */
} c4s_stream;

/* c4s_stream.flags: run every step of every row in one persistent kernel
 * instead of the two-phase path (scan of all steps, then the per-row chain). */
#define C4S_STREAM_SEQUENTIAL 1u
/* c4s_stream.flags: in the two-phase path, decide full-vocabulary rows one
 * step after the other (the pipelined row chain) instead of several steps at
 * once with each checked against the tokens drawn since (the default for
 * calls of at most 1024 steps). Both give the same tokens. */
#define C4S_STREAM_NO_SPECULATION 2u

/* LM head: LayerNorm(hidden) @ weight^T + bias -> f32 logits
 * (text2semantic.cpp:118-121; nn.cpp:73-83 eps/biased variance, nn.cpp:11-16
 * weight stored (out, in)). The LayerNorm is folded into the product, never
 * materialised: logits[m][n] = inv_m (G[m][n] - mu_m c[n]) + d[n] + bias[n],
 * G = (W gamma) x^T with W gamma split into two bf16 terms, c = W gamma and
 * d = W beta over the inputs, mu_m and inv_m = 1 / sqrt(var_m + eps) from the
 * row's sums; accumulation in fp32 (the tests hold it within 2e-4 absolute of
 * an fp64 evaluation for logits up to 4 in magnitude). hidden_dim must be a positive multiple of 32; hidden, gamma,
 * beta and weight must be 16-byte aligned (8-bit weights: 8), else C4S_EINVAL. */
typedef struct c4s_head {
  const uint16_t* hidden;       /* [M][D] bf16 */
  const float* gamma;           /* [D] */
  const float* beta;            /* [D] */
  float eps;                    /* 1e-5 in the reference (nn.h:49-50) */
  const void* weight;           /* [V][D] in wdtype (semantic_head.weight, [out][in]) */
  const float* bias;            /* [V] */
  int32_t M, D, V;
  float* logits;                /* [M][ld_out] f32 */
  int64_t ld_out;
  int32_t wdtype;               /* C4S_W_*; 0 (zero-initialised descriptor) is bf16 */
  int32_t group;                /* C4S_W_Q8: inputs per scale group: 32, 64 or 128 */
  const float* wscale;          /* C4S_W_Q8: [V][D / group] */
  const float* wbias;           /* C4S_W_Q8: [V][D / group]; w[n][k] = wscale * q[n][k] + wbias */
} c4s_head;

int c4s_create(int device, c4s_ctx** out);
int c4s_destroy(c4s_ctx* ctx);
const char* c4s_last_error(const c4s_ctx* ctx);
const char* c4s_version(void);

/* text2semantic.cpp:303-337 (batched) / :142-166 (single row). */
int c4s_sample_rows(c4s_ctx* ctx, const c4s_rows* rows, void* stream);
/* text2semantic.cpp:296-337 over n_steps with precomputed logits. Queued on
 * `stream` like the other entry points, except that with the overlapped
 * schedule (rows at most the chains' CUs, 256 steps or more) the calling
 * thread first waits until the previous such call of this context has ended
 * on the GPU: one call in flight per context. Not capturable: returns
 * C4S_EINVAL while `stream` is being captured into a graph. */
int c4s_sample_stream(c4s_ctx* ctx, const c4s_stream* st, void* stream);
/* The speculative chains of c4s_sample_stream (no counterpart in the
 * reference, which decides each step on the host) wait on each other with
 * bounded waits. A wait that expires (about 0.3 s by default; it does not
 * happen on a working device) stops that row: its tokens from that step of
 * the call are -1 and its RNG state stays at the step where it stopped. The
 * context records it, and the next c4s_sample_stream call returns
 * C4S_ETIMEOUT without queuing anything once the failing call has ended (the
 * overlapped schedule waits for it; otherwise a call reports what has ended
 * by then). c4s_stream_status synchronizes `stream` and returns C4S_ETIMEOUT
 * or C4S_OK; either report clears the record. */
int c4s_stream_status(c4s_ctx* ctx, void* stream);
/* Polls of those bounded waits before they give up (<= 0: the default,
 * 4194304). For tests of the C4S_ETIMEOUT path. */
int c4s_set_wait_limit(c4s_ctx* ctx, int32_t polls);
/* text2semantic.cpp:118-121 / :283-286 (head(cur)). */
int c4s_lmhead(c4s_ctx* ctx, const c4s_head* head, void* stream);
/* head(cur) then the chain on its logits (text2semantic.cpp:297-337 in one
 * call); rows->logits/ld/dtype/vocab/n_rows are taken from `head`. */
int c4s_lmhead_sample(c4s_ctx* ctx, const c4s_head* head, const c4s_rows* rows, void* stream);

/* c4s_lmhead_sample without any allocation: no counterpart in the reference.
 * For callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The same kernels as
 * c4s_lmhead_sample; when head->logits is NULL the logits live in a static
 * device array of 8 MiB that the library holds on each GPU until the process
 * ends. Limits: M x V x 4 bytes within 8 MiB when no logits buffer is given,
 * and vocab <= 12288; otherwise C4S_EINVAL. Every call on one GPU shares that GPU's array (the
 * kernels overwrite all of it that they read; nothing needs clearing): calls
 * that overlap on one GPU, from any context or stream, race. */
int c4s_lmhead_sample_noalloc(c4s_ctx* ctx, const c4s_head* head, const c4s_rows* rows, void* stream);

/* The LM head's tensors read from the reference's weight store
 * (src/core/weights.cpp:13-58: <root>.safetensors when that file exists, else
 * <root>/<name>.npy per tensor; names of src/t2s/text2semantic.cpp:114-115:
 * final_norm.weight, final_norm.bias, semantic_head.weight [V][D],
 * semantic_head.bias), converted to the storage `wdtype` and copied to the
 * calling thread's current HIP device. C4S_W_Q8 from float weights makes
 * groups of `group` inputs (bias = the group's minimum, scale = its range / 255);
 * a file that already holds an 8-bit head (u32 weight words of four codes,
 * least significant byte first, plus semantic_head.scales and
 * semantic_head.biases of [V][D / group]) is taken as it is. The pointers go
 * into c4s_head (hidden, logits and M are the caller's). Errors: C4S_EINVAL or
 * C4S_EHIP, text from c4s_weights_last_error() (this thread's last failure). */
typedef struct c4s_head_weights {
  float* gamma;                 /* [D] device */
  float* beta;                  /* [D] device */
  void* weight;                 /* [V][D] device, in wdtype */
  float* bias;                  /* [V] device */
  float* wscale;                /* C4S_W_Q8: [V][D / group] device */
  float* wbias;                 /* C4S_W_Q8: [V][D / group] device */
  int32_t D, V, wdtype, group;
} c4s_head_weights;
int c4s_head_weights_load(const char* root, int32_t wdtype, int32_t group, c4s_head_weights* out);
int c4s_head_weights_free(c4s_head_weights* w);
/* Host only (no device): one tensor of the store as fp32 (f16/bf16/f32/f64
 * data), its shape in shape[0 .. *ndim) (up to 8 dimensions); out may be NULL
 * to ask for the shape, else it must hold cap >= the element count. The
 * reference's npy loader (include/c4tts/npy.h:47-137) / load_safetensors. */
int c4s_tensor_read_f32(const char* root, const char* name, float* out, int64_t cap, int64_t* shape,
                        int32_t* ndim);
const char* c4s_weights_last_error(void);

/* hist_bits[b] = the set of row b's CSR history ids in [0, vocab) (ids
 * outside are skipped, sampling.cpp:24); the starting state of
 * c4s_rows.hist_bits (text2semantic.cpp:196-372 keeps gen[b] across steps). */
int c4s_hist_bits_init(c4s_ctx* ctx, const int32_t* hist_ids, const int64_t* hist_offsets, int32_t n_rows,
                       int32_t vocab, uint32_t* hist_bits, void* stream);

/* Seeds (host only): text2semantic.cpp:109 and :292-294. */
uint64_t c4s_seed_single(uint64_t seed);
void c4s_seed_batch(uint64_t seed, int32_t n, uint64_t* out);

/* Host-buffer single-row helpers: synchronous, copy in/out through the
 * context's staging memory. They back the reference's five C++ entry points
 * (include/c4tts/t2s.h:82-89, bodies sampling.cpp:14-76) and the inline draw
 * (text2semantic.cpp:150-165). n == 0 is a no-op (argmax returns 0). */
int c4s_host_temperature(c4s_ctx* ctx, float* logits, int32_t n, float temp);
int c4s_host_repetition_penalty(c4s_ctx* ctx, float* logits, int32_t n, const int32_t* ids,
                                int64_t n_ids, float penalty);
int c4s_host_top_k(c4s_ctx* ctx, float* logits, int32_t n, int32_t k);
int c4s_host_top_p(c4s_ctx* ctx, float* logits, int32_t n, float p, int32_t min_keep);
int c4s_host_argmax(c4s_ctx* ctx, const float* logits, int32_t n, int32_t* out);
int c4s_host_draw(c4s_ctx* ctx, const float* logits, int32_t n, uint64_t* rng, int32_t* out);

/* Achievable-bandwidth probe: mode 0 copies `bytes` from src to dst, mode 1
 * only reads src (dst needs 4 bytes). bytes must be a multiple of 16. */
int c4s_hbm_probe(c4s_ctx* ctx, const void* src, void* dst, int64_t bytes, int32_t mode,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* C4S_SAMPLING_H */
