// Implementation of c4tts/t2s_sampling.h over the C ABI (include/c4s_sampling.h).
// One process-wide context per thread, created on first use on the selected device.

#include "c4tts/t2s_sampling.h"

#include <memory>
#include <stdexcept>
#include <string>

#include "../../include/c4s_sampling.h"

namespace c4 {
namespace t2s {
namespace sampling {
namespace {

int g_device = 0;

struct CtxHolder {
  c4s_ctx* ctx = nullptr;
  ~CtxHolder() { c4s_destroy(ctx); }
};

c4s_ctx* ctx() {
  thread_local CtxHolder h;
  if (!h.ctx) {
    const int rc = c4s_create(g_device, &h.ctx);
    if (rc != C4S_OK)
      throw std::runtime_error("c4s: no usable gfx950 device " + std::to_string(g_device) +
                               " (code " + std::to_string(rc) + ")");
  }
  return h.ctx;
}

void check(int rc, const char* what) {
  if (rc != C4S_OK)
    throw std::runtime_error(std::string("c4s ") + what + ": " + c4s_last_error(ctx()));
}

}  // namespace

void set_device(int device) { g_device = device; }

void temperature(std::vector<float>& logits, float temp) {
  check(c4s_host_temperature(ctx(), logits.data(), static_cast<int32_t>(logits.size()), temp),
        "temperature");
}

void repetition_penalty(std::vector<float>& logits, const std::vector<int>& prev_tokens,
                        float penalty) {
  static_assert(sizeof(int) == sizeof(int32_t), "int must be 32-bit");
  check(c4s_host_repetition_penalty(ctx(), logits.data(), static_cast<int32_t>(logits.size()),
                                    reinterpret_cast<const int32_t*>(prev_tokens.data()),
                                    static_cast<int64_t>(prev_tokens.size()), penalty),
        "repetition_penalty");
}

void top_k(std::vector<float>& logits, int k) {
  check(c4s_host_top_k(ctx(), logits.data(), static_cast<int32_t>(logits.size()), k), "top_k");
}

void top_p(std::vector<float>& logits, float p, int min_tokens_to_keep) {
  check(c4s_host_top_p(ctx(), logits.data(), static_cast<int32_t>(logits.size()), p,
                       min_tokens_to_keep),
        "top_p");
}

int argmax(const std::vector<float>& logits) {
  int32_t out = 0;
  check(c4s_host_argmax(ctx(), logits.data(), static_cast<int32_t>(logits.size()), &out), "argmax");
  return out;
}

int draw(const std::vector<float>& logits, uint64_t& rng) {
  int32_t out = 0;
  check(c4s_host_draw(ctx(), logits.data(), static_cast<int32_t>(logits.size()), &rng, &out),
        "draw");
  return out;
}

uint64_t seed_single(uint64_t seed) { return c4s_seed_single(seed); }

}  // namespace sampling
}  // namespace t2s
}  // namespace c4
