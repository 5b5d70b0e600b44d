// c4::t2s::sampling on MI355X -- drop-in for the reference declarations in
// include/c4tts/t2s.h:82-89 (same namespace, names, signatures and default
// argument), implemented over the C ABI of libc4s_sampling.so.
//
// Semantics are the reference's (src/t2s/sampling.cpp:14-76): in place on the
// caller's vector, degenerate parameters are silent no-ops, out-of-range
// history ids are skipped. The work runs on the GPU; there is no CPU path, so
// a missing or failing device raises std::runtime_error.
//
// Two additions the reference keeps inline in its AR loop:
//   draw()          text2semantic.cpp:150-165, xorshift64 + inverse-CDF draw
//   seed_single()   text2semantic.cpp:109
#pragma once

#include <cstdint>
#include <vector>

namespace c4 {
namespace t2s {
namespace sampling {

void temperature(std::vector<float>& logits, float temp);
void repetition_penalty(std::vector<float>& logits, const std::vector<int>& prev_tokens,
                        float penalty);
void top_k(std::vector<float>& logits, int k);
void top_p(std::vector<float>& logits, float p, int min_tokens_to_keep = 1);
int argmax(const std::vector<float>& logits);

// Draws one token from `logits` (already processed) and advances `rng`.
int draw(const std::vector<float>& logits, uint64_t& rng);
uint64_t seed_single(uint64_t seed);

// Device used by the functions above (default 0); set before the first call.
void set_device(int device);

}  // namespace sampling
}  // namespace t2s
}  // namespace c4
