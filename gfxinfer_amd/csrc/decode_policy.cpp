// Online MTP depth selection: pick each speculative round's draft count by the tokens
// per millisecond each candidate depth has delivered so far (the reference roadmap's
// "Online MTP depth selection based on accepted tokens per millisecond",
// docs/ROADMAP.md:51, which the reference does not implement).  Host only and
// deterministic: untried candidates first (shallowest first), then the best measured
// rate, with a periodic re-measurement of the other candidates in turn so that a depth
// whose rate improved (acceptance drifts with the text) is noticed.
#include <algorithm>
#include <new>

#include "common.hpp"
#include "runtime.hpp"

namespace {

constexpr uint32_t kCandidateDepths[] = {1, 2, 3, 4, 6, 8, 12, 16, 24, 31};
constexpr double kWeight = 0.25;       // exponential average weight of a new round
constexpr uint64_t kProbeInterval = 16;

}  // namespace

gfxinfer_depth_policy::gfxinfer_depth_policy(uint32_t maximum_depth) {
  for (const uint32_t d : kCandidateDepths) {
    if (d <= maximum_depth) candidates.push_back({d, 0, 0.0, 0.0});
  }
  if (candidates.empty() || candidates.back().depth != maximum_depth) {
    candidates.push_back({maximum_depth, 0, 0.0, 0.0});  // the configured depth is a candidate
  }
}

uint32_t gfxinfer_depth_policy::choose(uint32_t limit) {
  ++round;
  std::size_t usable = 0;  // candidates with depth <= limit: a prefix
  while (usable < candidates.size() && candidates[usable].depth <= limit) ++usable;
  if (usable == 0) return limit;
  for (std::size_t i = 0; i < usable; ++i) {
    if (candidates[i].rounds == 0) return candidates[i].depth;
  }
  std::size_t best = 0;
  for (std::size_t i = 1; i < usable; ++i) {
    const Candidate& c = candidates[i];
    const Candidate& b = candidates[best];
    if (c.tokens * b.ms > b.tokens * c.ms) best = i;  // c.tokens / c.ms > b.tokens / b.ms
  }
  if (round % kProbeInterval == 0 && usable > 1) {
    // re-measure the other candidates in turn
    const std::size_t other = probe++ % (usable - 1);
    return candidates[other < best ? other : other + 1].depth;
  }
  return candidates[best].depth;
}

bool gfxinfer_depth_policy::record(uint32_t depth, uint32_t emitted, double milliseconds) {
  if (!(milliseconds > 0.0)) return false;
  for (Candidate& c : candidates) {
    if (c.depth != depth) continue;
    if (c.rounds == 0) {
      c.tokens = emitted;
      c.ms = milliseconds;
    } else {
      c.tokens += kWeight * (emitted - c.tokens);
      c.ms += kWeight * (milliseconds - c.ms);
    }
    ++c.rounds;
    return true;
  }
  return false;  // not a candidate (a short final round's depth): nothing to learn
}

extern "C" int32_t gfxinfer_depth_policy_create(uint32_t maximum_depth, gfxinfer_depth_policy** out) {
  if (out == nullptr || maximum_depth == 0 || maximum_depth > 31) {
    return gfx950::fail(GFXI_INVALID_ARGUMENT, "depth policy needs a maximum depth in [1, 31]");
  }
  try {
    *out = new gfxinfer_depth_policy(maximum_depth);
  } catch (const std::bad_alloc&) {
    return gfx950::fail(GFXI_OUT_OF_MEMORY, "depth policy allocation failed");
  }
  return gfx950::ok();
}

extern "C" void gfxinfer_depth_policy_destroy(gfxinfer_depth_policy* policy) { delete policy; }

extern "C" uint32_t gfxinfer_depth_policy_choose(gfxinfer_depth_policy* policy, uint32_t limit) {
  return policy == nullptr || limit == 0 ? 0u : policy->choose(limit);
}

extern "C" int32_t gfxinfer_depth_policy_record(gfxinfer_depth_policy* policy, uint32_t depth,
                                                uint32_t emitted_tokens, double milliseconds) {
  if (policy == nullptr || emitted_tokens == 0 || emitted_tokens > depth + 1 || !(milliseconds > 0.0)) {
    return gfx950::fail(GFXI_INVALID_ARGUMENT, "depth policy record needs 1..depth+1 tokens and a time");
  }
  policy->record(depth, emitted_tokens, milliseconds);
  return gfx950::ok();
}
