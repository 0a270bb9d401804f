// Host side of the activation observer: Algorithm R decisions and
// percentiles (reference src/quant/observer.cpp:8-51).
#include "observer.hpp"

#include <algorithm>
#include <cmath>

namespace esm_gfx950 {
namespace obs {

size_t plan(Reservoir& r, size_t n, uint32_t* slots, uint32_t* positions) {
  constexpr uint32_t kNone = UINT32_MAX;
  // newest[j]: position in this batch of slot j's newest value.
  std::vector<uint32_t> newest(kReservoirSize, kNone);
  size_t i = 0;
  // Fill phase: the first kReservoirSize values of the site's history take
  // the slots in order and draw nothing.
  for (; i < n && r.samples.size() < kReservoirSize; ++i) {
    newest[r.samples.size()] = static_cast<uint32_t>(i);
    r.samples.push_back(0.0f);
    ++r.total_seen;
  }
  // Replacement phase: one draw over [0, total_seen] per value.
  for (; i < n; ++i) {
    std::uniform_int_distribution<size_t> pick(0, r.total_seen);
    const size_t j = pick(r.rng);
    if (j < kReservoirSize) newest[j] = static_cast<uint32_t>(i);
    ++r.total_seen;
  }
  size_t count = 0;
  for (uint32_t j = 0; j < kReservoirSize; ++j) {
    if (newest[j] == kNone) continue;
    slots[count] = j;
    positions[count] = newest[j];
    ++count;
  }
  return count;
}

float percentile(const Reservoir& r, float pctile) {
  if (r.samples.empty()) return 0.0f;
  // Index floor(clamp(pctile / 100) * (size - 1)), formed in float as the
  // reference forms it (observer.cpp:41-45); selection instead of a full
  // sort returns the same order statistic.
  const float frac = std::clamp(pctile / 100.0f, 0.0f, 1.0f);
  size_t idx = static_cast<size_t>(std::floor(frac * static_cast<float>(r.samples.size() - 1)));
  if (idx >= r.samples.size()) idx = r.samples.size() - 1;
  std::vector<float> v = r.samples;
  std::nth_element(v.begin(), v.begin() + static_cast<std::ptrdiff_t>(idx), v.end());
  return v[idx];
}

}  // namespace obs
}  // namespace esm_gfx950
