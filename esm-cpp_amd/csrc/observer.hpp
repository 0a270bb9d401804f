// Activation observer for static-quantisation calibration: per site, a
// reservoir of |values| kept by Algorithm R, then percentiles
// (reference include/esm_cpp/observer.h:13-47, src/quant/observer.cpp:8-51).
//
// Algorithm R's decisions depend only on how many values a site has seen,
// never on the values: element i (0-based over the site's whole history)
// fills slot i while the reservoir is short, and afterwards replaces slot j =
// uniform(0, i) when j < the reservoir size. plan() draws those decisions for
// a batch of n values on the host, with the same generator and distribution
// as the reference (std::mt19937 seeded 0xc1b1ce, std::uniform_int_distribution
// over [0, total_seen]), and returns the batch positions whose values end up
// in the reservoir. The values themselves are gathered on the device.
#pragma once

#include <cstddef>
#include <cstdint>
#include <random>
#include <vector>

namespace esm_gfx950 {
namespace obs {

constexpr size_t kReservoirSize = 65536;  // ActivationObserver::kReservoirSize

struct Reservoir {
  std::vector<float> samples;  // |values|, at most kReservoirSize
  size_t total_seen = 0;
  std::mt19937 rng{0xc1b1ce};
};

// Advances r over n more values (n < 2^32 - 1). Writes, for every slot whose
// newest value comes from this batch, the slot and the value's position in
// the batch; returns how many (at most kReservoirSize). Slots opened by the
// fill phase hold 0 until the caller stores the gathered values.
size_t plan(Reservoir& r, size_t n, uint32_t* slots, uint32_t* positions);

// The pctile-th percentile (0..100) of r's samples, 0 when empty
// (ActivationObserver::Percentile, src/quant/observer.cpp:32-49).
float percentile(const Reservoir& r, float pctile);

}  // namespace obs
}  // namespace esm_gfx950
