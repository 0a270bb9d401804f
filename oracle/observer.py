"""CPU restatement of esm::ActivationObserver (reference
src/quant/observer.cpp:8-51, include/esm_cpp/observer.h:13-47).

TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker of the device
observer; the product never imports it.

The reservoir's decisions come from two pieces of the C++ standard library
as shipped with GCC 11.4 (libstdc++, the toolchain the reference and this
repository compile with; not vendored in the reference), restated here from
their published algorithms:
  - std::mt19937: MT19937 (Matsumoto & Nishimura, ACM TOMACS 8(1), 1998),
    seeded as C++ [rand.eng.mers] specifies (x[i] = 1812433253 *
    (x[i-1] ^ (x[i-1] >> 30)) + i); pinned by the standard's known answer
    (the 10000th output of a default-seeded engine is 4123659995);
  - std::uniform_int_distribution<size_t>(0, b) driven by a 32-bit engine:
    libstdc++ 11 downscales with Lemire's nearly divisionless method (Lemire,
    ACM TOMACS 29(1), 2019) using a 64-bit product
    (/usr/include/c++/11/bits/uniform_int_dist.h, _S_nd and the
    __urngrange == UINT32_MAX branch). Restated for b + 1 < 2^32, i.e. a
    site's first 2^32 - 1 values.
Pinned against the reference's own observer compiled from source
(oracle/_ref) in tests/test_observer.py.
"""
from __future__ import annotations

import math
from typing import Dict, List

import numpy as np

RESERVOIR_SIZE = 65536  # ActivationObserver::kReservoirSize (observer.h:24)
SEED = 0xC1B1CE  # Reservoir::rng seed (observer.h:43)


class MT19937:
    """32-bit Mersenne Twister, outputs drawn in blocks of 624."""

    N, M = 624, 397
    A, UPPER, LOWER = 0x9908B0DF, 0x80000000, 0x7FFFFFFF

    def __init__(self, seed: int = 5489):
        mt = [seed & 0xFFFFFFFF]
        for i in range(1, self.N):
            prev = mt[-1]
            mt.append((1812433253 * (prev ^ (prev >> 30)) + i) & 0xFFFFFFFF)
        self.mt = np.array(mt, np.uint64)
        self.block = np.zeros(0, np.uint64)
        self.pos = 0

    def _twist(self):
        mt, N, M = self.mt, self.N, self.M

        def step(i_lo, i_hi, src_lo):
            y = (mt[i_lo:i_hi] & self.UPPER) | (mt[i_lo + 1:i_hi + 1] & self.LOWER)
            mag = np.where((y & 1) == 1, np.uint64(self.A), np.uint64(0))
            mt[i_lo:i_hi] = mt[src_lo:src_lo + (i_hi - i_lo)] ^ (y >> np.uint64(1)) ^ mag

        # mt[i] takes mt[i + M] (i < N - M: old values) or mt[i + M - N]
        # (already replaced); chunks of at most N - M keep every source final.
        step(0, N - M, M)
        step(N - M, 2 * (N - M), 0)
        step(2 * (N - M), N - 1, N - M)
        y = (int(mt[N - 1]) & self.UPPER) | (int(mt[0]) & self.LOWER)
        mt[N - 1] = int(mt[M - 1]) ^ (y >> 1) ^ (self.A if y & 1 else 0)
        y = mt.copy()
        y ^= y >> np.uint64(11)
        y ^= (y << np.uint64(7)) & np.uint64(0x9D2C5680)
        y ^= (y << np.uint64(15)) & np.uint64(0xEFC60000)
        y ^= y >> np.uint64(18)
        self.block = (y & np.uint64(0xFFFFFFFF)).tolist()
        self.pos = 0

    def __call__(self) -> int:
        if self.pos >= len(self.block):
            self._twist()
        v = self.block[self.pos]
        self.pos += 1
        return v


def uniform_index(g: MT19937, b: int) -> int:
    """std::uniform_int_distribution<size_t>(0, b)(g) for b + 1 < 2^32."""
    rng = b + 1
    assert rng < (1 << 32)
    product = g() * rng
    low = product & 0xFFFFFFFF
    if low < rng:
        threshold = ((1 << 32) - rng) % rng
        while low < threshold:
            product = g() * rng
            low = product & 0xFFFFFFFF
    return product >> 32


class Reservoir:
    def __init__(self):
        self.samples: List[float] = []
        self.total_seen = 0
        self.rng = MT19937(SEED)


class ActivationObserver:
    """Observe / Percentile / Clear with the reference's semantics."""

    def __init__(self):
        self.sites: Dict[str, Reservoir] = {}

    def observe(self, site: str, values):
        """ActivationObserver::Observe (observer.cpp:8-30)."""
        v = np.abs(np.asarray(values, np.float32).ravel())
        if v.size == 0:
            return
        r = self.sites.setdefault(site, Reservoir())
        i = 0
        while i < v.size and len(r.samples) < RESERVOIR_SIZE:
            r.samples.append(float(v[i]))
            r.total_seen += 1
            i += 1
        vals = v.tolist()
        for i in range(i, v.size):
            j = uniform_index(r.rng, r.total_seen)
            if j < RESERVOIR_SIZE:
                r.samples[j] = vals[i]
            r.total_seen += 1

    def percentile(self, pctile: float) -> Dict[str, float]:
        """ActivationObserver::Percentile (observer.cpp:32-49), float32 index math."""
        out = {}
        for key, r in self.sites.items():
            if not r.samples:
                out[key] = 0.0
                continue
            s = np.sort(np.array(r.samples, np.float32))
            frac = np.float32(pctile) / np.float32(100.0)
            frac = min(max(frac, np.float32(0.0)), np.float32(1.0))
            idx = int(math.floor(np.float32(frac) * np.float32(s.size - 1)))
            out[key] = float(s[min(idx, s.size - 1)])
        return out

    def clear(self):
        self.sites.clear()
