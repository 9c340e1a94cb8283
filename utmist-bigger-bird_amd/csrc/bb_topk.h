// Top-k histogram layout shared by the routes top-k kernels (bb_routes.hip) and the decode-routing pool kernel
// (bb_decode.hip), which fills the histogram while it writes the keys.
#pragma once
#include "bb_common.h"

namespace bb {

constexpr int kTopBins = 2080;        // log-linear bins: 0 for a zero key, then 32 per octave
constexpr int kTopMetaWords = 8;      // uint32 words of one row's TopMeta (cleared before the counts accumulate)
// Float keys (fp32 bits of a positive value in the low 32 bits): bin = (bits >> 18) - kTopFloatBin0 + 1, clamped to
// [1, kTopBins - 1]: 32 bins per octave over [2^-40, 2^25), everything smaller in bin 1, larger in the top bin.
constexpr int kTopFloatBin0 = 87 << 5;

struct TopMeta {
  int32_t bstar, above, need, flags;
  uint32_t nsel, ncand, pad0, pad1;
};
static_assert(sizeof(TopMeta) == 4 * kTopMetaWords, "TopMeta is cleared as kTopMetaWords words");

// Monotone in the key (non-decreasing), so every key above the threshold bin is larger than every key in it.
BB_DEV int top_bin(uint64_t v, bool float_keys) {
  if (!v) return 0;
  if (float_keys) {
    const int b = (int)((uint32_t)v >> 18) - kTopFloatBin0 + 1;
    return b < 1 ? 1 : (b > kTopBins - 1 ? kTopBins - 1 : b);
  }
  const int lz = __clzll((long long)v);
  return 32 * (64 - lz) + (int)((v << lz) >> 58 & 31u);
}

// Order-preserving key of a float: its bits for a positive value, 0 (ranked last) for zero, negatives and NaN.
BB_DEV uint64_t float_key(float x) { return x > 0.0f ? (uint64_t)__float_as_uint(x) : 0ull; }

}  // namespace bb
