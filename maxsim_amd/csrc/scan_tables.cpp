// scan_tables.cpp -- host-side work split of the int8q scan kernel: contiguous
// document ranges per wave, balanced by cost ceil(len / 16) + 1 (16-token
// tiles plus the per-document finish), and the per-wave table of non-empty
// document ends that the kernel walks.
#include <algorithm>

#include "internal.hpp"

namespace msim {

void build_scan_tables(const int64_t* off, int64_t n, int64_t waves, std::vector<int64_t>& info,
                       std::vector<uint64_t>& table, std::vector<uint32_t>& ring) {
  info.clear();
  table.clear();
  ring.clear();
  if (n <= 0) return;
  waves = std::max<int64_t>(1, waves);
  constexpr int64_t kMaxWaveTokens = int64_t(1) << 25;  // (T1 - T0) * 64 stays below 2^31
  std::vector<int64_t> cost(n + 1, 0);
  for (int64_t d = 0; d < n; ++d) cost[d + 1] = cost[d] + (off[d + 1] - off[d] + 15) / 16 + 1;
  auto emit = [&](int64_t d0, int64_t d1) {
    const int64_t T0 = off[d0];
    int64_t tiles = 0, n_ne = 0, first_end = 0;
    bool has_empty = false;
    const int64_t tab0 = (int64_t)table.size();
    for (int64_t d = d0; d < d1; ++d) {
      const int64_t len = off[d + 1] - off[d];
      if (len == 0) {
        has_empty = true;
        continue;
      }
      const uint64_t end_rel = (uint64_t)(off[d + 1] - T0);
      if (n_ne == 0) first_end = (int64_t)end_rel;
      table.push_back(end_rel | ((uint64_t)(d - d0) << 32));
      ++n_ne;
      tiles += (len + 15) / 16;
    }
    const int64_t row[kWaveInfoWords] = {d0, d1 - d0, T0, off[d1], tiles, n_ne, tab0,
                                         first_end | (has_empty ? (int64_t(1) << 32) : 0)};
    info.insert(info.end(), row, row + kWaveInfoWords);
    // The kernel's load cursor over the first kScanPrefetch tiles (the same
    // steps as its issue()).
    int64_t k = 0;
    uint32_t t = n_ne > 0 ? 0u : kScanPastEnd, e = (uint32_t)first_end;
    for (int s = 0; s < kScanPrefetch; ++s) {
      ring.push_back(t);
      if (t == kScanPastEnd) continue;
      const uint32_t nt = t + 16u;
      if (nt >= e) {
        ++k;
        if (k < n_ne) {
          t = e;
          e = (uint32_t)table[tab0 + k];
        } else {
          t = kScanPastEnd;
        }
      } else {
        t = nt + 16u <= e ? nt : e - 16u;
      }
    }
    ring.push_back((uint32_t)k);
    ring.push_back(t);
    ring.push_back(e);
  };
  int64_t d0 = 0;
  for (int64_t w = 1; w <= waves && d0 < n; ++w) {
    int64_t d1 = w == waves ? n : std::lower_bound(cost.begin(), cost.end(), (cost[n] * w) / waves) - cost.begin();
    d1 = std::min(d1, n);
    while (d0 < d1) {
      // At most kScanMaxDocsPerWave documents, and a token span that keeps
      // the kernel's 32-bit byte offsets in range (a longer single document
      // still gets a wave of its own).
      int64_t e = std::min(d1, d0 + kScanMaxDocsPerWave);
      while (e > d0 + 1 && off[e] - off[d0] > kMaxWaveTokens) --e;
      emit(d0, e);
      d0 = e;
    }
  }
}

}  // namespace msim
