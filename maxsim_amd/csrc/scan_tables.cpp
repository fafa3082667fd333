// scan_tables.cpp -- host-side work split of the int8q scan kernel: contiguous
// document ranges per wave, balanced by cost ceil(len / 16) + 1 (16-token
// tiles plus the per-document finish), and the per-tile entries the kernel
// walks (tile start, valid rows, document end flag, document index).
#include <algorithm>

#include "internal.hpp"

namespace msim {

void build_scan_tables(const int64_t* off, int64_t n, int64_t waves, std::vector<int64_t>& info,
                       std::vector<uint64_t>& table, int64_t& stride) {
  info.clear();
  table.clear();
  stride = 0;
  if (n <= 0) return;
  std::vector<uint64_t> tiles;
  waves = std::max<int64_t>(1, waves);
  constexpr int64_t kMaxWaveTokens = int64_t(1) << 25;  // (T1 - T0) * 64 stays below 2^31
  std::vector<int64_t> cost(n + 1, 0);
  for (int64_t d = 0; d < n; ++d) cost[d + 1] = cost[d] + (off[d + 1] - off[d] + 15) / 16 + 1;
  auto emit = [&](int64_t d0, int64_t d1) {
    const int64_t T0 = off[d0];
    const int64_t tab0 = (int64_t)tiles.size();
    bool has_empty = false;
    for (int64_t d = d0; d < d1; ++d) {
      const int64_t s = off[d] - T0, e = off[d + 1] - T0;
      if (e == s) {
        has_empty = true;
        continue;
      }
      // Tiles at s, s + 16, ...; the last one ends at e (or holds the whole
      // document when it is shorter than 16 tokens).
      for (int64_t t = s;; t += 16) {
        const bool last = t + 16 >= e;
        const int64_t start = last ? std::max(s, e - 16) : t;
        const uint64_t rows = (uint64_t)std::min<int64_t>(16, e - start);
        const uint64_t hi = (rows - 1) | ((uint64_t)last << 5) | ((uint64_t)(d - d0) << 8);
        tiles.push_back((uint64_t)start | (hi << 32));
        if (last) break;
      }
    }
    const int64_t ntiles = (int64_t)tiles.size() - tab0;
    for (int k = 0; k <= kScanPrefetch; ++k) tiles.push_back(kScanPastEnd);
    const int64_t row[kWaveInfoWords] = {d0, d1 - d0, T0, off[d1], ntiles, tab0, has_empty ? 1 : 0, 0};
    info.insert(info.end(), row, row + kWaveInfoWords);
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
  // Padding waves (no documents, no tiles) up to whole workgroups.
  while ((info.size() / kWaveInfoWords) % kScanWavesPerGroup != 0) {
    const int64_t tab0 = (int64_t)tiles.size();
    for (int k = 0; k <= kScanPrefetch; ++k) tiles.push_back(kScanPastEnd);
    const int64_t row[kWaveInfoWords] = {n, 0, off[n], off[n], 0, tab0, 0, 0};
    info.insert(info.end(), row, row + kWaveInfoWords);
  }
  // Every wave's entries at a fixed stride (a multiple of 8 entries, 64 B),
  // so a wave finds them from its index alone, without reading its row of
  // `info` first; the rest of a slot is padding.
  const int64_t nw = (int64_t)info.size() / kWaveInfoWords;
  int64_t longest = 0;
  for (int64_t w = 0; w < nw; ++w) longest = std::max<int64_t>(longest, info[w * kWaveInfoWords + 4]);
  stride = ((longest + kScanPrefetch + 1 + 7) / 8) * 8;
  table.assign((size_t)(nw * stride), kScanPastEnd);
  for (int64_t w = 0; w < nw; ++w) {
    int64_t* row = &info[w * kWaveInfoWords];
    const int64_t cnt = row[4];
    std::copy(tiles.begin() + row[5], tiles.begin() + row[5] + cnt, table.begin() + w * stride);
    row[5] = w * stride;
  }
}

}  // namespace msim
