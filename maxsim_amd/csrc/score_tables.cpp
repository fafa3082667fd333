// score_tables.cpp -- host-side work split of the generalized scoring kernel
// (score.hip): contiguous target ranges per wave, balanced by tiles + 1 per
// target, and one table entry per 16-token tile (the last tile of a target
// holds its remaining 1..16 tokens; an empty target gets one empty tile).
#include <algorithm>

#include "internal.hpp"

namespace msim {

namespace {
constexpr int64_t kMaxLocal = 0xFFFF;  // 16-bit relative target index
uint64_t tile_entry(int64_t start, int64_t rows, bool last, bool empty, int64_t local) {
  return (uint64_t)start | ((uint64_t)(rows - 1) << 40) | ((uint64_t)last << 45) | ((uint64_t)empty << 46) |
         ((uint64_t)local << 48);
}
}  // namespace

void build_score_tables(const int64_t* off, const int64_t* targets, int64_t n, int64_t waves,
                        std::vector<int64_t>& info, std::vector<uint64_t>& tiles) {
  info.clear();
  tiles.clear();
  waves = std::max<int64_t>(1, std::min(waves, std::max<int64_t>(1, n)));
  auto doc_of = [&](int64_t t) { return targets ? targets[t] : t; };
  std::vector<int64_t> cost(n + 1, 0);
  for (int64_t t = 0; t < n; ++t) {
    const int64_t d = doc_of(t);
    const int64_t len = off[d + 1] - off[d];
    cost[t + 1] = cost[t] + std::max<int64_t>(1, (len + 15) / 16) + 1;
  }
  auto emit = [&](int64_t t0, int64_t t1) {
    const int64_t tab0 = (int64_t)tiles.size();
    for (int64_t t = t0; t < t1; ++t) {
      const int64_t d = doc_of(t);
      const int64_t s = off[d], e = off[d + 1];
      if (s == e) {
        tiles.push_back(tile_entry(0, 1, true, true, t - t0));
        continue;
      }
      for (int64_t x = s; x < e; x += 16) {
        const bool last = x + 16 >= e;
        tiles.push_back(tile_entry(x, std::min<int64_t>(16, e - x), last, false, t - t0));
      }
    }
    const int64_t ntiles = (int64_t)tiles.size() - tab0;
    tiles.push_back(tile_entry(0, 1, false, false, 0));
    const int64_t row[kScoreInfoWords] = {t0, t1 - t0, ntiles, tab0};
    info.insert(info.end(), row, row + kScoreInfoWords);
  };
  int64_t t0 = 0;
  for (int64_t w = 1; w <= waves && t0 < n; ++w) {
    int64_t t1 = w == waves ? n : std::lower_bound(cost.begin(), cost.end(), (cost[n] * w) / waves) - cost.begin();
    t1 = std::min(t1, n);
    while (t0 < t1) {
      const int64_t e = std::min(t1, t0 + kMaxLocal);
      emit(t0, e);
      t0 = e;
    }
  }
  while ((info.size() / kScoreInfoWords) % kScanWavesPerGroup != 0 || info.empty()) {
    const int64_t tab0 = (int64_t)tiles.size();
    tiles.push_back(tile_entry(0, 1, false, false, 0));
    const int64_t row[kScoreInfoWords] = {n, 0, 0, tab0};
    info.insert(info.end(), row, row + kScoreInfoWords);
  }
}

}  // namespace msim
