// score_tables.cpp -- host-side work split of the generalized scoring kernel
// (score.hip): which targets each wave scores, and one table entry per
// 16-token tile (the last tile of a target holds its remaining 1..16 tokens;
// an empty target gets one empty tile).  A target costs its tiles + 1; targets
// go to waves longest first, each onto the least-loaded wave (LPT), as in
// scan_tables.cpp, with absolute target indices; more than 2^24 targets fall
// back to contiguous cost-balanced ranges.
#include <algorithm>
#include <queue>

#include "internal.hpp"

namespace msim {

namespace {
constexpr int64_t kMaxLocal = int64_t(1) << 24;  // target index bits of a tile entry
}  // namespace

void build_score_tables(const int64_t* off, const int64_t* targets, int64_t n, int64_t waves,
                        std::vector<int64_t>& info, std::vector<uint64_t>& tiles) {
  info.clear();
  tiles.clear();
  waves = std::max<int64_t>(1, std::min(waves, std::max<int64_t>(1, n)));
  auto doc_of = [&](int64_t t) { return targets ? targets[t] : t; };
  auto cost_of = [&](int64_t t) {
    const int64_t d = doc_of(t);
    return std::max<int64_t>(1, (off[d + 1] - off[d] + 15) / 16) + 1;
  };
  // Tiles of target t (index `local` relative to the wave's base).
  auto emit_target = [&](int64_t t, int64_t local) {
    const int64_t d = doc_of(t);
    const int64_t s = off[d], e = off[d + 1];
    if (s == e) {
      tiles.push_back(score_tile_entry(0, 1, true, true, local));
      return;
    }
    for (int64_t x = s; x < e; x += 16)
      tiles.push_back(score_tile_entry(x, std::min<int64_t>(16, e - x), x + 16 >= e, false, local));
  };
  auto close_wave = [&](int64_t base, int64_t count, int64_t tab0) {
    const int64_t ntiles = (int64_t)tiles.size() - tab0;
    tiles.push_back(score_tile_entry(0, 1, false, false, 0));
    const int64_t row[kScoreInfoWords] = {base, count, ntiles, tab0};
    info.insert(info.end(), row, row + kScoreInfoWords);
  };
  if (n < kMaxLocal) {
    std::vector<int64_t> order((size_t)n);
    for (int64_t t = 0; t < n; ++t) order[(size_t)t] = t;
    std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return cost_of(a) > cost_of(b); });
    using Load = std::pair<int64_t, int64_t>;  // (cost so far, wave)
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int64_t w = 0; w < waves; ++w) heap.push({0, w});
    std::vector<std::vector<int64_t>> mine((size_t)waves);
    for (int64_t t : order) {
      Load l = heap.top();
      heap.pop();
      mine[(size_t)l.second].push_back(t);
      heap.push({l.first + cost_of(t), l.second});
    }
    for (auto& ts : mine) {
      std::sort(ts.begin(), ts.end());
      const int64_t tab0 = (int64_t)tiles.size();
      for (int64_t t : ts) emit_target(t, t);
      close_wave(0, (int64_t)ts.size(), tab0);
    }
  } else {
    std::vector<int64_t> cost(n + 1, 0);
    for (int64_t t = 0; t < n; ++t) cost[t + 1] = cost[t] + cost_of(t);
    int64_t t0 = 0;
    for (int64_t w = 1; w <= waves && t0 < n; ++w) {
      int64_t t1 = w == waves ? n : std::lower_bound(cost.begin(), cost.end(), (cost[n] * w) / waves) - cost.begin();
      t1 = std::min(t1, n);
      while (t0 < t1) {
        const int64_t e = std::min(t1, t0 + kMaxLocal - 1);
        const int64_t tab0 = (int64_t)tiles.size();
        for (int64_t t = t0; t < e; ++t) emit_target(t, t - t0);
        close_wave(t0, e - t0, tab0);
        t0 = e;
      }
    }
  }
  while ((info.size() / kScoreInfoWords) % kScanWavesPerGroup != 0 || info.empty()) {
    const int64_t tab0 = (int64_t)tiles.size();
    close_wave(n, 0, tab0);
  }
}

int64_t build_score_units(const int64_t* off, const int64_t* targets, int64_t n, int64_t workgroups,
                          std::vector<int64_t>& info, std::vector<uint64_t>& tiles) {
  info.clear();
  tiles.clear();
  workgroups = std::max<int64_t>(1, std::min(workgroups, std::max<int64_t>(1, n)));
  auto doc_of = [&](int64_t t) { return targets ? targets[t] : t; };
  auto tiles_of = [&](int64_t t) {
    const int64_t d = doc_of(t);
    return std::max<int64_t>(1, (off[d + 1] - off[d] + 15) / 16);
  };
  std::vector<int64_t> order((size_t)n);
  for (int64_t t = 0; t < n; ++t) order[(size_t)t] = t;
  std::stable_sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return tiles_of(a) > tiles_of(b); });
  using Load = std::pair<int64_t, int64_t>;  // (cost so far, list)
  std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
  for (int64_t w = 0; w < workgroups; ++w) heap.push({0, w});
  std::vector<std::vector<int64_t>> mine((size_t)workgroups);  // each longest first
  for (int64_t t : order) {
    Load l = heap.top();
    heap.pop();
    mine[(size_t)l.second].push_back(t);
    heap.push({l.first + tiles_of(t) + 1, l.second});
  }
  std::vector<std::vector<int64_t>> units((size_t)workgroups);  // records, kScoreInfoWords each
  int64_t most = 1;
  for (int64_t w = 0; w < workgroups; ++w) {
    auto& rec = units[(size_t)w];
    int64_t tab0 = (int64_t)tiles.size(), count = 0;
    auto close = [&]() {
      const int64_t row[kScoreInfoWords] = {0, count, (int64_t)tiles.size() - tab0, tab0};
      rec.insert(rec.end(), row, row + kScoreInfoWords);
      tab0 = (int64_t)tiles.size();
      count = 0;
    };
    for (int64_t t : mine[(size_t)w]) {
      const int64_t d = doc_of(t);
      const int64_t s = off[d], e = off[d + 1];
      if (s == e) tiles.push_back(score_tile_entry(0, 1, true, true, t));
      for (int64_t x = s; x < e; x += 16)
        tiles.push_back(score_tile_entry(x, std::min<int64_t>(16, e - x), x + 16 >= e, false, t));
      ++count;
      if ((int64_t)tiles.size() - tab0 >= kScoreUnitMinTiles) close();
    }
    if (count > 0) close();
    most = std::max<int64_t>(most, (int64_t)rec.size() / kScoreInfoWords);
  }
  for (auto& rec : units) {
    while ((int64_t)rec.size() / kScoreInfoWords < most) {
      const int64_t pad[kScoreInfoWords] = {0, 0, 0, 0};
      rec.insert(rec.end(), pad, pad + kScoreInfoWords);
    }
    info.insert(info.end(), rec.begin(), rec.end());
  }
  if (tiles.empty()) tiles.push_back(score_tile_entry(0, 1, false, false, 0));
  return most;
}

}  // namespace msim
