// scan_tables.cpp -- host-side work split of the int8q scan kernel: which
// documents each wave scores, and the per-tile entries the kernel walks
// (tile start, valid rows, document end flag, document index).
//
// A document costs ceil(len / 16) + 1 (its 16-token tiles plus the finish).
// Documents go to waves longest first, each to the least-loaded wave (LPT),
// so that the slowest wave -- the kernel's duration -- carries about the
// mean cost: with a few documents per wave, contiguous ranges cut at
// document boundaries leave waves up to a whole document above the mean.
// Corpora too large for the kernel's 32-bit byte offsets over the whole
// token range fall back to contiguous ranges (each with its own base).
#include <algorithm>
#include <queue>

#include "internal.hpp"

namespace msim {

namespace {

constexpr int64_t kMaxWaveTokens = int64_t(1) << 25;  // token span * 64 stays below 2^31
constexpr int64_t kMaxLocalDoc = int64_t(1) << 24;    // document index bits of a tile entry

int64_t doc_cost(const int64_t* off, int64_t d) { return (off[d + 1] - off[d] + 15) / 16 + 1; }

// Tiles of document d (tokens [s, e) relative to the wave base, local index
// `local`): at s, s + 16, ...; the last one ends at e (or holds the whole
// document when it is shorter than 16 tokens).
void emit_doc_tiles(int64_t s, int64_t e, int64_t local, std::vector<uint64_t>& tiles) {
  for (int64_t t = s;; t += 16) {
    const bool last = t + 16 >= e;
    const int64_t start = last ? std::max(s, e - 16) : t;
    const uint64_t rows = (uint64_t)std::min<int64_t>(16, e - start);
    const uint64_t hi = (rows - 1) | ((uint64_t)last << 5) | ((uint64_t)local << 8);
    tiles.push_back((uint64_t)start | (hi << 32));
    if (last) break;
  }
}

}  // namespace

void build_scan_tables(const int64_t* off, int64_t n, int64_t waves, bool contiguous, std::vector<int64_t>& info,
                       std::vector<uint64_t>& table, int64_t& stride, int64_t& num_waves) {
  info.clear();
  table.clear();
  stride = 0;
  num_waves = 0;
  if (n <= 0) return;
  waves = std::max<int64_t>(1, waves);
  std::vector<uint64_t> tiles;
  std::vector<int64_t> empties;
  // Per wave: d0, ndocs, T0, T1, ntiles, tab0 (into `tiles`, replaced by the
  // first position below), nempty, first empty; called after the wave's
  // tiles, before its padding entries.  `all_docs` counts the wave's empty
  // documents too (the positions it takes).
  std::vector<int64_t> wave_docs;
  auto add_wave = [&](int64_t d0, int64_t ndocs, int64_t T0, int64_t T1, int64_t tab0, int64_t e0, int64_t all_docs) {
    const int64_t ntiles = (int64_t)tiles.size() - tab0;
    const int64_t row[kWaveInfoWords] = {d0, ndocs, T0, T1, ntiles, tab0, (int64_t)empties.size() - e0, e0};
    info.insert(info.end(), row, row + kWaveInfoWords);
    wave_docs.push_back(all_docs);
  };

  const int64_t T = off[n];
  if (!contiguous && T < kMaxWaveTokens && n < kMaxLocalDoc) {
    // LPT over the whole corpus: absolute token starts and document ids
    // (every wave's base is token 0, document 0).
    waves = std::min(waves, n);
    // With more than one workgroup, the first one gets no documents: in a
    // fused launch it selects the top-k, and its polling would otherwise
    // slow its own scan work and that of the workgroup sharing its CU.
    const int64_t first = waves > kScanWavesPerGroup ? kScanWavesPerGroup : 0;
    std::vector<int64_t> order;
    order.reserve((size_t)n);
    for (int64_t d = 0; d < n; ++d)
      if (off[d + 1] > off[d]) order.push_back(d);
    std::stable_sort(order.begin(), order.end(),
                     [&](int64_t a, int64_t b) { return doc_cost(off, a) > doc_cost(off, b); });
    using Load = std::pair<int64_t, int64_t>;  // (cost so far, wave)
    std::priority_queue<Load, std::vector<Load>, std::greater<Load>> heap;
    for (int64_t w = first; w < waves; ++w) heap.push({0, w});
    std::vector<std::vector<int64_t>> docs((size_t)waves), empty_docs((size_t)waves);
    for (int64_t d : order) {
      Load l = heap.top();
      heap.pop();
      docs[(size_t)l.second].push_back(d);
      heap.push({l.first + doc_cost(off, d), l.second});
    }
    for (int64_t d = 0, w = 0; d < n; ++d)
      if (off[d + 1] == off[d]) empty_docs[(size_t)(first + w++ % (waves - first))].push_back(d);
    for (int64_t w = 0; w < waves; ++w) {
      auto& ds = docs[(size_t)w];
      std::sort(ds.begin(), ds.end());  // ascending tokens within the wave
      const int64_t tab0 = (int64_t)tiles.size(), e0 = (int64_t)empties.size();
      for (int64_t d : ds) emit_doc_tiles(off[d], off[d + 1], d, tiles);
      empties.insert(empties.end(), empty_docs[(size_t)w].begin(), empty_docs[(size_t)w].end());
      add_wave(0, (int64_t)ds.size(), 0, T, tab0, e0, (int64_t)(ds.size() + empty_docs[(size_t)w].size()));
      for (int k = 0; k <= kScanPrefetch; ++k) tiles.push_back(kScanPadEntry);
    }
  } else {
    // Contiguous ranges balanced by cost, at most kScanMaxDocsPerWave
    // documents and kMaxWaveTokens tokens each (a longer single document
    // still gets a wave of its own).
    std::vector<int64_t> cost(n + 1, 0);
    for (int64_t d = 0; d < n; ++d) cost[d + 1] = cost[d] + doc_cost(off, d);
    int64_t d0 = 0;
    for (int64_t w = 1; w <= waves && d0 < n; ++w) {
      int64_t d1 = w == waves ? n : std::lower_bound(cost.begin(), cost.end(), (cost[n] * w) / waves) - cost.begin();
      d1 = std::min(d1, n);
      while (d0 < d1) {
        int64_t e = std::min(d1, d0 + kScanMaxDocsPerWave);
        while (e > d0 + 1 && off[e] - off[d0] > kMaxWaveTokens) --e;
        const int64_t T0 = off[d0], tab0 = (int64_t)tiles.size(), e0 = (int64_t)empties.size();
        for (int64_t d = d0; d < e; ++d) {
          if (off[d + 1] == off[d]) empties.push_back(d);
          else emit_doc_tiles(off[d] - T0, off[d + 1] - T0, d - d0, tiles);
        }
        add_wave(d0, e - d0, T0, off[e], tab0, e0, e - d0);
        for (int k = 0; k <= kScanPrefetch; ++k) tiles.push_back(kScanPadEntry);
        d0 = e;
      }
    }
  }
  // Padding waves (no documents, no tiles) up to whole workgroups.
  while ((info.size() / kWaveInfoWords) % kScanWavesPerGroup != 0) {
    const int64_t tab0 = (int64_t)tiles.size(), e0 = (int64_t)empties.size();
    add_wave(n, 0, T, T, tab0, e0, 0);
    for (int k = 0; k <= kScanPrefetch; ++k) tiles.push_back(kScanPadEntry);
  }
  // Every wave's entries at a fixed stride (a multiple of 8 entries, 64 B),
  // so a wave finds them from its index alone, without reading its row of
  // `info` first; the rest of a slot is padding.  At least kScanMinStride
  // entries: a wave reads its first 11 entries while it fills its ring,
  // whatever its tile count.
  num_waves = (int64_t)info.size() / kWaveInfoWords;
  int64_t longest = 0;
  for (int64_t w = 0; w < num_waves; ++w) longest = std::max<int64_t>(longest, info[w * kWaveInfoWords + 4]);
  stride = std::max<int64_t>(kScanMinStride, ((longest + kScanPrefetch + 1 + 7) / 8) * 8);
  table.assign((size_t)(num_waves * stride), kScanPadEntry);
  // Positions in wave order: wave w's documents take [pos0, pos0 + all_docs).
  std::vector<int64_t> block_pos;
  int64_t pos = 0;
  for (int64_t w = 0; w < num_waves; ++w) {
    int64_t* row = &info[w * kWaveInfoWords];
    const int64_t cnt = row[4];
    std::copy(tiles.begin() + row[5], tiles.begin() + row[5] + cnt, table.begin() + w * stride);
    if (w % kScanWavesPerGroup == 0) block_pos.push_back(pos);
    row[5] = pos;
    pos += wave_docs[(size_t)w];
  }
  block_pos.push_back(pos);  // == n
  // The empty-document list, then the workgroup start positions, follow the
  // wave rows.
  info.insert(info.end(), empties.begin(), empties.end());
  info.insert(info.end(), block_pos.begin(), block_pos.end());
}

}  // namespace msim
