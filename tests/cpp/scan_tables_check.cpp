// Property checks of the host work splits on random ragged corpora.
// build_scan_tables (scan_tables.cpp), both partition modes: every token of
// every non-empty document lies in a tile of its own document, exactly one
// tile per document is marked last and ends at the document end, every empty
// document is listed once, tile slots are padded, the wave count is a
// multiple of the workgroup size, and the fused selection's positions (each
// wave's empty documents, then its documents in tile order, from the wave's
// first position) number the documents 0..n-1 once each, with every
// workgroup's first position in the block_pos list after the empty list.  build_score_tables (score_tables.cpp),
// documents or candidate targets (with duplicates): every target's tokens are
// covered by its tiles in order, exactly once, its last tile flagged, an empty
// target gets one empty tile, and every wave ends with a padding entry.
// build_score_units (score_tables.cpp): the same coverage over the units of
// every workgroup's list, each unit whole targets (its last tile ends one),
// tile entries with absolute target indices, every unit but a list's last of
// at least kScoreUnitMinTiles tiles, and every list padded to the returned
// count with empty records at its end.
#include <cstdio>
#include <vector>
#include <cstdint>
#include <random>
#include "internal.hpp"
int main() {
  std::mt19937 rng(1);
  for (int trial = 0; trial < 200; ++trial) {
    int n = 1 + rng() % 300; std::vector<int64_t> off(n + 1, 0);
    for (int d = 0; d < n; ++d) off[d + 1] = off[d] + (rng() % 5 == 0 ? 0 : rng() % 200);
    for (int contiguous = 0; contiguous < 2; ++contiguous) {
      int64_t waves = 1 + rng() % 64;
      std::vector<int64_t> info; std::vector<uint64_t> table; int64_t stride, nw;
      msim::build_scan_tables(off.data(), n, waves, contiguous, info, table, stride, nw);
      std::vector<int> seen_tok(off[n], 0), seen_empty(n, 0), doc_tiles_last(n, 0), pos_of(n, -1), doc_at(n, -1);
      int64_t total_empty = 0;
      for (int64_t w = 0; w < nw; ++w) total_empty += info[w * 8 + 6];
      const int64_t* block_pos = &info[nw * 8 + total_empty];
      if ((int64_t)info.size() != nw * 8 + total_empty + nw / 4 + 1 || block_pos[nw / 4] != n) { printf("BAD block_pos size\n"); return 1; }
      // The kernel reads entries 0 .. max(ntiles + prefetch, 10) of its row.
      if (stride < msim::kScanMinStride || stride % 8 != 0) { printf("BAD stride\n"); return 1; }
      for (int64_t w = 0; w < nw; ++w) {
        const int64_t* r = &info[w * 8];
        if (r[4] + msim::kScanPrefetch + 1 > stride) { printf("BAD stride for w%ld\n", (long)w); return 1; }
        if (w % 4 == 0 && block_pos[w / 4] != r[5]) { printf("BAD block_pos\n"); return 1; }
        int64_t next = r[5];
        auto place = [&](int64_t doc) -> bool {
          if (next < 0 || next >= n || doc_at[next] >= 0 || pos_of[doc] >= 0) return false;
          doc_at[next] = (int)doc; pos_of[doc] = (int)next; ++next; return true;
        };
        for (int64_t e = 0; e < r[6]; ++e) if (!place(info[nw * 8 + r[7] + e])) { printf("BAD empty position\n"); return 1; }
        for (int64_t i = 0; i < r[4]; ++i) {
          uint64_t e = table[w * stride + i];
          if ((e >> 37) & 1) if (!place((int64_t)(e >> 40) + r[0])) { printf("BAD doc position\n"); return 1; }
        }
        if (w + 1 < nw && next != info[(w + 1) * 8 + 5]) { printf("BAD next position\n"); return 1; }
        for (int64_t i = 0; i < r[4]; ++i) {
          uint64_t e = table[w * stride + i]; int64_t start = (int64_t)(e & 0xFFFFFFFFu) + r[2];
          uint32_t hi = (uint32_t)(e >> 32); int rows = (hi & 31) + 1; bool last = (hi >> 5) & 1; int64_t doc = (hi >> 8) + r[0];
          if (doc < 0 || doc >= n || start < off[doc] || start + rows > off[doc + 1]) { printf("BAD tile w%ld\n", (long)w); return 1; }
          for (int t = 0; t < rows; ++t) seen_tok[start + t]++;
          if (last) doc_tiles_last[doc]++;
          if (last != (start + rows == off[doc + 1])) { printf("BAD last\n"); return 1; }
        }
        for (int64_t i = r[4]; i < stride; ++i) if (table[w * stride + i] != msim::kScanPadEntry) { printf("BAD pad\n"); return 1; }
        for (int64_t e = 0; e < r[6]; ++e) seen_empty[info[nw * 8 + r[7] + e]]++;
      }
      for (int d = 0; d < n; ++d) {
        bool empty = off[d + 1] == off[d];
        if (empty ? (seen_empty[d] != 1 || doc_tiles_last[d]) : (doc_tiles_last[d] != 1 || seen_empty[d])) { printf("BAD doc %d\n", d); return 1; }
      }
      for (int64_t t = 0; t < off[n]; ++t) if (seen_tok[t] < 1) { printf("BAD token %ld\n", (long)t); return 1; }
      for (int d = 0; d < n; ++d) if (pos_of[d] < 0) { printf("BAD unplaced doc %d\n", d); return 1; }
      if (nw % 4) { printf("BAD nw\n"); return 1; }
    }
  }
  // build_score_tables
  for (int trial = 0; trial < 200; ++trial) {
    int n = 1 + rng() % 300; std::vector<int64_t> off(n + 1, 0);
    for (int d = 0; d < n; ++d) off[d + 1] = off[d] + (rng() % 5 == 0 ? 0 : rng() % 200);
    std::vector<int64_t> targets;
    const bool cand = trial % 2 == 1;
    const int nt = cand ? 1 + rng() % 200 : n;
    for (int t = 0; t < nt && cand; ++t) targets.push_back(rng() % n);
    std::vector<int64_t> info; std::vector<uint64_t> tiles;
    msim::build_score_tables(off.data(), cand ? targets.data() : nullptr, nt, 1 + rng() % 64, info, tiles);
    std::vector<int64_t> next_tok(nt, -1); std::vector<int> lasts(nt, 0);
    const int64_t nw = (int64_t)info.size() / msim::kScoreInfoWords;
    if (nw % 4) { printf("BAD score nw\n"); return 1; }
    for (int64_t w = 0; w < nw; ++w) {
      const int64_t* r = &info[w * msim::kScoreInfoWords];
      for (int64_t i = 0; i < r[2]; ++i) {
        const uint64_t e = tiles[r[3] + i];
        const int64_t start = (int64_t)(e & msim::kTileStartMask);
        const int rows = (int)((e >> msim::kTileRowsShift) & 15) + 1;
        const bool last = (e >> msim::kTileLastShift) & 1, empty = (e >> msim::kTileEmptyShift) & 1;
        const int64_t t = r[0] + (int64_t)(e >> msim::kTileLocalShift);
        if (t < 0 || t >= nt) { printf("BAD score target\n"); return 1; }
        const int64_t d = cand ? targets[t] : t;
        if (empty) {
          if (off[d + 1] != off[d] || !last) { printf("BAD score empty\n"); return 1; }
        } else {
          const int64_t expect = next_tok[t] < 0 ? off[d] : next_tok[t];
          if (start != expect || start + rows > off[d + 1]) { printf("BAD score tile\n"); return 1; }
          next_tok[t] = start + rows;
          if (last != (start + rows == off[d + 1])) { printf("BAD score last\n"); return 1; }
        }
        lasts[t] += last ? 1 : 0;
      }
      const uint64_t pad = tiles[r[3] + r[2]];
      if ((pad & msim::kTileStartMask) != 0 || ((pad >> msim::kTileLastShift) & 1)) { printf("BAD score pad\n"); return 1; }
    }
    for (int t = 0; t < nt; ++t) {
      const int64_t d = cand ? targets[t] : t;
      if (lasts[t] != 1) { printf("BAD score lasts %d\n", t); return 1; }
      if (off[d + 1] != off[d] && next_tok[t] != off[d + 1]) { printf("BAD score cover\n"); return 1; }
    }
  }
  // build_score_units
  for (int trial = 0; trial < 200; ++trial) {
    int n = 1 + rng() % 3000; std::vector<int64_t> off(n + 1, 0);
    for (int d = 0; d < n; ++d) off[d + 1] = off[d] + (rng() % 5 == 0 ? 0 : rng() % (trial % 2 ? 40 : 200));
    std::vector<int64_t> targets;
    const bool cand = trial % 3 == 2;
    const int nt = cand ? 1 + rng() % 500 : n;
    for (int t = 0; t < nt && cand; ++t) targets.push_back(rng() % n);
    const int64_t wgs = 1 + rng() % 300;
    std::vector<int64_t> info; std::vector<uint64_t> tiles;
    const int64_t U = msim::build_score_units(off.data(), cand ? targets.data() : nullptr, nt, wgs, info, tiles);
    const int64_t G = std::min<int64_t>(wgs, nt);
    if (U < 1 || (int64_t)info.size() != G * U * msim::kScoreInfoWords) { printf("BAD units size\n"); return 1; }
    std::vector<int64_t> next_tok(nt, -1); std::vector<int> lasts(nt, 0);
    for (int64_t g = 0; g < G; ++g) {
      bool ended = false;
      for (int64_t k = 0; k < U; ++k) {
        const int64_t* r = &info[(g * U + k) * msim::kScoreInfoWords];
        if (r[2] == 0) { ended = true; continue; }
        const bool last_unit = k + 1 == U || info[(g * U + k + 1) * msim::kScoreInfoWords + 2] == 0;
        if (ended || r[0] != 0 || (!last_unit && r[2] < msim::kScoreUnitMinTiles)) { printf("BAD unit\n"); return 1; }
        int64_t ends = 0;
        for (int64_t i = 0; i < r[2]; ++i) {
          const uint64_t e = tiles[r[3] + i];
          const int64_t start = (int64_t)(e & msim::kTileStartMask);
          const int rows = (int)((e >> msim::kTileRowsShift) & 15) + 1;
          const bool last = (e >> msim::kTileLastShift) & 1, empty = (e >> msim::kTileEmptyShift) & 1;
          const int64_t t = (int64_t)(e >> msim::kTileLocalShift);
          if (t < 0 || t >= nt) { printf("BAD unit target\n"); return 1; }
          const int64_t d = cand ? targets[t] : t;
          if (empty) {
            if (off[d + 1] != off[d] || !last) { printf("BAD unit empty\n"); return 1; }
          } else {
            const int64_t expect = next_tok[t] < 0 ? off[d] : next_tok[t];
            if (start != expect || start + rows > off[d + 1]) { printf("BAD unit tile\n"); return 1; }
            next_tok[t] = start + rows;
            if (last != (start + rows == off[d + 1])) { printf("BAD unit last\n"); return 1; }
          }
          lasts[t] += last ? 1 : 0;
          ends += last ? 1 : 0;
          if (i + 1 == r[2] && !last) { printf("BAD unit splits a target\n"); return 1; }
        }
        if (ends != r[1]) { printf("BAD unit count\n"); return 1; }
      }
    }
    for (int t = 0; t < nt; ++t) {
      const int64_t d = cand ? targets[t] : t;
      if (lasts[t] != 1 || (off[d + 1] != off[d] && next_tok[t] != off[d + 1])) { printf("BAD unit cover %d\n", t); return 1; }
    }
  }
  printf("ok\n");
}
