// Property check of the decode work planner (orionserve-rs_amd/csrc/
// decode_plan.cpp), host only.  For random batches (rows, contexts, block
// sizes, KV heads, wave slots, skipped rows) every plan must:
//   * cover each planned (row, KV head) context [0, position] exactly once,
//     and plan nothing for a skipped row;
//   * give each piece a 16-token-aligned start, at most 64 table entries, the
//     table offset of its first block, and split indices 0 .. n-1 of the
//     row's n = row_nsplit pieces, with n <= max_splits;
//   * cut every row into pieces of one length, the last piece no longer;
//   * when balanced, fit in at most four rounds of wave slots;
//   * flag exactly the items whose blocks another planned row (or the same
//     row twice) also attends, and choose streaming / mixed loads to match.
// Prints one line per failure and a summary; exit status 1 on any failure.
#include "kernels.hpp"

#include <algorithm>
#include <cstdio>
#include <map>
#include <random>
#include <vector>

using orion::DecodePlanHost;
using orion::DecodeWork;

int main(int argc, char** argv) {
  const int trials = argc > 1 ? atoi(argv[1]) : 2000;
  std::mt19937 rng(20261202);
  int fails = 0, balanced = 0;
  long packed_items = 0;
  auto fail = [&](int trial, const char* what, int row) {
    if (fails++ < 20) printf("trial %d: %s (row %d)\n", trial, what, row);
  };
  for (int trial = 0; trial < trials; ++trial) {
    const int rows = 1 + rng() % 200;
    const int bs = 1 << (rng() % 9);  // 1 .. 256
    const int hkv = 1 + rng() % 8;
    const int64_t slots = (trial % 3 == 0) ? 2048 : (64 + rng() % 4000);
    const int maxctx = (trial % 4 == 0) ? 16384 : (trial % 4 == 1 ? 64 : 4096);
    std::vector<uint32_t> pos(rows);
    std::vector<int32_t> row_seq(rows);
    std::vector<int64_t> off(rows + 1, 0);
    std::vector<uint32_t> ids;
    // every seventh trial: rows start with the leading blocks of row 0 (a
    // shared prefix, as prefix caching produces)
    // (every third trial of those: deep prefixes of up to 64 blocks, which
    // the packing planner groups)
    const bool prefix = trial % 7 == 3 || trial % 11 == 5;
    const int64_t share = trial % 11 == 5 ? 1 + rng() % 64 : 8;
    for (int r = 0; r < rows; ++r) {
      pos[r] = rng() % maxctx;
      row_seq[r] = r;
      const int nb = (int)pos[r] / bs + 1;
      for (int j = 0; j < nb; ++j)
        ids.push_back(prefix && r > 0 && j < std::min<int64_t>(share, off[1]) ? ids[j]
                                                                              : rng() % 100000);
      off[r + 1] = off[r] + nb;
    }
    const int G = 1 + rng() % 8;
    const int pack_r = (trial % 2) ? 16 / G : 0;
    std::vector<uint8_t> skip(rows, 0);
    const bool use_skip = trial % 5 == 0;
    if (use_skip)
      for (int r = 0; r < rows; ++r) skip[r] = rng() % 3 == 0;
    DecodePlanHost plan;
    orion::build_decode_plan(pos.data(), row_seq.data(), off.data(), ids.data(), rows, hkv, bs,
                             slots, use_skip ? skip.data() : nullptr, &plan, pack_r);
    balanced += plan.balanced;
    packed_items += plan.num_packed;
    int bs_log2 = 0;
    while ((1 << bs_log2) < bs) ++bs_log2;
    std::map<int, std::vector<std::pair<int, int>>> cover;  // item -> [start, end)
    std::map<std::pair<int, int>, int> seen_split;
    std::vector<int> in_pack(rows, 0);
    int counted_packed = 0;
    for (const DecodeWork& w : plan.work) {
      const int nblk = ((w.end - 1) >> bs_log2) - (w.start >> bs_log2) + 1;
      if (w.shared == 2) {  // packed: one piece of every row of the pack
        ++counted_packed;
        const int pk = w.item / hkv, h = w.item % hkv;
        if (pack_r < 2 || pk < 0 || (size_t)(pk + 1) * pack_r > plan.pack_rows.size()) {
          fail(trial, "packed item without a pack", pk);
          continue;
        }
        if (w.start % 16 || w.end <= w.start || nblk > 64) fail(trial, "bad packed bounds", pk);
        if (w.nsplit < 2) fail(trial, "packed item finishes in place", pk);
        int members = 0;
        for (int j = 0; j < pack_r; ++j) {
          const int r = plan.pack_rows[pk * pack_r + j];
          if (r < 0) continue;
          ++members;
          in_pack[r] = 1;
          if ((int)w.end > (int)pos[r]) fail(trial, "packed piece reaches a row's position", r);
          for (int b = 0; b < nblk; ++b)
            if (ids[w.tbl_off + b] != ids[off[r] + (w.start >> bs_log2) + b])
              fail(trial, "packed row does not share the piece's blocks", r);
          if (w.split < 0 || w.split >= plan.row_nsplit[r]) fail(trial, "bad packed split", r);
          if (seen_split[{r * hkv + h, w.split}]++) fail(trial, "split index repeated", r);
          cover[r * hkv + h].push_back({w.start, w.end});
        }
        if (members < 2) fail(trial, "pack of fewer than two rows", pk);
        if ((uint32_t)w.blk0 != ids[w.tbl_off]) fail(trial, "bad packed blk0", pk);
        continue;
      }
      const int row = w.item / hkv;
      if (row < 0 || row >= rows) {
        fail(trial, "row out of range", row);
        continue;
      }
      if (w.start % 16 || w.end <= w.start || nblk > 64) fail(trial, "bad piece bounds", row);
      if (w.tbl_off != off[row] + (w.start >> bs_log2) || (uint32_t)w.blk0 != ids[w.tbl_off])
        fail(trial, "bad table slice", row);
      if (w.nsplit != plan.row_nsplit[row] || w.split < 0 || w.split >= w.nsplit ||
          w.nsplit > plan.max_splits)
        fail(trial, "bad split index", row);
      if (seen_split[{w.item, w.split}]++) fail(trial, "split index repeated", row);
      cover[w.item].push_back({w.start, w.end});
    }
    if (counted_packed != plan.num_packed) fail(trial, "num_packed", counted_packed);
    if (pack_r < 2 && plan.num_packed) fail(trial, "packed without pack_r", -1);
    for (int r = 0; r < rows; ++r) {
      const bool planned = !(use_skip && skip[r]);
      if (!planned && plan.row_nsplit[r] != 0) fail(trial, "skipped row has pieces", r);
      for (int h = 0; h < hkv; ++h) {
        auto it = cover.find(r * hkv + h);
        if (!planned) {
          if (it != cover.end()) fail(trial, "skipped row planned", r);
          continue;
        }
        if (it == cover.end()) {
          fail(trial, "row not planned", r);
          continue;
        }
        auto v = it->second;
        std::sort(v.begin(), v.end());
        int at = 0, lo = 1 << 30, hi = 0;
        for (size_t i = 0; i < v.size(); ++i) {
          if (v[i].first != at) fail(trial, "gap or overlap", r);
          at = v[i].second;
          if (i + 1 < v.size()) {  // all but the last piece
            lo = std::min(lo, v[i].second - v[i].first);
            hi = std::max(hi, v[i].second - v[i].first);
          }
        }
        if (at != (int)pos[r] + 1) fail(trial, "context not covered", r);
        if ((int)v.size() != plan.row_nsplit[r]) fail(trial, "row_nsplit mismatch", r);
        if (!in_pack[r] && v.size() > 1 && (lo != hi || v.back().second - v.back().first > hi))
          fail(trial, "uneven pieces", r);
      }
    }
    if (plan.balanced && (int64_t)plan.work.size() > 4 * slots)
      fail(trial, "balanced plan overfills four rounds", -1);
    // shared blocks: attended twice over the planned rows
    std::vector<int> uses(100000, 0);  // block ids are drawn below 100000
    for (int r = 0; r < rows; ++r) {
      if (use_skip && skip[r]) continue;
      const int nb = ((int)pos[r] + bs) >> bs_log2;
      for (int j = 0; j < nb; ++j) uses[ids[off[r] + j]]++;
    }
    bool any_shared = false, any_private = false;
    for (const DecodeWork& w : plan.work) {
      if (w.shared == 2) continue;
      const int nblk = ((w.end - 1) >> bs_log2) - (w.start >> bs_log2) + 1;
      bool sh = false;
      for (int j = 0; j < nblk; ++j) sh = sh || uses[ids[w.tbl_off + j]] > 1;
      if ((w.shared != 0) != sh) fail(trial, "shared flag", w.item / hkv);
      any_shared = any_shared || sh;
      any_private = any_private || !sh;
    }
    bool any_shared_block = false;
    for (int u : uses) any_shared_block = any_shared_block || u > 1;
    if (plan.stream_kv != !any_shared_block) fail(trial, "stream_kv", -1);
    if (plan.mixed_kv != (any_shared_block && any_private)) fail(trial, "mixed_kv", -1);
  }
  printf("%d trials, %d balanced, %ld packed items, %d failures\n", trials, balanced,
         packed_items, fails);
  return fails ? 1 : 0;
}
