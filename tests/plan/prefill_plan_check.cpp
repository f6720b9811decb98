// Property check of the chunked-prefill work planner (orionserve-rs_amd/csrc/
// prefill_plan.cpp), host only.
//
//   prefill_plan_check random TRIALS
//     For random batches (chunk lengths, prefixes, query-head groups, KV
//     heads, CU counts, head_dim 128 and 256) every plan must give each (sequence, tile of packed
//     rows) exactly `nparts` entries, parts 0 .. nparts-1 in key order, whose
//     key-tile ranges tile [0, key tiles the tile's last row attends) with no
//     gap or overlap; nparts must be the same for every tile of a sequence;
//     row_parts / split_rows must list exactly the rows of split sequences;
//     and the list must be sorted longest first.
//   prefill_plan_check case CUS GROUP HKV P0,P1,... C0,C1,... [HEAD_DIM]
//     Plans one batch (prefixes P, chunk lengths C) and prints
//       parts=<max parts> entries=<n> empty=<parts reading no key>
//       straddle=<parts whose first key lies inside the positions of one
//                 16-row MFMA tile of queries: some of its queries attend no
//                 key of the part while others do>
//     after checking the same properties.
// Exit status 1 on any failure.
#include "kernels.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <random>
#include <sstream>
#include <string>
#include <vector>

using orion::PrefillPlan;
using orion::PrefillTile;

namespace {

int g_fails = 0;
void fail(const char* what, long a, long b) {
  if (g_fails++ < 20) printf("FAIL: %s (%ld, %ld)\n", what, a, b);
}

struct Stats {
  int empty = 0, straddle = 0;
};

Stats check(const std::vector<int32_t>& prefix, const std::vector<int32_t>& chunk, int group,
            int hkv, int cus, int head_dim = 128) {
  const int S = (int)chunk.size();
  std::vector<int32_t> start(S);
  std::vector<uint32_t> first(S);
  int rows = 0;
  for (int s = 0; s < S; ++s) {
    start[s] = rows;
    rows += chunk[s];
    first[s] = (uint32_t)prefix[s];
  }
  PrefillPlan plan;
  orion::build_prefill_order(start.data(), chunk.data(), first.data(), S, group, hkv, cus, &plan,
                             head_dim);
  const int64_t kBM = orion::prefill_tile_rows(head_dim);
  Stats st;
  // expected tiles and their key-tile counts
  std::map<std::pair<int, int>, std::vector<const PrefillTile*>> by_tile;
  for (const PrefillTile& t : plan.order) by_tile[{t.seq, t.tile}].push_back(&t);
  std::vector<int> seq_np(S, 0);
  size_t expected = 0;
  for (int s = 0; s < S; ++s) {
    const int64_t packed = (int64_t)chunk[s] * group;
    for (int64_t t = 0; t * kBM < packed; ++t) {
      const int64_t kv_len = (int64_t)prefix[s] + (std::min(packed, (t + 1) * kBM) - 1) / group + 1;
      const int64_t kvt = (kv_len + 63) / 64;
      auto it = by_tile.find({s, (int)t});
      if (it == by_tile.end()) {
        fail("tile missing from the plan", s, t);
        continue;
      }
      auto parts = it->second;
      std::sort(parts.begin(), parts.end(),
                [](const PrefillTile* a, const PrefillTile* b) { return a->part < b->part; });
      const int np = parts[0]->nparts;
      expected += np;
      if ((int)parts.size() != np) fail("entries per tile != nparts", s, t);
      if (seq_np[s] == 0) seq_np[s] = np;
      if (seq_np[s] != np) fail("nparts differs between tiles of a sequence", s, t);
      int64_t next = 0;
      for (int k = 0; k < (int)parts.size(); ++k) {
        const PrefillTile* p = parts[k];
        if (p->part != k || p->nparts != np) fail("part index", s, k);
        if (p->kt0 != next || p->kt1 < p->kt0) fail("key ranges not contiguous", s, k);
        next = p->kt1;
        if (p->kt0 == p->kt1) ++st.empty;
        if (np > 1 && p->kt1 > p->kt0 && p->kt0 > 0) {
          // 16-row MFMA tiles of this workgroup: packed rows [t*kBM + 16j, +16)
          const int64_t key0 = (int64_t)p->kt0 * 64;
          for (int64_t r0 = t * kBM; r0 < std::min(packed, (t + 1) * kBM); r0 += 16) {
            const int64_t r1 = std::min(packed, r0 + 16) - 1;
            const int64_t pmin = prefix[s] + r0 / group, pmax = prefix[s] + r1 / group;
            if (pmin < key0 && key0 <= pmax) {
              ++st.straddle;
              break;
            }
          }
        }
      }
      if (next != kvt) fail("key ranges do not end at the tile's keys", s, next);
    }
  }
  if (plan.order.size() != expected) fail("extra entries", (long)plan.order.size(), expected);
  for (size_t i = 1; i < plan.order.size(); ++i) {
    const auto len = [](const PrefillTile& t) { return t.kt1 - t.kt0; };
    if (len(plan.order[i]) > len(plan.order[i - 1])) fail("not longest first", (long)i, 0);
  }
  int max_np = 1;
  std::vector<int32_t> want_rows;
  for (int s = 0; s < S; ++s) {
    const int np = std::max(seq_np[s], 1);
    max_np = std::max(max_np, np);
    for (int r = 0; r < chunk[s]; ++r) {
      if ((int)plan.row_parts.size() <= start[s] + r) {
        fail("row_parts too short", s, r);
        break;
      }
      if (plan.row_parts[start[s] + r] != (np > 1 ? np : 0)) fail("row_parts", s, r);
      if (np > 1) want_rows.push_back(start[s] + r);
    }
  }
  if (plan.split_rows != want_rows) fail("split_rows", (long)plan.split_rows.size(), want_rows.size());
  if (plan.max_parts != max_np) fail("max_parts", plan.max_parts, max_np);
  return st;
}

std::vector<int32_t> parse_list(const char* s) {
  std::vector<int32_t> v;
  std::stringstream ss(s);
  std::string tok;
  while (std::getline(ss, tok, ',')) v.push_back(atoi(tok.c_str()));
  return v;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc >= 3 && std::string(argv[1]) == "random") {
    const int trials = atoi(argv[2]);
    std::mt19937 rng(20261203);
    long split = 0, empty = 0, straddle = 0;
    for (int trial = 0; trial < trials; ++trial) {
      const int S = 1 + rng() % 12;
      const int group = 1 + rng() % 8, hkv = 1 + rng() % 8;
      const int cus = (trial % 3 == 0) ? 256 : (int)(rng() % 300);
      std::vector<int32_t> prefix(S), chunk(S);
      for (int s = 0; s < S; ++s) {
        chunk[s] = (rng() % 6 == 0) ? 0 : 1 + rng() % 3000;
        prefix[s] = (rng() % 3 == 0) ? 0 : (int)(rng() % 30000);
      }
      // head_dim 256 plans tiles of half as many packed rows
      const Stats st = check(prefix, chunk, group, hkv, cus, trial % 2 ? 256 : 128);
      empty += st.empty;
      straddle += st.straddle;
      split += st.empty + st.straddle > 0;
    }
    printf("%d trials empty=%ld straddle=%ld failures=%d\n", trials, empty, straddle, g_fails);
    return g_fails ? 1 : 0;
  }
  if ((argc == 7 || argc == 8) && std::string(argv[1]) == "case") {
    const int cus = atoi(argv[2]), group = atoi(argv[3]), hkv = atoi(argv[4]);
    const int head_dim = argc == 8 ? atoi(argv[7]) : 128;
    const auto prefix = parse_list(argv[5]), chunk = parse_list(argv[6]);
    if (prefix.size() != chunk.size()) {
      printf("prefix and chunk lists differ in length\n");
      return 2;
    }
    std::vector<int32_t> start(chunk.size());
    const Stats st = check(prefix, chunk, group, hkv, cus, head_dim);
    // max parts, entries
    PrefillPlan plan;
    std::vector<uint32_t> first(prefix.begin(), prefix.end());
    int rows = 0;
    for (size_t s = 0; s < chunk.size(); ++s) {
      start[s] = rows;
      rows += chunk[s];
    }
    orion::build_prefill_order(start.data(), chunk.data(), first.data(), (int64_t)chunk.size(),
                               group, hkv, cus, &plan, head_dim);
    printf("parts=%d entries=%zu empty=%d straddle=%d failures=%d\n", plan.max_parts,
           plan.order.size(), st.empty, st.straddle, g_fails);
    return g_fails ? 1 : 0;
  }
  printf("usage: prefill_plan_check random TRIALS | case CUS GROUP HKV PREFIXES CHUNKS "
         "[HEAD_DIM]\n");
  return 2;
}
