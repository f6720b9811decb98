// Host-side prefill planning: the work list of the chunked-prefill kernel
// (attention_prefill.hip) -- tiles of packed rows, longest first, and the
// key parts of long-prefix sequences.  Pure host code, so it builds and is
// tested without a GPU (tests/plan/prefill_plan_check.cpp).
#include "kernels.hpp"

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <utility>
#include <vector>

namespace orion {

// Workgroup shape: 8 waves with a 3-stage K/V ring (one workgroup per CU,
// 96 KiB of LDS at d = 128), or 4 waves with 2 stages (two per CU).
// ORION_PREFILL_WAVES=4 selects the latter (measurement knob).
int prefill_waves() {
  static const int w = [] {
    const char* e = getenv("ORION_PREFILL_WAVES");
    return (e && atoi(e) == 4) ? 4 : 8;
  }();
  return w;
}

// (head_dim 256 always runs 8 waves: its 2-stage ring fills 128 KiB of LDS)
int prefill_tile_rows(int64_t head_dim) {
  return (head_dim > 128 ? 8 : prefill_waves()) * 16 * prefill_wave_row_tiles(head_dim);
}

// Key parts: a sequence is cut into nparts key ranges when its longest tile
// reads more than an even share of all the tiles' key reads over the CUs
// (and at least kMinPartTiles key tiles per part), so one long-prefix chunk
// no longer sets the launch's length while the other CUs idle.  Every tile
// of the sequence gets the same nparts (a row's heads can straddle two
// tiles, and the merge counts parts per row).
constexpr int kMinPartTiles = 16;

void build_prefill_order(const int32_t* row_start, const int32_t* row_count,
                         const uint32_t* first_pos, int64_t num_seqs, int64_t group, int64_t hkv,
                         int64_t cus, PrefillPlan* plan, int64_t head_dim) {
  const int64_t kBM = prefill_tile_rows(head_dim);
  struct Tile {
    int64_t seq, tile, kv_tiles;
  };
  std::vector<Tile> tiles;
  int64_t total = 0;
  for (int64_t s = 0; s < num_seqs; ++s) {
    const int64_t packed = (int64_t)row_count[s] * group;
    for (int64_t t = 0; t * kBM < packed; ++t) {
      // keys the tile's last packed row attends (the kernel's kv_len)
      const int64_t kv_len = (int64_t)first_pos[s] + (std::min(packed, (t + 1) * kBM) - 1) / group + 1;
      const int64_t kvt = (kv_len + 63) / 64;
      tiles.push_back({s, t, kvt});
      total += kvt;
    }
  }
  // ORION_PREFILL_SPLIT=0 keeps every sequence whole (measurement knob, read per call)
  const char* split_env = getenv("ORION_PREFILL_SPLIT");
  if (split_env && split_env[0] == '0') cus = 0;
  const int64_t share = cus > 0 ? std::max<int64_t>((total * hkv + cus - 1) / cus, kMinPartTiles)
                                : INT64_MAX;
  std::vector<int64_t> seq_parts(num_seqs, 1);
  for (const Tile& t : tiles)
    if (t.kv_tiles > share)
      seq_parts[t.seq] = std::max(seq_parts[t.seq], (t.kv_tiles + share - 1) / share);
  std::vector<std::pair<int64_t, PrefillTile>> items;
  for (const Tile& t : tiles) {
    // every tile of a split sequence writes all nparts parts (a short tile's
    // last parts may read no key: they write empty partials the merge weighs 0)
    const int64_t np = seq_parts[t.seq];
    const int64_t per = (t.kv_tiles + np - 1) / np;
    const int32_t nparts = (int32_t)np;
    for (int64_t k = 0; k < np; ++k) {
      const int64_t a = std::min(t.kv_tiles, k * per), b = std::min(t.kv_tiles, a + per);
      items.push_back({b - a, PrefillTile{(int32_t)t.seq, (int32_t)t.tile, (int32_t)a, (int32_t)b,
                                          (int32_t)k, nparts}});
    }
  }
  std::stable_sort(items.begin(), items.end(),
                   [](const auto& a, const auto& b) { return a.first > b.first; });
  plan->order.clear();
  for (const auto& it : items) plan->order.push_back(it.second);
  // rows whose results come in parts
  int64_t rows = 0;
  for (int64_t s = 0; s < num_seqs; ++s)
    rows = std::max<int64_t>(rows, (int64_t)row_start[s] + row_count[s]);
  plan->row_parts.assign(rows, 0);
  plan->split_rows.clear();
  plan->max_parts = 1;
  for (int64_t s = 0; s < num_seqs; ++s) {
    if (seq_parts[s] < 2) continue;
    plan->max_parts = std::max<int>(plan->max_parts, (int)seq_parts[s]);
    for (int64_t r = 0; r < row_count[s]; ++r) {
      plan->row_parts[row_start[s] + r] = (int32_t)seq_parts[s];
      plan->split_rows.push_back((int32_t)(row_start[s] + r));
    }
  }
}

}  // namespace orion
