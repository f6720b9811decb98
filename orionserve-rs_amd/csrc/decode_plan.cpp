// Host-side decode planning: the work list of the paged decode kernels
// (attention_decode.hip) and the size of their split-K workspace.  Pure host
// code, so it builds and is tested without a GPU.
#include "kernels.hpp"

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <map>
#include <tuple>
#include <unordered_map>
#include <utility>
#include <vector>

namespace orion {

// Decode work decomposition.  A work item is (row, KV head, piece of the
// row's context) and runs on one wave; a row split into several pieces is
// merged afterwards by the combine kernel.  Items are ordered longest first,
// so the last waves to be dispatched are the shortest.  Two ways to cut:
//  * balanced: each row is cut into equal pieces, as few as keep the items
//    within one round of the resident wave slots (or within R rounds when
//    one cannot hold them; see build_decode_plan), when the same fluid model
//    rates it faster than the best fixed chunk (bandwidth-bound batches);
//  * fixed chunks of C tokens, C a power of two chosen with a fluid model of
//    the split kernel, in token-equivalents of one wave's streaming:
//      time(C) = max((sum of item sizes + items * kItemOverhead) / wave_slots
//                    + C / 2,                       (bandwidth-bound, mean tail)
//                    largest item + kItemOverhead)  (latency-bound: one wave)
//    The per-item overhead (setup, split-K partial write and merge read) and
//    the half-item tail were fitted to measured config-2 times at C = 128 ...
//    1024.  Latency-bound (small) batches keep them: short chunks give
//    short dependent chains per wave.

// Shortest piece a balanced plan cuts: below it the per-item set-up and the
// merge of many partials cost more than the even spread gains.
constexpr int kMinBalancedPiece = 128;
// Most rounds of wave slots a balanced plan fills (beyond: fixed chunks).
constexpr int64_t kMaxBalancedRounds = 4;

// Per-item overhead of the fluid model, in token-equivalents of one wave's
// streaming (set-up, split-K partial write and merge read).
constexpr int64_t kItemOverhead = 96;

// C is a power of two (2^c_log2).
static int64_t estimate_split_time(const std::vector<int>& lens, int64_t hkv, int C, int c_log2,
                                   int64_t slots) {
  int64_t total = 0, items = 0, largest = 0;
  for (int L : lens) {
    const int64_t full = L >> c_log2, tail = L & (C - 1);
    items += hkv * (full + (tail ? 1 : 0));
    total += (int64_t)hkv * L;
    largest = std::max<int64_t>(largest, full ? C : tail);
  }
  if (items == 0) return 0;
  const int64_t fluid = (total + items * kItemOverhead) / std::max<int64_t>(slots, 1) +
                        std::min<int64_t>(C, largest) / 2;
  return std::max(fluid, largest + kItemOverhead);
}

// Shortest shared prefix worth a packed item (tokens).
constexpr int kMinPackPrefix = 256;

void build_decode_plan(const uint32_t* positions, const int32_t* row_seq,
                       const int64_t* bt_offsets, const uint32_t* bt_ids, int64_t rows,
                       int64_t hkv, int64_t block_size, int64_t wave_slots,
                       const uint8_t* skip_rows, DecodePlanHost* plan, int pack_r) {
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  const int unit = (int)std::max<int64_t>(16, block_size);
  // Rows flagged in skip_rows get no work (another kernel covers them);
  // their length counts as 0 for the chunk choice and the split bound.
  std::vector<int> lens(rows);
  plan->rows.clear();
  for (int64_t r = 0; r < rows; ++r) {
    const bool skip = skip_rows && skip_rows[r];
    lens[r] = skip ? 0 : (int)positions[r] + 1;
    if (skip_rows && !skip) plan->rows.push_back((int32_t)r);
  }

  // ---- packs: rows whose tables start with the same block ids (a shared
  // prefix) attend that prefix together, pack_r rows per item.  Rows are
  // grouped by their first block id and ordered by how many leading blocks
  // they share with the group's first row; each pack's prefix is the part
  // all its rows share, in whole units, short of every row's last position
  // (so each row keeps a private piece). ORION_DECODE_PACK=0 disables
  // packing (measurement knob, read per call). ----
  const char* pack_env = getenv("ORION_DECODE_PACK");
  if (pack_env && pack_env[0] == '0') pack_r = 0;
  std::vector<int> prefix(rows, 0), pack_of(rows, -1);
  std::vector<int> pack_len;  // shared prefix tokens of each pack
  plan->pack_rows.clear();
  plan->pack_r = pack_r >= 2 ? pack_r : 0;
  if (pack_r >= 2) {
    std::unordered_map<uint32_t, std::vector<int64_t>> by_first;
    for (int64_t r = 0; r < rows; ++r)
      if (lens[r] > kMinPackPrefix) by_first[bt_ids[bt_offsets[row_seq[r]]]].push_back(r);
    std::vector<uint32_t> keys;
    for (const auto& kv : by_first)
      if (kv.second.size() >= 2) keys.push_back(kv.first);
    std::sort(keys.begin(), keys.end());  // deterministic pack order
    for (uint32_t key : keys) {
      std::vector<int64_t>& grp = by_first[key];
      const int64_t r0 = grp[0];
      const uint32_t* t0 = bt_ids + bt_offsets[row_seq[r0]];
      const int64_t nb0 = ((int64_t)lens[r0] + block_size - 1) >> bs_log2;
      std::vector<std::pair<int64_t, int64_t>> lcp;  // (shared blocks with r0, row)
      for (int64_t r : grp) {
        const uint32_t* t = bt_ids + bt_offsets[row_seq[r]];
        const int64_t nb = std::min<int64_t>(nb0, ((int64_t)lens[r] + block_size - 1) >> bs_log2);
        int64_t k = 0;
        while (k < nb && t[k] == t0[k]) ++k;
        lcp.push_back({k, r});
      }
      std::stable_sort(lcp.begin(), lcp.end(),
                       [](const auto& a, const auto& b) { return a.first > b.first; });
      for (size_t i = 0; i + 2 <= lcp.size(); i += pack_r) {
        const size_t e = std::min(lcp.size(), i + (size_t)pack_r);
        int64_t L = INT64_MAX;
        for (size_t j = i; j < e; ++j)
          L = std::min<int64_t>(L, std::min<int64_t>(lcp[j].first * block_size,
                                                     lens[lcp[j].second] - 1));
        L = L / unit * unit;
        if (L < kMinPackPrefix) continue;
        const int pk = (int)pack_len.size();
        pack_len.push_back((int)L);
        for (size_t j = i; j < i + (size_t)pack_r; ++j) {
          const int64_t r = j < e ? lcp[j].second : -1;
          plan->pack_rows.push_back((int32_t)r);
          if (r >= 0) prefix[r] = (int)L, pack_of[r] = pk;
        }
      }
    }
  }
  const int npacks = (int)pack_len.size();

  // The segments the pieces are cut from: each row's private part [prefix,
  // len) and each pack's prefix [0, L).  Empty ones (skipped rows) are left
  // out: they add no items, bytes or length to any estimate below.
  std::vector<int> seg;
  seg.reserve(rows + pack_len.size());
  int max_len = 0;
  for (int64_t r = 0; r < rows; ++r)
    if (lens[r] - prefix[r] > 0) seg.push_back(lens[r] - prefix[r]);
  for (int L : pack_len) seg.push_back(L);
  for (int L : seg) max_len = std::max(max_len, L);

  int best_c = 0;
  int64_t best_t = 0;
  for (int C = 64, c_log2 = 6; C <= 2048; C <<= 1, ++c_log2) {
    if (C < block_size || C / block_size > 64) continue;
    const int64_t t = estimate_split_time(seg, hkv, C, c_log2, wave_slots);
    if (best_c == 0 || t < best_t) {
      best_c = C;
      best_t = t;
    }
  }
  if (best_c == 0) best_c = (int)std::max<int64_t>(block_size, 64);
  // ORION_DECODE_CHUNK overrides the choice (measurement knob).
  static const int forced = [] {
    const char* e = getenv("ORION_DECODE_CHUNK");
    return e ? atoi(e) : 0;
  }();
  if (forced >= 16 && (forced & (forced - 1)) == 0 && forced >= block_size &&
      forced / block_size <= 64)
    best_c = forced;
  const int C = best_c;
  // Balanced pieces: segment s is cut into n_s = ceil(L_s / P) pieces of
  // equal length (rounded up to whole blocks of at least 16 tokens), with the
  // bound P the smallest for which every item fits in one round of the
  // resident wave slots, so no wave starts after the first round and the
  // pieces of a row end together.  ORION_DECODE_BALANCE=0 keeps fixed chunks.
  // (Pieces are at most 64 table entries: the waves hold a piece's block ids
  // one per lane.)
  const char* balance_env = getenv("ORION_DECODE_BALANCE");
  const bool balance_knob = !(balance_env && balance_env[0] == '0');
  const int max_piece = (int)std::max<int64_t>(unit, 64 * block_size / unit * unit);
  auto pieces_of = [&](int L, int P, int* piece) {
    const int n = (L + P - 1) / P;
    *piece = ((L + n - 1) / n + unit - 1) / unit * unit;
    return (L + *piece - 1) / *piece;
  };
  auto items_at = [&](int P) {
    int64_t items = 0;
    for (int L : seg) {
      int piece;
      if (L) items += hkv * pieces_of(L, P, &piece);
    }
    return items;
  };
  // Rounds: when even the longest pieces overfill one round of wave slots,
  // the pieces fill R rounds instead (R <= kMaxBalancedRounds), again as
  // evenly as the smallest bound P for R * slots items allows.
  int bal_p = 0;
  if (balance_knob && forced == 0 && max_len > 0) {
    const int64_t slots = std::max<int64_t>(wave_slots, 1);
    const int64_t rounds = (items_at(max_piece) + slots - 1) / slots;
    if (rounds <= kMaxBalancedRounds) {
      const int64_t target = rounds * slots;
      int lo = 1, hi = max_piece / unit;  // P = k * unit; items_at is non-increasing in k
      while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (items_at(mid * unit) <= target) hi = mid; else lo = mid + 1;
      }
      bal_p = std::max(lo * unit, kMinBalancedPiece);
      if (bal_p > max_piece) bal_p = 0;
      // Keep it only where the fluid model prefers it: evenly cut rounds
      // (R rounds of the longest piece, or the bandwidth term) against the
      // best fixed chunk.  Small batches are latency-bound and keep short
      // fixed chunks.
      if (bal_p) {
        int64_t items = 0, total = 0, largest = 0;
        for (int L : seg) {
          if (!L) continue;
          int piece;
          const int n = pieces_of(L, bal_p, &piece);
          items += hkv * n;
          total += hkv * (int64_t)L;
          largest = std::max<int64_t>(largest, std::min(piece, L));
        }
        const int64_t r = (items + slots - 1) / slots;
        const int64_t t_bal = std::max((total + items * kItemOverhead) / slots,
                                       r * (largest + kItemOverhead));
        if (t_bal >= best_t) bal_p = 0;
      }
    }
  }
  plan->balanced = bal_p > 0;
  plan->work.clear();
  plan->row_nsplit.assign(rows, 0);
  plan->chunk = 0;
  plan->max_splits = 0;
  auto piece_len = [&](int L) {
    int piece = C;
    if (bal_p) pieces_of(L, bal_p, &piece);
    return piece;
  };
  // pack prefixes: np pieces each, splits 0 .. np-1 of every row of the pack
  std::vector<int> pack_np(npacks), pack_piece(npacks);
  for (int pk = 0; pk < npacks; ++pk) {
    pack_piece[pk] = piece_len(pack_len[pk]);
    pack_np[pk] = (pack_len[pk] + pack_piece[pk] - 1) / pack_piece[pk];
    plan->chunk = std::max(plan->chunk, std::min(pack_piece[pk], pack_len[pk]));
  }
  // (start, length, row or pack, split) of every piece, then ordered longest
  // first (stable: a row's pieces stay in order, full chunks before tails)
  struct Piece {
    int start, len;
    int64_t row;  // pack index for packed pieces
    int split;
    bool packed;
  };
  std::vector<Piece> pcs;
  for (int64_t r = 0; r < rows; ++r) {
    const int L = lens[r] - prefix[r];
    if (!lens[r]) continue;
    const int piece = piece_len(L);
    const int n = (L + piece - 1) / piece;
    const int np = pack_of[r] >= 0 ? pack_np[pack_of[r]] : 0;
    plan->row_nsplit[r] = np + n;
    plan->max_splits = std::max(plan->max_splits, np + n);
    plan->chunk = std::max(plan->chunk, std::min(piece, L));
    for (int s = 0; s < n; ++s)
      pcs.push_back({prefix[r] + s * piece, std::min(L - s * piece, piece), r, np + s, false});
  }
  for (int pk = 0; pk < npacks; ++pk)
    for (int s = 0; s < pack_np[pk]; ++s)
      pcs.push_back({s * pack_piece[pk], std::min(pack_len[pk] - s * pack_piece[pk],
                                                  pack_piece[pk]), pk, s, true});
  std::stable_sort(pcs.begin(), pcs.end(),
                   [](const Piece& a, const Piece& b) { return a.len > b.len; });
  plan->work.reserve(pcs.size() * hkv);
  plan->num_packed = 0;
  auto tbl_of = [&](const Piece& pc) {
    const int64_t r0 = pc.packed ? plan->pack_rows[pc.row * pack_r] : pc.row;
    return bt_offsets[row_seq[r0]] + (pc.start >> bs_log2);
  };
  // Packed items first.  Packs on one prefix share its pieces' blocks, so a
  // piece is taken by kItemsPerWorkgroup packs at a time with the KV head
  // outer: the waves of one workgroup (adjacent items) then read the same
  // K/V rows together and the repeats hit the CU's cache.  (A packed item
  // always writes partials, nsplit 2 -- every row of a pack has a private
  // piece too -- and is flagged shared = 2.)
  constexpr int kItemsPerWorkgroup = 4;
  std::vector<std::vector<const Piece*>> same_piece;  // packs reading one piece
  std::map<std::tuple<int, int, uint32_t>, size_t> piece_index;
  for (const Piece& pc : pcs) {
    if (!pc.packed) continue;
    const auto key = std::make_tuple(pc.start, pc.len, bt_ids[tbl_of(pc)]);
    auto it = piece_index.find(key);
    if (it == piece_index.end()) {
      piece_index[key] = same_piece.size();
      same_piece.push_back({&pc});
    } else {
      same_piece[it->second].push_back(&pc);
    }
  }
  for (const auto& packs : same_piece)
    for (size_t g = 0; g < packs.size(); g += kItemsPerWorkgroup) {
      const size_t ge = std::min(packs.size(), g + kItemsPerWorkgroup);
      for (int64_t h = 0; h < hkv; ++h)
        for (size_t j = g; j < ge; ++j) {
          const Piece& pc = *packs[j];
          const int64_t tbl_off = tbl_of(pc);
          plan->work.push_back({(int32_t)(pc.row * hkv + h), pc.start, pc.start + pc.len, 2,
                                (int32_t)tbl_off, (int32_t)bt_ids[tbl_off], 2, pc.split});
          ++plan->num_packed;
        }
    }
  for (const Piece& pc : pcs) {
    if (pc.packed) continue;
    const int64_t tbl_off = tbl_of(pc);
    const int32_t n = plan->row_nsplit[pc.row];
    for (int64_t h = 0; h < hkv; ++h)
      plan->work.push_back({(int32_t)(pc.row * hkv + h), pc.start, pc.start + pc.len, n,
                            (int32_t)tbl_off, (int32_t)bt_ids[tbl_off], 0, pc.split});
  }
  const int64_t num_plain = (int64_t)plan->work.size() - plan->num_packed;
  // Shared blocks: a block id attended by two planned rows (two rows of one
  // sequence share their prefix blocks too).  Two passes over the attended
  // ids: the first finds their range (the bitmap words touched), the second
  // sets two bitmaps (seen, seen again) without branches; both are cleared
  // afterwards.  Then each plain work item is flagged when its token range
  // reads a shared block (packed items, shared = 2, keep cached loads).
  static thread_local std::vector<uint64_t> seen, again;
  uint32_t id_lo = UINT32_MAX, id_hi = 0;
  for (int64_t r = 0; r < rows; ++r) {
    if (lens[r] == 0) continue;
    const uint32_t* t = bt_ids + bt_offsets[row_seq[r]];
    const int64_t nb = ((int64_t)lens[r] + block_size - 1) >> bs_log2;
    for (int64_t j = 0; j < nb; ++j) {
      id_lo = std::min(id_lo, t[j]);
      id_hi = std::max(id_hi, t[j]);
    }
  }
  bool shared = false;
  const size_t w_lo = id_lo >> 6, w_hi = id_hi >> 6;  // words touched (when id_lo <= id_hi)
  if (id_lo <= id_hi) {
    if (w_hi >= seen.size()) seen.resize(w_hi + 1, 0), again.resize(w_hi + 1, 0);
    uint64_t* sn = seen.data();
    uint64_t* ag = again.data();
    for (int64_t r = 0; r < rows; ++r) {
      if (lens[r] == 0) continue;
      const uint32_t* t = bt_ids + bt_offsets[row_seq[r]];
      const int64_t nb = ((int64_t)lens[r] + block_size - 1) >> bs_log2;
      for (int64_t j = 0; j < nb; ++j) {
        const uint32_t id = t[j];
        const uint64_t bit = 1ull << (id & 63);
        ag[id >> 6] |= sn[id >> 6] & bit;
        sn[id >> 6] |= bit;
      }
    }
    for (size_t w = w_lo; w <= w_hi && !shared; ++w) shared = again[w] != 0;
  }
  int64_t shared_items = 0;
  if (shared) {
    // the hkv items of a piece are adjacent and read the same blocks
    for (size_t i = 0; i < plan->work.size(); i += hkv) {
      const DecodeWork& wk = plan->work[i];
      if (wk.shared == 2) continue;
      const int nb = ((wk.end - 1) >> bs_log2) - (wk.start >> bs_log2) + 1;
      bool s = false;
      for (int j = 0; j < nb && !s; ++j) {
        const uint32_t id = bt_ids[wk.tbl_off + j];
        s = (again[id >> 6] >> (id & 63)) & 1;
      }
      for (int64_t h = 0; h < hkv; ++h) plan->work[i + h].shared = s ? 1 : 0;
      shared_items += s ? hkv : 0;
    }
  }
  if (id_lo <= id_hi) {
    std::fill(seen.begin() + w_lo, seen.begin() + w_hi + 1, 0);
    std::fill(again.begin() + w_lo, again.begin() + w_hi + 1, 0);
  }
  plan->stream_kv = !shared;
  plan->mixed_kv = shared && shared_items < num_plain;
}

int decode_pack_rows(const KvGeom& kv, int64_t hq) {
  if (!kv.dtype_bf16 || (kv.head_dim != 64 && kv.head_dim != 128) || kv.num_kv_heads <= 0)
    return 0;
  const int64_t G = hq / kv.num_kv_heads;
  return G >= 1 && G <= 8 ? (int)(16 / G) : 0;
}

size_t decode_workspace_bytes(int64_t rows, int64_t hq, int64_t D, int64_t max_splits) {
  if (max_splits <= 1) return 0;
  return (size_t)(rows * hq * max_splits) * (size_t)(D + 2) * sizeof(float);
}

}  // namespace orion
