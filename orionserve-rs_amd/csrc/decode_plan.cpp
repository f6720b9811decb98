// Host-side decode planning: the work list of the paged decode kernels
// (attention_decode.hip) and the size of their split-K workspace.  Pure host
// code, so it builds and is tested without a GPU.
#include "kernels.hpp"

#include <algorithm>
#include <cstdint>
#include <cstdlib>
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

static int64_t estimate_split_time(const std::vector<int>& lens, int64_t hkv, int C,
                                   int64_t slots) {
  int64_t total = 0, items = 0, largest = 0;
  for (int L : lens) {
    const int64_t full = L / C, tail = L % C;
    items += hkv * (full + (tail ? 1 : 0));
    total += (int64_t)hkv * L;
    largest = std::max<int64_t>(largest, full ? C : tail);
  }
  if (items == 0) return 0;
  const int64_t fluid = (total + items * kItemOverhead) / std::max<int64_t>(slots, 1) +
                        std::min<int64_t>(C, largest) / 2;
  return std::max(fluid, largest + kItemOverhead);
}

void build_decode_plan(const uint32_t* positions, const int32_t* row_seq,
                       const int64_t* bt_offsets, const uint32_t* bt_ids, int64_t rows,
                       int64_t hkv, int64_t block_size, int64_t wave_slots,
                       const uint8_t* skip_rows, DecodePlanHost* plan) {
  int bs_log2 = 0;
  while ((1 << bs_log2) < block_size) ++bs_log2;
  // Rows flagged in skip_rows get no work (another kernel covers them);
  // their length counts as 0 for the chunk choice and the split bound.
  std::vector<int> lens(rows);
  int max_len = 0;
  plan->rows.clear();
  for (int64_t r = 0; r < rows; ++r) {
    const bool skip = skip_rows && skip_rows[r];
    lens[r] = skip ? 0 : (int)positions[r] + 1;
    max_len = std::max(max_len, lens[r]);
    if (skip_rows && !skip) plan->rows.push_back((int32_t)r);
  }
  int best_c = 0;
  int64_t best_t = 0;
  for (int C = 64; C <= 2048; C <<= 1) {
    if (C < block_size || C / block_size > 64) continue;
    const int64_t t = estimate_split_time(lens, hkv, C, wave_slots);
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
  // Balanced pieces: row r is cut into n_r = ceil(L_r / P) pieces of equal
  // length (rounded up to whole blocks of at least 16 tokens), with the
  // bound P the smallest for which every item fits in one round of the
  // resident wave slots, so no wave starts after the first round and the
  // pieces of a row end together.  ORION_DECODE_BALANCE=0 keeps fixed chunks.
  // (Pieces are at most 64 table entries: the waves hold a piece's block ids
  // one per lane.)
  const char* balance_env = getenv("ORION_DECODE_BALANCE");
  const bool balance_knob = !(balance_env && balance_env[0] == '0');
  const int unit = (int)std::max<int64_t>(16, block_size);
  const int max_piece = (int)std::max<int64_t>(unit, 64 * block_size / unit * unit);
  auto pieces_of = [&](int L, int P, int* piece) {
    const int n = (L + P - 1) / P;
    *piece = ((L + n - 1) / n + unit - 1) / unit * unit;
    return (L + *piece - 1) / *piece;
  };
  auto items_at = [&](int P) {
    int64_t items = 0;
    for (int L : lens) {
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
        for (int L : lens) {
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
  // (start, length, row) of every piece, then ordered longest first (stable:
  // a row's pieces stay in order, full chunks before tails)
  struct Piece {
    int start, len;
    int64_t row;
  };
  std::vector<Piece> pcs;
  std::vector<int> row_piece(rows, 1);
  for (int64_t r = 0; r < rows; ++r) {
    const int L = lens[r];
    if (!L) continue;
    int piece = C;
    if (bal_p) pieces_of(L, bal_p, &piece);
    const int n = (L + piece - 1) / piece;
    row_piece[r] = piece;
    plan->row_nsplit[r] = n;
    plan->max_splits = std::max(plan->max_splits, n);
    plan->chunk = std::max(plan->chunk, std::min(piece, L));
    for (int s = 0; s < n; ++s) pcs.push_back({s * piece, std::min(L - s * piece, piece), r});
  }
  std::stable_sort(pcs.begin(), pcs.end(),
                   [](const Piece& a, const Piece& b) { return a.len > b.len; });
  plan->work.reserve(pcs.size() * hkv);
  for (const Piece& pc : pcs) {
    const int64_t tbl_off = bt_offsets[row_seq[pc.row]] + (pc.start >> bs_log2);
    const int32_t n = plan->row_nsplit[pc.row];
    const int32_t split = pc.start / row_piece[pc.row];
    for (int64_t h = 0; h < hkv; ++h)
      plan->work.push_back({(int32_t)(pc.row * hkv + h), pc.start, pc.start + pc.len, n,
                            (int32_t)tbl_off, (int32_t)bt_ids[tbl_off], 0, split});
  }
  // Shared blocks: a block id attended by two planned rows (two rows of one
  // sequence share their prefix blocks too).  One pass over the attended
  // ids with two bitmaps (seen, seen again) that are cleared afterwards;
  // then each work item is flagged when its token range reads a shared
  // block.
  static thread_local std::vector<uint64_t> seen, again;
  bool shared = false;
  size_t w_lo = SIZE_MAX, w_hi = 0;  // words touched (cleared afterwards)
  auto attended = [&](auto&& f) {
    for (int64_t r = 0; r < rows; ++r) {
      if (lens[r] == 0) continue;
      const int64_t o = bt_offsets[row_seq[r]];
      const int64_t nb = ((int64_t)lens[r] + block_size - 1) >> bs_log2;
      for (int64_t j = 0; j < nb; ++j) f(bt_ids[o + j]);
    }
  };
  attended([&](uint32_t id) {
    const size_t w = id >> 6;
    if (w >= seen.size()) seen.resize(w + 1, 0), again.resize(w + 1, 0);
    w_lo = std::min(w_lo, w);
    w_hi = std::max(w_hi, w);
    const uint64_t bit = 1ull << (id & 63);
    if (seen[w] & bit) {
      again[w] |= bit;
      shared = true;
    }
    seen[w] |= bit;
  });
  int64_t shared_items = 0;
  if (shared) {
    // the hkv items of a piece are adjacent and read the same blocks
    for (size_t i = 0; i < plan->work.size(); i += hkv) {
      const DecodeWork& wk = plan->work[i];
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
  if (w_lo <= w_hi) {
    std::fill(seen.begin() + w_lo, seen.begin() + w_hi + 1, 0);
    std::fill(again.begin() + w_lo, again.begin() + w_hi + 1, 0);
  }
  plan->stream_kv = !shared;
  plan->mixed_kv = shared && shared_items < (int64_t)plan->work.size();
}

size_t decode_workspace_bytes(int64_t rows, int64_t hq, int64_t D, int64_t max_splits) {
  if (max_splits <= 1) return 0;
  return (size_t)(rows * hq * max_splits) * (size_t)(D + 2) * sizeof(float);
}

}  // namespace orion
