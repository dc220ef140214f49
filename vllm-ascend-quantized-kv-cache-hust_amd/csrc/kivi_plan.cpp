// SPDX-License-Identifier: Apache-2.0
// Host-side work planning for the fused KIVI INT4 decode (no GPU code).
//
// The decode kernel takes a work list -- items of (request, position range,
// kind) -- and optionally "pieces", runs of consecutive items that one wave
// per (piece, kv head) walks in a single pass.  This file builds both from
// each request's decode geometry, the part of the reference's decode step
// (pkg/methods/kivi_int4/attention_backend.py:1193-1230) that decides which
// positions read int4 pages and which read the residual window.  It runs on
// the host every decode step and every layer, so it is native code: a
// config-3 batch (32 requests, ~300 items) plans in a few microseconds.
//
// Request geometry, int32 [batch, 6]:
//   {seq_len, k_hist, v_hist, ring_row, k_first_lane, v_first_lane}
// Output seq_meta, int32 [batch, 8]: the geometry plus {first_work, num_work}.
// Work items, int32 [num_work, 4]: {request, pos_begin, pos_end, kind}
//   kind 0: both sides int4; kind 1: the mixed-source tail (64 positions per
//   item in split plans); kinds 2 / 3: the even / odd 64-position chunks of
//   an int4 range, issued as a pair at indices 2P, 2P + 1.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "kvq_hip.h"

namespace {

// (piece, kv head) slots per CU: the decode kernel keeps 8 waves resident per
// CU, one per (piece, kv head) (8 / kDecodeWavesPerHead of decode_mfma.hip)
constexpr int kHeadSlotsPerCu = 8;
constexpr double kPieceMaxCost = 4096;  // int4 positions per piece before a second round
constexpr int kTailItemTokens = 64;     // positions per tail item in split plans
// One-round page-streaming plans run two workgroups per CU, and the first
// half of the pieces are the first workgroup dispatched to each CU.  While
// both run, the SIMD arbiter issues the older workgroup's waves first, so
// those pieces stream faster (config 3 on MI355X with equal pieces: about 5.3
// against 6.8 us per page); they get this much more cost per piece, so that both workgroups of a
// CU finish together instead of the younger one streaming alone, at half the
// CU's requests in flight, at the end.
constexpr double kFirstWaveShare = 1.4;

struct Planner {
  const int32_t* seqs;
  int64_t batch;
  int32_t* meta;
  int32_t* work;
  int64_t cap_work;
  int64_t n = 0;
  bool overflow = false;

  int64_t hist_both(int64_t b) const {
    const int32_t* s = seqs + 6 * b;
    return std::max<int64_t>(0, std::min({s[1], s[2], s[0]}));
  }
  void add(int64_t b, int64_t p, int64_t e, int kind) {
    if (n >= cap_work) {
      overflow = true;
      return;
    }
    int32_t* w = work + 4 * n++;
    w[0] = static_cast<int32_t>(b);
    w[1] = static_cast<int32_t>(p);
    w[2] = static_cast<int32_t>(e);
    w[3] = kind;
  }
  void close(int64_t b, int64_t first) {
    const int32_t* s = seqs + 6 * b;
    int32_t* m = meta + 8 * b;
    for (int i = 0; i < 6; ++i) m[i] = s[i];
    m[6] = static_cast<int32_t>(first);
    m[7] = static_cast<int32_t>(n - first);
  }
};

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int64_t slots_for(int kvh, int cu_count) {
  return std::max<int64_t>(1, static_cast<int64_t>(cu_count) * kHeadSlotsPerCu / std::max(1, kvh));
}

// Cost of the whole batch in int4-position units: int4 ranges in `tile`-position
// tiles, tail positions at `tail_cost` each.
double total_cost(const Planner& pl, double tail_cost, int64_t tile = 64) {
  double total = 0;
  for (int64_t b = 0; b < pl.batch; ++b) {
    const int64_t end_a = pl.hist_both(b);
    total += static_cast<double>(ceil_div(end_a, tile) * tile) +
             static_cast<double>(pl.seqs[6 * b] - end_a) * tail_cost;
  }
  return total;
}

// Fixed split: int4 ranges every `split` positions (paired: two items per
// range of 2 * split, kinds 2 and 3), then tail items of 64 positions.
void plan_split(Planner& pl, int64_t split, bool paired) {
  split = std::max<int64_t>(128, ceil_div(split, 128) * 128);
  for (int64_t b = 0; b < pl.batch; ++b) {
    const int64_t first = pl.n;
    const int64_t seq_len = pl.seqs[6 * b];
    const int64_t end_a = pl.hist_both(b);
    if (paired && end_a > 0 && pl.n % 2) pl.add(b, 0, 0, 1);  // pairs start at even indices
    for (int64_t p = 0; p < end_a;) {
      if (paired) {
        const int64_t e = std::min(end_a, p + 2 * split);
        pl.add(b, p, e, 2);
        pl.add(b, p, e, 3);
        p = e;
      } else {
        const int64_t e = std::min(end_a, p + split);
        pl.add(b, p, e, 0);
        p = e;
      }
    }
    for (int64_t p = end_a; p < seq_len;) {
      const int64_t e = std::min(seq_len, p + kTailItemTokens);
      pl.add(b, p, e, 1);
      p = e;
    }
    if (seq_len == 0) pl.add(b, 0, 0, 1);
    pl.close(b, first);
  }
}

// Cost-balanced pieces: every request's positions laid end to end (int4 in
// `tile`-position tiles -- 64, or 128 for the page-streaming kernel, whose
// workgroups must not share a page -- tail in 32-position steps at `tail_cost`
// per position), cut where the running cost crosses a multiple of total / slots
// (one-round page-streaming plans: kFirstWaveShare times that for the first
// half; several rounds: the last round in pieces of half that).
int64_t plan_pieces(Planner& pl, int kvh, int cu_count, double tail_cost, int64_t tile,
                    int32_t* pieces, int64_t cap_pieces) {
  const int64_t per_round = slots_for(kvh, cu_count);
  const double total = total_cost(pl, tail_cost, tile);
  const int64_t rounds = std::max<int64_t>(
      1, static_cast<int64_t>(std::ceil(total / (static_cast<double>(per_round) * kPieceMaxCost))));
  int64_t slots = per_round * rounds;
  const double dtile = static_cast<double>(tile);
  const double step = std::max(dtile, total / static_cast<double>(slots));
  // Page-streaming plans of several rounds: the hardware hands the pieces to
  // CUs as earlier ones finish, so the last pieces to start set the end; the
  // last round is cut into twice as many pieces of half the cost, which halves
  // the spread of those last starts and ends.
  const bool split_last = tile == 128 && rounds >= 2 && step >= 8 * dtile;
  const int64_t full = split_last ? per_round * (rounds - 1) : slots;
  if (split_last) slots = full + 2 * per_round;
  // the page-streaming kernel's single round: pieces [0, slots / 2) are the
  // first workgroups on their CUs (two per CU, slots == CUs)
  const bool skew = tile == 128 && rounds == 1 && slots == cu_count && slots >= 2 &&
                    total / static_cast<double>(slots) >= 4 * dtile;
  const int64_t first = slots / 2;
  const double share_unit =
      total / (kFirstWaveShare * static_cast<double>(first) + static_cast<double>(slots - first));
  // cumulative cost at the end of piece j
  auto target = [&](int64_t j) -> double {
    if (split_last && j >= full)
      return step * static_cast<double>(full) + 0.5 * step * static_cast<double>(j + 1 - full);
    if (!skew) return step * static_cast<double>(j + 1);
    return j < first ? share_unit * kFirstWaveShare * static_cast<double>(j + 1)
                     : share_unit * (kFirstWaveShare * static_cast<double>(first) +
                                     static_cast<double>(j + 1 - first));
  };
  int64_t np = 0;
  auto push = [&](int64_t v) {
    if (np >= cap_pieces + 1) {
      pl.overflow = true;
      return;
    }
    pieces[np++] = static_cast<int32_t>(v);
  };
  push(0);
  int64_t cut_j = 0;
  double cum = 0.0, cut = target(0);
  // close the piece once the running cost reaches the cut
  auto after = [&](double unit) {
    if (cum >= cut - unit / 2 && np < slots && pl.n > pieces[np - 1]) {
      push(pl.n);
      while (cut - unit / 2 <= cum) cut = target(++cut_j);
    }
  };
  for (int64_t b = 0; b < pl.batch && !pl.overflow; ++b) {
    const int64_t first = pl.n;
    const int64_t seq_len = pl.seqs[6 * b];
    const int64_t end_a = pl.hist_both(b);
    for (int64_t p = 0; p < end_a;) {
      const int64_t tiles =
          std::max<int64_t>(1, static_cast<int64_t>((cut - cum) / dtile + 0.5));
      const int64_t e = std::min(end_a, p + tile * tiles);
      pl.add(b, p, e, 0);
      cum += static_cast<double>(ceil_div(e - p, tile) * tile);
      p = e;
      after(dtile);
    }
    const double unit = 32 * tail_cost;
    for (int64_t p = end_a; p < seq_len;) {
      const int64_t k = std::max<int64_t>(1, static_cast<int64_t>((cut - cum) / unit + 0.5)) * 32;
      const int64_t e = std::min(seq_len, p + k);
      pl.add(b, p, e, 1);
      cum += static_cast<double>(e - p) * tail_cost;
      p = e;
      after(unit);
    }
    if (seq_len == 0) pl.add(b, 0, 0, 1);
    pl.close(b, first);
  }
  if (pl.n > pieces[np - 1]) push(pl.n);
  return np - 1;
}

}  // namespace

extern "C" int64_t kvq_plan_kivi_decode(const int32_t* seqs, int64_t batch, int num_kv_heads,
                                        int cu_count, int mode, int64_t split_tokens,
                                        double tail_cost, int32_t* seq_meta, int32_t* work,
                                        int64_t cap_work, int32_t* pieces, int64_t cap_pieces,
                                        int64_t* num_pieces) {
  if (batch < 0 || (batch > 0 && (!seqs || !seq_meta || !work)) || !num_pieces ||
      num_kv_heads <= 0 || cu_count <= 0 || cap_work < 0 || tail_cost <= 0)
    return KVQ_ERR_INVALID;
  *num_pieces = 0;
  Planner pl{seqs, batch, seq_meta, work, cap_work};
  if (mode == KVQ_PLAN_DEFAULT) {
    const int64_t slots = slots_for(num_kv_heads, cu_count);
    if (total_cost(pl, tail_cost) <= static_cast<double>(slots) * kPieceMaxCost) {
      mode = KVQ_PLAN_PIECES;
    } else {
      // items of up to 8192 positions
      int64_t positions = 0;
      for (int64_t b = 0; b < batch; ++b) positions += seqs[6 * b];
      const int64_t per_item = ceil_div(ceil_div(positions, slots), 128) * 128;
      split_tokens = std::min<int64_t>(8192, std::max<int64_t>(256, per_item));
      mode = KVQ_PLAN_SPLIT;
    }
  }
  switch (mode) {
    case KVQ_PLAN_PIECES: {
      // split_tokens, when given, is the int4 tile: 64 or 128 positions
      const int64_t tile = split_tokens > 0 ? split_tokens : 64;
      if (!pieces || cap_pieces <= 0 || (tile != 64 && tile != 128)) return KVQ_ERR_INVALID;
      *num_pieces = plan_pieces(pl, num_kv_heads, cu_count, tail_cost, tile, pieces, cap_pieces);
      break;
    }
    case KVQ_PLAN_SPLIT:
    case KVQ_PLAN_SPLIT_PAIRED:
      if (split_tokens <= 0) return KVQ_ERR_INVALID;
      plan_split(pl, split_tokens, mode == KVQ_PLAN_SPLIT_PAIRED);
      break;
    default:
      return KVQ_ERR_INVALID;
  }
  if (pl.overflow) return KVQ_ERR_CAPACITY;
  return pl.n;
}

// Host checks of one decode step, in one pass over the step's metadata (the
// Python forms are check_gather_metadata_host and
// KiviResidualRing.suspect_rows; this one runs per step on the fast path).
extern "C" int64_t kvq_kivi_step_check(const int64_t* table, int64_t batch, int64_t max_blocks,
                                       const int64_t* seq_lens, int64_t num_blocks,
                                       int64_t block_size, const int64_t* rows,
                                       const int64_t* k_slot, const int64_t* k_pos,
                                       const int64_t* v_slot, const int64_t* v_pos,
                                       int64_t ring_rows, int64_t ring_len, int32_t* suspect,
                                       int32_t* kind) {
  if (batch < 0 || max_blocks < 0 || block_size <= 0 || ring_len < 0 || !kind) return KVQ_ERR_INVALID;
  *kind = 0;
  if (batch == 0) return 0;
  if (!table || !seq_lens || !rows || !suspect) return KVQ_ERR_INVALID;
  // coverage of the longest sequence
  int64_t longest = 0;
  for (int64_t i = 0; i < batch; ++i) longest = seq_lens[i] > longest ? seq_lens[i] : longest;
  if (longest > max_blocks * block_size) {
    *kind = 3;
    return 0;
  }
  // live block ids: the first request with a bad one, negative before too large
  for (int64_t i = 0; i < batch; ++i) {
    const int64_t live = seq_lens[i] > 0 ? (seq_lens[i] + block_size - 1) / block_size : 0;
    bool neg = false, out = false;
    for (int64_t c = 0; c < live; ++c) {
      const int64_t b = table[i * max_blocks + c];
      neg |= b < 0;
      out |= b >= num_blocks;
    }
    if (neg || out) {
      *kind = neg ? 1 : 2;
      return i;
    }
  }
  // window entries that may no longer be live: an entry at position p with
  // slot s is live when p < seq_len and the table still has s's block at
  // column p / block_size
  const int64_t* slots[2] = {k_slot, v_slot};
  const int64_t* poss[2] = {k_pos, v_pos};
  for (int64_t i = 0; i < batch; ++i) {
    suspect[i] = 0;
    const int64_t row = rows[i];
    if (row < 0) continue;
    if (row >= ring_rows || !k_slot || !k_pos || !v_slot || !v_pos) return KVQ_ERR_INVALID;
    for (int side = 0; side < 2 && !suspect[i]; ++side) {
      const int64_t* ls = slots[side] + row * ring_len;
      const int64_t* lp = poss[side] + row * ring_len;
      for (int64_t lane = 0; lane < ring_len; ++lane) {
        if (ls[lane] < 0) continue;
        const int64_t p = lp[lane];
        bool ok = p >= 0 && p < seq_lens[i] && p / block_size < max_blocks;
        if (ok) ok = table[i * max_blocks + p / block_size] == ls[lane] / block_size;
        if (!ok) {
          suspect[i] = 1;
          break;
        }
      }
    }
  }
  return 0;
}
