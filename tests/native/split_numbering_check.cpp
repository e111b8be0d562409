// Host-only check of the eight-wave kernel's grid numbering (attn_fwd_split.h): for every
// block id of the whole-row and split grids, over a range of shapes, chunk lengths and
// both issue orders, the items must cover every key step of every (b, h, query block)
// exactly once, partial slots must be unique, in range and used exactly by the blocks of
// more than one chunk, and the merge grid must name exactly those blocks with their
// chunks' slots in key order; the pair grid must cover every query block exactly once with
// nq + 1 key steps an item; the paired split must cover every key step once, within
// (nq + f + 3) / 2 steps a workgroup, and merge exactly its cut blocks.  Prints
// "ok <cases>" or the first failure.
#include <algorithm>
#include <cstdio>
#include <map>
#include <set>
#include <tuple>
#include <vector>

#include "attn_fwd_split.h"

static int fails = 0;
#define CHECK(cond, ...)                                             \
  do {                                                               \
    if (!(cond)) {                                                   \
      if (fails++ < 10) {                                            \
        printf("FAIL %s:%d: %s: ", __FILE__, __LINE__, #cond);       \
        printf(__VA_ARGS__);                                         \
        printf("\n");                                                \
      }                                                              \
    }                                                                \
  } while (0)

static void check_case(int S, int n_bh, bool causal, int c, int sched) {
  const int nq = (S + ta::kPPRows - 1) / ta::kPPRows;
  const int len = (S + ta::kPPKeys - 1) / ta::kPPKeys;
  auto steps_of = [&](int qt) {
    // key steps a query block needs: causal rows stop at the block's last row
    if (!causal) return len;
    const int kv_end = (qt + 1) * ta::kPPRows < S ? (qt + 1) * ta::kPPRows : S;
    return (kv_end + ta::kPPKeys - 1) / ta::kPPKeys;
  };
  ta::SplitLayout l;
  const bool split = ta::split_layout(S, causal, c, &l);
  // whole-row grid
  if (c == 0) {
    std::vector<int> seen((size_t)n_bh * nq, 0);
    for (int blk = 0; blk < n_bh * nq; ++blk) {
      const ta::WorkItem w = ta::whole_item(blk, n_bh, nq, sched, causal);
      CHECK(w.bh >= 0 && w.bh < n_bh && w.qt >= 0 && w.qt < nq, "blk %d", blk);
      if (w.bh >= 0 && w.bh < n_bh && w.qt >= 0 && w.qt < nq) seen[(size_t)w.bh * nq + w.qt]++;
      CHECK(w.slot == -1 && w.t_beg == 0 && w.t_end == -1, "blk %d", blk);
    }
    for (size_t i = 0; i < seen.size(); ++i) CHECK(seen[i] == 1, "S=%d tile %zu seen %d", S, i, seen[i]);
    return;
  }
  if (!split) {
    // no split: every block fits in one chunk
    for (int qt = 0; qt < nq; ++qt) CHECK(steps_of(qt) <= c, "S=%d c=%d qt=%d", S, c, qt);
    return;
  }
  // split grid: coverage of key steps
  std::map<std::pair<int, int>, std::vector<std::tuple<int, int, int>>> chunks;  // (bh,qt) -> (beg,end,slot)
  std::map<std::pair<int, int>, std::pair<int, int>> block_of;  // (bh,qt) -> (slot0, ns) of its chunks
  std::set<int> slots;
  const int total = (int)(n_bh * l.items);
  for (int blk = 0; blk < total; ++blk) {
    const ta::WorkItem w = ta::split_item(blk, n_bh, (int)l.items, sched, causal, c, (int)l.ns,
                                          (int)l.slots, S);
    CHECK(w.bh >= 0 && w.bh < n_bh && w.qt >= 0 && w.qt < nq, "S=%d c=%d blk %d bh %d qt %d", S, c, blk, w.bh, w.qt);
    CHECK(w.t_beg >= 0 && w.t_beg < w.t_end && w.t_end <= steps_of(w.qt) && w.t_end - w.t_beg <= c,
          "S=%d c=%d blk %d [%d,%d) steps %d", S, c, blk, w.t_beg, w.t_end, steps_of(w.qt));
    if (w.slot >= 0) {
      CHECK(w.slot < n_bh * l.slots, "slot %d of %lld", w.slot, (long long)(n_bh * l.slots));
      CHECK(slots.insert(w.slot).second, "slot %d reused", w.slot);
      // the block's chunk-0 slot and chunk count, as the in-kernel merge reads them
      auto ins = block_of.emplace(std::make_pair(w.bh, w.qt), std::make_pair(w.slot0, w.ns));
      const auto& bi = ins.first->second;
      CHECK(bi.first == w.slot0 && bi.second == w.ns, "S=%d c=%d chunk slot0/ns %d/%d vs %d/%d", S, c,
            w.slot0, w.ns, bi.first, bi.second);
      CHECK(w.slot0 <= w.slot && w.slot < w.slot0 + w.ns, "slot %d outside [%d, +%d)", w.slot, w.slot0, w.ns);
    } else {
      CHECK(w.slot0 == -1 && w.ns == 1, "whole block slot0/ns %d/%d", w.slot0, w.ns);
    }
    chunks[{w.bh, w.qt}].emplace_back(w.t_beg, w.t_end, w.slot);
  }
  CHECK((int)chunks.size() == n_bh * nq, "S=%d c=%d blocks %zu of %d", S, c, chunks.size(), n_bh * nq);
  std::map<std::pair<int, int>, std::vector<int>> split_blocks;  // -> slots in key order
  for (auto& kv : chunks) {
    auto v = kv.second;
    std::sort(v.begin(), v.end());
    int at = 0;
    for (auto& t : v) {
      CHECK(std::get<0>(t) == at, "S=%d c=%d bh %d qt %d gap at %d", S, c, kv.first.first, kv.first.second, at);
      at = std::get<1>(t);
    }
    CHECK(at == steps_of(kv.first.second), "S=%d c=%d qt %d ends at %d", S, c, kv.first.second, at);
    if (v.size() == 1) {
      CHECK(std::get<2>(v[0]) == -1, "single chunk with slot %d", std::get<2>(v[0]));
    } else {
      std::vector<int> sl;
      for (auto& t : v) {
        CHECK(std::get<2>(t) >= 0, "chunk of a split block without a slot");
        sl.push_back(std::get<2>(t));
      }
      split_blocks[kv.first] = sl;
    }
  }
  CHECK((int64_t)slots.size() <= n_bh * l.slots, "slots");
  // merge grid
  std::set<std::pair<int, int>> merged;
  for (int blk = 0; blk < n_bh * l.merge; ++blk) {
    const ta::MergeItem m = ta::merge_item(blk, nq, causal, c, (int)l.ns, (int)l.slots);
    auto it = split_blocks.find({m.bh, m.qt});
    CHECK(it != split_blocks.end(), "merge blk %d names unsplit block (%d, %d)", blk, m.bh, m.qt);
    if (it == split_blocks.end()) continue;
    CHECK((int)it->second.size() == m.ns, "merge ns %d vs %zu", m.ns, it->second.size());
    for (int i = 0; i < m.ns && i < (int)it->second.size(); ++i)
      CHECK(it->second[i] == m.slot0 + i, "merge slot %d vs %d", m.slot0 + i, it->second[i]);
    const auto bi = block_of.count({m.bh, m.qt}) ? block_of[{m.bh, m.qt}] : std::make_pair(-2, -2);
    CHECK(bi.first == m.slot0 && bi.second == m.ns, "chunks' slot0/ns %d/%d vs merge %d/%d", bi.first, bi.second,
          m.slot0, m.ns);
    CHECK(merged.insert({m.bh, m.qt}).second, "block merged twice");
  }
  CHECK(merged.size() == split_blocks.size(), "S=%d c=%d merged %zu of %zu", S, c, merged.size(), split_blocks.size());
}

// Pair grid: every (b, h, query block) exactly once over the first and second blocks of
// all items, the first block the heavier one, and every item nq + 1 key steps (the middle
// block of an odd nq alone).
static void check_pairs(int S, int n_bh, int sched) {
  const int nq = (S + ta::kPPRows - 1) / ta::kPPRows;
  const int np = (nq + 1) / 2;
  std::set<std::pair<int, int>> seen;
  for (int blk = 0; blk < n_bh * np; ++blk) {
    ta::WorkItem a, b;
    ta::pair_items(blk, n_bh, nq, sched, &a, &b);
    CHECK(a.bh >= 0 && a.bh < n_bh && a.bh == b.bh, "pair bh %d %d", a.bh, b.bh);
    CHECK(a.qt >= 0 && a.qt < nq, "pair a.qt %d", a.qt);
    CHECK(seen.insert({a.bh, a.qt}).second, "S=%d block (%d, %d) twice", S, a.bh, a.qt);
    if (b.qt >= 0) {
      CHECK(b.qt < a.qt, "second block %d not lighter than %d", b.qt, a.qt);
      CHECK(seen.insert({b.bh, b.qt}).second, "S=%d block (%d, %d) twice", S, b.bh, b.qt);
      CHECK(a.qt + 1 + b.qt + 1 == nq + 1, "pair steps %d + %d", a.qt + 1, b.qt + 1);
    } else {
      CHECK(nq % 2 == 1 && a.qt == nq / 2, "single item qt %d of nq %d", a.qt, nq);
    }
    CHECK(a.t_beg == 0 && a.t_end == -1 && a.slot == -1 && b.t_beg == 0 && b.slot == -1, "pair ranges");
  }
  CHECK((int)seen.size() == n_bh * nq, "S=%d n_bh=%d pairs cover %zu of %d", S, n_bh, seen.size(), n_bh * nq);
}

// Paired split (psplit_items) with cut offset f: every key step of every causal (b, h,
// query block) exactly once, a workgroup's items of one head, at most (nq + f + 3) / 2
// steps a workgroup, slots unique and in range, two chunks (slots 2p and 2p + 1 of the
// head, in key order) exactly for the blocks the merge grid names, one chunk and no slot
// for every other block; the layout agrees (nq items, 2 P slots, P merges).
static void check_psplit(int S, int n_bh, int sched, int f) {
  const int nq = (S + ta::kPPRows - 1) / ta::kPPRows;
  ta::SplitLayout l;
  const bool split = ta::split_layout(S, true, ta::kSplitPairs, &l, f);
  const int P = ta::psplit_cut_pairs(nq, f);
  CHECK(split == (P > 0), "S=%d f=%d layout %d P %d", S, f, split, P);
  ta::SplitLayout lnc;
  CHECK(!ta::split_layout(S, false, ta::kSplitPairs, &lnc, f), "non-causal paired layout");
  if (split) CHECK(l.items == nq && l.slots == 2 * P && l.merge == P, "S=%d layout", S);
  std::map<std::pair<int, int>, std::vector<std::tuple<int, int, int>>> chunks;
  std::set<int> slots;
  std::map<std::pair<int, int>, std::set<int>> ps_slot0;  // (bh,qt) -> slot0 of its chunks
  for (int blk = 0; blk < n_bh * nq; ++blk) {
    ta::WorkItem it[2];
    ta::psplit_items(blk, n_bh, nq, sched, f, &it[0], &it[1]);
    int steps = 0;
    for (int i = 0; i < 2; ++i) {
      const ta::WorkItem& w = it[i];
      if (i == 1 && w.qt < 0) break;
      CHECK(w.bh >= 0 && w.bh < n_bh && w.qt >= 0 && w.qt < nq, "S=%d blk %d bh %d qt %d", S, blk, w.bh, w.qt);
      if (!(w.bh >= 0 && w.bh < n_bh && w.qt >= 0 && w.qt < nq)) return;
      CHECK(w.bh == it[0].bh, "one head a workgroup");
      CHECK(w.t_beg >= 0 && w.t_beg < w.t_end && w.t_end <= w.qt + 1, "S=%d blk %d [%d,%d) qt %d", S,
            blk, w.t_beg, w.t_end, w.qt);
      steps += w.t_end - w.t_beg;
      if (w.slot >= 0) {
        CHECK(w.slot < n_bh * 2 * P, "slot %d of %d", w.slot, n_bh * 2 * P);
        CHECK(slots.insert(w.slot).second, "slot %d reused", w.slot);
        CHECK(w.ns == 2 && (w.slot == w.slot0 || w.slot == w.slot0 + 1), "psplit slot0/ns %d/%d slot %d", w.slot0,
              w.ns, w.slot);
        ps_slot0[{w.bh, w.qt}].insert(w.slot0);
      } else {
        CHECK(w.slot0 == -1 && w.ns == 1, "psplit whole block slot0/ns %d/%d", w.slot0, w.ns);
      }
      chunks[{w.bh, w.qt}].emplace_back(w.t_beg, w.t_end, w.slot);
    }
    CHECK(2 * steps <= nq + f + 3, "S=%d f=%d blk %d: %d steps of nq %d", S, f, blk, steps, nq);
  }
  CHECK((int)chunks.size() == n_bh * nq, "S=%d blocks %zu of %d", S, chunks.size(), n_bh * nq);
  std::map<std::pair<int, int>, std::vector<int>> cut;
  for (auto& kv : chunks) {
    auto v = kv.second;
    std::sort(v.begin(), v.end());
    int at = 0;
    for (auto& t : v) {
      CHECK(std::get<0>(t) == at, "S=%d bh %d qt %d gap at %d", S, kv.first.first, kv.first.second, at);
      at = std::get<1>(t);
    }
    CHECK(at == kv.first.second + 1, "S=%d qt %d ends at %d", S, kv.first.second, at);
    if (v.size() == 1) {
      CHECK(std::get<2>(v[0]) == -1, "whole block with slot %d", std::get<2>(v[0]));
    } else {
      CHECK(v.size() == 2, "paired split block in %zu chunks", v.size());
      cut[kv.first] = {std::get<2>(v[0]), std::get<2>(v[1])};
    }
  }
  std::set<std::pair<int, int>> merged;
  for (int blk = 0; blk < n_bh * P; ++blk) {
    const ta::MergeItem m = ta::psplit_merge_item(blk, nq, f);
    auto itc = cut.find({m.bh, m.qt});
    CHECK(itc != cut.end(), "merge blk %d names uncut block (%d, %d)", blk, m.bh, m.qt);
    if (itc == cut.end()) continue;
    CHECK(m.ns == 2 && itc->second[0] == m.slot0 && itc->second[1] == m.slot0 + 1,
          "merge slots %d vs %d %d", m.slot0, itc->second[0], itc->second[1]);
    const auto& s0 = ps_slot0[{m.bh, m.qt}];
    CHECK(s0.size() == 1 && *s0.begin() == m.slot0, "psplit chunks' slot0 vs merge %d", m.slot0);
    CHECK(merged.insert({m.bh, m.qt}).second, "block merged twice");
  }
  CHECK(merged.size() == cut.size(), "S=%d f=%d merged %zu of %zu", S, f, merged.size(), cut.size());
}

int main() {
  int cases = 0;
  const int seqs[] = {1, 100, 128, 129, 255, 256, 300, 1000, 1024, 2048, 2100, 4096, 8192, 16384};
  const int bhs[] = {1, 2, 3, 4, 6, 8, 16};
  for (int S : seqs)
    for (int n_bh : bhs)
      for (int causal = 0; causal < 2; ++causal)
        for (int sched = 0; sched < 3; ++sched) {
          const int len = (S + 127) / 128;
          for (int c = 0; c <= len + 1; c += (c < 8 ? 1 : 1 + c / 4)) {
            check_case(S, n_bh, causal != 0, c, sched);
            ++cases;
          }
        }
  for (int S : seqs)
    for (int n_bh : bhs)
      for (int sched = 0; sched < 4; ++sched) {
        if (S > 128) check_pairs(S, n_bh, sched);
        ++cases;
      }
  for (int n_bh = 1; n_bh <= 40; ++n_bh)
    for (int nq = 2; nq <= 70; ++nq) {
      check_pairs(nq * 128 - 5, n_bh, 1);
      ++cases;
    }
  for (int S : seqs)
    for (int n_bh : bhs)
      for (int sched = 0; sched < 3; ++sched)
        for (int f = 0; f <= 8; ++f) {
          check_psplit(S, n_bh, sched, f);
          ++cases;
        }
  for (int n_bh = 1; n_bh <= 12; ++n_bh)
    for (int nq = 1; nq <= 70; ++nq) {
      check_psplit(nq * 128 - 5, n_bh, 1, 4);
      check_psplit(nq * 128, n_bh, 1, 0);
      cases += 2;
    }
  if (fails) {
    printf("%d failures\n", fails);
    return 1;
  }
  printf("ok %d\n", cases);
  return 0;
}
