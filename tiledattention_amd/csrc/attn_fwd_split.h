// Work numbering of the eight-wave kernel's grid (attn_fwd_pp.hip): which query block and
// which key steps a workgroup takes, for the whole-row grid and for split key ranges, and
// which partials the merge kernel combines.  Compiled into the kernels, the host launcher
// (grid sizes, workspace, dispatch model) and a host-only test, so all of them use one
// numbering.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define TA_HD __host__ __device__
#else
#define TA_HD
#endif

namespace ta {

constexpr int kPPRows = 128;  // query rows per block
constexpr int kPPKeys = 128;  // keys per step

// Chunk length that selects the paired split (psplit_items below).
constexpr int kSplitPairs = -1;

TA_HD inline int psplit_cut(int nq, int p, int f) {
  const int x = nq - 2 * p - 1 - f;
  return x >= 2 ? x / 2 : 0;
}

// Pairs with a cut (k_p > 0), the pairs 0 .. P - 1.
TA_HD inline int psplit_cut_pairs(int nq, int f) {
  const int x = nq - 3 - f;
  if (x < 0) return 0;
  const int P = x / 2 + 1;
  return P < (nq >> 1) ? P : (nq >> 1);
}

// Merge kernel workgroup: one thread per (row, 16-byte output chunk), the largest power of
// two of rows whose D / 8 threads each fit 256 (32 rows at D = 64, 16 at D = 128, 8 at
// D = 160 with 160 threads), so a workgroup covers whole rows and a block whole workgroups.
constexpr int merge_rows_per_wg(int d) {
  return d / 8 <= 8 ? 32 : d / 8 <= 16 ? 16 : 8;
}
constexpr int merge_threads(int d) { return merge_rows_per_wg(d) * (d / 8); }

// Split key ranges with chunks of C steps: a query block with `len` key steps is cut
// into ns = ceil(len / C) chunks counted back from its last step (chunk 0 takes the
// remainder), one work item each.  Causal block qt has qt + 1 steps, so blocks
// [a C, (a + 1) C) have a + 1 chunks each; non-causal blocks all have the same ns.
struct SplitLayout {
  int64_t items = 0;  // work items per (b, h)
  int64_t ns = 0;     // chunks per block (non-causal; 0 for causal)
  int64_t slots = 0;  // partial slots per (b, h)
  int64_t merge = 0;  // blocks of more than one chunk per (b, h)
};

// Items of causal blocks [0, x).
TA_HD inline int64_t split_causal_items(int64_t x, int64_t c) {
  const int64_t a = x / c, b = x - a * c;
  return c * a * (a + 1) / 2 + b * (a + 1);
}

// False when chunks of c steps split nothing (every block fits in one chunk).  c =
// kSplitPairs is the paired split (below; causal only) with cut offset f: items = nq
// workgroups, slots = 2 P, merge = P for the P pairs it cuts.
TA_HD inline bool split_layout(int64_t S, bool causal, int64_t c, SplitLayout* out, int f = 0) {
  const int64_t nq = (S + kPPRows - 1) / kPPRows;
  const int64_t len = (S + kPPKeys - 1) / kPPKeys;
  if (c == kSplitPairs) {
    if (!causal || nq > 0x7fffffffLL) return false;
    const int P = psplit_cut_pairs((int)nq, f);
    if (P == 0) return false;
    out->items = nq;
    out->ns = 0;
    out->slots = 2 * (int64_t)P;
    out->merge = P;
    return true;
  }
  if (c < 1) return false;
  if (causal) {
    if (nq <= c) return false;
    out->items = split_causal_items(nq, c);
    out->ns = 0;
    out->slots = out->items - c;  // blocks 0 .. C-1 are one chunk each
    out->merge = nq - c;
  } else {
    const int64_t ns = (len + c - 1) / c;
    if (ns <= 1) return false;
    out->items = nq * ns;
    out->ns = ns;
    out->slots = out->items;
    out->merge = nq;
  }
  return true;
}

// Block id -> (b*h, rank r of the item within its head, 0 = issued first) for a grid of
// n_bh * per_head items with sched >= 1 and a total divisible by 8.  The hardware hands
// block ids to the 8 XCDs round-robin (XCD = id % 8, k-th block of that XCD = id / 8), and
// each XCD runs its blocks in k order on whichever CU frees first:
// * n_bh = 1, 2 or 4: head h gets XCDs [h X, (h + 1) X), X = 8 / n_bh, and its items are
//   dealt out round-robin over them in rank order, so every XCD gets heavy and light items
//   of one head (balanced work, the head's K/V in those XCDs' L2);
// * otherwise each XCD gets a contiguous run of total / 8 items, whole heads when 8 | n_bh.
TA_HD inline void xcd_order(int blk, int n_bh, int per_head, int* bh, int* r) {
  const int total = n_bh * per_head;
  const int x = blk & 7, k = blk >> 3;
  if (n_bh < 8 && (8 % n_bh) == 0) {
    const int X = 8 / n_bh;
    *bh = x / X;
    *r = k * X + (x - *bh * X);
  } else {
    const int lin = x * (total >> 3) + k;
    *bh = lin / per_head;
    *r = lin - *bh * per_head;
  }
}

struct WorkItem {
  int bh;     // b * H + h
  int qt;     // query block
  int t_beg;  // key steps [t_beg, t_end); t_end = -1 for "every step the block needs"
  int t_end;
  int slot;   // partial slot, or -1 when the item is the block's only chunk
  int slot0;  // with slot >= 0: the slot of the block's chunk 0 (chunk i is in slot0 + i),
              // which also names the block among the launch's split blocks
  int ns;     // with slot >= 0: the block's chunk count
};

// Whole-row grid: one item per (b, h, query block).  sched >= 1 (with 8 | total) maps
// block ids per XCD as xcd_order describes; otherwise block ids run head by head.  Causal
// blocks are ranked heaviest (longest key range) first; with sched 2, for grids whose
// workgroups are all resident at once (each CU then holds two, and an XCD fills one slot
// per CU before the next), the heavier half comes first and the lighter half follows from
// the lightest up, so the j-th and (j + nq/2)-th blocks of a head, which share a CU, add up
// to the same work.
TA_HD inline WorkItem whole_item(int blk, int n_bh, int nq, int sched, bool causal) {
  const int total = nq * n_bh;
  WorkItem w;
  int j;
  if (sched >= 1 && (total & 7) == 0) {
    xcd_order(blk, n_bh, nq, &w.bh, &j);
  } else {
    w.bh = blk / nq;
    j = blk - w.bh * nq;
  }
  if (causal) {
    const int half = (nq + 1) >> 1;
    w.qt = (sched == 2 && j >= half) ? j - half : nq - 1 - j;
  } else {
    w.qt = j;
  }
  w.t_beg = 0;
  w.t_end = -1;
  w.slot = -1;
  w.slot0 = -1;
  w.ns = 1;
  return w;
}

// Pair grid (causal whole rows): ceil(nq / 2) items per (b, h); item j of a head covers
// query blocks nq - 1 - j (first) and j, nq + 1 key steps in all, or the middle block alone
// when nq is odd (b->qt = -1 then).  sched >= 1 (with 8 | total) maps block ids per XCD as
// xcd_order describes; otherwise block ids run head by head.
TA_HD inline void pair_items(int blk, int n_bh, int nq, int sched, WorkItem* a, WorkItem* b) {
  const int np = (nq + 1) >> 1;
  int bh, j;
  if (sched >= 1 && ((np * n_bh) & 7) == 0) {
    xcd_order(blk, n_bh, np, &bh, &j);
  } else {
    bh = blk / np;
    j = blk - bh * np;
  }
  a->bh = b->bh = bh;
  a->qt = nq - 1 - j;
  b->qt = j < nq - 1 - j ? j : -1;
  a->t_beg = b->t_beg = 0;
  a->t_end = b->t_end = -1;
  a->slot = b->slot = -1;
  a->slot0 = b->slot0 = -1;
  a->ns = b->ns = 1;
}

// Split grid: `items` per (b, h), ranked from the heaviest block down; sched >= 1 (with
// 8 | total) maps block ids per XCD as xcd_order describes, otherwise block ids run
// item-major across heads (heavy items of every head first).  A block of more than one
// chunk leaves chunk `part` in slot bh * slots + (item - C) (causal) or bh * slots + item
// (non-causal).
TA_HD inline WorkItem split_item(int blk, int n_bh, int items, int sched, bool causal, int c,
                                 int ns_nc, int slots, int S) {
  const int total = items * n_bh;
  int r;
  WorkItem w;
  if (sched >= 1 && (total & 7) == 0) {
    xcd_order(blk, n_bh, items, &w.bh, &r);
  } else {
    r = blk / n_bh;
    w.bh = blk - r * n_bh;
  }
  const int item = items - 1 - r;  // counted from the lightest block up
  int len, ns, part;
  if (causal) {
    int a = 0;
    while (c * (a + 1) * (a + 2) / 2 <= item) ++a;
    const int off = item - c * a * (a + 1) / 2;
    const int q = off / (a + 1);
    w.qt = a * c + q;
    part = off - q * (a + 1);
    ns = a + 1;
    len = w.qt + 1;
    w.slot = item - c;
  } else {
    ns = ns_nc;
    w.qt = item / ns;
    part = item - w.qt * ns;
    len = (S + kPPKeys - 1) / kPPKeys;
    w.slot = item;
  }
  w.t_beg = part == 0 ? 0 : len - (ns - part) * c;
  w.t_end = len - (ns - 1 - part) * c;
  w.slot = ns > 1 ? w.bh * slots + w.slot : -1;
  w.slot0 = ns > 1 ? w.slot - part : -1;
  w.ns = ns;
  return w;
}

// Paired split (chunk length kSplitPairs, causal only): the whole-row grid's nq workgroups
// per (b, h), with the work balanced.  Query blocks p (p + 1 key steps) and nq - 1 - p
// (nq - p steps) share workgroups 2p and 2p + 1: workgroup 2p runs block p whole and then
// the first k_p steps of block nq - 1 - p, workgroup 2p + 1 the remaining steps of block
// nq - 1 - p, so each takes about (nq + 1) / 2 steps where the whole-row grid's heaviest
// workgroup takes nq.  k_p = (nq - 2p - 1 - f) / 2 when positive (f: the fixed cost of a
// workgroup's second block, in key steps, given to the workgroup with one block), else
// the pair is not cut.  A cut block leaves its two chunks in slots 2p and 2p + 1 of its
// head (2 P slots a head for the P pairs that are cut); the middle block of an odd nq is
// one workgroup of its own.
//
// Workgroup blk of the paired-split grid (nq per (b, h); sched >= 1 with 8 | total maps
// block ids per XCD as xcd_order describes): its first item `a` and, on the light block's
// workgroup of a cut pair, the heavy block's first chunk `b` (b->qt = -1 otherwise).
// Every item carries its step range; slot -1 marks a whole block.
TA_HD inline void psplit_items(int blk, int n_bh, int nq, int sched, int f, WorkItem* a,
                               WorkItem* b) {
  int bh, r;
  if (sched >= 1 && ((nq * n_bh) & 7) == 0) {
    xcd_order(blk, n_bh, nq, &bh, &r);
  } else {
    bh = blk / nq;
    r = blk - bh * nq;
  }
  const int P = psplit_cut_pairs(nq, f);
  a->bh = b->bh = bh;
  b->qt = -1;
  b->t_beg = b->t_end = 0;
  b->slot = -1;
  a->slot = -1;
  a->slot0 = b->slot0 = -1;
  a->ns = b->ns = 1;
  const int np = nq >> 1;
  if (r >= 2 * np) {  // the middle block of an odd nq
    a->qt = np;
    a->t_beg = 0;
    a->t_end = np + 1;
    return;
  }
  const int pr = r >> 1;
  const int heavy = nq - 1 - pr;
  const int k = psplit_cut(nq, pr, f);
  if (r & 1) {
    a->qt = heavy;
    a->t_beg = k;
    a->t_end = heavy + 1;
    if (k > 0) {
      a->slot = bh * 2 * P + 2 * pr + 1;
      a->slot0 = a->slot - 1;
      a->ns = 2;
    }
  } else {
    a->qt = pr;
    a->t_beg = 0;
    a->t_end = pr + 1;
    if (k > 0) {
      b->qt = heavy;
      b->t_beg = 0;
      b->t_end = k;
      b->slot = bh * 2 * P + 2 * pr;
      b->slot0 = b->slot;
      b->ns = 2;
    }
  }
}

struct MergeItem {
  int bh;
  int qt;
  int ns;     // chunks
  int slot0;  // slot of chunk 0; chunk i is in slot0 + i
};

// Merge grid of the paired split: one block per (b, h, cut pair p), the heavy block
// nq - 1 - p with its two chunks in slots 2p and 2p + 1 of the head.
TA_HD inline MergeItem psplit_merge_item(int blk, int nq, int f) {
  const int P = psplit_cut_pairs(nq, f);
  MergeItem m;
  m.bh = blk / P;
  const int pr = blk - m.bh * P;
  m.qt = nq - 1 - pr;
  m.ns = 2;
  m.slot0 = m.bh * 2 * P + 2 * pr;
  return m;
}

// Merge grid: one block per (b, h, split query block): causal blocks qt >= C, or every
// non-causal block.
TA_HD inline MergeItem merge_item(int blk, int nq, bool causal, int c, int ns_nc, int slots) {
  const int nsb = causal ? nq - c : nq;
  MergeItem m;
  m.bh = blk / nsb;
  const int idx = blk - m.bh * nsb;
  if (causal) {
    m.qt = c + idx;
    const int a = m.qt / c;
    m.ns = a + 1;
    m.slot0 = (int)split_causal_items(m.qt, c) - c;
  } else {
    m.qt = idx;
    m.ns = ns_nc;
    m.slot0 = m.qt * ns_nc;
  }
  m.slot0 += m.bh * slots;
  return m;
}

}  // namespace ta
