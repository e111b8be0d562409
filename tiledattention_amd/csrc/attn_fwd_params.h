// Kernel argument block shared by the HIP kernels and the host launcher.
// Plain C layout: it is passed by value as the kernels' only argument.
#pragma once
#include <stdint.h>

namespace ta {

struct FwdParams {
  const uint16_t* q;  // [B,H,S,D] fp16/bf16 bit patterns, last-dim stride 1
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t q_sb, q_sh, q_ss;  // element strides of batch, head, sequence
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int32_t H;
  int32_t S;
  int32_t n_qblk;      // ceil(S / TILE_M)
  int32_t n_bh;        // B * H
  float scale_log2;    // softmax scale * log2(e)
  int32_t sched;       // block -> tile order: 0 plain, 1 XCD-grouped
  // Split key ranges (split kernels and the merge kernel only; see SplitLayout).
  float* part_o;       // [slots][128][D] fp32 partial outputs, each normalised by its own l
  float* part_lse;     // [slots][128] log2 of the partial's softmax denominator, m*c + log2(l)
  int32_t split_c;     // key steps (of 128 keys) per chunk, or kSplitPairs (paired split)
  int32_t split_items; // work items per (b, h)
  int32_t split_ns;    // chunks per query block (non-causal; causal derives it per block);
                       // the cut offset f of the paired split
  int32_t split_slots; // partial slots per (b, h)
  int32_t d_real;      // head-dim columns present in q/k/v/o (eight-wave kernel; <= D,
                       // multiple of 8): columns d_real..D-1 read as zero, are not written
  int32_t pad0;
  // Split launches merged in the kernel: arrival counters of this launch's split blocks
  // (counter slot0 of a block, see WorkItem), zero on entry and left zero; null when a
  // merge kernel follows instead.
  unsigned* merge_cnt;
};

// In-kernel merge counters (attn_fwd_pp.hip's ta_merge_counters): kMergeRegions regions of
// kMergeRegionCounters, one region per stream that launches split work, so launches that
// may overlap never share counters.
constexpr int kMergeRegions = 16;
constexpr int kMergeRegionCounters = 16384;

}  // namespace ta
