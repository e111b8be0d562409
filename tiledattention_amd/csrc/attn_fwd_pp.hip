// SDPA forward for CDNA4 (gfx950), fp32 accumulation, 128 query rows per workgroup:
// eight waves in a barrier-locked ping-pong.
//
// Math: the reference's tiled forward with fp32 accumulation
// (src/tiledattention/kernels/flash_fwd.py:374-446, unmasked form :533-574): per query row
// keep (m, l, acc), stream key tiles, finish with acc / l.  Schedule and layout are this
// file's own:
//
// * Waves w and w + 4 of the workgroup share a SIMD and the same 32 query rows
//   (row block w % 4).  The workgroup walks the keys in steps of 128; in each step wave
//   group 0 (waves 0-3) takes the first 64 keys and group 1 (waves 4-7) the last 64.  Each
//   wave keeps its own online-softmax state over its keys; the two states of a row block
//   are merged through LDS at the end (m = max, weights 2^((m_g - m) * c)).
// * Each wave alternates two clusters: the MFMA cluster (S of the next step,
//   S^T = K Q^T, and O^T += V^T P^T of the current one) and the VALU cluster (mask, row
//   max, rescale, exp, pack of P).  Group 1 runs one cluster behind group 0 and every
//   cluster ends at a workgroup barrier, so on every SIMD one wave issues MFMAs while the
//   other does the softmax arithmetic of its own step.
// * K/V go HBM -> LDS directly (buffer loads with the LDS-write form, 16 bytes a lane,
//   1 KiB a wave instruction), two stages each, with 16-byte chunks XOR-swizzled per row so
//   the K reads (b128) and the transposed V reads (ds_read_b64_tr_b16) are free of bank
//   conflicts.  Each wave group loads and reads only its own 64-key halves of the stages;
//   a group's loads for the next step but one are spread over its MFMA cluster and waited
//   for at the end of its next softmax cluster.
// * Operand layouts are those of the 128 x 64 kernel (attn_fwd.hip): scores transposed so
//   a lane owns one query, row reductions in-lane plus v_permlane32_swap, P packed from the
//   score registers straight into the B operand of the P.V MFMA, exp2 with scale*log2(e)
//   folded into one FMA, lazy rescale of O with a 2^15 threshold, l summed from the rounded
//   P.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_fwd_common.h"
#include "attn_fwd_params.h"
#include "attn_fwd_split.h"


namespace ta {

// Stage size of the eight-wave kernel at head dim D: 128 key rows of 2 D bytes.
constexpr int pp_stage_bytes(int d) { return kPPKeys * 2 * d; }

// Partials of split blocks (part_o, part_lse) are written and, by the in-kernel merge,
// read with agent-scope cache policy (SC1: the form the compiler gives agent-scope atomic
// stores and loads), through a buffer resource over the workspace.  Such a store is
// visible to SC1 loads on every CU, whatever its XCD, once it has completed (vmcnt), so the
// merge needs no flush or invalidation of the L2 (agent-scope fences cost 8-9 us a launch
// at C3 S = 4096).  The workspace of an in-kernel merge is below 2^31 bytes (at most
// kMergeRegionCounters slots of 128 rows of D <= 160 floats).
constexpr int kAgentScope = 16;  // cache policy bit SC1
__device__ inline __amdgpu_buffer_rsrc_t partial_rsrc(const FwdParams& p) {
  return __builtin_amdgcn_make_buffer_rsrc(p.part_o, (short)0, 0x7fffffff, 0x00020000);
}
__device__ inline int partial_offset(const FwdParams& p, const float* at) {
  return (int)((const char*)at - (const char*)p.part_o);
}
// (A launch followed by the merge kernel stores plainly: its workspace may exceed 2^31
// bytes, and the kernel boundary makes the stores visible.)
__device__ inline void store_partial(const FwdParams& p, float* at, f32x4 v) {
  if (p.merge_cnt == nullptr) {
    *(f32x4*)at = v;
    return;
  }
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), partial_rsrc(p), partial_offset(p, at), 0,
                                         kAgentScope);
}
__device__ inline void store_partial(const FwdParams& p, float* at, float v) {
  if (p.merge_cnt == nullptr) {
    *at = v;
    return;
  }
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), partial_rsrc(p), partial_offset(p, at), 0, kAgentScope);
}
__device__ inline f32x4 load_partial4(const FwdParams& p, const float* at) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(partial_rsrc(p), partial_offset(p, at), 0,
                                                                         kAgentScope));
}
__device__ inline float load_partial(const FwdParams& p, const float* at) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(partial_rsrc(p), partial_offset(p, at), 0, kAgentScope));
}

// One query block (or, with SPLIT, one chunk of its key steps) on the whole workgroup: the
// prologue, the key loop and the merge of the key slices with the output stores.  TMR is
// the block's query rows: 128 (four 32-row blocks; a wave group's four waves take one row
// block each and the group's 64 keys of every step), or 64 (two row blocks; a group's
// waves are two row blocks x two 32-key slots, so four waves share each row block).
// LOWP: input-dtype accumulation (the reference's flash_fwd.py:301-372): every step of a
// wave takes the exact running max, l sums the unrounded P in fp32, and O is rounded to the
// input dtype once per TILE_N keys of the wave's key slice (kLowpSteps steps),
// rnd((acc + P.V) rnd(alpha)), the P.V products accumulated onto the rounded acc in fp32
// by the MFMAs.  The
// key slices of a row (each accumulated that way) are combined in fp32 at the end, rounded
// to the input dtype, and multiplied by rnd(1/l) (one more rounding).
template <int DT, int D, bool CAUSAL, bool TAIL, bool SPLIT, int TMR = 128, int LOWP_TN = 0>
__device__ __forceinline__ void attn_fwd_pp_block(const FwdParams& p, const WorkItem wi, char* lds_k0,
                                                  char* lds_k1, char* lds_v0, char* lds_v1) {
  constexpr int TM = TMR;            // query rows per workgroup
  constexpr int TK = 128;            // keys per workgroup step (64 per wave group)
  // 256 rows (non-causal whole rows): the two groups own different rows, 128 each, and every
  // wave takes all 128 keys of a step (64 MFMAs a cluster, 64 scores a lane).
  constexpr bool R256 = TMR == 256;
  constexpr int NRB = R256 ? 4 : TM / 32;   // 32-row blocks of a group
  constexpr int NKS = R256 ? 1 : 4 / NRB;   // key slots of a group's 64 keys (1 or 2)
  constexpr int KB = R256 ? 4 : 2 / NKS;    // 32-key blocks per wave per step
  // A stage holds 128 key rows: the first DA columns of each row in a main part (rows of
  // 2 DA bytes; DA = 128 at D = 160, 64 at D = 96, D otherwise), the rest (32 columns at
  // D = 96 and 160) in a tail part of 64-byte rows behind it, so both parts have
  // power-of-two rows.
  constexpr int DA = D > 128 ? 128 : D == 96 ? 64 : D;
  constexpr int DT2 = D - DA;        // tail columns
  static_assert(DT2 == 0 || DT2 == 32, "head dims 64, 96, 128 and 160");
  constexpr int DK = D / 16;         // k-steps of the QK^T product
  constexpr int DKA = DA / 16;       // ... whose K operand is in the main part
  constexpr int DB = D / 32;         // 32-wide d blocks of O
  constexpr int DBA = DA / 32;       // ... whose V operand is in the main part
  constexpr int CPR = DA / 8;        // 16-byte chunks per main-part row
  constexpr int RB = 2 * DA;         // bytes per main-part row
  constexpr int RBT = 2 * DT2;       // bytes per tail row
  constexpr int STAGE_A = TK * RB;   // bytes of a stage's main part
  constexpr int STAGE = TK * (RB + RBT);  // bytes of one K or V stage
  constexpr int RPL = 1024 / RB;     // main-part rows one wave instruction fills
  constexpr int NLD = STAGE_A / 1024 / 8;  // main-part loads per wave per tensor per step
  constexpr int NLDT = DT2 ? 1 : 0;  // tail loads (a group's 64 tail rows are 4 KiB)
  constexpr int NLDS = NLD + NLDT;   // loads per wave per tensor per step (own half)
  static_assert(STAGE_A % (8 * 1024) == 0, "stage must split over the eight waves");
  static_assert(TK == kPPKeys && (TM == kPPRows || TM == 64 || R256),
                "steps of 128 keys, blocks of 64, 128 or 256 rows");
  static_assert(!R256 || (!CAUSAL && !SPLIT && LOWP_TN == 0 && (D == 64 || D == 128)),
                "256-row blocks: non-causal whole rows, fp32 accumulation, D 64 or 128");
  static_assert(TM != 64 || D == 64 || D == 96 || D == 128 || D == 160, "64-row blocks: D 64, 96, 128 or 160");
  constexpr bool LOWP = LOWP_TN != 0;
  static_assert(!LOWP || (!SPLIT && (D == 64 || D == 128)), "input-dtype accumulation: whole rows, D 64 or 128");
  // Input-dtype accumulation: key steps between roundings of a wave's O, TILE_N keys of its
  // key slice (64 keys a step with 128-row blocks, 32 with 64-row ones).
  constexpr int kLowpSteps = LOWP ? LOWP_TN / (TMR == 128 ? 64 : 32) : 1;
  static_assert(!LOWP || (kLowpSteps >= 1 && kLowpSteps <= 4), "TILE_N 64 or 128");
  // Raised MFMA-cluster priority only in the kernels built for two workgroups per CU (the
  // non-causal D = 64 whole-row ones, TA_PP_WAVES below).
  constexpr bool kPrioMfma = !SPLIT && D == 64 && !CAUSAL && !R256;
  // Those kernels have 128 VGPRs a lane (four waves per SIMD): P is formed two scores at a
  // time there, since a phased softmax holds 32 exponent arguments beside the 32 scores.
  constexpr bool kPhasedP = !kPrioMfma && !R256;  // R256: 64 scores a lane, no room for 64 more
  using DTy = DType<DT>;
  // P.V MFMAs of a cluster issued after its closing barrier, in the wave's softmax phase
  // (operands read in the cluster, held in registers): the 128-row input-dtype kernels, 3
  // (C4 D = 128 -1.8 to -2.4 %, D = 64 -2 %, against the one the compiler moves there;
  // 5 measured slower).  The other kernels leave it to the compiler (see barrier below).
  constexpr int kLateMfma = TM == 128 && LOWP ? 3 : 0;

  static_assert(STAGE == pp_stage_bytes(D), "stage layout");

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps it in SGPRs
  const int grp = wave >> 2;  // key half of every step
  const int wr = wave & 3;    // wave within its group
  const int rb = wr % NRB;    // row block
  const int ks = wr / NRB;    // key slot within the group's 64 keys of a step
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // ---- the work item: (bh, q tile, key steps) -----------------------------------------
  const int S = p.S;
  const int bh = wi.bh;
  const int qt = wi.qt;
  const int t_beg = wi.t_beg;
  const int slot = wi.slot;
  const int b = bh / p.H;
  const int h = bh - b * p.H;

  const uint16_t* __restrict__ qp = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* __restrict__ kp = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* __restrict__ vp = p.v + b * p.v_sb + h * p.v_sh;
  uint16_t* __restrict__ op = p.o + b * p.o_sb + h * p.o_sh;
  const int k_rb = (int)p.k_ss * 2;  // global row bytes
  const int v_rb = (int)p.v_ss * 2;

  const int q0 = qt * TM;
  const int wq0 = R256 ? q0 + 128 * grp + 32 * wr : q0 + rb * 32;  // first query row of this wave
  const int my_q = wq0 + l32;    // this lane's query row

  // ---- Q fragment: B operand of S^T = K Q^T, kept for the whole key loop ------------
  // (staged through LDS in the prologue, below)
  u32x4 qf[DK];
  // Columns at or past d_real (a head dim narrower than the kernel's) are zero.
  const int d_real = p.d_real;

  // ---- key range --------------------------------------------------------------------
  // Steps [t_beg, t_end) of TK keys; without a split, every step up to the last key the
  // block needs.
  const int t_end = SPLIT ? wi.t_end : ((CAUSAL ? min(S, q0 + TM) : S) + TK - 1) / TK;
  const int wave_kv_end = CAUSAL ? min(S, wq0 + 32) : S;
  const int gkoff = 64 * grp;              // the group's keys in a step: [TK t + gkoff, + 64)
  const int koff = R256 ? 0 : gkoff + 32 * KB * ks;   // this wave's: [TK t + koff, + 32 KB)

  // ---- staging: HBM -> LDS directly -------------------------------------------------
  // A stage is 1 KiB chunks g; lane l of the wave instruction that fills chunk g writes
  // physical chunk l % CPR of row g * RPL + l / CPR, so it loads logical chunk
  // (l % CPR) ^ swz(row) of that row.  Each wave group reads only its own half of a stage
  // (rows gkoff .. gkoff + 63) and loads it itself: wave (grp, wr) fills the chunks
  // g = 64 grp / RPL + wr + 4 i.  swz depends on g only through g & 3 (K, D = 128) or g & 1
  // (K, D = 64), fixed by wr, so one per-lane byte offset plus 4 i RPL rows serves every
  // load of a tensor.  One buffer resource per step starts at the step's first key; rows
  // past S are outside it and read as zero, and a step past the last gets an empty
  // resource (its loads write zeros into a stage half nobody reads any more).
  // R256: both groups read whole stages, so the eight waves fill every chunk, wave w the
  // chunks w + 8 i (g & 3 and g & 1 stay fixed per wave, so one per-lane offset still serves).
  constexpr int LS = R256 ? 8 : 4;     // chunk stride of a wave's loads
  const int ld_g0 = R256 ? wave : gkoff / RPL + wr;  // first chunk this wave fills
  const int ld_row = ld_g0 * RPL + lane / CPR;
  const int ld_pc = lane % CPR;
  // A logical chunk at or past d_real gets an offset of 2^31 or more: every buffer resource
  // here spans less than 2^31 bytes, so it reads zero (and the per-load row steps added
  // below stay far from 2^32).
  constexpr int kZeroChunk = INT32_MIN;
  const int lck = ld_pc ^ pp_swz_k<DA>(ld_row);
  const int lcv = ld_pc ^ pp_swz_v<DA>(ld_row);
  const int kvo = 8 * lck < d_real ? ld_row * k_rb + (lck << 4) : kZeroChunk;
  const int vvo = 8 * lcv < d_real ? ld_row * v_rb + (lcv << 4) : kZeroChunk;
  // Tail part: wave (grp, wr) fills the group's tail rows gkoff + 16 wr .. + 15, lane l
  // writing physical chunk l % 4 of row l / 4 of them.  K's tail chunks are swizzled with
  // (row >> 2) & 3 (a b128 read pass covers 16 consecutive rows at one chunk, rows 256
  // bytes apart repeat every 4); V's tail needs none (a transposed read pass covers 4 rows
  // x 64 bytes).  For these rows (row >> 2) & 3 = (l >> 4) & 3.
  const int tl_row = gkoff + 16 * wr + (lane >> 2);
  const int tl_lck = (lane & 3) ^ ((lane >> 4) & 3);
  const int tl_lcv = lane & 3;
  const int tkvo = DA + 8 * tl_lck < d_real ? tl_row * k_rb + 2 * DA + (tl_lck << 4) : kZeroChunk;
  const int tvvo = DA + 8 * tl_lcv < d_real ? tl_row * v_rb + 2 * DA + (tl_lcv << 4) : kZeroChunk;
  // Q is staged like a K stage (same swizzle, same per-lane rows and chunks).
  const int q_rb = (int)p.q_ss * 2;
  const int qvo = 8 * lck < d_real ? ld_row * q_rb + (lck << 4) : kZeroChunk;
  const int tqvo = DA + 8 * tl_lck < d_real ? tl_row * q_rb + 2 * DA + (tl_lck << 4) : kZeroChunk;
  auto dma = [&](const uint16_t* gbase, int64_t row_stride, int rb, int vo, int tvo, int t,
                 char* stage) {
    const int row0 = t * TK;
    const int rows = t < t_end ? S - row0 : 0;
    const __amdgpu_buffer_rsrc_t r = row_rsrc(gbase + (int64_t)row0 * row_stride, rows, rb);
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)(stage + (ld_g0 + LS * i) * 1024), 16,
          vo + i * LS * RPL * rb, 0, 0, 0);
    }
    if constexpr (NLDT != 0) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)(stage + STAGE_A + gkoff * RBT + wr * 1024),
          16, tvo, 0, 0, 0);
    }
  };
  // The Q tile into `stage` in a K stage's layout, each group loading its half of the rows;
  // rows past S are outside the resource and read as zero.  Against per-lane global loads
  // of each wave's own rows (both groups loading the same rows, 32 rows an instruction)
  // this halves the Q traffic and makes it 1 KiB-contiguous: B1 H8 causal D = 128
  // S = 1024 -8 %, S = 8192 -1.6 %; C4 D = 128 -1.7 %.
  auto dma_q = [&](char* stage) {
    const __amdgpu_buffer_rsrc_t r = row_rsrc(qp + (int64_t)q0 * p.q_ss, S - q0, q_rb);
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)(stage + (ld_g0 + 4 * i) * 1024), 16,
          qvo + i * 4 * RPL * q_rb, 0, 0, 0);
    }
    if constexpr (NLDT != 0) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)(stage + STAGE_A + gkoff * RBT + wr * 1024),
          16, tqvo, 0, 0, 0);
    }
  };
  // Wait for this wave's direct-to-LDS loads (vmcnt = 0; expcnt and lgkmcnt left at their
  // maxima) before the barrier that publishes them to the rest of its group.
  auto wait_dma = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };

  // ---- per-lane LDS read offsets --------------------------------------------------------
  // K: lane reads row koff + 32 bk + l32 at logical chunk 2 kk + hl; with m = swz_k(l32)
  // that is byte (koff + l32) * RB + (32 * (m >> 1) + 16 * (hl ^ (m & 1))) ^ (32 kk), plus
  // 32 * bk * RB.
  const int mk = pp_swz_k<DA>(l32);
  const int k_rd = (koff + l32) * RB + 32 * (mk >> 1) + 16 * (hl ^ (mk & 1));
  // K tail (k-steps DKA, DKA + 1): logical chunk 2 (kk - DKA) + hl of tail row
  // koff + 32 bk + l32, physical chunk logical ^ ((l32 >> 2) & 3): byte
  // kt_rd ^ (32 (kk - DKA)) of the tail part, plus 32 * bk * RBT.
  const int kt_rd = (koff + l32) * RBT + 16 * (hl ^ ((l32 >> 2) & 3));
  // V^T via the transposed read: lane l of 16-lane group G addresses row 4 hl + r,
  // r = (l % 16) / 4, of a 16-key chunk and d = 32 db + 16 (G % 2) + 4 (l % 4); the hardware
  // hands lane l column 32 db + 16 (G % 2) + l % 16 of those 4 rows.  swz_v depends only on
  // r, so the byte address is v_rd ^ (64 db), plus (koff + 32 bk + 16 kc) * RB.
  const int tr_r = (lane & 15) >> 2;
  const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int v_rd = (koff + 4 * hl + tr_r) * RB +
                   16 * ((tr_d >> 3) ^ pp_swz_v<DA>(4 * hl + tr_r)) + 2 * (tr_d & 7);
  // V tail (d block DBA): the same rows and columns tr_d of the unswizzled 64-byte tail rows.
  const int vt_rd = (koff + 4 * hl + tr_r) * RBT + 2 * tr_d;

  // ---- running state (lane = query l32 of this wave) ----------------------------------
  float m_run = kNegLarge;
  float l_part = 0.0f;
  f32x16 o_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o_acc[db] = f32x16{};
  const float c = p.scale_log2;

  // Step t, from this wave's point of view: first key, whether all 32-key blocks hold keys
  // it needs, and whether no score needs a mask.
  auto key0 = [&](int t) { return t * TK + koff; };
  auto all_active = [&](int t) { return key0(t) + 32 * (KB - 1) < wave_kv_end; };
  auto no_mask = [&](int t) {
    return (!CAUSAL || key0(t) + 32 * KB - 1 <= wq0) && (!TAIL || key0(t) + 32 * KB <= S);
  };

  f32x16 s[KB];        // S^T blocks of the step whose softmax comes next
  uint32_t pk[KB][8];  // packed P of the step whose P.V comes next

  // S^T = K Q^T of a step from stage `kst`, every block (blocks holding no key the wave
  // needs are masked whole by the softmax).
  auto qk = [&](const char* kst) {
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
        const char* ap = kk < DKA ? kst + bk * 32 * RB + (k_rd ^ (32 * kk))
                                  : kst + STAGE_A + bk * 32 * RBT + (kt_rd ^ (32 * (kk - DKA)));
        const u32x4 a = *(const u32x4*)ap;
        s[bk] = DTy::mfma(a, qf[kk], kk == 0 ? f32x16{} : s[bk]);
      }
    }
  };

  // O^T += V^T P^T of the step held in pk, from stage `vst`.  Every block: P is exactly 0
  // for masked keys.
  u32x4 late_a[kLateMfma > 0 ? kLateMfma : 1];  // A operands of the late MFMAs
  auto pv = [&](const char* vst) {
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const u32x4 bfrag = {pk[bk][4 * kc + 0], pk[bk][4 * kc + 1], pk[bk][4 * kc + 2],
                             pk[bk][4 * kc + 3]};
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const int rbd = db < DBA ? RB : RBT;  // row bytes of the part holding d block db
          const char* a0p = db < DBA ? vst + (v_rd ^ (64 * db)) + (32 * bk + 16 * kc) * RB
                                     : vst + STAGE_A + vt_rd + (32 * bk + 16 * kc) * RBT;
          s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a0p);
          s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0p + 8 * rbd));
          u32x2 w0 = __builtin_bit_cast(u32x2, r0);
          u32x2 w1 = __builtin_bit_cast(u32x2, r1);
          const u32x4 a = {w0[0], w0[1], w1[0], w1[1]};
          const int li = (bk * 2 + kc) * DB + db;  // issue order
          if (li >= KB * 2 * DB - kLateMfma) {
            late_a[li - (KB * 2 * DB - kLateMfma)] = a;
            continue;
          }
          o_acc[db] = DTy::mfma(a, bfrag, o_acc[db]);
        }
      }
    }
  };

  // Row max of the scores in s (NaN-propagating), over the wave's two lane halves.
  auto row_max = [&]() {
    float mxa = kMasked, mxb = kMasked;
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
      for (int r = 0; r < 16; r += 4) {
        mxa = vmax3(mxa, s[bk][r], s[bk][r + 1]);
        mxb = vmax3(mxb, s[bk][r + 2], s[bk][r + 3]);
      }
    }
    float a0, a1;
    swap32(vmax(mxa, mxb), a0, a1);
    return vmax(a0, a1);
  };

  // VALU cluster of step t: mask, row max, rescale, P = 2^(s*c - m*c) packed, l.  One
  // code path for every step (blocks without a needed key are masked whole), so the
  // rescale of O exists once and O keeps one register assignment through the loop.
  auto softmax = [&](int t, auto par_tag) {
    constexpr int PAR = decltype(par_tag)::value;
    // Blocks past the wave's last key are masked whole by the same test: all their keys
    // are past the wave's last query (causal) or past S.
    if (!(no_mask(t) && all_active(t))) {
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
        const int kb0 = key0(t) + 32 * bk;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kb0 + (r >> 2) * 8 + hl * 4 + (r & 3);
          bool bad = false;
          if (CAUSAL) bad = key > my_q;
          if (TAIL) bad = bad || key >= S;
          s[bk][r] = bad ? kMasked : s[bk][r];
        }
      }
    }
    // P = 2^(s c - mc) packed into pk, and the sum of the rounded P.  Each kind of op runs
    // over all 32 of the lane's scores before the next kind (FMA, exp, pack), so dependent
    // ops sit many instructions apart (C3 -1 %); the sum uses four independent dot2 chains,
    // each started without a zeroed accumulator (four VALU ops fewer; 0.3-2 %).
    auto make_p = [&](float mc) {
      if constexpr (kPhasedP) {
        float x[KB][16];
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
          for (int r = 0; r < 16; ++r) x[bk][r] = __builtin_fmaf(s[bk][r], c, -mc);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
          for (int r = 0; r < 16; ++r) x[bk][r] = fast_exp2(x[bk][r]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) pk[bk][r >> 1] = DTy::pack(x[bk][r], x[bk][r + 1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      } else {
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            pk[bk][r >> 1] = DTy::pack(fast_exp2(__builtin_fmaf(s[bk][r], c, -mc)),
                                       fast_exp2(__builtin_fmaf(s[bk][r + 1], c, -mc)));
          }
        }
      }
      float l4[4];
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const int j = (r >> 1) & 3;
          l4[j] = bk == 0 && r < 8 ? DTy::sum2_head(pk[bk][r >> 1]) : DTy::sum2(pk[bk][r >> 1], l4[j]);
        }
      }
      return (l4[0] + l4[1]) + (l4[2] + l4[3]);
    };
    // The reference point m moves only when the row max grows by more than the rescale
    // threshold (some P above 2^kRescaleLog2), so P is first computed with the current m.
    // P >= 0, so a lane whose sum of P stays below that bound has no such P and needs no
    // max at all: the row max is reduced only in the rare wave where some lane's sum
    // reaches it (every row's first step, a jump of the max), and there the rule is the
    // exact one (max grew by more than the threshold -> rescale O and l, recompute P).
    // A VALU cluster is bound by one wave's issue rate, so the skipped reduction is time
    // saved.
    if constexpr (LOWP) {
      // Exact running max; P from it (fp32), packed for P.V; l from the unrounded P.
      const float mx = row_max();
      const float m_new = vmax(m_run, mx);
      const float alpha = fast_exp2((m_run - m_new) * c);  // 1 where the max holds
      m_run = m_new;
      const float mc = m_run * c;
      float l4[4];
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = fast_exp2(__builtin_fmaf(s[bk][r], c, -mc));
          const float p1 = fast_exp2(__builtin_fmaf(s[bk][r + 1], c, -mc));
          pk[bk][r >> 1] = DTy::pack(p0, p1);
          const int j = (r >> 1) & 3;
          l4[j] = bk == 0 && r < 8 ? p0 + p1 : l4[j] + (p0 + p1);
        }
      }
      l_part = l_part * alpha + ((l4[0] + l4[1]) + (l4[2] + l4[3]));
      // The accumulation since the last rounding (acc + P.V in fp32) rounded to the input
      // dtype once per kLowpSteps steps (TILE_N keys of the wave's key slice), rescaled
      // first when some row's max moved: rnd((acc + P.V) rnd(alpha)); the steps between
      // only rescale.  t & 1 is PAR (whole rows start at step 0): the cadence is known at
      // compile time unless kLowpSteps is 4.
      const bool moved = __ballot(!(alpha == 1.0f)) != 0;
      const float al = DTy::round(alpha);
      const bool round_now = kLowpSteps == 1 || (kLowpSteps == 2 ? PAR == 1 : (PAR == 1 && (t & 2)));
      // `moved` is uniform: one branch per case (as a per-element select the compiler
      // formed both packs, the products and a select for every value on every step).
      if (round_now && moved) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const uint32_t w = DTy::pack(o_acc[db][r] * al, o_acc[db][r + 1] * al);
            o_acc[db][r] = DTy::lo(w);
            o_acc[db][r + 1] = DTy::hi(w);
          }
        }
      } else if (round_now) {
#pragma unroll
        for (int db = 0; db < DB; ++db) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const uint32_t w = DTy::pack(o_acc[db][r], o_acc[db][r + 1]);
            o_acc[db][r] = DTy::lo(w);
            o_acc[db][r + 1] = DTy::hi(w);
          }
        }
      } else if (moved) {
#pragma unroll
        for (int db = 0; db < DB; ++db) o_acc[db] *= al;
      }
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
        for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(pk[bk][i]));
      }
      return;
    }
    float l_step = make_p(m_run * c);
    if (__ballot(!(l_step < kRescaleBound))) {
      const float mx = row_max();
      const bool need = (mx - m_run) * c > kRescaleLog2;
      if (__ballot(need)) {
        const float m_new = need ? mx : m_run;
        const float alpha = fast_exp2((m_run - m_new) * c);
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < DB; ++db) o_acc[db] *= alpha;
        l_part *= alpha;
        l_step = make_p(m_run * c);
      }
    }
    l_part += l_step;
    // Keep the P computation in this cluster: without a use here the compiler sinks it
    // past the barrier to its consumers, the P.V MFMAs of the other cluster.
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
      for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(pk[bk][i]));
    }
  };

  // Issue order of the MFMA cluster: AHEAD LDS reads first, then each MFMA followed by the
  // reads of the MFMA AHEAD places later (1 for a K operand, 2 for a transposed V operand)
  // and, on every (NQ + NP) / nv-th MFMA, one of the cluster's nv loads into LDS.
  auto mfma_cluster_order = [&](int nv) {
    constexpr int NQ = KB * DK;      // QK^T MFMAs
    constexpr int NP = KB * 2 * DB;  // P.V MFMAs
    constexpr int AHEAD = 4;
    constexpr int NC = NQ + NP - kLateMfma;  // MFMAs in the cluster
    const int every = nv ? NC / nv : 0;
    __builtin_amdgcn_sched_group_barrier(0x100, AHEAD, 0);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      const int j = i + AHEAD;  // MFMA whose operands are read now
      if (j < NQ) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      } else if (j < NQ + NP) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      if (every && i % every == 0) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    }
    // operand reads of late MFMAs not yet covered
    constexpr int REM = NC + AHEAD < NQ + NP ? 2 * (NQ + NP - NC - AHEAD) : 0;
    if constexpr (REM > 0) __builtin_amdgcn_sched_group_barrier(0x100, REM, 0);
  };

  // Workgroup barrier without a memory fence: a fence would also wait for this wave's
  // direct-to-LDS loads, which are meant to stay in flight across the next barrier.  The
  // wave's LDS accesses are complete first (lgkmcnt = 0); the empty asm statements keep
  // the compiler from moving memory accesses across the barrier.  Loads into LDS are
  // waited for explicitly (wait_dma) by the wave that issued them before the barrier that
  // publishes them.
  // The barrier orders memory accesses only: the compiler issues the last few P.V MFMAs of
  // a cluster (operands already in registers) after it, in the wave's softmax phase, where
  // the MFMA pipe has room (3 of 32 at 128 rows; pinning all 32 in the cluster, or moving
  // 5 or 8 out, measured 2-4 % slower).  The fp32 64-row kernels are pinned (sched_barrier):
  // C3 S = 512 / 2048 -0.2 / -0.5 us against the one MFMA the compiler moves there (their
  // input-dtype variants measured 2.4 % slower pinned and are not).  Kernels with late
  // MFMAs (kLateMfma) are pinned too, so that exactly those cross the barrier.
  constexpr bool kPinPhases = (TM == 64 && !LOWP) || kLateMfma > 0;
  auto barrier = [&]() {
    if constexpr (kPinPhases) __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if constexpr (kPinPhases) __builtin_amdgcn_sched_barrier(0);
  };

  // ---- prologue and key loop ---------------------------------------------------------
  // Global phases: phase 0 = group 0 computes S_0 (group 1 idles); phase 2t + 1 = group 0's
  // softmax of step t with group 1's MFMA cluster of step t - 1 (S_0 for t = 0); phase
  // 2t + 2 = group 0's MFMA cluster of step t (S_{t+1}, P_t.V_t) with group 1's softmax of
  // step t.  Every phase ends at a workgroup barrier.
  //
  // A group reads only its own halves of the stages: its half of K_u in the MFMA cluster of
  // step u - 1 and its half of V_u in the MFMA cluster of step u.  It loads its halves of
  // K_{t+2} and V_{t+1} during its MFMA cluster of step t (into the halves that cluster's
  // predecessor read last) and waits for them at the end of its next softmax cluster.
  // Both groups run the same sequence, group 1 one phase later.
  //
  // Prologue: every wave issues its share of K_0, of the Q tile (into lds_v1, free until
  // the first MFMA cluster loads V_1 into it), and its group's halves of K_1 and V_0, then
  // waits until at most the last 2 NLDS loads (K_1 and V_0) are in flight: K_0 and Q have
  // landed, and the latencies of all four overlap.  After the barrier every wave reads its
  // Q fragment from lds_v1.  K_1 and V_0 are waited for at the end of the group's first
  // softmax cluster, like the loads of every MFMA cluster.
  static_assert(2 * NLDS < 16, "vmcnt field");
  dma(kp, p.k_ss, k_rb, kvo, tkvo, t_beg, lds_k0);
  if constexpr (R256) {
    // Q straight into the B-operand registers: lane l holds row wq0 + l % 32, columns
    // 16 kk + 8 (l / 32) .. + 8 (the layout the LDS read below produces); rows past S and
    // columns past d_real are zero.  Counted by vmcnt before K_1 and V_0.
    const uint16_t* qrow = qp + (int64_t)(my_q < S ? my_q : 0) * p.q_ss;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      const int d0 = 16 * kk + 8 * hl;
      qf[kk] = my_q < S && d0 < d_real ? *(const u32x4*)(qrow + d0) : u32x4{0u, 0u, 0u, 0u};
    }
  } else if (TM == 128 || grp == 0) {
    dma_q(lds_v1);  // 64-row blocks: group 0's chunks hold every row
  }
  dma(kp, p.k_ss, k_rb, kvo, tkvo, t_beg + 1, lds_k1);
  dma(vp, p.v_ss, v_rb, vvo, tvvo, t_beg, lds_v0);
  // R256: every prologue load, since the first MFMA cluster of each group reads K_1 and
  // V_0 shares loaded by the other group's waves.
  __builtin_amdgcn_s_waitcnt(R256 ? 0x0F70 : 0x0F70 | (2 * NLDS));
  barrier();
  // Q fragment from lds_v1 (rows 32 wr + l32, read like a K operand); lds_v1 receives V_1
  // only in the first MFMA cluster, at least two barriers later.
  if constexpr (!R256) {
    const int qr = 32 * rb + l32;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      const char* ap = kk < DKA ? lds_v1 + qr * RB + ((k_rd - (koff + l32) * RB) ^ (32 * kk))
                                : lds_v1 + STAGE_A + qr * RBT +
                                      ((kt_rd - (koff + l32) * RBT) ^ (32 * (kk - DKA)));
      qf[kk] = *(const u32x4*)ap;
    }
  }
  // S_0.
  // The reference point for a row's first step is its row max when that step needs no
  // mask, so the first softmax computes P once (from the initial point it would find every
  // P above the bound, reduce the max and compute P again); a masked first step keeps the
  // initial point and takes the exact rule over its masked scores.  O and l start at zero,
  // so the result is the same either way.
  auto first = [&]() {
    qk(lds_k0);
    if (!LOWP && no_mask(t_beg) && all_active(t_beg)) m_run = row_max();
  };

  // Step t with stage parity PAR: the stages of K_t (consumed; receives K_{t+2}), K_{t+1},
  // V_t and V_{t-1} (consumed; receives V_{t+1}).
  auto iter = [&](int t, auto par_tag, auto g1_tag) {
    constexpr int PAR = decltype(par_tag)::value;
    char* k_cur = PAR ? lds_k1 : lds_k0;
    char* k_nxt = PAR ? lds_k0 : lds_k1;
    char* v_cur = PAR ? lds_v1 : lds_v0;
    char* v_nxt = PAR ? lds_v0 : lds_v1;
    // R256: group 1 issues its share of K_{t+2} and V_{t+1} at the start of its softmax
    // (the phase of group 0's MFMA cluster, which loads the rest; both stages are free:
    // their last readers were the two MFMA clusters of step t - 1) and waits for it at the
    // end of its MFMA cluster, so both shares have landed before group 0 reads the stages.
    constexpr bool loads_in_softmax = R256 && decltype(g1_tag)::value;
    if constexpr (loads_in_softmax) {
      dma(kp, p.k_ss, k_rb, kvo, tkvo, t + 2, k_cur);
      dma(vp, p.v_ss, v_rb, vvo, tvvo, t + 1, v_nxt);
    }
    softmax(t, par_tag);
    if constexpr (!loads_in_softmax) wait_dma();  // this wave's K_{t+1} and V_t loads (one cluster ago)
    barrier();
    // MFMA cluster: S of step t + 1 (past the last step it reads a stale or zero stage and
    // is never used) and P.V of step t, one straight-line block whose LDS reads run AHEAD
    // MFMAs in front of their consumers, with this wave's loads of K_{t+2} and V_{t+1}
    // spread over it.  Both clusters run at the same priority (the softmax cluster is the
    // longer one, and giving the MFMA cluster priority cost 1-4 %), except in the kernels
    // that share a CU between two workgroups, where raising it keeps the two workgroups'
    // MFMA clusters from delaying each other (2.5 % there).
    if constexpr (kPrioMfma) __builtin_amdgcn_s_setprio(1);
    qk(k_nxt);
    pv(v_cur);
    if constexpr (loads_in_softmax) {
      mfma_cluster_order(0);
      wait_dma();
    } else {
      dma(kp, p.k_ss, k_rb, kvo, tkvo, t + 2, k_cur);
      dma(vp, p.v_ss, v_rb, vvo, tvvo, t + 1, v_nxt);
      mfma_cluster_order(2 * NLDS);
    }
    if constexpr (kPrioMfma) __builtin_amdgcn_s_setprio(0);
    barrier();
    if constexpr (kLateMfma > 0) {
#pragma unroll
      for (int x = 0; x < kLateMfma; ++x) {
        const int li = KB * 2 * DB - kLateMfma + x;
        const int db = li % DB, bk = li / DB / 2, kc = li / DB % 2;
        const u32x4 bfrag = {pk[bk][4 * kc + 0], pk[bk][4 * kc + 1], pk[bk][4 * kc + 2], pk[bk][4 * kc + 3]};
        o_acc[db] = DTy::mfma(late_a[x], bfrag, o_acc[db]);
      }
    }
  };
  using G0 = std::false_type;
  using G1 = std::integral_constant<bool, R256>;  // group 1's own load schedule (R256 only)
  if (grp == 0) {
    first();
    barrier();
    for (int t = t_beg; t < t_end; t += 2) {
      iter(t, std::integral_constant<int, 0>{}, G0{});
      if (t + 1 < t_end) iter(t + 1, std::integral_constant<int, 1>{}, G0{});
    }
    barrier();  // phase 2 n_steps + 1: group 1's last MFMA cluster
  } else {
    barrier();  // phase 0: group 0's S_0
    first();
    barrier();
    for (int t = t_beg; t < t_end; t += 2) {
      iter(t, std::integral_constant<int, 0>{}, G1{});
      if (t + 1 < t_end) iter(t + 1, std::integral_constant<int, 1>{}, G1{});
    }
  }
  wait_dma();  // the zero-filling loads of the last two steps, before the merge reuses LDS
  barrier();

  // R256: every wave holds all keys of its 32 rows: O / l straight to the output (the lane
  // pair l, l + 32 shares a row and holds half of its l each).
  if constexpr (R256) {
    float la, lb;
    swap32(l_part, la, lb);
    const float inv = 1.0f / (la + lb);
    if (TAIL && my_q >= S) return;
    uint16_t* orow = op + (int64_t)my_q * p.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * db + 8 * g + 4 * hl;
        if (d < d_real)
          *(u32x2*)(orow + d) = u32x2{DTy::pack(o_acc[db][4 * g] * inv, o_acc[db][4 * g + 1] * inv),
                                      DTy::pack(o_acc[db][4 * g + 2] * inv, o_acc[db][4 * g + 3] * inv)};
      }
    }
    return;
  }

  // Merge of d blocks [LO, LO + DB/2) of this wave's row block with the partner wave's
  // (same rows, the other key half).  Exchange regions: group 0's waves send from lds_k0,
  // group 1's from lds_k1 (DB/2 blocks x 16 floats x 64 lanes each, laid out as 16-byte
  // chunks [block][g][lane]: conflict-free 16-byte writes and reads), (m, l) at the start
  // of lds_v0; the merged tile is staged in lds_v1 for row-contiguous stores.
  auto merge_half = [&](auto lo_tag) {
    constexpr int LO = decltype(lo_tag)::value;
    constexpr int NB = DB / 2;
    constexpr int RGN = NB * 16 * 64 * 4;  // bytes a wave sends
    static_assert(4 * RGN <= STAGE, "a group's exchange regions fit one stage");
    constexpr int PLO = LO == 0 ? NB : 0;  // first block the partner merges
    f32x4* mine = (f32x4*)((grp == 0 ? lds_k0 : lds_k1) + wr * RGN);
    const f32x4* theirs = (const f32x4*)((grp == 0 ? lds_k1 : lds_k0) + wr * RGN);
    float* ml = (float*)lds_v0;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int db = PLO + b;
        mine[(b * 4 + g) * 64 + lane] =
            f32x4{o_acc[db][4 * g], o_acc[db][4 * g + 1], o_acc[db][4 * g + 2], o_acc[db][4 * g + 3]};
      }
    }
    ml[(grp * 4 + wr) * 128 + lane] = m_run;
    ml[(grp * 4 + wr) * 128 + 64 + lane] = l_part;
    barrier();
    f32x4 x1[NB][4];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) x1[b][g] = theirs[(b * 4 + g) * 64 + lane];
    }
    const float m1 = ml[((1 - grp) * 4 + wr) * 128 + lane];
    const float l1 = ml[((1 - grp) * 4 + wr) * 128 + 64 + lane];
    __builtin_amdgcn_sched_barrier(0);
    const float m = vmax(m_run, m1);
    const float a0 = fast_exp2((m_run - m) * c);
    const float a1 = fast_exp2((m1 - m) * c);
    float la, lb;
    swap32(l_part * a0 + l1 * a1, la, lb);
    const float l_tot = la + lb;
    const float inv = 1.0f / l_tot;
    const float w0s = a0 * inv, w1s = a1 * inv;
    // Input-dtype accumulation: the two halves (each rounded per tile) combined in fp32 and
    // rounded to the input dtype, then rnd(acc rnd(1/l)) (flash_fwd.py:366-368).
    const float ri = DTy::round(inv);
    auto merged = [&](int b, int g) {
      f32x4 o4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (LOWP) {
          o4[e] = DTy::round(DTy::round(o_acc[LO + b][4 * g + e] * a0 + x1[b][g][e] * a1) * ri);
        } else {
          o4[e] = o_acc[LO + b][4 * g + e] * w0s + x1[b][g][e] * w1s;
        }
      }
      return o4;
    };
    if (SPLIT && slot >= 0) {
      // One chunk of a split block: its output normalised by its own l, in fp32, and
      // log2 of its softmax denominator in units of the scaled scores, m c + log2(l).
      if (TAIL && my_q >= S) return;
      float* prow = p.part_o + ((int64_t)slot * TM + (my_q - q0)) * D;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) store_partial(p, prow + 32 * (LO + b) + 8 * g + 4 * hl, merged(b, g));
      }
      if (grp == 0 && hl == 0) store_partial(p, p.part_lse + (int64_t)slot * TM + (my_q - q0), m * c + fast_log2(l_tot));
      return;
    }
    // Whole-row kernels at D = 128, and causal ones at D = 64, stage the wave's 32 rows x
    // D/2 columns in lds_v1 (16-byte chunks swizzled with the row's low bits, CH a row) so
    // each store writes 16 bytes a lane, CH lanes a row; the non-causal D = 64 kernels (two
    // workgroups per CU) store 8 bytes a lane directly.
    constexpr bool kStageOut = !SPLIT && (D == 128 || (D == 64 && CAUSAL));
    if constexpr (kStageOut) {
      constexpr int CH = 4 * NB;           // 16-byte chunks per staged row (D/2 columns)
      constexpr int RPI = 64 / CH;         // rows per store instruction
      constexpr int SWZ = CH - 1;
      char* ob = lds_v1 + (grp * 4 + wr) * (32 * CH * 16);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x4 o4 = merged(b, g);
          const int ch = 4 * b + g;
          *(u32x2*)(ob + l32 * (CH * 16) + 16 * (ch ^ (l32 & SWZ)) + 8 * hl) =
              u32x2{DTy::pack(o4[0], o4[1]), DTy::pack(o4[2], o4[3])};
        }
      }
      asm volatile("" ::: "memory");
      const int ch = lane % CH;
#pragma unroll
      for (int i = 0; i < 32 / RPI; ++i) {
        const int row = RPI * i + lane / CH;
        const u32x4 v = *(const u32x4*)(ob + row * (CH * 16) + 16 * (ch ^ (row & SWZ)));
        const int q = wq0 + row;
        const int col = 32 * LO + 8 * ch;
        if ((!TAIL || q < S) && col < d_real) {
          // D = 128: non-temporal stores (C3 S = 4096 / 8192 -0.9 / -0.6 %, C4 unchanged);
          // at D = 64, and on the other store paths, they measured slower.
          if constexpr (D == 128) {
            __builtin_nontemporal_store(v, (u32x4*)(op + (int64_t)q * p.o_ss + col));
          } else {
            *(u32x4*)(op + (int64_t)q * p.o_ss + col) = v;
          }
        }
      }
      return;
    }
    if (TAIL && my_q >= S) return;
    uint16_t* orow = op + (int64_t)my_q * p.o_ss;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 o4 = merged(b, g);
        const int d = 32 * (LO + b) + 8 * g + 4 * hl;
        if (d < d_real) *(u32x2*)(orow + d) = u32x2{DTy::pack(o4[0], o4[1]), DTy::pack(o4[2], o4[3])};
      }
    }
  };

  // ---- 64-row blocks: merge the four key slices of each row block, O = acc / l ----------
  // Waves (g, rb + 2 k) of both groups g and key slots k hold the same 32 rows over
  // different keys.  Part P = 2 g + k of them merges the lane's 16-byte O^T chunks
  // [P DB, (P + 1) DB) (chunk u = 4 db + j holds d = 32 db + 8 j + 4 hl + e, e < 4): each
  // wave sends the other three the chunks they merge, in slots ordered by part (its own
  // part skipped), plus its (m, l); region of wave w: half w % 2 of stage w / 2, (m, l)
  // behind both halves.  The stages are free: every load has landed and every read has
  // retired before the last barrier.
  if constexpr (TM == 64) {
    constexpr int CPW = DB;                // chunks a part merges
    constexpr int RG = 3 * CPW * 64 * 16;  // bytes a wave sends
    static_assert(2 * RG + 2 * 512 <= STAGE, "exchange regions fit the stages");
    auto stage_of = [&](int i) -> char* {
      return i == 0 ? lds_k0 : i == 1 ? lds_k1 : i == 2 ? lds_v0 : lds_v1;
    };
    const int part = 2 * grp + ks;
    {
      f32x4* mine = (f32x4*)(stage_of(wave >> 1) + (wave & 1) * RG);
#pragma unroll
      for (int u = 0; u < 4 * DB; ++u) {
        const int tp = u / CPW;  // the part that merges chunk u
        if (tp == part) continue;
        const int slot = tp < part ? tp : tp - 1;
        mine[(slot * CPW + u % CPW) * 64 + lane] =
            f32x4{o_acc[u / 4][4 * (u % 4)], o_acc[u / 4][4 * (u % 4) + 1], o_acc[u / 4][4 * (u % 4) + 2],
                  o_acc[u / 4][4 * (u % 4) + 3]};
      }
      float* ml = (float*)(stage_of(wave >> 1) + 2 * RG + (wave & 1) * 512);
      ml[lane] = m_run;
      ml[64 + lane] = l_part;
    }
    barrier();
    auto merge_part = [&](auto p_tag) {
      constexpr int P = decltype(p_tag)::value;
      f32x4 x[3][CPW];
      float mq[3], lq[3];
#pragma unroll
      for (int n = 0; n < 3; ++n) {
        const int q = n < P ? n : n + 1;  // partner part
        const int wq = 4 * (q >> 1) + rb + 2 * (q & 1);
        const f32x4* src = (const f32x4*)(stage_of(wq >> 1) + (wq & 1) * RG);
        const int slot = P < q ? P : P - 1;  // our part's slot in the partner's region
#pragma unroll
        for (int cc = 0; cc < CPW; ++cc) x[n][cc] = src[(slot * CPW + cc) * 64 + lane];
        const float* ml = (const float*)(stage_of(wq >> 1) + 2 * RG + (wq & 1) * 512);
        mq[n] = ml[lane];
        lq[n] = ml[64 + lane];
      }
      __builtin_amdgcn_sched_barrier(0);
      const float m = vmax(vmax(m_run, mq[0]), vmax(mq[1], mq[2]));
      const float a0 = fast_exp2((m_run - m) * c);
      float an[3];
#pragma unroll
      for (int n = 0; n < 3; ++n) an[n] = fast_exp2((mq[n] - m) * c);
      float la, lb;
      swap32(l_part * a0 + (lq[0] * an[0] + lq[1] * an[1]) + lq[2] * an[2], la, lb);
      const float l_tot = la + lb;
      const float inv = 1.0f / l_tot;
      const float w0 = a0 * inv;
      float wn[3];
#pragma unroll
      for (int n = 0; n < 3; ++n) wn[n] = an[n] * inv;
      if (TAIL && my_q >= S) return;
      if (SPLIT && slot >= 0) {
        // One chunk of a split block: rows of this 64-row half of the 128-row slot, each
        // normalised by its own l, in fp32, and m c + log2(l) (the 128-row split's partial
        // format, merged by the same kernel).
        const int srow = my_q - (q0 & ~(kPPRows - 1));
        float* prow = p.part_o + ((int64_t)slot * kPPRows + srow) * D;
#pragma unroll
        for (int cc = 0; cc < CPW; ++cc) {
          constexpr int U0 = P * CPW;
          const int u = U0 + cc;
          f32x4 o4;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o4[e] = o_acc[u / 4][4 * (u % 4) + e] * w0 + (x[0][cc][e] * wn[0] + x[1][cc][e] * wn[1]) +
                    x[2][cc][e] * wn[2];
          store_partial(p, prow + 32 * (u / 4) + 8 * (u % 4) + 4 * hl, o4);
        }
        if (P == 0 && hl == 0) store_partial(p, p.part_lse + (int64_t)slot * kPPRows + srow, m * c + fast_log2(l_tot));
        return;
      }
      uint16_t* orow = op + (int64_t)my_q * p.o_ss;
#pragma unroll
      for (int cc = 0; cc < CPW; ++cc) {
        constexpr int U0 = P * CPW;
        const int u = U0 + cc;
        f32x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (LOWP) {
            // the four slices (each rounded per tile) combined in fp32 and rounded to the
            // input dtype, then rnd(acc rnd(1/l))
            const float h = o_acc[u / 4][4 * (u % 4) + e] * a0 + (x[0][cc][e] * an[0] + x[1][cc][e] * an[1]) +
                            x[2][cc][e] * an[2];
            o4[e] = DTy::round(DTy::round(h) * DTy::round(inv));
          } else {
            o4[e] = o_acc[u / 4][4 * (u % 4) + e] * w0 + (x[0][cc][e] * wn[0] + x[1][cc][e] * wn[1]) +
                    x[2][cc][e] * wn[2];
          }
        }
        const int d = 32 * (u / 4) + 8 * (u % 4) + 4 * hl;
        if (d < d_real) *(u32x2*)(orow + d) = u32x2{DTy::pack(o4[0], o4[1]), DTy::pack(o4[2], o4[3])};
      }
    };
    switch (part) {
      case 0: merge_part(std::integral_constant<int, 0>{}); break;
      case 1: merge_part(std::integral_constant<int, 1>{}); break;
      case 2: merge_part(std::integral_constant<int, 2>{}); break;
      default: merge_part(std::integral_constant<int, 3>{}); break;
    }
    return;
  } else if constexpr (DB % 2 == 0) {
    // Both groups merge, each half of the d blocks (group 0 blocks [0, DB/2), group 1 the
    // rest): every wave sends its partner (the wave of the other group with the same row
    // block) the blocks the partner merges, as 16-byte chunks, and its (m, l).  The stages
    // are free: every load has landed and every read has retired before the last barrier.
    if (grp == 0) merge_half(std::integral_constant<int, 0>{});
    else merge_half(std::integral_constant<int, DB / 2>{});
    return;
  }
  // Group 1 leaves (m, l, O^T) in LDS; group 0 merges and writes O.
  float* xo = (float*)((wr < 2 ? lds_k0 : lds_k1) + (wr & 1) * (STAGE / 2));
  float* xml = (float*)lds_v0 + wr * 128;
  static_assert(DB * 16 * 64 * 4 <= STAGE / 2, "merge buffer must fit half a stage");
  if (grp == 1) {
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int r = 0; r < 16; ++r) xo[(db * 16 + r) * 64 + lane] = o_acc[db][r];
    }
    xml[lane] = m_run;
    xml[64 + lane] = l_part;
  }
  barrier();
  if (grp == 1) return;
  // Group 1's O^T: every LDS read issued before the first use, so their latencies overlap.
  float x1[DB][16];
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int r = 0; r < 16; ++r) x1[db][r] = xo[(db * 16 + r) * 64 + lane];
  }
  const float m1 = xml[lane];
  const float l1 = xml[64 + lane];
  __builtin_amdgcn_sched_barrier(0);
  const float m = vmax(m_run, m1);
  const float a0 = fast_exp2((m_run - m) * c);
  const float a1 = fast_exp2((m1 - m) * c);
  float la, lb;
  swap32(l_part * a0 + l1 * a1, la, lb);
  const float l_tot = la + lb;
  // Whole-row kernels at D = 128 and 160, and causal ones at D = 64, stage O through this
  // wave's merge region, so that each store instruction writes whole rows (16 bytes a lane)
  // instead of 8 bytes in each of 32 rows; every lane takes part in that exchange, rows
  // past S included.  It shortens the time to the last store (B1 H8 causal, D = 128:
  // S = 1024 -7 %, S = 8192 -0.7 %; D = 64: S = 2048 -6.6 %, S = 8192 -1 %; D = 160: -0.7 to
  // -2.8 %); the non-causal D = 64 kernels, two workgroups per CU, measured 3-10 % slower
  // with it.
  constexpr bool kStageOut = !SPLIT && (D == 128 || D == 160 || (D == 64 && CAUSAL));
  if (!kStageOut && TAIL && my_q >= S) return;
  const float inv = 1.0f / l_tot;
  const float w0s = a0 * inv, w1s = a1 * inv;
  if (SPLIT && slot >= 0) {
    // One chunk of a split block: its output normalised by its own l, in fp32, and
    // log2 of its softmax denominator in units of the scaled scores, m c + log2(l).
    float* prow = p.part_o + ((int64_t)slot * TM + (my_q - q0)) * D;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 o4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          o4[e] = o_acc[db][r] * w0s + x1[db][r] * w1s;
        }
        store_partial(p, prow + 32 * db + 8 * g + 4 * hl, o4);
      }
    }
    if (hl == 0) store_partial(p, p.part_lse + (int64_t)slot * TM + (my_q - q0), m * c + fast_log2(l_tot));
    return;
  }
  if constexpr (kStageOut && D == 160) {
    // 20 chunks a row: rows padded to 336 bytes instead of swizzled, so the 8-byte writes of
    // one instruction (one chunk, 32 rows) conflict only 2-way (rows 16 apart share banks);
    // the 16-byte reads run over the tile's 640 chunks in row-major order (a 2-way conflict
    // where a read pass crosses a row pad).
    char* ob = (char*)xo;
    constexpr int RBL = 2 * D + 16;  // LDS bytes per staged row
    constexpr int CPO = D / 8;       // 16-byte chunks per output row
    static_assert(32 * CPO % 64 == 0 && 32 * RBL <= STAGE / 2, "staged tile in the region");
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          o4[e] = o_acc[db][r] * w0s + x1[db][r] * w1s;
        }
        *(u32x2*)(ob + l32 * RBL + 16 * (4 * db + g) + 8 * hl) =
            u32x2{DTy::pack(o4[0], o4[1]), DTy::pack(o4[2], o4[3])};
      }
    }
    asm volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < 32 * CPO / 64; ++i) {
      const int idx = 64 * i + lane;
      const int row = idx / CPO;
      const int ch = idx - row * CPO;
      const u32x4 v = *(const u32x4*)(ob + row * RBL + 16 * ch);
      const int q = wq0 + row;
      if ((!TAIL || q < S) && 8 * ch < d_real) *(u32x4*)(op + (int64_t)q * p.o_ss + 8 * ch) = v;
    }
    return;
  } else if constexpr (kStageOut) {
    // 32 rows x 2D bytes in the wave's own merge region (its group-1 values are in
    // registers by now), 16-byte chunks swizzled per row as the K stages are (chunk ^
    // swz_k(row)): the 16-byte row-major reads are conflict-free and the 8-byte writes of
    // one instruction (one chunk, 32 rows) conflict 2-way (rows 16 apart share banks;
    // 64 cycles a wave).
    char* ob = (char*)xo;
    constexpr int RBO = 2 * D;
    constexpr int CPO = D / 8;      // 16-byte chunks per output row
    constexpr int RPI = 64 / CPO;   // rows per read instruction
#pragma unroll
    for (int db = 0; db < DB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float o4[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g + e;
          o4[e] = o_acc[db][r] * w0s + x1[db][r] * w1s;
        }
        const int ch = 4 * db + g;
        *(u32x2*)(ob + l32 * RBO + 16 * (ch ^ pp_swz_k<D>(l32)) + 8 * hl) =
            u32x2{DTy::pack(o4[0], o4[1]), DTy::pack(o4[2], o4[3])};
      }
    }
    asm volatile("" ::: "memory");
    const int ch = lane % CPO;
#pragma unroll
    for (int i = 0; i < 32 / RPI; ++i) {
      const int row = RPI * i + lane / CPO;
      const u32x4 v = *(const u32x4*)(ob + row * RBO + 16 * (ch ^ pp_swz_k<D>(row)));
      const int q = wq0 + row;
      if ((!TAIL || q < S) && 8 * ch < d_real) *(u32x4*)(op + (int64_t)q * p.o_ss + 8 * ch) = v;
    }
    return;
  }
  uint16_t* orow = op + (int64_t)my_q * p.o_ss;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float o4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * g + e;
        o4[e] = o_acc[db][r] * w0s + x1[db][r] * w1s;
      }
      const uint32_t w0 = DTy::pack(o4[0], o4[1]);
      const uint32_t w1 = DTy::pack(o4[2], o4[3]);
      const int d = 32 * db + 8 * g + 4 * hl;
      if (d < d_real) *(u32x2*)(orow + d) = u32x2{w0, w1};
    }
  }
}

// A workgroup's work: one query block of the whole-row grid, one chunk of the split grid,
// or (PAIR) the causal pair of query blocks nq - 1 - j and j of one head, one after the
// other, so that every pair has nq + 1 key steps (balanced without relying on the order in
// which the hardware hands out workgroups) and the grid is half as many workgroups; with
// SPLIT as well, the paired split (psplit_items): a light block whole and then the first
// chunk of its partner, or the partner's remaining steps.
// One workgroup per CU (LDS and registers).  The numbering (attn_fwd_split.h) regroups
// block ids per XCD with sched >= 1 (one head's K/V in one L2) and issues causal tiles
// heaviest first, so each CU takes the next tile when its current one ends and heavy
// tiles pair with light ones.  Split items cover a chunk of key steps of a block and
// leave a partial (slot >= 0) when the block has more than one chunk.
template <int DT, int D, bool CAUSAL, bool TAIL, bool SPLIT, bool PAIR, int TMR = 128, int LOWP_TN = 0>
__device__ __forceinline__ void attn_fwd_pp_body(const FwdParams& p) {
  constexpr int STAGE = pp_stage_bytes(D);
  // One array per (tensor, stage): the stage of every access is a compile-time constant
  // (the key loop is unrolled by two), so the compiler can tell the loads in flight into
  // one stage from the reads of the other and does not wait on the former for the latter.
  __shared__ __attribute__((aligned(1024))) char lds_k0[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds_k1[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds_v0[STAGE];
  __shared__ __attribute__((aligned(1024))) char lds_v1[STAGE];
  // In-kernel merge: whether this workgroup arrived last at its block, in the last word of
  // a stage (every stage access of the block has completed at the arrival, and the next
  // block's loads start only after the barrier that follows every wave's read of it; D = 160
  // fills the LDS).
  int* const s_last = (int*)(lds_v1 + STAGE - sizeof(int));
  const bool merge_here = SPLIT && p.merge_cnt != nullptr;
  if constexpr (PAIR) {
    static_assert(CAUSAL, "pairs of causal query blocks");
    WorkItem a, b;
    if constexpr (SPLIT)
      psplit_items(blockIdx.x, p.n_bh, p.n_qblk, p.sched, p.split_ns, &a, &b);
    else
      pair_items(blockIdx.x, p.n_bh, p.n_qblk, p.sched, &a, &b);
    attn_fwd_pp_block<DT, D, CAUSAL, TAIL, SPLIT>(p, a, lds_k0, lds_k1, lds_v0, lds_v1);
    if (b.qt >= 0) {
      // Every wave is past its last LDS access of the first block before the second
      // block's prologue loads overwrite the stages.
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
      attn_fwd_pp_block<DT, D, CAUSAL, TAIL, SPLIT>(p, b, lds_k0, lds_k1, lds_v0, lds_v1);
    }
    if (merge_here) {
      // At most one of a workgroup's items is a chunk of a cut block (psplit_items: the
      // heavy block's remainder as `a`, or its first chunk as `b`), and it is the last one.
      const WorkItem& w = b.qt >= 0 ? b : a;
      if (w.slot >= 0) split_arrive_and_merge<DT, D>(p, w, w.qt, 1, s_last);
    }
  } else {
    WorkItem wi;
    if constexpr (SPLIT && TMR == 64) {
      // Each item of the 128-row split numbering runs as two 64-row halves, the second half
      // of the grid taking the second halves (an item's halves land on the same XCD): the
      // same key chunk, rows 64 h .. 64 h + 63 of the block and of its partial slot.
      const int total = p.split_items * p.n_bh;
      const int half = (int)blockIdx.x >= total ? 1 : 0;
      wi = split_item((int)blockIdx.x - half * total, p.n_bh, p.split_items, p.sched, CAUSAL, p.split_c,
                      p.split_ns, p.split_slots, p.S);
      wi.qt = 2 * wi.qt + half;
    } else {
      wi = SPLIT ? split_item(blockIdx.x, p.n_bh, p.split_items, p.sched, CAUSAL, p.split_c, p.split_ns,
                              p.split_slots, p.S)
                 : whole_item(blockIdx.x, p.n_bh, p.n_qblk, p.sched, CAUSAL);
    }
    attn_fwd_pp_block<DT, D, CAUSAL, TAIL, SPLIT, TMR, LOWP_TN>(p, wi, lds_k0, lds_k1, lds_v0, lds_v1);
    if (merge_here && wi.slot >= 0)
      split_arrive_and_merge<DT, D>(p, wi, TMR == 64 ? wi.qt >> 1 : wi.qt, TMR == 64 ? 2 : 1, s_last);
  }
}

// Merge of the chunks of one split query block (after the split kernel on the same
// stream): per row, with L_i the chunks' log-sum-exps, O = sum_i 2^(L_i - max L) O_i /
// sum_i 2^(L_i - max L), the same rescale the online softmax applies between key tiles,
// here folded into one pass over the chunks (running max, weights rescaled when it grows).
// One thread per (row, 16-byte output chunk): a workgroup covers merge_rows_per_wg(D) rows
// (merge_threads(D) threads), so a split block takes 128 / merge_rows_per_wg(D)
// workgroups; the partial reads of the chunks are independent and contiguous across the
// D/8 threads of a row, and a row is written by those threads as one contiguous run.
// One (row, 16-byte output chunk) of a split block: the block's ns partials in slots
// slot0 .. slot0 + ns - 1 combined and written to O.
template <int DT, int D>
__device__ __forceinline__ void merge_row_chunk(const FwdParams& p, int bh, int qt, int slot0, int ns, int row,
                                                int c8) {
  constexpr int TM = kPPRows;
  using DTy = DType<DT>;
  const int q = qt * TM + row;
  if (q >= p.S || 8 * c8 >= p.d_real) return;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const float* lse = p.part_lse + (int64_t)slot0 * TM + row;
  const float* po = p.part_o + ((int64_t)slot0 * TM + row) * D + 8 * c8;
  float mx = lse[0];
  f32x4 acc0 = *(const f32x4*)po;
  f32x4 acc1 = *(const f32x4*)(po + 4);
  float wsum = 1.0f;
  for (int i = 1; i < ns; ++i) {
    const float li = lse[i * TM];
    const f32x4 x0 = *(const f32x4*)(po + (int64_t)i * TM * D);
    const f32x4 x1 = *(const f32x4*)(po + (int64_t)i * TM * D + 4);
    const float m_new = vmax(mx, li);
    const float a = fast_exp2(mx - m_new);  // rescale of what is summed so far
    const float w = fast_exp2(li - m_new);
    mx = m_new;
    wsum = wsum * a + w;
    acc0 = acc0 * a + w * x0;
    acc1 = acc1 * a + w * x1;
  }
  const float inv = 1.0f / wsum;
  const u32x4 o = {DTy::pack(acc0[0] * inv, acc0[1] * inv), DTy::pack(acc0[2] * inv, acc0[3] * inv),
                   DTy::pack(acc1[0] * inv, acc1[1] * inv), DTy::pack(acc1[2] * inv, acc1[3] * inv)};
  *(u32x4*)(p.o + b * p.o_sb + h * p.o_sh + (int64_t)q * p.o_ss + 8 * c8) = o;
}

template <int DT, int D, bool CAUSAL>
__device__ __forceinline__ void attn_merge_body(const FwdParams& p) {
  constexpr int TM = kPPRows;
  constexpr int CH = D / 8;        // 16-byte output chunks per row
  constexpr int RPW = merge_rows_per_wg(D);  // rows per workgroup
  constexpr int WPB = TM / RPW;              // workgroups per split block
  static_assert(merge_threads(D) <= 256 && TM % RPW == 0, "workgroups must cover whole rows");
  const int blk = blockIdx.x / WPB;
  const MergeItem mi = CAUSAL && p.split_c == kSplitPairs
                           ? psplit_merge_item(blk, p.n_qblk, p.split_ns)
                           : merge_item(blk, p.n_qblk, CAUSAL, p.split_c, p.split_ns, p.split_slots);
  const int row = (blockIdx.x - blk * WPB) * RPW + threadIdx.x / CH;
  merge_row_chunk<DT, D>(p, mi.bh, mi.qt, mi.slot0, mi.ns, row, threadIdx.x % CH);
}

// The merge of one split block by one workgroup (512 threads): thread t takes the
// (row, 16-byte chunk) items t, t + 512, ... of the block's 128 rows, with the merge
// kernel's arithmetic (merge_row_chunk: the same running max, the same order, so both give
// the same bits).  The loads of an item's chunks do not depend on the running sums, so
// with the chunk loop unrolled they are in flight together.
template <int DT, int D>
__device__ __forceinline__ void merge_block_in_kernel(const FwdParams& p, int bh, int qt, int slot0, int ns) {
  constexpr int TM = kPPRows;
  constexpr int CH = D / 8;
  constexpr int NI = (TM * CH + 511) / 512;  // items a thread
  using DTy = DType<DT>;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  int row[NI], c8[NI];
  bool ok[NI];
  const float* lse[NI];
  const float* po[NI];
  float mx[NI], wsum[NI];
  f32x4 acc0[NI], acc1[NI];
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int idx = threadIdx.x + 512 * j;
    row[j] = idx / CH;
    c8[j] = idx - row[j] * CH;
    ok[j] = idx < TM * CH && qt * TM + row[j] < p.S && 8 * c8[j] < p.d_real;
    const int r = ok[j] ? row[j] : 0;
    lse[j] = p.part_lse + (int64_t)slot0 * TM + r;
    po[j] = p.part_o + ((int64_t)slot0 * TM + r) * D + 8 * (ok[j] ? c8[j] : 0);
    mx[j] = load_partial(p, lse[j]);
    acc0[j] = load_partial4(p, po[j]);
    acc1[j] = load_partial4(p, po[j] + 4);
    wsum[j] = 1.0f;
  }
#pragma unroll 4
  for (int i = 1; i < ns; ++i) {
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const float li = load_partial(p, lse[j] + i * TM);
      const f32x4 x0 = load_partial4(p, po[j] + (int64_t)i * TM * D);
      const f32x4 x1 = load_partial4(p, po[j] + (int64_t)i * TM * D + 4);
      const float m_new = vmax(mx[j], li);
      const float a = fast_exp2(mx[j] - m_new);
      const float w = fast_exp2(li - m_new);
      mx[j] = m_new;
      wsum[j] = wsum[j] * a + w;
      acc0[j] = acc0[j] * a + w * x0;
      acc1[j] = acc1[j] * a + w * x1;
    }
  }
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    if (!ok[j]) continue;
    const float inv = 1.0f / wsum[j];
    const u32x4 o = {DTy::pack(acc0[j][0] * inv, acc0[j][1] * inv), DTy::pack(acc0[j][2] * inv, acc0[j][3] * inv),
                     DTy::pack(acc1[j][0] * inv, acc1[j][1] * inv), DTy::pack(acc1[j][2] * inv, acc1[j][3] * inv)};
    *(u32x4*)(p.o + b * p.o_sb + h * p.o_sh + (int64_t)(qt * TM + row[j]) * p.o_ss + 8 * c8[j]) = o;
  }
}

// In-kernel merge of a split launch (p.merge_cnt set; no merge kernel follows): after a
// workgroup has written its chunk's partial (its slot's rows of part_o and part_lse), it
// counts itself in at the block's counter; the workgroup that arrives last, which knows
// that every chunk's partial is in memory, combines them into O.  `per_chunk` workgroups
// write each chunk (two 64-row halves on the 64-row split), so a block of ns chunks counts
// per_chunk * ns arrivals.  The counter wraps to zero on the last arrival (atomicInc), so
// it is zero again for the launch after.  Visibility across CUs and XCDs: the partials are
// stored and loaded at agent scope (store_partial / load_partial, SC1); every wave's stores
// have completed (vmcnt 0) before the workgroup barrier that precedes the increment, and
// the last workgroup loads them only after its increment has returned, so every chunk's
// stores completed before the loads are issued.  Every wave of the workgroup runs this
// (uniform: the item is the workgroup's), so its two barriers match.
template <int DT, int D>
__device__ __forceinline__ void split_arrive_and_merge(const FwdParams& p, const WorkItem& w, int qt128,
                                                       int per_chunk, int* s_last) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // this wave's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned last = (unsigned)(per_chunk * w.ns) - 1u;
    const unsigned old = atomicInc(p.merge_cnt + w.slot0, last);
    *s_last = old == last ? 1 : 0;
  }
  __syncthreads();
  if (*s_last == 0) return;
  merge_block_in_kernel<DT, D>(p, w.bh, qt128, w.slot0, w.ns);
}
}  // namespace ta

// Arrival counters of the in-kernel merge (FwdParams::merge_cnt points into one region).
// The host zeroes them once when it loads this code object; every launch leaves them zero.
__device__ unsigned ta_merge_counters[ta::kMergeRegions * ta::kMergeRegionCounters];

// Two extern "C" entries per (dtype, D, causal, tail): the whole-row kernel
// ta_fwd_pp_<f16|bf16>_d<D>_c<0|1>_t<0|1> and the split-key-range kernel
// ta_fwd_pp_split_<...>; 512 threads, one workgroup per CU (two for non-causal D = 64
// whole rows).
// Non-causal D = 64 whole-row kernels are built for two workgroups per CU (at most 128
// VGPRs; LDS 2 x 64 KiB): four waves per SIMD give the VALU-heavy D = 64 softmax more waves
// to issue from (C4 D=64 +7 %).  Causal ones stay at one per CU, where each CU takes the
// next, lighter tile as its heavy one ends (two resident from the start measured 5 % slower
// on B1 H8 S8192), and so do the split kernels, the residency the split planner models.
#define TA_PP_WAVES(D, C) ((D) == 64 && (C) == 0 ? 4 : 2)
#define TA_PP_DEFINE(DTN, DT, D, C, T)                                                    \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(TA_PP_WAVES(D, C), TA_PP_WAVES(D, C))))           \
      ta_fwd_pp_##DTN##_d##D##_c##C##_t##T(ta::FwdParams p) {                              \
    ta::attn_fwd_pp_body<DT, D, (C != 0), (T != 0), false, false>(p);                     \
  }                                                                                       \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(2, 2)))                                          \
      ta_fwd_pp_split_##DTN##_d##D##_c##C##_t##T(ta::FwdParams p) {                        \
    ta::attn_fwd_pp_body<DT, D, (C != 0), (T != 0), true, false>(p);                      \
  }

// Causal query-block pairs (whole rows, D = 64, 96 and 128): ta_fwd_pp_pair_<f16|bf16>_d<D>_c1_t<0|1>.
#define TA_PP_PAIR_DEFINE(DTN, DT, D, T)                                                   \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(2, 2)))                                          \
      ta_fwd_pp_pair_##DTN##_d##D##_c1_t##T(ta::FwdParams p) {                             \
    ta::attn_fwd_pp_body<DT, D, true, (T != 0), false, true>(p);                          \
  }

// Paired split (causal, D = 64, 96, 128 and 160): ta_fwd_pp_psplit_<f16|bf16>_d<D>_c1_t<0|1>,
// merged by ta_fwd_merge_<...>_c1.
#define TA_PP_PSPLIT_DEFINE(DTN, DT, D, T)                                                 \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(2, 2)))                                          \
      ta_fwd_pp_psplit_##DTN##_d##D##_c1_t##T(ta::FwdParams p) {                           \
    ta::attn_fwd_pp_body<DT, D, true, (T != 0), true, true>(p);                           \
  }

// 256-row blocks (non-causal whole rows, fp32 accumulation, D = 64 and 128; the C ABI picks
// them for grids of two or more blocks per CU): ta_fwd_pp256_<f16|bf16>_d<D>_c0_t<0|1>.
#define TA_PP256_DEFINE(DTN, DT, D, T)                                                     \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(2, 2)))                                          \
      ta_fwd_pp256_##DTN##_d##D##_c0_t##T(ta::FwdParams p) {                               \
    ta::attn_fwd_pp_body<DT, D, false, (T != 0), false, false, 256>(p);                   \
  }

// 64-row blocks (tiles (64, 64) and (64, 128) with fp32 accumulation, D = 64, 96, 128 and 160):
// ta_fwd_pp64_<f16|bf16>_d<D>_c<0|1>_t<0|1>.  Two workgroups per CU at D = 64, causal or not
// (104 VGPRs; causal B1 H8 S8192 bf16 87.2 -> 81.1 us, B4 H16 S4096 194.3 -> 171.0 us, small
// grids within 1 %, outputs bit-identical); one at D = 96-160, whose stages fill the LDS.
#define TA_PP64_DEFINE(DTN, DT, D, C, T)                                                   \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu((D) == 64 ? 4 : 2, (D) == 64 ? 4 : 2)))           \
      ta_fwd_pp64_##DTN##_d##D##_c##C##_t##T(ta::FwdParams p) {                            \
    ta::attn_fwd_pp_body<DT, D, (C != 0), (T != 0), false, false, 64>(p);                 \
  }
// Their split-key-range form (ta_fwd_pp64_split_<...>): the 128-row split numbering, each
// item as two 64-row halves, partials in the 128-row slots the merge kernel reads.
#define TA_PP64_SPLIT_DEFINE(DTN, DT, D, C, T)                                             \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(2, 2)))                                          \
      ta_fwd_pp64_split_##DTN##_d##D##_c##C##_t##T(ta::FwdParams p) {                      \
    ta::attn_fwd_pp_body<DT, D, (C != 0), (T != 0), true, false, 64>(p);                  \
  }
#define TA_PP64_DEFINE_CT(DTN, DT, D)   \
  TA_PP64_DEFINE(DTN, DT, D, 0, 0)      \
  TA_PP64_DEFINE(DTN, DT, D, 0, 1)      \
  TA_PP64_DEFINE(DTN, DT, D, 1, 0)      \
  TA_PP64_DEFINE(DTN, DT, D, 1, 1)      \
  TA_PP64_SPLIT_DEFINE(DTN, DT, D, 0, 0) \
  TA_PP64_SPLIT_DEFINE(DTN, DT, D, 0, 1) \
  TA_PP64_SPLIT_DEFINE(DTN, DT, D, 1, 0) \
  TA_PP64_SPLIT_DEFINE(DTN, DT, D, 1, 1)

// Input-dtype accumulation (D = 64 and 128, whole rows), one kernel per TILE_N (the keys of
// a wave's slice between roundings of O): ta_fwd_ppl_n<TN>_<f16|bf16>_d<D>_c_t (128-row
// blocks, tiles (128, TN)) and ta_fwd_ppl64_n<TN>_<...> (64-row blocks, tiles (64, TN)).
// Two workgroups per CU for the 64-row kernels at D = 64 (113-123 VGPRs at that bound; one
// at D = 128, where the LDS takes the CU): the second workgroup's waves to issue from make
// them faster, outputs bit-identical (C4 D = 64 bf16 tile (64, 64) 613 -> 690 TFLOP/s, causal
// B1 H8 S8192 bf16 127.9 -> 108.8 us).  The 128-row kernels stay at one: at 128 VGPRs they
// spill 6-15 registers to scratch.
#define TA_PPL_WAVES(D, C, TMR) ((D) == 64 && (TMR) == 64 ? 4 : 2)
#define TA_PPL_DEFINE(NAME, TN, DTN, DT, D, C, T, TMR)                                      \
  extern "C" __global__ void __launch_bounds__(512)                                       \
      __attribute__((amdgpu_waves_per_eu(TA_PPL_WAVES(D, C, TMR), TA_PPL_WAVES(D, C, TMR)))) \
      ta_fwd_##NAME##_n##TN##_##DTN##_d##D##_c##C##_t##T(ta::FwdParams p) {                \
    ta::attn_fwd_pp_body<DT, D, (C != 0), (T != 0), false, false, TMR, TN>(p);            \
  }
#define TA_PPL_DEFINE_TCT(NAME, TN, DTN, DT, D, TMR) \
  TA_PPL_DEFINE(NAME, TN, DTN, DT, D, 0, 0, TMR)     \
  TA_PPL_DEFINE(NAME, TN, DTN, DT, D, 0, 1, TMR)     \
  TA_PPL_DEFINE(NAME, TN, DTN, DT, D, 1, 0, TMR)     \
  TA_PPL_DEFINE(NAME, TN, DTN, DT, D, 1, 1, TMR)
#define TA_PPL_DEFINE_CT(DTN, DT, D)              \
  TA_PPL_DEFINE_TCT(ppl, 64, DTN, DT, D, 128)     \
  TA_PPL_DEFINE_TCT(ppl, 128, DTN, DT, D, 128)    \
  TA_PPL_DEFINE_TCT(ppl64, 64, DTN, DT, D, 64)    \
  TA_PPL_DEFINE_TCT(ppl64, 128, DTN, DT, D, 64)

// Merge kernels of the split path: ta_fwd_merge_<f16|bf16>_d<D>_c<0|1>, merge_threads(D)
// threads.
#define TA_MERGE_DEFINE(DTN, DT, D, C)                                                     \
  extern "C" __global__ void __launch_bounds__(256) ta_fwd_merge_##DTN##_d##D##_c##C(      \
      ta::FwdParams p) {                                                                  \
    ta::attn_merge_body<DT, D, (C != 0)>(p);                                              \
  }

#define TA_PP_DEFINE_CT(DTN, DT, D) \
  TA_PP_DEFINE(DTN, DT, D, 0, 0)    \
  TA_PP_DEFINE(DTN, DT, D, 0, 1)    \
  TA_PP_DEFINE(DTN, DT, D, 1, 0)    \
  TA_PP_DEFINE(DTN, DT, D, 1, 1)    \
  TA_MERGE_DEFINE(DTN, DT, D, 0)    \
  TA_MERGE_DEFINE(DTN, DT, D, 1)

TA_PP_DEFINE_CT(f16, 0, 64)
TA_PP_DEFINE_CT(f16, 0, 96)
TA_PP_DEFINE_CT(f16, 0, 128)
TA_PP_DEFINE_CT(f16, 0, 160)
TA_PP_DEFINE_CT(bf16, 1, 64)
TA_PP_DEFINE_CT(bf16, 1, 96)
TA_PP_DEFINE_CT(bf16, 1, 128)
TA_PP_DEFINE_CT(bf16, 1, 160)
TA_PP_PAIR_DEFINE(f16, 0, 64, 0)
TA_PP_PAIR_DEFINE(f16, 0, 64, 1)
TA_PP_PAIR_DEFINE(f16, 0, 96, 0)
TA_PP_PAIR_DEFINE(f16, 0, 96, 1)
TA_PP_PAIR_DEFINE(f16, 0, 128, 0)
TA_PP_PAIR_DEFINE(f16, 0, 128, 1)
TA_PP_PAIR_DEFINE(bf16, 1, 64, 0)
TA_PP_PAIR_DEFINE(bf16, 1, 64, 1)
TA_PP_PAIR_DEFINE(bf16, 1, 96, 0)
TA_PP_PAIR_DEFINE(bf16, 1, 96, 1)
TA_PP_PAIR_DEFINE(bf16, 1, 128, 0)
TA_PP_PAIR_DEFINE(bf16, 1, 128, 1)
TA_PP_PSPLIT_DEFINE(f16, 0, 64, 0)
TA_PP_PSPLIT_DEFINE(f16, 0, 64, 1)
TA_PP_PSPLIT_DEFINE(f16, 0, 96, 0)
TA_PP_PSPLIT_DEFINE(f16, 0, 96, 1)
TA_PP_PSPLIT_DEFINE(f16, 0, 128, 0)
TA_PP_PSPLIT_DEFINE(f16, 0, 128, 1)
TA_PP_PSPLIT_DEFINE(f16, 0, 160, 0)
TA_PP_PSPLIT_DEFINE(f16, 0, 160, 1)
TA_PP_PSPLIT_DEFINE(bf16, 1, 64, 0)
TA_PP_PSPLIT_DEFINE(bf16, 1, 64, 1)
TA_PP_PSPLIT_DEFINE(bf16, 1, 96, 0)
TA_PP_PSPLIT_DEFINE(bf16, 1, 96, 1)
TA_PP_PSPLIT_DEFINE(bf16, 1, 128, 0)
TA_PP_PSPLIT_DEFINE(bf16, 1, 128, 1)
TA_PP_PSPLIT_DEFINE(bf16, 1, 160, 0)
TA_PP_PSPLIT_DEFINE(bf16, 1, 160, 1)
TA_PP256_DEFINE(f16, 0, 64, 0)
TA_PP256_DEFINE(f16, 0, 64, 1)
TA_PP256_DEFINE(f16, 0, 128, 0)
TA_PP256_DEFINE(f16, 0, 128, 1)
TA_PP256_DEFINE(bf16, 1, 64, 0)
TA_PP256_DEFINE(bf16, 1, 64, 1)
TA_PP256_DEFINE(bf16, 1, 128, 0)
TA_PP256_DEFINE(bf16, 1, 128, 1)
TA_PP64_DEFINE_CT(f16, 0, 64)
TA_PP64_DEFINE_CT(f16, 0, 96)
TA_PP64_DEFINE_CT(f16, 0, 128)
TA_PP64_DEFINE_CT(f16, 0, 160)
TA_PP64_DEFINE_CT(bf16, 1, 64)
TA_PP64_DEFINE_CT(bf16, 1, 96)
TA_PP64_DEFINE_CT(bf16, 1, 128)
TA_PP64_DEFINE_CT(bf16, 1, 160)
TA_PPL_DEFINE_CT(f16, 0, 64)
TA_PPL_DEFINE_CT(f16, 0, 128)
TA_PPL_DEFINE_CT(bf16, 1, 64)
TA_PPL_DEFINE_CT(bf16, 1, 128)
