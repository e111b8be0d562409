// SDPA forward for CDNA4 (gfx950), fp32 accumulation, short rows: 32 query rows per
// workgroup, the key range split across its eight waves.
//
// Math: the reference's tiled forward with fp32 accumulation
// (src/tiledattention/kernels/flash_fwd.py:374-446): per query row (m, l, acc) over the
// keys, then acc / l.  Here each wave keeps its own (m, l, acc) over its keys and the eight
// states of a row are combined once at the end (m = max, weights 2^((m_w - m) c)), the same
// rescale the online softmax applies between key tiles.
//
// Layout and schedule (this file's own), for the grids where the eight-wave kernel's chain
// of 128-key steps is the latency (few query blocks, at most ~1-2 K keys a row):
//
// * A pass covers 512 keys at D = 128 (1024 at D = 64): wave w takes keys
//   [512 p + 64 w, + 64) (128 at D = 64), 2 (4) blocks of 32 keys.  LDS holds a pass as
//   128 KiB of 128-key stages in the eight-wave kernel's swizzled layout (the same K and
//   transposed V reads).
// * Every wave loads exactly the rows it reads (direct-to-LDS buffer loads, 16 bytes a
//   lane, 1 KiB a wave instruction; rows past the block's last key read as zero) and waits
//   only for its own loads: K of its keys, then S^T = K Q^T, then V of its keys over the
//   same rows, issued as soon as its K reads are done and landing under its softmax, then
//   O^T += V^T P^T.  Only the Q tile (one barrier before the first S) and the final merge
//   are shared, so no wave waits for another's loads.
// * Softmax per pass with the exact running max (P = 2^(s c - m c) <= 1 packs to either
//   input dtype; O and l are rescaled when a later pass raises m), l summed from the
//   rounded P that the P.V MFMAs use.
// * Merge: every wave writes its O (fp32, 16-byte chunks XOR-swizzled by row), m and l as
//   soon as its own P.V is done, over its own rows of the stages; after one barrier each
//   wave sums the eight states of 4 rows with the weights 2^((m_w - m) c) and stores them,
//   divided by the weighted sum of l.
//
// One workgroup per CU (138 KiB of LDS); the host runs it when its grid of 32-row blocks
// fits one round of the CUs.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_fwd_common.h"
#include "attn_fwd_params.h"

namespace ta {

template <int DT, int D, bool CAUSAL, bool TAIL>
__device__ __forceinline__ void attn_fwd_wide_body(const FwdParams& p) {
  static_assert(D == 64 || D == 128, "wide kernel: D 64 or 128");
  constexpr int TK = 128;                // key rows per stage
  constexpr int RB = 2 * D;              // LDS bytes per key row
  constexpr int STAGE = TK * RB;         // 32 KiB (D = 128), 16 KiB (D = 64)
  constexpr int REGION = 128 * 1024;     // the stages of one pass
  constexpr int NST = REGION / STAGE;    // stages per pass: 4 / 8
  constexpr int PK = NST * TK;           // keys per pass: 512 / 1024
  constexpr int KW = PK / 8;             // keys per wave per pass: 64 / 128
  constexpr int KB = KW / 32;            // 32-key blocks per wave: 2 / 4
  constexpr int DK = D / 16;             // k-steps of S^T = K Q^T
  constexpr int DB = D / 32;             // 32-wide d blocks of O
  constexpr int CPR = D / 8;             // 16-byte chunks per key row
  constexpr int RPL = 1024 / RB;         // key rows per 1 KiB chunk: 4 / 8
  constexpr int OWN = KW / RPL;          // 1 KiB chunks of a wave's rows: 16
  constexpr int QCH = 32 * RB / 1024;    // 1 KiB chunks of the Q tile: 8 / 4
  constexpr int SLOT = OWN * 1024;       // a wave's own rows of the stages: 16 KiB
  static_assert(32 * D * 4 <= SLOT && 8 * SLOT == REGION && QCH <= 8,
                "a wave's fp32 O fits its own rows; Q chunks <= waves");
  __shared__ __attribute__((aligned(1024))) char region[REGION];
  __shared__ __attribute__((aligned(1024))) char lds_q[32 * RB];
  __shared__ float ml[2][8][32];  // per wave and row: m, then 2^((m_w - m) c) l_w
  using DTy = DType<DT>;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: kept in SGPRs
  const int l32 = lane & 31;
  const int hl = lane >> 5;

  // ---- the block: (bh, 32-row query block), the longest (causal: last) blocks first
  const int S = p.S;
  const int nqb = p.n_qblk;  // 32-row blocks a head
  const int bh = (int)(blockIdx.x % (unsigned)p.n_bh);
  const int qb = nqb - 1 - (int)(blockIdx.x / (unsigned)p.n_bh);
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const uint16_t* __restrict__ qp = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* __restrict__ kp = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* __restrict__ vp = p.v + b * p.v_sb + h * p.v_sh;
  uint16_t* __restrict__ op = p.o + b * p.o_sb + h * p.o_sh;
  const int k_rb = (int)p.k_ss * 2;  // global row bytes
  const int v_rb = (int)p.v_ss * 2;
  const int q_rb = (int)p.q_ss * 2;
  const int d_real = p.d_real;  // columns at or past it read as zero and are not written
  const float c = p.scale_log2;

  const int q0 = 32 * qb;
  const int my_q = q0 + l32;  // this lane's query row
  const int key_end = CAUSAL ? min(S, q0 + 32) : S;
  const int n_pass = (key_end + PK - 1) / PK;

  const int kw0 = wave * KW;  // this wave's keys of a pass: kbase + kw0 .. + KW,
  const int sw = kw0 / TK;    // rows koff .. koff + KW of stage sw
  const int koff = kw0 % TK;

  auto wait_vm = [&]() { __builtin_amdgcn_s_waitcnt(0x0F70); };  // vmcnt(0)
  auto wait_lds = [&]() {                                          // lgkmcnt(0)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    asm volatile("" ::: "memory");
  };
  auto barrier = [&]() {
    wait_lds();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };

  // ---- loads: 1 KiB chunk g of a stage holds rows g RPL .. + RPL; lane l writes physical
  // chunk l % CPR of row g RPL + l / CPR, i.e. loads that row's logical chunk
  // (l % CPR) ^ swz(row).  A logical chunk at or past d_real gets an offset of 2^31 or more,
  // outside every resource here (each spans less than 2^31 bytes), so it reads zero.
  constexpr int kZeroChunk = INT32_MIN;
  auto chunk_off = [&](int g, int rb, bool is_k) {
    const int row = g * RPL + lane / CPR;
    const int lc = (lane % CPR) ^ (is_k ? pp_swz_k<D>(row) : pp_swz_v<D>(row));
    return 8 * lc < d_real ? (lane / CPR) * rb + (lc << 4) : kZeroChunk;
  };
  // A wave's chunks are koff / RPL + i (i < OWN) of stage sw; the K swizzle of chunk i
  // depends on i only through i % 4 (D = 128) or i % 2 (D = 64), V's not at all.
  constexpr int KPH = D == 128 ? 4 : 2;
  int kvo[KPH];
#pragma unroll
  for (int i = 0; i < KPH; ++i) kvo[i] = chunk_off(koff / RPL + i, k_rb, true);
  const int vvo = chunk_off(koff / RPL, v_rb, false);
  // This wave's rows of K or V for the pass at kbase; rows at or past key_end read as zero.
  auto load_own = [&](const uint16_t* gbase, int64_t row_stride, int rb, bool is_k, int kbase) {
    const int wk0 = kbase + kw0;
    const __amdgpu_buffer_rsrc_t r = row_rsrc(gbase + (int64_t)wk0 * row_stride, key_end - wk0, rb);
#pragma unroll
    for (int i = 0; i < OWN; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          r, (__attribute__((address_space(3))) void*)(region + sw * STAGE + (koff / RPL + i) * 1024), 16,
          (is_k ? kvo[i % KPH] : vvo) + i * RPL * rb, 0, 0, 0);
    }
  };

  // ---- LDS reads (the eight-wave kernel's operand layouts) -----------------------------
  // K: lane reads row koff + 32 bk + l32 at logical chunk 2 kk + hl; the Q tile (rows l32)
  // likewise.  V^T via the transposed read: lane l of 16-lane group G addresses row
  // 4 hl + (l % 16) / 4 of a 16-key chunk and d = 32 db + 16 (G % 2) + 4 (l % 4).
  const int mk = pp_swz_k<D>(l32);
  const int q_rd = l32 * RB + 32 * (mk >> 1) + 16 * (hl ^ (mk & 1));
  const int k_rd = koff * RB + q_rd;
  const int tr_r = (lane & 15) >> 2;
  const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const int v_rd = (koff + 4 * hl + tr_r) * RB + 16 * ((tr_d >> 3) ^ pp_swz_v<D>(4 * hl + tr_r)) + 2 * (tr_d & 7);
  const char* st = region + sw * STAGE;

  // Issue order of a run of N MFMAs whose operands come from LDS (RPM reads each): the
  // reads of the first AHEAD MFMAs, then each MFMA followed by the reads of the MFMA AHEAD
  // places later, so that no MFMA waits on a read issued just before it.
  auto run_order = [&](auto n_tag, auto rpm_tag) {
    constexpr int N = decltype(n_tag)::value;
    constexpr int RPM = decltype(rpm_tag)::value;
    constexpr int AHEAD = 4;
    __builtin_amdgcn_sched_group_barrier(0x100, AHEAD * RPM, 0);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (i + AHEAD < N) __builtin_amdgcn_sched_group_barrier(0x100, RPM, 0);
    }
  };

  // ---- state (lane = query l32 of the block, half hl of each 32-key block's keys) -------
  u32x4 qf[DK];  // B operand of S^T = K Q^T
  float m_run = kNegLarge;
  float l_part = 0.0f;
  f32x16 o_acc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db) o_acc[db] = f32x16{};
  f32x16 s[KB];
  uint32_t pk[KB][8];  // packed P, B operand of O^T += V^T P^T

  for (int ps = 0; ps < n_pass; ++ps) {
    const int kbase = ps * PK;
    const int wk0 = kbase + kw0;  // this wave's first key of the pass
    const bool active = wk0 < key_end;
    if (ps == 0) {
      // The Q tile (rows past S read as zero), one chunk a wave, issued before the wave's
      // K so that waiting for all but the K loads waits for it.
      if (wave < QCH) {
        const __amdgpu_buffer_rsrc_t r = row_rsrc(qp + (int64_t)q0 * p.q_ss, S - q0, q_rb);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(lds_q + wave * 1024),
                                                 16, chunk_off(wave, q_rb, true) + wave * RPL * q_rb, 0, 0, 0);
      }
      if (active) {
        load_own(kp, p.k_ss, k_rb, true, kbase);
        __builtin_amdgcn_s_waitcnt(0x0F70 | (OWN & 15) | ((OWN >> 4) << 14));  // vmcnt(OWN)
      } else {
        wait_vm();
      }
      barrier();  // the Q tile
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) qf[kk] = *(const u32x4*)(lds_q + (q_rd ^ (32 * kk)));
    } else if (active) {
      load_own(kp, p.k_ss, k_rb, true, kbase);
    }
    if (active) {
      wait_vm();  // this wave's K rows
      asm volatile("" ::: "memory");
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
          const u32x4 a = *(const u32x4*)(st + bk * 32 * RB + (k_rd ^ (32 * kk)));
          s[bk] = DTy::mfma(a, qf[kk], kk == 0 ? f32x16{} : s[bk]);
        }
      }
      run_order(std::integral_constant<int, DK * KB>{}, std::integral_constant<int, 1>{});
      wait_lds();  // its K reads are done: its V over the same rows
      load_own(vp, p.v_ss, v_rb, false, kbase);

      // mask (keys past the row, causal; past S, ragged non-causal), exact max, P, l
      const bool need_mask = (CAUSAL && wk0 + KW - 1 > q0) || (TAIL && wk0 + KW > S);
      if (need_mask) {
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = wk0 + 32 * bk + (r >> 2) * 8 + hl * 4 + (r & 3);
            bool bad = false;
            if (CAUSAL) bad = key > my_q;
            if (TAIL) bad = bad || key >= S;
            s[bk][r] = bad ? kMasked : s[bk][r];
          }
        }
      }
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
      const float m_new = vmax(m_run, vmax(a0, a1));  // a row whose keys are all masked keeps m
      if (ps > 0 && __ballot(m_new > m_run)) {
        const float alpha = fast_exp2((m_run - m_new) * c);
#pragma unroll
        for (int db = 0; db < DB; ++db) o_acc[db] *= alpha;
        l_part *= alpha;
      }
      m_run = m_new;
      const float mc = m_new * c;
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          pk[bk][r >> 1] = DTy::pack(fast_exp2(__builtin_fmaf(s[bk][r], c, -mc)),
                                     fast_exp2(__builtin_fmaf(s[bk][r + 1], c, -mc)));
        }
      }
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
        for (int i = 0; i < 8; ++i) l_part = DTy::sum2(pk[bk][i], l_part);
      }

      wait_vm();  // this wave's V rows
      asm volatile("" ::: "memory");
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
          const u32x4 bfrag = {pk[bk][4 * kc + 0], pk[bk][4 * kc + 1], pk[bk][4 * kc + 2], pk[bk][4 * kc + 3]};
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const char* a0p = st + (v_rd ^ (64 * db)) + (32 * bk + 16 * kc) * RB;
            s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a0p);
            s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0p + 8 * RB));
            u32x2 w0 = __builtin_bit_cast(u32x2, r0);
            u32x2 w1 = __builtin_bit_cast(u32x2, r1);
            const u32x4 a = {w0[0], w0[1], w1[0], w1[1]};
            o_acc[db] = DTy::mfma(a, bfrag, o_acc[db]);
          }
        }
      }
      run_order(std::integral_constant<int, KB * 2 * DB>{}, std::integral_constant<int, 2>{});
      wait_lds();  // its V reads are done before the next pass's K over the same rows
    }
  }

  // ---- merge of the eight waves' states of each row -----------------------------------
  // Each wave writes its O (unweighted, fp32), m and l as soon as its last P.V is done: O
  // into its own rows of the stages (bytes [16 w, 16 w + 16) KiB, which no other wave reads
  // or loads), m and l beside; one barrier, then wave w sums rows 4 w .. 4 w + 3 of the
  // eight states with the weights 2^((m_w - m) c), m = max_w m_w.  A wave that never had a
  // key keeps m = kNegLarge, l = 0, O = 0: its weight is 0 (every row has at least one key,
  // so the row max is a real score).
  float la, lb;
  swap32(l_part, la, lb);
  if (hl == 0) {
    ml[0][wave][l32] = m_run;
    ml[1][wave][l32] = la + lb;
  }
  // O^T lane layout: row l32, d = 32 db + 8 g + 4 hl + e (e < 4): 16-byte chunk
  // ch = 8 db + 2 g + hl of the row, stored at chunk ch ^ (row & 15) (conflict-free)
  char* part = region + wave * SLOT;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int ch = 8 * db + 2 * g + hl;
      *(f32x4*)(part + l32 * (D * 4) + 16 * (ch ^ (l32 & 15))) =
          f32x4{o_acc[db][4 * g], o_acc[db][4 * g + 1], o_acc[db][4 * g + 2], o_acc[db][4 * g + 3]};
    }
  }
  barrier();
  // lane l takes row 4 w + l / 16 and the D / 16 columns from (l % 16) D / 16
  constexpr int VPL = D / 16;   // values per lane: 8 / 4
  constexpr int CPL = VPL / 4;  // 16-byte chunks per lane: 2 / 1
  const int row = 4 * wave + (lane >> 4);
  const int ch0 = (lane & 15) * CPL;
  float mx = ml[0][0][row];
#pragma unroll
  for (int w = 1; w < 8; ++w) mx = vmax(mx, ml[0][w][row]);
  float acc[VPL];
#pragma unroll
  for (int e = 0; e < VPL; ++e) acc[e] = 0.0f;
  float lsum = 0.0f;
#pragma unroll
  for (int w = 0; w < 8; ++w) {
    const float aw = fast_exp2((ml[0][w][row] - mx) * c);
    lsum += aw * ml[1][w][row];
    const char* pw = region + w * SLOT + row * (D * 4);
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) {
      const f32x4 v = *(const f32x4*)(pw + 16 * ((ch0 + cc) ^ (row & 15)));
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[4 * cc + e] += aw * v[e];
    }
  }
  const float inv = 1.0f / lsum;
  const int q = q0 + row;
  const int col = 4 * ch0;
  if ((!TAIL || q < S) && col < d_real) {
    uint32_t w2[VPL / 2];
#pragma unroll
    for (int e = 0; e < VPL / 2; ++e) w2[e] = DTy::pack(acc[2 * e] * inv, acc[2 * e + 1] * inv);
    uint16_t* dst = op + (int64_t)q * p.o_ss + col;
    if constexpr (VPL == 8) {
      *(u32x4*)dst = u32x4{w2[0], w2[1], w2[2], w2[3]};
    } else {
      *(u32x2*)dst = u32x2{w2[0], w2[1]};
    }
  }
}

}  // namespace ta

// ta_fwd_wide_<dtype>_d<D>_c<causal>_t<tail>: one workgroup of 512 threads per (b, h, 32-row
// query block), grid B * H * ceil(S / 32).  The t0 variants need S to be a multiple of 32,
// and non-causal ones a multiple of a wave's keys per pass (64 at D = 128, 128 at D = 64).
#define TA_WIDE_DEFINE(DTN, DT, D, C, T)                                                     \
  extern "C" __global__ __launch_bounds__(512, 1) void ta_fwd_wide_##DTN##_d##D##_c##C##_t##T( \
      ta::FwdParams p) {                                                                     \
    ta::attn_fwd_wide_body<DT, D, (C != 0), (T != 0)>(p);                                    \
  }
#define TA_WIDE_DEFINE_CT(DTN, DT, D) \
  TA_WIDE_DEFINE(DTN, DT, D, 0, 0)   \
  TA_WIDE_DEFINE(DTN, DT, D, 0, 1)   \
  TA_WIDE_DEFINE(DTN, DT, D, 1, 0)   \
  TA_WIDE_DEFINE(DTN, DT, D, 1, 1)

TA_WIDE_DEFINE_CT(f16, 0, 64)
TA_WIDE_DEFINE_CT(f16, 0, 128)
TA_WIDE_DEFINE_CT(bf16, 1, 64)
TA_WIDE_DEFINE_CT(bf16, 1, 128)
