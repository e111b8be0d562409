// SDPA forward for CDNA4 (gfx950): online-softmax attention over K/V tiles.
//
// Math follows the reference's tiled forward (src/tiledattention/kernels/flash_fwd.py:374-446
// for fp32 accumulation, :301-372 for input-dtype accumulation, :533-574 / :486-531 for the
// unmasked "aligned" forms): per query tile keep (m, l, acc), stream K/V tiles, and finish with
// acc / l.  The schedule and data layout below are this file's own, written for CDNA4:
//
// * One workgroup owns TM query rows; each of its TM/32 waves owns 32 rows.
// * Scores are computed transposed, S^T = K * Q^T, with v_mfma_f32_32x32x16_{f16,bf16}:
//   A = K (rows = keys, from LDS), B = Q^T (columns = queries, held in VGPRs for the whole
//   key loop).  In the 32x32 accumulator lane l then holds query (l % 32) and 16 of the
//   block's 32 keys, so the row max / row sum are in-lane plus one lane<->lane^32 exchange
//   (v_permlane32_swap).
// * O is computed transposed too, O^T += V^T * P^T: A = V^T read with ds_read_b64_tr_b16
//   from the row-major V tile, B = P^T straight from the score registers (after packing to
//   the input dtype).  The key order P carries in its registers is a fixed permutation and
//   the transposed V reads use the same permutation, so no lane shuffle is needed.  Each
//   lane again holds one query, so the per-query rescale by alpha and the final 1/l are
//   lane-local.
// * K/V tiles go HBM -> VGPR -> LDS through two LDS stages (one for the 64-row tiles):
//   tile t+1 is fetched (buffer loads, range-checked so rows past S read as zero) while
//   tile t is consumed; one barrier per tile (two with one stage).  LDS rows are padded (K: 2D+16 bytes, V: 2D+64 bytes) so the b128 K
//   reads and the b64 transposed V reads are free of bank conflicts on the 64-bank LDS.
//   At D = 256 the tiles go HBM -> LDS directly instead (buffer loads with the LDS-write
//   form) into unpadded rows with XOR-swizzled 16-byte chunks: the 64-128 staging
//   registers per lane would not fit beside O (128) and Q (64).
// * exp is v_exp_f32 (2^x) with scale*log2(e) folded into one FMA per score.
// * Causal: tiles above the diagonal are never loaded by a wave that does not need them,
//   32-key blocks above a wave's rows are skipped, and only the diagonal block is masked.
// * fp32 accumulation rescales O lazily: the running max used for the exponent is only
//   raised (and O rescaled) when a row's max grows by more than 2^kRescaleLog2 (2^15);
//   final O = acc / l is independent of the reference point, and P stays at or below
//   2^15, inside fp16/bf16 range.  l is summed from the rounded P that feeds P.V (consistent normalisation).
//   Input-dtype accumulation rescales every tile and follows the reference's rounding
//   sequence (acc = rnd(rnd(acc*rnd(alpha)) + rnd(P.V)), l from the unrounded P).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_fwd_common.h"
#include "attn_fwd_params.h"

#ifndef TA_TILE_M
#define TA_TILE_M 128
#endif
#ifndef TA_TILE_N
#define TA_TILE_N 64
#endif

// LDS stages of K/V tiles: two (the next tile is stored while the current one is read,
// one barrier per tile), except for the 64-row tiles, whose two-wave workgroups are too
// small to fill a CU at two stages (64 x 128: 151 KiB at D = 128, one workgroup per CU;
// 64 x 64: 76 KiB, two): with one stage, at the cost of a second barrier per tile, two
// (64 x 128) or four (64 x 64, with two waves per SIMD below) share a CU.  C4 D = 128 bf16:
// 64 x 128 308 -> 573 TFLOP/s, 64 x 64 584 -> 836; 64 x 64 at D = 256 105 -> 211.
#ifndef TA_STAGES
#if TA_TILE_M == 64
#define TA_STAGES 1
#else
#define TA_STAGES 2
#endif
#endif

namespace ta {

// LDS rows are padded so that every LDS address is a per-lane base plus an immediate
// offset and both read patterns are free of bank conflicts on the 64-bank LDS (16 units of
// 16 bytes per 256-byte bank row):
// * K: stride 2D + 16 bytes, an odd number of 16-byte units (D is a multiple of 16): one
//   b128 read pass covers 16 consecutive rows at one 16-byte column -> 16 distinct units;
// * V: stride 2D padded to 4 (mod 8) units (2D + 64 bytes for D = 64, 128, 256; 2D for
//   D = 160): one b64 transposed read pass covers 4 consecutive rows x 4 units -> 16
//   distinct units.
template <int D>
struct LdsLayout {
  static_assert(D % 16 == 0, "head dim must be a multiple of 16");
  static constexpr int KS = 2 * D + 16;                        // K row stride, bytes
  static constexpr int VS = 2 * D + 16 * ((12 - (D / 8) % 8) % 8);  // V row stride, bytes
  static_assert((KS / 16) % 2 == 1 && (VS / 16) % 8 == 4, "conflict-free strides");
};

// D = 256, loaded straight into LDS: rows of 512 bytes (two 64-bank rows), 16-byte chunks
// XOR-swizzled per row instead of padded:
// * K: physical chunk = logical ^ (row & 15).  A b128 read pass covers 16 consecutive rows
//   at one logical chunk -> 16 distinct chunks mod 16 -> conflict-free.
// * V: physical chunk = logical ^ 4 (row & 3).  A b64 transposed read pass covers 4
//   consecutive rows x 4 logical chunks (64 bytes) -> 4 distinct 64-byte groups.
template <int D>
struct LdsSwizzled {
  static_assert(D == 256, "swizzled staging is built for D = 256");
  static constexpr int KS = 2 * D;
  static constexpr int VS = 2 * D;
  __device__ static inline int swz_k(int row) { return row & 15; }
  __device__ static inline int swz_v(int row) { return (row & 3) << 2; }
};

template <int DT, int D, int TM, int TN, bool CAUSAL, bool TAIL, bool LOWP>
__device__ __forceinline__ void attn_fwd_body(const FwdParams& p) {
  constexpr int NW = TM / 32;        // waves per workgroup
  constexpr int NT = NW * 64;        // threads per workgroup
  constexpr int KB = TN / 32;        // 32-key blocks per tile
  constexpr int DK = D / 16;         // k-steps of the QK^T product
  constexpr int DB = D / 32;         // 32-wide d blocks of O
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int LD = TN * CPR / NT;  // 16-byte chunks per thread per tensor per tile
  // Rows one staging pass covers when a pass is whole rows (CPR divides NT), else 0.
  constexpr int RPP = (NT % CPR == 0) ? NT / CPR : 0;
  static_assert((TN * CPR) % NT == 0, "tile must split evenly over threads");
  constexpr bool DMA = D == 256;  // tiles straight into LDS (swizzled rows)
  using L = std::conditional_t<DMA, LdsSwizzled<D>, LdsLayout<D>>;
  constexpr int K_BYTES = TN * L::KS;
  constexpr int STAGE = K_BYTES + TN * L::VS;
  using DTy = DType<DT>;

  constexpr int NST = TA_STAGES;
  __shared__ __attribute__((aligned(16))) char smem[NST * STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hl = lane >> 5;  // which half of the wave

  // ---- block -> (bh, q tile) ------------------------------------------------------
  // sched 0: block ids in (bh, q tile) order.  sched >= 1: hardware hands block ids to
  // the 8 XCDs round-robin (block b runs on XCD b % 8), so consecutive logical tiles are
  // regrouped onto one XCD, keeping a head's K/V in one L2.  Causal tiles get heavier
  // with the tile index; sched <= 1 issues them heaviest first, sched 2 issues the
  // heavier half first and then the lighter half from the top, so the j-th and
  // (j + nq/2)-th tiles of a head - which land on the same CU when each XCD fills one
  // workgroup slot per CU before the next - add up to the same amount of work.
  const int nq = p.n_qblk;
  const int total = nq * p.n_bh;
  int lin = blockIdx.x;
  if (p.sched >= 1 && (total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
  const int bh = lin / nq;
  const int j = lin - bh * nq;
  int qt = j;
  if (CAUSAL) {
    const int half = (nq + 1) >> 1;
    qt = (p.sched == 2) ? (j < half ? nq - 1 - j : j - half) : nq - 1 - j;
  }
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int S = p.S;

  const uint16_t* __restrict__ qp = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* __restrict__ kp = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* __restrict__ vp = p.v + b * p.v_sb + h * p.v_sh;
  uint16_t* __restrict__ op = p.o + b * p.o_sb + h * p.o_sh;
  const int k_rb = (int)p.k_ss * 2;  // row bytes
  const int v_rb = (int)p.v_ss * 2;

  const int q0 = qt * TM;
  const int wq0 = q0 + wave * 32;  // first query row of this wave
  const int my_q = wq0 + l32;      // this lane's query row

  // ---- Q fragment: B operand of S^T = K Q^T, kept for the whole key loop ------------
  u32x4 qf[DK];
  {
    const bool ok = !TAIL || my_q < S;
    const uint16_t* row = qp + (int64_t)(ok ? my_q : 0) * p.q_ss;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      u32x4 v = *(const u32x4*)(row + 16 * kk + 8 * hl);
      qf[kk] = ok ? v : u32x4{0, 0, 0, 0};
    }
  }

  // ---- key range --------------------------------------------------------------------
  const int kv_end = CAUSAL ? min(S, q0 + TM) : S;
  const int n_tiles = (kv_end + TN - 1) / TN;
  const int wave_kv_end = CAUSAL ? min(S, wq0 + 32) : S;

  // ---- staging: HBM -> VGPR -> LDS --------------------------------------------------
  // Thread t moves 16-byte chunks t, t + NT, ... of each tile: chunk c is row c / CPR,
  // column chunk c % CPR.  When a pass is whole rows (CPR divides NT) every chunk of a
  // thread sits in one column, RPP rows apart: a fixed per-thread byte offset plus
  // immediates on both sides.  Otherwise (D = 160) each chunk's row and column are
  // computed once.  Global side: buffer loads from a per-tile resource.
  const int st_row = tid / CPR;  // whole-row passes: first row and column of the thread
  const int st_ch = tid % CPR;
  const int st_koff = st_row * k_rb + st_ch * 16;
  const int st_voff = st_row * v_rb + st_ch * 16;
  const int st_klds = st_row * L::KS + st_ch * 16;
  const int st_vlds = K_BYTES + st_row * L::VS + st_ch * 16;
  // Byte offset of chunk i of this thread: `base` + i rows-per-pass for whole-row passes,
  // else from the chunk's own row and column (`lds` adds the V tile's LDS base).
  auto st_off = [&](int i, int base, int stride, int lds) {
    if constexpr (RPP != 0) {
      return base + i * RPP * stride;
    } else {
      const int c = tid + i * NT;
      return lds + (c / CPR) * stride + (c % CPR) * 16;
    }
  };
  u32x4 stk[LD], stv[LD];
  auto load_tile = [&](int kt) {
    const int rows = S - kt * TN;
    const __amdgpu_buffer_rsrc_t kr = row_rsrc(kp + (int64_t)kt * TN * p.k_ss, rows, k_rb);
    const __amdgpu_buffer_rsrc_t vr = row_rsrc(vp + (int64_t)kt * TN * p.v_ss, rows, v_rb);
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      stk[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(kr, st_off(i, st_koff, k_rb, 0), 0, 0));
      stv[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(vr, st_off(i, st_voff, v_rb, 0), 0, 0));
    }
  };
  auto store_tile = [&](int stage) {
    char* base = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      *(u32x4*)(base + st_off(i, st_klds, L::KS, 0)) = stk[i];
      *(u32x4*)(base + st_off(i, st_vlds, L::VS, K_BYTES)) = stv[i];
    }
  };
  // Direct-to-LDS tiles (D = 256).  A tile of one tensor is NCH chunks of 1 KiB (RPC rows
  // each); wave w fills chunks g = w + NW i, lane l writing physical chunk l % CPR of row
  // RPC g + l / CPR, so it loads logical chunk (l % CPR) ^ swz(row) of that row.  Rows
  // RPC NW i apart: K's swizzle repeats every 16 rows (KP distinct per-lane offsets, the
  // rest a uniform row step), V's every 4 (one offset).  Rows past S are outside the
  // tile's buffer resource and read as zero.
  constexpr int RPC = 1024 / (2 * D);
  constexpr int NCH = TN * 2 * D / 1024;
  constexpr int NLW = NCH / NW;  // loads per wave per tensor per tile
  // s_waitcnt immediate: vmcnt(NLW) (its low 4 bits at 3:0, the high 2 at 15:14), expcnt
  // and lgkmcnt at their maxima.
  constexpr int kWaitNLW = 0x0F70 | (NLW & 15) | ((NLW >> 4) << 14);
  static_assert(NLW < 64, "vmcnt field");
  constexpr int RSTEP = RPC * NW;  // rows between a wave's consecutive chunks
  constexpr int KP = DMA ? 16 / RSTEP : 1;
  static_assert(!DMA || (NCH % NW == 0 && 16 % RSTEP == 0 && RSTEP % 4 == 0), "DMA tiling");
  int dm_k[KP];
  int dm_v = 0;
  if constexpr (DMA) {
    const int row0 = RPC * wave + lane / CPR;
    const int pc = lane % CPR;
#pragma unroll
    for (int j = 0; j < KP; ++j) {
      const int row = row0 + RSTEP * j;
      dm_k[j] = row * k_rb + ((pc ^ L::swz_k(row)) << 4);
    }
    dm_v = row0 * v_rb + ((pc ^ L::swz_v(row0)) << 4);
  }
  auto dma_k = [&](int kt, int stage) {
    const __amdgpu_buffer_rsrc_t kr = row_rsrc(kp + (int64_t)kt * TN * p.k_ss, S - kt * TN, k_rb);
    char* base = smem + stage * STAGE;
#pragma unroll
    for (int i = 0; i < NLW; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          kr, (__attribute__((address_space(3))) void*)(base + (wave + NW * i) * 1024), 16,
          dm_k[i % KP], (i / KP) * 16 * k_rb, 0, 0);
    }
  };
  auto dma_v = [&](int kt, int stage) {
    const __amdgpu_buffer_rsrc_t vr = row_rsrc(vp + (int64_t)kt * TN * p.v_ss, S - kt * TN, v_rb);
    char* base = smem + stage * STAGE + K_BYTES;
#pragma unroll
    for (int i = 0; i < NLW; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          vr, (__attribute__((address_space(3))) void*)(base + (wave + NW * i) * 1024), 16,
          dm_v, i * RSTEP * v_rb, 0, 0);
    }
  };

  // ---- per-lane LDS read offsets --------------------------------------------------------
  // K (A operand of S^T = K Q^T): lane reads row l32 of a 32-key block, 16 bytes at
  // column 16 * (2 kk + hl).
  // With swizzled rows: row l32 of a block has m = swz_k(l32) (blocks are 32 rows, so
  // swz_k(32 bk + l32) = swz_k(l32)); logical chunk 2 kk + hl is physical
  // (2 kk + hl) ^ m, i.e. byte 32 (kk ^ (m >> 1)) + 16 (hl ^ (m & 1)) of the row: k_rd
  // below XOR 32 kk.
  int k_rd = l32 * L::KS + hl * 16;
  if constexpr (DMA) {
    const int m = L::swz_k(l32);
    k_rd = l32 * L::KS + 32 * (m >> 1) + 16 * (hl ^ (m & 1));
  }
  // V^T (A operand of O^T = V^T P^T) via the transposed read: lane l of 16-lane group G
  // addresses row (key) 4 * hl + (l % 16) / 4 of a 16-key chunk and d = 16 * (G % 2) +
  // 4 * (l % 4); the hardware hands lane l column d = 16 * (G % 2) + l % 16 of those 4 rows.
  int v_rd = K_BYTES + (4 * hl + ((lane & 15) >> 2)) * L::VS +
             (16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2;
  // With swizzled rows: the row's swizzle 4 r (r = row & 3 = (lane >> 2) & 3, the same for
  // every 16-key chunk and its + 8 rows) moves the 64-byte group of d block db to
  // db ^ r: v_rd below XOR 64 db.
  if constexpr (DMA) {
    const int r = (lane >> 2) & 3;
    v_rd = K_BYTES + (4 * hl + r) * L::VS + ((64 * r) ^ ((16 * ((lane >> 4) & 1) + 4 * (lane & 3)) * 2));
  }
  auto k_addr = [&](int bk, int kk) {
    return DMA ? bk * 32 * L::KS + (k_rd ^ (32 * kk)) : k_rd + bk * 32 * L::KS + 32 * kk;
  };
  auto v_addr = [&](int bk, int kc, int db) {
    return DMA ? (v_rd ^ (64 * db)) + (32 * bk + 16 * kc) * L::VS
               : v_rd + (32 * bk + 16 * kc) * L::VS + 64 * db;
  };

  // ---- running state (lane = query l32 of this wave) ----------------------------------
  float m_run = kNegLarge;   // reference point of the exponent, raw score units
  float l_part = 0.0f;       // this lane's share of the row sum (keys it holds)
  f32x16 o_acc[DB];          // fp32 accumulation: O^T blocks
  uint32_t o_lp[LOWP ? DB : 1][8];  // input-dtype accumulation: packed O^T blocks
#pragma unroll
  for (int db = 0; db < DB; ++db) {
    o_acc[db] = f32x16{};
    if (LOWP) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) o_lp[db][jj] = 0u;
    }
  }
  const float c = p.scale_log2;

  // P of the current tile (packed) and its rescale factor, kept between the two parts of a
  // tile when it runs in two parts (a whole tile keeps its own).
  uint32_t pk_part[KB][8];
  float alpha_part = 1.0f;

  // One key tile.  FULL: every 32-key block of the tile is visible to every row of the
  // wave (no mask, no skipped block) - the common case, compiled without any per-block
  // condition.  PART 0 is the whole tile; PART 1 ends with P (reads the K tile), PART 2 is
  // P.V (reads the V tile), for the loop that refills K and V separately.
  auto tile = [&](const char* st, int k0, auto full_tag, auto part_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    constexpr int PART = decltype(part_tag)::value;
    uint32_t pk_whole[KB][8];
    float alpha_whole = 1.0f;
    uint32_t(&pk)[KB][8] = PART == 0 ? pk_whole : pk_part;
    float& alpha = PART == 0 ? alpha_whole : alpha_part;
    bool active[KB];
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) active[bk] = FULL || (k0 + 32 * bk) < wave_kv_end;
    if constexpr (PART != 2) {

    // -- S^T blocks ------------------------------------------------------------------
    f32x16 s[KB];
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) {
      if (active[bk]) {
        f32x16 acc = DTy::mfma(*(const u32x4*)(st + k_addr(bk, 0)), qf[0], f32x16{});
#pragma unroll
        for (int kk = 1; kk < DK; ++kk) acc = DTy::mfma(*(const u32x4*)(st + k_addr(bk, kk)), qf[kk], acc);
        s[bk] = acc;
      }
    }

    // -- mask (diagonal block for causal, keys past S for ragged tails) ---------------
    if (!FULL) {
      const bool need_tail = TAIL && (k0 + TN > S);
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
        const int kb0 = k0 + 32 * bk;
        const bool diag = CAUSAL && (kb0 + 31 > wq0);
        if (active[bk] && (diag || need_tail)) {
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
    }

    // -- row max -----------------------------------------------------------------------
    float mxa = kMasked, mxb = kMasked;  // two independent 3-input chains
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) {
      if (active[bk]) {
#pragma unroll
        for (int r = 0; r < 16; r += 4) {
          mxa = vmax3(mxa, s[bk][r], s[bk][r + 1]);
          mxb = vmax3(mxb, s[bk][r + 2], s[bk][r + 3]);
        }
      }
    }
    float mx;
    {
      float a0, a1;
      swap32(vmax(mxa, mxb), a0, a1);
      mx = vmax(a0, a1);
    }

    // -- new reference point, rescale of running state ---------------------------------
    alpha = 1.0f;
    if (LOWP) {
      const float m_new = vmax(m_run, mx);
      alpha = fast_exp2((m_run - m_new) * c);
      m_run = m_new;
    } else {
      const bool need = (mx - m_run) * c > kRescaleLog2;
      if (__ballot(need)) {
        const float m_new = need ? mx : m_run;
        alpha = fast_exp2((m_run - m_new) * c);
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < DB; ++db) o_acc[db] *= alpha;
      }
    }
    l_part *= alpha;

    // -- P = 2^(s*c - m*c), packed to the input dtype -------------------------------------
    // fp32 accumulation sums l from the same rounded P that feeds P.V, so the weights
    // are normalised consistently (with the lazy reference point the dominant key's P
    // is not exactly 1 and its rounding would otherwise not cancel).  Input-dtype
    // accumulation keeps the reference's fp32 sum of the unrounded P (flash_fwd.py:429).
    const float mc = m_run * c;
#pragma unroll
    for (int bk = 0; bk < KB; ++bk) {
      if (active[bk]) {
        float la = 0.0f, lb = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
          const float p0 = fast_exp2(__builtin_fmaf(s[bk][r], c, -mc));
          const float p1 = fast_exp2(__builtin_fmaf(s[bk][r + 1], c, -mc));
          const uint32_t w = DTy::pack(p0, p1);
          pk[bk][r >> 1] = w;
          if (LOWP) {
            l_part += p0 + p1;
          } else if (r & 2) {
            lb = DTy::sum2(w, lb);
          } else {
            la = DTy::sum2(w, la);
          }
        }
        if (!LOWP) l_part += la + lb;
      }
    }

    }  // PART != 2
    if constexpr (PART == 1) return;

    // -- O^T += V^T P^T ------------------------------------------------------------------
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      f32x16 acc = LOWP ? f32x16{} : o_acc[db];
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
        if (active[bk]) {
#pragma unroll
          for (int kc = 0; kc < 2; ++kc) {
            const char* a0p = st + v_addr(bk, kc, db);
            s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a0p);
            s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a0p + 8 * L::VS));
            u32x2 w0 = __builtin_bit_cast(u32x2, r0);
            u32x2 w1 = __builtin_bit_cast(u32x2, r1);
            u32x4 a = {w0[0], w0[1], w1[0], w1[1]};
            u32x4 bfrag = {pk[bk][4 * kc + 0], pk[bk][4 * kc + 1], pk[bk][4 * kc + 2],
                           pk[bk][4 * kc + 3]};
            acc = DTy::mfma(a, bfrag, acc);
          }
        }
      }
      if (LOWP) {
        const float al = DTy::round(alpha);
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const float t0 = DTy::round(DTy::lo(o_lp[db][jj]) * al);
          const float t1 = DTy::round(DTy::hi(o_lp[db][jj]) * al);
          const float u0 = DTy::round(acc[2 * jj]);
          const float u1 = DTy::round(acc[2 * jj + 1]);
          o_lp[db][jj] = DTy::pack(t0 + u0, t1 + u1);
        }
      } else {
        o_acc[db] = acc;
      }
    }
  };

  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  // Fully visible: every key of the tile is <= the wave's first query (causal) and < S.
  auto is_full = [&](int k0) { return (!CAUSAL || k0 + TN - 1 <= wq0) && (!TAIL || k0 + TN <= S); };
  // The unmasked tile body is a second copy of the tile in the code.  At D = 256, and at
  // D >= 128 with 64-row tiles, the two copies together need more registers than the
  // kernel has (the tail-masked kernels spilled 14-168 registers to scratch), so there
  // every tile takes the masked body, whose masks are wave-uniform per-block branches that
  // unmasked tiles skip.
  constexpr bool kFullBody = D <= 64 || (TM == 128 && D <= 160);
  auto run_tile = [&](const char* st, int k0, auto part_tag) {
    if (kFullBody && is_full(k0)) {
      tile(st, k0, std::true_type{}, part_tag);
    } else if (k0 < wave_kv_end) {
      tile(st, k0, std::false_type{}, part_tag);
    }
  };

  if constexpr (!DMA) {
    if (n_tiles > 0) {
      load_tile(0);
      store_tile(0);
    }
  } else if (n_tiles > 0) {
    dma_k(0, 0);
    dma_v(0, 0);
  }
  // Drain the Q-fragment loads (and the first tile's direct loads) here, on every path into
  // the loop: otherwise the waitcnt insertion merges a "Q still in flight" state into the
  // loop header and puts a vmcnt wait on the next tile's prefetch in front of every QK^T
  // MFMA.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  for (int kt = 0; kt < n_tiles; ++kt) {
    const bool has_next = kt + 1 < n_tiles;
    const int k0 = kt * TN;
    const char* st = smem + (NST == 2 ? (kt & 1) * STAGE : 0);
    if constexpr (!DMA) {
      if (has_next) load_tile(kt + 1);
      run_tile(st, k0, P0{});
      if constexpr (NST == 2) {
        if (has_next) store_tile((kt + 1) & 1);
        __syncthreads();
      } else {
        // One stage: the next tile (in registers since the top of this iteration) replaces
        // the current one once every wave is done reading it.
        __syncthreads();
        if (has_next) {
          store_tile(0);
          __syncthreads();
        }
      }
    } else if constexpr (NST == 2) {
      // The other stage was read last in the previous tile, before its closing barrier.
      if (has_next) {
        dma_k(kt + 1, (kt + 1) & 1);
        dma_v(kt + 1, (kt + 1) & 1);
      }
      run_tile(st, k0, P0{});
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads of the next tile
      __syncthreads();
    } else {
      // One stage, K and V refilled separately: K(kt + 1) once every wave has its P of
      // tile kt (its latency hidden by P.V), V(kt + 1) once every wave is done with P.V
      // (hidden by the next tile's S and softmax).  On entry V(kt) may be in flight (kt >
      // 0); every wave runs the same barriers whether or not it has keys in this tile.
      run_tile(st, k0, P1{});
      __syncthreads();
      if (has_next) dma_k(kt + 1, 0);
      // V(kt) was issued before K(kt + 1): wait until at most K(kt + 1)'s loads are left.
      if (has_next) {
        __builtin_amdgcn_s_waitcnt(kWaitNLW);
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);
      }
      __syncthreads();
      run_tile(st, k0, P2{});
      __syncthreads();
      if (has_next) {
        dma_v(kt + 1, 0);
        __builtin_amdgcn_s_waitcnt(kWaitNLW);  // K(kt + 1) landed, V(kt + 1) may not have
        __syncthreads();
      }
    }
  }

  // ---- epilogue: O = acc / l, written back as [q][d] ------------------------------------
  float la, lb;
  swap32(l_part, la, lb);
  const float l_tot = la + lb;
  if (TAIL && my_q >= S) return;
  const float inv = 1.0f / l_tot;
  uint16_t* orow = op + (int64_t)my_q * p.o_ss;
#pragma unroll
  for (int db = 0; db < DB; ++db) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      uint32_t w0, w1;
      if (LOWP) {
        const float il = DTy::round(inv);
        w0 = DTy::pack(DTy::lo(o_lp[db][2 * g]) * il, DTy::hi(o_lp[db][2 * g]) * il);
        w1 = DTy::pack(DTy::lo(o_lp[db][2 * g + 1]) * il, DTy::hi(o_lp[db][2 * g + 1]) * il);
      } else {
        w0 = DTy::pack(o_acc[db][4 * g + 0] * inv, o_acc[db][4 * g + 1] * inv);
        w1 = DTy::pack(o_acc[db][4 * g + 2] * inv, o_acc[db][4 * g + 3] * inv);
      }
      const int d = 32 * db + 8 * g + 4 * hl;
      *(u32x2*)(orow + d) = u32x2{w0, w1};
    }
  }
}

}  // namespace ta

// Waves per SIMD the register allocation is sized for: two when enough workgroups fit a
// CU by LDS for 8 waves (TM = 128, TN = 64: two workgroups; 64 x 64 with one stage: four),
// so one wave's MFMAs overlap another's softmax; one otherwise, and always one for head
// dims above 128 (whose O, Q and staging registers need the whole register file).
#if (TA_TILE_M == 128 && TA_TILE_N == 64) || (TA_TILE_M == 64 && TA_TILE_N == 64)
#define TA_WAVES_PER_SIMD 2
#else
#define TA_WAVES_PER_SIMD 1
#endif

// One extern "C" entry per (dtype, D, causal, tail, accumulation) at this file's (TM, TN).
// Name: ta_fwd_<f16|bf16>_d<D>_m<TM>_n<TN>_c<0|1>_t<0|1>_a<0|1>.
#define TA_NAME2(DTN, D, M, N, C, T, A) ta_fwd_##DTN##_d##D##_m##M##_n##N##_c##C##_t##T##_a##A
#define TA_NAME(DTN, D, M, N, C, T, A) TA_NAME2(DTN, D, M, N, C, T, A)

#define TA_DEFINE(DTN, DT, D, C, T, A, WPS)                                                 \
  extern "C" __global__ void __launch_bounds__(TA_TILE_M * 2)                               \
      __attribute__((amdgpu_waves_per_eu(WPS, WPS)))                                        \
      TA_NAME(DTN, D, TA_TILE_M, TA_TILE_N, C, T, A)(ta::FwdParams p) {                     \
    ta::attn_fwd_body<DT, D, TA_TILE_M, TA_TILE_N, (C != 0), (T != 0), (A != 0)>(p);         \
  }

#define TA_DEFINE_CTA(DTN, DT, D, WPS) \
  TA_DEFINE(DTN, DT, D, 0, 0, 0, WPS)  \
  TA_DEFINE(DTN, DT, D, 0, 0, 1, WPS)  \
  TA_DEFINE(DTN, DT, D, 0, 1, 0, WPS)  \
  TA_DEFINE(DTN, DT, D, 0, 1, 1, WPS)  \
  TA_DEFINE(DTN, DT, D, 1, 0, 0, WPS)  \
  TA_DEFINE(DTN, DT, D, 1, 0, 1, WPS)  \
  TA_DEFINE(DTN, DT, D, 1, 1, 0, WPS)  \
  TA_DEFINE(DTN, DT, D, 1, 1, 1, WPS)

TA_DEFINE_CTA(f16, 0, 64, TA_WAVES_PER_SIMD)
TA_DEFINE_CTA(f16, 0, 128, TA_WAVES_PER_SIMD)
TA_DEFINE_CTA(bf16, 1, 64, TA_WAVES_PER_SIMD)
TA_DEFINE_CTA(bf16, 1, 128, TA_WAVES_PER_SIMD)

// Head dims 160 and 256: 64-key tiles only (two stages of padded K and V rows take 84 KiB
// and 141 KiB of LDS; 128-key tiles would not fit).
#if TA_TILE_N == 64
TA_DEFINE_CTA(f16, 0, 160, 1)
TA_DEFINE_CTA(f16, 0, 256, 1)
TA_DEFINE_CTA(bf16, 1, 160, 1)
TA_DEFINE_CTA(bf16, 1, 256, 1)
#endif
