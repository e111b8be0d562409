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
// * K/V tiles go HBM -> VGPR -> LDS through two LDS stages: tile t+1 is fetched while
//   tile t is consumed; one barrier per tile.  Rows are unpadded and 16-byte chunks are
//   XOR-swizzled per row (different swizzles for K and V) so the b128 K reads and the b64
//   transposed V reads are free of bank conflicts on the 64-bank LDS.
// * exp is v_exp_f32 (2^x) with scale*log2(e) folded into one FMA per score.
// * Causal: tiles above the diagonal are never loaded by a wave that does not need them,
//   32-key blocks above a wave's rows are skipped, and only the diagonal block is masked.
// * fp32 accumulation rescales O lazily: the running max used for the exponent is only
//   raised (and O rescaled) when a row's max grows by more than 2^8; final O = acc / l is
//   independent of the reference point, and P stays below 256, well inside fp16/bf16
//   range.  l is summed from the rounded P that feeds P.V (consistent normalisation).
//   Input-dtype accumulation rescales every tile and follows the reference's rounding
//   sequence (acc = rnd(rnd(acc*rnd(alpha)) + rnd(P.V)), l from the unrounded P).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_fwd_params.h"

#ifndef TA_TILE_M
#define TA_TILE_M 128
#endif
#ifndef TA_TILE_N
#define TA_TILE_N 64
#endif

namespace ta {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;

// Initial running max, raw score units (the reference starts from -1e30, flash_fwd.py:14).
// Finite, so the first rescale factor 2^((m0 - m)*c) is exactly 0 rather than NaN.
constexpr float kNegLarge = -1.0e30f;
// Masked scores are -inf: 2^(-inf) = 0 whatever the running max is, and a lane whose keys
// are all masked keeps max = -inf without ever forming inf - inf against kNegLarge.
constexpr float kMasked = -__builtin_huge_valf();
// Lazy-rescale threshold in log2 units: P = 2^(s*c - m*c) stays <= 2^8.
constexpr float kRescaleLog2 = 8.0f;

template <int DT>
struct DType;

template <>
struct DType<0> {  // float16
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (v_cvt_pk_f16_f32).
  __device__ static inline uint32_t pack(float a, float b) {
    f16x2 h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static inline float lo(uint32_t u) {
    return (float)__builtin_bit_cast(f16x2, u)[0];
  }
  __device__ static inline float hi(uint32_t u) {
    return (float)__builtin_bit_cast(f16x2, u)[1];
  }
  __device__ static inline float round(float x) { return (float)(_Float16)x; }
  // acc + lo(u) + hi(u) in fp32 (v_dot2c_f32_f16 against (1, 1); keeps fp16 subnormals).
  __device__ static inline float sum2(uint32_t u, float acc) {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, u), one, acc, false);
  }
};

template <>
struct DType<1> {  // bfloat16
  __device__ static inline f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // Round-to-nearest-even pack of two floats (v_cvt_pk_bf16_f32).
  __device__ static inline uint32_t pack(float a, float b) {
    bf16x2 h = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
  __device__ static inline float lo(uint32_t u) { return __uint_as_float(u << 16); }
  __device__ static inline float hi(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }
  __device__ static inline float round(float x) { return (float)(__bf16)x; }
  // acc + lo(u) + hi(u) in fp32 (v_dot2c_f32_bf16 against (1, 1)).
  __device__ static inline float sum2(uint32_t u, float acc) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, u), one, acc, false);
  }
};

// Symmetric exchange with lane ^ 32: returns (own, partner) in some order; callers only
// combine the pair with a commutative op.
__device__ static inline void swap32(float x, float& a, float& b) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(r[0]);
  b = __uint_as_float(r[1]);
}

__device__ static inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 16-byte chunk swizzles (chunk index within a row, row index within the tile).
// K: the 16 lanes of one b128 read pass hit 16 consecutive rows at one logical chunk.
// V: one b64 transposed read pass covers 4 rows x 4 consecutive logical chunks.
template <int D>
__device__ static inline int swz_k(int row) {
  return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
template <int D>
__device__ static inline int swz_v(int row) {
  return D == 128 ? ((row & 3) << 2) : (((row >> 1) & 1) << 2);
}

template <int DT, int D, int TM, int TN, bool CAUSAL, bool TAIL, bool LOWP>
__device__ __forceinline__ void attn_fwd_body(const FwdParams& p) {
  constexpr int NW = TM / 32;        // waves per workgroup
  constexpr int NT = NW * 64;        // threads per workgroup
  constexpr int KB = TN / 32;        // 32-key blocks per tile
  constexpr int DK = D / 16;         // k-steps of the QK^T product
  constexpr int DB = D / 32;         // 32-wide d blocks of O
  constexpr int CPR = D / 8;         // 16-byte chunks per row
  constexpr int TILE_CHUNKS = TN * CPR;
  constexpr int LD_PER_THREAD = TILE_CHUNKS / NT;  // chunks per thread per tensor per tile
  static_assert(TILE_CHUNKS % NT == 0, "tile must split evenly over threads");
  constexpr int TILE_ELEMS = TN * D;  // halves per K (or V) tile
  using DTy = DType<DT>;

  __shared__ __attribute__((aligned(16))) uint16_t smem[2 * 2 * TILE_ELEMS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int l32 = lane & 31;
  const int hl = lane >> 5;  // which half of the wave

  // ---- block -> (bh, q tile) ------------------------------------------------------
  const int nq = p.n_qblk;
  const int total = nq * p.n_bh;
  int lin = blockIdx.x;
  if (p.sched == 1) {
    // Group consecutive logical tiles onto one XCD: hardware hands block ids to the 8
    // XCDs round-robin, so block id b runs on XCD b % 8.
    const int per = total >> 3;
    if ((total & 7) == 0) lin = (lin & 7) * per + (lin >> 3);
  }
  const int bh = lin / nq;
  int qt = lin - bh * nq;
  if (CAUSAL) qt = nq - 1 - qt;  // heaviest query tiles first
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int S = p.S;

  const uint16_t* __restrict__ qp = p.q + b * p.q_sb + h * p.q_sh;
  const uint16_t* __restrict__ kp = p.k + b * p.k_sb + h * p.k_sh;
  const uint16_t* __restrict__ vp = p.v + b * p.v_sb + h * p.v_sh;
  uint16_t* __restrict__ op = p.o + b * p.o_sb + h * p.o_sh;

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

  // ---- staging: HBM -> VGPR -> LDS ----------------------------------------------------
  u32x4 stk[LD_PER_THREAD], stv[LD_PER_THREAD];
  auto load_tile = [&](int kt) {
#pragma unroll
    for (int i = 0; i < LD_PER_THREAD; ++i) {
      const int idx = tid + i * NT;
      const int row = idx / CPR;
      const int pc = idx % CPR;
      const int key = kt * TN + row;
      const bool ok = !TAIL || key < S;
      const int kr = ok ? key : 0;
      u32x4 kv = *(const u32x4*)(kp + (int64_t)kr * p.k_ss + ((pc ^ swz_k<D>(row)) << 3));
      u32x4 vv = *(const u32x4*)(vp + (int64_t)kr * p.v_ss + ((pc ^ swz_v<D>(row)) << 3));
      stk[i] = ok ? kv : u32x4{0, 0, 0, 0};
      stv[i] = ok ? vv : u32x4{0, 0, 0, 0};
    }
  };
  auto store_tile = [&](int stage) {
    uint16_t* kd = smem + stage * 2 * TILE_ELEMS;
    uint16_t* vd = kd + TILE_ELEMS;
#pragma unroll
    for (int i = 0; i < LD_PER_THREAD; ++i) {
      const int idx = tid + i * NT;
      *(u32x4*)(kd + idx * 8) = stk[i];
      *(u32x4*)(vd + idx * 8) = stv[i];
    }
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
      for (int j = 0; j < 8; ++j) o_lp[db][j] = 0u;
    }
  }
  const float c = p.scale_log2;

  if (n_tiles > 0) {
    load_tile(0);
    store_tile(0);
  }
  __syncthreads();

  for (int kt = 0; kt < n_tiles; ++kt) {
    const bool has_next = kt + 1 < n_tiles;
    if (has_next) load_tile(kt + 1);

    const int k0 = kt * TN;
    if (k0 < wave_kv_end) {
      const uint16_t* ks = smem + (kt & 1) * 2 * TILE_ELEMS;
      const uint16_t* vs = ks + TILE_ELEMS;

      // -- S^T blocks ------------------------------------------------------------------
      f32x16 s[KB];
      bool active[KB];
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
        active[bk] = (k0 + 32 * bk) < wave_kv_end;
        s[bk] = f32x16{};
        if (active[bk]) {
          const int row = 32 * bk + l32;
#pragma unroll
          for (int kk = 0; kk < DK; ++kk) {
            const int ch = (2 * kk + hl) ^ swz_k<D>(row);
            u32x4 a = *(const u32x4*)(ks + row * D + ch * 8);
            s[bk] = DTy::mfma(a, qf[kk], s[bk]);
          }
        }
      }

      // -- mask (diagonal block for causal, keys past S for ragged tails) ---------------
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

      // -- row max -----------------------------------------------------------------------
      float mx = kMasked;
#pragma unroll
      for (int bk = 0; bk < KB; ++bk) {
        if (active[bk]) {
#pragma unroll
          for (int r = 0; r < 16; r += 2) mx = fmaxf(mx, fmaxf(s[bk][r], s[bk][r + 1]));
        }
      }
      {
        float a0, a1;
        swap32(mx, a0, a1);
        mx = fmaxf(a0, a1);
      }

      // -- new reference point, rescale of running state ---------------------------------
      float alpha = 1.0f;
      if (LOWP) {
        const float m_new = fmaxf(m_run, mx);
        alpha = fast_exp2((m_run - m_new) * c);
        m_run = m_new;
      } else {
        const bool need = (mx - m_run) * c > kRescaleLog2;
        if (__builtin_amdgcn_read_exec() & __ballot(need)) {
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
      uint32_t pk[KB][8];
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

      // -- O^T += V^T P^T ------------------------------------------------------------------
      // Transposed V read: lane l of 16-lane group G reads row (key) r = (l%16)/4 of the
      // 4-key group and 4 consecutive d at 4*(l%4); the hardware hands lane l column
      // d = 16*(G%2) + l%16 of those 4 rows.
      const int tr_r = (lane & 15) >> 2;
      const int tr_d = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        f32x16 acc = LOWP ? f32x16{} : o_acc[db];
#pragma unroll
        for (int bk = 0; bk < KB; ++bk) {
          if (active[bk]) {
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) {
              const int kbase = 32 * bk + 16 * kc + 4 * hl + tr_r;
              const int d = 32 * db + tr_d;
              const int row0 = kbase, row1 = kbase + 8;
              const uint16_t* a0p = vs + row0 * D + (((d >> 3) ^ swz_v<D>(row0)) << 3) + (d & 7);
              const uint16_t* a1p = vs + row1 * D + (((d >> 3) ^ swz_v<D>(row1)) << 3) + (d & 7);
              s16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a0p);
              s16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a1p);
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
          for (int j = 0; j < 8; ++j) {
            const float t0 = DTy::round(DTy::lo(o_lp[db][j]) * al);
            const float t1 = DTy::round(DTy::hi(o_lp[db][j]) * al);
            const float u0 = DTy::round(acc[2 * j]);
            const float u1 = DTy::round(acc[2 * j + 1]);
            o_lp[db][j] = DTy::pack(t0 + u0, t1 + u1);
          }
        } else {
          o_acc[db] = acc;
        }
      }
    }

    if (has_next) store_tile((kt + 1) & 1);
    __syncthreads();
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

// One extern "C" entry per (dtype, D, causal, tail, accumulation) at this file's (TM, TN).
// Name: ta_fwd_<f16|bf16>_d<D>_m<TM>_n<TN>_c<0|1>_t<0|1>_a<0|1>.
#define TA_NAME2(DTN, D, M, N, C, T, A) ta_fwd_##DTN##_d##D##_m##M##_n##N##_c##C##_t##T##_a##A
#define TA_NAME(DTN, D, M, N, C, T, A) TA_NAME2(DTN, D, M, N, C, T, A)

#define TA_DEFINE(DTN, DT, D, C, T, A)                                                      \
  extern "C" __global__ void __launch_bounds__(TA_TILE_M * 2)                               \
      TA_NAME(DTN, D, TA_TILE_M, TA_TILE_N, C, T, A)(ta::FwdParams p) {                     \
    ta::attn_fwd_body<DT, D, TA_TILE_M, TA_TILE_N, (C != 0), (T != 0), (A != 0)>(p);         \
  }

#define TA_DEFINE_CTA(DTN, DT, D) \
  TA_DEFINE(DTN, DT, D, 0, 0, 0)  \
  TA_DEFINE(DTN, DT, D, 0, 0, 1)  \
  TA_DEFINE(DTN, DT, D, 0, 1, 0)  \
  TA_DEFINE(DTN, DT, D, 0, 1, 1)  \
  TA_DEFINE(DTN, DT, D, 1, 0, 0)  \
  TA_DEFINE(DTN, DT, D, 1, 0, 1)  \
  TA_DEFINE(DTN, DT, D, 1, 1, 0)  \
  TA_DEFINE(DTN, DT, D, 1, 1, 1)

TA_DEFINE_CTA(f16, 0, 64)
TA_DEFINE_CTA(f16, 0, 128)
TA_DEFINE_CTA(bf16, 1, 64)
TA_DEFINE_CTA(bf16, 1, 128)
