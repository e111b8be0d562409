// Device helpers shared by the SDPA forward kernels (gfx950): operand types, per-dtype
// MFMA / pack / round / pair-sum, cross-half lane exchange, exp2, NaN-propagating max and
// range-checked buffer resources.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ta {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Initial running max, raw score units (the reference starts from -1e30, flash_fwd.py:14).
// Finite, so the first rescale factor 2^((m0 - m)*c) is exactly 0 rather than NaN.
constexpr float kNegLarge = -1.0e30f;
// Masked scores are -inf: 2^(-inf) = 0 whatever the running max is, and a lane whose keys
// are all masked keeps max = -inf without ever forming inf - inf against kNegLarge.
constexpr float kMasked = -__builtin_huge_valf();
// Lazy-rescale threshold in log2 units: P = 2^(s*c - m*c) stays <= 2^15, the largest power
// of two below fp16's maximum, so P packs to either input dtype without overflow (P.V and l
// accumulate in fp32).  Against 2^8, the running max moves (O rescaled, P recomputed) less
// often where it jumps, e.g. keys with outliers: C5b 0.564 -> 0.527 ms, C3 / C4 / C5
// unchanged.
constexpr float kRescaleLog2 = 15.0f;
constexpr float kRescaleBound = 32768.0f;  // 2^kRescaleLog2
static_assert(kRescaleBound == (float)(1 << (int)kRescaleLog2), "bound = 2^threshold");

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
  // lo(u) + hi(u): the same dot2 with an inline-constant zero accumulator (VOP3P form; the
  // compiler would materialise the zero with a v_mov for the accumulating form).
  __device__ static inline float sum2_head(uint32_t u) {
    float x;
    asm("v_dot2_f32_f16 %0, %1, %2, 0" : "=v"(x) : "v"(u), "s"(0x3c003c00u));
    return x;
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
  // lo(u) + hi(u) (VOP3P dot2 with an inline-constant zero accumulator, as for fp16).
  __device__ static inline float sum2_head(uint32_t u) {
    float x;
    asm("v_dot2_f32_bf16 %0, %1, %2, 0" : "=v"(x) : "v"(u), "s"(0x3f803f80u));
    return x;
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
__device__ static inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// IEEE 754-2019 maximum (NaN-propagating): lowers to v_maximum3_f32 on gfx950 without the
// operand canonicalisation fmaxf needs in IEEE mode.
__device__ static inline float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ static inline float vmax3(float a, float b, float c) { return vmax(a, vmax(b, c)); }

// 16-byte chunk swizzle of the unpadded LDS key tiles of the eight-wave and wide kernels
// (row = 2D bytes, 64 banks x 4 bytes):
// * K: a b128 read pass covers 16 consecutive rows at one logical chunk;
//   physical chunk = logical ^ (row & 15) for D = 128, ^ ((row >> 1) & 7) for D = 64.
// * V: a b64 transposed read pass covers 4 consecutive rows x 4 logical chunks;
//   physical chunk = logical ^ 4 * (row & 3) for D = 128, ^ 4 * ((row >> 1) & 1) for D = 64.
template <int D>
__device__ static inline int pp_swz_k(int row) {
  return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
template <int D>
__device__ static inline int pp_swz_v(int row) {
  return D == 128 ? ((row & 3) << 2) : (((row >> 1) & 1) << 2);
}

// Buffer resource for rows [0, rows) of a row-major tensor with `row_bytes` between rows:
// loads past the last row return zeros (the hardware range check), which zero-fills the
// ragged last key tile without any per-lane select.
__device__ static inline __amdgpu_buffer_rsrc_t row_rsrc(const void* base, int rows, int row_bytes) {
  const int bytes = rows > 0 ? rows * row_bytes : 0;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

}  // namespace ta
