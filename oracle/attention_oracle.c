/*
 * CPU oracle for the SDPA forward path.  TEST INFRASTRUCTURE ONLY: only tests/, the
 * smoke() check and bench.py's cpu_baseline leg may load this; the product never does.
 *
 * Three restatements, all reading fp16/bf16 bit patterns and upcasting exactly:
 *
 *  ora_explicit_f32 / ora_explicit_f64
 *      The north-star oracle: explicit softmax(Q K^T * scale + mask) V with every operation
 *      in fp32 (or fp64), one query row at a time.  Mask: key j allowed for query i iff
 *      j <= i when causal (the reference's `row >= col`, flash_fwd.py:420-421).
 *
 *  ora_flash_tiled
 *      The reference kernel's own algorithm, flash_fwd.py:374-446 (fp32 accumulation) and
 *      :301-372 (accumulation in the input dtype): query tiles of TM rows, key tiles of TN,
 *      running (m, l, acc) from m = -1e30, masked scores = -1e30 (:14, :415-423),
 *      alpha = exp(m - m'), p = exp(s - m'), l = l*alpha + sum(p) in fp32 (:425-430),
 *      p rounded to the input dtype before P.V (:432-433), causal key-tile bound
 *      ceil(min((qt+1)*TM, S)/TN) (:393-398), epilogue acc * (1/l) (:438-444).
 *      In input-dtype mode: acc = rnd(rnd(acc * rnd(alpha)) + rnd(P.V)) (:360-362) and
 *      out = rnd(acc * rnd(1/l)) (:365-368).  `score_lowp` = 1 additionally rounds Q K^T to
 *      the input dtype before the fp32 scale (:410-413 read as a matmul returning the input
 *      dtype); the result dtype of cuTile's matmul is not pinned by anything in the
 *      reference, so both readings are offered.
 *
 * Rounding: fp32 -> fp16 / bf16 round-to-nearest-even, written from the IEEE 754 binary16
 * and bfloat16 formats.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- conversions */

static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else { /* subnormal: value = man * 2^-24 */
      float f = (float)man * 5.9604644775390625e-8f;
      memcpy(&bits, &f, 4);
      bits |= sign;
    }
  } else if (exp == 31) {
    bits = sign | 0x7f800000u | (man << 13);
  } else {
    bits = sign | ((exp + 112u) << 23) | (man << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static uint16_t f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u); /* NaN */
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520: inf */
  if (ax < 0x38800000u) { /* below 2^-14: subnormal or zero, quantum 2^-24 */
    float a;
    memcpy(&a, &ax, 4);
    float q = a * 16777216.0f;     /* exact scaling by 2^24 */
    float r = nearbyintf(q);        /* ties to even under the default rounding mode */
    return (uint16_t)(sign | (uint32_t)r);
  }
  /* normal: keep 10 mantissa bits, round to nearest even on the 13 dropped bits */
  uint32_t e = (ax >> 23) - 112u;
  uint32_t m = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)(sign | h);
}

static float bf16_to_f32(uint16_t b) {
  uint32_t bits = (uint32_t)b << 16;
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

static uint16_t f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  uint32_t lsb = (x >> 16) & 1u;
  x += 0x7fffu + lsb;
  return (uint16_t)(x >> 16);
}

static inline float up(uint16_t v, int dtype) { return dtype ? bf16_to_f32(v) : f16_to_f32(v); }
static inline uint16_t down(float v, int dtype) { return dtype ? f32_to_bf16(v) : f32_to_f16(v); }
static inline float rnd(float v, int dtype) { return up(down(v, dtype), dtype); }

void ora_round(const float* x, uint16_t* out, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) out[i] = down(x[i], dtype);
}

void ora_upcast(const uint16_t* x, float* out, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) out[i] = up(x[i], dtype);
}

/* ---------------------------------------------------------------- explicit oracle */

/* Rows: if `rows` is non-NULL, only the n_rows listed query rows of every (b,h) are
 * computed and `out` is [B*H, n_rows, D]; otherwise all S rows and out is [B*H, S, D]. */
void ora_explicit_f32(const uint16_t* q, const uint16_t* k, const uint16_t* v, int dtype,
                      int64_t BH, int64_t S, int64_t D, int causal, float scale,
                      const int64_t* rows, int64_t n_rows, float* out) {
  int64_t nr = rows ? n_rows : S;
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)(S > 0 ? S : 1));
    float* qr = (float*)malloc(sizeof(float) * (size_t)(D > 0 ? D : 1));
    float* acc = (float*)malloc(sizeof(float) * (size_t)(D > 0 ? D : 1));
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < BH * nr; ++t) {
      int64_t bh = t / nr, ri = t % nr;
      int64_t i = rows ? rows[ri] : ri;
      const uint16_t* qb = q + (bh * S + i) * D;
      const uint16_t* kb = k + bh * S * D;
      const uint16_t* vb = v + bh * S * D;
      for (int64_t d = 0; d < D; ++d) qr[d] = up(qb[d], dtype);
      int64_t nj = causal ? (i + 1 < S ? i + 1 : S) : S;
      float m = -INFINITY;
      for (int64_t j = 0; j < nj; ++j) {
        float s = 0.0f;
        const uint16_t* kr = kb + j * D;
        for (int64_t d = 0; d < D; ++d) s += qr[d] * up(kr[d], dtype);
        s *= scale;
        sc[j] = s;
        if (s > m) m = s;
      }
      float l = 0.0f;
      for (int64_t j = 0; j < nj; ++j) {
        sc[j] = expf(sc[j] - m);
        l += sc[j];
      }
      for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
      for (int64_t j = 0; j < nj; ++j) {
        const uint16_t* vr = vb + j * D;
        float p = sc[j];
        for (int64_t d = 0; d < D; ++d) acc[d] += p * up(vr[d], dtype);
      }
      float* o = out + (bh * nr + ri) * D;
      for (int64_t d = 0; d < D; ++d) o[d] = acc[d] / l;
    }
    free(sc);
    free(qr);
    free(acc);
  }
}

void ora_explicit_f64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int dtype,
                      int64_t BH, int64_t S, int64_t D, int causal, double scale,
                      const int64_t* rows, int64_t n_rows, double* out) {
  int64_t nr = rows ? n_rows : S;
#pragma omp parallel
  {
    double* sc = (double*)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
    double* qr = (double*)malloc(sizeof(double) * (size_t)(D > 0 ? D : 1));
    double* acc = (double*)malloc(sizeof(double) * (size_t)(D > 0 ? D : 1));
#pragma omp for schedule(dynamic, 4)
    for (int64_t t = 0; t < BH * nr; ++t) {
      int64_t bh = t / nr, ri = t % nr;
      int64_t i = rows ? rows[ri] : ri;
      const uint16_t* qb = q + (bh * S + i) * D;
      const uint16_t* kb = k + bh * S * D;
      const uint16_t* vb = v + bh * S * D;
      for (int64_t d = 0; d < D; ++d) qr[d] = (double)up(qb[d], dtype);
      int64_t nj = causal ? (i + 1 < S ? i + 1 : S) : S;
      double m = -INFINITY;
      for (int64_t j = 0; j < nj; ++j) {
        double s = 0.0;
        const uint16_t* kr = kb + j * D;
        for (int64_t d = 0; d < D; ++d) s += qr[d] * (double)up(kr[d], dtype);
        s *= scale;
        sc[j] = s;
        if (s > m) m = s;
      }
      double l = 0.0;
      for (int64_t j = 0; j < nj; ++j) {
        sc[j] = exp(sc[j] - m);
        l += sc[j];
      }
      for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
      for (int64_t j = 0; j < nj; ++j) {
        const uint16_t* vr = vb + j * D;
        for (int64_t d = 0; d < D; ++d) acc[d] += sc[j] * (double)up(vr[d], dtype);
      }
      double* o = out + (bh * nr + ri) * D;
      for (int64_t d = 0; d < D; ++d) o[d] = acc[d] / l;
    }
    free(sc);
    free(qr);
    free(acc);
  }
}

/* ---------------------------------------------------------------- tiled restatement */

#define ORA_NEG_LARGE (-1.0e30f) /* flash_fwd.py:14 */

void ora_flash_tiled(const uint16_t* q, const uint16_t* k, const uint16_t* v, int dtype,
                     int64_t BH, int64_t S, int64_t D, int causal, float scale, int64_t TM,
                     int64_t TN, int accum_lowp, int score_lowp, int l_rounded, uint16_t* out) {
  int64_t n_qt = (S + TM - 1) / TM;
#pragma omp parallel
  {
    float* m = (float*)malloc(sizeof(float) * (size_t)TM);
    float* l = (float*)malloc(sizeof(float) * (size_t)TM);
    float* acc = (float*)malloc(sizeof(float) * (size_t)(TM * D));
    float* sc = (float*)malloc(sizeof(float) * (size_t)(TM * TN));
    float* pv = (float*)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (int64_t t = 0; t < BH * n_qt; ++t) {
      int64_t bh = t / n_qt, qt = t % n_qt;
      const uint16_t* qb = q + bh * S * D;
      const uint16_t* kb = k + bh * S * D;
      const uint16_t* vb = v + bh * S * D;
      int64_t n_kt = (S + TN - 1) / TN;
      if (causal) {
        int64_t cols = (qt + 1) * TM < S ? (qt + 1) * TM : S;
        n_kt = (cols + TN - 1) / TN;
      }
      for (int64_t r = 0; r < TM; ++r) {
        m[r] = ORA_NEG_LARGE;
        l[r] = 0.0f;
      }
      for (int64_t x = 0; x < TM * D; ++x) acc[x] = 0.0f;
      for (int64_t kt = 0; kt < n_kt; ++kt) {
        for (int64_t r = 0; r < TM; ++r) {
          int64_t row = qt * TM + r;
          int row_ok = row < S;
          float tile_max = -INFINITY;
          for (int64_t c = 0; c < TN; ++c) {
            int64_t col = kt * TN + c;
            int valid = row_ok && col < S && (!causal || row >= col);
            float s = ORA_NEG_LARGE;
            if (valid) {
              float dot = 0.0f;
              for (int64_t d = 0; d < D; ++d)
                dot += up(qb[row * D + d], dtype) * up(kb[col * D + d], dtype);
              if (score_lowp) dot = rnd(dot, dtype);
              s = dot * scale;
            }
            sc[r * TN + c] = s;
            if (s > tile_max) tile_max = s;
          }
          float m_next = m[r] > tile_max ? m[r] : tile_max;
          float alpha = expf(m[r] - m_next);
          float psum = 0.0f;
          for (int64_t c = 0; c < TN; ++c) {
            float p = expf(sc[r * TN + c] - m_next);
            float pl = rnd(p, dtype); /* p_lowp */
            psum += l_rounded ? pl : p;
            sc[r * TN + c] = pl;
          }
          l[r] = l[r] * alpha + psum;
          for (int64_t d = 0; d < D; ++d) pv[d] = 0.0f;
          for (int64_t c = 0; c < TN; ++c) {
            int64_t col = kt * TN + c;
            if (col >= S) continue; /* out-of-range V rows read as zero */
            float p = sc[r * TN + c];
            for (int64_t d = 0; d < D; ++d) pv[d] += p * up(vb[col * D + d], dtype);
          }
          float* a = acc + r * D;
          if (accum_lowp) {
            float al = rnd(alpha, dtype);
            for (int64_t d = 0; d < D; ++d)
              a[d] = rnd(rnd(a[d] * al, dtype) + rnd(pv[d], dtype), dtype);
          } else {
            for (int64_t d = 0; d < D; ++d) a[d] = a[d] * alpha + pv[d];
          }
          m[r] = m_next;
        }
      }
      for (int64_t r = 0; r < TM; ++r) {
        int64_t row = qt * TM + r;
        if (row >= S) continue;
        float inv = 1.0f / l[r];
        uint16_t* o = out + (bh * S + row) * D;
        if (accum_lowp) {
          float il = rnd(inv, dtype);
          for (int64_t d = 0; d < D; ++d) o[d] = down(acc[r * D + d] * il, dtype);
        } else {
          for (int64_t d = 0; d < D; ++d) o[d] = down(acc[r * D + d] * inv, dtype);
        }
      }
    }
    free(m);
    free(l);
    free(acc);
    free(sc);
    free(pv);
  }
}
