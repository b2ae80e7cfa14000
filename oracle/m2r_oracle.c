/*
 * CPU oracle for the MI355X state codec and FP4 weight decode.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests compare
 * the HIP library against; only tests/, __graft_entry__.smoke() and bench.py's
 * CPU-baseline leg may load it.  No product code path calls it.
 *
 * It restates the reference's arithmetic literally, one IEEE binary32
 * operation per Python/Triton operation, compiled with -ffp-contract=off:
 *   - state rows: scripts/fp4_zero_predictor_codec_v1.py:76-181 (_latent_scan)
 *     and :221-225 (ridge correction), scripts/state_ppl_codec_v10.py:78-154
 *     (_tier_scan), scripts/state_ppl_codec_v6.py:52-61 (_stored_quantize),
 *     mamba2_recall/state_codec.py:105-176 (_sq_scan)
 *   - dense 3-bit rows: mamba2_recall/state_codec_dense3.py:82-148 (_scan)
 *   - FP4 decode: mamba2_recall/fp4.py:100-103,151-154,225-250
 *   - legacy diagnostic encode: mamba2_recall/state_codec.py:299-331
 * Division is C's correctly rounded `/` (the reference's div_rn; its `/`
 * sites are defined the same way), rounding is C roundf (half away from
 * zero), binary16/E4M3FN conversions round to nearest even.  The dead-tier
 * latent dot products use the canonical adjacent-pair tree over
 * next_pow2(nz) zero-padded products.  exp/log are the codec's binary64
 * recipe rounded once to binary32 (same algorithm as the device).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- formats */

static float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static double bits_d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static uint64_t d_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

float orc_f16_to_f32(uint16_t h) {
  uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  if (e == 0) {
    float v = (float)m * 0x1p-24f; /* exact */
    return s ? -v : v;
  }
  if (e == 31) return bits_f(s | 0x7F800000u | (m << 13));
  return bits_f(s | ((e + 112) << 23) | (m << 13));
}

/* binary32 -> binary16, round to nearest even, subnormals, overflow to inf */
uint16_t orc_f32_to_f16(float f) {
  uint32_t u = f_bits(f);
  uint32_t s = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint16_t)(s | 0x7E00u | ((a >> 13) & 0x3FF));
  if (a >= 0x477FF000u) return (uint16_t)(s | 0x7C00u); /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                 /* below 2^-14: subnormal */
    /* value / 2^-24 rounded to nearest even integer */
    float q = bits_f(a) * 0x1p24f;                       /* exact scaling */
    float r = rintf(q);                                  /* RNE (default mode) */
    return (uint16_t)(s | (uint32_t)r);
  }
  uint32_t r = a + 0xFFFu + ((a >> 13) & 1u);
  r &= ~0x1FFFu;
  return (uint16_t)(s | (((r >> 23) - 112) << 10) | ((r >> 13) & 0x3FF));
}

float orc_e4m3_to_f32(uint8_t b) {
  uint32_t s = (uint32_t)(b >> 7) << 31, e = (b >> 3) & 15, m = b & 7;
  if ((b & 0x7F) == 0x7F) return bits_f(s | 0x7FC00000u);
  if (e == 0) {
    float v = (float)m * 0x1p-9f;
    return s ? -v : v;
  }
  return bits_f(s | ((e + 120) << 23) | (m << 20));
}

/* binary32 -> E4M3FN round to nearest even; callers clamp to +-448 first. */
uint8_t orc_f32_to_e4m3(float f) {
  uint32_t u = f_bits(f);
  uint32_t s = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return (uint8_t)(s | 0x7F);
  if (a >= 0x43E80000u) return (uint8_t)(s | 0x7F);       /* >= 464: not representable */
  if (a < 0x3C800000u) {                                   /* below 2^-6 */
    float r = rintf(bits_f(a) * 512.0f);
    return (uint8_t)(s | (uint32_t)r);
  }
  uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
  r &= ~0xFFFFFu;
  return (uint8_t)(s | ((((r >> 23) - 120) << 3) | ((r >> 20) & 7)));
}

/* ------------------------------------------------------- transcendentals */

double orc_exp_d(double x) {
  if (x > 100.0) return INFINITY;
  if (x < -110.0) return 0.0;
  const double inv_ln2 = 1.4426950408889634;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  const double magic = 6755399441055744.0;
  double kd = (x * inv_ln2 + magic) - magic;
  double r = (x - kd * ln2_hi) - kd * ln2_lo;
  double p = 1.0 / 6227020800.0;
  p = fma(p, r, 1.0 / 479001600.0);
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  int64_t k = (int64_t)kd;
  double scale = bits_d((uint64_t)(k + 1023) << 52);
  return p * scale;
}

double orc_log_d(double x) {
  uint64_t u = d_bits(x);
  int64_t e = (int64_t)((u >> 52) & 0x7FF) - 1023;
  double m = bits_d((u & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
  if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
  double s = (m - 1.0) / (m + 1.0);
  double s2 = s * s;
  double p = 1.0 / 23.0;
  p = fma(p, s2, 1.0 / 21.0);
  p = fma(p, s2, 1.0 / 19.0);
  p = fma(p, s2, 1.0 / 17.0);
  p = fma(p, s2, 1.0 / 15.0);
  p = fma(p, s2, 1.0 / 13.0);
  p = fma(p, s2, 1.0 / 11.0);
  p = fma(p, s2, 1.0 / 9.0);
  p = fma(p, s2, 1.0 / 7.0);
  p = fma(p, s2, 1.0 / 5.0);
  p = fma(p, s2, 1.0 / 3.0);
  p = fma(p, s2, 1.0);
  double logm = 2.0 * s * p;
  double ed = (double)e;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  return (ed * ln2_hi + logm) + ed * ln2_lo;
}

float orc_expf(float x) { return (float)orc_exp_d((double)x); }
float orc_logf(float x) { return (float)orc_log_d((double)x); }

/* dt activation inside the codec kernels (fp4_zero_predictor_codec_v1.py:123-124) */
float orc_softplus_dt(float v) {
  if (v <= 20.0f) {
    float e = orc_expf(v);
    float ep1 = e + 1.0f;
    return orc_logf(ep1);
  }
  return v;
}

/* The recurrent update of every codec, written in the reference kernels as
 * `state * decay + (b * dt) * x` (fp4_zero_predictor_codec_v1.py:135-136,149-150;
 * state_ppl_codec_v10.py:123-124; state_codec.py:91,149-150;
 * state_codec_dense3.py:129).  Triton compiles with floating-point fusion
 * enabled by default, which contracts this sum into one fused multiply-add
 * on its first product: state = fma(state, decay, RN(RN(b * dt) * x)).  The
 * build defines the update that way (one rounding of state * decay + the
 * rounded input term). */
float orc_update(float state, float decay, float input_term) { return fmaf(state, decay, input_term); }

/* _stored_quantize (state_ppl_codec_v6.py:52-61) */
int32_t orc_stored_quantize(float value, float scale, float limit) {
  float safe = scale > 0.0f ? scale : 1.0f;
  float quotient = value / safe;
  float rounded = roundf(quotient);
  float clipped = fminf(fmaxf(rounded, -limit), limit);
  return scale > 0.0f ? (int32_t)clipped : 0;
}

/* Canonical adjacent-pair tree over `n` (a power of two) values. */
static float pair_tree(float* v, int n) {
  for (int w = n; w > 1; w >>= 1)
    for (int i = 0; i < w / 2; ++i) v[i] = v[2 * i] + v[2 * i + 1];
  return v[0];
}

static int next_pow2(int v) { int r = 1; while (r < v) r <<= 1; return r; }

static float load_param(const void* p, int f32, int64_t i) {
  return f32 ? ((const float*)p)[i] : orc_f16_to_f32(((const uint16_t*)p)[i]);
}

/* ------------------------------------------------ FP16-carry control step
 * _s16_scan (mamba2_recall/state_codec.py:65-102): per row the FP32 carry is
 * fma(state, decay, RN(RN(b*dt)*x)) (the contracted update, see
 * orc_update), read out against C with D*x,
 * then rounded to FP16.  Statistics (optional, may be NULL): for every
 * (b, h, 16-row tile of P, coordinate) the sum over tokens and tile rows of
 * |FP16 carry| in binary32, in this order: each row's sum over the tokens in
 * token order (the per-program accumulator of state_codec.py:100-101), the
 * rows of each 4-row sub-tile as (r0 + r1) + (r2 + r3) (the tl.sum of :102;
 * rows past P add zero), then the four sub-tiles of the 16-row tile in order,
 * ((T0 + T1) + T2) + T3 (the host sum over sub-tiles, state_codec.py:255-261,
 * missing sub-tiles zero).  state is [B,H,P,128] f16 bits, stats
 * [B,H,ceil(P/16),128] f32.
 */
int orc_s16_step(const uint16_t* X, const uint16_t* DT, const float* A, const uint16_t* Bm, const uint16_t* Cm,
                 const void* D, int d_f32, const void* DB, int db_f32, uint16_t* S, uint16_t* Y, float* stats,
                 int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G) {
  if (H % G) return 1;
  const int64_t hpg = H / G, tiles = (P + 15) / 16;
  if (stats) memset(stats, 0, sizeof(float) * batch * H * tiles * 128);
  #pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t h = 0; h < H; ++h) {
      const int64_t g = h / hpg;
      const float av = A[h], dv = load_param(D, d_f32, h), bias = load_param(DB, db_f32, h);
      /* per-row sums over the tokens, rows padded to whole 16-row tiles */
      float* acc = stats ? (float*)calloc((size_t)tiles * 16 * 128, sizeof(float)) : NULL;
      for (int64_t p = 0; p < P; ++p) {
        uint16_t* st = S + ((b * H + h) * P + p) * 128;
        float v[128];
        for (int n = 0; n < 128; ++n) v[n] = orc_f16_to_f32(st[n]);
        for (int64_t t = 0; t < L; ++t) {
          const int64_t bt = b * L + t;
          const float x = orc_f16_to_f32(X[(bt * H + h) * P + p]);
          const float dtv = orc_softplus_dt(orc_f16_to_f32(DT[bt * H + h]) + bias);
          const float decay = orc_expf(av * dtv);
          const uint16_t* bv = Bm + (bt * G + g) * 128;
          const uint16_t* cv = Cm + (bt * G + g) * 128;
          double out = 0.0;
          for (int n = 0; n < 128; ++n) {
            const float db = orc_f16_to_f32(bv[n]) * dtv;
            v[n] = orc_update(v[n], decay, db * x);
            out += (double)v[n] * (double)orc_f16_to_f32(cv[n]);
          }
          Y[(bt * H + h) * P + p] = orc_f32_to_f16((float)out + x * dv);
          for (int n = 0; n < 128; ++n) {
            v[n] = orc_f16_to_f32(orc_f32_to_f16(v[n]));
            if (acc) acc[p * 128 + n] = acc[p * 128 + n] + fabsf(v[n]);
          }
        }
        for (int n = 0; n < 128; ++n) st[n] = orc_f32_to_f16(v[n]);
      }
      if (acc) {
        for (int64_t tile = 0; tile < tiles; ++tile)
          for (int n = 0; n < 128; ++n) {
            float sub[4];
            for (int j = 0; j < 4; ++j) {
              const float* r = acc + (tile * 16 + 4 * j) * 128 + n;
              sub[j] = (r[0] + r[128]) + (r[256] + r[384]);
            }
            stats[((b * H + h) * tiles + tile) * 128 + n] = ((sub[0] + sub[1]) + sub[2]) + sub[3];
          }
        free(acc);
      }
    }
  return 0;
}

/* ------------------------------------------------ packed 52-byte state step
 * mode 0: legacy sq3p25 (FP32 denominator quantize, state_codec.py:156-163)
 * mode 1: stored-scale tiers (state_ppl_codec_v10.py:110-141)
 * mode 2: ridge latent (fp4_zero_predictor_codec_v1.py:115-162)
 * Arrays are the reference's SoA tensors, contiguous, f16 as raw bits.
 */
int orc_state_step(int mode, int n8, int n4, int nz, const uint16_t* X, const uint16_t* DT, const float* A,
                   const uint16_t* Bm, const uint16_t* Cm, const void* D, int d_f32, const void* DB, int db_f32,
                   const uint8_t* perm, const uint16_t* basis, const uint16_t* lscale, const uint16_t* pred,
                   uint8_t* lo, uint8_t* hi, uint8_t* q4, uint8_t* latent, uint16_t* S8, uint16_t* S4,
                   uint16_t* Y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G) {
  if (n8 + n4 + nz != 128 || n8 % 2 || n4 % 2 || H % G) return 1;
  const int F = n8 + n4 + 2;
  const int RZ = next_pow2(nz);
  const int64_t hpg = H / G;
  /* per (b, t, g) shared values */
  const int64_t nbtg = batch * L * G;
  float* bperm = (float*)malloc(sizeof(float) * nbtg * 128);
  float* cperm = (float*)malloc(sizeof(float) * nbtg * 128);
  float* corr = (float*)malloc(sizeof(float) * nbtg * F);
  float* dots = (float*)malloc(sizeof(float) * nbtg * 5);
  if (!bperm || !cperm || !corr || !dots) return 2;
  for (int64_t i = 0; i < nbtg; ++i) {
    int64_t g = i % G;
    for (int n = 0; n < 128; ++n) {
      int pos = perm[g * 128 + n];
      bperm[i * 128 + n] = orc_f16_to_f32(Bm[i * 128 + pos]);
      cperm[i * 128 + n] = orc_f16_to_f32(Cm[i * 128 + pos]);
    }
    if (mode == 2) {
      const float* bb = bperm + i * 128 + n8 + n4;
      const float* cc = cperm + i * 128 + n8 + n4;
      /* correction[f] = sum_d float(Cdead[d]) * float(pred[g,f,d]) (:221-223) */
      for (int f = 0; f < F; ++f) {
        float acc = 0.0f;
        for (int d = 0; d < nz; ++d) acc = acc + cc[d] * orc_f16_to_f32(pred[(g * F + f) * nz + d]);
        corr[i * F + f] = acc;
      }
      float t[128];
      for (int k = 0; k < 5; ++k) {
        for (int d = 0; d < RZ; ++d) {
          float v = 0.0f;
          if (d < nz) {
            float e0 = orc_f16_to_f32(basis[(g * nz + d) * 2]);
            float e1 = orc_f16_to_f32(basis[(g * nz + d) * 2 + 1]);
            switch (k) {
              case 0: v = bb[d] * cc[d]; break; /* dot_bc */
              case 1: v = e0 * cc[d]; break;    /* dot_c0 */
              case 2: v = e1 * cc[d]; break;    /* dot_c1 */
              case 3: v = e0 * bb[d]; break;    /* dot_b0 */
              default: v = e1 * bb[d]; break;   /* dot_b1 */
            }
          }
          t[d] = v;
        }
        dots[i * 5 + k] = pair_tree(t, RZ);
      }
    }
  }
  const int64_t rows = batch * H * P;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t b = r / (H * P), h = (r / P) % H, p = r % P;
    const int64_t g = h / hpg;
    float st8[128], st4[128], prior8[128], prior4[128];
    int32_t q8[128], q4v[128];
    float s8 = orc_f16_to_f32(S8[r]), s4 = orc_f16_to_f32(S4[r]);
    for (int n = 0; n < n8; ++n) {
      int lon = (lo[r * (n8 / 2) + n / 2] >> ((n % 2) * 4)) & 15;
      int hin = (hi[r * (n8 / 2) + n / 2] >> ((n % 2) * 4)) & 15;
      int ub = (hin << 4) | lon;
      q8[n] = ub - 256 * (ub > 127);
      st8[n] = (float)q8[n] * s8;
    }
    for (int n = 0; n < n4; ++n) {
      int nib = (q4[r * (n4 / 2) + n / 2] >> ((n % 2) * 4)) & 15;
      q4v[n] = nib - 16 * (nib > 7);
      st4[n] = (float)q4v[n] * s4;
    }
    const float av = A[h], dv = load_param(D, d_f32, h), bias = load_param(DB, db_f32, h);
    float ls0 = 0, ls1 = 0, z0 = 0, z1 = 0;
    uint8_t qz0 = 0, qz1 = 0;
    if (mode == 2) {
      ls0 = orc_f16_to_f32(lscale[g * 2]);
      ls1 = orc_f16_to_f32(lscale[g * 2 + 1]);
      qz0 = latent[r * 2];
      qz1 = latent[r * 2 + 1];
      z0 = orc_e4m3_to_f32(qz0) * ls0;
      z1 = orc_e4m3_to_f32(qz1) * ls1;
    }
    for (int64_t t = 0; t < L; ++t) {
      const int64_t bt = b * L + t, i = bt * G + g;
      const float* bv = bperm + i * 128;
      const float* cv = cperm + i * 128;
      const int64_t xoff = (bt * H + h) * P + p;
      float x = orc_f16_to_f32(X[xoff]);
      float dtv = orc_f16_to_f32(DT[bt * H + h]) + bias;
      dtv = orc_softplus_dt(dtv);
      float decay = orc_expf(av * dtv);
      for (int n = 0; n < n8; ++n) { prior8[n] = st8[n]; st8[n] = orc_update(prior8[n], decay, (bv[n] * dtv) * x); }
      for (int n = 0; n < n4; ++n) {
        prior4[n] = st4[n];
        st4[n] = orc_update(prior4[n], decay, (bv[n8 + n] * dtv) * x);
      }
      float out = 0.0f;
      for (int n = 0; n < n8; ++n) out += st8[n] * cv[n];
      for (int n = 0; n < n4; ++n) out += st4[n] * cv[n8 + n];
      if (mode == 2) {
        const float* d5 = dots + i * 5;
        const float* pc = corr + i * F;
        out += decay * (z0 * d5[1] + z1 * d5[2]) + (x * dtv) * d5[0] + x * dv;
        float ap = 0.0f;
        for (int n = 0; n < n8; ++n) ap += prior8[n] * pc[n];
        for (int n = 0; n < n4; ++n) ap += prior4[n] * pc[n8 + n];
        out += decay * (ap + z0 * pc[n8 + n4] + z1 * pc[n8 + n4 + 1]);
        Y[xoff] = orc_f32_to_f16(out);
        z0 = orc_update(z0, decay, (x * dtv) * d5[3]);
        z1 = orc_update(z1, decay, (x * dtv) * d5[4]);
        qz0 = orc_f32_to_e4m3(fminf(fmaxf(z0 / ls0, -448.0f), 448.0f));
        qz1 = orc_f32_to_e4m3(fminf(fmaxf(z1 / ls1, -448.0f), 448.0f));
        z0 = orc_e4m3_to_f32(qz0) * ls0;
        z1 = orc_e4m3_to_f32(qz1) * ls1;
      } else {
        float dead = 0.0f;
        for (int d = 0; d < nz; ++d) dead += ((bv[n8 + n4 + d] * dtv) * x) * cv[n8 + n4 + d];
        out += dead + x * dv;
        Y[xoff] = orc_f32_to_f16(out);
      }
      float amax8 = 0.0f, amax4 = 0.0f;
      for (int n = 0; n < n8; ++n) amax8 = fmaxf(amax8, fabsf(st8[n]));
      for (int n = 0; n < n4; ++n) amax4 = fmaxf(amax4, fabsf(st4[n]));
      if (mode == 0) {
        float den8 = fmaxf(amax8 / 127.0f, 1e-8f);
        float den4 = fmaxf(amax4 / 7.0f, 1e-8f);
        for (int n = 0; n < n8; ++n) q8[n] = (int32_t)fminf(fmaxf(roundf(st8[n] / den8), -127.0f), 127.0f);
        for (int n = 0; n < n4; ++n) q4v[n] = (int32_t)fminf(fmaxf(roundf(st4[n] / den4), -7.0f), 7.0f);
        s8 = orc_f16_to_f32(orc_f32_to_f16(den8));
        s4 = orc_f16_to_f32(orc_f32_to_f16(den4));
      } else {
        float den8 = fmaxf(amax8 / 127.0f, 1e-8f);
        float den4 = fmaxf(amax4 / 7.0f, 1e-8f);
        s8 = orc_f16_to_f32(orc_f32_to_f16(den8));
        s4 = orc_f16_to_f32(orc_f32_to_f16(den4));
        for (int n = 0; n < n8; ++n) q8[n] = orc_stored_quantize(st8[n], s8, 127.0f);
        for (int n = 0; n < n4; ++n) q4v[n] = orc_stored_quantize(st4[n], s4, 7.0f);
      }
      for (int n = 0; n < n8; ++n) st8[n] = (float)q8[n] * s8;
      for (int n = 0; n < n4; ++n) st4[n] = (float)q4v[n] * s4;
    }
    for (int j = 0; j < n8 / 2; ++j) {
      lo[r * (n8 / 2) + j] = (uint8_t)((q8[2 * j] & 15) | ((q8[2 * j + 1] & 15) << 4));
      hi[r * (n8 / 2) + j] = (uint8_t)(((q8[2 * j] >> 4) & 15) | (((q8[2 * j + 1] >> 4) & 15) << 4));
    }
    for (int j = 0; j < n4 / 2; ++j)
      q4[r * (n4 / 2) + j] = (uint8_t)((q4v[2 * j] & 15) | ((q4v[2 * j + 1] & 15) << 4));
    S8[r] = orc_f32_to_f16(s8);
    S4[r] = orc_f32_to_f16(s4);
    if (mode == 2) {
      /* final store re-rounds clamp(z / ls) (:176-179); z = e4m3 * ls exactly */
      latent[r * 2] = orc_f32_to_e4m3(fminf(fmaxf(z0 / ls0, -448.0f), 448.0f));
      latent[r * 2 + 1] = orc_f32_to_e4m3(fminf(fmaxf(z1 / ls1, -448.0f), 448.0f));
    }
  }
  free(bperm); free(cperm); free(corr); free(dots);
  return 0;
}

/* ----------------------------------------------------------- dense 3-bit
 * state_codec_dense3.py:82-148.  table_kind 0 = permutation (u8),
 * 1 = power-of-two equalizer (i8 exponents).  codes [rows,3,16], scales
 * [rows,2] f16.
 */
int orc_dense3_step(int table_kind, const uint16_t* X, const uint16_t* DT, const float* A, const uint16_t* Bm,
                    const uint16_t* Cm, const void* D, int d_f32, const void* DB, int db_f32, const void* table,
                    uint8_t* codes, uint16_t* scales, uint16_t* Y, int64_t batch, int64_t L, int64_t H, int64_t P,
                    int64_t G) {
  if (H % G) return 1;
  const int64_t hpg = H / G;
  const int64_t rows = batch * H * P;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t b = r / (H * P), h = (r / P) % H, p = r % P;
    const int64_t g = h / hpg;
    float st[128];
    int32_t q[128];
    float sc[2] = {orc_f16_to_f32(scales[r * 2]), orc_f16_to_f32(scales[r * 2 + 1])};
    for (int n = 0; n < 128; ++n) {
      int u = 0;
      for (int k = 0; k < 3; ++k) u |= ((codes[r * 48 + 16 * k + n / 8] >> (n % 8)) & 1) << k;
      q[n] = u - 8 * (u >= 4);
      st[n] = (float)q[n] * sc[n / 64];
    }
    int pos[128];
    float wf[128], rf[128];
    for (int n = 0; n < 128; ++n) {
      if (table_kind == 0) {
        pos[n] = ((const uint8_t*)table)[g * 128 + n];
      } else {
        int k = ((const int8_t*)table)[g * 128 + n];
        pos[n] = n;
        wf[n] = ldexpf(1.0f, -k); /* exp2(-k), exact */
        rf[n] = ldexpf(1.0f, k);
      }
    }
    const float av = A[h], dv = load_param(D, d_f32, h), bias = load_param(DB, db_f32, h);
    for (int64_t t = 0; t < L; ++t) {
      const int64_t bt = b * L + t;
      const int64_t xoff = (bt * H + h) * P + p;
      float x = orc_f16_to_f32(X[xoff]);
      float dtv = orc_softplus_dt(orc_f16_to_f32(DT[bt * H + h]) + bias);
      float decay = orc_expf(av * dtv);
      float out = 0.0f;
      for (int n = 0; n < 128; ++n) {
        float bv = orc_f16_to_f32(Bm[(bt * G + g) * 128 + pos[n]]);
        float cv = orc_f16_to_f32(Cm[(bt * G + g) * 128 + pos[n]]);
        if (table_kind == 1) { bv = bv * wf[n]; cv = cv * rf[n]; }
        st[n] = orc_update(st[n], decay, (bv * dtv) * x);
        out += st[n] * cv;
      }
      out += x * dv;
      Y[xoff] = orc_f32_to_f16(out);
      for (int half = 0; half < 2; ++half) {
        float amax = 0.0f;
        for (int n = 64 * half; n < 64 * half + 64; ++n) amax = fmaxf(amax, fabsf(st[n]));
        float den = fmaxf(amax / 3.0f, 1e-8f);
        for (int n = 64 * half; n < 64 * half + 64; ++n)
          q[n] = (int32_t)fminf(fmaxf(roundf(st[n] / den), -3.0f), 3.0f);
        sc[half] = orc_f16_to_f32(orc_f32_to_f16(den));
        for (int n = 64 * half; n < 64 * half + 64; ++n) st[n] = (float)q[n] * sc[half];
      }
    }
    for (int k = 0; k < 3; ++k)
      for (int j = 0; j < 16; ++j) {
        int byte = 0;
        for (int bit = 0; bit < 8; ++bit) byte |= (((q[8 * j + bit] & 7) >> k) & 1) << bit;
        codes[r * 48 + 16 * k + j] = (uint8_t)byte;
      }
    scales[r * 2] = orc_f32_to_f16(sc[0]);
    scales[r * 2 + 1] = orc_f32_to_f16(sc[1]);
  }
  return 0;
}

/* ------------------------------------------------- legacy diagnostic encode
 * mamba2_recall/state_codec.py:299-331 (encode_state_, mode sq3p25): for each
 * row of 128 FP32 coordinates in packed order, s8 = max(amax(|v[0:16]|) /
 * 127, 1e-8), s4 = max(amax(|v[16:80]|) / 7, 1e-8) in binary32; codes
 * sign(z) * floor(|z| + 0.5) of z = v / s, clamped to +-127 / +-7; nibble
 * planes lo/hi (INT8 low and high nibbles, two coordinates per byte) and q4;
 * stored scales half(s).  Coordinates 80..127 are not stored.
 */
static int32_t legacy_code(float v, float s, float limit) {
  float z = v / s;
  float sgn = z > 0.0f ? 1.0f : (z < 0.0f ? -1.0f : 0.0f);
  float m = sgn * floorf(fabsf(z) + 0.5f);
  return (int32_t)fminf(fmaxf(m, -limit), limit);
}

void orc_encode_legacy(const float* v, uint8_t* lo, uint8_t* hi, uint8_t* q4, uint16_t* s8, uint16_t* s4,
                       int64_t rows) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = v + r * 128;
    float m8 = 0.0f, m4 = 0.0f;
    for (int n = 0; n < 16; ++n) m8 = fmaxf(m8, fabsf(x[n]));
    for (int n = 16; n < 80; ++n) m4 = fmaxf(m4, fabsf(x[n]));
    const float d8 = fmaxf(m8 / 127.0f, 1e-8f), d4 = fmaxf(m4 / 7.0f, 1e-8f);
    int32_t q[80];
    for (int n = 0; n < 16; ++n) q[n] = legacy_code(x[n], d8, 127.0f);
    for (int n = 16; n < 80; ++n) q[n] = legacy_code(x[n], d4, 7.0f);
    for (int j = 0; j < 8; ++j) {
      lo[r * 8 + j] = (uint8_t)((q[2 * j] & 15) | ((q[2 * j + 1] & 15) << 4));
      hi[r * 8 + j] = (uint8_t)(((q[2 * j] >> 4) & 15) | (((q[2 * j + 1] >> 4) & 15) << 4));
    }
    for (int j = 0; j < 32; ++j) q4[r * 32 + j] = (uint8_t)((q[16 + 2 * j] & 15) | ((q[17 + 2 * j] & 15) << 4));
    s8[r] = orc_f32_to_f16(d8);
    s4[r] = orc_f32_to_f16(d4);
  }
}

/* ---------------------------------------------------------------- FP4 decode
 * fp4.py:151-154 + decode_packet's checks (:236, :245, :247, :249).  Returns
 * the same error bits as the device kernel; out is [rows, cols] f16 bits.
 * group 16: scales are E4M3FN bytes and `global_scale` applies; group 64:
 * scales are f16 bits and global_scale is ignored.
 */
uint32_t orc_fp4_decode(int group, const uint8_t* packed, const void* scales, float global_scale, uint16_t* out,
                        int64_t rows, int64_t cols) {
  static const float lev[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  const int64_t groups = (cols + group - 1) / group, padded = groups * group;
  uint32_t err = 0;
  if (group == 16 && !(global_scale > 0.0f && isfinite(global_scale))) err |= 32u;
#pragma omp parallel for reduction(| : err) schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t q = 0; q < groups; ++q) {
      float sf;
      if (group == 16) sf = orc_e4m3_to_f32(((const uint8_t*)scales)[r * groups + q]);
      else sf = orc_f16_to_f32(((const uint16_t*)scales)[r * groups + q]);
      if (!isfinite(sf)) err |= 1u;
      else if (!(sf >= 0.0f)) err |= 2u;
      for (int64_t j = 0; j < group; ++j) {
        int64_t c = q * group + j;
        int code = (packed[r * (padded / 2) + c / 2] >> ((c % 2) * 4)) & 15;
        if (c >= cols) { if (code) err |= 16u; continue; }
        if (sf == 0.0f && code != 0 && code != 8) err |= 4u;
        float sign = (code & 8) ? -1.0f : 1.0f;
        float v = lev[code & 7] * sign; /* _decode_e2m1_codes */
        v = v * sf;                     /* * scales.float() */
        if (group == 16) v = v * global_scale;
        uint16_t hbits = orc_f32_to_f16(v); /* .half() */
        if ((hbits & 0x7FFF) >= 0x7C00) err |= 8u;
        out[r * cols + c] = hbits;
      }
    }
  }
  return err;
}

/* Elementwise primitive table, mirroring the device probe op numbering. */
void orc_unary(const uint32_t* in, uint32_t* out, int64_t n, int op) {
  for (int64_t i = 0; i < n; ++i) {
    uint32_t u = in[i];
    float f = bits_f(u);
    uint32_t r = 0;
    switch (op) {
      case 0: r = orc_f32_to_f16(f); break;
      case 1: r = f_bits(orc_f16_to_f32((uint16_t)u)); break;
      case 2: r = orc_f32_to_e4m3(f); break;
      case 3: r = f_bits(orc_e4m3_to_f32((uint8_t)u)); break;
      case 4: r = f_bits(roundf(f)); break;
      case 5: r = f_bits(orc_expf(f)); break;
      case 6: r = f_bits(orc_logf(f)); break;
      case 7: r = f_bits(orc_softplus_dt(f)); break;
      default: r = 0; break;
    }
    out[i] = r;
  }
}

void orc_stored_quantize_n(const float* v, const uint16_t* s, int32_t* q, int64_t n, int limit) {
  for (int64_t i = 0; i < n; ++i) q[i] = orc_stored_quantize(v[i], orc_f16_to_f32(s[i]), (float)limit);
}

/* Exhaustive check helper: counts inputs x in [lo_bits, hi_bits] (positive
 * float bit patterns) where trunc(x + pred(0.5)) != roundf(x); also for -x. */
int64_t orc_check_round_identity(uint32_t lo_bits, uint32_t hi_bits) {
  int64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (int64_t u = lo_bits; u <= (int64_t)hi_bits; ++u) {
    float x = bits_f((uint32_t)u);
    for (int s = 0; s < 2; ++s) {
      float y = s ? -x : x;
      float a = truncf(y + copysignf(0x1.fffffep-2f, y));
      float b = roundf(y);
      if (f_bits(a) != f_bits(b)) ++bad;
    }
  }
  return bad;
}

/* Checks the device's reciprocal-form quantizer against the literal one:
 * code(a) = (int)clamp(trunc(q + copysign(pred(0.5), q)), +-lim) with
 * q = fma(fma(-a*y, d, a), y, a*y), y = 1/d, versus
 * (int)clamp(roundf(a / d), +-lim).  Inputs: deterministic pseudo-random
 * (a, d) pairs with a = fl(u*d) for a random quotient u in [0, 256) moved
 * by a few ulps, plus every half-integer boundary (k + 1/2) * d +- 4 ulps,
 * plus zeros and subnormal dividends.  Returns the number of differing
 * codes.  `div_bad` receives the number of nonzero normal-range dividends
 * whose quotient bits differ from IEEE division (Markstein's theorem says
 * none). */
int64_t orc_check_markstein(uint64_t seed, int64_t n_random, int n_boundary_scales, int64_t* div_bad) {
  int64_t bad = 0, dbad = 0;
#pragma omp parallel for reduction(+ : bad, dbad) schedule(static)
  for (int64_t i = 0; i < n_random; ++i) {
    uint64_t z = seed + (uint64_t)i * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    float d;
    if (z & 1) d = orc_f16_to_f32((uint16_t)(((z >> 1) % 0x7BFF) + 1));
    else d = bits_f((uint32_t)(0x2E000000u + ((z >> 1) % 0x1E000000u)));
    float u = bits_f((uint32_t)(0x3F800000u | ((z >> 20) & 0x7FFFFFu))) * (float)(1u << ((z >> 43) & 7)) - 1.0f;
    float a;
    switch ((z >> 56) & 15) {
      case 0: a = 0.0f; break;                                         /* zero */
      case 1: a = bits_f((uint32_t)((z >> 8) & 0x7FFFFFu)); break;     /* subnormal */
      default: a = bits_f(f_bits(u * d) + (int32_t)((z >> 50) & 7) - 3); break;
    }
    if (!isfinite(a) || !isfinite(d) || d == 0.0f) continue;
    if (z & 2) a = -a;
    float lim = (z & 4) ? 127.0f : ((z & 8) ? 7.0f : 3.0f);
    float y = 1.0f / d;
    float q0 = a * y;
    float r = fmaf(-q0, d, a);
    float q = fmaf(r, y, q0);
    if (a != 0.0f && fabsf(a) >= 0x1p-100f && f_bits(q) != f_bits(a / d)) ++dbad;
    /* device form: clamp below +-(lim+1) and let the int conversion truncate */
    const float top = nextafterf(lim + 1.0f, 0.0f);
    int c1 = (int)fminf(fmaxf(q + copysignf(0x1.fffffep-2f, q), -top), top);
    int c2 = (int)fminf(fmaxf(roundf(a / d), -lim), lim);
    if (c1 != c2) ++bad;
  }
  for (int si = 0; si < n_boundary_scales; ++si) {
    float d = orc_f16_to_f32((uint16_t)(0x0001 + (si * 7919) % 0x7BFF));
    float y = 1.0f / d;
    for (int k = 0; k <= 128; ++k) {
      float m = ((float)k + 0.5f) * d; /* exact */
      uint32_t mb = f_bits(m);
      for (int du = -4; du <= 4; ++du) {
        float a = bits_f(mb + du);
        for (int s = 0; s < 2; ++s) {
          float aa = s ? -a : a;
          float q0 = aa * y;
          float r = fmaf(-q0, d, aa);
          float q = fmaf(r, y, q0);
          if (fabsf(aa) >= 0x1p-100f && f_bits(q) != f_bits(aa / d)) ++dbad;
          int c1 = (int)fminf(fmaxf(q + copysignf(0x1.fffffep-2f, q), -0x1.fffffep+6f), 0x1.fffffep+6f);
          int c2 = (int)fminf(fmaxf(roundf(aa / d), -127.0f), 127.0f);
          if (c1 != c2) ++bad;
        }
      }
    }
  }
  if (div_bad) *div_bad = dbad;
  return bad;
}

/* The latent quotient z / ls is taken on the device as
 * copysign(fma(fma(-z*y, ls, z), y, z*y), z) with y = RN(1/ls); the E4M3 byte
 * of clamp(quotient, +-448) must equal the one from IEEE division.  Checks
 * every binary16 ls in [2^-24, 65504] against dense z: all E4M3 values times
 * ls and their midpoints (+-2 ulps), zeros of both signs, subnormal z, and
 * pseudo-random z.  Returns the number of differing bytes. */
int64_t orc_check_latent_division(uint64_t seed, int n_random_per_scale) {
  int64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 64)
  for (int sb = 1; sb < 0x7C00; ++sb) {
    const float ls = orc_f16_to_f32((uint16_t)sb);
    const float y = 1.0f / ls;
    uint64_t z = seed ^ ((uint64_t)sb * 0x9E3779B97F4A7C15ull);
    for (int i = -n_random_per_scale - 520; i < n_random_per_scale; ++i) {
      float zv;
      if (i < -n_random_per_scale) {
        int k = i + n_random_per_scale + 520;        /* 0..519 structured cases */
        if (k < 256) {
          float e = orc_e4m3_to_f32((uint8_t)(k & 0x7F));
          zv = bits_f(f_bits(e * ls) + (k >> 7) * 2 - 1);
        } else if (k < 512) {
          int kk = k - 256;
          float e0 = orc_e4m3_to_f32((uint8_t)(kk & 0x7E)), e1 = orc_e4m3_to_f32((uint8_t)((kk & 0x7E) + 1));
          zv = ((e0 + e1) * 0.5f) * ls;                /* near every rounding midpoint */
          zv = bits_f(f_bits(zv) + (kk & 1 ? 1 : -1));
        } else if (k == 512) zv = 0.0f;
        else if (k == 513) zv = -0.0f;
        else zv = bits_f((uint32_t)(k * 977));          /* subnormals */
        if (!isfinite(zv)) continue;                     /* NaN is outside the contract */
      } else {
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        zv = bits_f((uint32_t)(z & 0x7FFFFFFFu));
        if (!isfinite(zv)) continue;
      }
      const float top = 464.0f * ls;   /* exact; beyond it both quotients clamp to 448 */
      for (int sgn = 0; sgn < 2; ++sgn) {
        const float a = sgn ? -zv : zv;
        const float ac = fminf(fmaxf(a, -top), top);
        float q0 = ac * y;
        float r = fmaf(-q0, ls, ac);
        float q = copysignf(fmaf(r, y, q0), a);
        uint8_t b1 = orc_f32_to_e4m3(fminf(fmaxf(q, -448.0f), 448.0f));
        uint8_t b2 = orc_f32_to_e4m3(fminf(fmaxf(a / ls, -448.0f), 448.0f));
        if (b1 != b2) ++bad;
      }
    }
  }
  return bad;
}

/* The device's fast quantizer for quotients that need no clamping: with
 * y = RN(1/d) and magic = 1.5 * 2^23 + bias, t = fma(v, y, magic) holds
 * bias + rint(v*y) in its low bits and f = fma(v, y, -(t - magic)) is the
 * rounding residual.  The device keeps that code unless |f| exceeds the
 * residual bound thr (thr8 for lim 127, thr4 for lim 7 and 3), in which case
 * it requantizes with the exact quotient.  Counts the (v, d) pairs with
 * |f| <= thr whose fast code differs from roundf(v / d) (IEEE division), or
 * whose low byte is not (code + bias) mod 256.  Inputs: pseudo-random scales
 * (normal binary16 values, and binary32 values >= 2^-26 for the binary32
 * denominators of the legacy codec) with quotients uniform in
 * |v / d| <= lim + 0.49, and every half-integer boundary (k + 1/2) * d moved
 * by up to +-40 ulps, both signs.  `flagged` receives the number of pairs
 * sent to the exact path. */
int64_t orc_check_residual_round(uint64_t seed, int64_t n_random, int n_boundary_scales, float thr8, float thr4,
                                 int64_t* flagged) {
  int64_t bad = 0, flg = 0;
#pragma omp parallel for reduction(+ : bad, flg) schedule(static)
  for (int64_t i = 0; i < n_random + (int64_t)n_boundary_scales; ++i) {
    uint64_t z = seed + (uint64_t)i * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const int li = (int)((z >> 3) % 3);
    const float lim = li == 0 ? 127.0f : (li == 1 ? 7.0f : 3.0f);
    const float bias = li == 0 ? 128.0f : (li == 1 ? 8.0f : 4.0f);
    const float thr = li == 0 ? thr8 : thr4;
    float d;
    if (z & 1) d = orc_f16_to_f32((uint16_t)(0x0400 + (uint16_t)((z >> 8) % (0x7BFF - 0x0400 + 1))));
    else d = bits_f((uint32_t)(0x32800000u + ((z >> 8) % (0x7F000000u - 0x32800000u))));
    const float y = 1.0f / d;
    const float magic = 0x1.8p23f + bias;
    float vs[2 * 81 * 2 + 1];
    int nv = 0;
    if (i < n_random) {
      const float u = (bits_f((uint32_t)(0x3F800000u | ((z >> 20) & 0x7FFFFFu))) - 1.5f) * 2.0f * (lim + 0.49f);
      vs[nv++] = u * d;
    } else {
      const int k = (int)((z >> 40) % (uint64_t)lim);     /* boundary k + 1/2 for k < lim */
      const uint32_t mb = f_bits(((float)k + 0.5f) * d);  /* exact */
      for (int du = -40; du <= 40; ++du) {
        vs[nv++] = bits_f(mb + du);
        vs[nv++] = -bits_f(mb + du);
      }
    }
    for (int j = 0; j < nv; ++j) {
      const float v = vs[j];
      if (!isfinite(v) || fabsf(v / d) > lim + 0.49f) continue;
      const float t = fmaf(v, y, magic);
      const float f = fmaf(v, y, -(t - magic));
      if (fabsf(f) > thr) { ++flg; continue; }
      const int fast = (int)(t - magic);
      const int exact = (int)roundf(v / d);
      if (fast != exact || ((f_bits(t) - (uint32_t)(exact + (int)bias)) & 0xFFu) != 0u) ++bad;
    }
  }
  if (flagged) *flagged = flg;
  return bad;
}

/* The device's two-sided magic-number quantizer (m2r_device.h,
 * two_sided_code): with y = RN(1/d), y_hi = RN(y + y rel), y_lo = RN(y - y rel)
 * and magic = 1.5 2^23 + bias, the codes t_hi = RN(v y_hi + magic) and
 * t_lo = RN(v y_lo + magic) are kept when equal; then t - magic must equal
 * roundf(v / d) with IEEE division, and the low byte of t the biased code.
 * Same case mix as orc_check_residual_round: random quotients in
 * (-lim - 1/2, lim + 1/2) over binary16 and binary32 divisors, and for every
 * boundary scale the values k + 1/2 (times d, exact) and +-40 ulps around
 * them.  Returns the number of kept codes that differ; *flagged counts the
 * cases sent to the exact path. */
int64_t orc_check_two_sided_round(uint64_t seed, int64_t n_random, int n_boundary_scales, float rel,
                                  int64_t* flagged) {
  int64_t bad = 0, flg = 0;
#pragma omp parallel for reduction(+ : bad, flg) schedule(static)
  for (int64_t i = 0; i < n_random + (int64_t)n_boundary_scales; ++i) {
    uint64_t z = seed + (uint64_t)i * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    const int li = (int)((z >> 3) % 3);
    const float lim = li == 0 ? 127.0f : (li == 1 ? 7.0f : 3.0f);
    const float bias = li == 0 ? 128.0f : (li == 1 ? 8.0f : 4.0f);
    float d;
    if (z & 1) d = orc_f16_to_f32((uint16_t)(0x0400 + (uint16_t)((z >> 8) % (0x7BFF - 0x0400 + 1))));
    else d = bits_f((uint32_t)(0x32800000u + ((z >> 8) % (0x7F000000u - 0x32800000u))));
    const float y = 1.0f / d;
    const float yh = fmaf(y, rel, y), yl = fmaf(y, -rel, y);
    const float magic = 0x1.8p23f + bias;
    float vs[2 * 81 * 2 + 1];
    int nv = 0;
    if (i < n_random) {
      const float u = (bits_f((uint32_t)(0x3F800000u | ((z >> 20) & 0x7FFFFFu))) - 1.5f) * 2.0f * (lim + 0.49f);
      vs[nv++] = u * d;
    } else {
      const int k = (int)((z >> 40) % (uint64_t)lim);     /* boundary k + 1/2 for k < lim */
      const uint32_t mb = f_bits(((float)k + 0.5f) * d);  /* exact */
      for (int du = -40; du <= 40; ++du) {
        vs[nv++] = bits_f(mb + du);
        vs[nv++] = -bits_f(mb + du);
      }
    }
    for (int j = 0; j < nv; ++j) {
      const float v = vs[j];
      if (!isfinite(v) || fabsf(v / d) > lim + 0.49f) continue;
      const float th = fmaf(v, yh, magic), tl = fmaf(v, yl, magic);
      if (th != tl) { ++flg; continue; }
      const int fast = (int)(th - magic);
      const int exact = (int)roundf(v / d);
      if (fast != exact || ((f_bits(th) - (uint32_t)(exact + (int)bias)) & 0xFFu) != 0u) ++bad;
    }
  }
  if (flagged) *flagged = flg;
  return bad;
}
