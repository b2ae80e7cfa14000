// Device-side arithmetic primitives for the MI355X (gfx950) state codec and
// FP4 weight decode.  Every function here is exact in the sense stated in its
// comment: it returns bit-for-bit the value the reference semantics define
// (IEEE-754 binary32 round-to-nearest-even operations, C `roundf`, binary16
// and E4M3FN round-to-nearest-even conversions), using cheaper gfx950
// instruction sequences where a proof of equality exists.
//
// Build requirement: the translation units including this header are compiled
// with -ffp-contract=off, so `a * b + c` is two rounded operations.  Fused
// multiply-adds are only ever written explicitly (__builtin_fmaf), and only in
// places where the fusion is part of an exactness argument or where the value
// only feeds the tolerance-checked readout y.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace m2r {

// ---------------------------------------------------------------------------
// binary16 <-> binary32.  v_cvt_f16_f32 rounds to nearest even (MODE default)
// and keeps binary16 subnormals; v_cvt_f32_f16 is exact.
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float x) {
  return __builtin_bit_cast(uint16_t, (_Float16)x);
}
// float(half(x)): the stored-scale rounding of a float denominator.
__device__ __forceinline__ float round_to_half(float x) {
  return (float)(_Float16)x;
}

// ---------------------------------------------------------------------------
// E4M3FN (OCP FP8, bias 7, no infinities, 0x7F/0xFF NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  // both forms computed and selected: subnormal m * 2^-9 (exact) or normal
  const float sub = (float)m * 0x1p-9f;
  const float nrm = __builtin_bit_cast(float, ((e + 120u) << 23) | (m << 20));
  float mag = (e == 0) ? sub : nrm;
  mag = ((b & 0x7Fu) == 0x7Fu) ? __builtin_nanf("") : mag;
  return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, mag) | sign);
}

// Round-to-nearest-even binary32 -> E4M3FN for |x| <= 448 (callers clamp
// first, as the reference does).  NaN maps to 0x7F with the input's sign.
// Both magnitude paths are computed and selected (no divergent branches).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  // below 2^-6: multiples of 2^-9; scaling by 512 is exact, rint is RNE, and
  // a carry to 8 is exactly the code of 2^-6
  const float sub = __builtin_rintf(__builtin_fminf(__builtin_bit_cast(float, a), 0x1p-6f) * 512.0f);
  const uint32_t cs = (uint32_t)sub;
  const uint32_t r = (a + 0x7FFFFu + ((a >> 20) & 1u)) & ~0xFFFFFu;   // RNE at 3 mantissa bits
  const uint32_t cn = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
  uint32_t code = (a < 0x3C800000u) ? cs : cn;
  code = (a > 0x7F800000u) ? 0x7Fu : code;
  return sign | code;
}

// The same conversions by gfx950's FP8 instructions, which use the OCP
// E4M3FN format and round to nearest even.  Decoding byte SEL of w: the
// hardware returns a negative quiet NaN for both NaN codes, so the sign is
// taken from the code's own bit 7 (0x7F then decodes to the positive NaN, as
// e4m3_to_f32 gives); every other code decodes to the same bits.  Encoding a
// pair: defined for non-NaN |x| <= 448 (callers clamp first), where it equals
// f32_to_e4m3 bit for bit; byte 0 of the result holds a, byte 1 b.  Both
// identities are checked on the GPU (every code; encode over a dense sweep of
// [-448, 448]).
template <int SEL>
__device__ __forceinline__ float e4m3_byte_to_f32(uint32_t w) {
  const uint32_t f = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_f32_fp8((int)w, SEL));
  const uint32_t sign = (w << (24 - 8 * SEL)) & 0x80000000u;
  return __builtin_bit_cast(float, (f & 0x7FFFFFFFu) | sign);
}
__device__ __forceinline__ uint32_t f32x2_to_e4m3(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}

// z / ls for the latent byte, in reciprocal form (y = RN(1/ls)).  z is first
// clamped to +-464*ls (exact: 464 has 5 significant bits, ls 11), beyond which
// both this and IEEE division clamp to +-448 downstream; the sign of z is then
// restored so signed zeros and underflowed quotients keep the IEEE sign.  The
// E4M3 byte of clamp(result, +-448) equals that of IEEE z / ls for every
// finite z and binary16 ls > 0 (exhaustive over ls in the CPU checks).
__device__ __forceinline__ float latent_quotient(float z, float ls, float y) {
  const float top = 464.0f * ls;
  const float c = __builtin_fminf(__builtin_fmaxf(z, -top), top);
  const float q0 = c * y;
  const float r = __builtin_fmaf(-q0, ls, c);
  return __builtin_copysignf(__builtin_fmaf(r, y, q0), z);
}

// RN(1/s) for a positive finite binary16 value s (held in binary32): the
// hardware reciprocal estimate plus one Newton step, y0 + y0 (1 - s y0).  With
// an estimate within 2^-22 relative, the pre-rounding error is below 2^-44
// relative, while 1/s for an 11-bit significand lies at least 2^-12 ulp from
// every rounding midpoint, so the final fma rounds to RN(1/s).  The parity
// tests check all 31743 positive finite binary16 values.  Not valid for
// general binary32 s.
__device__ __forceinline__ float recip_half(float s) {
  const float y0 = __builtin_amdgcn_rcpf(s);
  const float e = __builtin_fmaf(-s, y0, 1.0f);
  return __builtin_fmaf(e, y0, y0);
}

// ---------------------------------------------------------------------------
// C roundf (half away from zero) for every binary32 input:
// trunc(x + copysign(pred(0.5), x)).  The exhaustive CPU check of this
// identity lives with the parity tests.
__device__ __forceinline__ float round_half_away(float x) {
  return __builtin_truncf(x + __builtin_copysignf(0x1.fffffep-2f, x));
}

// Correctly rounded a/d given y = RN(1/d) (Markstein's theorem: y within half
// an ulp of 1/d and q0 within one ulp of a/d => RN(q0 + RN(a - d*q0)*y) is
// RN(a/d)).  The residual fma is exact.  y == 0 with d == 1 yields 0, which
// the stored-scale quantizer uses for the zero-scale case.
__device__ __forceinline__ float div_by_recip(float a, float d, float y) {
  float q0 = a * y;
  float r = __builtin_fmaf(-q0, d, a);
  return __builtin_fmaf(r, y, q0);
}

// The requantization denominator max(amax / lim, 1e-8) for amax >= 0 (a
// maximum of absolute values, never NaN), with y = RN(1 / lim): the
// reciprocal form is RN(amax / lim) for finite amax; an infinite amax gives
// an infinite den, as IEEE division does (the reciprocal form's residual
// would be NaN there).
__device__ __forceinline__ float requant_den(float amax, float lim, float y) {
  const float den = __builtin_fmaxf(div_by_recip(amax, lim, y), 1e-8f);
  return amax == __builtin_inff() ? amax : den;
}

// roundf(RN(v/d)) as an integer, with y = RN(1/d), for quotients that need
// no clamping (|RN(v/d)| < lim + 1/2).
__device__ __forceinline__ int quantize_code_unclamped(float v, float d, float y) {
  const float q = div_by_recip(v, d, y);
  return (int)(q + __builtin_copysignf(0x1.fffffep-2f, q));
}

// clamp(roundf(RN(v/d)), -lim, lim) as an integer, with y = RN(1/d) and
// top = the largest binary32 below lim + 1.  roundf(q) is trunc(q + copysign(
// pred(0.5), q)); clamping that sum to +-top before the truncating integer
// conversion equals clamping the rounded value to +-lim.
// (An infinite v with a finite divisor gives NaN here, where IEEE division
// gives an infinity: the state kernels never divide an infinite update by a
// finite scale, since that update's maximum makes the scale infinite.)
__device__ __forceinline__ int quantize_code(float v, float d, float y, float top) {
  const float q = div_by_recip(v, d, y);
  const float t = q + __builtin_copysignf(0x1.fffffep-2f, q);
  return (int)__builtin_fminf(__builtin_fmaxf(t, -top), top);
}
constexpr float QTOP127 = 0x1.fffffep+6f;   // below 128
constexpr float QTOP7 = 0x1.fffffep+2f;     // below 8
constexpr float QTOP3 = 0x1.fffffep+1f;     // below 4

// Biased code by the magic-number rounding, for a quotient that needs no
// clamping: t = RN(v y + 1.5 2^23 + bias) lies in [2^23, 2^24), where the
// spacing is 1, so t = 1.5 2^23 + bias + rint(v y) (one rounding of the exact
// product) and the low bits of t are the code plus its bias.  rint(v y) is
// roundf(RN(v / d)) unless v / d lies near a half-integer.
//
// Two-sided form: with y = RN(1/d) for a positive normal binary32 d,
// yh = RN(y + y 2^-22) and yl = RN(y - y 2^-22), the
// biased codes th = RN(v yh + magic) and tl = RN(v yl + magic) (each one
// rounding of an exact product plus magic, as above) bracket roundf(RN(v/d)):
//   v yh >= (v/d) (1 - 2^-24)^2 (1 + 2^-22) > (v/d)(1 + 2^-24) >= RN(v/d)
// for v > 0 (mirrored for v < 0, and v yl below RN(v/d) alike), so RN(v/d)
// lies strictly between v yl and v yh.  When th == tl == magic + k, both
// products lie within 1/2 of k, hence |RN(v/d) - k| < 1/2 and roundf gives
// k: the code is kept.  Otherwise a half-integer lies between them (or on an
// end) and the tier is requantized with the exact quotients.  Per coordinate
// two fmas and one bitwise accumulation of th ^ tl, against three
// instructions and half a maximum for a residual test (f = RN(v y - (t -
// magic)) against a bound).  The CPU checks verify it on random quotients and
// every half-integer boundary, and that an offset of 0 or 2^-25 is not
// enough.
constexpr float TWO_SIDED_REL = 0x1p-22f;
__device__ __forceinline__ uint32_t two_sided_code(float v, float yh, float yl, float bias, uint32_t& diff) {
  const float magic = 0x1.8p23f + bias;
  const uint32_t th = __builtin_bit_cast(uint32_t, __builtin_fmaf(v, yh, magic));
  const uint32_t tl = __builtin_bit_cast(uint32_t, __builtin_fmaf(v, yl, magic));
  diff |= th ^ tl;
  return th;
}

// q * s exactly, for a code q held as binary16 (an integer of at most 11
// bits) and any binary32 s: one mixed-precision fma with a -0 addend (x + -0
// is x, also for signed zeros), so infinite and NaN scales give the IEEE
// product as well.  `mz` is -0.0 passed through an empty asm by the caller
// (a known -0 addend is folded into a plain product, which has no
// mixed-precision form).
__device__ __forceinline__ float dequant_h(_Float16 q, float s, float mz) {
  return __builtin_fmaf((float)q, s, mz);
}
__device__ __forceinline__ float opaque_neg_zero() {
  float mz = -0.0f;
  asm volatile("" : "+s"(mz));
  return mz;
}
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Packed binary16 a + b kept as one packed add (the empty asm stops the
// compiler from splitting it into two half-word adds).
__device__ __forceinline__ f16x2 pk_add_h(f16x2 a, f16x2 b) {
  uint32_t r = __builtin_bit_cast(uint32_t, a + b);
  asm volatile("" : "+v"(r));
  return __builtin_bit_cast(f16x2, r);
}

// The recurrent update of every codec: fma(state, decay, input) with
// input = RN(RN(b * dt) * x) rounded separately, i.e. the reference's
// `state * decay + (b * dt) * x` as Triton's floating-point fusion contracts
// it (one rounding of state * decay + input).
__device__ __forceinline__ float state_update(float state, float decay, float input) {
  return __builtin_fmaf(state, decay, input);
}

// ---------------------------------------------------------------------------
// Transcendentals.  The codec defines exp/log of a binary32 argument as the
// binary32 rounding of a fixed binary64 evaluation that uses only IEEE
// add/sub/mul/fma/div, so the host oracle and the device compute identical
// bits.  Range reduction: x = k*ln2 + r, |r| <= ln2/2, exp(r) by a degree-13
// Taylor polynomial (relative truncation error < 2^-58).  Log: x = m*2^e with
// m in [sqrt(1/2), sqrt(2)), log(m) = 2*atanh(s), s = (m-1)/(m+1), series to
// s^23.  Constants are the binary64 roundings of the named values.
//
// The binary64 constants of both recipes, by index (name, value).
#define M2R_TRANS_CONSTS(X)                                                    \
  X(KC_EXP_BIG, 100.0)                                                         \
  X(KC_EXP_TINY, 110.0)                                                        \
  X(KC_INV_LN2, 1.4426950408889634)              /* 1/ln2 */                   \
  X(KC_LN2_HI, 6.93147180369123816490e-01)       /* high 32 bits of ln2 */     \
  X(KC_LN2_LO, 1.90821492927058770002e-10)       /* ln2 - ln2_hi */            \
  X(KC_MAGIC, 6755399441055744.0)                /* 1.5 * 2^52 */              \
  X(KC_E13, 1.0 / 6227020800.0)                                                \
  X(KC_E12, 1.0 / 479001600.0)                                                 \
  X(KC_E11, 1.0 / 39916800.0)                                                  \
  X(KC_E10, 1.0 / 3628800.0)                                                   \
  X(KC_E9, 1.0 / 362880.0)                                                     \
  X(KC_E8, 1.0 / 40320.0)                                                      \
  X(KC_E7, 1.0 / 5040.0)                                                       \
  X(KC_E6, 1.0 / 720.0)                                                        \
  X(KC_E5, 1.0 / 120.0)                                                        \
  X(KC_E4, 1.0 / 24.0)                                                         \
  X(KC_E3, 1.0 / 6.0)                                                          \
  X(KC_SQRT2, 1.4142135623730951)                                              \
  X(KC_L23, 1.0 / 23.0)                                                        \
  X(KC_L21, 1.0 / 21.0)                                                        \
  X(KC_L19, 1.0 / 19.0)                                                        \
  X(KC_L17, 1.0 / 17.0)                                                        \
  X(KC_L15, 1.0 / 15.0)                                                        \
  X(KC_L13, 1.0 / 13.0)                                                        \
  X(KC_L11, 1.0 / 11.0)                                                        \
  X(KC_L9, 1.0 / 9.0)                                                          \
  X(KC_L7, 1.0 / 7.0)                                                          \
  X(KC_L5, 1.0 / 5.0)                                                          \
  X(KC_L3, 1.0 / 3.0)
#define M2R_KC_NAME(n, v) n,
#define M2R_KC_VALUE(n, v) v,
enum TransConst { M2R_TRANS_CONSTS(M2R_KC_NAME) KC_COUNT };
constexpr double kTransValue[KC_COUNT] = {M2R_TRANS_CONSTS(M2R_KC_VALUE)};
#undef M2R_KC_NAME
#undef M2R_KC_VALUE

// How a recipe's binary64 constant is materialized (the value is the same):
//  - KM_ASM: an immediate passed through an empty volatile asm, so the
//    compiler can no longer hoist its materialization out of loops (keeping
//    ~20 such constants in registers for a whole kernel); VREG materializes
//    it in vector registers instead of scalar ones (for code whose scalar
//    issue is the bottleneck);
//  - KM_PLAIN: a plain immediate, for code that evaluates the recipes once
//    (one token per launch): the compiler then materializes each constant
//    once, shares it between the two exponentials and needs no copies.
template <bool VREG = false>
__device__ __forceinline__ double kconst(double v) {
  if constexpr (VREG) asm volatile("" : "+v"(v));
  else asm volatile("" : "+s"(v));
  return v;
}
enum { KM_ASM = 0, KM_PLAIN = 1 };
template <bool VREG, int KM>
__device__ __forceinline__ double kc(TransConst i) {
  if constexpr (KM == KM_PLAIN) return kTransValue[i];
  else return kconst<VREG>(kTransValue[i]);
}

// VREG: branch-free, the out-of-range cases selected at the end (the
// polynomial then runs on an in-range stand-in argument); otherwise early
// returns.  Both give the same bits.
template <bool VREG = false, int KM = 0>
__device__ __forceinline__ double xexp_d(double x) {
  if constexpr (!VREG) {
    if (x > kc<VREG, KM>(KC_EXP_BIG)) return __builtin_inf();
    if (x < -kc<VREG, KM>(KC_EXP_TINY)) return 0.0;
  }
  const bool big = VREG && x > kc<VREG, KM>(KC_EXP_BIG), tiny = VREG && x < -kc<VREG, KM>(KC_EXP_TINY);
  const double xr = (big || tiny) ? 0.0 : x;
  const double magic = kc<VREG, KM>(KC_MAGIC);
  double kd = (xr * kc<VREG, KM>(KC_INV_LN2) + magic) - magic;   // rint(x/ln2)
  double r = (xr - kd * kc<VREG, KM>(KC_LN2_HI)) - kd * kc<VREG, KM>(KC_LN2_LO);
  double p = kc<VREG, KM>(KC_E13);                                 // 1/13!
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E12));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E11));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E10));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E9));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E8));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E7));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E6));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E5));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E4));
  p = __builtin_fma(p, r, kc<VREG, KM>(KC_E3));
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  int64_t k = (int64_t)kd;
  double scale = __builtin_bit_cast(double, (uint64_t)(k + 1023) << 52);
  const double y = p * scale;
  return big ? __builtin_inf() : (tiny ? 0.0 : y);
}

template <bool VREG = false, int KM = 0>
__device__ __forceinline__ double xlog_d(double x) {
  // Domain used by the codec: finite x >= 1 (softplus argument exp(d)+1).
  uint64_t u = __builtin_bit_cast(uint64_t, x);
  int64_t e = (int64_t)((u >> 52) & 0x7FF) - 1023;
  double m = __builtin_bit_cast(double, (u & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
  if constexpr (VREG) {
    const bool upper = m > kc<VREG, KM>(KC_SQRT2);
    m = upper ? m * 0.5 : m;
    e += upper ? 1 : 0;
  } else if (m > kc<VREG, KM>(KC_SQRT2)) {
    m = m * 0.5;
    e += 1;
  }
  double s = (m - 1.0) / (m + 1.0);
  double s2 = s * s;
  double p = kc<VREG, KM>(KC_L23);
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L21));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L19));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L17));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L15));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L13));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L11));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L9));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L7));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L5));
  p = __builtin_fma(p, s2, kc<VREG, KM>(KC_L3));
  p = __builtin_fma(p, s2, 1.0);
  double logm = 2.0 * s * p;
  double ed = (double)e;
  const double ln2_hi = kc<VREG, KM>(KC_LN2_HI);
  const double ln2_lo = kc<VREG, KM>(KC_LN2_LO);
  return (ed * ln2_hi + logm) + ed * ln2_lo;
}

template <bool VREG = false, int KM = 0>
__device__ __forceinline__ float xexpf(float x) {
  return (float)xexp_d<VREG, KM>((double)x);
}
template <bool VREG = false, int KM = 0>
__device__ __forceinline__ float xlogf(float x) {
  return (float)xlog_d<VREG, KM>((double)x);
}

// Mamba-2 dt activation of the codec kernels: v = dt + dt_bias;
// v <= 20 ? log(exp(v) + 1) : v, with the inner +1 rounded in binary32
// (VREG: branch-free, arguments above 20, and NaN, select v itself).
template <bool VREG = false, int KM = 0>
__device__ __forceinline__ float softplus_dt(float v) {
  if constexpr (!VREG) {
    if (v <= 20.0f) return xlogf<VREG, KM>(xexpf<VREG, KM>(v) + 1.0f);
    return v;
  }
  const bool soft = v <= 20.0f;
  const float e = xexpf<VREG, KM>(soft ? v : 0.0f);
  const float l = xlogf<VREG, KM>(e + 1.0f);
  return soft ? l : v;
}

// dt activation and decay for one head (inline; its binary64 constants are
// rematerialized at each use, see kconst).
template <bool VREG = false, int KM = 0>
__device__ __forceinline__ float2 dt_activation(float dt_plus_bias, float A) {
  const float dtv = softplus_dt<VREG, KM>(dt_plus_bias);
  return make_float2(dtv, xexpf<VREG, KM>(A * dtv));
}

}  // namespace m2r
