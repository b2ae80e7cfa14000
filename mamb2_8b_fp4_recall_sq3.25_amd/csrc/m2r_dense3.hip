// Dense 3-bit state step (all 128 coordinates as 3-bit codes in three bit
// planes + two FP16 half-row scales) and the diagnostic packed-state decode /
// legacy encode, for gfx950 (the FP16-carry control scan is m2r_s16.hip).
//
//   dense3  mamba2_recall/state_codec_dense3.py:82-148 (_scan)
//   decode  mamba2_recall/state_codec.py:269-296, state_codec_dense3.py:189-212,
//           scripts/w4_state_repair_codec_v2.py:141-162
//   encode  mamba2_recall/state_codec.py:299-331 (encode_state_)
//
// The dense3 kernel follows the packed-row kernel's structure: one lane per
// row, the carry held between tokens as biased code bytes (q + 4), rows staged
// through LDS, per-token B/C table gather and B*dt computed once per
// workgroup.  Quantization uses the binary32 denominator
// max(RN(amax_half / 3), 1e-8) through the exact reciprocal-form quotient.
#include "m2r_device.h"
#include "m2r_abi_util.h"
#include "m2r_tile.h"

#include <type_traits>

namespace m2r {

struct Dense3Args {
  const uint16_t* x; const uint16_t* dt; const float* A; const uint16_t* Bm; const uint16_t* Cm;
  const void* D; const void* dt_bias; const void* table;
  uint8_t* codes;      // u8 [rows, 3, 16]
  uint16_t* scales;    // f16 [rows, 2]
  uint16_t* y;
  int B, L, H, P, G;
  int d_f32, db_f32, equalizer;
};

template <int WPB>
__global__ __launch_bounds__(64 * WPB) void k_dense3_step(Dense3Args a) {
  constexpr int NT = 64 * WPB;
  constexpr int W = 48;
  __shared__ __align__(16) uint8_t s_tile[WPB][64 * W + 16];
  __shared__ __align__(16) float s_c[128];
  __shared__ __align__(16) float s_b[128];
  __shared__ __align__(16) float s_bdt[WPB][128];
  __shared__ float s_dtv[WPB], s_decay[WPB];
  __shared__ int s_pos[128];
  __shared__ float s_wf[128], s_rf[128];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.z, h0 = blockIdx.y * WPB, h = h0 + wave;
  const int H = a.H, P = a.P, G = a.G, L = a.L;
  const int g = h0 / (H / G);
  const int pbase = blockIdx.x * 64;
  const int nvalid = min(64, P - pbase);
  const bool valid = lane < nvalid;
  const int row0 = (b * H + h) * P + pbase, row = row0 + lane;

  for (int n = tid; n < 128; n += NT) {
    if (a.equalizer) {
      int k = ((const int8_t*)a.table)[g * 128 + n];
      s_pos[n] = n;
      s_wf[n] = __builtin_ldexpf(1.0f, -k);   // exp2(-k), exact
      s_rf[n] = __builtin_ldexpf(1.0f, k);
    } else {
      s_pos[n] = ((const uint8_t*)a.table)[g * 128 + n] & 127;   // in-bounds for any table
    }
  }
  const float Dh = load_param(a.D, a.d_f32, h);
  uint8_t* tile = s_tile[wave];
  wave_copy_in<W>(tile, a.codes, row0, nvalid, lane);
  float sc0 = 0.f, sc1 = 0.f;
  if (valid) {
    uint32_t sw = ((const uint32_t*)a.scales)[row];
    sc0 = h2f((uint16_t)(sw & 0xFFFFu));
    sc1 = h2f((uint16_t)(sw >> 16));
  }
  __syncthreads();

  // carry: byte k of c[i] = q[4i+k] + 4 (== 3-bit code ^ 4).  Coordinate n
  // is bit n % 32 of word 4j + n / 32 of plane j.  Four bits of a plane
  // spread to bit 0 of four bytes as (nibble * 0x204081) & 0x01010101 (the
  // partial products land on distinct bits, so nothing carries); the bias
  // flips bit 2, i.e. plane 2 is read inverted.
  uint32_t c[32];
  {
    uint32_t w[12];
    lds_read_row<W>(tile, lane * W, w);
#pragma unroll
    for (int j = 8; j < 12; ++j) w[j] = ~w[j];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int wi = i >> 3, sh = 4 * (i & 7);
      const uint32_t s0 = __umul24(__builtin_amdgcn_ubfe(w[wi], sh, 4), 0x204081u) & 0x01010101u;
      const uint32_t s1 = __umul24(__builtin_amdgcn_ubfe(w[4 + wi], sh, 4), 0x204081u) & 0x01010101u;
      const uint32_t s2 = __umul24(__builtin_amdgcn_ubfe(w[8 + wi], sh, 4), 0x204081u) & 0x01010101u;
      c[i] = valid ? (s0 | (s1 << 1) | (s2 << 2)) : 0x04040404u;
    }
  }
  const float y3 = 1.0f / 3.0f;

  for (int t = 0; t < L; ++t) {
    const int bt = b * L + t;
    for (int n = tid; n < 128; n += NT) {
      int pos = s_pos[n];
      float bv = h2f(a.Bm[((size_t)bt * G + g) * 128 + pos]);
      float cv = h2f(a.Cm[((size_t)bt * G + g) * 128 + pos]);
      if (a.equalizer) { bv = bv * s_wf[n]; cv = cv * s_rf[n]; }
      s_b[n] = bv;
      s_c[n] = cv;
    }
    if (tid < WPB) {
      int hh = h0 + tid;
      float v = h2f(a.dt[(size_t)bt * H + hh]) + load_param(a.dt_bias, a.db_f32, hh);
      const float2 act = dt_activation(v, a.A[hh]);
      s_dtv[tid] = act.x;
      s_decay[tid] = act.y;
    }
    __syncthreads();
    for (int i = tid; i < WPB * 128; i += NT) {
      int w = i >> 7, n = i & 127;
      s_bdt[w][n] = s_b[n] * s_dtv[w];
    }
    __syncthreads();

    const float decay = s_decay[wave];
    const float x = valid ? h2f(a.x[((size_t)bt * H + h) * P + pbase + lane]) : 0.f;
    float acc = 0.f, amax0 = 0.f, amax1 = 0.f;
    float v[128];
    const f32x4* bdt4 = (const f32x4*)s_bdt[wave];
    const f32x4* c4v = (const f32x4*)s_c;
#pragma unroll
    for (int i0 = 0; i0 < 128; i0 += 4) {
      const f32x4 cb = bdt4[i0 / 4], cc = c4v[i0 / 4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = i0 + j;
        // q * s as the exact product (also for infinite or NaN scales)
        float prior = (ubyte_f(c[i / 4], j) - 4.0f) * ((i < 64) ? sc0 : sc1);
        float u = state_update(prior, decay, cb[j] * x);
        v[i] = u;
        acc = __builtin_fmaf(u, cc[j], acc);
        if (i < 64) amax0 = __builtin_fmaxf(amax0, __builtin_fabsf(u));
        else amax1 = __builtin_fmaxf(amax1, __builtin_fabsf(u));
      }
    }
    asm volatile("" : "+v"(acc));
    float out = acc + x * Dh;
    if (valid) a.y[((size_t)bt * H + h) * P + pbase + lane] = f2h(out);

    const float den0 = requant_den(amax0, 3.0f, y3);
    const float den1 = requant_den(amax1, 3.0f, y3);
    sc0 = round_to_half(den0);
    sc1 = round_to_half(den1);
    // an infinite den divides through d = 1, y = 0 (RN(v / inf) = 0 for finite v)
    const bool inf0 = den0 == __builtin_inff(), inf1 = den1 == __builtin_inff();
    const float d0 = inf0 ? 1.0f : den0, d1 = inf1 ? 1.0f : den1;
    const float r0 = inf0 ? 0.0f : 1.0f / den0, r1 = inf1 ? 0.0f : 1.0f / den1;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float d = (i < 16) ? d0 : d1, r = (i < 16) ? r0 : r1;
      int q0 = quantize_code(v[4 * i], d, r, QTOP3);
      int q1 = quantize_code(v[4 * i + 1], d, r, QTOP3);
      int q2 = quantize_code(v[4 * i + 2], d, r, QTOP3);
      int q3 = quantize_code(v[4 * i + 3], d, r, QTOP3);
      c[i] = (pack4(q0, q1, q2, q3) & 0x07070707u) ^ 0x04040404u;   // (q & 7) ^ 4 == q + 4
    }
    __syncthreads();
  }

  // planes: byte j of plane k holds bit k of (q & 7) for lanes 8j..8j+7.
  // For 8 coordinates (two code words a, b), plane k's bits sit at bit k of
  // each byte; (a & m) | (b & m) << 4 with m = 0x01010101 << k, times
  // 0x01020408 >> k, leaves the 8 bits in the top byte (distinct partial
  // products, no carries).  Bit 2 is read inverted (the bias).
  if (valid) {
    uint32_t w[12];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const uint32_t m = 0x01010101u << k, mul = 0x01020408u >> k;
      uint32_t top[16];
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const uint32_t ca = k == 2 ? ~c[2 * t] : c[2 * t], cb = k == 2 ? ~c[2 * t + 1] : c[2 * t + 1];
        top[t] = ((ca & m) | ((cb & m) << 4)) * mul;
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {   // top bytes of products 4q .. 4q+3 -> plane word q
        const uint32_t lo = __builtin_amdgcn_perm(top[4 * q + 1], top[4 * q], 0x0c0c0703u);
        const uint32_t hi = __builtin_amdgcn_perm(top[4 * q + 3], top[4 * q + 2], 0x07030c0cu);
        w[4 * k + q] = lo | hi;
      }
    }
    lds_write_row<W>(tile, lane * W, w);
  }
  __syncthreads();
  wave_copy_out<W>(a.codes, tile, row0, nvalid, lane);
  if (valid) ((uint32_t*)a.scales)[row] = (uint32_t)f2h(sc0) | ((uint32_t)f2h(sc1) << 16);
}

// ---------------------------------------------------------------------------
// Streaming dense 3-bit step: the packed-row kernel's structure applied to
// the three-plane format.  One lane owns one row; a wave owns HPW head slots
// of 64 rows (the same P block of HPW heads); a workgroup owns NH = WPB * HPW
// heads of one B/C group and one batch row.  Every slot's packed rows stay in
// LDS for all L tokens; the first token streams them in (slot k + 1 is
// fetched while slot k computes) and the last streams them out.  Each wave
// builds the per-token values it reads itself (no workgroup barrier).
//
// Internal coordinate order.  Position i = 32 wi + 8 j + 4 h + m (wi, m in
// 0..3, j in 0..3, h in 0..1) holds coordinate n = 32 wi + 8 m + 4 h + j, i.e.
// bit b = 8 m + 4 h + j of plane word wi.  A word X_j whose byte m holds the
// code of (m, h = 0, j) in bits 0..2 and that of (m, 1, j) in bits 4..6 is
// then a rotation away from every plane: with M_k = 0x11111111 << k,
//   plane_k = rotr(OR_j (rotl(X_j, j) & rotl(M_k, j)), k)
// (the four masked terms occupy disjoint bits, and rotation distributes over
// OR), and, the other way round, X_j = rotr(OR_k (rotl(plane_k, k) &
// rotl(M_k, j)), j).  Both directions take about one and a half bit
// operations per coordinate; neither needs a multiply.

// internal position i -> coordinate n
__host__ __device__ constexpr int d3_coord(int i) { return (i & ~31) | ((i & 3) << 3) | (i & 4) | ((i >> 3) & 3); }

constexpr uint32_t rotl32(uint32_t x, int n) { return n == 0 ? x : (x << n) | (x >> (32 - n)); }
// rotl(M_k, j)
constexpr uint32_t d3_mask(int k, int j) { return rotl32(0x11111111u << k, j); }

__device__ __forceinline__ uint32_t rotl_dev(uint32_t x, int n) {
  return n == 0 ? x : __builtin_amdgcn_alignbit(x, x, 32 - n);
}
__device__ __forceinline__ uint32_t rotr_dev(uint32_t x, int n) {
  return n == 0 ? x : __builtin_amdgcn_alignbit(x, x, n);
}

// Per-token values of one wave (its own LDS region; only its lanes read them).
template <int HPW>
struct D3Token {
  alignas(16) float c[128];          // C (times the equalizer's 2^k), internal order
  alignas(16) float bdt[HPW][128];   // RN(RN(B 2^-k) * dt) per head slot, internal order
  uint16_t x[HPW][64];               // x of the wave's rows, per head slot
  float dtv[HPW], decay[HPW], D[HPW];
  // per head slot: 1 when B*dt and the decay are bounded so that the update
  // of finite operands is finite
  uint32_t bounded[HPW];
  float sbc;                         // sum of b * c over the 128 coordinates (readout)
};

// Inputs of one token a wave loads (one token ahead in the multi-token
// instance): its lane's pairs of the group's B and C rows, x of its rows in
// every head slot and, for lanes < HPW, dt and dt_bias of head slot `lane`.
template <int HPW>
struct D3Raw {
  uint32_t bp, cp;
  uint16_t xv[HPW];
  uint16_t dt, db_lo, db_hi;
};

template <int WPB, int HPW>
__device__ __forceinline__ void d3_load(const Dense3Args& a, D3Raw<HPW>& r, int bt, int g, int h0, int pbase,
                                        int lane, int wave) {
  const int hl = h0 + min(lane, HPW - 1) * WPB + wave;   // lanes >= HPW repeat the last slot
  const uint16_t* db = (const uint16_t*)a.dt_bias;
  r.dt = a.dt[(size_t)bt * a.H + hl];
  r.db_lo = db[a.db_f32 ? 2 * hl : hl];
  r.db_hi = db[a.db_f32 ? 2 * hl + 1 : hl];
  const size_t row = ((size_t)bt * a.G + g) * 128 + 2 * lane;
  r.bp = *(const uint32_t*)(a.Bm + row);
  r.cp = *(const uint32_t*)(a.Cm + row);
  const int p = min(pbase + lane, a.P - 1);   // rows past P read row P-1 (never stored)
#pragma unroll
  for (int k = 0; k < HPW; ++k) r.xv[k] = a.x[((size_t)bt * a.H + h0 + k * WPB + wave) * a.P + p];
}

template <int HPW>
__device__ __forceinline__ float2 d3_activation(const D3Raw<HPW>& r, float Ah, int db_f32) {
  const float db = db_f32 ? __builtin_bit_cast(float, (uint32_t)r.db_lo | ((uint32_t)r.db_hi << 16)) : h2f(r.db_lo);
  return dt_activation(h2f(r.dt) + db, Ah);
}

// Builds the wave's token values: lane l gathers internal positions l and
// l + 64 (raw B/C indices pv0, pv1; equalizer weights wf = 2^-k, rf = 2^k, 1
// for a permutation table) from the lanes holding them.
template <int HPW>
__device__ __forceinline__ void d3_token_build(D3Token<HPW>& wt, const D3Raw<HPW>& r, float2 act, int pv0, int pv1,
                                               float wf0, float wf1, float rf0, float rf1, int lane) {
#pragma unroll
  for (int k = 0; k < HPW; ++k) wt.x[k][lane] = r.xv[k];
  const uint32_t bw0 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv0 >> 1), (int)r.bp);
  const uint32_t bw1 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv1 >> 1), (int)r.bp);
  const uint32_t cw0 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv0 >> 1), (int)r.cp);
  const uint32_t cw1 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv1 >> 1), (int)r.cp);
  __builtin_amdgcn_sched_barrier(0);   // all four exchanges in flight before the first use
  const float b0 = h2f((uint16_t)(bw0 >> (16 * (pv0 & 1)))) * wf0;
  const float b1 = h2f((uint16_t)(bw1 >> (16 * (pv1 & 1)))) * wf1;
  const float c0 = h2f((uint16_t)(cw0 >> (16 * (pv0 & 1)))) * rf0;
  const float c1 = h2f((uint16_t)(cw1 >> (16 * (pv1 & 1)))) * rf1;
  // |b| < 2^30, |dt| < 2^60 and |decay| < 2^100 keep every update of finite
  // operands (|prior| <= 4 * 65504) below 2^120
  const bool b_lane_ok = __builtin_fabsf(b0) < 0x1p30f && __builtin_fabsf(b1) < 0x1p30f;
  const bool b_ok = __builtin_amdgcn_ballot_w64(!b_lane_ok) == 0;
  const float dtv = act.x;
  if (lane < HPW) {
    wt.dtv[lane] = act.x;
    wt.decay[lane] = act.y;
    wt.bounded[lane] = b_ok && __builtin_fabsf(act.x) < 0x1p60f && __builtin_fabsf(act.y) < 0x1p100f;
  }
  wt.c[lane] = c0;
  wt.c[64 + lane] = c1;
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const float dk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dtv), k));
    wt.bdt[k][lane] = b0 * dk;
    wt.bdt[k][64 + lane] = b1 * dk;
  }
  const float sbc = wave_sum(b0 * c0 + b1 * c1);
  if (lane == 0) wt.sbc = sbc;
  wave_sync();
}

// One half row (coordinates with n / 64 == HF, internal positions 64 HF ..
// 64 HF + 63): unpack the two plane words of each plane, dequantize with the
// stored scale, update, accumulate the readout (prior * c), requantize with
// den = max(RN(amax / 3), 1e-8) and the binary32 quotient, and repack.  `w`
// holds the row's 12 plane words (plane k word wi at 4 k + wi); the new ones
// are written to `nw` at the same positions.  Returns the new stored scale.
//
// The clamp to +-3 acts only when an update is not finite (a NaN quotient
// then clamps to -3, as fminf(fmaxf(NaN, -3), 3) does): with every update
// finite, |RN(v / den)| <= 3 / (1 - 2^-24) rounds to at most 3.  `ok` (per
// lane) says the updates are finite by construction; when it holds on every
// lane the wave takes the quantizer without the clamp.
//
// prior = q * s exactly from binary16 1024 + b (b = q + 4, low nibble) or
// 1024 + 16 b (high nibble) and s (s / 16, exact).  EXACT false (every scale
// of the wave finite): (1024 + b) s - 1028 s ((1024 + 16 b) s/16 - 1088 s/16),
// one fma (both products have at most 22 significant bits); true: the packed
// binary16 difference (q, 16 q) times s (s / 16), also the IEEE product for
// infinite and NaN scales, where the fused form gives inf - inf.
template <int HF, bool EXACT>
__device__ __forceinline__ float d3_half(const uint32_t (&w)[12], uint32_t (&nw)[12], float sc, float decay, float x,
                                         const f32x4* bdt4, const f32x4* c4, float& acc, bool ok) {
  const float so = sc * 0.0625f;
  const float nbe = -1028.0f * sc, nbo = -1088.0f * so;
  const f16x2 hbe = {(_Float16)-1028.0f, (_Float16)-1028.0f}, hbo = {(_Float16)-1088.0f, (_Float16)-1088.0f};
  const float mz = EXACT ? opaque_neg_zero() : 0.f;
  float v[64];
  float amax = 0.f;
  f32x4 cb_next = bdt4[0], cw_next = c4[0];
#pragma unroll
  for (int wl = 0; wl < 2; ++wl) {
    const int wi = 2 * HF + wl;
    const uint32_t z0 = w[wi], z1 = rotl_dev(w[4 + wi], 1), z2 = rotl_dev(~w[8 + wi], 2);   // plane 2 read inverted: b = q + 4
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t y = (z0 & d3_mask(0, j)) | (z1 & d3_mask(1, j)) | (z2 & d3_mask(2, j));
      const uint32_t xw = rotr_dev(y, j);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int i0 = 32 * wl + 8 * j + 4 * h;
        const f32x4 cb = cb_next, cw = cw_next;
        if (i0 + 4 < 64) {
          cb_next = bdt4[i0 / 4 + 1];
          cw_next = c4[i0 / 4 + 1];
        }
        const uint32_t word = h ? (xw & 0xF0F0F0F0u) : (xw & 0x0F0F0F0Fu);
        const float s = h ? so : sc, nb = h ? nbo : nbe;
        const uint32_t h01 = __builtin_amdgcn_perm(0x64646464u, word, 0x04010400u);
        const uint32_t h23 = __builtin_amdgcn_perm(0x64646464u, word, 0x04030402u);
        float pr[4];
        if constexpr (EXACT) {
          const f16x2 q01 = pk_add_h(__builtin_bit_cast(f16x2, h01), h ? hbo : hbe);
          const f16x2 q23 = pk_add_h(__builtin_bit_cast(f16x2, h23), h ? hbo : hbe);
#pragma unroll
          for (int m = 0; m < 4; ++m) pr[m] = dequant_h((m < 2 ? q01 : q23)[m & 1], s, mz);
        } else {
#pragma unroll
          for (int m = 0; m < 4; ++m)
            pr[m] = __builtin_fmaf(h2f((uint16_t)((m < 2 ? h01 : h23) >> (16 * (m & 1)))), s, nb);
        }
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float prior = pr[m];
          acc = __builtin_fmaf(prior, cw[m], acc);
          float u = state_update(prior, decay, cb[m] * x);
          asm volatile("" : "+v"(u));
          v[i0 + m] = u;
        }
        amax = max3_abs(amax, v[i0], v[i0 + 1]);
        amax = max3_abs(amax, v[i0 + 2], v[i0 + 3]);
      }
    }
  }
  asm volatile("" : "+v"(acc), "+v"(amax));
  const float den = requant_den(amax, 3.0f, 1.0f / 3.0f);
  const float stored = round_to_half(den);
  // an infinite den (an infinite update) divides through d = 1, y = 0: RN(v /
  // inf) is 0 for finite v, and the residual then stays finite
  const bool inf = den == __builtin_inff();
  const float d = inf ? 1.0f : den;
  const float r = inf ? 0.0f : 1.0f / den;
  const bool fast = __builtin_amdgcn_ballot_w64(!ok) == 0;
  // codes (two's complement bytes: bits 0..2 are the 3-bit code) into the
  // plane words; `codes4(i0)` packs the codes of internal positions i0..i0+3
  auto to_planes = [&](auto codes4) {
#pragma unroll
    for (int wl = 0; wl < 2; ++wl) {
      uint32_t z[3] = {0u, 0u, 0u};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t pk0 = codes4(32 * wl + 8 * j), pk1 = codes4(32 * wl + 8 * j + 4);
        // bits 0..2: codes of h = 0, bits 4..6: h = 1 (bits 3 and 7 are never selected)
        const uint32_t xw = (pk0 & 0x07070707u) | ((pk1 << 4) & 0xF8F8F8F8u);
        const uint32_t yw = rotl_dev(xw, j);
#pragma unroll
        for (int k = 0; k < 3; ++k) z[k] |= yw & d3_mask(k, j);
      }
#pragma unroll
      for (int k = 0; k < 3; ++k) nw[4 * k + 2 * HF + wl] = rotr_dev(z[k], k);
    }
  };
  if (fast) {
    // the code as the low bits of th = RN(v yh + 1.5 2^23) = 1.5 2^23 +
    // rint(v yh), kept where the code of the other side, RN(v yl + ...),
    // agrees (two_sided_code; r = RN(1/den) of a positive normal den here)
    const float yh = __builtin_fmaf(r, TWO_SIDED_REL, r), yl = __builtin_fmaf(r, -TWO_SIDED_REL, r);
    uint32_t diff = 0u;
    to_planes([&](int i0) {
      uint32_t tb[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        tb[m] = two_sided_code(v[i0 + m], yh, yl, 0.0f, diff);
        asm volatile("" : "+v"(diff));   // one three-input bitwise operation per coordinate
      }
      return pack4((int)tb[0], (int)tb[1], (int)tb[2], (int)tb[3]);
    });
    // a lane near a rounding boundary: the half row again with exact quotients
    if (__builtin_amdgcn_ballot_w64(diff != 0u) != 0)
      to_planes([&](int i0) {
        return pack4(quantize_code_unclamped(v[i0], d, r), quantize_code_unclamped(v[i0 + 1], d, r),
                     quantize_code_unclamped(v[i0 + 2], d, r), quantize_code_unclamped(v[i0 + 3], d, r));
      });
  } else {
    to_planes([&](int i0) {
      return pack4(quantize_code(v[i0], d, r, QTOP3), quantize_code(v[i0 + 1], d, r, QTOP3),
                   quantize_code(v[i0 + 2], d, r, QTOP3), quantize_code(v[i0 + 3], d, r, QTOP3));
    });
  }
  return stored;
}

template <int WPB, int HPW, bool ONE>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(2, 8)))
void k_dense3_slots(Dense3Args a) {
  constexpr int NH = WPB * HPW;
  constexpr int O_SC = 64 * 48;                 // scales after the 64 code rows
  constexpr int TILE = O_SC + 64 * 4 + 16;
  constexpr int SLOT_OPS = chunk_ops(48) + chunk_ops(4);   // transfers (and stores) per slot
  static_assert(TILE % 16 == 0, "tiles stay 16-byte aligned");
  static_assert(2 * SLOT_OPS + 1 <= 63, "vmcnt range");
  __shared__ __align__(16) D3Token<HPW> s_wt[WPB];
  __shared__ __align__(16) uint8_t s_tile[NH][TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.z;
  const int h0 = blockIdx.y * NH;
  const int H = a.H, P = a.P;
  const int L = ONE ? 1 : a.L;
  const int g = h0 / (H / a.G);
  const int pbase = blockIdx.x * 64;
  const int nvalid = min(64, P - pbase);
  const bool valid = lane < nvalid;
  D3Token<HPW>& wt = s_wt[wave];

  auto slot_row0 = [&](int hh) { return (b * H + h0 + hh) * P + pbase; };
  // LDS byte address of the tiles (integer offsets from it, no generic-pointer casts)
  const uint32_t tiles_lds = lds_address(&s_tile[0][0]);
  auto slot_dma = [&](int hh) {
    const int row0 = slot_row0(hh);
    const uint32_t t = tiles_lds + (uint32_t)(hh * TILE);
    field_dma16_at<48>(t, a.codes, row0, nvalid, lane);
    field_dma16_at<4>(t + O_SC, (const uint8_t*)a.scales, row0, nvalid, lane);
  };
  // before slot k is first read: only operations issued after its transfers
  // may be outstanding (slot k-2's copy-out when the first token is also the
  // last, and slot k-1's y store)
  auto slot_wait = [&](int k) {
    if (k == 0) wait_vmcnt<0>();
    else if (L == 1 && k >= 2) wait_vmcnt<SLOT_OPS + 1>();
    else wait_vmcnt<1>();
  };
  auto slot_copy_out = [&](int hh) {
    const int row0 = slot_row0(hh);
    u32x4 v[SLOT_OPS];
    field_read16<48>(s_tile[hh], lane, v);
    field_read16<4>(s_tile[hh] + O_SC, lane, v + chunk_ops(48));
    field_write16<48>(a.codes, v, row0, nvalid, lane);
    field_write16<4>((uint8_t*)a.scales, v + chunk_ops(48), row0, nvalid, lane);
  };

  // ---- prologue: register loads (dt first), the dt activation while they
  // land, then the first slot's transfer, which lands while the token is built
  D3Raw<HPW> raw;
  d3_load<WPB, HPW>(a, raw, b * L, g, h0, pbase, lane, wave);
  const int hl = h0 + min(lane, HPW - 1) * WPB + wave;
  const float Ah = a.A[hl];
  const uint32_t d_bits = a.d_f32 ? ((const uint32_t*)a.D)[hl] : (uint32_t)((const uint16_t*)a.D)[hl];
  const int n0 = d3_coord(lane);
  const uint32_t tb0 = ((const uint8_t*)a.table)[g * 128 + n0];
  const uint32_t tb1 = ((const uint8_t*)a.table)[g * 128 + n0 + 64];
  float2 act = d3_activation<HPW>(raw, Ah, a.db_f32);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): no compiler wait may cover a slot transfer
  __builtin_amdgcn_sched_barrier(0);
  slot_dma(wave);
  if (lane < HPW) wt.D[lane] = a.d_f32 ? __builtin_bit_cast(float, d_bits) : h2f((uint16_t)d_bits);
  int pv0, pv1;
  float wf0 = 1.f, wf1 = 1.f, rf0 = 1.f, rf1 = 1.f;
  if (a.equalizer) {
    const int k0 = (int)(int8_t)tb0, k1 = (int)(int8_t)tb1;
    pv0 = n0;
    pv1 = n0 + 64;
    wf0 = __builtin_ldexpf(1.0f, -k0);   // exp2(-k), exact
    wf1 = __builtin_ldexpf(1.0f, -k1);
    rf0 = __builtin_ldexpf(1.0f, k0);
    rf1 = __builtin_ldexpf(1.0f, k1);
  } else {
    pv0 = (int)(tb0 & 127);   // in-bounds for any table
    pv1 = (int)(tb1 & 127);
  }

  for (int t = 0; t < L; ++t) {
    const int bt = b * L + t;
    const D3Raw<HPW> cur = raw;
    if (t + 1 < L) d3_load<WPB, HPW>(a, raw, bt + 1, g, h0, pbase, lane, wave);
    d3_token_build<HPW>(wt, cur, act, pv0, pv1, wf0, wf1, rf0, rf1, lane);

    for (int k = 0; k < HPW; ++k) {
      int hh = k * WPB + wave;
      asm volatile("" : "+s"(hh));
      const int h = h0 + hh;
      wave_priority_by_slots_left(HPW - k);
      if (t == 0) slot_wait(k);
      uint8_t* tile = s_tile[hh];
      uint32_t w[12];
      {
        const u32x4* rp = (const u32x4*)(tile + 48 * lane);
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          const u32x4 v4 = rp[q];
          w[4 * q] = v4.x; w[4 * q + 1] = v4.y; w[4 * q + 2] = v4.z; w[4 * q + 3] = v4.w;
        }
      }
      const uint32_t sw = ((const uint32_t*)(tile + O_SC))[lane];
      float sc0 = h2f((uint16_t)(sw & 0xFFFFu)), sc1 = h2f((uint16_t)(sw >> 16));
      if (!valid) {   // rows past P: zero placeholders, never stored
#pragma unroll
        for (int q = 0; q < 12; ++q) w[q] = 0u;
        sc0 = sc1 = 0.f;
      }
      const float x = h2f(wt.x[k][lane]);
      const float decay = wt.decay[k];
      const bool base_ok = wt.bounded[k] != 0 && __builtin_fabsf(x) <= 65504.f;
      const f32x4* bdt4 = (const f32x4*)wt.bdt[k];
      const f32x4* c4 = (const f32x4*)wt.c;
      float acc = 0.f;
      uint32_t nw[12];
      const bool fin0 = __builtin_fabsf(sc0) <= 65504.f, fin1 = __builtin_fabsf(sc1) <= 65504.f;
      // one wave-uniform choice per slot between the fused dequantization
      // (every scale of the wave finite) and the exact products
      auto halves = [&](auto exact) {
        constexpr bool EX = decltype(exact)::value;
        sc0 = d3_half<0, EX>(w, nw, sc0, decay, x, bdt4, c4, acc, base_ok && fin0);
        __builtin_amdgcn_sched_barrier(0);
        if (t == 0 && k + 1 < HPW) slot_dma(hh + WPB);
        sc1 = d3_half<1, EX>(w, nw, sc1, decay, x, bdt4 + 16, c4 + 16, acc, base_ok && fin1);
        __builtin_amdgcn_sched_barrier(0);
        if (t == L - 1 && k > 0) slot_copy_out(hh - WPB);
        __builtin_amdgcn_sched_barrier(0);
      };
      if (__builtin_amdgcn_ballot_w64(!(fin0 && fin1)) == 0) halves(std::false_type{});
      else halves(std::true_type{});
      const float out = decay * acc + x * (wt.dtv[k] * wt.sbc + wt.D[k]);
      {
        const __amdgpu_buffer_rsrc_t ry = raw_buffer(a.y + ((size_t)bt * H + h) * P + pbase, 2 * nvalid);
        __builtin_amdgcn_raw_buffer_store_b16(f2h(out), ry, 2 * lane, 0, STORE_THROUGH);
      }
      if (valid) {
        u32x4* wp = (u32x4*)(tile + 48 * lane);
#pragma unroll
        for (int q = 0; q < 3; ++q) wp[q] = u32x4{nw[4 * q], nw[4 * q + 1], nw[4 * q + 2], nw[4 * q + 3]};
        ((uint32_t*)(tile + O_SC))[lane] = (uint32_t)f2h(sc0) | ((uint32_t)f2h(sc1) << 16);
      }
      wave_sync();
    }
    if (t == L - 1) slot_copy_out((HPW - 1) * WPB + wave);
    if (t + 1 < L) act = d3_activation<HPW>(raw, Ah, a.db_f32);
  }
}

// ---------------------------------------------------------------------------
// Diagnostic decode of packed rows to FP32 [rows, 128] in packed lane order:
// kind 0 = INT8/INT4 tiers (dead tier zero), kind 1 = dense 3-bit planes
// (`lo` holds the [rows, 3, 16] codes, `s8` the [rows, 2] scales).
__global__ void k_state_decode(int kind, int n8, int n4, const uint8_t* lo, const uint8_t* hi, const uint8_t* q4,
                               const uint16_t* s8, const uint16_t* s4, float* out, int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  float* o = out + r * 128;
  if (kind == 1) {
    const uint8_t* cd = lo + r * 48;
    float sc0 = h2f(s8[2 * r]), sc1 = h2f(s8[2 * r + 1]);
    for (int n = 0; n < 128; ++n) {
      int u = 0;
      for (int k = 0; k < 3; ++k) u |= ((cd[16 * k + n / 8] >> (n % 8)) & 1) << k;
      int q = u - 8 * (u >= 4);
      o[n] = (float)q * (n < 64 ? sc0 : sc1);
    }
    return;
  }
  const float a8 = h2f(s8[r]), a4 = h2f(s4[r]);
  for (int n = 0; n < n8; ++n) {
    int l = (lo[r * (n8 / 2) + n / 2] >> (4 * (n % 2))) & 15;
    int hh = (hi[r * (n8 / 2) + n / 2] >> (4 * (n % 2))) & 15;
    o[n] = (float)(int)(int8_t)(uint8_t)((hh << 4) | l) * a8;
  }
  for (int n = 0; n < n4; ++n) {
    int nib = (q4[r * (n4 / 2) + n / 2] >> (4 * (n % 2))) & 15;
    o[n8 + n] = (float)(nib - 16 * (nib > 7)) * a4;
  }
  for (int n = n8 + n4; n < 128; ++n) o[n] = 0.f;
}

// Diagnostic legacy encode of FP32 packed-order rows (state_codec.py:313-330):
// den = max(amax / lim, 1e-8); code = clamp(sign(z) * floor(|z| + 0.5)),
// z = v / den; stored scales half(den).
__global__ void k_encode_legacy(const float* v, uint8_t* lo, uint8_t* hi, uint8_t* q4, uint16_t* s8, uint16_t* s4,
                                int64_t rows) {
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  const float* x = v + r * 128;
  float m8 = 0.f, m4 = 0.f;
  for (int n = 0; n < 16; ++n) m8 = __builtin_fmaxf(m8, __builtin_fabsf(x[n]));
  for (int n = 16; n < 80; ++n) m4 = __builtin_fmaxf(m4, __builtin_fabsf(x[n]));
  const float d8 = __builtin_fmaxf(m8 / 127.0f, 1e-8f), d4 = __builtin_fmaxf(m4 / 7.0f, 1e-8f);
  int q[80];
  for (int n = 0; n < 80; ++n) {
    const float d = n < 16 ? d8 : d4, lim = n < 16 ? 127.0f : 7.0f;
    float z = x[n] / d;
    float sgn = z > 0.f ? 1.f : (z < 0.f ? -1.f : 0.f);
    float m = sgn * __builtin_floorf(__builtin_fabsf(z) + 0.5f);
    q[n] = (int)__builtin_fminf(__builtin_fmaxf(m, -lim), lim);
  }
  for (int j = 0; j < 8; ++j) {
    lo[r * 8 + j] = (uint8_t)((q[2 * j] & 15) | ((q[2 * j + 1] & 15) << 4));
    hi[r * 8 + j] = (uint8_t)(((q[2 * j] >> 4) & 15) | (((q[2 * j + 1] >> 4) & 15) << 4));
  }
  for (int j = 0; j < 32; ++j) q4[r * 32 + j] = (uint8_t)((q[16 + 2 * j] & 15) | ((q[17 + 2 * j] & 15) << 4));
  s8[r] = f2h(d8);
  s4[r] = f2h(d4);
}

}  // namespace m2r

using namespace m2r;

extern "C" int m2r_state_step_dense3(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                     const void* D, int d_is_f32, const void* dt_bias, int db_is_f32,
                                     const void* table, int table_is_equalizer, uint8_t* codes, void* scales,
                                     void* y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G,
                                     hipStream_t stream) {
  if (batch <= 0 || L <= 0 || H <= 0 || P <= 0 || G <= 0 || H % G) return m2r_fail("dense3 step: bad geometry");
  if ((double)batch * L * H * P >= 2147483647.0 || batch > 65535) return m2r_fail("dense3 step: size limits");
  Dense3Args args{(const uint16_t*)x, (const uint16_t*)dt, A, (const uint16_t*)B, (const uint16_t*)C, D, dt_bias,
                  table, codes, (uint16_t*)scales, (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G,
                  d_is_f32, db_is_f32, table_is_equalizer};
  const int pblocks = (int)((P + 63) / 64);
  const int hpg = (int)(H / G);
  // streaming kernel: 16-byte transfers of whole slots need P % 4 == 0 and
  // 16-byte aligned codes and scales; paired B/C loads need 4-byte alignment
  const bool stream_ok = P % 4 == 0 && (((uintptr_t)codes | (uintptr_t)scales) & 15) == 0 &&
                         (((uintptr_t)B | (uintptr_t)C) & 3) == 0;
  if (stream_ok) {
    const long long slots = (long long)batch * H * pblocks;
    int wpb = 1, hpw = 1;
    const int forced = m2r_forced_step_shape();
    if (forced && (forced & 15) && hpg % ((forced >> 4) * (forced & 15)) == 0 && (forced >> 4) != 8) {
      wpb = forced >> 4;
      hpw = forced & 15;
    } else if (hpg % 16 == 0 && slots >= 16LL * 512) {
      wpb = 4; hpw = 4;
    } else if (hpg % 8 == 0 && slots >= 8LL * 512) {
      wpb = 4; hpw = 2;
    } else if (hpg % 4 == 0) {
      wpb = 4; hpw = 1;
    }
    const dim3 grid((unsigned)pblocks, (unsigned)(H / (wpb * hpw)), (unsigned)batch), block(64 * wpb);
#define M2R_D3(W, K)                                                                     \
    if (wpb == W && hpw == K) {                                                          \
      if (L == 1) hipLaunchKernelGGL((k_dense3_slots<W, K, true>), grid, block, 0, stream, args);  \
      else hipLaunchKernelGGL((k_dense3_slots<W, K, false>), grid, block, 0, stream, args);        \
      return m2r_check(hipGetLastError(), "dense3 step launch");                         \
    }
    M2R_D3(4, 4)
    M2R_D3(4, 2)
    M2R_D3(4, 1)
    M2R_D3(1, 1)
#undef M2R_D3
    return m2r_fail("dense3 step: unsupported workgroup shape");
  }
  if (hpg % 4 == 0 && batch * H * pblocks >= 4096) {
    hipLaunchKernelGGL(k_dense3_step<4>, dim3(pblocks, (unsigned)(H / 4), (unsigned)batch), dim3(256), 0, stream,
                       args);
  } else {
    hipLaunchKernelGGL(k_dense3_step<1>, dim3(pblocks, (unsigned)H, (unsigned)batch), dim3(64), 0, stream, args);
  }
  return m2r_check(hipGetLastError(), "dense3 step launch");
}

extern "C" int m2r_state_decode(int kind, int n8, int n4, int nz, const uint8_t* lo, const uint8_t* hi,
                                const uint8_t* q4, const uint8_t* latent, const void* s8, const void* s4,
                                const void* extra, float* out, int64_t batch, int64_t H, int64_t P, int64_t flags,
                                hipStream_t stream) {
  (void)nz; (void)latent; (void)extra; (void)flags;
  int64_t rows = batch * H * P;
  if (rows <= 0) return m2r_fail("state decode: bad geometry");
  if (kind == 0 && (n8 < 0 || n4 < 0 || n8 + n4 > 128 || n8 % 2 || n4 % 2)) return m2r_fail("state decode: tiers");
  hipLaunchKernelGGL(k_state_decode, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, kind, n8, n4, lo,
                     hi, q4, (const uint16_t*)s8, (const uint16_t*)s4, out, rows);
  return m2r_check(hipGetLastError(), "state decode launch");
}

extern "C" int m2r_state_encode_legacy(const float* v, uint8_t* lo, uint8_t* hi, uint8_t* q4, void* s8, void* s4,
                                       int64_t rows, hipStream_t stream) {
  if (rows <= 0) return m2r_fail("legacy encode: bad geometry");
  hipLaunchKernelGGL(k_encode_legacy, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream, v, lo, hi, q4,
                     (uint16_t*)s8, (uint16_t*)s4, rows);
  return m2r_check(hipGetLastError(), "legacy encode launch");
}
