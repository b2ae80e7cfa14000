// Dense 3-bit state step (all 128 coordinates as 3-bit codes in three bit
// planes + two FP16 half-row scales), the FP16-carry control scan, and the
// diagnostic packed-state decode / legacy encode, for gfx950.
//
//   dense3  mamba2_recall/state_codec_dense3.py:82-148 (_scan)
//   s16     mamba2_recall/state_codec.py:65-102 (_s16_scan)
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
    const float nb0 = -4.0f * sc0, nb1 = -4.0f * sc1;
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
        float prior = (i < 64) ? __builtin_fmaf(ubyte_f(c[i / 4], j), sc0, nb0)
                               : __builtin_fmaf(ubyte_f(c[i / 4], j), sc1, nb1);
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

    float den0 = __builtin_fmaxf(div_by_recip(amax0, 3.0f, y3), 1e-8f);
    float den1 = __builtin_fmaxf(div_by_recip(amax1, 3.0f, y3), 1e-8f);
    float r0 = 1.0f / den0, r1 = 1.0f / den1;
    sc0 = round_to_half(den0);
    sc1 = round_to_half(den1);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const float d = (i < 16) ? den0 : den1, r = (i < 16) ? r0 : r1;
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
// FP16-carry control: state = half(fma(state, decay, (B*dt) * x)) after the
// readout y = sum(state * C) + x * D.  Optional statistics: sum over tokens
// and the rows of each 16-row P tile of |FP16 carry| per coordinate.
struct S16Args {
  const uint16_t* x; const uint16_t* dt; const float* A; const uint16_t* Bm; const uint16_t* Cm;
  const void* D; const void* dt_bias;
  uint16_t* state; uint16_t* y; float* stats;
  int B, L, H, P, G;
  int d_f32, db_f32;
};

// STAGED (state 16-byte aligned): the slot's 64 rows of 256 B move between
// HBM and registers through LDS, as 1 KiB wave-wide transfers (16 per slot);
// rows sit in LDS at a 272-byte pitch, so each group of 16 lanes reading
// 16 bytes of its own row covers the 64 banks once.  Otherwise every lane
// reads its row directly.
constexpr int S16_PITCH = 68;   // dwords per staged row (64 + 4 padding)
typedef uint32_t s16x4 __attribute__((ext_vector_type(4)));

template <bool STAGED>
__global__ __launch_bounds__(64) void k_s16_step(S16Args a) {
  __shared__ __align__(16) float s_b[128];
  __shared__ __align__(16) float s_c[128];
  __shared__ float s_acc[4][128];
  __shared__ __align__(16) uint32_t s_rows[STAGED ? 64 * S16_PITCH : 4];
  const int lane = threadIdx.x;
  const int b = blockIdx.z, h = blockIdx.y;
  const int H = a.H, P = a.P, G = a.G, L = a.L;
  const int g = h / (H / G);
  const int pbase = blockIdx.x * 64;
  const int nvalid = min(64, P - pbase);
  const bool valid = lane < nvalid;
  const size_t row0 = (size_t)(b * H + h) * P + pbase;
  const size_t row = row0 + lane;
  float st[128];
  if constexpr (STAGED) {
    const s16x4* src = (const s16x4*)(a.state + row0 * 128);
#pragma unroll
    for (int k = 0; k < 16; ++k) {   // chunk q = 64k + lane: row q / 16, 16-byte part q % 16
      const int r = 4 * k + (lane >> 4), part = lane & 15;
      const s16x4 v = r < nvalid ? src[64 * k + lane] : s16x4{0u, 0u, 0u, 0u};
      *(s16x4*)(s_rows + r * S16_PITCH + 4 * part) = v;
    }
    __syncthreads();
#pragma unroll
    for (int part = 0; part < 16; ++part) {
      const s16x4 v = *(const s16x4*)(s_rows + lane * S16_PITCH + 4 * part);
#pragma unroll
      for (int e = 0; e < 8; ++e) st[8 * part + e] = h2f((uint16_t)(v[e >> 1] >> (16 * (e & 1))));
    }
  } else {
#pragma unroll
    for (int n = 0; n < 128; ++n) st[n] = valid ? h2f(a.state[row * 128 + n]) : 0.f;
  }
  for (int n = lane; n < 512; n += 64) (&s_acc[0][0])[n] = 0.f;
  const float av = a.A[h], Dh = load_param(a.D, a.d_f32, h), bias = load_param(a.dt_bias, a.db_f32, h);
  for (int t = 0; t < L; ++t) {
    const int bt = b * L + t;
    for (int n = lane; n < 128; n += 64) {
      s_b[n] = h2f(a.Bm[((size_t)bt * G + g) * 128 + n]);
      s_c[n] = h2f(a.Cm[((size_t)bt * G + g) * 128 + n]);
    }
    __syncthreads();
    const float2 act = dt_activation(h2f(a.dt[(size_t)bt * H + h]) + bias, av);
    const float dtv = act.x, decay = act.y;
    float x = valid ? h2f(a.x[((size_t)bt * H + h) * P + pbase + lane]) : 0.f;
    float acc = 0.f;
#pragma unroll
    for (int n = 0; n < 128; ++n) {
      float dB = s_b[n] * dtv;
      st[n] = state_update(st[n], decay, dB * x);
      acc = __builtin_fmaf(st[n], s_c[n], acc);
    }
    asm volatile("" : "+v"(acc));
    if (valid) a.y[((size_t)bt * H + h) * P + pbase + lane] = f2h(acc + x * Dh);
#pragma unroll
    for (int n = 0; n < 128; ++n) st[n] = round_to_half(st[n]);
    if (a.stats && valid) {
      const int tile = lane >> 4;
#pragma unroll
      for (int n = 0; n < 128; ++n) atomicAdd(&s_acc[tile][n], __builtin_fabsf(st[n]));
    }
    __syncthreads();
  }
  if constexpr (STAGED) {
    __syncthreads();   // every lane has read its row before the buffer is reused
#pragma unroll
    for (int part = 0; part < 16; ++part) {
      s16x4 v;
#pragma unroll
      for (int w = 0; w < 4; ++w)
        v[w] = (uint32_t)f2h(st[8 * part + 2 * w]) | ((uint32_t)f2h(st[8 * part + 2 * w + 1]) << 16);
      *(s16x4*)(s_rows + lane * S16_PITCH + 4 * part) = v;
    }
    __syncthreads();
    s16x4* dst = (s16x4*)(a.state + row0 * 128);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int r = 4 * k + (lane >> 4), part = lane & 15;
      if (r < nvalid) dst[64 * k + lane] = *(const s16x4*)(s_rows + r * S16_PITCH + 4 * part);
    }
  } else if (valid) {
#pragma unroll
    for (int n = 0; n < 128; ++n) a.state[row * 128 + n] = f2h(st[n]);
  }
  if (a.stats) {
    const int tiles = (P + 15) / 16;
    for (int i = lane; i < 512; i += 64) {
      int tl = i >> 7, n = i & 127;
      int tile = pbase / 16 + tl;
      if (tile < tiles && pbase + 16 * tl < P)
        a.stats[(((size_t)b * H + h) * tiles + tile) * 128 + n] = s_acc[tl][n];
    }
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
  if ((H / G) % 4 == 0 && batch * H * pblocks >= 4096) {
    hipLaunchKernelGGL(k_dense3_step<4>, dim3(pblocks, (unsigned)(H / 4), (unsigned)batch), dim3(256), 0, stream,
                       args);
  } else {
    hipLaunchKernelGGL(k_dense3_step<1>, dim3(pblocks, (unsigned)H, (unsigned)batch), dim3(64), 0, stream, args);
  }
  return m2r_check(hipGetLastError(), "dense3 step launch");
}

extern "C" int m2r_state_step_s16(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                  const void* D, int d_is_f32, const void* dt_bias, int db_is_f32, void* state,
                                  void* y, float* stats, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G,
                                  hipStream_t stream) {
  if (batch <= 0 || L <= 0 || H <= 0 || P <= 0 || G <= 0 || H % G) return m2r_fail("s16 step: bad geometry");
  if ((double)batch * L * H * P >= 2147483647.0 || batch > 65535) return m2r_fail("s16 step: size limits");
  S16Args args{(const uint16_t*)x, (const uint16_t*)dt, A, (const uint16_t*)B, (const uint16_t*)C, D, dt_bias,
               (uint16_t*)state, (uint16_t*)y, stats, (int)batch, (int)L, (int)H, (int)P, (int)G, d_is_f32,
               db_is_f32};
  const dim3 grid((unsigned)((P + 63) / 64), (unsigned)H, (unsigned)batch);
  if (((uintptr_t)state & 15) == 0)
    hipLaunchKernelGGL(k_s16_step<true>, grid, dim3(64), 0, stream, args);
  else
    hipLaunchKernelGGL(k_s16_step<false>, grid, dim3(64), 0, stream, args);
  return m2r_check(hipGetLastError(), "s16 step launch");
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
