// FP16-carry control scan (the reference's s16 mode) for gfx950, with the
// optional calibration statistics.
//
//   s16     mamba2_recall/state_codec.py:65-102 (_s16_scan)
//
// A translation unit of its own: it is compiled with the default machine
// scheduler, the dense3 and packed-row steps with the max-ILP one.
#include "m2r_device.h"
#include "m2r_abi_util.h"
#include "m2r_tile.h"

namespace m2r {

// ---------------------------------------------------------------------------
// FP16-carry control: state = half(fma(state, decay, (B*dt) * x)) after the
// readout y = sum(state * C) + x * D.  Optional statistics: sum over tokens
// and the rows of each 16-row P tile of |FP16 carry| per coordinate, in one
// fixed order (so they are the same on every run): each row's sum over the
// tokens in token order (state_codec.py:100-101), the rows of each 4-row
// sub-tile as (r0 + r1) + (r2 + r3) (the per-program tl.sum of :102), and
// the four sub-tiles of a 16-row tile in order, ((T0 + T1) + T2) + T3 (the
// host-side sum of state_codec.py:255-261).
struct S16Args {
  const uint16_t* x; const uint16_t* dt; const float* A; const uint16_t* Bm; const uint16_t* Cm;
  const void* D; const void* dt_bias;
  uint16_t* state; uint16_t* y; float* stats;
  int B, L, H, P, G;
  int d_f32, db_f32;
};

// STAGED (state 16-byte aligned): the slot's 64 rows of 256 B move between
// HBM and registers through LDS, one half-row (128 B) of every row at a
// time, as 1 KiB wave-wide transfers (8 per half, each 8 rows x 128 B);
// half-rows sit in LDS at a 144-byte pitch, so each group of 16 lanes
// reading 16 bytes of its own row covers the 64 banks once.  The half-size
// buffer (9 KiB) leaves room for more workgroups per CU.  Otherwise every
// lane reads its row directly.
constexpr int S16_PITCH = 36;   // dwords per staged half-row (32 + 4 padding)
constexpr int S16_SUM_PITCH = 132;   // dwords per row of the statistics' per-row sums
typedef uint32_t s16x4 __attribute__((ext_vector_type(4)));

// STATS: each lane keeps its row's sums over the tokens in LDS (its own row:
// no other lane adds to it), reduced in the fixed order above at the end.
template <bool STAGED, bool STATS>
__global__ __launch_bounds__(64) void k_s16_step(S16Args a) {
  __shared__ __align__(16) float s_b[128];
  __shared__ __align__(16) float s_c[128];
  __shared__ __align__(16) float s_sum[STATS ? 64 * S16_SUM_PITCH : 4];
  __shared__ __align__(16) uint32_t s_rows[STAGED ? 64 * S16_PITCH : 4];   // one half-row per row
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
    for (int hf = 0; hf < 2; ++hf) {
      if (hf) __syncthreads();   // every lane has read the first half-rows
#pragma unroll
      for (int k = 0; k < 8; ++k) {   // row 8k + lane / 8, 16-byte part 8 hf + lane % 8
        const int r = 8 * k + (lane >> 3), part = 8 * hf + (lane & 7);
        const s16x4 v = r < nvalid ? src[16 * r + part] : s16x4{0u, 0u, 0u, 0u};
        *(s16x4*)(s_rows + r * S16_PITCH + 4 * (lane & 7)) = v;
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        const s16x4 v = *(const s16x4*)(s_rows + lane * S16_PITCH + 4 * p);
#pragma unroll
        for (int e = 0; e < 8; ++e) st[8 * (8 * hf + p) + e] = h2f((uint16_t)(v[e >> 1] >> (16 * (e & 1))));
      }
    }
  } else {
#pragma unroll
    for (int n = 0; n < 128; ++n) st[n] = valid ? h2f(a.state[row * 128 + n]) : 0.f;
  }
  if constexpr (STATS) {   // the lane's own row of sums (rows past P stay zero)
#pragma unroll
    for (int q = 0; q < 32; ++q) *(f32x4*)(s_sum + lane * S16_SUM_PITCH + 4 * q) = f32x4{0.f, 0.f, 0.f, 0.f};
  }
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
    if constexpr (STATS) {
      if (valid) {   // the row's sums over the tokens, in token order
        float* row_sum = s_sum + lane * S16_SUM_PITCH;
#pragma unroll
        for (int q = 0; q < 32; ++q) {
          f32x4 v = *(const f32x4*)(row_sum + 4 * q);
          v.x = v.x + __builtin_fabsf(st[4 * q]);
          v.y = v.y + __builtin_fabsf(st[4 * q + 1]);
          v.z = v.z + __builtin_fabsf(st[4 * q + 2]);
          v.w = v.w + __builtin_fabsf(st[4 * q + 3]);
          *(f32x4*)(row_sum + 4 * q) = v;
        }
      }
    }
    __syncthreads();
  }
  if constexpr (STAGED) {
    s16x4* dst = (s16x4*)(a.state + row0 * 128);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      __syncthreads();   // every lane has read (or stored) the buffer's previous contents
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        s16x4 v;
        const int part = 8 * hf + p;
#pragma unroll
        for (int w = 0; w < 4; ++w)
          v[w] = (uint32_t)f2h(st[8 * part + 2 * w]) | ((uint32_t)f2h(st[8 * part + 2 * w + 1]) << 16);
        *(s16x4*)(s_rows + lane * S16_PITCH + 4 * p) = v;
      }
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int r = 8 * k + (lane >> 3), part = 8 * hf + (lane & 7);
        if (r < nvalid) dst[16 * r + part] = *(const s16x4*)(s_rows + r * S16_PITCH + 4 * (lane & 7));
      }
    }
  } else if (valid) {
#pragma unroll
    for (int n = 0; n < 128; ++n) a.state[row * 128 + n] = f2h(st[n]);
  }
  if constexpr (STATS) {
    __syncthreads();   // every row's sums are complete
    const int tiles = (P + 15) / 16;
    for (int i = lane; i < 512; i += 64) {
      const int tl = i >> 7, n = i & 127;
      const int tile = pbase / 16 + tl;
      float sub[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {   // 4-row sub-tile j of the 16-row tile
        const float* r = s_sum + (16 * tl + 4 * j) * S16_SUM_PITCH + n;
        sub[j] = (r[0] + r[S16_SUM_PITCH]) + (r[2 * S16_SUM_PITCH] + r[3 * S16_SUM_PITCH]);
      }
      if (tile < tiles && pbase + 16 * tl < P)
        a.stats[(((size_t)b * H + h) * tiles + tile) * 128 + n] = ((sub[0] + sub[1]) + sub[2]) + sub[3];
    }
  }
}

}  // namespace m2r

using namespace m2r;

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
  const bool staged = ((uintptr_t)state & 15) == 0;
  if (staged && stats) hipLaunchKernelGGL((k_s16_step<true, true>), grid, dim3(64), 0, stream, args);
  else if (staged) hipLaunchKernelGGL((k_s16_step<true, false>), grid, dim3(64), 0, stream, args);
  else if (stats) hipLaunchKernelGGL((k_s16_step<false, true>), grid, dim3(64), 0, stream, args);
  else hipLaunchKernelGGL((k_s16_step<false, false>), grid, dim3(64), 0, stream, args);
  return m2r_check(hipGetLastError(), "s16 step launch");
}
