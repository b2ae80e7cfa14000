// Packed-resident FP4 (E2M1, G16) matrix-vector products for gfx950:
// y[m, n] = sum_k u[m, k] * w[n, k] for M <= 4 activation rows, with the
// weights read straight from the checkpoint format (two codes per byte, one
// E4M3 block scale per 16 weights, one FP32 global scale) instead of from a
// decoded FP16 copy: 0.5625 bytes per weight instead of 2.
//
// Every weight is the binary16 value fp4.decode_packet produces
// (mamba2_recall/fp4.py:151-154): half(RN(RN(lev * block) * global)), lev in
// {0, .5, 1, 1.5, 2, 3, 4, 6}, sign from bit 3 of the code.  Each workgroup
// builds that value for every (block byte, level) pair in an LDS table (128 x
// 8 binary16, stored as low-byte and high-byte planes), so a weight costs one
// byte-permute lookup: the code nibbles select their entries' low and high
// bytes with v_perm_b32, each code's sign bit is or-ed into bit 7 of its high
// byte (the binary16 sign), two more permutes form the binary16 pairs, and
// v_dot2_f32_f16 multiplies weight pairs by activation pairs and accumulates
// in binary32: about 2.25 VALU instructions per weight and activation row.  The packet must satisfy decode_packet's checks
// (the loader validates each matrix once); block bytes with the sign bit set
// other than 0x80 are outside that contract.
//
// Mapping: a workgroup of four waves takes 4 / KCH rows at a time (rows
// strided over the grid); wave w works on 2048-wide chunk c = w % KCH of row
// w / KCH, lane l on k in [2048 c + 32 l, 2048 c + 32 l + 32): one 16-byte
// code load, one 2-byte scale load and two table reads per row.  The loads of
// the next two rows are in flight while a row computes; the grid is one
// resident round of workgroups.  The activations of the
// lane's k range stay in registers, reordered once into the weight pairs'
// order.  A wave sum per chunk, then the chunks' partial sums in a fixed
// order through LDS, finish each output.  One activation row (the batch-1
// decode) takes k_fp4_gemv_rows instead where it fills the chip in one
// resident round: whole rows per wave, no barrier per row, the same sums.
#include "m2r_device.h"
#include "m2r_abi_util.h"
#include "m2r_tile.h"

#include <algorithm>
#include <atomic>

namespace m2r {

typedef _Float16 gh2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(gh2, a), __builtin_bit_cast(gh2, b), c, false);
}

// 8 weights of code word cw against the activation pairs ue (k = 0,2 | 4,6)
// and uo (1,3 | 5,7) of the same 8 positions, with the block's table t.
__device__ __forceinline__ void fp4_dot8(uint32_t cw, const uint32_t (&t)[4], const uint32_t* ue, const uint32_t* uo,
                                         float& acc) {
  const uint32_t even = cw & 0x07070707u, odd = (cw >> 4) & 0x07070707u;
  // low and high bytes of the magnitudes; the code's sign bit (bit 3 of the
  // nibble: bit 3 of byte j for the even weight 2j, bit 7 for the odd weight
  // 2j+1) becomes bit 7 of the high byte, i.e. the binary16 sign (the
  // magnitudes' high bytes have it clear)
  const uint32_t le = __builtin_amdgcn_perm(t[1], t[0], even), lo = __builtin_amdgcn_perm(t[1], t[0], odd);
  const uint32_t he = __builtin_amdgcn_perm(t[3], t[2], even) | ((cw & 0x08080808u) << 4);
  const uint32_t ho = __builtin_amdgcn_perm(t[3], t[2], odd) | (cw & 0x80808080u);
  // binary16 pairs (w0, w2), (w4, w6), (w1, w3), (w5, w7): low byte, high byte
  const uint32_t e01 = __builtin_amdgcn_perm(he, le, 0x05010400u), e23 = __builtin_amdgcn_perm(he, le, 0x07030602u);
  const uint32_t o01 = __builtin_amdgcn_perm(ho, lo, 0x05010400u), o23 = __builtin_amdgcn_perm(ho, lo, 0x07030602u);
  acc = dot2(e01, ue[0], acc);
  acc = dot2(e23, ue[1], acc);
  acc = dot2(o01, uo[0], acc);
  acc = dot2(o23, uo[1], acc);
}

template <int M, int KCH>
__global__ __launch_bounds__(256) void k_fp4_gemv(const uint8_t* __restrict__ codes, const uint8_t* __restrict__ scales,
                                                  const float* __restrict__ gscale, const uint16_t* __restrict__ u,
                                                  int64_t u_stride, uint16_t* __restrict__ y, int64_t y_stride,
                                                  int N) {
  static_assert(KCH == 1 || KCH == 2 || KCH == 4, "the four waves split a row's chunks evenly");
  constexpr int K = KCH * 2048;
  constexpr int RPI = 4 / KCH;   // rows per workgroup iteration: wave w takes chunk w % KCH of row w / KCH
  __shared__ __align__(16) uint32_t s_tab[128][4];   // per block byte: low bytes of T[0..7], then high bytes
  __shared__ float s_part[2][RPI][KCH][M];           // per-chunk partial sums, double-buffered by iteration
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = wave % KCH, r = wave / KCH;
  const int stride = (int)gridDim.x * RPI;
  int n = (int)blockIdx.x * RPI + r;
  // the first row's loads go out before the table is built
  auto load_row = [&](int row, u32x4& cv, uint32_t& sb) {
    const int rr = min(row, N - 1);   // rows past N re-read row N-1 (never stored)
    cv = __builtin_nontemporal_load((const u32x4*)(codes + (size_t)rr * (K / 2) + c * 1024) + lane);
    sb = *(const uint16_t*)(scales + (size_t)rr * (K / 16) + c * 128 + 2 * lane);
  };
  // two rows ahead: the loads of iterations it + 1 and it + 2 are in flight
  // while iteration it computes
  u32x4 cv, cv2;
  uint32_t sb, sb2;
  load_row(n, cv, sb);
  load_row(n + stride, cv2, sb2);
  const float gl = *gscale;
  for (int e = threadIdx.x; e < 128 * 8; e += 256) {
    const int blk = e >> 3, i = e & 7;
    // 2 * lev as an integer, times block / 2: RN(lev * block) exactly
    const float lev2 = (float)((i < 4) ? i : (i == 4 ? 4 : (i == 5 ? 6 : (i == 6 ? 8 : 12))));
    const float hb = e4m3_byte_to_f32<0>((uint32_t)blk) * 0.5f;
    const uint16_t h = f2h((lev2 * hb) * gl);
    uint8_t* row = (uint8_t*)s_tab[blk];
    row[i] = (uint8_t)(h & 0xFFu);
    row[8 + i] = (uint8_t)(h >> 8);
  }
  // activations of the lane's k range of chunk c, as pairs in the weights'
  // order: per 8 positions (u0,u2), (u4,u6) | (u1,u3), (u5,u7)
  uint32_t ue[M][8], uo[M][8];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const uint32_t* src = (const uint32_t*)(u + m * u_stride + c * 2048 + 32 * lane);
    uint32_t p[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 v = ((const u32x4*)src)[q];
      p[4 * q] = v.x; p[4 * q + 1] = v.y; p[4 * q + 2] = v.z; p[4 * q + 3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {   // 8 positions = natural pairs p[4q .. 4q+3]
      ue[m][2 * q] = __builtin_amdgcn_perm(p[4 * q + 1], p[4 * q], 0x05040100u);
      ue[m][2 * q + 1] = __builtin_amdgcn_perm(p[4 * q + 3], p[4 * q + 2], 0x05040100u);
      uo[m][2 * q] = __builtin_amdgcn_perm(p[4 * q + 1], p[4 * q], 0x07060302u);
      uo[m][2 * q + 1] = __builtin_amdgcn_perm(p[4 * q + 3], p[4 * q + 2], 0x07060302u);
    }
  }
  __syncthreads();   // the table is complete
  for (int it = 0; (int)blockIdx.x * RPI + it * stride < N; ++it) {
    const u32x4 cur = cv;
    const uint32_t scur = sb;
    cv = cv2;
    sb = sb2;
    load_row(n + 2 * stride, cv2, sb2);
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.f;
#pragma unroll
    for (int gidx = 0; gidx < 2; ++gidx) {   // two 16-weight groups per lane
      const u32x4 tv = *(const u32x4*)s_tab[(scur >> (8 * gidx)) & 0x7Fu];
      const uint32_t t[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int q = 2 * gidx + h;   // code word of the 16-byte load: positions 8q .. 8q+7
        const uint32_t cw = q == 0 ? cur.x : q == 1 ? cur.y : q == 2 ? cur.z : cur.w;
#pragma unroll
        for (int m = 0; m < M; ++m) fp4_dot8(cw, t, &ue[m][2 * q], &uo[m][2 * q], acc[m]);
      }
    }
    float (&part)[RPI][KCH][M] = s_part[it & 1];
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const float sum = wave_sum(acc[m]);
      if (lane == 0) part[r][c][m] = sum;
    }
    __syncthreads();   // one barrier per iteration: the other buffer is free again by the next one
    if (c == 0 && lane < M && n < N) {
      float tot = part[r][0][lane];
#pragma unroll
      for (int cc = 1; cc < KCH; ++cc) tot += part[r][cc][lane];
      y[lane * y_stride + n] = f2h(tot);
    }
    n += stride;
  }
}

// One activation row (M == 1): each wave takes D whole rows (rows strided
// over every wave of the grid, W waves: rows w, w + W, ..., w + (D - 1) W),
// lane l the same k ranges as above in each of the row's KCH chunks, so a row
// needs no workgroup barrier: the KCH chunk sums are wave sums added in chunk
// order, the same bits as k_fp4_gemv<1, KCH>.  The host sizes the grid so
// that D W >= N with every workgroup resident at once: all of a wave's loads
// are issued first (rows past N re-read row N - 1, which is never stored),
// then the table is built, and each row is computed as soon as its loads
// have landed, while the later rows' loads are still in flight.
template <int KCH, int D, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_fp4_gemv_rows(const uint8_t* __restrict__ codes,
                                                           const uint8_t* __restrict__ scales,
                                                           const float* __restrict__ gscale,
                                                           const uint16_t* __restrict__ u,
                                                           uint16_t* __restrict__ y, int N) {
  static_assert(KCH == 1 || KCH == 2 || KCH == 4, "K of 2048, 4096 or 8192");
  constexpr int K = KCH * 2048;
  __shared__ __align__(16) uint32_t s_tab[128][4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int W = (int)gridDim.x * WPB;
  const int n0 = (int)blockIdx.x * WPB + wave;
  // the activations first (shared by every wave, cache hits), so that
  // waiting for them does not wait for the rows
  u32x4 uv[KCH][4];
#pragma unroll
  for (int cc = 0; cc < KCH; ++cc)
#pragma unroll
    for (int q = 0; q < 4; ++q) uv[cc][q] = ((const u32x4*)(u + cc * 2048 + 32 * lane))[q];
  u32x4 cv[D][KCH];
  uint32_t sb[D][KCH];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    const int row = min(n0 + j * W, N - 1);
#pragma unroll
    for (int cc = 0; cc < KCH; ++cc) {
      cv[j][cc] = __builtin_nontemporal_load((const u32x4*)(codes + (size_t)row * (K / 2) + cc * 1024) + lane);
      sb[j][cc] = *(const uint16_t*)(scales + (size_t)row * (K / 16) + cc * 128 + 2 * lane);
    }
  }
  const float gl = *gscale;
  for (int e = threadIdx.x; e < 128 * 8; e += 64 * WPB) {
    const int blk = e >> 3, i = e & 7;
    const float lev2 = (float)((i < 4) ? i : (i == 4 ? 4 : (i == 5 ? 6 : (i == 6 ? 8 : 12))));
    const float hb = e4m3_byte_to_f32<0>((uint32_t)blk) * 0.5f;
    const uint16_t h = f2h((lev2 * hb) * gl);
    uint8_t* row = (uint8_t*)s_tab[blk];
    row[i] = (uint8_t)(h & 0xFFu);
    row[8 + i] = (uint8_t)(h >> 8);
  }
  // activation pairs in the weights' order: per 8 positions (u0,u2), (u4,u6)
  // | (u1,u3), (u5,u7)
  uint32_t ue[KCH][8], uo[KCH][8];
#pragma unroll
  for (int cc = 0; cc < KCH; ++cc) {
    uint32_t p[16];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      p[4 * q] = uv[cc][q].x; p[4 * q + 1] = uv[cc][q].y; p[4 * q + 2] = uv[cc][q].z; p[4 * q + 3] = uv[cc][q].w;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ue[cc][2 * q] = __builtin_amdgcn_perm(p[4 * q + 1], p[4 * q], 0x05040100u);
      ue[cc][2 * q + 1] = __builtin_amdgcn_perm(p[4 * q + 3], p[4 * q + 2], 0x05040100u);
      uo[cc][2 * q] = __builtin_amdgcn_perm(p[4 * q + 1], p[4 * q], 0x07060302u);
      uo[cc][2 * q + 1] = __builtin_amdgcn_perm(p[4 * q + 3], p[4 * q + 2], 0x07060302u);
    }
  }
  __syncthreads();   // the table is complete
#pragma unroll
  for (int j = 0; j < D; ++j) {
    float tot = 0.f;
#pragma unroll
    for (int cc = 0; cc < KCH; ++cc) {
      const u32x4 cur = cv[j][cc];
      const uint32_t scur = sb[j][cc];
      float acc = 0.f;
#pragma unroll
      for (int gidx = 0; gidx < 2; ++gidx) {
        const u32x4 tv = *(const u32x4*)s_tab[(scur >> (8 * gidx)) & 0x7Fu];
        const uint32_t t[4] = {tv.x, tv.y, tv.z, tv.w};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int q = 2 * gidx + h;
          const uint32_t cw = q == 0 ? cur.x : q == 1 ? cur.y : q == 2 ? cur.z : cur.w;
          fp4_dot8(cw, t, &ue[cc][2 * q], &uo[cc][2 * q], acc);
        }
      }
      const float sum = wave_sum(acc);
      tot = cc == 0 ? sum : tot + sum;
    }
    const int n = n0 + j * W;
    if (lane == 0 && n < N) y[n] = f2h(tot);
  }
}

}  // namespace m2r

using namespace m2r;

// The whole-row kernel for one activation row: the smallest rows-per-wave D
// for which one resident round of eight-wave workgroups covers N rows, if
// that round has a workgroup for every CU (D <= 6; D <= 2 for K = 8192,
// whose larger D leave two waves per SIMD, slower than the general kernel).
// Returns 1 when launched, 0 when the general kernel is to be used, or a
// negative error.
template <int KCH, int D>
static int launch_rows_d(const uint8_t* packed, const uint8_t* sc, const float* gs, const uint16_t* u, uint16_t* y,
                         int64_t N, int cus, hipStream_t stream) {
  constexpr int WPB = 8;
  // resident workgroups per CU of this instance (a property of the code
  // object, the same on every gfx950 device), queried once
  static std::atomic<int> per_cu_cache{-1};
  int per_cu = per_cu_cache.load(std::memory_order_relaxed);
  if (per_cu < 0) {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, (const void*)k_fp4_gemv_rows<KCH, D, WPB>, 64 * WPB, 0) !=
        hipSuccess)
      return -m2r_fail("fp4 gemv: occupancy query failed");
    per_cu = b;
    per_cu_cache.store(b, std::memory_order_relaxed);
  }
  const int64_t waves = (N + D - 1) / D, blocks = (waves + WPB - 1) / WPB;
  if (per_cu <= 0 || blocks > (int64_t)per_cu * cus || blocks < cus) return 0;
  hipLaunchKernelGGL((k_fp4_gemv_rows<KCH, D, WPB>), dim3((unsigned)blocks), dim3(64 * WPB), 0, stream, packed, sc,
                     gs, u, y, (int)N);
  return 1;
}

template <int KCH>
static int launch_rows_k(const uint8_t* packed, const uint8_t* sc, const float* gs, const uint16_t* u, uint16_t* y,
                         int64_t N, int cus, hipStream_t stream) {
  int r = 0;
  if (!r) r = launch_rows_d<KCH, 1>(packed, sc, gs, u, y, N, cus, stream);
  if (!r) r = launch_rows_d<KCH, 2>(packed, sc, gs, u, y, N, cus, stream);
  if constexpr (KCH < 4) {
    if (!r) r = launch_rows_d<KCH, 3>(packed, sc, gs, u, y, N, cus, stream);
    if (!r) r = launch_rows_d<KCH, 4>(packed, sc, gs, u, y, N, cus, stream);
    if (!r) r = launch_rows_d<KCH, 5>(packed, sc, gs, u, y, N, cus, stream);
    if (!r) r = launch_rows_d<KCH, 6>(packed, sc, gs, u, y, N, cus, stream);
  }
  return r;
}

static int launch_rows(int kch, const uint8_t* packed, const uint8_t* sc, const float* gs, const uint16_t* u,
                       uint16_t* y, int64_t N, hipStream_t stream) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return -m2r_fail("fp4 gemv: device query failed");
  if (kch == 1) return launch_rows_k<1>(packed, sc, gs, u, y, N, cus, stream);
  if (kch == 2) return launch_rows_k<2>(packed, sc, gs, u, y, N, cus, stream);
  return launch_rows_k<4>(packed, sc, gs, u, y, N, cus, stream);
}

extern "C" int m2r_fp4_gemv_g16(const uint8_t* packed, const uint8_t* e4m3_scales, const float* global_scale,
                                const void* u, int64_t u_stride, void* y, int64_t y_stride, int64_t M, int64_t N,
                                int64_t K, hipStream_t stream) {
  if (M <= 0 || N <= 0 || K <= 0) return m2r_fail("fp4 gemv: non-positive shape");
  if (K % 2048) return m2r_fail("fp4 gemv: K must be a multiple of 2048");
  if (N > (1 << 30) || u_stride < K || y_stride < N) return m2r_fail("fp4 gemv: size or stride limits");
  if ((((uintptr_t)packed | (uintptr_t)u) & 15) || (u_stride % 8) || ((uintptr_t)e4m3_scales & 1))
    return m2r_fail("fp4 gemv: codes and activation rows must be 16-byte aligned, scales 2-byte aligned");
  const int kch = (int)(K / 2048);
  if (M == 1) {
    if (int e = launch_rows(kch, packed, e4m3_scales, global_scale, (const uint16_t*)u, (uint16_t*)y, N, stream))
      return e > 0 ? m2r_check(hipGetLastError(), "fp4 gemv launch") : 1;
  }
  const int rpi = 4 / kch > 0 ? 4 / kch : 1;
  // one resident round: eight four-wave workgroups per CU
  const int blocks = (int)std::min<int64_t>((N + rpi - 1) / rpi, 2048);
  const dim3 grid(blocks), block(256);
#define M2R_GEMV(MM, KK)                                                                                       \
  if (M == MM && kch == KK) {                                                                                  \
    hipLaunchKernelGGL((k_fp4_gemv<MM, KK>), grid, block, 0, stream, packed, e4m3_scales, global_scale,         \
                       (const uint16_t*)u, u_stride, (uint16_t*)y, y_stride, (int)N);                          \
    return m2r_check(hipGetLastError(), "fp4 gemv launch");                                                   \
  }
  M2R_GEMV(1, 1) M2R_GEMV(1, 2) M2R_GEMV(1, 4)
  M2R_GEMV(2, 1) M2R_GEMV(2, 2) M2R_GEMV(2, 4)
  M2R_GEMV(4, 1) M2R_GEMV(4, 2) M2R_GEMV(4, 4)
#undef M2R_GEMV
  return m2r_fail("fp4 gemv: supported are M in {1, 2, 4} rows of u and K in {2048, 4096, 8192}");
}
