// One-token causal depthwise convolution update of the Mamba-2 mixer, for
// gfx950: the cached window rolls by one step, takes the new projection
// column, and the output is silu(sum(window * weight) + bias).
//
// Arithmetic: the reference's PyTorch fallback of the update
// (mamba2_recall/state_quant.py:289-297), operation for operation:
//   window <- roll(window, -1) along time; window[..., K-1] <- value
//   p_t = half(window_t * w_t)                 (binary16 products)
//   s   = half(((p_0 + p_1) + p_2) + p_3)      (binary32 sum in time order)
//   s   = half(s + bias)                       (when a bias is given)
//   out = half(s / (1 + exp(-s)))              (silu in binary32)
// One thread per (batch row, channel); the window is read and written
// through its strides (the controller keeps it time-major: [B, K, C] memory).
#include "m2r_device.h"
#include "m2r_abi_util.h"
#include "m2r_tile.h"

#include <initializer_list>

namespace m2r {

template <int K>
__global__ __launch_bounds__(256) void k_conv_update(uint16_t* window, int64_t ws_b, int64_t ws_c, int64_t ws_t,
                                                     const uint16_t* value, int64_t vs_b, const uint16_t* weight,
                                                     const uint16_t* bias, uint16_t* out, int64_t batch,
                                                     int64_t channels, int silu) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= batch * channels) return;
  const int64_t b = i / channels, c = i - b * channels;
  uint16_t* w = window + b * ws_b + c * ws_c;
  uint16_t win[K];
#pragma unroll
  for (int t = 0; t < K - 1; ++t) win[t] = w[(t + 1) * ws_t];
  win[K - 1] = value[b * vs_b + c];
  float acc = 0.f;
#pragma unroll
  for (int t = 0; t < K; ++t) {
    w[t * ws_t] = win[t];
    acc = acc + h2f(f2h(h2f(win[t]) * h2f(weight[c * K + t])));
  }
  float s = h2f(f2h(acc));
  if (bias) s = h2f(f2h(s + h2f(bias[c])));
  if (silu) s = s / (1.0f + expf(-s));
  out[i] = f2h(s);
}

}  // namespace m2r

using namespace m2r;

extern "C" int m2r_causal_conv_update(void* window, int64_t ws_b, int64_t ws_c, int64_t ws_t, const void* value,
                                      int64_t vs_b, const void* weight, const void* bias, void* out, int64_t batch,
                                      int64_t channels, int width, int silu, hipStream_t stream) {
  if (batch <= 0 || channels <= 0) return m2r_fail("conv update: non-positive shape");
  if (width != 4) return m2r_fail("conv update: the Mamba-2 convolution width is 4");
  if (batch * channels > (int64_t)1 << 40) return m2r_fail("conv update: size limits");
  const int64_t n = batch * channels;
  hipLaunchKernelGGL(k_conv_update<4>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, (uint16_t*)window,
                     ws_b, ws_c, ws_t, (const uint16_t*)value, vs_b, (const uint16_t*)weight,
                     (const uint16_t*)bias, (uint16_t*)out, batch, channels, silu);
  return m2r_check(hipGetLastError(), "conv update launch");
}

// ---------------------------------------------------------------------------
// Gated RMS norm of the Mamba-2 mixer (mamba_ssm's RMSNormGated with
// norm_before_gate = False, which the reference's controllers call as
// mx.norm(y, z), mamba2_recall/state_quant.py:298-300), per group of
// `gs` channels of a row, in binary32:
//   v   = y * (z * sigmoid(z)),  sigmoid(z) = 1 / (1 + exp(-z))
//   r   = 1 / sqrt(sum_group(v^2) / gs + eps)
//   out = half((v * r) * weight)
// One 256-thread workgroup per (row, group); a thread holds up to four
// chunks of four channels in registers.  The sum of squares is a fixed tree
// (per thread in chunk order, then the wave's adjacent-pair butterfly, then
// the four waves in order), so results do not vary from run to run.
namespace m2r {

typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_gated_rmsnorm(const uint16_t* y, int64_t ys, const uint16_t* z, int64_t zs,
                                                       const uint16_t* weight, uint16_t* out, int64_t os, int gs,
                                                       float eps) {
  __shared__ float part[4];
  const int64_t row = blockIdx.y;
  const int c0 = blockIdx.x * gs;
  const int tid = threadIdx.x;
  const u16x4* yr = (const u16x4*)(y + row * ys + c0);
  const u16x4* zr = (const u16x4*)(z + row * zs + c0);
  float v[4][4];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int q = k * 256 + tid;   // chunk of channels 4q .. 4q + 3 of the group
    if (4 * q < gs) {
      const u16x4 yv = yr[q], zv = zr[q];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float zf = h2f(zv[j]);
        const float sg = 1.0f / (1.0f + expf(-zf));
        v[k][j] = h2f(yv[j]) * (zf * sg);
        ss = __builtin_fmaf(v[k][j], v[k][j], ss);
      }
    }
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = 1.0f / __builtin_sqrtf(tot / (float)gs + eps);
  const u16x4* wr = (const u16x4*)(weight + c0);
  u16x4* orow = (u16x4*)(out + row * os + c0);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int q = k * 256 + tid;
    if (4 * q < gs) {
      const u16x4 wv = wr[q];
      u16x4 o;
#pragma unroll
      for (int j = 0; j < 4; ++j) o[j] = f2h((v[k][j] * r) * h2f(wv[j]));
      orow[q] = o;
    }
  }
}

}  // namespace m2r

extern "C" int m2r_gated_rmsnorm(const void* y, int64_t y_stride, const void* z, int64_t z_stride,
                                 const void* weight, void* out, int64_t out_stride, int64_t rows, int64_t channels,
                                 int64_t group_size, float eps, hipStream_t stream) {
  if (rows <= 0 || channels <= 0 || group_size <= 0) return m2r_fail("gated norm: non-positive shape");
  if (channels % group_size) return m2r_fail("gated norm: channels must be a multiple of the group size");
  if (group_size % 4 || group_size > 4096) return m2r_fail("gated norm: group size must be a multiple of 4, at most 4096");
  if (rows > 65535 || channels / group_size > 65535) return m2r_fail("gated norm: grid limits exceeded");
  if (!(eps >= 0.f)) return m2r_fail("gated norm: eps must be non-negative");
  if (!y || !z || !weight || !out) return m2r_fail("gated norm: null pointer");
  for (const void* p : {y, z, weight, (const void*)out})
    if ((uintptr_t)p & 7) return m2r_fail("gated norm: y, z, weight and out must be 8-byte aligned");
  if ((y_stride | z_stride | out_stride) & 3 || y_stride < channels || z_stride < channels || out_stride < channels)
    return m2r_fail("gated norm: row strides must be multiples of 4 elements, at least the channel count");
  hipLaunchKernelGGL(k_gated_rmsnorm, dim3((unsigned)(channels / group_size), (unsigned)rows), dim3(256), 0, stream,
                     (const uint16_t*)y, y_stride, (const uint16_t*)z, z_stride, (const uint16_t*)weight,
                     (uint16_t*)out, out_stride, (int)group_size, eps);
  return m2r_check(hipGetLastError(), "gated norm launch");
}
