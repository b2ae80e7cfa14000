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
