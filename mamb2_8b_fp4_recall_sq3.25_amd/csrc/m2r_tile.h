// Wave-level tiling helpers shared by the state-step kernels: LDS staging of
// SoA packed rows, broadcast-friendly vector types, code-byte packing, and the
// canonical adjacent-pair reduction tree.
#pragma once
#include "m2r_device.h"

namespace m2r {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int next_pow2(int v) { int r = 1; while (r < v) r <<= 1; return r; }

__device__ __forceinline__ float load_param(const void* p, int f32, int i) {
  return f32 ? ((const float*)p)[i] : h2f(((const uint16_t*)p)[i]);
}

// Sum of `v` with the value held by lane ^ (1 << level), for the butterfly
// levels 0..5 of a 64-lane wave.  Levels 0-1 use quad_perm DPP; levels 2-3
// use half-row / row mirrors, which pair each lane with a lane of the other
// aligned half-block (equal to the xor partner's value once every lane of a
// block holds the block sum); levels 4-5 use ds_bpermute lane exchanges.
// IEEE addition is commutative, so all lanes of a pair obtain identical bits.
template <int LEVEL>
__device__ __forceinline__ float butterfly_add(float v) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (LEVEL == 0) return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xF, 0xF, false));
  if constexpr (LEVEL == 1) return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xF, 0xF, false));
  if constexpr (LEVEL == 2) return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x141, 0xF, 0xF, false));
  if constexpr (LEVEL == 3) return v + __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(iv, 0x140, 0xF, 0xF, false));
  if constexpr (LEVEL == 4) return v + __shfl_xor(v, 16, 64);
  if constexpr (LEVEL == 5) return v + __shfl_xor(v, 32, 64);
  return v;
}

// Adjacent-pair binary tree over RZ = next_pow2(NZ) products, zero padded:
// level k adds elements (2i, 2i+1) of level k-1.  The butterfly computes
// exactly this tree.  Every lane receives the total.  `v0`/`v1` are the
// products at 2*lane and 2*lane+1 when RZ == 128, else `v0` is the product
// at `lane`.
template <int RZ>
__device__ __forceinline__ float wave_pair_tree(float v0, float v1) {
  float s = (RZ == 128) ? v0 + v1 : v0;
  constexpr int levels = (RZ >= 64) ? 6 : (RZ >= 32 ? 5 : (RZ >= 16 ? 4 : (RZ >= 8 ? 3 : (RZ >= 4 ? 2 : (RZ >= 2 ? 1 : 0)))));
  if constexpr (levels > 0) s = butterfly_add<0>(s);
  if constexpr (levels > 1) s = butterfly_add<1>(s);
  if constexpr (levels > 2) s = butterfly_add<2>(s);
  if constexpr (levels > 3) s = butterfly_add<3>(s);
  if constexpr (levels > 4) s = butterfly_add<4>(s);
  if constexpr (levels > 5) s = butterfly_add<5>(s);
  return s;
}

// Wave sum in any order (readout-only quantities).
__device__ __forceinline__ float wave_sum(float v) { return wave_pair_tree<64>(v, 0.f); }

// Dword-granular tile transfers split into a load phase (registers) and a
// store phase, so that all of a wave's global loads can be in flight before
// the first wait.  KW = dwords per lane = ceil(16 * W / 64).
template <int W>
struct TileRegs { uint32_t r[(16 * W + 63) / 64]; };

template <int W>
__device__ __forceinline__ void tile_load(TileRegs<W>& t, const uint8_t* g, int row0, int nvalid, int lane) {
  const uint32_t* src = (const uint32_t*)(g + (size_t)row0 * W);
  const int ndw = nvalid * W / 4;
#pragma unroll
  for (int k = 0; k < (16 * W + 63) / 64; ++k) {
    int i = k * 64 + lane;
    t.r[k] = (i < ndw) ? src[i] : 0u;
  }
}

template <int W>
__device__ __forceinline__ void tile_store_lds(const TileRegs<W>& t, uint8_t* lds, int nvalid, int lane) {
  uint32_t* dst = (uint32_t*)lds;
  const int ndw = nvalid * W / 4;
#pragma unroll
  for (int k = 0; k < (16 * W + 63) / 64; ++k) {
    int i = k * 64 + lane;
    if (i < ndw) dst[i] = t.r[k];
  }
}

// Reads W (even) bytes at lds[off .. off+W) (off even) as little-endian
// words: aligned dword reads plus one funnel shift per word.  The tile keeps
// 4 bytes of slack so the last dword read stays inside the allocation.
template <int W>
__device__ __forceinline__ void lds_read_row(const uint8_t* lds, int off, uint32_t (&w)[(W + 3) / 4]) {
  constexpr int NW = (W + 3) / 4;
  const uint32_t* d = (const uint32_t*)(lds + (off & ~3));
  const uint32_t sh = (uint32_t)(off & 3) * 8u;
  uint32_t v[NW + 1];
#pragma unroll
  for (int i = 0; i <= NW; ++i) v[i] = d[i];
#pragma unroll
  for (int i = 0; i < NW; ++i) w[i] = __builtin_amdgcn_alignbit(v[i + 1], v[i], sh);
}

template <int W>
__device__ __forceinline__ void lds_write_row(uint8_t* lds, int off, const uint32_t (&w)[(W + 3) / 4]) {
  uint16_t* h = (uint16_t*)(lds + off);
#pragma unroll
  for (int i = 0; i < (W + 3) / 4; ++i) {
    h[2 * i] = (uint16_t)(w[i] & 0xFFFFu);
    if (2 * i + 1 < W / 2) h[2 * i + 1] = (uint16_t)(w[i] >> 16);
  }
}

// Wave-cooperative copy of the wave's rows of one SoA field (W bytes per
// row, W even) between global memory and LDS.  Dword transfers when both the
// start and the length are dword multiples (always the case for even P),
// 16-bit transfers otherwise.  Trip counts are compile-time.
template <int W>
__device__ __forceinline__ void wave_copy_in(uint8_t* lds, const uint8_t* g, int row0, int nvalid, int lane) {
  const size_t start = (size_t)row0 * W;
  const int nbytes = nvalid * W;
  if (((start | (size_t)nbytes) & 3) == 0) {
    const uint32_t* src = (const uint32_t*)(g + start);
    uint32_t* dst = (uint32_t*)lds;
#pragma unroll
    for (int k = 0; k < (16 * W + 63) / 64; ++k) {
      int i = k * 64 + lane;
      if (i < nbytes / 4) dst[i] = src[i];
    }
  } else {
    const uint16_t* src = (const uint16_t*)(g + start);
    uint16_t* dst = (uint16_t*)lds;
#pragma unroll
    for (int k = 0; k < (32 * W + 63) / 64; ++k) {
      int i = k * 64 + lane;
      if (i < nbytes / 2) dst[i] = src[i];
    }
  }
}

template <int W>
__device__ __forceinline__ void wave_copy_out(uint8_t* g, const uint8_t* lds, int row0, int nvalid, int lane) {
  const size_t start = (size_t)row0 * W;
  const int nbytes = nvalid * W;
  if (((start | (size_t)nbytes) & 3) == 0) {
    const uint32_t* src = (const uint32_t*)lds;
    uint32_t* dst = (uint32_t*)(g + start);
#pragma unroll
    for (int k = 0; k < (16 * W + 63) / 64; ++k) {
      int i = k * 64 + lane;
      if (i < nbytes / 4) dst[i] = src[i];
    }
  } else {
    const uint16_t* src = (const uint16_t*)lds;
    uint16_t* dst = (uint16_t*)(g + start);
#pragma unroll
    for (int k = 0; k < (32 * W + 63) / 64; ++k) {
      int i = k * 64 + lane;
      if (i < nbytes / 2) dst[i] = src[i];
    }
  }
}

// Byte k of a carried word as a float (exact); selected as v_cvt_f32_ubyteK.
__device__ __forceinline__ float ubyte_f(uint32_t w, int k) {
  return (float)((w >> (8 * k)) & 0xFFu);
}

// Packs the low bytes of four ints into one word (byte k <- q[k]).
__device__ __forceinline__ uint32_t pack4(int q0, int q1, int q2, int q3) {
  uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u);  // q0.b0, q1.b0
  uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x04000c0cu);  // q2.b0, q3.b0 in bytes 2,3
  return lo | hi;
}

}  // namespace m2r
