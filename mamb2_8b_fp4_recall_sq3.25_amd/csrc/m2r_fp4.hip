// FP4 (E2M1) weight decode to resident FP16, for gfx950.
//
// Semantics (mamba2_recall/fp4.py:100-103, 151-154, 225-250;
// docs/FP4_WEIGHT_V1_PROTOCOL.md "Normative FP4 representation"):
//   nibble c: magnitude lev[c & 7] with lev = [0, .5, 1, 1.5, 2, 3, 4, 6],
//   bit 3 is the sign; the low nibble of byte i is column 2i.
//   G16: w = half( f32( f32(lev*sign * f32(e4m3 block)) * global ) )
//   G64: w = half( f32(lev*sign * f32(f16 scale)) )
// lev*|block| has at most 6 significant bits, so it is exact in binary32 and
// the only roundings are the product with `global` and the binary16
// conversion, both round-to-nearest-even.  IEEE sign rules give the sign of
// zero results as sign(code) xor sign(block); the kernel reproduces that by
// computing the magnitude and xoring the two sign bits into the binary16 word.
//
// Work unit: 8 consecutive weights = one 32-bit code word and one 16-byte
// output vector.  A wave moves 256 B of codes and 1 KiB of FP16 per step,
// each a single contiguous wave-wide access.  Validation of the reference's
// ValueError conditions is folded into the same pass: any violation sets a
// bit in a device word with one atomic OR per offending wave.
#include "m2r_device.h"
#include "m2r_abi_util.h"

#include <atomic>

namespace m2r {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

enum : uint32_t {
  FP4_ERR_SCALE_NONFINITE = 1u,    // 'Invalid stored scale' (nonfinite)
  FP4_ERR_SCALE_NEGATIVE = 2u,     // 'Invalid stored scale' (negative)
  FP4_ERR_ZERO_SCALE_CODE = 4u,    // 'Nonzero code in a zero-scale group'
  FP4_ERR_DECODED_NONFINITE = 8u,  // 'Nonfinite decoded FP16 weights'
  FP4_ERR_PADDING = 16u,           // 'Nonzero final-group padding'
  FP4_ERR_GLOBAL = 32u,            // 'Global scale must be finite and positive'
};

// 2*lev[c] for c in 0..7 as bytes: {0,1,2,3} and {4,6,8,12}.
constexpr uint32_t LEV2_LO = 0x03020100u;
constexpr uint32_t LEV2_HI = 0x0C080604u;

// Decodes 8 nibbles of `cw` with magnitude multiplier `hb` (= |block|/2 for
// G16, |scale|/2 for G64) and global multiplier `gl` (1 is not used for G64:
// G64 has a single rounding, selected by USE_GLOBAL).  `zsign` is the sign bit
// of the block scale (only observable on zero products).
template <bool USE_GLOBAL>
__device__ __forceinline__ u32x4 decode8(uint32_t cw, float hb, float gl, uint32_t zsign, uint32_t& err) {
  // byte j of `sel` = (nibble j) & 7 for the low and high nibble of each byte
  uint32_t even = cw & 0x07070707u;              // nibbles 0,2,4,6 (low nibbles)
  uint32_t odd = (cw >> 4) & 0x07070707u;        // nibbles 1,3,5,7
  uint32_t le = __builtin_amdgcn_perm(LEV2_HI, LEV2_LO, even);
  uint32_t lo = __builtin_amdgcn_perm(LEV2_HI, LEV2_LO, odd);
  uint32_t out[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    float m0 = (float)((le >> (8 * k)) & 0xFFu) * hb;
    float m1 = (float)((lo >> (8 * k)) & 0xFFu) * hb;
    if (USE_GLOBAL) { m0 = m0 * gl; m1 = m1 * gl; }
    uint32_t h0 = f2h(m0), h1 = f2h(m1);
    err |= ((h0 & 0x7FFFu) >= 0x7C00u || (h1 & 0x7FFFu) >= 0x7C00u) ? FP4_ERR_DECODED_NONFINITE : 0u;
    uint32_t s0 = ((cw >> (8 * k + 3)) & 1u) ^ zsign;
    uint32_t s1 = ((cw >> (8 * k + 7)) & 1u) ^ zsign;
    out[k] = h0 | (s0 << 15) | (h1 << 16) | (s1 << 31);
  }
  return u32x4{out[0], out[1], out[2], out[3]};
}

__device__ __forceinline__ void report(uint32_t err, uint32_t* flag) {
  // one atomic per wave that saw a violation
  uint64_t any = __ballot(err != 0u);
  if (any) {
    uint32_t werr = err;
    for (int k = 1; k < 64; k <<= 1) werr |= __shfl_xor(werr, k, 64);
    if ((threadIdx.x & 63) == 0 && flag) atomicOr(flag, werr);
  }
}

// G16, cols % 16 == 0: unit u covers weights [8u, 8u+8) of the flattened
// matrix; its block scale byte is u/2.
template <int UPT, bool NT>
__global__ __launch_bounds__(256) void k_fp4_g16(const uint32_t* __restrict__ codes,
                                                 const uint8_t* __restrict__ scales,
                                                 const float* __restrict__ global_scale,
                                                 u32x4* __restrict__ out, int64_t n_units, uint32_t* flag) {
  const float gl = *global_scale;
  uint32_t err = (gl > 0.f && gl < __builtin_inff()) ? 0u : FP4_ERR_GLOBAL;
  const int64_t stride = (int64_t)gridDim.x * 256 * UPT;
  for (int64_t base = (int64_t)blockIdx.x * 256 * UPT; base < n_units; base += stride) {
    uint32_t cw[UPT];
    uint32_t sb[UPT];
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      int64_t u = base + k * 256 + threadIdx.x;
      cw[k] = u < n_units ? __builtin_nontemporal_load(codes + u) : 0u;
      sb[k] = u < n_units ? scales[u >> 1] : 0u;
    }
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      int64_t u = base + k * 256 + threadIdx.x;
      if (u >= n_units) continue;
      uint32_t s = sb[k];
      uint32_t mag = s & 0x7Fu;
      err |= (mag == 0x7Fu) ? FP4_ERR_SCALE_NONFINITE : 0u;
      err |= ((s & 0x80u) && mag != 0u) ? FP4_ERR_SCALE_NEGATIVE : 0u;
      // a zero block may only hold codes 0 and 8 (both magnitudes zero)
      err |= (mag == 0u && (cw[k] & 0x77777777u) != 0u) ? FP4_ERR_ZERO_SCALE_CODE : 0u;
      float hb = e4m3_byte_to_f32<0>(mag) * 0.5f;   // FP8 instruction (0x7F: NaN, flagged above)
      u32x4 v = decode8<true>(cw[k], hb, gl, s >> 7, err);
      if constexpr (NT) __builtin_nontemporal_store(v, out + u);
      else out[u] = v;
    }
  }
  report(err, flag);
}

// G16 over whole blocks of 1024 units, wide loads: thread t of workgroup w
// decodes the four consecutive units 4(256 w + t) .. +3 from one 16-byte code
// load and one 2-byte load of their two block scales, stages the four 16-byte
// results in LDS and stores them transposed, so that every store instruction
// of a wave is again a contiguous 1 KiB (four units per lane stored directly
// would leave each instruction a 16-byte stripe every 64 bytes: partial-line
// writes, several times slower).  Needs 16-byte aligned codes and 2-byte
// aligned scales; the same values and error bits as k_fp4_g16.
__global__ __launch_bounds__(256) void k_fp4_g16_wide(const u32x4* __restrict__ codes,
                                                      const uint16_t* __restrict__ scales,
                                                      const float* __restrict__ global_scale,
                                                      u32x4* __restrict__ out, uint32_t* flag) {
  __shared__ u32x4 stage[1024];
  const float gl = *global_scale;
  uint32_t err = (gl > 0.f && gl < __builtin_inff()) ? 0u : FP4_ERR_GLOBAL;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const u32x4 c4 = __builtin_nontemporal_load(codes + t);
  const uint32_t s2 = scales[t];   // block scales of units 4t, 4t+1 (low byte) and 4t+2, 4t+3
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t cw = c4[k], s = (s2 >> (8 * (k >> 1))) & 0xFFu;
    const uint32_t mag = s & 0x7Fu;
    err |= (mag == 0x7Fu) ? FP4_ERR_SCALE_NONFINITE : 0u;
    err |= ((s & 0x80u) && mag != 0u) ? FP4_ERR_SCALE_NEGATIVE : 0u;
    err |= (mag == 0u && (cw & 0x77777777u) != 0u) ? FP4_ERR_ZERO_SCALE_CODE : 0u;
    const float hb = e4m3_byte_to_f32<0>(mag) * 0.5f;
    stage[4 * threadIdx.x + k] = decode8<true>(cw, hb, gl, s >> 7, err);
  }
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * 1024;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    __builtin_nontemporal_store(stage[k * 256 + threadIdx.x], out + base + k * 256 + threadIdx.x);
  report(err, flag);
}

// G64 over whole blocks of 1024 units, the layout of k_fp4_g16_wide: the four
// units of a thread share one FP16 scale (64 weights = 8 units); 16-byte
// aligned codes, 2-byte aligned scales.
__global__ __launch_bounds__(256) void k_fp4_g64_wide(const u32x4* __restrict__ codes,
                                                      const uint16_t* __restrict__ scales, u32x4* __restrict__ out,
                                                      uint32_t* flag) {
  __shared__ u32x4 stage[1024];
  uint32_t err = 0u;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const u32x4 c4 = __builtin_nontemporal_load(codes + t);
  const uint32_t s = scales[t >> 1];
  const uint32_t mag = s & 0x7FFFu;
  err |= (mag >= 0x7C00u) ? FP4_ERR_SCALE_NONFINITE : 0u;
  err |= ((s & 0x8000u) && mag != 0u) ? FP4_ERR_SCALE_NEGATIVE : 0u;
  const float hb = h2f((uint16_t)mag) * 0.5f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    err |= (mag == 0u && (c4[k] & 0x77777777u) != 0u) ? FP4_ERR_ZERO_SCALE_CODE : 0u;
    stage[4 * threadIdx.x + k] = decode8<false>(c4[k], hb, 1.0f, s >> 15, err);
  }
  __syncthreads();
  const int64_t base = (int64_t)blockIdx.x * 1024;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    __builtin_nontemporal_store(stage[k * 256 + threadIdx.x], out + base + k * 256 + threadIdx.x);
  report(err, flag);
}

// G64, cols % 64 == 0: unit u uses the FP16 scale u/8; one rounding.
template <int UPT>
__global__ __launch_bounds__(256) void k_fp4_g64(const uint32_t* __restrict__ codes,
                                                 const uint16_t* __restrict__ scales,
                                                 u32x4* __restrict__ out, int64_t n_units, uint32_t* flag) {
  uint32_t err = 0u;
  const int64_t stride = (int64_t)gridDim.x * 256 * UPT;
  for (int64_t base = (int64_t)blockIdx.x * 256 * UPT; base < n_units; base += stride) {
    uint32_t cw[UPT];
    uint32_t sb[UPT];
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      int64_t u = base + k * 256 + threadIdx.x;
      cw[k] = u < n_units ? __builtin_nontemporal_load(codes + u) : 0u;
      sb[k] = u < n_units ? scales[u >> 3] : 0u;
    }
#pragma unroll
    for (int k = 0; k < UPT; ++k) {
      int64_t u = base + k * 256 + threadIdx.x;
      if (u >= n_units) continue;
      uint32_t s = sb[k];
      uint32_t mag = s & 0x7FFFu;
      err |= (mag >= 0x7C00u) ? FP4_ERR_SCALE_NONFINITE : 0u;
      err |= ((s & 0x8000u) && mag != 0u) ? FP4_ERR_SCALE_NEGATIVE : 0u;
      err |= (mag == 0u && (cw[k] & 0x77777777u) != 0u) ? FP4_ERR_ZERO_SCALE_CODE : 0u;
      float hb = h2f((uint16_t)mag) * 0.5f;
      u32x4 v = decode8<false>(cw[k], hb, 1.0f, s >> 15, err);
      __builtin_nontemporal_store(v, out + u);
    }
  }
  report(err, flag);
}

// Generic path for widths that are not a multiple of the group: one thread
// per (row, group); padding codes must be zero (fp4.py:245).
template <int GROUP>
__global__ __launch_bounds__(256) void k_fp4_padded(const uint8_t* __restrict__ packed, const void* __restrict__ scales,
                                                    const float* __restrict__ global_scale, uint16_t* __restrict__ out,
                                                    int64_t rows, int64_t cols, uint32_t* flag) {
  const int64_t groups = (cols + GROUP - 1) / GROUP;
  const int64_t padded = groups * GROUP;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t err = 0u;
  float gl = 1.0f;
  if (GROUP == 16) {
    gl = *global_scale;
    err |= (gl > 0.f && gl < __builtin_inff()) ? 0u : FP4_ERR_GLOBAL;
  }
  if (idx < rows * groups) {
    const int64_t r = idx / groups, q = idx - r * groups;
    uint32_t s, mag, zsign;
    float hb;
    if (GROUP == 16) {
      s = ((const uint8_t*)scales)[idx];
      mag = s & 0x7Fu; zsign = s >> 7;
      err |= (mag == 0x7Fu) ? FP4_ERR_SCALE_NONFINITE : 0u;
      hb = e4m3_to_f32(mag) * 0.5f;
    } else {
      s = ((const uint16_t*)scales)[idx];
      mag = s & 0x7FFFu; zsign = s >> 15;
      err |= (mag >= 0x7C00u) ? FP4_ERR_SCALE_NONFINITE : 0u;
      hb = h2f((uint16_t)mag) * 0.5f;
    }
    err |= (zsign && mag != 0u) ? FP4_ERR_SCALE_NEGATIVE : 0u;
    const uint8_t* row = packed + r * (padded / 2);
    for (int j = 0; j < GROUP; ++j) {
      int64_t c = q * GROUP + j;
      uint32_t code = (row[c >> 1] >> (4 * (c & 1))) & 15u;
      if (c >= cols) {
        err |= code ? FP4_ERR_PADDING : 0u;
        continue;
      }
      err |= (mag == 0u && (code & 7u)) ? FP4_ERR_ZERO_SCALE_CODE : 0u;
      uint32_t lev2 = (__builtin_amdgcn_perm(LEV2_HI, LEV2_LO, code & 7u)) & 0xFFu;
      float m = (float)lev2 * hb;
      if (GROUP == 16) m = m * gl;
      uint32_t hbits = f2h(m);
      err |= ((hbits & 0x7FFFu) >= 0x7C00u) ? FP4_ERR_DECODED_NONFINITE : 0u;
      out[r * cols + c] = (uint16_t)(hbits | ((((code >> 3) & 1u) ^ zsign) << 15));
    }
  }
  report(err, flag);
}

static int grid_for(int64_t n_units, int upt, int64_t cap) {
  int64_t per_block = 256LL * upt;
  int64_t blocks = (n_units + per_block - 1) / per_block;
  if (cap > 0 && blocks > cap) blocks = cap;   // the grid-stride loop covers the rest
  if (blocks < 1) blocks = 1;
  if (blocks > 0x7FFFFFFF) blocks = 0x7FFFFFFF;
  return (int)blocks;
}

// G16 decode shape forced through m2r_set_fp4_decode_shape (0 = automatic):
// units per thread, grid cap in workgroups, non-temporal stores.
static std::atomic<int> g_fp4_upt{0}, g_fp4_cap{0}, g_fp4_nt{1};

template <int UPT>
static void launch_g16(bool nt, dim3 grid, hipStream_t stream, const uint32_t* codes, const uint8_t* scales,
                       const float* gl, u32x4* out, int64_t n_units, uint32_t* flag) {
  if (nt) hipLaunchKernelGGL((k_fp4_g16<UPT, true>), grid, dim3(256), 0, stream, codes, scales, gl, out, n_units, flag);
  else hipLaunchKernelGGL((k_fp4_g16<UPT, false>), grid, dim3(256), 0, stream, codes, scales, gl, out, n_units, flag);
}

}  // namespace m2r

using namespace m2r;

extern "C" int m2r_fp4_decode_g16(const uint8_t* packed, const uint8_t* e4m3_scales, const float* global_scale,
                                  void* out_f16, int64_t rows, int64_t cols, uint32_t* err_flag, hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return m2r_fail("fp4 g16: non-positive shape");
  if (cols % 16 == 0) {
    const int64_t n_units = rows * cols / 8;
    const int forced = g_fp4_upt.load(std::memory_order_relaxed);
    const int upt = forced ? forced : 4;
    // per-unit kernel: four units per thread, one pass (no grid cap),
    // non-temporal stores: the fastest of 1/2/4/8 units x caps
    // 2048/4096/16384/none x store policies on the full 8B weight set
    const int64_t cap = forced ? g_fp4_cap.load(std::memory_order_relaxed) : 0;
    const bool nt = forced ? g_fp4_nt.load(std::memory_order_relaxed) != 0 : true;
    const uint32_t* codes = (const uint32_t*)packed;
    u32x4* out = (u32x4*)out_f16;
    // automatic: whole blocks of 1024 units with the wide-load kernel, the
    // rest (fewer than 1024 units) with the per-unit kernel
    const int64_t n_wide = forced || ((uintptr_t)packed & 15) || ((uintptr_t)e4m3_scales & 1) ? 0 : n_units / 1024 * 1024;
    if (n_wide > 0) {
      if (n_wide / 1024 > 0x7FFFFFFF) return m2r_fail("fp4 g16: matrix too large");
      hipLaunchKernelGGL(k_fp4_g16_wide, dim3((unsigned)(n_wide / 1024)), dim3(256), 0, stream, (const u32x4*)packed,
                         (const uint16_t*)e4m3_scales, global_scale, out, err_flag);
      if (n_wide == n_units) return m2r_check(hipGetLastError(), "fp4 g16 launch");
      codes += n_wide;
      e4m3_scales += n_wide / 2;
      out += n_wide;
    }
    const int64_t n_rest = n_units - n_wide;
    const dim3 grid(grid_for(n_rest, upt, cap));
    if (upt == 1) launch_g16<1>(nt, grid, stream, codes, e4m3_scales, global_scale, out, n_rest, err_flag);
    else if (upt == 2) launch_g16<2>(nt, grid, stream, codes, e4m3_scales, global_scale, out, n_rest, err_flag);
    else if (upt == 8) launch_g16<8>(nt, grid, stream, codes, e4m3_scales, global_scale, out, n_rest, err_flag);
    else launch_g16<4>(nt, grid, stream, codes, e4m3_scales, global_scale, out, n_rest, err_flag);
  } else {
    int64_t groups = (cols + 15) / 16;
    int64_t n = rows * groups;
    hipLaunchKernelGGL((k_fp4_padded<16>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, packed,
                       (const void*)e4m3_scales, global_scale, (uint16_t*)out_f16, rows, cols, err_flag);
  }
  return m2r_check(hipGetLastError(), "fp4 g16 launch");
}

extern "C" int m2r_fp4_decode_g64(const uint8_t* packed, const void* f16_scales, void* out_f16, int64_t rows,
                                  int64_t cols, uint32_t* err_flag, hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return m2r_fail("fp4 g64: non-positive shape");
  if (cols % 64 == 0) {
    const int64_t n_units = rows * cols / 8;
    constexpr int UPT = 4;
    const bool forced = g_fp4_upt.load(std::memory_order_relaxed) != 0;
    const int64_t cap = forced ? g_fp4_cap.load(std::memory_order_relaxed) : 0;
    const uint32_t* codes = (const uint32_t*)packed;
    const uint16_t* sc = (const uint16_t*)f16_scales;
    u32x4* out = (u32x4*)out_f16;
    // automatic: whole blocks of 1024 units with the wide-load kernel, the rest per unit
    const int64_t n_wide = forced || ((uintptr_t)packed & 15) || ((uintptr_t)f16_scales & 1) ? 0 : n_units / 1024 * 1024;
    if (n_wide > 0) {
      if (n_wide / 1024 > 0x7FFFFFFF) return m2r_fail("fp4 g64: matrix too large");
      hipLaunchKernelGGL(k_fp4_g64_wide, dim3((unsigned)(n_wide / 1024)), dim3(256), 0, stream, (const u32x4*)packed,
                         sc, out, err_flag);
      if (n_wide == n_units) return m2r_check(hipGetLastError(), "fp4 g64 launch");
      codes += n_wide;
      sc += n_wide / 8;
      out += n_wide;
    }
    const int64_t n_rest = n_units - n_wide;
    hipLaunchKernelGGL((k_fp4_g64<UPT>), dim3(grid_for(n_rest, UPT, cap)), dim3(256), 0, stream, codes, sc, out, n_rest,
                       err_flag);
  } else {
    int64_t groups = (cols + 63) / 64;
    int64_t n = rows * groups;
    hipLaunchKernelGGL((k_fp4_padded<64>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, packed,
                       f16_scales, (const float*)nullptr, (uint16_t*)out_f16, rows, cols, err_flag);
  }
  return m2r_check(hipGetLastError(), "fp4 g64 launch");
}

extern "C" int m2r_set_fp4_decode_shape(int units_per_thread, int max_blocks, int nontemporal) {
  const int u = units_per_thread;
  if (!(u == 0 || u == 1 || u == 2 || u == 4 || u == 8) || max_blocks < 0)
    return m2r_fail("fp4 decode shape: units per thread 1, 2, 4 or 8 (0 = automatic), max_blocks >= 0");
  g_fp4_cap.store(max_blocks, std::memory_order_relaxed);
  g_fp4_nt.store(nontemporal ? 1 : 0, std::memory_order_relaxed);
  g_fp4_upt.store(u, std::memory_order_relaxed);
  return 0;
}
