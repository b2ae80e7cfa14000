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
// block holds the block sum); levels 4-5 use the row-swap permutes.
// IEEE addition is commutative, so all lanes of a pair obtain identical bits.
// Levels 0-3 are written as DPP updates of a zero with every row and bank
// enabled and out-of-range sources reading zero: every source lane of these
// patterns lies in its own row, so the value is the moved one, and the form
// lets the compiler fold the move into the add (one v_add_f32 with a DPP
// operand per level instead of a move and an add).
template <int LEVEL>
__device__ __forceinline__ float butterfly_add(float v) {
  const int iv = __builtin_bit_cast(int, v);
  if constexpr (LEVEL == 0) return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, true));
  if constexpr (LEVEL == 1) return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, true));
  if constexpr (LEVEL == 2) return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, true));
  if constexpr (LEVEL == 3) return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, iv, 0x140, 0xF, 0xF, true));
  // levels 4-5: v_permlane16_swap / v_permlane32_swap of two copies of v
  // leave, in every lane, the values of the lower and the upper half-block
  // of its aligned 32- / 64-lane block; their sum is v + v[lane ^ 16 (32)]
  if constexpr (LEVEL == 4) {
    const auto r = __builtin_amdgcn_permlane16_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  }
  if constexpr (LEVEL == 5) {
    const auto r = __builtin_amdgcn_permlane32_swap(iv, iv, false, false);
    return __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  }
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

// Direct global -> LDS transfers (LDS DMA): every lane reads SIZE bytes at
// its own global address; they land at LDS byte address lds + SIZE * lane.
// Issued as inline assembly on purpose: the compiler then neither counts
// them in its own vmcnt bookkeeping nor guards later LDS stores with waits
// for them, so the callers own the ordering.  A caller must (1) let every
// compiler-visible global load complete before issuing transfers (otherwise
// the compiler's wait for such a load would also wait for the transfers),
// and (2) wait with wait_vmcnt before reading the destination.  M0, which
// carries the LDS address (wave-uniform by contract), is an operand of the
// statement: the compiler writes it (once for a run of transfers with the
// same base) and knows it changed.  The leading s_nop is the wait state
// between an M0 write and an LDS transfer that reads it.
// The LDS address of a generic pointer into LDS is its low 32 bits (the
// high half is the shared aperture's base), taken here without the
// address-space cast's null test.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return (uint32_t)(uintptr_t)p;
}
__device__ __forceinline__ void lds_dma_b32(const void* g, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

// Raw buffer resource over `bytes` bytes at `base` (gfx9-family dword 3:
// 32-bit raw data, no swizzle): accesses at offsets >= bytes are dropped
// (stores) or read 0 (loads) by the hardware range check.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_buffer(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

// The 16-byte form: lane l's 16 bytes at g land at M0 + 16 l.  NT: marked
// non-temporal (a launch whose state is too large for the L2 reads every
// state byte once); without it the lines stay in the L2 for the next launch
// of the same layer, which hits there when the state of every layer fits.
template <bool NT = true>
__device__ __forceinline__ void lds_dma_b128(const void* g, uint32_t lds) {
  if constexpr (NT)
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
  else
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}
// The same with an instruction offset, which moves the global and the LDS
// address alike: lane l's 16 bytes at g + IMM land at lds + IMM + 16 l, so
// transfers into one tile share M0.
template <int IMM, bool NT = true>
__device__ __forceinline__ void lds_dma_b128_imm(const void* g, uint32_t lds) {
  static_assert(IMM >= 0 && IMM < 4096, "instruction offset range");
  if constexpr (NT)
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off offset:%2 nt" ::"v"(g),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)), "n"(IMM)
                 : "memory");
  else
    asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off offset:%2" ::"v"(g),
                 "{m0}"(__builtin_amdgcn_readfirstlane(lds)), "n"(IMM)
                 : "memory");
}

// 16-byte transfers of one SoA field of a 64-row slot (64 * W bytes at
// g + row0 * W) to or from the slot's LDS tile: one vector memory operation
// per started 1 KiB chunk.
constexpr int chunk_ops(int W) { return (64 * W + 1023) / 1024; }

// Global -> LDS.  Lanes past the field stay idle; lanes past the nvalid valid
// rows re-read the last valid chunk, whose copy lands in rows nobody reads.
// Requires g + row0 * W to be 16-byte aligned and nvalid * W a multiple of
// 16.  Issues exactly chunk_ops(W) operations.
// field_dma16_at takes the LDS byte address itself.
template <int W>
__device__ __forceinline__ void field_dma16_at(uint32_t l0, const uint8_t* g, int row0, int nvalid, int lane) {
  constexpr int FB = 64 * W;
  const uint8_t* base = g + (size_t)row0 * W;
  const int last = nvalid * W - 16;
#pragma unroll
  for (int k = 0; k < chunk_ops(W); ++k) {
    const int o = k * 1024 + 16 * lane;
    if (k * 1024 + 1024 <= FB || o < FB) lds_dma_b128(base + min(o, last), l0 + 1024 * k);
  }
}
template <int W>
__device__ __forceinline__ void field_dma16(uint8_t* lds, const uint8_t* g, int row0, int nvalid, int lane) {
  constexpr int FB = 64 * W;
  const uint8_t* base = g + (size_t)row0 * W;
  const uint32_t l0 = lds_address(lds);
  const int last = nvalid * W - 16;
#pragma unroll
  for (int k = 0; k < chunk_ops(W); ++k) {
    const int o = k * 1024 + 16 * lane;
    if (k * 1024 + 1024 <= FB || o < FB) lds_dma_b128(base + min(o, last), l0 + 1024 * k);
  }
}

// The same transfers into a slot tile whose LDS base `tile` is M0 for every
// field of the slot: the field sits at tile byte offset O and chunk k goes
// by instruction offset O + 1024 k.
template <int W, int O, bool NT = true, int K = 0>
__device__ __forceinline__ void field_dma16_tile(uint32_t tile, const uint8_t* g, int row0, int nvalid, int lane) {
  static_assert(chunk_ops(W) <= 4, "fields of at most 4 KiB per slot");
  if constexpr (K < chunk_ops(W)) {
    constexpr int FB = 64 * W, IMM = O + 1024 * K;
    const uint8_t* base = g + (size_t)row0 * W;
    const int o = K * 1024 + 16 * lane;
    if (K * 1024 + 1024 <= FB || o < FB) lds_dma_b128_imm<IMM, NT>(base + (min(o, nvalid * W - 16) - IMM), tile);
    field_dma16_tile<W, O, NT, K + 1>(tile, g, row0, nvalid, lane);
  }
}
// NF two-byte fields of a slot (128 bytes each: f0, f1, f2), which sit back
// to back in the tile from byte offset O, in one transfer: lane l moves
// 16 bytes of field l / 8 (lanes past the nvalid valid rows re-read the
// field's last valid chunk, which lands in rows nobody reads).  Requires
// nvalid % 8 == 0.
template <int NF, int O, bool NT = true>
__device__ __forceinline__ void scale_fields_dma16_tile(uint32_t tile, const uint8_t* f0, const uint8_t* f1,
                                                        const uint8_t* f2, int row0, int nvalid, int lane) {
  static_assert(NF >= 1 && NF <= 3, "one to three fields");
  const int f = lane >> 3, c = min(lane & 7, nvalid / 8 - 1);
  const uint8_t* fb = f == 0 ? f0 : (f == 1 ? f1 : f2);
  if (lane < 8 * NF) lds_dma_b128_imm<O, NT>(fb + (size_t)row0 * 2 + (16 * c - O), tile);
}

// Cache policies of the state and output stores.  STORE_THROUGH: device
// scope (sc1) and non-temporal, so they are written through during the
// launch instead of staying dirty in the issuing XCD's L2 until the
// end-of-kernel writeback.  STORE_DEVICE: device scope only (written
// through, the lines kept in the L2), for launches whose state of every
// layer fits the L2s.
constexpr int STORE_THROUGH = 16 | 2, STORE_DEVICE = 16;

// LDS -> global in two halves, so that a caller reads every field of a slot
// before its first store (the compiler does not move LDS reads above a
// buffer store, and each read-wait-store round trip is an LDS latency):
// field_read16 reads the chunk_ops(W) 16-byte chunks of lane `lane`;
// field_write16 stores them with unguarded buffer stores whose range check
// drops everything past nvalid * W bytes (whole chunks, under the same
// alignment requirements) and issues exactly chunk_ops(W) store
// instructions.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <int W>
__device__ __forceinline__ void field_read16(const uint8_t* lds, int lane, u32x4* v) {
  constexpr int FB = 64 * W;
#pragma unroll
  for (int k = 0; k < chunk_ops(W); ++k) v[k] = *(const u32x4*)(lds + min(k * 1024 + 16 * lane, FB - 16));
}
template <int W, int CP = STORE_THROUGH>
__device__ __forceinline__ void field_write16(uint8_t* g, const u32x4* v, int row0, int nvalid, int lane) {
  const __amdgpu_buffer_rsrc_t rsrc = raw_buffer(g + (size_t)row0 * W, nvalid * W);
#pragma unroll
  for (int k = 0; k < chunk_ops(W); ++k)
    __builtin_amdgcn_raw_buffer_store_b128(v[k], rsrc, k * 1024 + 16 * lane, 0, CP);
}

// LDS DMA of one SoA field of a 64-row slot: 64 * W bytes at g + row0 * W
// land at lds[0 .. 64 * W).  W / 4 dword transfers (64 lanes x 4 bytes)
// plus, for W % 4 == 2, one transfer by lanes 0..31 cover the field exactly
// (narrower transfers still advance the LDS address by 4 bytes per lane, so
// they cannot pack 16-bit elements).  Lanes past the nvalid valid rows
// re-read the last valid dword; their copies land in rows nobody reads.
// Every transfer has active lanes, so a call issues exactly dma_ops(W)
// vector memory operations.  Requires row0 * W and nvalid * W to be dword
// multiples.
constexpr int dma_ops(int W) { return W / 4 + (W % 4 ? 1 : 0); }

// Same transfer with a wave-uniform 64-bit base in SGPRs, a per-lane 32-bit
// offset and a compile-time instruction offset: no per-transfer VALU work.
// The instruction offset moves the global and the LDS address alike (LDS
// destination = M0 + IMM + 4 * lane), so M0 stays at the field base.
template <int IMM>
__device__ __forceinline__ void lds_dma_b32_sbase(uint32_t voff, const void* sbase, uint32_t lds) {
  static_assert(IMM >= 0 && IMM < 4096, "instruction offset range");
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1 offset:%3" ::"v"(voff), "s"(sbase),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds)), "n"(IMM)
               : "memory");
}

__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// full 64-row field: transfer K.. of N with offsets 256 * K
template <int K, int N>
struct FullFieldDma {
  static __device__ __forceinline__ void run(uint32_t lane4, const void* base, uint32_t l0) {
    if constexpr (K < N) {
      lds_dma_b32_sbase<256 * K>(lane4, base, l0);
      FullFieldDma<K + 1, N>::run(lane4, base, l0);
    }
  }
};

template <int W>
__device__ __forceinline__ void field_dma(uint8_t* lds, const uint8_t* g, int row0, int nvalid, int lane) {
  static_assert(W % 2 == 0, "even field widths");
  const uint8_t* base = (const uint8_t*)uniform_ptr(g + (size_t)row0 * W);
  const uint32_t l0 = lds_address(lds);
  if (nvalid == 64) {   // every row valid: constant offsets, nothing to clamp
    const uint32_t lane4 = 4u * (uint32_t)lane;
    FullFieldDma<0, W / 4>::run(lane4, base, l0);
    if constexpr (W % 4 != 0) {
      if (lane < 32) lds_dma_b32_sbase<256 * (W / 4)>(lane4, base, l0);
    }
    return;
  }
  const int last_dw = nvalid * W / 4 - 1;
#pragma unroll
  for (int k = 0; k < W / 4; ++k) lds_dma_b32(base + 4 * min(k * 64 + lane, last_dw), l0 + 256 * k);
  if constexpr (W % 4 != 0) {
    if (lane < 32) lds_dma_b32(base + 4 * min((W / 4) * 64 + lane, last_dw), l0 + 256 * (W / 4));
  }
}


// Stores one SoA field of a 64-row slot staged in LDS (64 * W bytes) to
// g + row0 * W, nvalid rows: all LDS reads first, then unguarded dword
// buffer stores whose range check drops everything past nvalid * W bytes.
// Requires row0 * W and nvalid * W to be dword multiples.
template <int W>
__device__ __forceinline__ void field_store(uint8_t* g, const uint8_t* lds, int row0, int nvalid, int lane) {
  constexpr int NW = (16 * W + 63) / 64;
  const uint32_t* src = (const uint32_t*)lds;
  const __amdgpu_buffer_rsrc_t rsrc = raw_buffer(g + (size_t)row0 * W, nvalid * W);
  uint32_t v[NW];
#pragma unroll
  for (int k = 0; k < NW; ++k) v[k] = src[(k * 64 + 64 <= 16 * W) ? k * 64 + lane : min(k * 64 + lane, 16 * W - 1)];
#pragma unroll
  // the chunk offset goes into the range-checked offset (the scalar offset
  // operand is outside the raw-buffer range check)
  for (int k = 0; k < NW; ++k) __builtin_amdgcn_raw_buffer_store_b32(v[k], rsrc, 4 * (k * 64 + lane), 0, 0);
}

// Waits until at most N vector memory operations of this wave are
// outstanding; also a compiler barrier for memory accesses.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
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

// Wave priority from the number of head slots the wave still has to step
// in this token (4 or more: highest).  Two workgroups share each CU, so each
// SIMD runs two waves; its issue arbitration otherwise favours the older
// wave, which runs ahead while the younger one finishes alone, a slot or more
// later, with no second wave to hide its latencies.  With the priority the
// wave that is behind wins the arbitration until it has caught up.
__device__ __forceinline__ void wave_priority_by_slots_left(int left) {
  if (left >= 4) __builtin_amdgcn_s_setprio(3);
  else if (left == 3) __builtin_amdgcn_s_setprio(2);
  else if (left == 2) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Orders a wave's LDS accesses across its lanes (the wave's own regions
// need no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// max(m, |a|, |b|) as one v_max3_f32 (IEEE maxNum: a quiet NaN operand is
// ignored, as fmaxf does).  Written out because the compiler otherwise
// canonicalizes each pinned operand first.
__device__ __forceinline__ float max3_abs(float m, float a, float b) {
  float r;
  asm("v_max3_f32 %0, %1, |%2|, |%3|" : "=v"(r) : "v"(m), "v"(a), "v"(b));
  return r;
}

}  // namespace m2r
