// Fused Mamba-2 selective-state step + per-token requantization of the packed
// 52-byte recurrent-state rows, for gfx950.
//
// One kernel template covers the three same-byte row formats of the
// reference:
//   MODE_LEGACY  sq3p25 16/64/48, quantized with the binary32 denominator
//                (mamba2_recall/state_codec.py:105-176, _sq_scan)
//   MODE_STORED  stored-scale INT8/INT4/zero tiers
//                (scripts/state_ppl_codec_v10.py:78-154, _tier_scan;
//                 scripts/state_ppl_codec_v6.py:83-195 stored_scale path)
//   MODE_RIDGE   INT8/INT4 tiers + two E4M3 latent coefficients + the static
//                zero-tier ridge predictor
//                (scripts/fp4_zero_predictor_codec_v1.py:76-236, _latent_scan
//                 and the einsum correction of scan())
//
// Mapping: one lane owns one state row r = (b, h, p); a wave owns 64
// consecutive p of one head; a workgroup owns WPB heads of the same B/C
// group.  The row's live coordinates (N8 + N4, compile-time) stay in VGPRs
// for all L tokens.  Packed SoA rows are staged through LDS so that every
// global access is a contiguous wave-wide transfer.  Per-token values shared
// by the group (permuted B/C, dt activation, B*dt, ridge correction, dead-tier
// dot products) are computed once per workgroup into LDS and read back as
// wave-uniform broadcasts.
#include "m2r_device.h"
#include "m2r_abi_util.h"
#include "m2r_tile.h"

#include <atomic>

namespace m2r {

enum { MODE_LEGACY = 0, MODE_STORED = 1, MODE_RIDGE = 2 };

struct StepArgs {
  const uint16_t* x;       // f16 [B, L, H, P]
  const uint16_t* dt;      // f16 [B, L, H]
  const float* A;          // f32 [H]
  const uint16_t* Bm;      // f16 [B, L, G, 128]
  const uint16_t* Cm;      // f16 [B, L, G, 128]
  const void* D;           // f16 or f32 [H]
  const void* dt_bias;     // f16 or f32 [H]
  const uint8_t* perm;     // u8 [G, 128]: packed lane n holds coordinate perm[g, n]
  const uint16_t* basis;   // f16 [G, NZ, 2]   (ridge)
  const uint16_t* lscale;  // f16 [G, 2]       (ridge)
  const uint16_t* pred;    // f16 [G, F, NZ]   (ridge), F = N8 + N4 + 2
  uint8_t* lo;             // u8 [rows, N8/2]  low nibbles of the INT8 tier
  uint8_t* hi;             // u8 [rows, N8/2]  high nibbles of the INT8 tier
  uint8_t* q4;             // u8 [rows, N4/2]  INT4 tier
  uint8_t* latent;         // e4m3 [rows, 2]   (ridge)
  uint16_t* s8;            // f16 [rows]
  uint16_t* s4;            // f16 [rows]
  uint16_t* y;             // f16 [B, L, H, P]
  int B, L, H, P, G;
  int d_f32, db_f32;
};

// Carried coordinates are held in an internal lane order that makes the
// conversion between the nibble planes and code bytes two bitfield inserts
// per four coordinates: within each tier, every full group of 8 packed lanes
// is ordered (0,2,4,6,1,3,5,7) and a final group of 4 is ordered (0,2,1,3).
// packed_lane<N8,N4>(j) is the packed lane of internal position j (< N8+N4);
// the zero tier keeps its natural order.
constexpr int tier_packed_of(int j, int T) {
  const int g = j / 8, k = j % 8;
  if (g * 8 + 8 <= T) return g * 8 + (k < 4 ? 2 * k : 2 * (k - 4) + 1);
  return g * 8 + (k < 2 ? 2 * k : 2 * (k - 2) + 1);
}
template <int N8, int N4>
__device__ __forceinline__ int packed_lane(int j) {
  return j < N8 ? tier_packed_of(j, N8) : (j < N8 + N4 ? N8 + tier_packed_of(j - N8, N4) : j);
}

// nibble-plane words -> carried code-byte words for one tier.
// INT8: lo/hi plane words (8 lanes per word); byte = (q + 128) = code ^ 0x80.
template <int N>
__device__ __forceinline__ void planes_to_bytes8(const uint32_t* wl, const uint32_t* wh, uint32_t* c) {
#pragma unroll
  for (int g = 0; g < (N + 7) / 8; ++g) {
    const uint32_t hb = wh[g] ^ 0x88888888u;                                   // bias via the high nibble
    const uint32_t e = (wl[g] & 0x0F0F0F0Fu) | ((hb << 4) & 0xF0F0F0F0u);
    const uint32_t o = ((wl[g] >> 4) & 0x0F0F0F0Fu) | (hb & 0xF0F0F0F0u);
    if (g * 8 + 8 <= N) { c[2 * g] = e; c[2 * g + 1] = o; }
    else c[2 * g] = (e & 0xFFFFu) | (o << 16);
  }
}
// INT4: q4 plane words; byte = (q + 8) = nibble ^ 8.
template <int N>
__device__ __forceinline__ void plane_to_bytes4(const uint32_t* wq, uint32_t* c) {
#pragma unroll
  for (int g = 0; g < (N + 7) / 8; ++g) {
    const uint32_t q = wq[g] ^ 0x88888888u;
    const uint32_t e = q & 0x0F0F0F0Fu, o = (q >> 4) & 0x0F0F0F0Fu;
    if (g * 8 + 8 <= N) { c[2 * g] = e; c[2 * g + 1] = o; }
    else c[2 * g] = (e & 0xFFFFu) | (o << 16);
  }
}
// carried bytes -> nibble-plane words (inverse of the two above)
template <int N>
__device__ __forceinline__ void bytes_to_planes8(const uint32_t* c, uint32_t* wl, uint32_t* wh) {
#pragma unroll
  for (int g = 0; g < (N + 7) / 8; ++g) {
    uint32_t e, o;
    if (g * 8 + 8 <= N) { e = c[2 * g]; o = c[2 * g + 1]; }
    else { e = c[2 * g] & 0xFFFFu; o = c[2 * g] >> 16; }
    wl[g] = (e & 0x0F0F0F0Fu) | ((o << 4) & 0xF0F0F0F0u);
    wh[g] = (((e >> 4) & 0x0F0F0F0Fu) | (o & 0xF0F0F0F0u)) ^ 0x88888888u;
  }
}
template <int N>
__device__ __forceinline__ void bytes_to_plane4(const uint32_t* c, uint32_t* wq) {
#pragma unroll
  for (int g = 0; g < (N + 7) / 8; ++g) {
    uint32_t e, o;
    if (g * 8 + 8 <= N) { e = c[2 * g]; o = c[2 * g + 1]; }
    else { e = c[2 * g] & 0xFFFFu; o = c[2 * g] >> 16; }
    wq[g] = ((e & 0x0F0F0F0Fu) | ((o << 4) & 0xF0F0F0F0u)) ^ 0x88888888u;
  }
}

// Per-token values shared by the workgroup (one B/C group, NH heads): the raw
// B/C rows and x, the permuted B and C, dt activation and decay per head, B*dt
// per head, the readout weights and the latent dot products.
template <int N8, int N4, int NZ, int MODE, int NH>
struct TokenShared {
  static constexpr int NL = N8 + N4;
  uint16_t raw[256];                                   // B row then C row of the group, original order
  uint16_t xr[NH * 64];                                // x of the NH heads, this P block
  alignas(16) float b[128];                            // internal order
  alignas(16) float c[128];
  alignas(16) float cp[MODE == MODE_RIDGE ? NL : 4];   // c + ridge correction of the live coordinates
  alignas(16) float bdt[NH][NL];                       // RN(b * dt) per head
  float dtv[NH], decay[NH];
  // 0: sum of b*c over all 128 coordinates (readout); 1, 2: dead-tier e0.c,
  // e1.c (readout); 3, 4: dead-tier e0.b, e1.b (canonical trees, exact);
  // 5, 6: ridge correction of the two latent coefficients (readout)
  float dots[8];
};

// Raw per-token inputs a thread loads one token ahead: its share of the
// group's B and C rows, x of the rows it owns in each of its HPW head slots,
// and, for the first NH threads, one head's dt and dt_bias bits.  Nothing is
// converted at load time, so no wait is needed until token_store.
template <int WPB, int HPW>
struct TokenRaw {
  static constexpr int NT = 64 * WPB;
  static constexpr int NBC = (256 + NT - 1) / NT;
  uint16_t bc[NBC];
  uint16_t xv[HPW];
  uint16_t dt, db_lo, db_hi;   // dt_bias: f16 bits, or the halves of f32 bits
};

template <int WPB, int HPW>
__device__ __forceinline__ void token_load(const StepArgs& a, TokenRaw<WPB, HPW>& r, int bt, int g, int h0,
                                           int pbase, int tid, int lane, int wave) {
  using R = TokenRaw<WPB, HPW>;
#pragma unroll
  for (int k = 0; k < R::NBC; ++k) {
    const int i = k * R::NT + tid;
    const uint16_t* src = (i < 128) ? a.Bm : a.Cm;
    r.bc[k] = (i < 256) ? src[((size_t)bt * a.G + g) * 128 + (i & 127)] : (uint16_t)0;
  }
  const int p = pbase + lane;
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int hh = k * WPB + wave;
    r.xv[k] = (p < a.P) ? a.x[((size_t)bt * a.H + h0 + hh) * a.P + p] : (uint16_t)0;
  }
  r.dt = r.db_lo = r.db_hi = 0;
  if (tid < WPB * HPW) {
    const int h = h0 + tid;
    const uint16_t* db = (const uint16_t*)a.dt_bias;
    r.dt = a.dt[(size_t)bt * a.H + h];
    r.db_lo = db[a.db_f32 ? 2 * h : h];
    r.db_hi = db[a.db_f32 ? 2 * h + 1 : h];
  }
}

template <int N8, int N4, int NZ, int MODE, int WPB, int HPW>
__device__ __forceinline__ void token_store(TokenShared<N8, N4, NZ, MODE, WPB * HPW>& sh,
                                            const TokenRaw<WPB, HPW>& r, float Ah, int db_f32, int tid, int lane,
                                            int wave) {
  using R = TokenRaw<WPB, HPW>;
#pragma unroll
  for (int k = 0; k < R::NBC; ++k) {
    const int i = k * R::NT + tid;
    if (i < 256) sh.raw[i] = r.bc[k];
  }
#pragma unroll
  for (int k = 0; k < HPW; ++k) sh.xr[(k * WPB + wave) * 64 + lane] = r.xv[k];
  if (tid < WPB * HPW) {
    const float db = db_f32 ? __builtin_bit_cast(float, (uint32_t)r.db_lo | ((uint32_t)r.db_hi << 16)) : h2f(r.db_lo);
    const float2 act = dt_activation(h2f(r.dt) + db, Ah);
    sh.dtv[tid] = act.x;
    sh.decay[tid] = act.y;
  }
}

// After token_store and a barrier: gather through the permutation, B*dt per
// head, readout weights and latent dot products; ends with a barrier.
template <int N8, int N4, int NZ, int MODE, int WPB, int HPW>
__device__ __forceinline__ void token_build(TokenShared<N8, N4, NZ, MODE, WPB * HPW>& sh, const uint8_t* s_perm,
                                            const float* s_basis, const uint16_t* s_pred, int tid, int lane,
                                            int wave) {
  constexpr int NL = N8 + N4, F = NL + 2, NT = 64 * WPB, NH = WPB * HPW;
  constexpr int RZ = next_pow2(NZ);
#pragma unroll
  for (int k = 0; k < (256 + NT - 1) / NT; ++k) {
    const int i = k * NT + tid;
    if (i < 256) {
      const int n = i & 127;   // internal position
      const float v = h2f(sh.raw[(i & 128) + (s_perm[packed_lane<N8, N4>(n)] & 127)]);
      if (i < 128) sh.b[n] = v; else sh.c[n] = v;
    }
  }
  __syncthreads();
  // compile-time trip counts: every LDS read of a loop is issued before the
  // first use, so each loop costs about one LDS latency
#pragma unroll
  for (int k = 0; k < (NH * NL + NT - 1) / NT; ++k) {
    const int i = k * NT + tid;
    if (i < NH * NL) {
      const int w = i / NL, n = i - w * NL;
      sh.bdt[w][n] = sh.b[n] * sh.dtv[w];
    }
  }
  if constexpr (MODE == MODE_RIDGE) {
    // corr[f] = sum_d C[dead d] * pred[g, f, d]: four threads per output,
    // interleaved d, combined inside the quad; live rows are folded into the
    // readout weight c + corr, latent rows kept apart (readout-only values)
#pragma unroll
    for (int k = 0; k < (4 * F + NT - 1) / NT; ++k) {
      const int idx = k * NT + tid;
      if (idx < 4 * F) {                            // whole quads take this branch together
        const int j = idx >> 2, part = idx & 3;     // internal feature position
        const int f = packed_lane<N8, N4>(j);       // predictor row (packed lane; latent rows last)
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < (NZ + 3) / 4; ++i) {
          const int d = part + 4 * i;
          if (d < NZ) acc = __builtin_fmaf(sh.c[NL + d], h2f(s_pred[f * NZ + d]), acc);
        }
        acc = butterfly_add<0>(acc);
        acc = butterfly_add<1>(acc);
        if (part == 0) {
          if (j < NL) sh.cp[j] = sh.c[j] + acc;
          else sh.dots[5 + (j - NL)] = acc;
        }
      }
    }
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      if (wave != k % WPB) continue;
      float t;
      if (k == 0) {
        t = wave_sum(sh.b[lane] * sh.c[lane] + sh.b[lane + 64] * sh.c[lane + 64]);
      } else {
        // dead-tier dot products: canonical adjacent-pair trees
        float v[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int d0 = (RZ == 128) ? 2 * lane + j : lane;
          const bool in = (RZ == 128 || j == 0) && d0 < NZ;
          const int d = in ? d0 : 0;
          const float bb = sh.b[NL + d], cc = sh.c[NL + d], e0 = s_basis[d], e1 = s_basis[NZ + d];
          const float pr = k == 1 ? e0 * cc : k == 2 ? e1 * cc : k == 3 ? e0 * bb : e1 * bb;
          v[j] = in ? pr : 0.f;
        }
        t = wave_pair_tree<RZ>(v[0], v[1]);
      }
      if (lane == 0) sh.dots[k] = t;
    }
  } else {
    if (wave == 0) {
      const float t = wave_sum(sh.b[lane] * sh.c[lane] + sh.b[lane + 64] * sh.c[lane + 64]);
      if (lane == 0) sh.dots[0] = t;
    }
  }
  __syncthreads();
}

// One tier of a row: update its N carried coordinates (biased code bytes in
// c[0 .. N/4)), accumulate the readout (prior * readout weight), then
// requantize with den = max(RN(amax / lim), 1e-8) and the stored (binary16)
// scale, writing the new codes back into c.  Returns the new stored scale.
// INT8: byte = q + 128, lim 127; INT4: byte = q + 8, lim 7.  Legacy mode
// quantizes with the binary32 denominator.
template <int N, bool INT8, int MODE>
__device__ __forceinline__ float tier_step(uint32_t* c, float sc, float decay, float x, const f32x4* bdt4,
                                           const f32x4* cw4, float& acc) {
  constexpr float BIAS = INT8 ? 128.0f : 8.0f;
  constexpr float LIM = INT8 ? 127.0f : 7.0f;
  constexpr float TOP = INT8 ? QTOP127 : QTOP7;
  const float nb = -BIAS * sc;   // exact
  float v[N];
  float amax = 0.f;
  // the shared operands of chunk i+1 are read while chunk i computes
  f32x4 cb_next = bdt4[0], cw_next = cw4[0];
#pragma unroll
  for (int i0 = 0; i0 < N; i0 += 4) {
    const f32x4 cb = cb_next, cw = cw_next;
    if (i0 + 4 < N) {
      cb_next = bdt4[i0 / 4 + 1];
      cw_next = cw4[i0 / 4 + 1];
    }
    float au[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // prior = q * s exactly: (q + bias) * s - bias * s, all exact
      const float prior = __builtin_fmaf(ubyte_f(c[i0 / 4], j), sc, nb);
      acc = __builtin_fmaf(prior, cw[j], acc);
      float u = prior * decay + cb[j] * x;
      // ordered pin: chunk by chunk, each prior dies as soon as it is used
      asm volatile("" : "+v"(u));
      v[i0 + j] = u;
      au[j] = __builtin_fabsf(u);
    }
    amax = __builtin_fmaxf(amax, __builtin_fmaxf(__builtin_fmaxf(au[0], au[1]), __builtin_fmaxf(au[2], au[3])));
    __builtin_amdgcn_sched_barrier(0);
  }
  // Materialize the accumulator and the maximum here: otherwise the compiler
  // sinks their chains (and every update behind the maximum) into the
  // requantization, which keeps every prior and LDS operand live at once.
  asm volatile("" : "+v"(acc), "+v"(amax));
  const float den = __builtin_fmaxf(div_by_recip(amax, LIM, 1.0f / LIM), 1e-8f);
  const float stored = round_to_half(den);
  float d, r;
  if constexpr (MODE == MODE_LEGACY) {
    d = den;
    r = 1.0f / den;
  } else {
    // zero (underflowed) or infinite stored scale: the reference's quotient
    // is 0 and so is the code
    const bool zero = !(stored > 0.f) || stored == __builtin_inff();
    d = zero ? 1.f : stored;
    r = zero ? 0.f : 1.0f / stored;
  }
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    const int q0 = quantize_code(v[4 * i], d, r, TOP);
    const int q1 = quantize_code(v[4 * i + 1], d, r, TOP);
    const int q2 = quantize_code(v[4 * i + 2], d, r, TOP);
    const int q3 = quantize_code(v[4 * i + 3], d, r, TOP);
    uint32_t packed = pack4(q0, q1, q2, q3);
    packed = INT8 ? (packed ^ 0x80808080u) : ((packed & 0x0F0F0F0Fu) ^ 0x08080808u);
    asm volatile("" : "+v"(packed));
    c[i] = packed;
    __builtin_amdgcn_sched_barrier(0);
  }
  return stored;
}

// Orders a wave's LDS accesses across its lanes (the wave's own staging
// tiles need no workgroup barrier).
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// One workgroup = WPB waves, each owning HPW head slots of 64 rows (the same
// P block of NH = WPB * HPW consecutive heads of one B/C group and batch
// row).  The packed rows of every slot stay in LDS, in the reference's SoA
// field layout, for all L tokens; a slot is unpacked into VGPRs, stepped and
// repacked in one pass per token.  The first token streams the slots in:
// the next slot's rows are loaded into VGPRs while the current one computes.
// Per-token shared values are built once per workgroup for all NH heads.
template <int N8, int N4, int NZ, int MODE, int WPB, int HPW>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(WPB == 8 ? 4 : 1, 8)))
void k_state_step(StepArgs a) {
  constexpr int W8 = N8 / 2;          // bytes per row of lo and of hi
  constexpr int W4 = N4 / 2;          // bytes per row of q4
  constexpr int NL = N8 + N4;         // carried coordinates
  constexpr int F = NL + 2;           // ridge predictor features
  constexpr int NT = 64 * WPB;
  constexpr int NH = WPB * HPW;
  constexpr bool RIDGE = MODE == MODE_RIDGE;
  constexpr int O_LO = 0, O_HI = 64 * W8, O_Q4 = 128 * W8, O_S8 = O_Q4 + 64 * W4, O_S4 = O_S8 + 128;
  constexpr int O_LAT = O_S4 + 128;
  constexpr int TILE = O_LAT + (RIDGE ? 128 : 0) + 16;   // 16 bytes of slack for row reads
  constexpr int C8 = N8 / 4, C4 = N4 / 4;   // carried code words (4 biased bytes each)
  constexpr int PRED_DW = RIDGE ? F * NZ / 2 : 1;   // F*NZ is even for every layout
  constexpr int PRED_OPS = (PRED_DW + 63) / 64;     // 64-dword transfers of the predictor
  constexpr int PERM_PT = (128 + NT - 1) / NT;      // permutation bytes per thread
  constexpr int BASIS_PT = (NZ + NT - 1) / NT;      // basis pairs per thread
  static_assert(N8 % 4 == 0 && N4 % 4 == 0 && N8 > 0 && N4 > 0, "tier widths must be positive multiples of 4");
  static_assert(!RIDGE || (F * NZ) % 2 == 0, "predictor staged as dwords");
  static_assert(TILE % 16 == 0, "tiles stay 16-byte aligned");

  // small, often-read arrays first: their LDS offsets fit instruction immediates
  __shared__ __align__(16) TokenShared<N8, N4, NZ, MODE, NH> sh;
  __shared__ float s_D[NH];
  __shared__ uint8_t s_perm[128];
  __shared__ float s_basis[RIDGE ? 2 * NZ : 1];
  __shared__ __align__(16) uint32_t s_pred32[PRED_OPS * 64];
  __shared__ __align__(16) uint8_t s_tile[NH][TILE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: per-wave values in SGPRs
  const int b = blockIdx.z;
  const int h0 = blockIdx.y * NH;
  const int H = a.H, P = a.P, L = a.L;
  const int g = h0 / (H / a.G);
  const int pbase = blockIdx.x * 64;
  const int nvalid = min(64, P - pbase);
  const bool valid = lane < nvalid;
  const bool dword_tiles = (P & 1) == 0;   // every slot's row0 * W and nvalid * W are dword multiples
  const uint16_t* s_pred = (const uint16_t*)s_pred32;

  // vector memory operations per slot transfer (field_dma counts)
  constexpr int SLOT_DMA = 2 * dma_ops(W8) + dma_ops(W4) + dma_ops(2) * (RIDGE ? 3 : 2);
  static_assert(SLOT_DMA <= 63, "a slot's transfers must fit the vmcnt range");
  auto slot_row0 = [&](int hh) { return (b * H + h0 + hh) * P + pbase; };
  auto slot_dma = [&](int hh) {   // even P: direct global -> LDS transfers
    const int row0 = slot_row0(hh);
    uint8_t* t = s_tile[hh];
    field_dma<W8>(t + O_LO, a.lo, row0, nvalid, lane);
    field_dma<W8>(t + O_HI, a.hi, row0, nvalid, lane);
    field_dma<W4>(t + O_Q4, a.q4, row0, nvalid, lane);
    field_dma<2>(t + O_S8, (const uint8_t*)a.s8, row0, nvalid, lane);
    field_dma<2>(t + O_S4, (const uint8_t*)a.s4, row0, nvalid, lane);
    if constexpr (RIDGE) field_dma<2>(t + O_LAT, a.latent, row0, nvalid, lane);
  };
  // at the first token, before slot k is read: issue slot k+1's transfers,
  // then wait until only those are outstanding (vector memory operations
  // complete in program order, so slot k's transfers and everything issued
  // before them have landed)
  auto slot_fetch_next_and_wait = [&](int k) {
    if (dword_tiles && k + 1 < HPW) {
      slot_dma((k + 1) * WPB + wave);
      wait_vmcnt<SLOT_DMA>();
    } else {
      wait_vmcnt<0>();
    }
  };
  auto slot_copy_in = [&](int hh) {   // odd P: 16-bit transfers
    const int row0 = slot_row0(hh);
    uint8_t* t = s_tile[hh];
    wave_copy_in<W8>(t + O_LO, a.lo, row0, nvalid, lane);
    wave_copy_in<W8>(t + O_HI, a.hi, row0, nvalid, lane);
    wave_copy_in<W4>(t + O_Q4, a.q4, row0, nvalid, lane);
    wave_copy_in<2>(t + O_S8, (const uint8_t*)a.s8, row0, nvalid, lane);
    wave_copy_in<2>(t + O_S4, (const uint8_t*)a.s4, row0, nvalid, lane);
    if constexpr (RIDGE) wave_copy_in<2>(t + O_LAT, a.latent, row0, nvalid, lane);
  };
  auto slot_copy_out = [&](int hh) {
    const int row0 = slot_row0(hh);
    const uint8_t* t = s_tile[hh];
    if (dword_tiles) {
      field_store<W8>(a.lo, t + O_LO, row0, nvalid, lane);
      field_store<W8>(a.hi, t + O_HI, row0, nvalid, lane);
      field_store<W4>(a.q4, t + O_Q4, row0, nvalid, lane);
      field_store<2>((uint8_t*)a.s8, t + O_S8, row0, nvalid, lane);
      field_store<2>((uint8_t*)a.s4, t + O_S4, row0, nvalid, lane);
      if constexpr (RIDGE) field_store<2>(a.latent, t + O_LAT, row0, nvalid, lane);
      return;
    }
    wave_copy_out<W8>(a.lo, t + O_LO, row0, nvalid, lane);
    wave_copy_out<W8>(a.hi, t + O_HI, row0, nvalid, lane);
    wave_copy_out<W4>(a.q4, t + O_Q4, row0, nvalid, lane);
    wave_copy_out<2>((uint8_t*)a.s8, t + O_S8, row0, nvalid, lane);
    wave_copy_out<2>((uint8_t*)a.s4, t + O_S4, row0, nvalid, lane);
    if constexpr (RIDGE) wave_copy_out<2>(a.latent, t + O_LAT, row0, nvalid, lane);
  };

  // ---- prologue: the predictor's LDS transfer, then the register loads of the
  // first token and the statics (one wait covers both), then the LDS transfer
  // of the wave's first slot, which lands during the token build; each later
  // slot is fetched while the previous one computes -----------------------------
  if constexpr (RIDGE) {   // predictor rows of the group, spread over the waves
    const uint8_t* pg = (const uint8_t*)(a.pred + (size_t)g * F * NZ);
    for (int j = wave; j < PRED_OPS; j += WPB) lds_dma_b32(pg + 4 * min(j * 64 + lane, PRED_DW - 1),
                                                           lds_address(s_pred32 + 64 * j));
  }
  TokenRaw<WPB, HPW> raw;
  token_load<WPB, HPW>(a, raw, b * L, g, h0, pbase, tid, lane, wave);
  const float Ah = (tid < NH) ? a.A[h0 + tid] : 0.f;
  const float Dv = (tid < NH) ? load_param(a.D, a.d_f32, h0 + tid) : 0.f;
  uint8_t permv[PERM_PT];
#pragma unroll
  for (int k = 0; k < PERM_PT; ++k) {
    const int n = k * NT + tid;
    permv[k] = (n < 128) ? a.perm[g * 128 + n] : (uint8_t)0;
  }
  uint32_t basisv[BASIS_PT];
  float ls0 = 0.f, ls1 = 0.f, rls0 = 0.f, rls1 = 0.f;
  if constexpr (RIDGE) {
#pragma unroll
    for (int k = 0; k < BASIS_PT; ++k) {
      const int i = k * NT + tid;
      basisv[k] = (i < NZ) ? ((const uint32_t*)a.basis)[g * NZ + i] : 0u;
    }
    ls0 = h2f(a.lscale[g * 2]);
    ls1 = h2f(a.lscale[g * 2 + 1]);
    rls0 = 1.0f / ls0;   // correctly rounded reciprocals
    rls1 = 1.0f / ls1;
  }
  // the predictor transfer and the register loads complete before any slot
  // transfer is issued (the compiler's own waits for the register loads then
  // never cover a slot transfer)
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
  if (dword_tiles) slot_dma(wave);
  if (tid < NH) s_D[tid] = Dv;
#pragma unroll
  for (int k = 0; k < PERM_PT; ++k) {
    const int n = k * NT + tid;
    if (n < 128) s_perm[n] = permv[k];
  }
  if constexpr (RIDGE) {
#pragma unroll
    for (int k = 0; k < BASIS_PT; ++k) {
      const int i = k * NT + tid;
      if (i < NZ) {
        s_basis[i] = h2f((uint16_t)(basisv[k] & 0xFFFFu));
        s_basis[NZ + i] = h2f((uint16_t)(basisv[k] >> 16));
      }
    }
  }
  if (!dword_tiles) {
    for (int k = 0; k < HPW; ++k) slot_copy_in(k * WPB + wave);
  }
  token_store<N8, N4, NZ, MODE, WPB, HPW>(sh, raw, Ah, a.db_f32, tid, lane, wave);
  __syncthreads();

  for (int t = 0; t < L; ++t) {
    const int bt = b * L + t;
    if (t > 0) {
      token_store<N8, N4, NZ, MODE, WPB, HPW>(sh, raw, Ah, a.db_f32, tid, lane, wave);
      __syncthreads();
    }
    if (t + 1 < L) token_load<WPB, HPW>(a, raw, bt + 1, g, h0, pbase, tid, lane, wave);   // prefetch
    token_build<N8, N4, NZ, MODE, WPB, HPW>(sh, s_perm, s_basis, s_pred, tid, lane, wave);

    for (int k = 0; k < HPW; ++k) {
      const int hh = k * WPB + wave;
      const int h = h0 + hh;
      if (t == 0) slot_fetch_next_and_wait(k);
      uint8_t* tile = s_tile[hh];
      uint16_t* t16 = (uint16_t*)tile;

      // ---- unpack the slot: carried codes, internal lane order ------------------
      // byte k of c8[i] is q8 + 128 of internal coordinate 4i+k, of c4[i] q4 + 8
      uint32_t c8[C8], c4[C4];
      {
        uint32_t wl[(W8 + 3) / 4], wh[(W8 + 3) / 4], wq[(W4 + 3) / 4];
        lds_read_row<W8>(tile + O_LO, lane * W8, wl);
        lds_read_row<W8>(tile + O_HI, lane * W8, wh);
        planes_to_bytes8<N8>(wl, wh, c8);
        lds_read_row<W4>(tile + O_Q4, lane * W4, wq);
        plane_to_bytes4<N4>(wq, c4);
      }
      float sc8 = h2f(t16[O_S8 / 2 + lane]);
      float sc4 = h2f(t16[O_S4 / 2 + lane]);
      float z0 = 0.f, z1 = 0.f;
      if constexpr (RIDGE) {
        const uint32_t lat = t16[O_LAT / 2 + lane];
        z0 = e4m3_to_f32(lat & 0xFFu) * ls0;
        z1 = e4m3_to_f32(lat >> 8) * ls1;
      }
      if (!valid) {   // rows past P: finite placeholders, never stored
#pragma unroll
        for (int i = 0; i < C8; ++i) c8[i] = 0x80808080u;
#pragma unroll
        for (int i = 0; i < C4; ++i) c4[i] = 0x08080808u;
        sc8 = sc4 = z0 = z1 = 0.f;
      }
      const float x = h2f(sh.xr[hh * 64 + lane]);
      const float decay = sh.decay[hh];
      const float dtv = sh.dtv[hh];

      // ---- per tier: update, readout accumulation, requantization ---------------
      // (each tier is requantized before the next is updated, so only one
      // tier's updated values are live at a time)
      const f32x4* bdt4 = (const f32x4*)sh.bdt[hh];
      const f32x4* cw4;
      if constexpr (RIDGE) cw4 = (const f32x4*)sh.cp; else cw4 = (const f32x4*)sh.c;
      float acc = 0.f;
      sc8 = tier_step<N8, true, MODE>(c8, sc8, decay, x, bdt4, cw4, acc);
      __builtin_amdgcn_sched_barrier(0);
      sc4 = tier_step<N4, false, MODE>(c4, sc4, decay, x, bdt4 + N8 / 4, cw4 + N8 / 4, acc);
      __builtin_amdgcn_sched_barrier(0);
      // readout: sum_i u_i c_i + corrections = decay * (sum_i prior_i (c_i +
      // corr_i) + latent terms) + x * (dt * sum_all b c + D)
      float out;
      uint32_t qz = 0;
      if constexpr (RIDGE) {
        const float kz0 = sh.dots[1] + sh.dots[5], kz1 = sh.dots[2] + sh.dots[6];
        out = decay * (acc + z0 * kz0 + z1 * kz1) + x * (dtv * sh.dots[0] + s_D[hh]);
        // latent step (bit-exact): z <- z * decay + (x * dt) * (e . b_dead), requantized
        const float xdt = x * dtv;
        const float zn0 = z0 * decay + xdt * sh.dots[3];
        const float zn1 = z1 * decay + xdt * sh.dots[4];
        const float q0 = __builtin_fminf(__builtin_fmaxf(latent_quotient(zn0, ls0, rls0), -448.f), 448.f);
        const float q1 = __builtin_fminf(__builtin_fmaxf(latent_quotient(zn1, ls1, rls1), -448.f), 448.f);
        qz = f32_to_e4m3(q0) | (f32_to_e4m3(q1) << 8);
      } else {
        out = decay * acc + x * (dtv * sh.dots[0] + s_D[hh]);
      }
      if (valid) a.y[((size_t)bt * H + h) * P + pbase + lane] = f2h(out);

      // ---- repack the slot row into the tile ---------------------------------------
      if (valid) {
        uint32_t wl[(W8 + 3) / 4], wh[(W8 + 3) / 4], wq[(W4 + 3) / 4];
        bytes_to_planes8<N8>(c8, wl, wh);
        lds_write_row<W8>(tile + O_LO, lane * W8, wl);
        lds_write_row<W8>(tile + O_HI, lane * W8, wh);
        bytes_to_plane4<N4>(c4, wq);
        lds_write_row<W4>(tile + O_Q4, lane * W4, wq);
        t16[O_S8 / 2 + lane] = f2h(sc8);
        t16[O_S4 / 2 + lane] = f2h(sc4);
        if constexpr (RIDGE) t16[O_LAT / 2 + lane] = (uint16_t)qz;
      }
      wave_sync();
      if (t == L - 1) slot_copy_out(hh);
    }
    if (t + 1 < L) __syncthreads();   // shared token values are rebuilt next iteration
  }
}

// ---------------------------------------------------------------------------
// Host dispatch over the supported tier layouts.  Heads per workgroup grow
// with the number of 64-row slots so that the per-token shared work is
// amortized while the grid still spans every CU; small grids keep four waves
// per workgroup, which splits the per-token shared work four ways.
// Workgroup shape forced through m2r_set_step_shape (0 = automatic), encoded
// as waves_per_block * 16 + heads_per_wave.
static std::atomic<int> g_forced_shape{0};

template <int N8, int N4, int NZ, int MODE>
static hipError_t launch_layout(const StepArgs& a, hipStream_t stream) {
  const int pblocks = (a.P + 63) / 64;
  const int hpg = a.H / a.G;
  const long long slots = (long long)a.B * a.H * pblocks;
  const int forced = g_forced_shape.load(std::memory_order_relaxed);
  if (forced && hpg % ((forced >> 4) * (forced & 15)) == 0) {
    const int wpb = forced >> 4, hpw = forced & 15;
    dim3 grid(pblocks, a.H / (wpb * hpw), a.B);
    if (wpb == 1) hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 1, 1>), grid, dim3(64), 0, stream, a);
    else if (hpw == 1) hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 4, 1>), grid, dim3(256), 0, stream, a);
    else if (wpb == 8) hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 8, 2>), grid, dim3(512), 0, stream, a);
    else if (hpw == 2) hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 4, 2>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 4, 4>), grid, dim3(256), 0, stream, a);
    return hipGetLastError();
  }
  if (hpg % 16 == 0 && slots >= 16LL * 512) {
    dim3 grid(pblocks, a.H / 16, a.B);
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 4, 4>), grid, dim3(256), 0, stream, a);
  } else if (hpg % 8 == 0 && slots >= 8LL * 512) {
    dim3 grid(pblocks, a.H / 8, a.B);
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 4, 2>), grid, dim3(256), 0, stream, a);
  } else if (hpg % 4 == 0) {
    dim3 grid(pblocks, a.H / 4, a.B);
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 4, 1>), grid, dim3(256), 0, stream, a);
  } else {
    dim3 grid(pblocks, a.H, a.B);
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, 1, 1>), grid, dim3(64), 0, stream, a);
  }
  return hipGetLastError();
}

#define M2R_LAYOUT(n8, n4, nz, mode)                                   \
  if (a.n8_ == n8 && a.n4_ == n4 && a.nz_ == nz) return launch_layout<n8, n4, nz, mode>(a.args, stream);

struct Dispatch { StepArgs args; int n8_, n4_, nz_; };

static hipError_t dispatch_ridge(const Dispatch& a, hipStream_t stream) {
  // scripts/fp4_zero_predictor_codec_v1.py:28-36 applied to the seven
  // published layouts of scripts/w4_state_repair_codec_v2.py:27-28.
  M2R_LAYOUT(36, 20, 72, MODE_RIDGE)
  M2R_LAYOUT(16, 60, 52, MODE_RIDGE)
  M2R_LAYOUT(32, 28, 68, MODE_RIDGE)
  M2R_LAYOUT(40, 12, 76, MODE_RIDGE)
  M2R_LAYOUT(24, 44, 60, MODE_RIDGE)
  M2R_LAYOUT(8, 76, 44, MODE_RIDGE)
  M2R_LAYOUT(44, 4, 80, MODE_RIDGE)
  return hipErrorInvalidValue;
}

static hipError_t dispatch_tier(const Dispatch& a, hipStream_t stream) {
  // scripts/state_ppl_codec_v10.py:24-26 and w4_state_repair_codec_v2.py:27-28
  M2R_LAYOUT(16, 64, 48, MODE_STORED)
  M2R_LAYOUT(8, 80, 40, MODE_STORED)
  M2R_LAYOUT(24, 48, 56, MODE_STORED)
  M2R_LAYOUT(32, 32, 64, MODE_STORED)
  M2R_LAYOUT(36, 24, 68, MODE_STORED)
  M2R_LAYOUT(40, 16, 72, MODE_STORED)
  M2R_LAYOUT(44, 8, 76, MODE_STORED)
  return hipErrorInvalidValue;
}

}  // namespace m2r

using namespace m2r;

static int check_geometry(int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G) {
  if (batch <= 0 || L <= 0 || H <= 0 || P <= 0 || G <= 0) return m2r_fail("state step: non-positive geometry");
  if (H % G) return m2r_fail("state step: heads must be divisible by groups");
  if (batch > 65535 || H > 65535 * 4) return m2r_fail("state step: grid limits exceeded");
  if ((double)batch * L * H * P >= 2147483647.0) return m2r_fail("state step: B*L*H*P must fit int32");
  return 0;
}

extern "C" int m2r_state_step_ridge(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                    const void* D, int d_is_f32, const void* dt_bias, int db_is_f32,
                                    const uint8_t* perm, const void* basis, const void* lscale, const void* pred,
                                    uint8_t* lo, uint8_t* hi, uint8_t* q4, uint8_t* latent, void* s8, void* s4,
                                    void* y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G, int n8,
                                    int n4, int nz, hipStream_t stream) {
  if (int e = check_geometry(batch, L, H, P, G)) return e;
  Dispatch d{};
  d.args = StepArgs{(const uint16_t*)x, (const uint16_t*)dt, A, (const uint16_t*)B, (const uint16_t*)C, D, dt_bias,
                    perm, (const uint16_t*)basis, (const uint16_t*)lscale, (const uint16_t*)pred, lo, hi, q4, latent,
                    (uint16_t*)s8, (uint16_t*)s4, (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G,
                    d_is_f32, db_is_f32};
  d.n8_ = n8; d.n4_ = n4; d.nz_ = nz;
  hipError_t e = dispatch_ridge(d, stream);
  if (e == hipErrorInvalidValue) return m2r_fail("ridge step: unsupported tier layout");
  return m2r_check(e, "ridge step launch");
}

extern "C" int m2r_state_step_tier(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                   const void* D, int d_is_f32, const void* dt_bias, int db_is_f32,
                                   const uint8_t* perm, uint8_t* lo, uint8_t* hi, uint8_t* q4, void* s8, void* s4,
                                   void* y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G, int n8,
                                   int n4, int nz, hipStream_t stream) {
  if (int e = check_geometry(batch, L, H, P, G)) return e;
  Dispatch d{};
  d.args = StepArgs{(const uint16_t*)x, (const uint16_t*)dt, A, (const uint16_t*)B, (const uint16_t*)C, D, dt_bias,
                    perm, nullptr, nullptr, nullptr, lo, hi, q4, nullptr, (uint16_t*)s8, (uint16_t*)s4,
                    (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G, d_is_f32, db_is_f32};
  d.n8_ = n8; d.n4_ = n4; d.nz_ = nz;
  hipError_t e = dispatch_tier(d, stream);
  if (e == hipErrorInvalidValue) return m2r_fail("tier step: unsupported tier layout");
  return m2r_check(e, "tier step launch");
}

extern "C" int m2r_set_step_shape(int waves_per_block, int heads_per_wave) {
  const int w = waves_per_block, k = heads_per_wave;
  const bool ok = (w == 0 && k == 0) || (w == 1 && k == 1) || (w == 4 && (k == 1 || k == 2 || k == 4)) ||
                  (w == 8 && k == 2);
  if (!ok)
    return m2r_fail("step shape: supported (waves, heads per wave) are (1,1), (4,1), (4,2), (4,4), (8,2) or (0,0)");
  g_forced_shape.store(w * 16 + k, std::memory_order_relaxed);
  return 0;
}

extern "C" int m2r_state_step_legacy(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                     const void* D, int d_is_f32, const void* dt_bias, int db_is_f32,
                                     const uint8_t* perm, uint8_t* lo, uint8_t* hi, uint8_t* q4, void* s8,
                                     void* s4, void* y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G,
                                     hipStream_t stream) {
  if (int e = check_geometry(batch, L, H, P, G)) return e;
  StepArgs args{(const uint16_t*)x, (const uint16_t*)dt, A, (const uint16_t*)B, (const uint16_t*)C, D, dt_bias,
                perm, nullptr, nullptr, nullptr, lo, hi, q4, nullptr, (uint16_t*)s8, (uint16_t*)s4,
                (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G, d_is_f32, db_is_f32};
  return m2r_check(launch_layout<16, 64, 48, MODE_LEGACY>(args, stream), "legacy step launch");
}
