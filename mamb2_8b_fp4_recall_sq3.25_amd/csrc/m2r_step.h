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
#pragma once
#include "m2r_device.h"
#include "m2r_tile.h"

#include <atomic>
#include <type_traits>
#include <initializer_list>

namespace m2r {

enum { MODE_LEGACY = 0, MODE_STORED = 1, MODE_RIDGE = 2 };

// Phase timeline of one launch, compiled only into the instrumented build
// (M2R_PHASE_TIMELINE; the library proper has none of it).  Lane 0 of every
// wave stamps the shader clock (s_memtime) at the phase boundaries below into
// LDS and, at the end, writes its 32 stamps to g_phase_stamps[(block * WPB +
// wave) * 32 + i], block = (z * gridDim.y + y) * gridDim.x + x.  Stamps 30 and
// 31 read the constant 100 MHz clock (s_memrealtime) at the start and the end,
// which gives the shader clock's rate.  Phases of slot k (k < 4) are stamps
// ST_SLOT + 4 k + {0: its data landed, 1: update (one wave per slot: INT8
// tier) done, 2: barrier passed (one wave per slot: INT4 tier done), 3: slot
// done}.  Multi-token launches of several waves per slot also stamp token
// ST_TL_TOKEN at ST_TL + {0: token start, 1: token values ready (record read
// or token built), 2: update half done, 3: maxima barrier passed, 4:
// requantization half done, 5: token end}.
enum {
  ST_START = 0, ST_ARGS = 1, ST_ISSUED = 2, ST_SLOT0_ISSUED = 3, ST_ACT = 4, ST_TOKEN = 5, ST_BARRIER = 6,
  ST_BUILD = 7, ST_SLOT = 8, ST_TL = 12, ST_COPYOUT = 24, ST_END = 25, ST_REAL0 = 30, ST_REAL1 = 31
};
constexpr int ST_TL_TOKEN = 100;
#ifdef M2R_PHASE_TIMELINE
__device__ unsigned long long* g_phase_stamps;
#define M2R_STAMP(i)                                                                     \
  do {                                                                                   \
    const unsigned long long t_ = __builtin_amdgcn_s_memtime();                          \
    if (lane == 0) sm.stamps[wave][(i)] = t_;                                            \
  } while (0)
#define M2R_STAMP_REAL(i)                                                                \
  do {                                                                                   \
    const unsigned long long t_ = __builtin_amdgcn_s_memrealtime();                      \
    if (lane == 0) sm.stamps[wave][(i)] = t_;                                            \
  } while (0)
#else
#define M2R_STAMP(i) do {} while (0)
#define M2R_STAMP_REAL(i) do {} while (0)
#endif

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
  int dma_tiles;           // bit 0: P % 8 == 0, 16-byte aligned state fields and predictor, 4-byte
                           // aligned B and C: 16-byte LDS transfers and paired B/C loads; bit 1: H
                           // even and 4-byte aligned x, dt, A, D, dt_bias, perm (and basis): the
                           // one-token instances may stage their inputs by dword transfers
  float rhpg;              // 1 / (H / G) rounded to binary32: group of head h = (int)((h + 0.5) * rhpg)
  // multi-token ridge launches of several waves per slot: the token records
  // k_token_records wrote ([B, L, G] records of REC_FLOATS), or null (each
  // workgroup builds its tokens itself)
  const float* rec;
};

// Loads every field of the arguments into scalar registers at once (one
// wait) instead of on first use (a wait per field, in series).
__device__ __forceinline__ void load_args(const StepArgs& a) {
  asm volatile("" ::"s"(a.x), "s"(a.dt), "s"(a.A), "s"(a.Bm), "s"(a.Cm), "s"(a.D), "s"(a.dt_bias), "s"(a.perm),
               "s"(a.basis), "s"(a.lscale), "s"(a.pred), "s"(a.lo), "s"(a.hi), "s"(a.q4), "s"(a.latent),
               "s"(a.s8), "s"(a.s4), "s"(a.y), "s"(a.B), "s"(a.H), "s"(a.P), "s"(a.G), "s"(a.d_f32),
               "s"(a.db_f32), "s"(a.rhpg));
  // nothing is scheduled above this point, so no field is loaded later
  __builtin_amdgcn_sched_barrier(0);
}

// Group of head h (wave-uniform): floor(h / hpg) as (int)((h + 0.5) * rhpg).
// Exact for H < 2^22: the float product is within G * 2^-23 of
// (h + 0.5) / hpg, whose distance to the integers is at least 0.5 / hpg.
__device__ __forceinline__ int group_of_head(int h, float rhpg) {
  return __builtin_amdgcn_readfirstlane((int)(((float)h + 0.5f) * rhpg));
}

// Scalar load of the dword at a wave-uniform address (the inputs are never
// written by the step kernels: constant address space).
__device__ __forceinline__ uint32_t scalar_dword(const void* p) {
  // both halves zero-extended (readfirstlane returns a signed int)
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)p);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uintptr_t)p >> 32));
  const uintptr_t u = (uintptr_t)lo | ((uintptr_t)hi << 32);
  return *(const __attribute__((address_space(4))) uint32_t*)u;
}
// N consecutive dwords at a wave-uniform, dword-aligned address: one scalar load.
template <int N>
__device__ __forceinline__ void scalar_dwords(const void* p, uint32_t* out) {
  if constexpr (N == 1) {
    out[0] = scalar_dword(p);
  } else {
    typedef uint32_t vec __attribute__((ext_vector_type(N), aligned(4)));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)p);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)((uintptr_t)p >> 32));
    const uintptr_t u = (uintptr_t)lo | ((uintptr_t)hi << 32);
    const vec v = *(const __attribute__((address_space(4))) vec*)u;
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = v[i];
  }
}

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
// Readout segments.  The carried coordinates, the INT8 tier then the INT4
// tier in one index space [0, NL), are cut into four segments.  A cut is a
// whole nibble-plane word into its tier (a multiple of 8 from the tier's
// start) or the tier boundary n8.  One cut is the two-wave split: the tier
// boundary, moved into the INT4 tier by the multiple of 8 that brings the two
// halves' coordinate counts closest when the INT4 tier is the wider one (the
// INT8 tier is never split between two waves); the other two are the valid
// cuts that make the largest segment smallest, then the sum of the segments'
// squares (the lowest cuts on a further tie).  Each
// segment's readout is one fma chain, and the row's readout their left fold
// ((s0 + s1) + s2) + s3 on every workgroup shape.  A slot stepped by four
// waves gives wave r segment r; by two waves, wave 0 the segments before the
// two-wave split and wave 1 the others.
constexpr bool seg_cut_ok(int n8, int p) { return p <= n8 ? (p % 8 == 0 || p == n8) : (p - n8) % 8 == 0; }
constexpr int pair_cut(int n8, int n4) { return n8 + (n4 > n8 ? 8 * ((n4 - n8 + 7) / 16) : 0); }
struct SegCuts { int c[3]; int j; };   // cuts c[0] < c[1] < c[2]; c[j] is the two-wave split
constexpr SegCuts seg_cuts(int n8, int n4) {
  const int nl = n8 + n4, c2 = pair_cut(n8, n4);
  int v[40] = {};   // the valid cut positions (at most 16 per tier and the boundary)
  int nv = 0;
  for (int p = 1; p < nl; ++p)
    if (seg_cut_ok(n8, p)) v[nv++] = p;
  SegCuts best{{0, 0, 0}, -1};
  int best_max = 1 << 30, best_sq = 1 << 30;
  for (int i = 0; i < nv; ++i)
    for (int j = i + 1; j < nv; ++j)
      for (int k = j + 1; k < nv; ++k) {
        const int a = v[i], b = v[j], c = v[k];
        if (a != c2 && b != c2 && c != c2) continue;
        int m = a;
        if (b - a > m) m = b - a;
        if (c - b > m) m = c - b;
        if (nl - c > m) m = nl - c;
        const int sq = a * a + (b - a) * (b - a) + (c - b) * (c - b) + (nl - c) * (nl - c);
        if (m < best_max || (m == best_max && sq < best_sq)) {
          best_max = m;
          best_sq = sq;
          best = SegCuts{{a, b, c}, a == c2 ? 0 : b == c2 ? 1 : 2};
        }
      }
  return best;
}
constexpr int seg_pos(int n8, int n4, int k) {
  return k <= 0 ? 0 : k >= 4 ? n8 + n4 : seg_cuts(n8, n4).c[k - 1];
}
// first segment of wave r of a WPS-wave slot (r = WPS: 4)
constexpr int role_seg(int n8, int n4, int wps, int r) {
  return wps == 4 ? r : wps == 2 ? (r == 0 ? 0 : r == 1 ? seg_cuts(n8, n4).j + 1 : 4) : (r == 0 ? 0 : 4);
}
constexpr bool seg_layout_ok(int n8, int n4) { return seg_cuts(n8, n4).j >= 0; }
static_assert(seg_pos(8, 76, 1) == 16 && seg_pos(8, 76, 2) == 40 && seg_pos(8, 76, 3) == 64 &&
                  seg_cuts(8, 76).j == 1 && seg_pos(32, 28, 1) == 16 && seg_pos(32, 28, 2) == 32 &&
                  seg_pos(32, 28, 3) == 48 && seg_pos(36, 20, 1) == 8 && seg_pos(36, 20, 2) == 24 &&
                  seg_pos(36, 20, 3) == 36 && seg_cuts(36, 20).j == 2 && seg_pos(44, 4, 3) == 44 &&
                  seg_cuts(44, 4).j == 2 && seg_pos(24, 44, 2) == 32 && seg_pos(16, 60, 3) == 56,
              "readout segments");
// segment of carried coordinate p (the cuts as template-level constants, so
// that a call with an unrolled loop index folds)
template <int N8, int N4>
__host__ __device__ __forceinline__ constexpr int seg_of(int p) {
  constexpr int S1 = seg_pos(N8, N4, 1), S2 = seg_pos(N8, N4, 2), S3 = seg_pos(N8, N4, 3);
  return p < S1 ? 0 : p < S2 ? 1 : p < S3 ? 2 : 3;
}
// bit r: wave r of a WPS-wave slot steps INT8 (TIER4 false) or INT4 coordinates
template <int N8, int N4, int WPS, bool TIER4>
constexpr unsigned tier_waves() {
  unsigned m = 0;
  for (int r = 0; r < WPS; ++r) {
    const int lo = seg_pos(N8, N4, role_seg(N8, N4, WPS, r)), hi = seg_pos(N8, N4, role_seg(N8, N4, WPS, r + 1));
    if (TIER4 ? hi > N8 : lo < N8) m |= 1u << r;
  }
  return m;
}

// Code words (four coordinates each) of wave r's part of one tier, and the
// most any wave of a WPS-wave slot has.
constexpr int role_words(int n8, int n4, int wps, int r, bool tier4) {
  const int lo = seg_pos(n8, n4, role_seg(n8, n4, wps, r)), hi = seg_pos(n8, n4, role_seg(n8, n4, wps, r + 1));
  const int a = tier4 ? (lo > n8 ? lo - n8 : 0) : (lo < n8 ? lo : n8);
  const int e = tier4 ? (hi > n8 ? hi - n8 : 0) : (hi < n8 ? hi : n8);
  return (e - a + 3) / 4;
}
constexpr int max_role_words(int n8, int n4, int wps, bool tier4) {
  int m = 1;
  for (int r = 0; r < wps; ++r) m = role_words(n8, n4, wps, r, tier4) > m ? role_words(n8, n4, wps, r, tier4) : m;
  return m;
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

// Per-token values of one wave, in the wave's own LDS region.  Only the
// wave's own lanes read them, so building them needs no workgroup barrier:
// the raw B/C rows, the permuted b and c, B*dt per head slot, the readout
// weights of the carried coordinates, x of the wave's rows and per-slot and
// per-token scalars.
template <int N8, int N4, int HPW>
struct WaveToken {
  static constexpr int NL = N8 + N4;
  alignas(16) float b[128];          // internal order
  alignas(16) float c[128];
  alignas(16) float cw[NL];          // readout weights of the carried coordinates: c (+ ridge correction)
  alignas(16) float bdt[HPW][NL];    // RN(b * dt) per head slot
  uint16_t x[HPW][64];               // x of the wave's rows, per head slot
  float dtv[HPW], decay[HPW], D[HPW];
  // per head slot: 1 when B*dt and the decay are bounded (|.| < 2^100), so
  // that the state update of finite operands is finite
  uint32_t bounded[HPW];
  // 0: sum of b*c over all 128 coordinates (readout); 1, 2: dead-tier e0.c,
  // e1.c plus the ridge correction of the latent coefficients (readout);
  // 3, 4: dead-tier e0.b, e1.b (canonical trees, exact)
  float dots[5];
};

// Per-token values of the ridge codec that the waves of a workgroup share
// when they split the predictor correction (four or more waves): the readout
// weights of the carried coordinates (c + correction), the latent
// coefficients' corrections and the dead-tier dot products e.c and e.b, each
// written by the wave that computes it and read after a workgroup barrier.
template <int NL>
struct GroupToken {
  alignas(16) float cw[NL + 2];   // readout weights, then the latent coefficients' corrections
  float tree[4];                  // e0.c, e1.c, e0.b, e1.b
};

// Token record of the ridge codec: the per-token values of one (batch row,
// group, token) that do not depend on the state, as the split token build
// (wave_token_build, four waves) computes them: [REC_CW, REC_CW + NL + 2)
// the readout weights and the latent coefficients' corrections (GroupToken
// cw), [REC_TREE, REC_TREE + 4) the dead-tier dot products, REC_SBC the sum
// of b.c, REC_BOK 1.0 when every carried b is finite (else 0.0), and
// [REC_B, REC_B + NL) the carried b in internal order.  1 KiB: one 16-byte
// load per lane of one wave.
constexpr int REC_FLOATS = 256, REC_CW = 0, REC_TREE = 88, REC_SBC = 92, REC_BOK = 93, REC_B = 96;
static_assert(REC_CW + 84 + 2 <= REC_TREE && REC_B + 84 <= REC_FLOATS, "every published layout fits (NL <= 84)");

// Token inputs of a one-token workgroup staged in LDS by direct transfers
// (the staged prologue): the group's B and C rows (f16 pairs) and statics,
// `stat`: [0, 32) the permutation bytes, [32, 32 + NZ) the dead-tier basis
// (f16 pairs).
struct TokenStage {
  alignas(16) uint32_t b[64];      // shared transfer 0
  alignas(16) uint32_t c[64];      // shared transfer 1
  alignas(16) uint32_t stat[128];  // shared transfers 2 and 3
};
static_assert(sizeof(TokenStage) == 1024, "shared transfer j lands at dword 64 j");
struct NoStage {};

// Inputs of one token that a wave loads one token ahead: its lane's two f16
// of the group's B and of its C row, x of its rows in every head slot, and
// for lanes < HPW the dt and dt_bias bits of head slot `lane`.  Nothing is
// converted at load time, so no wait is needed until the token is built.
template <int HPW>
struct WaveRaw {
  uint16_t bc[4];              // B[2 lane], B[2 lane + 1], C[2 lane], C[2 lane + 1]
  uint16_t xv[HPW];
  uint16_t dt, db_lo, db_hi;   // dt_bias: f16 bits, or the halves of f32 bits
};

// The dt inputs are loaded first: the dt activation of the first token
// starts as soon as they land, while the other loads are still in flight.
// Every load here is unconditional, with clamped indices (a conditional load
// makes the compiler wait for it at the end of its branch).
// A wave's head slots are HPW consecutive heads (slot k of wave w is
// workgroup head w * HPW + k); WPS > 1: WPS waves per head, a wave's only
// slot is head wave / WPS.
template <int WPB, int HPW, int WPS = 1>
__device__ __forceinline__ void wave_load_dt(const StepArgs& a, WaveRaw<HPW>& r, int bt, int h0, int lane,
                                             int wave) {
  // lanes >= HPW repeat the last slot
  const int h = h0 + (WPS > 1 ? wave / WPS : wave * HPW + min(lane, HPW - 1));
  const uint16_t* db = (const uint16_t*)a.dt_bias;
  r.dt = a.dt[(size_t)bt * a.H + h];
  r.db_lo = db[a.db_f32 ? 2 * h : h];
  r.db_hi = db[a.db_f32 ? 2 * h + 1 : h];
}
// x of the wave's rows in each head slot (a record-fed token loop loads
// only these: dt comes 64 tokens at a time, B and C with the records).
template <int WPB, int HPW, int WPS = 1>
__device__ __forceinline__ void wave_load_x(const StepArgs& a, WaveRaw<HPW>& r, int bt, int h0, int pbase, int lane,
                                            int wave) {
  const int p = min(pbase + lane, a.P - 1);   // rows past P read row P-1 (never stored)
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const int h = h0 + (WPS > 1 ? wave / WPS : wave * HPW + k);
    r.xv[k] = a.x[((size_t)bt * a.H + h) * a.P + p];
  }
}
// ALIGNED: B and C are 4-byte aligned, so a lane's pair is one load each.
template <int WPB, int HPW, bool ALIGNED, int WPS = 1>
__device__ __forceinline__ void wave_load_rest(const StepArgs& a, WaveRaw<HPW>& r, int bt, int g, int h0,
                                               int pbase, int lane, int wave) {
  const size_t row = ((size_t)bt * a.G + g) * 128 + 2 * lane;
  if constexpr (ALIGNED) {
    const uint32_t bp = *(const uint32_t*)(a.Bm + row), cp = *(const uint32_t*)(a.Cm + row);
    r.bc[0] = (uint16_t)bp;
    r.bc[1] = (uint16_t)(bp >> 16);
    r.bc[2] = (uint16_t)cp;
    r.bc[3] = (uint16_t)(cp >> 16);
  } else {
    r.bc[0] = a.Bm[row];
    r.bc[1] = a.Bm[row + 1];
    r.bc[2] = a.Cm[row];
    r.bc[3] = a.Cm[row + 1];
  }
  wave_load_x<WPB, HPW, WPS>(a, r, bt, h0, pbase, lane, wave);
}

// dt activation of head slot `lane` (lanes < HPW; the others compute a copy
// of the last slot's, unused).
template <int HPW, bool VREG = false, int KM = KM_ASM>
__device__ __forceinline__ float2 wave_dt_activation(const WaveRaw<HPW>& r, float Ah, int db_f32) {
  const float db = db_f32 ? __builtin_bit_cast(float, (uint32_t)r.db_lo | ((uint32_t)r.db_hi << 16)) : h2f(r.db_lo);
  return dt_activation<VREG, KM>(h2f(r.dt) + db, Ah);
}

// Builds the wave's token values from its landed raw inputs and the dt
// activation `act` of head slot `lane` (lanes < HPW): raw rows and x, dt and
// decay per head slot, b and c gathered through
// the permutation (lane holds internal positions lane and lane + 64, whose
// raw indices are pv0 and pv1), B*dt, sum b.c, the readout weights and, for
// the ridge codec, the correction of the readout weights by the static
// predictor and the dead-tier dot products.  `first`: the first token, whose
// ridge correction waits for the workgroup's predictor transfer.  STAGED:
// x already sits in wt.x (transferred there by the staged prologue, which
// also waited for the predictor).
template <int N8, int N4, int NZ, int MODE, int WPB, int HPW, bool STAGED = false>
__device__ __forceinline__ void wave_token_build(WaveToken<N8, N4, HPW>& wt, GroupToken<N8 + N4>& gt,
                                                 const WaveRaw<HPW>& r, float2 act, int pv0, int pv1,
                                                 const float (&e0v)[2], const float (&e1v)[2],
                                                 const uint16_t* s_pred, bool first, int lane, int wave) {
  constexpr int NL = N8 + N4, F = NL + 2, RZ = next_pow2(NZ);
  if constexpr (!STAGED) {
#pragma unroll
    for (int k = 0; k < HPW; ++k) wt.x[k][lane] = r.xv[k];
  }
  const float dtv = act.x;
  // gather: raw element i of the B (C) row is half i & 1 of lane i >> 1's pair
  const int braw = (int)((uint32_t)r.bc[0] | ((uint32_t)r.bc[1] << 16));
  const int craw = (int)((uint32_t)r.bc[2] | ((uint32_t)r.bc[3] << 16));
  const uint32_t bw0 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv0 >> 1), braw);
  const uint32_t bw1 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv1 >> 1), braw);
  const uint32_t cw0 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv0 >> 1), craw);
  const uint32_t cw1 = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (pv1 >> 1), craw);
  __builtin_amdgcn_sched_barrier(0);   // all four exchanges in flight before the first use
  const float b0 = h2f((uint16_t)(bw0 >> (16 * (pv0 & 1)))), b1 = h2f((uint16_t)(bw1 >> (16 * (pv1 & 1))));
  const float c0 = h2f((uint16_t)(cw0 >> (16 * (pv0 & 1)))), c1 = h2f((uint16_t)(cw1 >> (16 * (pv1 & 1))));
  // the carried coordinates' b are finite binary16 values (|b| <= 65504)
  const bool b_lane_ok = (lane >= NL || __builtin_fabsf(b0) <= 65504.f) &&
                         (64 + lane >= NL || __builtin_fabsf(b1) <= 65504.f);
  const bool b_ok = __builtin_amdgcn_ballot_w64(!b_lane_ok) == 0;
  if (lane < HPW) {
    wt.dtv[lane] = act.x;
    wt.decay[lane] = act.y;
    wt.bounded[lane] = (b_ok && 65504.f * __builtin_fabsf(act.x) < 0x1p100f && __builtin_fabsf(act.y) < 0x1p100f);
  }
  wt.b[lane] = b0;
  wt.b[64 + lane] = b1;
  wt.c[lane] = c0;
  wt.c[64 + lane] = c1;
#pragma unroll
  for (int k = 0; k < HPW; ++k) {
    const float dk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dtv), k));
    if (lane < NL) wt.bdt[k][lane] = b0 * dk;
    if (64 + lane < NL) wt.bdt[k][64 + lane] = b1 * dk;
  }
  const float sbc = wave_sum(b0 * c0 + b1 * c1);
  if (lane == 0) wt.dots[0] = sbc;
  if constexpr (MODE != MODE_RIDGE) {
    if (lane < NL) wt.cw[lane] = c0;
    if (64 + lane < NL) wt.cw[64 + lane] = c1;
  } else {
    wave_sync();                 // the dead-tier c and b are read across lanes below
    if (!STAGED && first) __syncthreads();  // every wave's share of the predictor transfer has landed
    if constexpr (WPB >= 4) {
      // Split across the workgroup: wave w computes the corrections of
      // internal outputs [w FW, (w + 1) FW), lanes l and l + 32 the two halves
      // of the dead-tier sum of output w FW + (l & 31), and dead-tier tree w
      // (w < 4); readout-only values, except the trees e.b (canonical, exact).
      constexpr int FW = 8 * ((F + 8 * WPB - 1) / (8 * WPB));
      static_assert(FW <= 32, "two lane halves per output");
      const int jo = wave * FW + (lane & 31);
      const uint16_t* pr = s_pred + packed_lane<N8, N4>(min(jo, F - 1)) * NZ;
      constexpr int Q = NZ / 4, QH = (Q + 1) / 2;
      const int qb = (lane >> 5) * QH;
      f32x4 cv[QH];
      uint2 w[QH];
#pragma unroll
      for (int i = 0; i < QH; ++i) {
        const int q = min(qb + i, Q - 1);
        cv[i] = *(const f32x4*)(wt.c + NL + 4 * q);
        w[i] = *(const uint2*)(pr + 4 * q);
      }
      const float cjo = wt.c[min(jo, NL - 1)];   // readout weight base of output jo (< NL)
      // tree `wave` operands (waves 0..3: e0.c, e1.c, e0.b, e1.b), read
      // unconditionally at clamped positions
      const float* src = wave < 2 ? wt.c : wt.b;
      float tv[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int d0 = (RZ == 128) ? 2 * lane + j : lane;
        tv[j] = src[NL + min(d0, NZ - 1)];
      }
      __builtin_amdgcn_sched_barrier(0);
      // tree `wave` (waves past 3 of an eight-wave group compute an unused
      // copy), interleaved by the scheduler with the correction below
      const float (&e)[2] = (wave & 1) ? e1v : e0v;
      float v[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int d0 = (RZ == 128) ? 2 * lane + j : lane;
        const bool in = (RZ == 128 || j == 0) && d0 < NZ;
        v[j] = in ? e[j] * tv[j] : 0.f;
      }
      const float tsum = wave_pair_tree<RZ>(v[0], v[1]);
      float a[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < QH; ++i) {
        f32x4 c4 = cv[i];
        if (Q % 2 && i == QH - 1 && qb + i >= Q) c4 = f32x4{0.f, 0.f, 0.f, 0.f};   // the upper half's extra quad
        a[0] = __builtin_fmaf(c4.x, h2f((uint16_t)w[i].x), a[0]);
        a[1] = __builtin_fmaf(c4.y, h2f((uint16_t)(w[i].x >> 16)), a[1]);
        a[2] = __builtin_fmaf(c4.z, h2f((uint16_t)w[i].y), a[2]);
        a[3] = __builtin_fmaf(c4.w, h2f((uint16_t)(w[i].y >> 16)), a[3]);
      }
      const int part = __builtin_bit_cast(int, (a[0] + a[1]) + (a[2] + a[3]));
      const auto sw = __builtin_amdgcn_permlane32_swap(part, part, false, false);
      const float corr = __builtin_bit_cast(float, (int)sw[0]) + __builtin_bit_cast(float, (int)sw[1]);
      if (lane < FW && jo < F) gt.cw[jo] = (jo < NL ? cjo : 0.f) + corr;
      if (lane == 0 && wave < 4) gt.tree[wave] = tsum;
      __syncthreads();   // the workgroup's shared token values are complete
      return;
    }
    // corr[j] = sum_d C[dead d] * pred[g, row(j), d] for output j = lane and
    // lane + 64 (rows past F recompute row F-1, unused); the dead-tier C is a
    // wave-uniform operand, the predictor row a per-lane one
    const int f0 = packed_lane<N8, N4>(min(lane, F - 1));
    const int f1 = packed_lane<N8, N4>(min(64 + lane, F - 1));
    const uint16_t* p0 = s_pred + f0 * NZ;
    const uint16_t* p1 = s_pred + f1 * NZ;
    // every LDS read of a half is issued before its first use; four partial
    // sums per output (readout-only value: summation order free)
    constexpr int Q = NZ / 4, QH = (Q + 1) / 2;
    float a0[4] = {0.f, 0.f, 0.f, 0.f}, a1[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      f32x4 cv[QH];
      uint2 w0[QH], w1[QH];
#pragma unroll
      for (int i = 0; i < QH; ++i) {
        const int d = 4 * min(h * QH + i, Q - 1);
        cv[i] = *(const f32x4*)(wt.c + NL + d);
        w0[i] = *(const uint2*)(p0 + d);
        if constexpr (F > 64) w1[i] = *(const uint2*)(p1 + d);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < QH; ++i) {
        if (h * QH + i >= Q) break;
        a0[0] = __builtin_fmaf(cv[i].x, h2f((uint16_t)w0[i].x), a0[0]);
        a0[1] = __builtin_fmaf(cv[i].y, h2f((uint16_t)(w0[i].x >> 16)), a0[1]);
        a0[2] = __builtin_fmaf(cv[i].z, h2f((uint16_t)w0[i].y), a0[2]);
        a0[3] = __builtin_fmaf(cv[i].w, h2f((uint16_t)(w0[i].y >> 16)), a0[3]);
        if constexpr (F > 64) {
          a1[0] = __builtin_fmaf(cv[i].x, h2f((uint16_t)w1[i].x), a1[0]);
          a1[1] = __builtin_fmaf(cv[i].y, h2f((uint16_t)(w1[i].x >> 16)), a1[1]);
          a1[2] = __builtin_fmaf(cv[i].z, h2f((uint16_t)w1[i].y), a1[2]);
          a1[3] = __builtin_fmaf(cv[i].w, h2f((uint16_t)(w1[i].y >> 16)), a1[3]);
        }
      }
    }
    const float acc0 = (a0[0] + a0[1]) + (a0[2] + a0[3]);
    const float acc1 = (a1[0] + a1[1]) + (a1[2] + a1[3]);
    if (lane < NL) wt.cw[lane] = c0 + acc0;
    if (64 + lane < NL) wt.cw[64 + lane] = c1 + acc1;
    // correction of the latent coefficients: outputs NL and NL + 1
    const float lc0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                    __builtin_bit_cast(int, NL < 64 ? acc0 : acc1), NL % 64));
    const float lc1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                    __builtin_bit_cast(int, NL + 1 < 64 ? acc0 : acc1), (NL + 1) % 64));
    // dead-tier dot products: canonical adjacent-pair trees (products at
    // 2 lane + j when RZ == 128, else at lane)
    float v[4][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int d0 = (RZ == 128) ? 2 * lane + j : lane;
      const bool in = (RZ == 128 || j == 0) && d0 < NZ;
      const int d = in ? d0 : 0;
      const float bb = wt.b[NL + d], cc = wt.c[NL + d];
      v[0][j] = in ? e0v[j] * cc : 0.f;
      v[1][j] = in ? e1v[j] * cc : 0.f;
      v[2][j] = in ? e0v[j] * bb : 0.f;
      v[3][j] = in ? e1v[j] * bb : 0.f;
    }
    const float ec0 = wave_pair_tree<RZ>(v[0][0], v[0][1]);
    const float ec1 = wave_pair_tree<RZ>(v[1][0], v[1][1]);
    const float eb0 = wave_pair_tree<RZ>(v[2][0], v[2][1]);
    const float eb1 = wave_pair_tree<RZ>(v[3][0], v[3][1]);
    if (lane == 0) {
      wt.dots[1] = ec0 + lc0;
      wt.dots[2] = ec1 + lc1;
      wt.dots[3] = eb0;
      wt.dots[4] = eb1;
    }
  }
  wave_sync();
}

// One tier of a row: update its N carried coordinates (biased code bytes in
// c[0 .. N/4)), accumulate the readout, then requantize with den =
// max(RN(amax / lim), 1e-8) and the stored (binary16) scale, writing the new
// codes back into c.  INT8: byte = q + 128, lim 127; INT4: byte = q + 8,
// lim 7.  Legacy mode quantizes with the binary32 denominator.
//
// Clamping the rounded quotient to +-lim only matters when the divisor is
// below den (a binary16-subnormal stored scale) or when an update is not
// finite.  `finite_in` (per lane) says the update cannot overflow or be NaN
// (finite scale, x, decay and B*dt of bounded size); when it holds on every
// lane and every stored scale is zero, infinite or a normal binary16 value,
// |RN(u / s)| <= lim (1 + 2^-11) / (1 - 2^-24) < lim + 1/2 and the wave takes
// the quantizer without the clamp.
//
// EXACT selects the dequantization form: false (every scale of the wave
// finite) the fused (1024 + q + bias) * s - (1024 + bias) * s, one fma per
// coordinate (exact: both products have at most 22 significant bits); true
// q * s as a packed binary16 subtraction and a product, which is also the
// IEEE product for infinite and NaN scales (where the fused form gives
// inf - inf).
//
// Readout: rs[sg] is set, for each readout segment sg the tier's
// coordinates reach, to the binary32 chain of prior * w over them (w the
// readout weights; one segment's chain is live at a time, segments being
// contiguous runs of chunks).  `bdt4` and `cw4` are the head's B*dt and the
// readout weights of the carried coordinates, as four-value chunks (BMUL:
// `bdt4` holds b, and B * dt is formed here with dtk).
//
// tier_update is the first half (dequantization, readout, update and the
// maximum of |update|), tier_requant the second (the new scale and codes
// from the maximum over the whole tier): a tier split between waves runs the
// halves on its parts with the parts' maxima combined in between.
template <int N, bool INT8, bool EXACT, int N8, int N4, int P0, bool BMUL = false>
__device__ __forceinline__ float tier_update(const uint32_t* c, float sc, float decay, float x, const f32x4* bdt4,
                                             const f32x4* cw4, float (&rs)[4], float (&v)[N], float dtk = 0.f) {
  constexpr float BIAS = INT8 ? 128.0f : 8.0f;
  static_assert(P0 % 4 == 0 && N % 4 == 0, "whole chunks");
  const float nb = -(1024.0f + BIAS) * sc;
  const f16x2 nbias = {(_Float16)(-(1024.0f + BIAS)), (_Float16)(-(1024.0f + BIAS))};
  const float mz = EXACT ? opaque_neg_zero() : 0.f;
  float amax = 0.f;
  float racc = 0.f;   // the current segment's readout chain
  // the shared operands of chunk i+1 are read while chunk i computes
  constexpr int C0 = P0 / 4;
  f32x4 cb_next = bdt4[C0], cw_next = cw4[C0];
#pragma unroll
  for (int i0 = 0; i0 < N; i0 += 4) {
    const int ci = C0 + i0 / 4;   // chunk index among the carried coordinates
    // BMUL: bdt4 holds b, and B * dt is formed here (the same RN(b * dt))
    const f32x4 cb = BMUL ? cb_next * dtk : cb_next, cw = cw_next;
    if (i0 + 4 < N) {
      cb_next = bdt4[ci + 1];
      cw_next = cw4[ci + 1];
    }
    // the chunk's code bytes as binary16 values 1024 + byte (exponent byte
    // 0x64), formed here (the empty asm keeps the compiler from forming every
    // chunk's pairs ahead of the tier, which would hold them all live)
    uint32_t cc = c[i0 / 4];
    asm volatile("" : "+v"(cc));
    const uint32_t h01 = __builtin_amdgcn_perm(0x64646464u, cc, 0x04010400u);
    const uint32_t h23 = __builtin_amdgcn_perm(0x64646464u, cc, 0x04030402u);
    const int sg = seg_of<N8, N4>(P0 + i0);   // a whole chunk lies in one segment
    float pr[4];
    if constexpr (EXACT) {
      const f16x2 q01 = pk_add_h(__builtin_bit_cast(f16x2, h01), nbias);
      const f16x2 q23 = pk_add_h(__builtin_bit_cast(f16x2, h23), nbias);
#pragma unroll
      for (int j = 0; j < 4; ++j) pr[j] = dequant_h((j < 2 ? q01 : q23)[j & 1], sc, mz);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) pr[j] = __builtin_fmaf(h2f((uint16_t)((j < 2 ? h01 : h23) >> (16 * (j & 1)))), sc, nb);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      racc = __builtin_fmaf(pr[j], cw[j], racc);
      float u = state_update(pr[j], decay, cb[j] * x);
      // ordered pin: chunk by chunk, each prior dies as soon as it is used
      asm volatile("" : "+v"(u));
      v[i0 + j] = u;
    }
    amax = max3_abs(amax, v[i0], v[i0 + 1]);
    amax = max3_abs(amax, v[i0 + 2], v[i0 + 3]);
    if (i0 + 4 == N || seg_of<N8, N4>(P0 + i0 + 4) != sg) {   // the segment's last chunk in this tier
      rs[sg] = racc;
      racc = 0.f;
    }
  }
  // Materialize the readout and the maximum here: otherwise the compiler
  // sinks their chains (and every update behind the maximum) into the
  // requantization, which keeps every prior and LDS operand live at once.
  constexpr int G0 = seg_of<N8, N4>(P0), G1 = seg_of<N8, N4>(P0 + N - 1);
#pragma unroll
  for (int sg = G0; sg <= G1; ++sg) asm volatile("" : "+v"(rs[sg]));
  asm volatile("" : "+v"(amax));
  return amax;
}

// Readout of segment sg: its INT8 tier contribution, then its INT4 one.
template <int N8, int N4>
__device__ __forceinline__ float segment_readout(int sg, float c8, float c4) {
  const bool h8 = seg_pos(N8, N4, sg) < N8, h4 = seg_pos(N8, N4, sg + 1) > N8;
  return (h8 && h4) ? c8 + c4 : (h8 ? c8 : c4);
}

template <int N, bool INT8, int MODE>
__device__ __forceinline__ float tier_requant(const float (&v)[N], uint32_t* c, float amax, bool finite_in) {
  constexpr float BIAS = INT8 ? 128.0f : 8.0f;
  constexpr float LIM = INT8 ? 127.0f : 7.0f;
  constexpr float TOP = INT8 ? QTOP127 : QTOP7;
  const float den = requant_den(amax, LIM, 1.0f / LIM);
  const float stored = round_to_half(den);
  float d, r;
  bool unclamped;
  // stored scale not > 0: the reference's code is 0 whatever the update
  // (also NaN): the clamp bound is then 0 (clamp(NaN, -0, 0) is -0 or 0)
  float top = TOP;
  if constexpr (MODE == MODE_LEGACY) {
    // an infinite den divides through d = 1, y = 0: RN(v / inf) is 0 for
    // finite v (NaN, clamped to -lim, for infinite v, as IEEE gives)
    const bool inf = den == __builtin_inff();
    d = inf ? 1.0f : den;
    r = inf ? 0.0f : 1.0f / den;
    unclamped = finite_in;
  } else {
    // zero (underflowed) or infinite stored scale: the reference's quotient
    // is 0 and so is the code
    const bool zero = !(stored > 0.f) || stored == __builtin_inff();
    d = zero ? 1.f : stored;
    r = zero ? 0.f : recip_half(stored);
    unclamped = finite_in && (zero || stored >= 0x1p-14f);
    top = stored > 0.f ? TOP : 0.0f;
  }
  // wave-uniform choice, re-tested per chunk (a branch around the whole loop
  // makes the register allocator keep both versions' values apart)
  const bool fast = __builtin_amdgcn_ballot_w64(!unclamped) == 0;
  if (fast) {
    // the biased code as the low byte of t = RN(u yh + 1.5 2^23 + bias) =
    // 1.5 2^23 + bias + rint(u yh), kept where the code of the other side,
    // RN(u yl + ...), agrees (two_sided_code)
    const float yh = __builtin_fmaf(r, TWO_SIDED_REL, r), yl = __builtin_fmaf(r, -TWO_SIDED_REL, r);
    uint32_t diff = 0u;
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      uint32_t tb[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tb[j] = two_sided_code(v[4 * i + j], yh, yl, BIAS, diff);
        asm volatile("" : "+v"(diff));   // one three-input bitwise operation per coordinate
      }
      uint32_t packed = pack4((int)tb[0], (int)tb[1], (int)tb[2], (int)tb[3]);
      asm volatile("" : "+v"(packed));
      c[i] = packed;
    }
    // A lane whose two codes differ has a half-integer between u yl and u
    // yh: the wave then requantizes the tier with the exact quotients (rare:
    // the window is 2^-21 of the quotient wide).
    if (__builtin_amdgcn_ballot_w64(diff != 0u) != 0) {
#pragma unroll
      for (int i = 0; i < N / 4; ++i) {
        const int q0 = quantize_code_unclamped(v[4 * i], d, r);
        const int q1 = quantize_code_unclamped(v[4 * i + 1], d, r);
        const int q2 = quantize_code_unclamped(v[4 * i + 2], d, r);
        const int q3 = quantize_code_unclamped(v[4 * i + 3], d, r);
        uint32_t packed = pack4(q0, q1, q2, q3);
        packed = INT8 ? (packed ^ 0x80808080u) : ((packed & 0x0F0F0F0Fu) ^ 0x08080808u);
        c[i] = packed;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const int q0 = quantize_code(v[4 * i], d, r, top);
      const int q1 = quantize_code(v[4 * i + 1], d, r, top);
      const int q2 = quantize_code(v[4 * i + 2], d, r, top);
      const int q3 = quantize_code(v[4 * i + 3], d, r, top);
      uint32_t packed = pack4(q0, q1, q2, q3);
      packed = INT8 ? (packed ^ 0x80808080u) : ((packed & 0x0F0F0F0Fu) ^ 0x08080808u);
      asm volatile("" : "+v"(packed));
      c[i] = packed;
    }
  }
  return stored;
}

// One workgroup = WPB waves, each owning HPW head slots of 64 rows (the same
// P block of NH = WPB * HPW consecutive heads of one B/C group and batch
// row).  The packed rows of every slot stay in LDS, in the reference's SoA
// field layout, for all L tokens; a slot is unpacked into VGPRs, stepped and
// repacked in one pass per token.  The first token streams the slots in:
// slot k+1 is fetched while slot k computes.  Every wave builds the token
// values it reads itself, so the only workgroup barrier is the one that
// publishes the ridge predictor (staged once, shared by all waves).
// LDS of one workgroup: the waves' token records, the shared ridge-correction
// record(s), the staged predictor and the slot tiles.
// WPS > 1: the small-batch layouts, two or four waves per head slot (HPW ==
// 1), each stepping the coordinates of its readout segments, so that each
// slot's serial chain is about half or a quarter as long; `pacc` and `pmax`
// pass the waves' readout partial sums and tier maxima (one buffer per token
// parity).
template <int N8, int N4, int NZ, int MODE, int WPB, int HPW, bool DMA, bool ONE, int WPS = 1, bool REC = false>
struct StepSmem {
  static constexpr bool PAIR = WPS > 1;
  static_assert(WPS == 1 || ((WPS == 2 || WPS == 4) && HPW == 1 && WPB % WPS == 0),
                "two or four waves per head slot, one slot each");
  static_assert(seg_layout_ok(N8, N4), "four non-empty readout segments");
  static constexpr int NL = N8 + N4, F = NL + 2, NH = PAIR ? WPB / WPS : WPB * HPW;
  static constexpr bool RIDGE = MODE == MODE_RIDGE, SPLIT = RIDGE && WPB >= 4;
  // one-token instances of four or more waves stage their token inputs in
  // LDS by direct transfers (one shared transfer per wave)
  static constexpr bool STAGED = DMA && ONE && WPB >= 4 && NH <= 16;
  // REC: the record-fed instance (multi-token ridge, several waves per slot,
  // 16-byte transfers): three record buffers (token t mod 3), and the prior
  // latent coefficients the last wave of a slot passes to its reading wave
  // (per token parity)
  static_assert(!REC || (RIDGE && PAIR && SPLIT && !ONE && DMA), "record-fed instances");
  // slot tile: lo, hi, q4, s8, s4 (and latent) fields of 64 rows, 16 bytes of slack
  static constexpr int TILE = 128 * (N8 / 2) + 64 * (N4 / 2) + 256 + (RIDGE ? 128 : 0) + 16;
  static constexpr int PRED_DW = RIDGE ? F * NZ / 2 : 1;
  static constexpr int PRED_WORDS = DMA ? (PRED_DW + 255) / 256 * 256 : (PRED_DW + 63) / 64 * 64;
  alignas(16) WaveToken<N8, N4, HPW> wt[WPB];
  // split ridge correction: one record per token parity (a wave may build
  // token t + 1 while another still reads token t)
  alignas(16) GroupToken<NL> gt[SPLIT && !ONE ? 2 : 1];
  alignas(16) uint32_t pred32[PRED_WORDS];
  alignas(16) std::conditional_t<STAGED, TokenStage, NoStage> stage;
  alignas(16) float rec[REC ? 3 : 1][REC ? REC_FLOATS : 4];
  alignas(16) float2 pz[REC ? 2 : 1][REC ? NH : 1][REC ? 64 : 1];
  // WPS > 1 (per token parity): the readout partial sums of waves 0 ..
  // WPS - 2 of a slot, and every wave's maxima of its INT8 and INT4 parts
  alignas(16) float pacc[PAIR ? 2 : 1][PAIR ? NH : 1][PAIR ? WPS : 1][PAIR ? 64 : 1];
  alignas(16) float pmax[PAIR ? 2 : 1][PAIR ? NH : 1][2][PAIR ? WPS : 1][PAIR ? 64 : 1];
  alignas(16) uint8_t tile[NH][TILE];
#ifdef M2R_PHASE_TIMELINE
  unsigned long long stamps[WPB][32];
#endif
};

// The step of one workgroup: block coordinates (bx, by) and batch row b,
// arguments `a`, LDS `sm`.  k_state_step runs it on its own grid; the
// multi-layer kernel runs it with arguments read from a table of layers.
template <int N8, int N4, int NZ, int MODE, int WPB, int HPW, bool DMA, bool ONE, int WPS = 1, bool REC = false>
__device__ __forceinline__ void state_step_body(const StepArgs& a,
                                                StepSmem<N8, N4, NZ, MODE, WPB, HPW, DMA, ONE, WPS, REC>& sm, int bx,
                                                int by, int b) {
  constexpr bool PAIR = WPS > 1;      // several waves per slot
  constexpr int W8 = N8 / 2;          // bytes per row of lo and of hi
  constexpr int W4 = N4 / 2;          // bytes per row of q4
  constexpr int NL = N8 + N4;         // carried coordinates
  constexpr int F = NL + 2;           // ridge predictor features
  constexpr int NH = PAIR ? WPB / WPS : WPB * HPW;
  constexpr int RZ = next_pow2(NZ);
  constexpr bool RIDGE = MODE == MODE_RIDGE;
  constexpr int O_LO = 0, O_HI = 64 * W8, O_Q4 = 128 * W8, O_S8 = O_Q4 + 64 * W4, O_S4 = O_S8 + 128;
  constexpr int O_LAT = O_S4 + 128;
  constexpr int TILE = O_LAT + (RIDGE ? 128 : 0) + 16;   // 16 bytes of slack for row reads
  constexpr int C8 = N8 / 4, C4 = N4 / 4;   // carried code words (4 biased bytes each)
  constexpr int PRED_DW = RIDGE ? F * NZ / 2 : 1;   // F*NZ is even for every layout
  constexpr int PRED_OPS = (PRED_DW + 63) / 64;     // 64-dword transfers of the predictor
  constexpr int PRED_OPS16 = (PRED_DW + 255) / 256; // 1 KiB transfers (aligned predictor)
  static_assert(!RIDGE || (F * NZ * 2) % 16 == 0, "a group's predictor is a whole number of 16-byte chunks");
  static_assert(N8 % 4 == 0 && N4 % 4 == 0 && N8 > 0 && N4 > 0, "tier widths must be positive multiples of 4");
  static_assert(NZ % 4 == 0 && NL + NZ == 128, "dead tier read as 4-wide vectors");
  static_assert(!RIDGE || (F * NZ) % 2 == 0, "predictor staged as dwords");
  static_assert(TILE % 16 == 0, "tiles stay 16-byte aligned");

  using Smem = StepSmem<N8, N4, NZ, MODE, WPB, HPW, DMA, ONE, WPS, REC>;
  static_assert(Smem::TILE == TILE && Smem::PRED_WORDS == (DMA ? PRED_OPS16 * 256 : PRED_OPS * 64), "LDS layout");
  constexpr bool SPLIT = Smem::SPLIT;
  // REC, the record-fed token loop (StepArgs::rec): every token's
  // state-independent values come from its record in LDS.  Wave REC_LOADER
  // loads record t + 2 while token t steps, and puts record t + 1 in LDS
  // before token t's maxima barrier, so that the maxima barrier is the only
  // workgroup barrier of a token (after the first).
  constexpr int REC_LOADER = 1;
  auto& s_wt = sm.wt;
  auto& s_gt = sm.gt;
  auto& s_pred32 = sm.pred32;
  auto& s_tile = sm.tile;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: per-wave values in SGPRs
  M2R_STAMP_REAL(ST_REAL0);
  M2R_STAMP(ST_START);
  // WPS > 1: the wave's role in its slot (0: also moves the INT8 fields;
  // WPS - 1: also moves the INT4 fields, steps the latent coefficients and
  // reads the rows out)
  const int role = PAIR ? (wave & (WPS - 1)) : 0;
  // workgroup-local head of the wave's slot k
  auto head_slot = [&](int k) { return PAIR ? wave / WPS : wave * HPW + k; };
  const int h0 = by * NH;
  const int H = a.H, P = a.P;
  // ONE: the one-token (decode) instance, with a compile-time token count:
  // no token loop, prefetch or loop-carried state
  const int L = ONE ? 1 : a.L;
  const int g = group_of_head(h0, a.rhpg);
  const int pbase = bx * 64;
  const int nvalid = min(64, P - pbase);
  const bool valid = lane < nvalid;
  // Rows past P need finite placeholders only when their tile rows hold
  // stale LDS: the 16-byte transfers fill them with copies of the last
  // valid chunk (finite codes and scales, stepped like any row and never
  // stored), the register copies leave them as they were.
  constexpr bool PLACEHOLDERS = !DMA;
  constexpr bool dma_tiles = DMA;   // a.dma_tiles: 16-byte LDS transfers, else staging through VGPRs
  // Cache policies.  The shapes of one slot per wave (HPW == 1, which the
  // launch picks below 4,096 slots when the heads per group allow wider
  // ones) read the state and the predictor as ordinary lines: at small
  // batches the next launch of the same layer finds them in the L2.  The
  // shapes of several slots per wave (large batches, whose states exceed
  // the L2s) read them non-temporal.  The multi-wave slots (at most 1,024)
  // also keep their stored lines in the L2 (written through at device
  // scope); the others store non-temporal.
  constexpr bool NT_LOAD = HPW > 1;
  constexpr int STORE_CP = PAIR ? STORE_DEVICE : STORE_THROUGH;
  const uint16_t* s_pred = (const uint16_t*)s_pred32;
  WaveToken<N8, N4, HPW>& wt = s_wt[wave];

  // vector memory operations per slot transfer (and per state copy-out); on
  // a slot of several waves wave 0 transfers the INT8 tier's fields (lo, hi
  // and s8: OPS8), the last wave the INT4 tier's (q4, s4 and the latent
  // bytes: OPS4), the others none (the two-byte fields of a transfer go in
  // one operation: s8, s4 and the latent bytes of a one-wave slot; s8, or s4
  // and the latent bytes, on a slot of several waves)
  constexpr int C8W = chunk_ops(W8), C4W = chunk_ops(W4);
  constexpr int OPS8 = 2 * C8W + 1;
  constexpr int OPS4 = C4W + 1;
  constexpr int SLOT_DMA = PAIR ? OPS8 + OPS4 : 2 * C8W + 1 + C4W;
  static_assert(SLOT_DMA <= 63, "a slot's transfers must fit the vmcnt range");
  static_assert(O_S4 == O_S8 + 128 && O_LAT == O_S4 + 128, "two-byte fields back to back in the tile");
  const bool own8 = !PAIR || role == 0, own4 = !PAIR || role == WPS - 1;   // the fields this wave moves
  auto slot_row0 = [&](int hh) { return (b * H + h0 + hh) * P + pbase; };
  auto slot_dma = [&](int hh) {   // direct global -> LDS transfers
    const int row0 = slot_row0(hh);
    uint8_t* t = s_tile[hh];
    // the INT8 tier's fields first (with all two-byte fields in a one-wave
    // slot): the first slot's INT8 tier starts when they have landed
    const uint32_t tl = lds_address(t);
    const uint8_t *s8 = (const uint8_t*)a.s8, *s4 = (const uint8_t*)a.s4;
    if constexpr (!PAIR) {
      field_dma16_tile<W8, O_LO, NT_LOAD>(tl, a.lo, row0, nvalid, lane);
      field_dma16_tile<W8, O_HI, NT_LOAD>(tl, a.hi, row0, nvalid, lane);
      scale_fields_dma16_tile<RIDGE ? 3 : 2, O_S8, NT_LOAD>(tl, s8, s4, RIDGE ? a.latent : s4, row0, nvalid, lane);
      field_dma16_tile<W4, O_Q4, NT_LOAD>(tl, a.q4, row0, nvalid, lane);
    } else if (own8) {
      field_dma16_tile<W8, O_LO, NT_LOAD>(tl, a.lo, row0, nvalid, lane);
      field_dma16_tile<W8, O_HI, NT_LOAD>(tl, a.hi, row0, nvalid, lane);
      scale_fields_dma16_tile<1, O_S8, NT_LOAD>(tl, s8, s8, s8, row0, nvalid, lane);
    } else if (own4) {
      field_dma16_tile<W4, O_Q4, NT_LOAD>(tl, a.q4, row0, nvalid, lane);
      scale_fields_dma16_tile<RIDGE ? 2 : 1, O_S4, NT_LOAD>(tl, s4, RIDGE ? a.latent : s4, s4, row0, nvalid, lane);
    }
  };
  // store instructions of a slot's copy-out (one per 1 KiB chunk of a field)
  constexpr int COPY_OPS = 2 * C8W + C4W + (RIDGE ? 3 : 2);
  static_assert(SLOT_DMA + COPY_OPS + 1 <= 63, "vmcnt range");
  // At the first token, before slot k is read: wait until only the
  // operations issued after slot k's transfers are outstanding (vector memory
  // operations complete in program order), so no wait covers a store's write
  // acknowledgement.  Slot k's transfers are issued in the middle of slot
  // k-1 (slot 0's by the prologue); after them come slot k-2's state
  // copy-out when the first token is also the last (copy-outs trail by one
  // slot, also issued mid-slot) and slot k-1's y store (one store
  // instruction).  (Loads the compiler issues in between, the next token's
  // prefetch, only make a wait longer.)
  // (The one-wave slot waits at slot 0 only for the INT8 fields, issued
  // first; it waits for the INT4 fields after the INT8 tier.)
  auto slot_wait = [&](int k) {
    const bool copy = L == 1 && k >= 2;
    if (k == 0) {
      if (dma_tiles && !PAIR) wait_vmcnt<C4W>();
      else wait_vmcnt<0>();
    }
    else if (copy) wait_vmcnt<COPY_OPS + 1>();
    else wait_vmcnt<1>();
  };
  auto slot_copy_in = [&](int hh) {   // other geometries: 16-bit transfers through VGPRs
    const int row0 = slot_row0(hh);
    uint8_t* t = s_tile[hh];
    if (own8) {
      wave_copy_in<W8>(t + O_LO, a.lo, row0, nvalid, lane);
      wave_copy_in<W8>(t + O_HI, a.hi, row0, nvalid, lane);
      wave_copy_in<2>(t + O_S8, (const uint8_t*)a.s8, row0, nvalid, lane);
    }
    if (own4) {
      wave_copy_in<W4>(t + O_Q4, a.q4, row0, nvalid, lane);
      wave_copy_in<2>(t + O_S4, (const uint8_t*)a.s4, row0, nvalid, lane);
      if constexpr (RIDGE) wave_copy_in<2>(t + O_LAT, a.latent, row0, nvalid, lane);
    }
  };
  auto slot_copy_out = [&](int hh) {
    const int row0 = slot_row0(hh);
    const uint8_t* t = s_tile[hh];
    if constexpr (dma_tiles && PAIR) {   // this wave's fields: every LDS read, then the stores
      constexpr int C8W = chunk_ops(W8), C4W = chunk_ops(W4), C2 = chunk_ops(2);
      // store chunks per role: lo, hi and s8; q4, s4 (and the latent bytes)
      constexpr int COPY8 = 2 * C8W + 1, COPY4 = C4W + (RIDGE ? 2 : 1);
      u32x4 v[COPY8 > COPY4 ? COPY8 : COPY4];
      if (own8) {
        field_read16<W8>(t + O_LO, lane, v);
        field_read16<W8>(t + O_HI, lane, v + C8W);
        field_read16<2>(t + O_S8, lane, v + 2 * C8W);
        field_write16<W8, STORE_CP>(a.lo, v, row0, nvalid, lane);
        field_write16<W8, STORE_CP>(a.hi, v + C8W, row0, nvalid, lane);
        field_write16<2, STORE_CP>((uint8_t*)a.s8, v + 2 * C8W, row0, nvalid, lane);
      } else if (own4) {
        field_read16<W4>(t + O_Q4, lane, v);
        field_read16<2>(t + O_S4, lane, v + C4W);
        if constexpr (RIDGE) field_read16<2>(t + O_LAT, lane, v + C4W + C2);
        field_write16<W4, STORE_CP>(a.q4, v, row0, nvalid, lane);
        field_write16<2, STORE_CP>((uint8_t*)a.s4, v + C4W, row0, nvalid, lane);
        if constexpr (RIDGE) field_write16<2, STORE_CP>(a.latent, v + C4W + C2, row0, nvalid, lane);
      }
      return;
    } else if constexpr (dma_tiles) {   // every LDS read of the slot, then its stores
      constexpr int C8W = chunk_ops(W8), C4W = chunk_ops(W4), C2 = chunk_ops(2);
      u32x4 v[COPY_OPS];
      field_read16<W8>(t + O_LO, lane, v);
      field_read16<W8>(t + O_HI, lane, v + C8W);
      field_read16<W4>(t + O_Q4, lane, v + 2 * C8W);
      field_read16<2>(t + O_S8, lane, v + 2 * C8W + C4W);
      field_read16<2>(t + O_S4, lane, v + 2 * C8W + C4W + C2);
      if constexpr (RIDGE) field_read16<2>(t + O_LAT, lane, v + 2 * C8W + C4W + 2 * C2);
      field_write16<W8>(a.lo, v, row0, nvalid, lane);
      field_write16<W8>(a.hi, v + C8W, row0, nvalid, lane);
      field_write16<W4>(a.q4, v + 2 * C8W, row0, nvalid, lane);
      field_write16<2>((uint8_t*)a.s8, v + 2 * C8W + C4W, row0, nvalid, lane);
      field_write16<2>((uint8_t*)a.s4, v + 2 * C8W + C4W + C2, row0, nvalid, lane);
      if constexpr (RIDGE) field_write16<2>(a.latent, v + 2 * C8W + C4W + 2 * C2, row0, nvalid, lane);
      return;
    }
    if (own8) {
      wave_copy_out<W8>(a.lo, t + O_LO, row0, nvalid, lane);
      wave_copy_out<W8>(a.hi, t + O_HI, row0, nvalid, lane);
      wave_copy_out<2>((uint8_t*)a.s8, t + O_S8, row0, nvalid, lane);
    }
    if (own4) {
      wave_copy_out<W4>(a.q4, t + O_Q4, row0, nvalid, lane);
      wave_copy_out<2>((uint8_t*)a.s4, t + O_S4, row0, nvalid, lane);
      if constexpr (RIDGE) wave_copy_out<2>(a.latent, t + O_LAT, row0, nvalid, lane);
    }
  };

  WaveRaw<HPW> raw;
  float Ah;
  // Multi-token instances compute the dt activation 64 tokens at a time:
  // lane j of act64[k] holds (dtv, decay) of token t0 + j for head slot k
  // (one binary64 chain per 64 tokens instead of one per token); each
  // token's values are read back with v_readlane.  Same arithmetic as
  // wave_dt_activation, so the same bits.
  float2 act64[ONE ? 1 : HPW];
  auto batch_activation = [&](int t0) {
    const int tt = min(t0 + lane, L - 1);
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const int h = h0 + head_slot(k);
      const float dtf = h2f(a.dt[((size_t)b * L + tt) * H + h]);
      const float db = a.db_f32 ? ((const float*)a.dt_bias)[h] : h2f(((const uint16_t*)a.dt_bias)[h]);
      act64[k] = dt_activation<true>(dtf + db, a.A[h]);   // (rare: constants in vector registers)
    }
  };
  auto token_act = [&](int t) {   // lane k < HPW: head slot k's values of token t
    const int j = t & 63;
    float2 r = make_float2(0.f, 0.f);
#pragma unroll
    for (int k = HPW - 1; k >= 0; --k) {
      const float x = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, act64[k].x), j));
      const float y = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, act64[k].y), j));
      if (k == HPW - 1 || lane == k) r = make_float2(x, y);
    }
    return r;
  };
  uint32_t d_bits, perm0, perm1;
  uint32_t basis_w[2] = {0u, 0u};
  uint32_t ls_w = 0u;
  float2 act;
  // record-fed loop: the loader's copies of records t + 1 and t + 2 (16
  // bytes per lane), and rec_load(t), this lane's 16 bytes of the record of
  // token t of the workgroup's batch row and group
  uint4 rnext = make_uint4(0u, 0u, 0u, 0u), rnext2 = make_uint4(0u, 0u, 0u, 0u);
  auto rec_load = [&](int t) {
    return ((const uint4*)(a.rec + ((size_t)(b * L + t) * a.G + g) * REC_FLOATS))[lane];
  };
  if constexpr (Smem::STAGED) {
    // ---- staged prologue (one token, LDS transfers): the vector inputs of
    // the token and the statics travel by direct transfers into LDS together
    // with the predictor and the wave's first slot, and the per-head scalars
    // by scalar loads, so that no compiler-visible vector load is
    // outstanding.  The dt activation runs while the transfers are in flight;
    // the wave then waits once for everything but its slot transfers (which
    // keep landing while the token is built), and the workgroup barrier
    // publishes every wave's share.  Shared transfers (B row, C row,
    // permutation and basis) are spread over the waves; each wave transfers x
    // of its own head slots straight into its token record.
    TokenStage& st = sm.stage;
    const int bt = b;   // b * L with L == 1
    load_args(a);
    M2R_STAMP(ST_ARGS);
    // shared transfer j by wave j, branch-free: the B row (0), the C row (1),
    // the permutation bytes and the first 32 basis pairs (2), basis pairs
    // 32 .. NZ - 1 (3)
    constexpr int SHARED_OPS = RIDGE ? 4 : 3;
    static_assert(WPB >= SHARED_OPS, "at most one shared transfer per wave");
    if (wave < SHARED_OPS) {
      const uint8_t* bc = (const uint8_t*)(wave == 0 ? a.Bm : a.Cm) + ((size_t)bt * a.G + g) * 256;
      const uint8_t* prm = a.perm + (size_t)g * 128;
      const uint8_t* bas = RIDGE ? (const uint8_t*)a.basis + (size_t)g * NZ * 4 : prm;
      const int bi = wave == 2 ? lane - 32 : lane + 32;   // basis pair of this lane (waves 2 and 3)
      const uint8_t* src = wave < 2 ? bc + 4 * lane
                           : ((wave == 2 && (lane < 32 || !RIDGE)) ? prm + 4 * (lane & 31) : bas + 4 * min(bi, NZ - 1));
      lds_dma_b32(src, lds_address(st.b + 64 * wave));
    }
    // (after the shared transfers, which the token build waits for first)
    // the per-head scalars of the wave's head slots, heads hf .. hf + HPW - 1
    // (one when HPW == 1; hf is even when HPW > 1, as h0 is): per array the
    // dwords holding them, by at most two scalar loads, all issued before the
    // first wait.  An array of binary16 or binary32 values (D, dt_bias) is
    // read as DW dwords, then DW more that only the binary32 case uses (the
    // binary16 case re-reads the first ones: nothing past the wave's heads
    // is read).
    constexpr int DW = (HPW + 1) / 2;   // dwords holding HPW binary16 values
    const int hf = h0 + head_slot(0), he = hf & ~1;
    uint32_t wdt[DW], wA[HPW], wD[2 * DW], wdb[2 * DW];
    scalar_dwords<DW>(a.dt + ((size_t)bt * H + he), wdt);
    scalar_dwords<HPW>(a.A + hf, wA);
    {
      const uint8_t* pd = a.d_f32 ? (const uint8_t*)((const uint32_t*)a.D + hf) : (const uint8_t*)((const uint16_t*)a.D + he);
      const uint8_t* pb = a.db_f32 ? (const uint8_t*)((const uint32_t*)a.dt_bias + hf)
                                   : (const uint8_t*)((const uint16_t*)a.dt_bias + he);
      scalar_dwords<DW>(pd, wD);
      scalar_dwords<DW>(a.d_f32 && HPW > 1 ? pd + 4 * DW : pd, wD + DW);
      scalar_dwords<DW>(pb, wdb);
      scalar_dwords<DW>(a.db_f32 && HPW > 1 ? pb + 4 * DW : pb, wdb + DW);
    }
    if constexpr (RIDGE) ls_w = scalar_dword(a.lscale + 2 * g);
    if constexpr (RIDGE) {   // the predictor: 16-byte chunks; lanes past the end re-read the last one
      const uint8_t* pg = (const uint8_t*)(a.pred + (size_t)g * F * NZ);
      for (int j = wave; j < PRED_OPS16; j += WPB)
        lds_dma_b128<NT_LOAD>(pg + 16 * min(j * 64 + lane, PRED_DW / 4 - 1), lds_address(s_pred32 + 256 * j));
    }
#pragma unroll
    for (int j = 0; j < (HPW + 1) / 2; ++j) {   // x of head slots 2j (lanes < 32) and 2j + 1
      const int k = 2 * j + (lane >> 5);
      const int hk = h0 + head_slot(min(k, HPW - 1));
      const uint16_t* src = a.x + ((size_t)bt * H + hk) * P + pbase + 2 * min(lane & 31, nvalid / 2 - 1);
      if (HPW % 2 == 0 || k < HPW) lds_dma_b32(src, lds_address(&wt.x[2 * j][0]));
    }
    M2R_STAMP(ST_ISSUED);
    slot_dma(head_slot(0));
    M2R_STAMP(ST_SLOT0_ISSUED);
    // head slot k's values (binary16 bits, or binary32 bits of D and
    // dt_bias), then head slot `lane`'s in lanes < HPW (the others take the
    // last slot's)
    uint32_t sdt[HPW], sdb[HPW], sA[HPW], sD[HPW];
#pragma unroll
    for (int k = 0; k < HPW; ++k) {
      const int hsh = HPW > 1 ? 16 * (k & 1) : 16 * (hf & 1);   // the head's half of its dword
      sdt[k] = (wdt[k / 2] >> hsh) & 0xFFFFu;
      sA[k] = wA[k];
      sD[k] = a.d_f32 ? wD[k] : (wD[k / 2] >> hsh) & 0xFFFFu;
      sdb[k] = a.db_f32 ? wdb[k] : (wdb[k / 2] >> hsh) & 0xFFFFu;
    }
    uint32_t vdt = sdt[HPW - 1], vdb = sdb[HPW - 1], vA = sA[HPW - 1], vD = sD[HPW - 1];
#pragma unroll
    for (int k = HPW - 2; k >= 0; --k) {
      vdt = lane == k ? sdt[k] : vdt;
      vdb = lane == k ? sdb[k] : vdb;
      vA = lane == k ? sA[k] : vA;
      vD = lane == k ? sD[k] : vD;
    }
    raw.dt = (uint16_t)vdt;
    raw.db_lo = (uint16_t)vdb;
    raw.db_hi = a.db_f32 ? (uint16_t)(vdb >> 16) : (uint16_t)vdb;
    Ah = __builtin_bit_cast(float, vA);
    d_bits = vD;
    // (with two waves per SIMD the prologue's scalar issue is its
    // bottleneck: the binary64 constants go in vector registers; the
    // multi-wave slots, one wave per SIMD, keep them in scalar ones; one
    // evaluation per launch, so plain immediates)
    act = wave_dt_activation<HPW, !PAIR, KM_PLAIN>(raw, Ah, a.db_f32);
#ifdef M2R_PHASE_TIMELINE
    asm volatile("" ::"v"(act.x), "v"(act.y));   // the activation is complete at its stamp
#endif
    M2R_STAMP(ST_ACT);
    // this wave's token, statics and predictor transfers have landed
    if (!PAIR) wait_vmcnt<SLOT_DMA>();
    else if (own8) wait_vmcnt<OPS8>();
    else if (own4) wait_vmcnt<OPS4>();
    else wait_vmcnt<0>();
    M2R_STAMP(ST_TOKEN);
    __syncthreads();          // ... and every other wave's
    M2R_STAMP(ST_BARRIER);
    const uint32_t bw = st.b[lane], cw = st.c[lane];
    raw.bc[0] = (uint16_t)bw;
    raw.bc[1] = (uint16_t)(bw >> 16);
    raw.bc[2] = (uint16_t)cw;
    raw.bc[3] = (uint16_t)(cw >> 16);
    const uint8_t* p8 = (const uint8_t*)st.stat;
    perm0 = p8[packed_lane<N8, N4>(lane)];
    perm1 = p8[packed_lane<N8, N4>(64 + lane)];
    if constexpr (RIDGE) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int d0 = (RZ == 128) ? 2 * lane + j : lane;
        basis_w[j] = st.stat[32 + min(d0, NZ - 1)];   // unused past NZ
      }
    }
  } else {
    // ---- prologue: the wave's share of the predictor's LDS transfer, then the
    // register loads of the first token and the statics (one wait covers both),
    // then the LDS transfer of the wave's first slot, which lands while the
    // token is built; each later slot is fetched while the previous computes --
    // (order: the dt inputs, the predictor transfer, then the rest; the dt
    // activation's wait for its inputs thus covers only the first two)
    wave_load_dt<WPB, HPW, WPS>(a, raw, b * L, h0, lane, wave);
    const int hl = h0 + head_slot(min(lane, HPW - 1));   // head of slot `lane` (lanes < HPW)
    Ah = a.A[hl];
    if constexpr (RIDGE && !REC) {   // (a record-fed loop never reads the predictor)
      const uint8_t* pg = (const uint8_t*)(a.pred + (size_t)g * F * NZ);
      if constexpr (DMA) {   // 16-byte chunks; lanes past the end re-read the last one
        for (int j = wave; j < PRED_OPS16; j += WPB)
          lds_dma_b128<NT_LOAD>(pg + 16 * min(j * 64 + lane, PRED_DW / 4 - 1), lds_address(s_pred32 + 256 * j));
      } else {
        for (int j = wave; j < PRED_OPS; j += WPB)
          lds_dma_b32(pg + 4 * min(j * 64 + lane, PRED_DW - 1), lds_address(s_pred32 + 64 * j));
      }
    }
    uint4 rec0 = make_uint4(0u, 0u, 0u, 0u);   // REC: record 0, put in LDS once the loads have landed
    if constexpr (REC) {
      if (wave == REC_LOADER) {
        rec0 = rec_load(0);
        if (L > 1) rnext = rec_load(1);
      }
    }
    wave_load_rest<WPB, HPW, DMA, WPS>(a, raw, b * L, g, h0, pbase, lane, wave);
    // statics, kept as loaded bits until the first token's full wait (a
    // conversion here would make the compiler wait for them before the dt
    // activation)
    d_bits = a.d_f32 ? ((const uint32_t*)a.D)[hl] : (uint32_t)((const uint16_t*)a.D)[hl];
    perm0 = a.perm[g * 128 + packed_lane<N8, N4>(lane)];
    perm1 = a.perm[g * 128 + packed_lane<N8, N4>(64 + lane)];
    if constexpr (RIDGE) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int d0 = (RZ == 128) ? 2 * lane + j : lane;
        basis_w[j] = ((const uint32_t*)a.basis)[g * NZ + min(d0, NZ - 1)];   // unused past NZ
      }
      ls_w = DMA ? *(const uint32_t*)(a.lscale + g * 2)
                 : (uint32_t)a.lscale[g * 2] | ((uint32_t)a.lscale[g * 2 + 1] << 16);
    }
    // dt activation of the first token (multi-token: of the first 64) while
    // the other loads are in flight
    if constexpr (ONE) {
      act = wave_dt_activation<HPW, false, KM_PLAIN>(raw, Ah, a.db_f32);
    } else {
      batch_activation(0);
      act = token_act(0);
    }
    // the predictor transfer and the register loads complete before any slot
    // transfer is issued (the compiler's own waits for the register loads then
    // never cover a slot transfer; no load may be scheduled past this wait)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (dma_tiles) slot_dma(head_slot(0));
    else {
      for (int k = 0; k < HPW; ++k) slot_copy_in(head_slot(k));
    }
    if constexpr (REC) {   // record 0, published by the first token's barrier
      if (wave == REC_LOADER) ((uint4*)sm.rec[0])[lane] = rec0;
    }
  }
  if (lane < HPW) wt.D[lane] = a.d_f32 ? __builtin_bit_cast(float, d_bits) : h2f((uint16_t)d_bits);
  const int pv0 = perm0 & 127, pv1 = perm1 & 127;   // raw B/C index of internal positions lane, lane + 64
  float e0v[2] = {0.f, 0.f}, e1v[2] = {0.f, 0.f};   // dead-tier basis at the pair-tree positions
  float ls0 = 0.f, ls1 = 0.f, rls0 = 0.f, rls1 = 0.f;
  if constexpr (RIDGE) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      e0v[j] = h2f((uint16_t)(basis_w[j] & 0xFFFFu));
      e1v[j] = h2f((uint16_t)(basis_w[j] >> 16));
    }
    ls0 = h2f((uint16_t)(ls_w & 0xFFFFu));
    ls1 = h2f((uint16_t)(ls_w >> 16));
    // correctly rounded reciprocals: the latent scales are positive finite
    // binary16 values (the statics contract every caller validates)
    rls0 = recip_half(ls0);
    rls1 = recip_half(ls1);
  }

  // WPS > 1: the wave's copies of its slot's INT8 and INT4 scales
  float sc8_carry = 0.f, sc4_carry = 0.f;
  // a wave steps coordinates of a field another wave moves (not so only for
  // two waves split at the tier boundary)
  constexpr bool CROSS = PAIR && !(WPS == 2 && pair_cut(N8, N4) == N8);
  int rbuf = 0;   // REC: the buffer of token t's record (t mod 3)
  // KEEP (several waves per slot, several tokens): a wave's code words stay
  // in registers from token to token, read from the tile at the first token
  // and written back at the last (no nibble-plane unpacking and repacking
  // per token); so do the latent bytes where only the last wave reads them
  constexpr bool KEEP = PAIR && !ONE;
  uint32_t keep8[max_role_words(N8, N4, PAIR ? WPS : 1, false)];
  uint32_t keep4[max_role_words(N8, N4, PAIR ? WPS : 1, true)];
  uint32_t keep_lat = 0u;
  for (int t = 0; t < L; ++t) {
    const int bt = b * L + t;
    const WaveRaw<HPW> cur = raw;
    if (PAIR && t == ST_TL_TOKEN) M2R_STAMP(ST_TL);
    if (t + 1 < L) {   // prefetch
      if constexpr (REC) {
        wave_load_x<WPB, HPW, WPS>(a, raw, bt + 1, h0, pbase, lane, wave);
      } else {
        wave_load_dt<WPB, HPW, WPS>(a, raw, bt + 1, h0, lane, wave);
        wave_load_rest<WPB, HPW, DMA, WPS>(a, raw, bt + 1, g, h0, pbase, lane, wave);
      }
    }
    // readout weights and dead-tier dot products of this token
    const float* cwt;
    float dot1, dot2, dot3, dot4;
    auto build_token = [&]() {
      GroupToken<NL>& gt = s_gt[SPLIT && !ONE ? (t & 1) : 0];
      wave_token_build<N8, N4, NZ, MODE, WPB, HPW, Smem::STAGED>(wt, gt, cur, act, pv0, pv1, e0v, e1v, s_pred,
                                                                t == 0, lane, wave);
      cwt = SPLIT ? gt.cw : wt.cw;
      dot1 = SPLIT ? gt.tree[0] + gt.cw[NL] : wt.dots[1];
      dot2 = SPLIT ? gt.tree[1] + gt.cw[NL + 1] : wt.dots[2];
      dot3 = SPLIT ? gt.tree[2] : wt.dots[3];
      dot4 = SPLIT ? gt.tree[3] : wt.dots[4];
    };
    // REC: record t sits in buffer rbuf (put there before token t - 1's
    // maxima barrier, or before the first token)
    const float* rv = sm.rec[REC ? rbuf : 0];
    if constexpr (REC) {
      if (t + 2 < L && wave == REC_LOADER) rnext2 = rec_load(t + 2);
      if (t == 0) __syncthreads();   // record 0 is in LDS
      cwt = rv + REC_CW;
      dot1 = rv[REC_TREE] + rv[REC_CW + NL];
      dot2 = rv[REC_TREE + 1] + rv[REC_CW + NL + 1];
      dot3 = rv[REC_TREE + 2];
      dot4 = rv[REC_TREE + 3];
    } else {
      build_token();
    }
    if (t == 0) M2R_STAMP(ST_BUILD);
    if (PAIR && t == ST_TL_TOKEN) M2R_STAMP(ST_TL + 1);

    for (int k = 0; k < HPW; ++k) {
      // The slot's head index, opaque to the optimizer: every address and
      // buffer descriptor derived from it is then built here, where scalar
      // work overlaps the other waves' vector work, instead of being hoisted
      // out of the token loop for all slots at once (more scalar registers
      // than exist: spills, and a long serial setup before the first token).
      int hh = head_slot(k);
      asm volatile("" : "+s"(hh));
      const int h = h0 + hh;
      wave_priority_by_slots_left(HPW - k);
      if (t == 0) {
        slot_wait(k);
        // a slot on several waves where a wave steps fields another one
        // moved: those transfers are visible to it after the barrier
        if constexpr (CROSS) __syncthreads();
        if (k < 4) M2R_STAMP(ST_SLOT + 4 * k);
      }
      uint8_t* tile = s_tile[hh];
      uint16_t* t16 = (uint16_t*)tile;

      if constexpr (PAIR) {
        // ---- one slot on WPS waves: wave r updates the coordinates of its
        // readout segments (dequantization, readout, update, maximum) and
        // publishes through LDS what the others need (waves 0 .. WPS - 2
        // their readout partial sum, every wave its INT8 and INT4 parts'
        // maxima); after the workgroup barrier each requantizes its
        // coordinates with the whole tiers' maxima (the same values on every
        // wave, so the same scales and codes as one wave gets) and the last
        // wave steps the latent coefficients and reads the row out. ---------
        // (REC: from registers and the record: x of the wave's rows, dt and
        // the decay, the bound flag with the record's flag for b, B * dt
        // formed in tier_update from the record's b, and sum b.c)
        const float x = REC ? h2f(cur.xv[0]) : h2f(wt.x[0][lane]);
        const float decay = REC ? act.y : wt.decay[0];
        const float dtv = REC ? act.x : wt.dtv[0];
        const bool bounded = REC ? (rv[REC_BOK] != 0.f && 65504.f * __builtin_fabsf(act.x) < 0x1p100f &&
                                    __builtin_fabsf(act.y) < 0x1p100f)
                                 : wt.bounded[0] != 0;
        const bool base_ok = bounded && __builtin_fabsf(x) <= 65504.f;
        const f32x4* bdt4 = (const f32x4*)(REC ? rv + REC_B : wt.bdt[0]);
        const f32x4* cw4 = (const f32x4*)cwt;
        const float sbc = REC ? rv[REC_SBC] : wt.dots[0];
        auto& pacc = sm.pacc[t & 1][hh];
        auto& pmax = sm.pmax[t & 1][hh];
        auto role_body = [&](auto role_c) {
          constexpr int R = decltype(role_c)::value;
          constexpr int G0 = role_seg(N8, N4, WPS, R), G1 = role_seg(N8, N4, WPS, R + 1);   // its segments
          constexpr int PLO = seg_pos(N8, N4, G0), PHI = seg_pos(N8, N4, G1);
          constexpr int A8 = PLO < N8 ? PLO : N8, E8 = PHI < N8 ? PHI : N8;
          constexpr int A4 = PLO > N8 ? PLO - N8 : 0, E4 = PHI > N8 ? PHI - N8 : 0;
          constexpr int M8 = E8 - A8, M4 = E4 - A4;   // this wave's INT8 and INT4 coordinates
          constexpr bool LAST = R == WPS - 1;
          // the wave that reads the rows out: four waves per slot, wave 0 (the
          // last one also steps the latent coefficients and stores their and
          // the INT4 scales); two, the last
          constexpr int RO = WPS == 4 ? 0 : WPS - 1;
          constexpr bool READS_OUT = R == RO;
          constexpr unsigned HAS8 = tier_waves<N8, N4, WPS, false>(), HAS4 = tier_waves<N8, N4, WPS, true>();
          // a tier's maximum is published only when another wave steps part of it
          constexpr bool SHARE8 = (HAS8 & (HAS8 - 1)) != 0, SHARE4 = (HAS4 & (HAS4 - 1)) != 0;
          // per segment: the tiers' readout chains, then the segment's readout
          float c8s[4] = {0.f, 0.f, 0.f, 0.f}, c4s[4] = {0.f, 0.f, 0.f, 0.f}, accs[4];
          uint32_t c8[M8 > 0 ? (M8 + 3) / 4 : 1], c4[M4 > 0 ? (M4 + 3) / 4 : 1];
          float v8[M8 > 0 ? M8 : 1], v4[M4 > 0 ? M4 : 1];
          float amax8 = 0.f, amax4 = 0.f, s8 = 0.f, s4 = 0.f, z0 = 0.f, z1 = 0.f;
          bool fin8 = true, fin4 = true;
          // a tier's scale: the tile's at the first token, then the value this
          // wave requantized with (every wave of the tier derives the same one)
          // (KEEP: the latent bytes stay in a register where only this last
          // wave reads them, i.e. unless a reading wave reads the tile's)
          constexpr bool KEEP_LAT = KEEP && (REC || RO == WPS - 1);
          if constexpr (M8 > 0) {
            if (KEEP && t > 0) {
#pragma unroll
              for (int i = 0; i < (M8 + 3) / 4; ++i) c8[i] = keep8[i];
            } else {
              uint32_t wl[(M8 / 2 + 3) / 4], wh[(M8 / 2 + 3) / 4];
              lds_read_row<M8 / 2>(tile + O_LO, lane * W8 + A8 / 2, wl);
              lds_read_row<M8 / 2>(tile + O_HI, lane * W8 + A8 / 2, wh);
              planes_to_bytes8<M8>(wl, wh, c8);
            }
            s8 = t == 0 ? h2f(t16[O_S8 / 2 + lane]) : sc8_carry;
            if (PLACEHOLDERS && !valid) {   // rows past P: finite placeholders, never stored
#pragma unroll
              for (int i = 0; i < (M8 + 3) / 4; ++i) c8[i] = 0x80808080u;
              s8 = 0.f;
            }
            fin8 = __builtin_fabsf(s8) <= 65504.f;
            if (__builtin_amdgcn_ballot_w64(!fin8) == 0)
              amax8 = tier_update<M8, true, false, N8, N4, A8, REC>(c8, s8, decay, x, bdt4, cw4, c8s, v8, dtv);
            else
              amax8 = tier_update<M8, true, true, N8, N4, A8, REC>(c8, s8, decay, x, bdt4, cw4, c8s, v8, dtv);
            if constexpr (SHARE8) pmax[0][R][lane] = amax8;
          }
          // the latent coefficients, read with the rows (REC: by the last
          // wave only, which passes them to the reading wave through pz: the
          // tile's latent bytes of token t are rewritten after the barrier
          // without another barrier before token t + 1)
          constexpr bool PASS_Z = REC && READS_OUT != LAST;
          if constexpr ((LAST || (READS_OUT && !PASS_Z)) && RIDGE) {
            const uint32_t lat = (KEEP_LAT && LAST && t > 0) ? keep_lat : (uint32_t)t16[O_LAT / 2 + lane];
            z0 = e4m3_byte_to_f32<0>(lat) * ls0;
            z1 = e4m3_byte_to_f32<1>(lat) * ls1;
            if (PLACEHOLDERS && !valid) z0 = z1 = 0.f;
            if constexpr (PASS_Z && LAST) sm.pz[t & 1][hh][lane] = make_float2(z0, z1);
          }
          if constexpr (M4 > 0) {
            if (KEEP && t > 0) {
#pragma unroll
              for (int i = 0; i < (M4 + 3) / 4; ++i) c4[i] = keep4[i];
            } else {
              uint32_t wq[(M4 / 2 + 3) / 4];
              lds_read_row<M4 / 2>(tile + O_Q4, lane * W4 + A4 / 2, wq);
              plane_to_bytes4<M4>(wq, c4);
            }
            s4 = t == 0 ? h2f(t16[O_S4 / 2 + lane]) : sc4_carry;
            if (PLACEHOLDERS && !valid) {
#pragma unroll
              for (int i = 0; i < (M4 + 3) / 4; ++i) c4[i] = 0x08080808u;
              s4 = 0.f;
            }
            fin4 = __builtin_fabsf(s4) <= 65504.f;
            if (__builtin_amdgcn_ballot_w64(!fin4) == 0)
              amax4 = tier_update<M4, false, false, N8, N4, N8 + A4, REC>(c4, s4, decay, x, bdt4, cw4, c4s, v4, dtv);
            else
              amax4 = tier_update<M4, false, true, N8, N4, N8 + A4, REC>(c4, s4, decay, x, bdt4, cw4, c4s, v4, dtv);
            if constexpr (SHARE4) pmax[1][R][lane] = amax4;
          }
          uint32_t qz = 0;
          if constexpr (LAST && RIDGE) {   // latent step (bit-exact), as in the one-wave slot below
            const float xdt = x * dtv;
            const float zn0 = state_update(z0, decay, xdt * dot3);
            const float zn1 = state_update(z1, decay, xdt * dot4);
            const float q0 = __builtin_fminf(__builtin_fmaxf(latent_quotient(zn0, ls0, rls0), -448.f), 448.f);
            const float q1 = __builtin_fminf(__builtin_fmaxf(latent_quotient(zn1, ls1, rls1), -448.f), 448.f);
            qz = f32x2_to_e4m3(q0, q1);
          }
          // the left fold of the readout segments: the other waves publish
          // the fold of their segments, the reading wave folds them in order
#pragma unroll
          for (int sg = G0; sg < G1; ++sg) accs[sg] = segment_readout<N8, N4>(sg, c8s[sg], c4s[sg]);
          float part = accs[G0];
#pragma unroll
          for (int sg = G0 + 1; sg < G1; ++sg) part = part + accs[sg];
          if constexpr (!READS_OUT) pacc[R][lane] = part;
          if constexpr (REC) {   // record t + 1 into the buffer token t - 2 used (every wave is past it)
            if (wave == REC_LOADER && t + 1 < L) ((uint4*)sm.rec[rbuf == 2 ? 0 : rbuf + 1])[lane] = rnext;
          }
          if (t == 0) M2R_STAMP(ST_SLOT + 1);
          if (t == ST_TL_TOKEN) M2R_STAMP(ST_TL + 2);
          __syncthreads();   // readout partials and tier maxima are published
          if (t == 0) M2R_STAMP(ST_SLOT + 2);
          if (t == ST_TL_TOKEN) M2R_STAMP(ST_TL + 3);
          if constexpr (READS_OUT) {
            if constexpr (PASS_Z && RIDGE) {
              const float2 zz = sm.pz[t & 1][hh][lane];
              z0 = zz.x;
              z1 = zz.y;
            }
            float acc = RO == 0 ? part : pacc[0][lane];
#pragma unroll
            for (int r = 1; r < WPS; ++r) {
              if (r < RO) acc = acc + pacc[r][lane];
              else if (r > RO) acc = acc + pacc[r][lane];
            }
            if constexpr (RO > 0) {   // the reading wave's own segments after the others' before it
#pragma unroll
              for (int sg = G0; sg < G1; ++sg) acc = acc + accs[sg];
            }
            float out;
            if constexpr (RIDGE) out = decay * (acc + z0 * dot1 + z1 * dot2) + x * (dtv * sbc + wt.D[0]);
            else out = decay * acc + x * (dtv * sbc + wt.D[0]);
            const __amdgpu_buffer_rsrc_t ry = raw_buffer(a.y + ((size_t)bt * H + h) * P + pbase, 2 * nvalid);
            __builtin_amdgcn_raw_buffer_store_b16(f2h(out), ry, 2 * lane, 0, STORE_CP);
          }
          // the whole tiers' maxima (maxima are exact: any order)
          auto tier_max = [&](int tier, float own, unsigned has) {
            float m = own;
#pragma unroll
            for (int r = 0; r < WPS; ++r)
              if (r != R && ((has >> r) & 1u)) m = max3_abs(m, pmax[tier][r][lane], 0.f);
            return m;
          };
          if constexpr (M8 > 0) {
            const float m8 = tier_max(0, amax8, HAS8);
            sc8_carry = tier_requant<M8, true, MODE>(v8, c8, m8, base_ok && fin8);
            if constexpr (KEEP) {
#pragma unroll
              for (int i = 0; i < (M8 + 3) / 4; ++i) keep8[i] = c8[i];
            }
            if (valid && (!KEEP || t == L - 1)) {
              uint32_t wl[(M8 / 2 + 3) / 4], wh[(M8 / 2 + 3) / 4];
              bytes_to_planes8<M8>(c8, wl, wh);
              lds_write_row<M8 / 2>(tile + O_LO, lane * W8 + A8 / 2, wl);
              lds_write_row<M8 / 2>(tile + O_HI, lane * W8 + A8 / 2, wh);
              if constexpr (R == 0) t16[O_S8 / 2 + lane] = f2h(sc8_carry);
            }
          }
          if constexpr (M4 > 0) {
            const float m4 = tier_max(1, amax4, HAS4);
            sc4_carry = tier_requant<M4, false, MODE>(v4, c4, m4, base_ok && fin4);
            if constexpr (KEEP) {
#pragma unroll
              for (int i = 0; i < (M4 + 3) / 4; ++i) keep4[i] = c4[i];
            }
            if (valid && (!KEEP || t == L - 1)) {
              uint32_t wq[(M4 / 2 + 3) / 4];
              bytes_to_plane4<M4>(c4, wq);
              lds_write_row<M4 / 2>(tile + O_Q4, lane * W4 + A4 / 2, wq);
              if constexpr (LAST) t16[O_S4 / 2 + lane] = f2h(sc4_carry);
            }
          }
          if constexpr (LAST && RIDGE) {
            if constexpr (KEEP_LAT) keep_lat = qz;
            if (valid && (!KEEP_LAT || t == L - 1)) t16[O_LAT / 2 + lane] = (uint16_t)qz;
          }
        };
        if constexpr (WPS == 2) {
          if (role == 0) role_body(std::integral_constant<int, 0>{});
          else role_body(std::integral_constant<int, 1>{});
        } else {
          if (role == 0) role_body(std::integral_constant<int, 0>{});
          else if (role == 1) role_body(std::integral_constant<int, 1>{});
          else if (role == 2) role_body(std::integral_constant<int, 2>{});
          else role_body(std::integral_constant<int, 3>{});
        }
      } else {
        const float x = h2f(wt.x[k][lane]);
        const float decay = wt.decay[k];
        const float dtv = wt.dtv[k];
        const bool base_ok = wt.bounded[k] != 0 && __builtin_fabsf(x) <= 65504.f;
        const f32x4* bdt4 = (const f32x4*)wt.bdt[k];
        const f32x4* cw4 = (const f32x4*)cwt;
        // the readout per readout segment: each tier's contribution, then the
        // segment's sum, folded after both tiers (the order of the multi-wave
        // slots, whose segments run on different waves)
        float c8s[4] = {0.f, 0.f, 0.f, 0.f}, c4s[4] = {0.f, 0.f, 0.f, 0.f};

        // ---- INT8 tier: unpack (byte k of c8[i] is q8 + 128 of internal
        // coordinate 4i+k), update with readout accumulation, requantize and
        // repack into the tile; each tier is done before the next is read, so
        // only one tier's values are live at a time.  Per tier, a wave-uniform
        // choice between two copies of the tier code: the fused
        // dequantization when every scale of the wave is finite, the exact
        // products otherwise (non-finite scales are rare: the reference's
        // controllers reject such states).
        {
          uint32_t c8[C8];
          {
            uint32_t wl[(W8 + 3) / 4], wh[(W8 + 3) / 4];
            lds_read_row<W8>(tile + O_LO, lane * W8, wl);
            lds_read_row<W8>(tile + O_HI, lane * W8, wh);
            planes_to_bytes8<N8>(wl, wh, c8);
          }
          float sc8 = h2f(t16[O_S8 / 2 + lane]);
          if (PLACEHOLDERS && !valid) {   // rows past P: finite placeholders, never stored
#pragma unroll
            for (int i = 0; i < C8; ++i) c8[i] = 0x80808080u;
            sc8 = 0.f;
          }
          const bool fin8 = __builtin_fabsf(sc8) <= 65504.f;
          {
            float v8[N8];
            if (__builtin_amdgcn_ballot_w64(!fin8) == 0) {
              const float m8 = tier_update<N8, true, false, N8, N4, 0>(c8, sc8, decay, x, bdt4, cw4, c8s, v8);
              sc8 = tier_requant<N8, true, MODE>(v8, c8, m8, base_ok);
            } else {
              const float m8 = tier_update<N8, true, true, N8, N4, 0>(c8, sc8, decay, x, bdt4, cw4, c8s, v8);
              sc8 = tier_requant<N8, true, MODE>(v8, c8, m8, base_ok && fin8);
            }
          }
          if (valid) {
            uint32_t wl[(W8 + 3) / 4], wh[(W8 + 3) / 4];
            bytes_to_planes8<N8>(c8, wl, wh);
            lds_write_row<W8>(tile + O_LO, lane * W8, wl);
            lds_write_row<W8>(tile + O_HI, lane * W8, wh);
            t16[O_S8 / 2 + lane] = f2h(sc8);
          }
        }
        if (t == 0 && k < 4) M2R_STAMP(ST_SLOT + 4 * k + 1);
        __builtin_amdgcn_sched_barrier(0);
        // the next slot's transfers are issued between the tiers, where the
        // other waves' arithmetic covers their issue time
        if (dma_tiles && t == 0 && k + 1 < HPW) slot_dma(hh + 1);   // head_slot(k + 1)
        // first slot, first token: its INT4 fields (transferred after the
        // INT8 ones) are waited for only now; later only the next slot's
        // transfers may be outstanding
        if (dma_tiles && t == 0 && k == 0) {
          if (HPW > 1) wait_vmcnt<SLOT_DMA>();
          else wait_vmcnt<0>();
        }

        // ---- INT4 tier and the latent coefficients ------------------------------
        uint32_t c4[C4];
        {
          uint32_t wq[(W4 + 3) / 4];
          lds_read_row<W4>(tile + O_Q4, lane * W4, wq);
          plane_to_bytes4<N4>(wq, c4);
        }
        float sc4 = h2f(t16[O_S4 / 2 + lane]);
        float z0 = 0.f, z1 = 0.f;
        if constexpr (RIDGE) {
          const uint32_t lat = t16[O_LAT / 2 + lane];
          z0 = e4m3_byte_to_f32<0>(lat) * ls0;
          z1 = e4m3_byte_to_f32<1>(lat) * ls1;
        }
        if (PLACEHOLDERS && !valid) {
#pragma unroll
          for (int i = 0; i < C4; ++i) c4[i] = 0x08080808u;
          sc4 = z0 = z1 = 0.f;
        }
        const bool fin4 = __builtin_fabsf(sc4) <= 65504.f;
        {
          float v4[N4];
          if (__builtin_amdgcn_ballot_w64(!fin4) == 0) {
            const float m4 = tier_update<N4, false, false, N8, N4, N8>(c4, sc4, decay, x, bdt4, cw4, c4s, v4);
            sc4 = tier_requant<N4, false, MODE>(v4, c4, m4, base_ok);
          } else {
            const float m4 = tier_update<N4, false, true, N8, N4, N8>(c4, sc4, decay, x, bdt4, cw4, c4s, v4);
            sc4 = tier_requant<N4, false, MODE>(v4, c4, m4, base_ok && fin4);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (t == 0 && k < 4) M2R_STAMP(ST_SLOT + 4 * k + 2);
        if (t == L - 1 && k > 0) slot_copy_out(hh - 1);   // the previous slot's state (head_slot(k - 1))
        __builtin_amdgcn_sched_barrier(0);
        float accs[4];
#pragma unroll
        for (int sg = 0; sg < 4; ++sg) accs[sg] = segment_readout<N8, N4>(sg, c8s[sg], c4s[sg]);
        const float acc = ((accs[0] + accs[1]) + accs[2]) + accs[3];   // the readout segments' left fold
        // readout: sum_i u_i c_i + corrections = decay * (sum_i prior_i (c_i +
        // corr_i) + latent terms) + x * (dt * sum_all b c + D)
        float out;
        uint32_t qz = 0;
        if constexpr (RIDGE) {
          out = decay * (acc + z0 * dot1 + z1 * dot2) + x * (dtv * wt.dots[0] + wt.D[k]);
          // latent step (bit-exact): z <- fma(z, decay, (x * dt) * (e . b_dead)), requantized
          const float xdt = x * dtv;
          const float zn0 = state_update(z0, decay, xdt * dot3);
          const float zn1 = state_update(z1, decay, xdt * dot4);
          const float q0 = __builtin_fminf(__builtin_fmaxf(latent_quotient(zn0, ls0, rls0), -448.f), 448.f);
          const float q1 = __builtin_fminf(__builtin_fmaxf(latent_quotient(zn1, ls1, rls1), -448.f), 448.f);
          qz = f32x2_to_e4m3(q0, q1);   // q0, q1 are clamped, never NaN (maxNum drops a NaN)
        } else {
          out = decay * acc + x * (dtv * wt.dots[0] + wt.D[k]);
        }
        {   // one unguarded store instruction: the range check drops rows past P
          const __amdgpu_buffer_rsrc_t ry = raw_buffer(a.y + ((size_t)bt * H + h) * P + pbase, 2 * nvalid);
          __builtin_amdgcn_raw_buffer_store_b16(f2h(out), ry, 2 * lane, 0, STORE_CP);
        }

        // ---- repack the INT4 tier and the latent bytes into the tile ------------------
        if (valid) {
          uint32_t wq[(W4 + 3) / 4];
          bytes_to_plane4<N4>(c4, wq);
          lds_write_row<W4>(tile + O_Q4, lane * W4, wq);
          t16[O_S4 / 2 + lane] = f2h(sc4);
          if constexpr (RIDGE) t16[O_LAT / 2 + lane] = (uint16_t)qz;
        }
      }
      wave_sync();
      if (t == 0 && k < 4) M2R_STAMP(ST_SLOT + 4 * k + 3);
      if (PAIR && t == ST_TL_TOKEN) M2R_STAMP(ST_TL + 4);
    }
    if constexpr (REC) {
      rbuf = rbuf == 2 ? 0 : rbuf + 1;
      if (wave == REC_LOADER) rnext = rnext2;
    }
    if (PAIR && t == ST_TL_TOKEN) M2R_STAMP(ST_TL + 5);
    if (t == L - 1) {
      // ... and the moving wave writes back every wave's last values
      if constexpr (CROSS) __syncthreads();
      slot_copy_out(head_slot(HPW - 1));
      M2R_STAMP(ST_COPYOUT);
    }
    if (t + 1 < L) {
      if (((t + 1) & 63) == 0) batch_activation(t + 1);
      act = token_act(t + 1);
    }
  }
#ifdef M2R_PHASE_TIMELINE
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): every store of the wave has completed
  M2R_STAMP(ST_END);
  M2R_STAMP_REAL(ST_REAL1);
  wave_sync();
  if (g_phase_stamps && lane < 32) {
    const size_t blk = ((size_t)b * gridDim.y + by) * gridDim.x + bx;
    g_phase_stamps[(blk * WPB + wave) * 32 + lane] = sm.stamps[wave][lane];
  }
#endif
}

template <int N8, int N4, int NZ, int MODE, int WPB, int HPW, bool DMA, bool ONE, int WPS = 1, bool REC = false>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(WPB == 8 && WPS == 1 ? 4 : 2, 8)))
void k_state_step(StepArgs a) {
  __shared__ StepSmem<N8, N4, NZ, MODE, WPB, HPW, DMA, ONE, WPS, REC> sm;
  state_step_body<N8, N4, NZ, MODE, WPB, HPW, DMA, ONE, WPS, REC>(a, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}

// ---------------------------------------------------------------------------
// Token records of a multi-token ridge launch (the record-fed token loop of
// k_state_step): one four-wave workgroup per (REC_TOKENS tokens, group,
// batch row) runs the split token build of every token (wave_token_build with
// four waves: the same gathers, sums, ridge correction and dead-tier trees,
// so the same bits) and wave 0 stores the state-independent values as the
// token's record at rec[((b L + t) G + g) REC_FLOATS].  Each token's inputs
// are loaded while the previous token is built.  Needs 16-byte
// aligned predictor and 4-byte aligned B and C (StepArgs::dma_tiles bit 0).
constexpr int REC_TOKENS = 8;

template <int N8, int N4, int NZ>
struct RecordSmem {
  static constexpr int NL = N8 + N4, F = NL + 2;
  static constexpr int PRED_DW = F * NZ / 2, PRED_WORDS = (PRED_DW + 255) / 256 * 256;
  alignas(16) WaveToken<N8, N4, 1> wt[4];
  alignas(16) GroupToken<NL> gt[2];   // by token parity: wave 0 reads token t's while the others build t + 1
  alignas(16) uint32_t pred32[PRED_WORDS];
};

template <int N8, int N4, int NZ>
__global__ __launch_bounds__(256) void k_token_records(StepArgs a, float* rec) {
  constexpr int NL = N8 + N4, F = NL + 2, RZ = next_pow2(NZ);
  using Smem = RecordSmem<N8, N4, NZ>;
  constexpr int PRED_OPS16 = (Smem::PRED_DW + 255) / 256;
  static_assert(NL <= 84, "record layout");
  __shared__ Smem sm;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.y, b = blockIdx.z;
  const int L = a.L, t0 = blockIdx.x * REC_TOKENS, t1 = min(t0 + REC_TOKENS, L);
  const int h0 = g * (a.H / a.G);   // a head of the group (the build also copies x of its rows: unused)
  // the group's predictor (16-byte chunks; lanes past the end re-read the
  // last one), permutation and dead-tier basis, as the step kernel loads them
  const uint8_t* pg = (const uint8_t*)(a.pred + (size_t)g * F * NZ);
  for (int j = wave; j < PRED_OPS16; j += 4)
    lds_dma_b128(pg + 16 * min(j * 64 + lane, Smem::PRED_DW / 4 - 1), lds_address(sm.pred32 + 256 * j));
  const uint32_t perm0 = a.perm[g * 128 + packed_lane<N8, N4>(lane)];
  const uint32_t perm1 = a.perm[g * 128 + packed_lane<N8, N4>(64 + lane)];
  float e0v[2], e1v[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int d0 = (RZ == 128) ? 2 * lane + j : lane;
    const uint32_t w = ((const uint32_t*)a.basis)[g * NZ + min(d0, NZ - 1)];   // unused past NZ
    e0v[j] = h2f((uint16_t)(w & 0xFFFFu));
    e1v[j] = h2f((uint16_t)(w >> 16));
  }
  WaveRaw<1> raw;   // the first token's inputs, in flight with the predictor
  wave_load_rest<4, 1, true, 4>(a, raw, b * L + t0, g, h0, 0, lane, wave);
  __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0): the predictor transfer has landed
  __syncthreads();                      // ... every wave's share
  const int pv0 = perm0 & 127, pv1 = perm1 & 127;
  const uint16_t* s_pred = (const uint16_t*)sm.pred32;
  for (int t = t0; t < t1; ++t) {
    const WaveRaw<1> r = raw;
    if (t + 1 < t1) wave_load_rest<4, 1, true, 4>(a, raw, b * L + t + 1, g, h0, 0, lane, wave);
    GroupToken<NL>& gt = sm.gt[t & 1];
    // dt 0, decay 0: the bound flag is then that of b alone
    wave_token_build<N8, N4, NZ, MODE_RIDGE, 4, 1, false>(sm.wt[wave], gt, r, make_float2(0.f, 0.f), pv0, pv1, e0v,
                                                         e1v, s_pred, false, lane, wave);
    // (the split build ends with a workgroup barrier: gt is complete)
    if (wave == 0) {
      const WaveToken<N8, N4, 1>& wt = sm.wt[0];
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = 4 * lane + i;
        const float cw = gt.cw[min(idx, NL + 1)];
        const float tr = gt.tree[min(max(idx - REC_TREE, 0), 3)];
        const float bv = wt.b[min(max(idx - REC_B, 0), NL - 1)];
        float x = 0.f;
        if (idx < NL + 2) x = cw;
        else if (idx >= REC_TREE && idx < REC_TREE + 4) x = tr;
        else if (idx == REC_SBC) x = wt.dots[0];
        else if (idx == REC_BOK) x = wt.bounded[0] ? 1.f : 0.f;
        else if (idx >= REC_B && idx < REC_B + NL) x = bv;
        v[i] = x;
      }
      float4* dst = (float4*)(rec + ((size_t)(b * L + t) * a.G + g) * REC_FLOATS);
      dst[lane] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
}

}  // namespace m2r
