// Host dispatch and C ABI of the fused state step (kernel in m2r_step.h).
#include "m2r_step.h"
#include "m2r_abi_util.h"

#include <atomic>
#include <type_traits>
#include <initializer_list>

namespace m2r {

// ---------------------------------------------------------------------------
// Host dispatch over the supported tier layouts.  Heads per workgroup grow
// with the number of 64-row slots so that the per-token shared work is
// amortized while the grid still spans every CU; small grids keep four waves
// per workgroup, which splits the per-token shared work four ways.
// Workgroup shape forced through m2r_set_step_shape (0 = automatic), encoded
// as waves_per_block * 16 + heads_per_wave; (4, 0) = 2 waves per head slot and
// FOUR_PER_SLOT = 4 waves per head slot, one head per workgroup.
static std::atomic<int> g_forced_shape{0};
static constexpr int FOUR_PER_SLOT = 256 + 4 * 16;

// a.dma_tiles: bit 0 = 16-byte LDS transfers of the state rows; bit 1 = the
// one-token inputs may be staged by dword transfers (the staged prologue of
// the one-token instances of four or more waves).
// WPS > 1: WPS waves per head slot (each steps a quarter or half of the
// carried coordinates), 4 waves per workgroup: the small-batch shapes (one
// wave per SIMD, the slots' work on two or four times the SIMDs).
template <int N8, int N4, int NZ, int MODE, int WPB, int HPW, int WPS = 1>
static void launch_shape(const StepArgs& a, dim3 grid, hipStream_t stream) {
  constexpr bool staged = StepSmem<N8, N4, NZ, MODE, WPB, HPW, true, true, WPS>::STAGED;
  if constexpr (MODE == MODE_RIDGE && WPS > 1) {   // the record-fed instance (a.rec: records written)
    if (a.rec) {
      hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, WPB, HPW, true, false, WPS, true>), grid, dim3(64 * WPB), 0,
                         stream, a);
      return;
    }
  }
  if ((a.dma_tiles & 1) && a.L == 1 && (!staged || (a.dma_tiles & 2))) {
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, WPB, HPW, true, true, WPS>), grid, dim3(64 * WPB), 0, stream,
                       a);
  } else if (a.dma_tiles & 1) {
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, WPB, HPW, true, false, WPS>), grid, dim3(64 * WPB), 0, stream,
                       a);
  } else {
    hipLaunchKernelGGL((k_state_step<N8, N4, NZ, MODE, WPB, HPW, false, false, WPS>), grid, dim3(64 * WPB), 0,
                       stream, a);
  }
}

// args.rec on entry: a token-record workspace of at least B * L * G records
// (or null).  The shapes of several waves per slot take it for a
// multi-token ridge launch with 16-byte transfers: k_token_records fills it
// and the step's token loop reads the records instead of building each
// token (the same values); every other launch runs with rec = null.
template <int N8, int N4, int NZ, int MODE>
static hipError_t launch_layout(const StepArgs& args, hipStream_t stream) {
  StepArgs a = args;
  a.rhpg = 1.0f / (float)(a.H / a.G);
  const int pblocks = (a.P + 63) / 64;
  const int hpg = a.H / a.G;
  const long long slots = (long long)a.B * a.H * pblocks;
  const int forced = g_forced_shape.load(std::memory_order_relaxed);
  float* const ws = (float*)args.rec;
  a.rec = nullptr;
  // the token records of a shape of several waves per slot
  auto records = [&]() {
    if constexpr (MODE == MODE_RIDGE) {
      if (ws && a.L > 1 && (a.dma_tiles & 1)) {
        hipLaunchKernelGGL((k_token_records<N8, N4, NZ>), dim3((a.L + REC_TOKENS - 1) / REC_TOKENS, a.G, a.B),
                           dim3(256), 0, stream, a, ws);
        a.rec = ws;
      }
    }
  };
  if (forced == 4 * 16 && hpg % 2 == 0) {   // (4, 0): two waves per head slot
    records();
    launch_shape<N8, N4, NZ, MODE, 4, 1, 2>(a, dim3(pblocks, a.H / 2, a.B), stream);
    return hipGetLastError();
  }
  if (forced == FOUR_PER_SLOT) {   // (4, -4): four waves per head slot
    records();
    launch_shape<N8, N4, NZ, MODE, 4, 1, 4>(a, dim3(pblocks, a.H, a.B), stream);
    return hipGetLastError();
  }
  if (forced && (forced & 15) && hpg % ((forced >> 4) * (forced & 15)) == 0) {
    const int wpb = forced >> 4, hpw = forced & 15;
    dim3 grid(pblocks, a.H / (wpb * hpw), a.B);
    if (wpb == 1) launch_shape<N8, N4, NZ, MODE, 1, 1>(a, grid, stream);
    else if (hpw == 1) launch_shape<N8, N4, NZ, MODE, 4, 1>(a, grid, stream);
    else if (wpb == 8) launch_shape<N8, N4, NZ, MODE, 8, 2>(a, grid, stream);
    else if (hpw == 2) launch_shape<N8, N4, NZ, MODE, 4, 2>(a, grid, stream);
    else launch_shape<N8, N4, NZ, MODE, 4, 4>(a, grid, stream);
    return hipGetLastError();
  }
  if (hpg % 16 == 0 && slots >= 16LL * 512) {
    launch_shape<N8, N4, NZ, MODE, 4, 4>(a, dim3(pblocks, a.H / 16, a.B), stream);
  } else if (slots <= 512) {   // four waves per slot, up to two waves per SIMD
    records();
    launch_shape<N8, N4, NZ, MODE, 4, 1, 4>(a, dim3(pblocks, a.H, a.B), stream);
  } else if (hpg % 2 == 0 && slots <= 1024) {   // two waves per slot, up to two waves per SIMD
    records();
    launch_shape<N8, N4, NZ, MODE, 4, 1, 2>(a, dim3(pblocks, a.H / 2, a.B), stream);
  } else if (hpg % 8 == 0 && slots >= 8LL * 512) {
    launch_shape<N8, N4, NZ, MODE, 4, 2>(a, dim3(pblocks, a.H / 8, a.B), stream);
  } else if (hpg % 4 == 0) {
    launch_shape<N8, N4, NZ, MODE, 4, 1>(a, dim3(pblocks, a.H / 4, a.B), stream);
  } else {
    launch_shape<N8, N4, NZ, MODE, 1, 1>(a, dim3(pblocks, a.H, a.B), stream);
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

// 16-byte LDS transfers need every slot's field start and valid length to be
// multiples of 16 bytes: P % 8 == 0 (fields are 2 to 38 bytes wide, all even)
// and 16-byte aligned field arrays.
// The transfer-friendly instances need P % 8 == 0, 16-byte aligned state
// fields (and ridge predictor), and 4-byte aligned B, C (and latent scales).
static int dma_tiles_ok(int64_t P, std::initializer_list<const void*> align16,
                        std::initializer_list<const void*> align4) {
  if (P % 8) return 0;
  for (const void* f : align16)
    if (f && ((uintptr_t)f & 15)) return 0;
  for (const void* f : align4)
    if (f && ((uintptr_t)f & 3)) return 0;
  return 1;
}

// Staged one-token inputs (bit 1 of StepArgs::dma_tiles): an even number of
// heads (so that every workgroup's heads start on a dword) and dword-aligned
// per-head, row and static arrays.
static int staged_ok(int64_t H, std::initializer_list<const void*> align4) {
  if (H % 2) return 0;
  for (const void* f : align4)
    if (f && ((uintptr_t)f & 3)) return 0;
  return 2;
}

static int check_geometry(int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G) {
  if (batch <= 0 || L <= 0 || H <= 0 || P <= 0 || G <= 0) return m2r_fail("state step: non-positive geometry");
  if (H % G) return m2r_fail("state step: heads must be divisible by groups");
  if (batch > 65535 || H > 65535 * 4) return m2r_fail("state step: grid limits exceeded");
  if ((double)batch * L * H * P >= 2147483647.0) return m2r_fail("state step: B*L*H*P must fit int32");
  return 0;
}

extern "C" int64_t m2r_ridge_records_bytes(int64_t batch, int64_t L, int64_t G) {
  if (batch <= 0 || L <= 0 || G <= 0) return 0;
  return batch * L * G * (int64_t)(REC_FLOATS * sizeof(float));
}

extern "C" int m2r_state_step_ridge_ws(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                       const void* D, int d_is_f32, const void* dt_bias, int db_is_f32,
                                       const uint8_t* perm, const void* basis, const void* lscale, const void* pred,
                                       uint8_t* lo, uint8_t* hi, uint8_t* q4, uint8_t* latent, void* s8, void* s4,
                                       void* y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G, int n8,
                                       int n4, int nz, void* workspace, int64_t workspace_bytes,
                                       hipStream_t stream) {
  if (int e = check_geometry(batch, L, H, P, G)) return e;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return m2r_fail("ridge step: workspace size without a workspace");
  if (workspace && ((uintptr_t)workspace & 15)) return m2r_fail("ridge step: workspace must be 16-byte aligned");
  if (workspace && workspace_bytes < m2r_ridge_records_bytes(batch, L, G))
    return m2r_fail("ridge step: workspace smaller than m2r_ridge_records_bytes(batch, L, G)");
  Dispatch d{};
  d.args = StepArgs{(const uint16_t*)x, (const uint16_t*)dt, A, (const uint16_t*)B, (const uint16_t*)C, D, dt_bias,
                    perm, (const uint16_t*)basis, (const uint16_t*)lscale, (const uint16_t*)pred, lo, hi, q4, latent,
                    (uint16_t*)s8, (uint16_t*)s4, (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G,
                    d_is_f32, db_is_f32,
                    dma_tiles_ok(P, {lo, hi, q4, latent, s8, s4, pred}, {B, C, lscale}) |
                        staged_ok(H, {x, dt, A, D, dt_bias, perm, basis})};
  d.args.rec = (const float*)workspace;
  d.n8_ = n8; d.n4_ = n4; d.nz_ = nz;
  hipError_t e = dispatch_ridge(d, stream);
  if (e == hipErrorInvalidValue) return m2r_fail("ridge step: unsupported tier layout");
  return m2r_check(e, "ridge step launch");
}

extern "C" int m2r_state_step_ridge(const void* x, const void* dt, const float* A, const void* B, const void* C,
                                    const void* D, int d_is_f32, const void* dt_bias, int db_is_f32,
                                    const uint8_t* perm, const void* basis, const void* lscale, const void* pred,
                                    uint8_t* lo, uint8_t* hi, uint8_t* q4, uint8_t* latent, void* s8, void* s4,
                                    void* y, int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G, int n8,
                                    int n4, int nz, hipStream_t stream) {
  return m2r_state_step_ridge_ws(x, dt, A, B, C, D, d_is_f32, dt_bias, db_is_f32, perm, basis, lscale, pred, lo, hi,
                                 q4, latent, s8, s4, y, batch, L, H, P, G, n8, n4, nz, nullptr, 0, stream);
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
                    (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G, d_is_f32, db_is_f32,
                    dma_tiles_ok(P, {lo, hi, q4, s8, s4}, {B, C}) | staged_ok(H, {x, dt, A, D, dt_bias, perm})};
  d.n8_ = n8; d.n4_ = n4; d.nz_ = nz;
  hipError_t e = dispatch_tier(d, stream);
  if (e == hipErrorInvalidValue) return m2r_fail("tier step: unsupported tier layout");
  return m2r_check(e, "tier step launch");
}

int m2r_forced_step_shape() { return g_forced_shape.load(std::memory_order_relaxed); }

extern "C" int m2r_set_step_shape(int waves_per_block, int heads_per_wave) {
  const int w = waves_per_block, k = heads_per_wave;
  const bool ok = (w == 0 && k == 0) || (w == 1 && k == 1) ||
                  (w == 4 && (k == 0 || k == 1 || k == 2 || k == 4 || k == -2 || k == -4)) || (w == 8 && k == 2);
  if (!ok)
    return m2r_fail("step shape: supported (waves, heads per wave) are (1,1), (4,1), (4,2), (4,4), (8,2), "
                    "(4,0) = (4,-2) = two waves per head, (4,-4) = four waves per head, or (0,0)");
  g_forced_shape.store(k == -4 ? FOUR_PER_SLOT : w * 16 + (k < 0 ? 0 : k), std::memory_order_relaxed);
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
                (uint16_t*)y, (int)batch, (int)L, (int)H, (int)P, (int)G, d_is_f32, db_is_f32,
                dma_tiles_ok(P, {lo, hi, q4, s8, s4}, {B, C}) | staged_ok(H, {x, dt, A, D, dt_bias, perm})};
  return m2r_check(launch_layout<16, 64, 48, MODE_LEGACY>(args, stream), "legacy step launch");
}
