// One launch of the one-token ridge-latent state step over many layers.
//
// The model runs one step launch per layer (m2r_state_step_ridge), because
// each layer's inputs come from the previous layer's projections.  When the
// layers' inputs are already resident (the synthetic 56-layer benchmark, or
// independent states stepped together), one launch can cover every layer:
// each workgroup reads its layer's arguments from a table in device memory
// and runs the same per-workgroup step as the per-layer kernel, dispatched
// on the layer's tier layout.  At batch 1 this removes 55 launch gaps and
// 55 serial prologues per token; the results are those of the per-layer
// launches, bit for bit.
//
// The table is staged by the entry point into device memory: into a
// workspace the caller passes (m2r_state_step_ridge_layers), or into a static
// device array that the library owns (m2r_state_step_ridge_layers_noalloc,
// for callers that cannot allocate).
#include "m2r_step.h"
#include "m2r_abi_util.h"
#include "../../include/m2r.h"

#include <mutex>
#include <vector>

namespace m2r {

struct LayerEntry {
  StepArgs args;
  int layout;       // index into the published-layout list below
  int pad[3];
};

// The seven published ridge layouts (scripts/fp4_zero_predictor_codec_v1.py:
// 28-36 applied to scripts/w4_state_repair_codec_v2.py:27-28), as (n8, n4, nz).
constexpr int kLayouts[7][3] = {{36, 20, 72}, {16, 60, 52}, {32, 28, 68}, {40, 12, 76},
                                {24, 44, 60}, {8, 76, 44},  {44, 4, 80}};

template <int WPB, int HPW>
struct LayersSmem {
  template <int K>
  using S = StepSmem<kLayouts[K][0], kLayouts[K][1], kLayouts[K][2], MODE_RIDGE, WPB, HPW, true, true>;
  static constexpr size_t bytes() {
    size_t m = sizeof(S<0>);
    m = sizeof(S<1>) > m ? sizeof(S<1>) : m;
    m = sizeof(S<2>) > m ? sizeof(S<2>) : m;
    m = sizeof(S<3>) > m ? sizeof(S<3>) : m;
    m = sizeof(S<4>) > m ? sizeof(S<4>) : m;
    m = sizeof(S<5>) > m ? sizeof(S<5>) : m;
    m = sizeof(S<6>) > m ? sizeof(S<6>) : m;
    return m;
  }
};

// Grid (P blocks, H / (WPB HPW), batch x layers): block z covers batch row
// z % batch of layer z / batch.
template <int WPB, int HPW>
__global__ __launch_bounds__(64 * WPB) __attribute__((amdgpu_waves_per_eu(2, 8)))
void k_state_step_layers(const LayerEntry* __restrict__ table, int batch) {
  __shared__ __align__(16) uint8_t smem[LayersSmem<WPB, HPW>::bytes()];
  const int layer = blockIdx.z / batch;
  const int b = blockIdx.z - layer * batch;
  const StepArgs a = table[layer].args;
  const int id = table[layer].layout;
#define M2R_LAYER_CASE(K)                                                                                  \
  case K:                                                                                                  \
    state_step_body<kLayouts[K][0], kLayouts[K][1], kLayouts[K][2], MODE_RIDGE, WPB, HPW, true, true>(      \
        a, *reinterpret_cast<typename LayersSmem<WPB, HPW>::template S<K>*>(smem), blockIdx.x, blockIdx.y, b); \
    break;
  switch (id) {
    M2R_LAYER_CASE(0)
    M2R_LAYER_CASE(1)
    M2R_LAYER_CASE(2)
    M2R_LAYER_CASE(3)
    M2R_LAYER_CASE(4)
    M2R_LAYER_CASE(5)
    M2R_LAYER_CASE(6)
    default: break;
  }
#undef M2R_LAYER_CASE
}

// Static staging area of the no-allocation entry point: the device copy of
// one call's layer table, at most M2R_LAYERS_NOALLOC_MAX layers (48 KiB).
// Each GPU the library runs on holds its own copy for the life of the
// process; calls that overlap on one GPU (other streams, other host threads)
// race on it.
__device__ __align__(256) uint8_t scratch[M2R_LAYERS_NOALLOC_MAX * sizeof(LayerEntry)];

// The device address of `scratch` on each device, resolved once per device
// with that device current (the array's name is a host-side stand-in that
// must never reach a kernel or a copy).
static constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

static int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return m2r_fail("layers step (no-alloc): no current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return m2r_check(e, "layers step (no-alloc): scratch address");
    if (!p) return m2r_fail("layers step (no-alloc): scratch address is null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Host staging of the no-allocation entry point's table: a fixed buffer
// under a lock (no host allocation either).
static LayerEntry g_noalloc_table[M2R_LAYERS_NOALLOC_MAX];
static std::mutex g_noalloc_mu;

static int layout_id(int n8, int n4, int nz) {
  for (int k = 0; k < 7; ++k)
    if (kLayouts[k][0] == n8 && kLayouts[k][1] == n4 && kLayouts[k][2] == nz) return k;
  return -1;
}

static bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Validates the call, fills `table` and picks the workgroup shape.
static int build_table(const m2r_ridge_layer* layers, int nlayers, int64_t batch, int64_t H, int64_t P, int64_t G,
                       LayerEntry* table, int& wpb, int& hpw) {
  if (!layers || nlayers <= 0) return m2r_fail("layers step: no layers");
  if (batch <= 0 || H <= 0 || P <= 0 || G <= 0) return m2r_fail("layers step: non-positive geometry");
  if (H % G) return m2r_fail("layers step: heads must be divisible by groups");
  if (batch * nlayers > 65535) return m2r_fail("layers step: batch x layers exceeds the grid limit 65535");
  if ((double)batch * H * P >= 2147483647.0) return m2r_fail("layers step: B*H*P must fit int32");
  if (P % 8) return m2r_fail("layers step: P must be a multiple of 8");
  if (H % 2) return m2r_fail("layers step: H must be even");
  const int64_t hpg = H / G;
  const int64_t slots = batch * H * ((P + 63) / 64);
  if (hpg % 16 == 0 && slots >= 16LL * 512) { wpb = 4; hpw = 4; }
  else if (hpg % 8 == 0 && slots >= 8LL * 512) { wpb = 4; hpw = 2; }
  else if (hpg % 4 == 0) { wpb = 4; hpw = 1; }
  else return m2r_fail("layers step: heads per group must be a multiple of 4");
  for (int i = 0; i < nlayers; ++i) {
    const m2r_ridge_layer& l = layers[i];
    const int id = layout_id(l.n8, l.n4, l.nz);
    if (id < 0) return m2r_fail("layers step: unsupported tier layout");
    const void* a16[] = {l.lo, l.hi, l.q4, l.latent, l.s8, l.s4, l.pred};
    const void* a4[] = {l.B, l.C, l.lscale};
    for (const void* q : a16)
      if (!q || !aligned(q, 16)) return m2r_fail("layers step: state arrays and pred must be 16-byte aligned");
    for (const void* q : a4)
      if (!q || !aligned(q, 4)) return m2r_fail("layers step: B, C and lscale must be 4-byte aligned");
    if (!l.x || !l.dt || !l.A || !l.D || !l.dt_bias || !l.perm || !l.basis || !l.y)
      return m2r_fail("layers step: null pointer");
    const void* a4s[] = {l.x, l.dt, l.A, l.D, l.dt_bias, l.perm, l.basis};
    for (const void* q : a4s)
      if (!aligned(q, 4)) return m2r_fail("layers step: x, dt, A, D, dt_bias, perm and basis must be 4-byte aligned");
    LayerEntry& e = table[(size_t)i];
    e = LayerEntry{};
    e.args = StepArgs{(const uint16_t*)l.x, (const uint16_t*)l.dt, l.A, (const uint16_t*)l.B, (const uint16_t*)l.C,
                      l.D, l.dt_bias, l.perm, (const uint16_t*)l.basis, (const uint16_t*)l.lscale,
                      (const uint16_t*)l.pred, l.lo, l.hi, l.q4, l.latent, (uint16_t*)l.s8, (uint16_t*)l.s4,
                      (uint16_t*)l.y, (int)batch, 1, (int)H, (int)P, (int)G, l.d_is_f32, l.db_is_f32, 3};
    e.args.rhpg = 1.0f / (float)hpg;
    e.layout = id;
  }
  return 0;
}

static int launch_layers(const LayerEntry* dev_table, int nlayers, int64_t batch, int64_t H, int64_t P, int wpb,
                         int hpw, hipStream_t stream) {
  const dim3 grid((unsigned)((P + 63) / 64), (unsigned)(H / (wpb * hpw)), (unsigned)(batch * nlayers));
  if (hpw == 4) hipLaunchKernelGGL((k_state_step_layers<4, 4>), grid, dim3(256), 0, stream, dev_table, (int)batch);
  else if (hpw == 2) hipLaunchKernelGGL((k_state_step_layers<4, 2>), grid, dim3(256), 0, stream, dev_table, (int)batch);
  else hipLaunchKernelGGL((k_state_step_layers<4, 1>), grid, dim3(256), 0, stream, dev_table, (int)batch);
  return m2r_check(hipGetLastError(), "layers step launch");
}

// Host copy of the table, per host thread (the copy into device memory is
// staged before hipMemcpyAsync returns, so the buffer is reusable at once).
static thread_local std::vector<LayerEntry> t_table;

// Both entry points copy the table from host memory that the next call
// overwrites.  Captured into a graph, that copy would read the host buffer at
// replay time, when it holds whatever table the latest call built: the
// replay would step another call's layers with the captured grid.  So a
// capturing stream is rejected before anything is enqueued.
static int reject_capture(hipStream_t stream, const char* what) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (int e = m2r_check(hipStreamIsCapturing(stream, &st), what)) return e;
  if (st != hipStreamCaptureStatusNone)
    return m2r_fail("layers step: the stream is capturing a graph; the layer table is copied from host memory "
                    "that later calls overwrite, so this entry point cannot be captured (launch it eagerly)");
  return 0;
}

}  // namespace m2r

using namespace m2r;

extern "C" int64_t m2r_state_step_ridge_layers_workspace(int nlayers) {
  return nlayers > 0 ? (int64_t)nlayers * (int64_t)sizeof(LayerEntry) : 0;
}

extern "C" int m2r_state_step_ridge_layers(const m2r_ridge_layer* layers, int nlayers, int64_t batch, int64_t H,
                                           int64_t P, int64_t G, void* workspace, int64_t workspace_bytes,
                                           hipStream_t stream) {
  int wpb = 0, hpw = 0;
  if (nlayers > 65535) return m2r_fail("layers step: batch x layers exceeds the grid limit 65535");
  if (nlayers > 0) t_table.resize((size_t)nlayers);
  if (int e = build_table(layers, nlayers, batch, H, P, G, t_table.data(), wpb, hpw)) return e;
  const int64_t need = m2r_state_step_ridge_layers_workspace(nlayers);
  if (!workspace || !aligned(workspace, 16) || workspace_bytes < need)
    return m2r_fail("layers step: workspace must be 16-byte aligned and hold m2r_state_step_ridge_layers_workspace(nlayers) bytes");
  if (int e = reject_capture(stream, "layers step: capture query")) return e;
  if (int e = m2r_check(hipMemcpyAsync(workspace, t_table.data(), (size_t)need, hipMemcpyHostToDevice, stream),
                        "layers step table copy"))
    return e;
  return launch_layers((const LayerEntry*)workspace, nlayers, batch, H, P, wpb, hpw, stream);
}

extern "C" int m2r_state_step_ridge_layers_noalloc(const m2r_ridge_layer* layers, int nlayers, int64_t batch,
                                                   int64_t H, int64_t P, int64_t G, hipStream_t stream) {
  if (nlayers > M2R_LAYERS_NOALLOC_MAX)
    return m2r_fail("layers step (no-alloc): more than M2R_LAYERS_NOALLOC_MAX (256) layers in one call");
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  int wpb = 0, hpw = 0;
  if (int e = build_table(layers, nlayers, batch, H, P, G, g_noalloc_table, wpb, hpw)) return e;
  if (int e = reject_capture(stream, "layers step (no-alloc): capture query")) return e;
  void* dev_table = nullptr;
  if (int e = scratch_address(&dev_table)) return e;
  const size_t bytes = (size_t)m2r_state_step_ridge_layers_workspace(nlayers);
  if (int e = m2r_check(hipMemcpyAsync(dev_table, g_noalloc_table, bytes, hipMemcpyHostToDevice, stream),
                        "layers step (no-alloc) table copy"))
    return e;
  return launch_layers((const LayerEntry*)dev_table, nlayers, batch, H, P, wpb, hpw, stream);
}
