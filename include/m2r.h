/*
 * m2r.h - C ABI of libm2r_hip.so, the MI355X (gfx950) state codec and FP4
 * weight decode of mamba2-recall.
 *
 * Conventions for every entry point:
 *   - all pointers are device pointers to contiguous buffers, binary16 data
 *     is passed as `const void*` / `void*` (IEEE binary16 bit patterns);
 *   - work is enqueued on `stream` (a hipStream_t) and never synchronizes,
 *     never allocates device memory;
 *   - the return value is 0 on success; nonzero means the call was rejected
 *     or the launch failed, and m2r_last_error() (per host thread) describes
 *     why.  Shape/dtype validation beyond what is stated here is the host
 *     wrapper's job (the Python package raises the reference's ValueError /
 *     RuntimeError / FloatingPointError types).
 *
 * Shapes: batch B, tokens L, heads H, head dim P, groups G (H % G == 0),
 * state coordinates 128.  Rows are r = (b*H + h)*P + p.
 */
#ifndef M2R_H
#define M2R_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Library identity and error text of the last failing call on this thread. */
int m2r_abi_version(void);
const char* m2r_last_error(void);

/*
 * Ridge-latent 52-byte state step: decode packed rows, run L selective-state
 * tokens (decay, dt*B x update, C readout with the latent and static ridge
 * predictor terms, D skip), requantize after every token, write y [B,L,H,P]
 * FP16 and the packed rows back in place.
 * Replaces scripts/fp4_zero_predictor_codec_v1.py:184-236 (scan, including the
 * einsum correction :221-225) and its Triton kernel _latent_scan :76-181.
 *   x f16[B,L,H,P]; dt f16[B,L,H]; A f32[H]; B,C f16[B,L,G,128];
 *   D, dt_bias f16 or f32 [H] (flag 1 = f32); perm u8[G,128];
 *   basis f16[G,nz,2]; lscale f16[G,2] (> 0); pred f16[G,n8+n4+2,nz];
 *   lo,hi u8[rows,n8/2]; q4 u8[rows,n4/2]; latent e4m3[rows,2];
 *   s8,s4 f16[rows]; (n8,n4,nz) one of the seven published layouts.
 * Fastest with P % 8 == 0, 16-byte aligned state arrays and pred, 4-byte
 * aligned B, C and lscale; other alignments give the same results, slower.
 */
int m2r_state_step_ridge(const void* x, const void* dt, const float* A, const void* B, const void* C,
                         const void* D, int d_is_f32, const void* dt_bias, int db_is_f32, const uint8_t* perm,
                         const void* basis, const void* lscale, const void* pred, uint8_t* lo, uint8_t* hi,
                         uint8_t* q4, uint8_t* latent, void* s8, void* s4, void* y, int64_t batch, int64_t L,
                         int64_t H, int64_t P, int64_t G, int n8, int n4, int nz, hipStream_t stream);

/*
 * The same step with a caller workspace for its token records.  The
 * reference computes the ridge correction of every token's readout weights
 * before its scan (scripts/fp4_zero_predictor_codec_v1.py:221-225, the einsum
 * over all L tokens); here, for L > 1 on the small-batch shapes (at most 1024
 * 64-row slots) with 16-byte transfers, a first kernel writes one record per
 * (batch row, token, group) of the state-independent token values (readout
 * weights with the correction, dead-tier dot products, sum b.c, the carried
 * b) into `workspace`, and the scan reads them instead of building each token
 * itself.  Results are identical to m2r_state_step_ridge bit for bit.
 * workspace: null (then exactly m2r_state_step_ridge), or 16-byte aligned
 * device memory of at least m2r_ridge_records_bytes(batch, L, G) bytes,
 * used on `stream` only (calls that overlap on one workspace race).
 */
int m2r_state_step_ridge_ws(const void* x, const void* dt, const float* A, const void* B, const void* C,
                            const void* D, int d_is_f32, const void* dt_bias, int db_is_f32, const uint8_t* perm,
                            const void* basis, const void* lscale, const void* pred, uint8_t* lo, uint8_t* hi,
                            uint8_t* q4, uint8_t* latent, void* s8, void* s4, void* y, int64_t batch, int64_t L,
                            int64_t H, int64_t P, int64_t G, int n8, int n4, int nz, void* workspace,
                            int64_t workspace_bytes, hipStream_t stream);
/* Workspace bytes of m2r_state_step_ridge_ws: batch * L * G records of 1 KiB. */
int64_t m2r_ridge_records_bytes(int64_t batch, int64_t L, int64_t G);

/*
 * Stored-scale tier step (INT8/INT4/zero-carry), same row format without the
 * latent.  Replaces scripts/state_ppl_codec_v10.py:157-192 (scan, _tier_scan
 * :78-154), scripts/w4_state_repair_codec_v2.py:103-137 (scan) and the
 * stored_scale path of scripts/state_ppl_codec_v6.py:198-254.
 */
int m2r_state_step_tier(const void* x, const void* dt, const float* A, const void* B, const void* C,
                        const void* D, int d_is_f32, const void* dt_bias, int db_is_f32, const uint8_t* perm,
                        uint8_t* lo, uint8_t* hi, uint8_t* q4, void* s8, void* s4, void* y, int64_t batch,
                        int64_t L, int64_t H, int64_t P, int64_t G, int n8, int n4, int nz, hipStream_t stream);

/*
 * Legacy sq3p25 step (16/64/48, binary32-denominator quantization).
 * Replaces mamba2_recall/state_codec.py:203-262 (scan, sq3p25 branch) and its
 * Triton kernel _sq_scan :105-176.
 */
int m2r_state_step_legacy(const void* x, const void* dt, const float* A, const void* B, const void* C,
                          const void* D, int d_is_f32, const void* dt_bias, int db_is_f32, const uint8_t* perm,
                          uint8_t* lo, uint8_t* hi, uint8_t* q4, void* s8, void* s4, void* y, int64_t batch,
                          int64_t L, int64_t H, int64_t P, int64_t G, hipStream_t stream);

/*
 * Test and tuning hook for the three steps above: force the workgroup shape
 * (waves per workgroup, 64-row head slots per wave) to one of (1,1), (4,1),
 * (4,2), (4,4), (8,2), (4,0) = (4,-2): four waves, two per head slot (the
 * automatic choice at small batches), or (4,-4): four waves, all on one head
 * slot (each wave steps a quarter of the carried coordinates); (0,0) restores
 * the automatic choice.  A forced shape whose head count does not divide the heads per group
 * falls back to the automatic choice.  Process-wide; results do not depend on the shape.  No counterpart
 * in the reference (its Triton launch grid is fixed per call).
 */
int m2r_set_step_shape(int waves_per_block, int heads_per_wave);

/*
 * Dense 3-bit step: codes u8[rows,3,16] (bit planes), scales f16[rows,2];
 * table u8[G,128] permutation (table_is_equalizer = 0) or i8[G,128] power-of-two
 * exponents in [-8, 8] (1).  Replaces mamba2_recall/state_codec_dense3.py:151-186
 * (scan) and its Triton kernel _scan :82-148.
 */
int m2r_state_step_dense3(const void* x, const void* dt, const float* A, const void* B, const void* C,
                          const void* D, int d_is_f32, const void* dt_bias, int db_is_f32, const void* table,
                          int table_is_equalizer, uint8_t* codes, void* scales, void* y, int64_t batch, int64_t L,
                          int64_t H, int64_t P, int64_t G, hipStream_t stream);

/*
 * FP16-carry control step: state f16[B,H,P,128] in original coordinates;
 * stats (may be NULL) f32[B,H,ceil(P/16),128] receives sum over tokens and the
 * 16 rows of each P tile of |FP16 carry|.  Replaces
 * mamba2_recall/state_codec.py:203-262 (scan, s16 branch) and _s16_scan :65-102.
 */
int m2r_state_step_s16(const void* x, const void* dt, const float* A, const void* B, const void* C, const void* D,
                       int d_is_f32, const void* dt_bias, int db_is_f32, void* state, void* y, float* stats,
                       int64_t batch, int64_t L, int64_t H, int64_t P, int64_t G, hipStream_t stream);

/*
 * Diagnostic decode of packed rows to f32 [rows,128] in packed lane order.
 * kind 0: INT8/INT4 tiers (lo, hi, q4, s8, s4; the zero tier decodes to 0);
 * kind 1: dense 3-bit (codes in `lo`, f16[rows,2] scales in `s8`).
 * Replaces the torch bodies of mamba2_recall/state_codec.py:269-296,
 * state_codec_dense3.py:189-212 and w4_state_repair_codec_v2.py:141-162
 * (before their permutation scatter).  `latent`, `extra`, `flags`: reserved.
 */
int m2r_state_decode(int kind, int n8, int n4, int nz, const uint8_t* lo, const uint8_t* hi, const uint8_t* q4,
                     const uint8_t* latent, const void* s8, const void* s4, const void* extra, float* out,
                     int64_t batch, int64_t H, int64_t P, int64_t flags, hipStream_t stream);

/*
 * Diagnostic legacy encode of f32 [rows,128] packed-order values into sq3p25
 * rows (binary32 denominators, sign(z)*floor(|z|+0.5) codes).  Replaces the
 * torch body of mamba2_recall/state_codec.py:299-331 (encode_state_).
 */
int m2r_state_encode_legacy(const float* v, uint8_t* lo, uint8_t* hi, uint8_t* q4, void* s8, void* s4, int64_t rows,
                            hipStream_t stream);

/*
 * FP4 E2M1 G16 decode: packed u8[rows, ceil(cols/16)*8], e4m3_scales
 * u8[rows, ceil(cols/16)] (E4M3FN bytes), global_scale f32[1] (device),
 * out f16[rows, cols].  err_flag (may be NULL) is a device u32 that receives
 * the OR of: 1 nonfinite scale, 2 negative scale, 4 nonzero code in a zero
 * group, 8 nonfinite decoded value, 16 nonzero padding, 32 bad global scale.
 * Replaces mamba2_recall/fp4.py:225-250 (decode_packet, G16 branch) with the
 * op chain :100-103, :125-130, :151-154.
 */
int m2r_fp4_decode_g16(const uint8_t* packed, const uint8_t* e4m3_scales, const float* global_scale, void* out_f16,
                       int64_t rows, int64_t cols, uint32_t* err_flag, hipStream_t stream);

/*
 * Tuning and test hook for m2r_fp4_decode_g16 (cols % 16 == 0): units of 8
 * weights per thread (1, 2, 4 or 8; 0 restores the automatic choice), the
 * grid cap in 256-thread workgroups (0: no cap, one pass; a cap makes the
 * workgroups stride over the matrix) and non-temporal (1) or default (0)
 * output stores.  While a shape is forced, m2r_fp4_decode_g64 takes the same
 * grid cap.  Process-wide; results do not depend on the shape.  No
 * counterpart in the reference.
 */
int m2r_set_fp4_decode_shape(int units_per_thread, int max_blocks, int nontemporal);

/* FP4 E2M1 G64 decode with f16 scales u16[rows, ceil(cols/64)]; same error bits
 * (32 unused).  Replaces mamba2_recall/fp4.py:225-250, G64 branch. */
int m2r_fp4_decode_g64(const uint8_t* packed, const void* f16_scales, void* out_f16, int64_t rows, int64_t cols,
                       uint32_t* err_flag, hipStream_t stream);

/*
 * Probes of the exact arithmetic primitives, for known-answer testing.
 * m2r_probe_stored_quantize replaces scripts/state_ppl_codec_v6.py:72-80
 * (quantize_stored_probe): q = s > 0 ? clamp(roundf(RN(v/s)), +-limit) : 0,
 * limit 7 or 127.  m2r_probe_unary applies primitive `op` (0 f32->f16 bits,
 * 1 f16->f32, 2 f32->e4m3, 3 e4m3->f32, 4 roundf, 5 exp, 6 log, 7 dt
 * softplus, 8 reciprocal of a binary16 value, 9 e4m3->f32 and 10 f32->e4m3
 * by the FP8 instructions) to u32 words; m2r_probe_div computes RN(a/d) in the kernels'
 * reciprocal form.  These three have no counterpart besides the first.
 */
int m2r_probe_stored_quantize(const float* v, const void* s_f16, int32_t* q, int64_t n, int limit, hipStream_t stream);
int m2r_probe_unary(const uint32_t* in, uint32_t* out, int64_t n, int op, hipStream_t stream);
int m2r_probe_div(const float* a, const float* d, float* q, int64_t n, hipStream_t stream);
/* One wave (in: 192 floats, out: 386 floats): out[64*l + lane] is the
 * level-l butterfly pair sum of in[lane] (l = 0..5); out[384] / out[385] are
 * the canonical adjacent-pair tree sums of in[64..191] / in[0..63]. */
int m2r_probe_butterfly(const float* in, float* out, hipStream_t stream);

/*
 * HBM streaming probe (measurement only; no counterpart in the reference):
 * `units` units, each reading `read_bytes` bytes (0, 4, 16 or 32) and writing
 * `writes` 16-byte vectors (src: units*read_bytes bytes, dst:
 * units*writes*16 bytes, at least 16; both 16-byte aligned); every store
 * instruction of a wave is a contiguous 1 KiB, every load a contiguous
 * 64*min(read_bytes,16) bytes; each lane issues `burst` units' loads before
 * their stores, over a grid-stride grid of `blocks` workgroups of 256 threads
 * (0: one step per wave), with the default (nontemporal = 0) or the
 * non-temporal cache policy.  (read_bytes, writes, burst) in {(16,0), (0,1),
 * (16,1), (32,7)} x burst {1, 8}, or (4,1) with burst 1 or 4; units a
 * multiple of 64*burst.  Gives the read-only, write-only, 1:1, 22:78 (the FP4
 * G16 decode's byte mix) and dword-read 20:80 (its access shape) ceilings.
 */
int m2r_stream_probe(const void* src, void* dst, int64_t units, int read_bytes, int writes, int burst, int blocks,
                     int nontemporal, hipStream_t stream);

/*
 * Read-fraction sweep and time-phased variants of the streaming probe (no
 * counterpart in the reference; a measurement aid).  Each of `steps`
 * workgroup steps (256 threads) loads read_vectors 16-byte vectors per thread
 * from a contiguous source block and stores write_vectors per thread to a
 * contiguous destination block (src: steps*256*read_vectors*16 bytes, dst:
 * steps*256*max(write_vectors,1)*16 bytes, 16-byte aligned), grid-stride over
 * `blocks` workgroups (0: one step each).  phase 0: a thread stores as soon as
 * its own loads land; 1: a workgroup barrier separates the step's loads from
 * its stores; 2: the step's stores also complete, behind a barrier, before
 * the next step's loads.  (read_vectors, write_vectors) in {(1,0), (0,1),
 * (1,9), (1,4), (4,16), (3,7), (1,1)}: 100, 0, 10, 20, 20, 30 and 50% of
 * the bytes read.
 */
int m2r_stream_probe_phased(const void* src, void* dst, int64_t steps, int read_vectors, int write_vectors,
                            int phase, int blocks, int nontemporal, hipStream_t stream);

/*
 * One launch of the one-token ridge-latent step over many layers whose inputs
 * are all resident: every workgroup reads its layer's arguments from a table
 * and runs the per-layer step on them (results identical to one
 * m2r_state_step_ridge call per layer with L = 1).  No counterpart in the
 * reference, which steps one layer per mixer call; it is the one-launch
 * all-layers variant of the batch-1 step (a 56-layer token otherwise takes
 * 56 launches).  Requirements on every layer: a published layout, P % 8 == 0,
 * 16-byte aligned lo, hi, q4, latent, s8, s4 and pred, 4-byte aligned B, C
 * and lscale; all layers share batch, H, P and G; batch * nlayers <= 65535.
 * The entry point copies the table (host array `layers`, reusable when the
 * call returns) into `workspace`, a 16-byte aligned device buffer of at
 * least m2r_state_step_ridge_layers_workspace(nlayers) bytes, on `stream`.
 */
typedef struct m2r_ridge_layer {
  const void* x;        /* f16 [B,1,H,P] */
  const void* dt;       /* f16 [B,1,H] */
  const float* A;       /* f32 [H] */
  const void* B;        /* f16 [B,1,G,128] */
  const void* C;        /* f16 [B,1,G,128] */
  const void* D;        /* f16 or f32 [H] */
  const void* dt_bias;  /* f16 or f32 [H] */
  const uint8_t* perm;  /* u8 [G,128] */
  const void* basis;    /* f16 [G,nz,2] */
  const void* lscale;   /* f16 [G,2] */
  const void* pred;     /* f16 [G,n8+n4+2,nz] */
  uint8_t* lo;
  uint8_t* hi;
  uint8_t* q4;
  uint8_t* latent;
  void* s8;
  void* s4;
  void* y;              /* f16 [B,1,H,P] */
  int32_t n8, n4, nz;
  int32_t d_is_f32, db_is_f32;
  int32_t reserved;
} m2r_ridge_layer;
int64_t m2r_state_step_ridge_layers_workspace(int nlayers);
int m2r_state_step_ridge_layers(const m2r_ridge_layer* layers, int nlayers, int64_t batch, int64_t H, int64_t P,
                                int64_t G, void* workspace, int64_t workspace_bytes, hipStream_t stream);

/*
 * The same one-launch multi-layer step with no workspace argument and no
 * allocation of any kind (no hipMalloc/hipFree, no host heap): the device copy
 * of the layer table goes to a static device array of the library, at most
 * M2R_LAYERS_NOALLOC_MAX layers per call (larger calls are rejected).  No
 * counterpart in the reference; it is for callers that cannot allocate
 * (tight serving loops, harnesses that forbid allocation).  Every call on
 * one GPU shares that GPU's array (and the library's host staging buffer,
 * under a lock): calls that overlap on one GPU, from other streams or host
 * threads, race; calls on one stream are ordered.  Results equal
 * m2r_state_step_ridge_layers'.  Neither multi-layer entry point can be
 * captured into a HIP graph: each copies the table from host memory that
 * later calls overwrite, so on a capturing stream both return an error
 * before enqueueing anything.
 */
#define M2R_LAYERS_NOALLOC_MAX 256
int m2r_state_step_ridge_layers_noalloc(const m2r_ridge_layer* layers, int nlayers, int64_t batch, int64_t H,
                                        int64_t P, int64_t G, hipStream_t stream);

/*
 * One-token causal depthwise convolution update of the Mamba-2 mixer: roll
 * the cached window one step, store the new projection column, and write
 * out = silu(sum_t half(window_t * weight[c,t]) + bias[c]) in binary16.
 * Replaces the PyTorch fallback of mamba2_recall/state_quant.py:289-297
 * (the update branch of _convolution), with the same rounding sequence.
 *   window f16 [B, C, width] addressed through element strides (ws_b, ws_c,
 *   ws_t), updated in place; value f16 [B, C] with batch stride vs_b (channel
 *   stride 1); weight f16 [C, width] contiguous; bias f16 [C] or NULL;
 *   out f16 [B, C] contiguous; width must be 4; silu 1 applies the SiLU.
 */
int m2r_causal_conv_update(void* window, int64_t ws_b, int64_t ws_c, int64_t ws_t, const void* value, int64_t vs_b,
                           const void* weight, const void* bias, void* out, int64_t batch, int64_t channels,
                           int width, int silu, hipStream_t stream);

/*
 * Gated RMS norm of the Mamba-2 mixer, norm_before_gate = False: per group of
 * group_size channels of each row, v = y * (z * sigmoid(z)) in binary32,
 * out = half((v / sqrt(mean(v^2) + eps)) * weight).  Replaces the gated norm
 * module the reference's controllers call as mx.norm(y, z)
 * (mamba2_recall/state_quant.py:298-300; mamba_ssm's RMSNormGated, a
 * third-party Triton kernel).  The sum of squares is a fixed tree, so the
 * results are deterministic; they agree with a binary32/binary64
 * restatement of the formula to one binary16 rounding.
 *   y, z f16 rows of `channels` with element row strides y_stride, z_stride;
 *   weight f16 [channels]; out f16 rows with stride out_stride.  Pointers
 *   8-byte aligned, strides multiples of 4 elements; group_size a multiple
 *   of 4, at most 4096, dividing channels; rows and groups at most 65535.
 */
int m2r_gated_rmsnorm(const void* y, int64_t y_stride, const void* z, int64_t z_stride, const void* weight, void* out,
                      int64_t out_stride, int64_t rows, int64_t channels, int64_t group_size, float eps,
                      hipStream_t stream);

/*
 * Packed-resident FP4 G16 matrix-vector product: y[m, n] = sum_k u[m, k] *
 * w[n, k] with W read directly in the checkpoint's packed format.  Every
 * weight is the binary16 value m2r_fp4_decode_g16 produces; products
 * accumulate in binary32; y is FP16.  No counterpart in the reference, which
 * decodes the whole model to resident FP16 before its GEMMs
 * (mamba2_recall/fp4_checkpoint.py:345-405); this is the packed-resident
 * GEMV that the reference lacks (README.md:40-41), for small-batch decode.
 *   packed u8[N, K/2] (16-byte aligned), e4m3_scales u8[N, K/16] (2-byte
 *   aligned), global_scale device f32; u f16 rows of K with row stride
 *   u_stride (16-byte aligned, u_stride % 8 == 0); y f16 rows of N with row
 *   stride y_stride.  M in {1, 2, 4}; K in {2048, 4096, 8192}.  The packet
 *   must satisfy the decode checks (no error word here).
 */
int m2r_fp4_gemv_g16(const uint8_t* packed, const uint8_t* e4m3_scales, const float* global_scale, const void* u,
                     int64_t u_stride, void* y, int64_t y_stride, int64_t M, int64_t N, int64_t K,
                     hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* M2R_H */
