/* svla.h — C-ABI of the MI355X (gfx950) SmolVLA bf16 hot-path library.
 *
 * Drop-in boundary for the reference's per-kernel AIE ABI
 * (`extern "C" void f(T in[R][C], ..., T out[R][C])`, caller-owned buffers,
 * outputs written in place, e.g. cc/bf16/rms_norm_960_bf16.cc:60) and for the
 * host tiling helpers that drive it from numpy (vla/text_encoder_bf16.py:398-475,
 * vla/action_expert_bf16.py:517-655).  Unlike the AIE ABI the shapes are
 * runtime arguments and every entry point reports errors.
 *
 * Conventions
 *  - All pointers are DEVICE pointers (hipMalloc / torch CUDA tensors) unless
 *    the parameter is documented as a host value.  bf16 tensors are IEEE
 *    bfloat16 (2 bytes), row-major with explicit leading dimensions counted in
 *    elements.  16-byte alignment and leading dimensions that are multiples of
 *    8 elements are required where noted ("aligned").
 *  - Linear weights are consumed PACKED as [N, K] (out-features x in-features,
 *    K contiguous, i.e. nn.Linear's own layout).  The reference stores them
 *    [in, out] (vla/text_encoder_bf16.py:601-611); svla_pack_weight_bf16 turns
 *    one into the other on the device.
 *  - Caller owns all memory except one split-K workspace per device (skinny
 *    GEMMs, see svla_linear_bf16), which svla_init allocates at set-up (or the
 *    first split call outside graph capture, if svla_init was not called); the
 *    library keeps no per-call state.  Calls are asynchronous on the given
 *    stream (NULL = default stream) and may be captured in a HIP graph (no
 *    memset / allocation inside).
 *  - Concurrency: calls on one stream, and replays of graphs captured from one
 *    stream, are ordered and bit-reproducible.  Kernels on different streams
 *    of one device may run at the same time (two engines' chunks replayed
 *    concurrently on two streams equal their serial runs bit for bit), except
 *    where a device-wide resource is shared:
 *      * the split-K workspace of the skinny GEMMs (svla_linear_bf16) and the
 *        static scratch array (svla_linear_scratch_bf16): split calls on
 *        different streams must not overlap in time (svla_gemm_set_split(1)
 *        turns splitting off);
 *      * the fused expert (svla_expert_run) keeps one workgroup on every CU
 *        for its whole run and they wait on each other: nothing else may run
 *        on the device meanwhile (its waits are bounded: a launch that cannot
 *        keep every CU ends within seconds with svla_expert_status != 0).
 *    An earlier corruption of concurrent runs came from a race in the
 *    pipelined GEMM and attention kernels: an LDS stage could be refilled
 *    before a wave's reads of its previous contents had completed (fixed).
 *  - Return value: 0 on success, SVLA_EINVAL for bad shapes/alignment, or a
 *    hipError_t (positive) from the launch.
 */
#ifndef SVLA_H
#define SVLA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SVLA_OK 0
#define SVLA_EINVAL (-22)
#define SVLA_ENOSPC (-28) /* svla_linear_scratch_bf16: the split needs more scratch than it has */

typedef void* svla_stream_t; /* hipStream_t */

/* activation codes (svla_linear_bf16 `act`) */
#define SVLA_ACT_NONE 0
#define SVLA_ACT_GELU_TANH 1
#define SVLA_ACT_GELU_ERF 2
#define SVLA_ACT_SILU 3

/* attention mask kinds */
#define SVLA_MASK_NONE 0
#define SVLA_MASK_CAUSAL 1
#define SVLA_MASK_PREFIX_LM 2

/* Layout flags of svla_linear_wide_bf16: slab-blocked A, W or C.  A blocked
 * [rows, K] matrix stores element (r, k) at (k / 32) * rows * 32 + r * 32 + k % 32. */
#define SVLA_LAYOUT_A_BLOCKED 1
#define SVLA_LAYOUT_W_BLOCKED 2
#define SVLA_LAYOUT_C_BLOCKED 4

/* Harness elementwise operations (svla_unary_*). */
#define SVLA_OP_SILU 0
#define SVLA_OP_GELU_TANH 1
#define SVLA_OP_GELU_ERF 2
#define SVLA_OP_SIN 3
#define SVLA_OP_COS 4

/* Harness row norms (svla_row_norm). */
#define SVLA_NORM_RMS 0     /* x * rsqrt(mean(x^2) + eps) * w                 (nn.RMSNorm) */
#define SVLA_NORM_RMS_ADD 1 /* x / (||x|| / sqrt(cols) + eps) * w             (harness RMSNorm module) */
#define SVLA_NORM_LAYER 2   /* (x - mean) / sqrt(var + eps) * w (+ b), biased var (LayerNorm) */

/* Library version (major*10000 + minor*100 + patch). */
int svla_version(void);

/* Set-up for the CURRENT device, once per device before any graph capture
 * (later calls return at once): allocates the split-K workspace of skinny
 * GEMMs (16 MB of fp32 partial tiles + 4096 arrival counters, kept until the
 * process ends), so that eager calls and calls captured into a graph split
 * long-K problems the same way, and resolves the device address of the static
 * scratch array of svla_linear_scratch_bf16 (allocating nothing for it),
 * clearing its counters.  Synchronises the device.  No counterpart in the
 * reference (its AIE modules are built per kernel by df.build at import,
 * vla/text_encoder_bf16.py:368-392). */
int svla_init(void);

/* ---------------------------------------------------------------- norms --
 * RMSNorm, y = x * rsqrt(mean(x^2) + eps) * w, fp32 math, one bf16 rounding.
 * Replaces rms_norm_960_bf16(bf16[4][960], bf16[960], bf16[4][960])
 * (cc/bf16/rms_norm_960_bf16.cc:60), rms_norm_bf16 (cc/bf16_old/rms_norm_bf16.cc:60)
 * and the tiling helper rmsnorm() (vla/text_encoder_bf16.py:398-404).
 * cols % 8 == 0, cols <= 2048, aligned. */
int svla_rmsnorm_bf16(const void* x, int ldx, const void* w, void* y, int ldy, int rows,
                      int cols, float eps, svla_stream_t stream);

/* LayerNorm with affine gamma/beta (beta may be NULL).
 * Replaces layer_norm_bf16 + the bias kernel (cc/bf16_old/layer_norm_bf16.cc:67;
 * vla/vision_block_bf16.py:101-127) and layernorm() (:272-280). */
int svla_layernorm_bf16(const void* x, int ldx, const void* gamma, const void* beta, void* y,
                        int ldy, int rows, int cols, float eps, svla_stream_t stream);

/* svla_layernorm_bf16 writing its output slab-blocked, [cols/32][rows][32] (the
 * A layout of svla_linear_wide_bf16 with SVLA_LAYOUT_A_BLOCKED); cols % 32 == 0.
 * Same values.  Replaces the same reference LayerNorm (vla/vision_block_bf16.py:101-127)
 * where its output feeds the big-batch ViT projections. */
int svla_layernorm_blocked_bf16(const void* x, int ldx, const void* gamma, const void* beta,
                                void* y, int rows, int cols, float eps, svla_stream_t stream);

/* ----------------------------------------------------------------- GEMM --
 * C[M,N] = epilogue(alpha * norm(A)[M,K] . W[N,K]^T) on bf16 MFMA (fp32 accumulate).
 * Replaces the Allo GEMM module GEMM(M,N,K,Pm,Pn,Pk,bf16,bf16) and its K-chunk
 * host accumulation (vla/text_encoder_bf16.py:174-225, 584-590; contract
 * cc/gemm.py:44-77), the attention-score kernel transpose_matmul_with_scale_bf16
 * (cc/bf16_old/transpose_matmul_with_scale_bf16.cc:52, alpha = 0.125) and the
 * residual adds (vla/text_encoder_bf16.py:532,592).
 * norm_w (may be NULL): the A rows are RMS-normalised on the fly,
 *   C[m,n] = sum_k bf16((x[m,k] * r[m]) * norm_w[k]) * W[n,k],
 *   r[m] = 1 / sqrt(mean_k(x[m,:]^2) + norm_eps)  (fp32),
 * the operand rounded exactly as svla_rmsnorm_bf16 rounds its output, so the
 * fused and the standalone norm give the same product; K <= 2048.
 * (the rmsnorm() that precedes every projection, vla/text_encoder_bf16.py:398-404).
 * Epilogue order (mirrors the torch modules' bf16 boundaries):
 *   v = alpha*acc (+ bias[n]) (+ bias_f32[n]); if out_f32: store fp32 v.
 *   else v = bf16(v); v = bf16(act(v)); if res: v = bf16(v + res[m,n]); store.
 * bias/bias_f32/res may be NULL; res may alias c (in-place residual update).
 * K % 8 == 0, N % 4 == 0, aligned.  Problems with few rows (M <= 256) split K
 * across the 8 waves of each workgroup and, when that grid is far smaller than
 * the chip, across workgroups too: the partial tiles go to a per-device
 * workspace (allocated by svla_init, or by the first such call that is not
 * being graph-captured; kept until exit; a split call captured before either
 * runs unsplit) and the last workgroup of each tile sums them in a fixed
 * order.  Split calls on different streams must not overlap in time (see
 * Concurrency above). */
int svla_linear_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                     const float* bias_f32, const void* res, int ldr, void* c, int ldc, int m,
                     int n, int k, float alpha, int act, int out_f32, const void* norm_w,
                     float norm_eps, svla_stream_t stream);

/* svla_linear_bf16 that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot call hipMalloc (code under HIP graph capture
 * before any set-up, tight serving loops, harnesses that forbid allocation).
 * Same arguments, kernels and results as svla_linear_bf16, bit for bit (the
 * same tile and the same K split); the split-K partial tiles of skinny
 * problems go to a static device array instead of the allocated workspace:
 * 4 MB of fp32 partials + 1024 arrival counters per device, held from module
 * load until the process ends.  A call whose split needs more (more than 1024
 * output tiles, or tiles x splits x (tile + 64) floats over 1M) returns
 * SVLA_ENOSPC and launches nothing; problems that do not split use no scratch
 * and have no limit.  The first call on a device (or svla_init) resolves the
 * array's device address (hipGetSymbolAddress, no allocation) and clears its
 * counters with a kernel on `stream`; every call leaves them at zero.  All
 * calls on one device share the array: calls that overlap in time on one
 * device race (see Concurrency above). */
int svla_linear_scratch_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                             const float* bias_f32, const void* res, int ldr, void* c, int ldc,
                             int m, int n, int k, float alpha, int act, int out_f32,
                             const void* norm_w, float norm_eps, svla_stream_t stream);

/* The big-problem GEMM of svla_linear_bf16 (persistent 256x256 tiles, plain
 * store epilogue: bias, fp32 bias, alpha, activation, residual) with optional
 * slab-blocked layouts (SVLA_LAYOUT_*): a slab-blocked operand streams into
 * LDS as contiguous kilobytes (measured on MI355X: ~41 B/clk/CU against
 * ~22 for the 64-byte row pieces of the row-major layout).  lda / ldw / ldc
 * are ignored for blocked matrices.  m % 256 == 0, n % 256 == 0,
 * k % 128 == 0, k >= 256; res (row-major) only with a row-major C.  Same numerics as
 * svla_linear_bf16.  Replaces the same reference GEMMs (the ViT projections,
 * vla/vision_block_bf16.py:135-169). */
int svla_linear_wide_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                          const float* bias_f32, const void* res, int ldr, void* c, int ldc, int m,
                          int n, int k, float alpha, int act, int layout, svla_stream_t stream);

/* Row-major [rows, k] (leading dimension ldx) -> slab-blocked [k/32][rows][32]
 * (for weights and inputs of svla_linear_wide_bf16).  k % 32 == 0. */
int svla_slab_block_bf16(const void* x, int ldx, void* out, int rows, int k, svla_stream_t stream);

/* Tuning hook: force the GEMM tile configuration for every later call
 * (0: 256x256/32x32-MFMA, 1: 128x128/32x32, 2: 64x128/16x16, 3: 64x64/16x16,
 * 4: skinny 64x64, 5: skinny 64x32, 6: 128x128/16x16, 7: 128x128 4-stage LDS-DMA
 * pipeline, 8: 256x256 5-stage LDS-DMA pipeline with 128x128 wave tiles, 9: 64x64
 * 4-stage LDS-DMA pipeline, 10: 128x64 and 11: 64x128 4-stage LDS-DMA pipelines, 12: skinny
 * 64x16, 13: 128x128, 14: 128x64, 15: 64x128 and 16: 64x64 2-stage line-DMA pipelines
 * (64-wide K stages fetched as whole cache lines), 17: 32x32, 18: 32x64 and 19: 96x96
 * 4-stage line-DMA pipelines with K split over the waves), or -1 for the automatic
 * shape-based choice (default).  A forced tile that cannot serve a problem (too
 * short a K for a pipelined tile, a paired RoPE / SiLU epilogue on a tile
 * without one, anything but a plain dense store on the 256x256 pipeline) is
 * replaced by the nearest tile that can, unless SVLA_TILE_STRICT is or-ed in:
 * then such calls return SVLA_EINVAL and launch nothing.  Process-wide; not
 * thread-safe. */
#define SVLA_TILE_STRICT 0x100
int svla_gemm_set_tile(int tile);

/* Query: the tile configuration (numbering of svla_gemm_set_tile) that
 * svla_linear_bf16 picks for a dense, un-normalised, packed (ldc = n) problem
 * of this shape, or SVLA_EINVAL.  For reports and tests. */
int svla_gemm_tile_choice(int m, int n, int k, int act);

/* Tuning hook: force the number of cross-workgroup K splits of skinny
 * (M <= 256) GEMMs, 1..64 (1 = never split), or -1 for the automatic choice
 * (default).  Process-wide; not thread-safe. */
int svla_gemm_set_split(int splits);

/* Fused (RMSNorm +) QKV projection with rotate-half RoPE in the epilogue.
 * Columns [0, rope_cols) are heads of 64 that get RoPE at position
 * (row % seq_len) with fp32 tables cos/sin [seq_len, 32]; the remaining columns
 * (V) are stored as projected.  Replaces rmsnorm + gemm_q/gemm_kv +
 * rope_apply_packed (vla/text_encoder_bf16.py:422-475, 486-500; kernels
 * cc/float/rope_vec_ops.cc, sine.cc, cosine.cc).  n % 64 == 0, rope_cols % 64 == 0. */
int svla_linear_rope_bf16(const void* a, int lda, const void* w, int ldw, void* c, int ldc,
                          int m, int n, int k, int rope_cols, int seq_len, const float* cos_t,
                          const float* sin_t, const void* norm_w, float norm_eps,
                          svla_stream_t stream);

/* svla_linear_rope_bf16 that also writes, for every rotated column, the bf16
 * remainder c_lo = o - bf16(o) of the fp32 RoPE output o (c_lo: same ldc and
 * row layout as c; columns past rope_cols are not written; NULL: none).  The
 * reference module keeps Q and K in fp32 after RoPE and scores them in fp32
 * (vla/text_encoder_bf16.py:92-104, 117-122); bf16 hi + lo carries o to about
 * 16 bits for svla_attention_lo_bf16. */
int svla_linear_rope_lo_bf16(const void* a, int lda, const void* w, int ldw, void* c,
                             void* c_lo, int ldc, int m, int n, int k, int rope_cols, int seq_len,
                             const float* cos_t, const float* sin_t, const void* norm_w,
                             float norm_eps, svla_stream_t stream);

/* Gated MLP up-projection: out[M, inter] = bf16(silu(gate)) * bf16(up) (bf16),
 * gate/up from one GEMM over the weight interleaved by svla_pack_gate_up_bf16
 * (optionally on RMS-normalised A).  Replaces rmsnorm + gemm_ffn_up x2 +
 * silu_*_bf16 + the numpy hadamard (vla/text_encoder_bf16.py:534-581;
 * vla/action_expert_bf16.py:629-642).  inter % 32 == 0. */
int svla_linear_silu_mul_bf16(const void* a, int lda, const void* w_gu, int ldw, void* out,
                              int ldo, int m, int inter, int k, const void* norm_w,
                              float norm_eps, svla_stream_t stream);

/* Patch embedding: Conv2d(C -> E, kernel = stride = P) as an im2col GEMM over
 * images [n_img, C, H, H] bf16, + conv bias, + learned position embedding
 * pos[(H/P)^2, E].  out [n_img*(H/P)^2, E].  w is the conv weight [E, C*P*P].
 * Replaces preprocessing_block/conv2d (vla/preprocessing_bf16.py:86-109;
 * cc/bf16_old/conv_bf16.cc:12) + the position add (vla/vit_emb.py:43-47). */
int svla_patch_embed_bf16(const void* images, const void* w, const void* bias, const void* pos,
                          void* out, int ldo, int n_img, int chans, int image, int patch,
                          int embed, svla_stream_t stream);

/* Pixel-shuffle connector: out = pixel_shuffle(x, scale) . W^T with the shuffle
 * folded into the A-operand addressing.  x [n_img, grid*grid, hidden]; the
 * n_img*(grid/scale)^2 output rows are written with leading dim ldo, row m at
 * (m / rows_per_sample) * sample_stride + m % rows_per_sample when
 * rows_per_sample > 0 (e.g. 3 cameras x 64 tokens into each sample's 241-row
 * prefix), contiguously when rows_per_sample == 0.  Replaces
 * connector_block/fused_op (vla/connector_bf16.py:97-139; formula
 * vla/vla.py:434-437). */
int svla_connector_bf16(const void* x, const void* w, int ldw, void* out, int ldo, int n_img,
                        int grid, int hidden, int scale, int n_out, int rows_per_sample,
                        int sample_stride, svla_stream_t stream);

/* Action output projection fused with the final expert RMSNorm (norm_w, may
 * be NULL) and the Euler update of the flow-matching loop:
 * v = bf16(norm(A) . W^T); x_f32 += dt * v; x_bf16 = bf16(x_f32) (x_bf16 may be
 * NULL).  Replaces postprocessing's RMSNorm + GEMM (vla/vla.py:218-222) and adds
 * the update the reference lacks. */
int svla_action_out_euler(const void* a, int lda, const void* w, int ldw, float* x_f32,
                          int ldx, void* x_bf16, int ldxb, int m, int n, int k,
                          const void* norm_w, float norm_eps, float dt, svla_stream_t stream);

/* ------------------------------------------------------- fused expert --
 * The whole flow-matching action expert of one chunk -- num_steps Euler steps,
 * each: action_in (Linear A->H + bias), time_in on [action | time] (the time
 * half precomputed per step into time_bias) + SiLU, time_out (+ bias), the
 * n_layers expert layers (self-attention, causal, when layer % 2 == 0, else
 * cross-attention on the projected prefix K/V; RMSNorm -> QKV (+RoPE) ->
 * attention -> O + residual -> RMSNorm -> gate|up + SiLU*up -> down +
 * residual), the final RMSNorm + action_out and x <- x + dt * v -- in ONE
 * persistent launch for small batches (batch * chunk rows; chunk <= 64).
 * Rounding points of the reference torch modules (as on the layer-by-layer
 * path): each RMSNorm output is rounded once, bf16((x * (1/rms)) * gain),
 * before its projection; projections round to bf16; RoPE runs in fp32 on the
 * bf16 projection and the scores take the fp32 result (bf16 hi + lo); the
 * attention softmax is normalised before its probabilities are rounded to
 * bf16; residual adds round to bf16.  Replaces
 * action_expert_self_forward / action_expert_cross_forward
 * (vla/action_expert_bf16.py:662-803) as driven by joint_transformer
 * (vla/vla.py:194-212) and postprocessing (vla/vla.py:218-222), plus the
 * Euler loop, time embedding and action input the reference lacks.
 * Weights are PACKED [out, in] as for svla_linear_bf16; w_gu interleaved by
 * svla_pack_gate_up_bf16; self layers' w_qkv is [q | k | v, hidden], cross
 * layers' w_qkv is Wq [q, hidden] and cross_k / cross_v are the already
 * projected prefix K/V [batch * prefix_len, kv] (leading dimension ld_cross).
 * rope_cos/sin [chunk, 32] (svla_rope_table).  x_in / x_out: fp32
 * [batch * chunk, action_dim] Euler state before / after (may alias). */
typedef struct svla_expert_layer {
  int cross;
  const void* w_qkv;
  const void* w_o;
  const void* w_gu;
  const void* w_down;
  const void* norm1;
  const void* norm2;
  const void* cross_k;
  const void* cross_v;
} svla_expert_layer;

typedef struct svla_expert_desc {
  int batch, chunk, hidden, n_q_heads, n_kv_heads, head_dim, inter, action_dim, n_layers,
      prefix_len, num_steps, ld_cross;
  float rms_eps, dt;
  const void* w_action_in; /* [hidden, action_dim] */
  const void* b_action_in; /* [hidden] */
  const void* w_time_in_a; /* [hidden, hidden]: the action half of time_in */
  const float* time_bias;  /* [num_steps, hidden] fp32: temb(t_s) . W_time_in[time half] + b */
  const void* w_time_out;  /* [hidden, hidden] */
  const void* b_time_out;  /* [hidden] */
  const void* norm_out;    /* [hidden] final RMSNorm gain */
  const void* w_action_out; /* [action_dim, hidden] */
  const float* rope_cos;
  const float* rope_sin;
  const float* x_in;
  float* x_out;
  const svla_expert_layer* layers; /* host array of n_layers */
} svla_expert_desc;

/* What svla_expert_run needs (filled by svla_expert_prepare; host memory). */
typedef struct svla_expert_plan {
  void* phases;
  int n_phases;
  unsigned* counters;
  long counter_words;
  unsigned* status;
  int grid;
  int team_xcd;
  int team_size;
  int spin_limit; /* polls before a wait gives up (svla_expert_prepare: 1 << 22,
                     about seconds); a caller may lower it, e.g. to exercise
                     the failure path: status 1 and NaN actions, every
                     workgroup still exits */
  unsigned long long* stamps; /* optional (prepare: NULL), device memory of
                     2 * n_phases counters: the first workgroup of the team
                     records the GPU's constant 100 MHz clock
                     (s_memrealtime) when phase p starts (its wait done) at
                     stamps[2p] and after its own arrival at stamps[2p + 1]
                     -- the per-phase timing of a run */
} svla_expert_plan;

/* Device workspace bytes svla_expert_prepare needs for d (phase table,
 * arrival counters, and one buffer per intermediate activation of the whole
 * chunk: about 9.4 MB per Euler step at batch 1), or 0 if d is invalid
 * (chunk > 64, head_dim != 64, hidden / inter / q width > 2048, prefix_len >
 * 256, a NULL pointer). */
long svla_expert_workspace_size(const svla_expert_desc* d);

/* Lays out the workspace (device, 256-byte aligned, ws_bytes >= the size
 * above), uploads the phase table (synchronous on `stream`) and fills
 * *plan.  team_xcd < 0: every CU takes part; 0..7: only the CUs of that XCD
 * (a performance choice: results are the same).  The pointers in d are
 * captured: later runs use them. */
int svla_expert_prepare(const svla_expert_desc* d, void* ws, long ws_bytes, int team_xcd,
                        svla_expert_plan* plan, svla_stream_t stream);

/* One chunk's expert: clears the arrival counters (a small kernel) and
 * launches the persistent kernel (one workgroup per CU) on `stream`;
 * graph-capturable.  Every wait inside is bounded: a launch that cannot
 * finish (workgroups not co-resident) gives up and sets the status word. */
int svla_expert_run(const svla_expert_plan* plan, svla_stream_t stream);

/* Status word of the last run (synchronous copy): 0 ok, 1 a wait gave up,
 * 2 the XCD team could not form.  A run that gave up also fills x_out with
 * NaN, so a caller that replays a graph without reading the status still
 * sees the failure. */
int svla_expert_status(const svla_expert_plan* plan, int* status);

/* Byte offset, inside the workspace laid out for d, of the activation that
 * enters expert layer `layer` (0..n_layers-1) at Euler step `step`;
 * layer == n_layers: the last layer's output (the input of the final norm
 * and action projection).  Each such buffer is written once per run and
 * keeps its value until the next run, so a caller can read every layer's
 * output of every step back after svla_expert_run -- the per-layer check of
 * the reference's layer tests (vla/action_expert_bf16.py:848-906).  Layout:
 * fragment-major bf16 [64 rows][hidden]: element (m, k) at
 * ((((k/32)*4 + m/16)*64 + m%16 + 16*((k/8)%4))*8 + k%8).  -1 if d, step or
 * layer is invalid. */
long svla_expert_trace_offset(const svla_expert_desc* d, int step, int layer);

/* ------------------------------------------------------------ attention --
 * Fused GQA attention: O = softmax(scale * Q K^T + mask) V per head, query
 * head h reading KV head h*hkv/hq.  Scores and softmax statistics fp32,
 * probabilities bf16 into the P.V MFMA, fp32 accumulate, bf16 out.
 * Q row r of batch b at q + b*q_bs + r*ldq + h*64 (same scheme for k, v, o).
 * head_dim must be 64.  mask: SVLA_MASK_NONE / CAUSAL / PREFIX_LM (keys
 * < prefix_len visible to all rows, later keys causal).
 * Replaces the per-head score GEMMs, masked_softmax_128_bf16 / softmax_bf16_* /
 * softmax_float32_seq1024 and the P.V GEMMs (vla/text_encoder_bf16.py:502-526;
 * vla/vision_block_bf16.py:325-367; vla/action_expert_bf16.py:689-713, 764-787). */
int svla_attention_bf16(const void* q, int ldq, long q_bs, const void* k, int ldk, long k_bs,
                        const void* v, int ldv, long v_bs, void* o, int ldo, long o_bs,
                        int batch, int sq, int sk, int hq, int hkv, int head_dim, float scale,
                        int mask_kind, int prefix_len, svla_stream_t stream);

/* svla_attention_bf16 with fp32-accurate scores for RoPE'd Q and K: q_lo /
 * k_lo (nullable; k_lo only with q_lo) are the bf16 remainders written by
 * svla_linear_rope_lo_bf16, with the strides of q / k; the scores are then
 * K . Q^T for Q = q + q_lo, K = k + k_lo (the k_lo . q_lo term, below 2^-16
 * relative, is dropped), as the reference module scores its fp32 post-RoPE
 * Q and K (vla/text_encoder_bf16.py:117-122; vla/action_expert_bf16.py:
 * 119-125, 194-199: Q only in cross layers, whose K is a plain projection). */
int svla_attention_lo_bf16(const void* q, const void* q_lo, int ldq, long q_bs, const void* k,
                           const void* k_lo, int ldk, long k_bs, const void* v, int ldv,
                           long v_bs, void* o, int ldo, long o_bs, int batch, int sq, int sk,
                           int hq, int hkv, int head_dim, float scale, int mask_kind,
                           int prefix_len, svla_stream_t stream);

/* -------------------------------------------------- per-kernel harness --
 * Standalone kernels matching the reference's per-kernel test harness. */

/* masked_softmax_128_bf16(bf16[R][C], int row_start, bf16[R][C])
 * (cc/bf16/masked_softmax_128_bf16.cc:251): causal mask at global row
 * row_start + r, fp32 softmax, bf16 out.  row_start is a HOST int. */
int svla_masked_softmax_bf16(const void* s, int row_start, void* p, int rows, int cols,
                             svla_stream_t stream);

/* Row softmax, input bf16 (in_f32 = 0) or fp32 (in_f32 = 1), output bf16
 * (out_f32 = 0) or fp32.  softmax_bf16_* (cc/bf16_old/v2_softmax_bf16.cc:552-663,
 * v1_softmax_bf16.cc:159) and softmax_float32_seq1024 (cc/float/v1_softmax_float.cc:117). */
int svla_softmax(const void* s, void* p, int rows, int cols, int in_f32, int out_f32,
                 svla_stream_t stream);

/* SiLU y = x * sigmoid(x) on n bf16 values (silu_{128,160,256}_bf16,
 * cc/bf16/silu_160_bf16.cc:124; silu_bf16 cc/bf16_old/silu_bf16.cc:192). */
int svla_silu_bf16(const void* x, void* y, long n, svla_stream_t stream);

/* GELU (kind = SVLA_ACT_GELU_TANH or SVLA_ACT_GELU_ERF) on n bf16 values
 * (gelu_bf16, cc/bf16_old/gelu_bf16.cc:83). */
int svla_gelu_bf16(const void* x, void* y, long n, int kind, svla_stream_t stream);

/* out = bf16(silu(gate)) * up (bf16), n values (the numpy hadamard step,
 * vla/text_encoder_bf16.py:581). */
int svla_silu_mul_bf16(const void* gate, const void* up, void* out, long n,
                       svla_stream_t stream);

/* RoPE on x [rows, heads*64] (leading dim ldx) at positions pos_offset+row,
 * fp32 tables [>= pos_offset+rows, 32].  in_f32/out_f32 select fp32 or bf16
 * storage.  rope_fused_float32 (cc/float/rope_fused.cc:17) and
 * rope_apply_packed (vla/text_encoder_bf16.py:422-475). */
int svla_rope(const void* x, int ldx, void* y, int ldy, int rows, int heads,
              const float* cos_t, const float* sin_t, int pos_offset, int in_f32, int out_f32,
              svla_stream_t stream);

/* ---------------------------------------------------------- utilities -- */

/* RoPE tables: cos/sin[pos][k] of pos / theta^(2k/head_dim), fp32,
 * pos < max_pos, k < head_dim/2 (apply_rope, vla/text_encoder_bf16.py:80-97). */
int svla_rope_table(float* cos_t, float* sin_t, int max_pos, int head_dim, float theta,
                    svla_stream_t stream);

/* Transpose-pack a reference [K, N] (in x out) bf16 weight to [N, K]. */
int svla_pack_weight_bf16(const void* w_kn, int ldw, void* out_nk, int k, int n,
                          svla_stream_t stream);

/* Interleave gate/up weights ([K, inter] each, reference layout) into the
 * [2*inter, K] layout consumed by svla_linear_silu_mul_bf16 (blocks of 32 rows
 * alternating gate/up).  inter % 32 == 0. */
int svla_pack_gate_up_bf16(const void* w_gate, const void* w_up, void* out, int k, int inter,
                           svla_stream_t stream);

/* Language embedding: out[r] = bf16(table[ids[r]] * scale) for r < n_tokens;
 * ids are int64 (an id outside [0, vocab) yields a zero row).  Row r goes to
 * out + (r / per_sample)*out_bs + (r % per_sample)*ldo
 * (create_text_emb, vla/vla.py:169-174). */
int svla_embed_bf16(const int64_t* ids, const void* table, long vocab, int hidden, float scale,
                    void* out, int ldo, long out_bs, long n_tokens, int per_sample,
                    svla_stream_t stream);

/* Sinusoidal flow-matching time embedding of the HOST scalar t, computed in
 * fp64 and rounded to bf16: [sin(2 pi t / p_j) | cos(2 pi t / p_j)], p_j
 * geometric from min_period to max_period, out [dim] bf16. */
int svla_time_embedding_bf16(double t, int dim, double min_period, double max_period, void* out,
                             svla_stream_t stream);

/* fp32 -> bf16 conversion (round to nearest even), n values. */
int svla_f32_to_bf16(const float* x, void* y, long n, svla_stream_t stream);

/* ------------------------------------------------------- pre-processing --
 * Camera frames -> vision-encoder input: n uint8 RGB frames [h, w, 3]
 * (HWC, frame stride src_bs bytes, host value h, w) resized with the aspect
 * ratio kept to round((h, w) * min(S/h, S/w)) by bilinear interpolation
 * (half-pixel centres, as torch interpolate(mode="bilinear",
 * align_corners=False)), placed top-left in an S x S canvas padded with black,
 * then mapped to [-1, 1] (x / 255 * 2 - 1) as bf16 [n, 3, S, S] (S = out_size).
 * The "resize/normalize to [-1, 1]" step in front of the patch embedding; the
 * reference feeds random images straight in (vla/vla.py:306, 396-408). */
int svla_image_to_bf16(const uint8_t* src, long src_bs, int n, int h, int w, void* dst,
                       int out_size, svla_stream_t stream);

/* ------------------------------------------------------ harness kernels --
 * The remaining per-kernel harness entry points, fp32 and bf16 variants
 * (computed in fp32; bf16 results rounded where the matching torch reference
 * rounds). */

/* y = op(x) elementwise on n fp32 / bf16 values (op = SVLA_OP_*).  Replaces
 * silu_float32 (cc/float/silu.cc), gelu (cc/float/gelu.cc,
 * cc/bf16_new/gelu_bf16.cc), silu_bf16 / silu_bf16_small (cc/bf16_new/silu_bf16.cc),
 * silu_{128,160}_float32 (cc/float/silu_128.cc, silu_160.cc), sin_float32 /
 * cos_float32 (cc/float/sine.cc:64, cosine.cc:66) and sin_bfloat16 /
 * cos_bfloat16 (cc/bf16_new/sine_bf16.cc, cosine_bf16.cc). */
int svla_unary_f32(const float* x, float* y, long n, int op, svla_stream_t stream);
int svla_unary_bf16(const void* x, void* y, long n, int op, svla_stream_t stream);

/* out = x + y on n bf16 values.  Replaces add (cc/bf16_old/add_32_32_bf16.cc). */
int svla_add_bf16(const void* x, const void* y, void* out, long n, svla_stream_t stream);

/* Row norms with fp32 (is_f32 = 1: x, w, b, y all fp32) or bf16 I/O, kind =
 * SVLA_NORM_*; b (LayerNorm only) may be NULL.  round_ops (bf16): round after
 * every step a torch bf16 op chain rounds (the "new" harness references);
 * otherwise round once.  cols <= 2048.  Replaces rms_norm (cc/float/rms_norm.cc,
 * cc/bf16_new/rms_norm_bf16.cc), rms_norm_small, rms_norm_960 (cc/float/rms_norm_960.cc),
 * layer_norm (cc/float/layer_norm.cc, cc/bf16_new/layer_norm_bf16.cc) and
 * layer_norm_small. */
int svla_row_norm(const void* x, int ldx, const void* w, const void* b, void* y, int ldy, int rows,
                  int cols, float eps, int kind, int is_f32, int round_ops,
                  svla_stream_t stream);

/* Row softmax over cols, rows with strides lds / ldp; row_start >= 0 masks key
 * c of row r when c > row_start + r / row_div (row_div > 1: several heads of
 * one query row stored consecutively).  Replaces masked_softmax_float32
 * (cc/float/masked_softmax.cc:72-127) and masked_softmax_128_float32
 * (cc/float/masked_softmax_128.cc). */
int svla_softmax_rows(const void* s, int lds, void* p, int ldp, int rows, int cols, int row_start,
                      int row_div, int in_f32, int out_f32, svla_stream_t stream);

/* fp32 Conv2d with kernel = stride = patch and no padding: images [n, C, H, W],
 * kernel [E, C, patch, patch], bias [E] or NULL -> out [n * (H/patch) * (W/patch), E]
 * (patches in row-major grid order).  Replaces conv (cc/float/conv.cc:12-55). */
int svla_conv_patch_f32(const float* images, const float* kernel, const float* bias, float* out,
                        int n_img, int chans, int height, int width, int patch, int embed,
                        svla_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SVLA_H */
