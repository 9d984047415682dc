// Fused action expert for small batches: every Euler step of the
// flow-matching loop -- action / time embedding, the 16 expert layers
// (self- and cross-attention alternating), the output head and the Euler
// update -- in ONE persistent launch.
//
// Replaces, at batch 1, the ~840 launches of the layer-by-layer path
// (vla/action_expert_bf16.py:662-803 per layer, the joint_transformer
// interleave vla/vla.py:194-212, postprocessing vla/vla.py:218-222, plus the
// flow-matching loop the reference lacks).  Each launch there costs ~4 us of
// dispatch and drain on top of a few microseconds of work spread over a
// small corner of the chip; here the work is a fixed list of PHASES (one per
// GEMM or attention of the step sequence) that every workgroup walks.
//
// Design (CDNA4; the figures are MI355X measurements of this build):
//  * One workgroup of 8 waves per CU.  A phase is split into UNITS (a
//    64-row x 16-column output tile of a GEMM, one (sample, head) of an
//    attention); unit u of a phase runs on team rank u % team_size.
//  * Phases hand over through device-scope arrival counters: a workgroup
//    that finished its units of phase p waits for its stores to be
//    acknowledged (vmcnt = 0), then adds its unit count to one of 8
//    sub-counters of phase p (spread so that 256 arrivals do not queue on
//    one address: a grid barrier measured 4.0 us with one counter, 2.0 us
//    with 8); a workgroup with units in phase p + 1 polls the 8
//    sub-counters (with the status word, one round trip per poll) until they
//    sum to phase p's unit count.  Completion of phase p implies completion
//    of every earlier phase (each of its units waited for p - 1), so one
//    wait per phase suffices.
//  * Every phase writes its output to a buffer that no other phase of the
//    launch writes (activation versions, not in-place updates), 256-byte
//    aligned, with write-through (agent-scope) stores.  No cache can then
//    hold a stale copy of data a phase reads: nobody reads an address before
//    the phase that writes it has completed, so the first read of a line by
//    an XCD misses its L2 and later reads by that XCD's CUs hit the fresh
//    line.  Activations are read with plain loads (L2-cached broadcast).
//  * Latency, not bandwidth, sets the time of a phase at these sizes
//    (per-phase timestamps: ~1.2 us hand-off, ~2-3 us for the activation
//    loads, the rest epilogue and bookkeeping), so everything that does not
//    depend on the previous phase is issued before or beside its wait: the
//    weights of a workgroup's first unit before the wait, the epilogue
//    operands (residual, bias, RoPE tables, Euler state) together with the
//    activations, the next phase's header during the current phase.
//  * GEMM units: the 8 waves split K (one pass for K <= 2048); each wave
//    holds its k-range of the 64 activation rows in registers and streams
//    its 16x16x32 MFMA weight fragments into a private LDS region by LDS-DMA
//    (no registers held while they fly); the partial tiles meet in LDS.
//    The RMSNorm in front of a projection is fused: the row sums of squares
//    come from the activation fragments and meet in LDS, then every wave
//    turns its fragments into bf16(x * (1/rms) * gain) before the MFMAs --
//    the single rounding of torch's bf16 RMSNorm, so each layer output
//    follows the reference module's rounding points.  Paired epilogues
//    (RoPE pairs (d, d+32), SiLU(gate) * up) use the 16-column tile of 8
//    columns + their partners.  The V columns of a
//    self layer's QKV projection are written transposed (V^T [kv][64 keys])
//    for the attention.
//  * Attention units: one (sample, head); K, V^T and the queries are staged
//    into LDS once per CU (cross layers: K and V^T before the phase wait),
//    then the 8 waves take 4 key quarters of 64 keys x 2 query groups.  Scores are fp32; the softmax is exact (the
//    maxima and sums of the key groups meet in LDS) and the probabilities
//    are rounded to bf16 before P.V, as the reference torch module does
//    (vla/text_encoder_bf16.py:117-126).  The P.V operand is V^T straight
//    from global memory (the cross layers' V is transposed by the launch's
//    first phase).
//  * Every wait is bounded: past the plan's spin limit (kSpin polls unless
//    the caller lowers it) or when another workgroup has already given up,
//    the workgroup sets the status word, fills the action output with NaN
//    and leaves, so the grid always drains and a failed chunk is loud.  The team is either every workgroup of the launch
//    or, optionally, the workgroups of one XCD (selected by the hardware
//    XCC_ID register); the write-through / write-once discipline keeps the
//    results correct whichever CUs take part.
#include <cstring>
#include <vector>

#include "svla_common.h"

namespace {

constexpr int XW = 8;              // waves per workgroup
constexpr int XT = XW * 64;        // threads per workgroup
constexpr int XKS = 64 / XW;       // 32-deep k-steps per wave: K <= XW * XKS * 32 = 2048
constexpr int XBM = 64;            // rows per GEMM unit (4 MFMA row tiles) = max batch * chunk
constexpr int XBN = 16;            // columns per GEMM unit
constexpr int XPS = XBN + 4;       // padded LDS row of a partial tile (floats)
constexpr int XMAXK = 256;         // attention: keys per sample
constexpr int XKW = 64;            // attention: keys of the one-wave-per-query-tile path
constexpr int XKG = XMAXK / XW;    // attention: keys per wave of the split path (32)
constexpr int XVTS = 64;           // self-attention V^T: keys per sample (leading dimension)
constexpr int kMaxCross = 16;      // cross layers (V^T transposes in the first phase)
constexpr int kSub = 8;            // sub-counters per phase
constexpr int kCntStride = 32;     // unsigned per sub-counter (128 bytes apart)
constexpr int kSpin = 1 << 22;     // polls before a wait gives up

enum XKind { XK_GEMM = 0, XK_ATTN = 1, XK_VT = 2 };
enum XEpi { XE_STORE = 0, XE_ROPE = 1, XE_SILU = 2, XE_EULER = 3 };
enum XStat { XS_OK = 0, XS_TIMEOUT = 1, XS_TEAM = 2 };

struct XPhase {
  int kind, epi, act, a_f32;
  int M, N, K, units, col_tiles;
  int row_groups, group_tiles;  // GEMM unit = (column tile, group of row tiles)
  // GEMM: C[M, N] = epilogue(norm(A)[M, K] . W[N, K]^T)
  const void* a;
  int lda;
  const bf16* w;
  int ldw;
  const bf16* bias;
  const float* bias_f32;
  const bf16* res;
  int ldr;
  void* c;
  int ldc;
  const bf16* norm_w;
  float norm_eps;
  const float* cos_t;
  const float* sin_t;
  int rope_cols, rope_period;
  bf16* vt;     // ROPE: columns >= rope_cols go here transposed, [sample][col][XVTS]
  bf16* c_lo;   // ROPE: the bf16 remainder o - bf16(o) of every rotated column (same layout as c)
  int chunk;    // rows per sample (ROPE V^T, attention queries)
  const float* x_in;  // Euler: x_out[m, n] = x_in[m, n] + dt * bf16(v) (fp32, leading dim N)
  float* x_out;
  float dt;
  // attention: unit = sample * heads + head; V given transposed
  const bf16* q;
  const bf16* q_lo;  // remainder of the fp32 RoPE output: Q = q + q_lo to ~16 bits
  const bf16* k_lo;  // the same for K (self layers; null: K is plain bf16)
  const bf16* k;
  const bf16* vt_in;
  bf16* o;
  int ldq, ldk, ldvt, ldo;
  long q_bs, k_bs, vt_bs, o_bs;
  int heads, kv_heads, lk, causal;
  int q_tiles;    // units per (sample, head): 16-query tiles, or 1 (every key in one wave)
  int kv_static;  // K and V^T were written before the previous phase (cross layers)
  float scale;
  // V^T transposes (first phase): unit = (layer, sample, 64-column block)
  int n_vt, vt_blocks, vt_ldv, vt_keys;
  long vt_src_bs, vt_dst_bs;
  const bf16* vt_src[kMaxCross];
  bf16* vt_dst[kMaxCross];
};

// The phase table does not change while the kernel runs: reading it through
// the constant address space lets uniform field reads become scalar loads
// (cached in the scalar cache) instead of one vector round trip each.
typedef const __attribute__((address_space(4))) XPhase CPhase;

struct XArgs {
  CPhase* ph;
  int n_ph;
  unsigned* cnt;     // [n_ph + 1][kSub][kCntStride]; the last row is the team registration
  unsigned* status;  // XStat of the launch (0 = ok)
  int team_xcd;      // < 0: every workgroup; else the workgroups on this XCD
  int team_size;     // participants expected when team_xcd >= 0
  int spin;          // polls before a wait gives up
  unsigned long long* stamps;  // optional per-phase clock stamps (team rank 0)
};

// Loads through pointers read from the phase table: tell the compiler they
// are global (flat loads would also count on lgkmcnt and force full waits).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef const __attribute__((address_space(1))) bf16x8* gbf8p;
typedef const __attribute__((address_space(1))) f32x4* gf4p;
typedef const __attribute__((address_space(1))) bf16x4* gbf4p;
typedef const __attribute__((address_space(1))) uint64_t* gu64cp;
typedef const __attribute__((address_space(1))) uint16_t* gu16cp;
__device__ __forceinline__ bf16x8 ldg8(const bf16* p) { return *(gbf8p)(p); }
__device__ __forceinline__ bf16x4 ldg4(const bf16* p) { return *(gbf4p)(p); }
__device__ __forceinline__ f32x4 ldgf4(const float* p) { return *(gf4p)(p); }
__device__ __forceinline__ uint64_t ldg64(const bf16* p) { return *(gu64cp)(p); }
__device__ __forceinline__ uint16_t ldg16(const bf16* p) { return *(gu16cp)(p); }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
// The thread index through an opaque copy: lane-derived values are then
// computed where they are used instead of being hoisted out of the phase loop
// (the kernel runs at the VGPR limit, hoisted values were spilled, and a
// spill reload is a memory load that returns in order behind the loads
// already issued -- the first poll of a phase, for one, waited for the wave's
// weight requests).
__device__ __forceinline__ int tidx() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// gfx9 s_waitcnt immediate: vmcnt split over bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8; the counters not named are left unconstrained
constexpr int wc_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int wc_lgkm0 = 15 | (3 << 14) | (7 << 4);

// LDS written by this wave visible to the whole workgroup, this wave's LDS
// reads complete (global memory operations in flight are not waited for)
__device__ __forceinline__ void wg_sync_lds() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(wc_lgkm0);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// 8 bytes stored write-through (agent-scope relaxed atomic store, global)
typedef __attribute__((address_space(1))) uint64_t* gu64p;
__device__ __forceinline__ void st8_wt(void* p, uint64_t v) {
  __hip_atomic_store((gu64p)(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t pack4(const float v[4]) {
  bf16x4 o;
  o[0] = f2bf(v[0]); o[1] = f2bf(v[1]); o[2] = f2bf(v[2]); o[3] = f2bf(v[3]);
  return __builtin_bit_cast(uint64_t, o);
}
__device__ __forceinline__ void st4_wt(bf16* p, const float v[4]) { st8_wt(p, pack4(v)); }
__device__ __forceinline__ void st2f_wt(float* p, float a, float b) {
  st8_wt(p, __builtin_bit_cast(uint64_t, u32x2{__builtin_bit_cast(uint32_t, a),
                                               __builtin_bit_cast(uint32_t, b)}));
}

// Wave 0 polls the 8 sub-counters of `row` (lanes 0..7) and the status word
// (lane 8) together until the counters sum to `target`; false when the wait
// gave up (status set).
__device__ bool wait_phase(const XArgs& g, int row, unsigned target) {
  const int lane = tidx() & 63;
  const unsigned* c = lane < kSub ? g.cnt + ((size_t)row * kSub + lane) * kCntStride : g.status;
  for (int n = 0;; ++n) {
    const unsigned v = lane <= kSub ? ld_agent(c) : 0u;
    unsigned s = lane < kSub ? v : 0u;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    const unsigned st = __shfl(v, kSub, 64);
    if (__builtin_amdgcn_readfirstlane(s) >= target) return true;
    if (__builtin_amdgcn_readfirstlane(st) != 0u) return false;
    if (n >= g.spin) {
      if (lane == 0)
        __hip_atomic_store(g.status, (unsigned)XS_TIMEOUT, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

// ---- GEMM units ---------------------------------------------------------------
struct GemmRegs {
  bf16x8 fx[XKS][4];  // activations: this wave's k-steps x 4 row tiles
  float ss[4];        // norm: this lane's row sums of squares (rows tm*16 + fr)
};

// LDS image of one wave's weight fragments: k-step j of the unit's 16 rows,
// 64 bytes per row, 16-byte chunk c of row r at slot c ^ ((r >> 1) & 3)
// (the 16 rows of a fragment read then spread over the banks)
constexpr int XWSTEP = 16 * 32;  // bf16 per k-step
__device__ __forceinline__ int wswz(int r, int c) { return c ^ ((r >> 1) & 3); }
typedef __attribute__((address_space(3))) bf16* lds_bf16p;

// bf16 activations passed between GEMM phases (GEMM inputs, residuals and
// the attention output) are stored fragment-major: the 16-row x 32-k
// B-operand fragment of (k-step k / 32, row tile m / 16) is one contiguous,
// lane-ordered 1 KB block (lane = m % 16 + 16 ((k / 8) % 4), 8 k per lane).
// A fragment load is then 8 whole cache lines; a row-major fragment touches
// 16 half-used lines, and a CU's L1 serves misses at a per-line rate (about
// half the bytes per second).  64 rows (the row limit of this kernel), so a
// K-column activation takes ceil(K / 32) * 4 KB.
__device__ __forceinline__ unsigned frag_off(int m, int k) {
  return ((((unsigned)k >> 5) * 4u + ((unsigned)m >> 4)) * 64u + (unsigned)(m & 15) +
          16u * (((unsigned)k >> 3) & 3u)) * 8u + ((unsigned)k & 7u);
}

// epilogue operands, loaded with the activations
struct EpiPre {
  f32x4 u, w;      // fp32 bias | RoPE cos, sin | Euler x
  bf16x4 b, r;     // bf16 bias, residual
};

__device__ __forceinline__ bool paired(int epi) { return epi == XE_ROPE || epi == XE_SILU; }

// first packed column of unit column tile ct (16-column tile; a paired tile
// holds 8 columns of a first half and their 8 partners 32 columns on)
__device__ __forceinline__ int tile_base(int epi, int ct) {
  const int n0 = ct * XBN;
  return paired(epi) ? (n0 >> 6) * 64 + ((n0 & 63) >> 4) * 8 : n0;
}

// This wave's k-steps: [ks0, ks0 + kcnt) of the ceil(K / 32) steps.
__device__ __forceinline__ void wave_krange(int K, int wave, int& ks0, int& kcnt) {
  const int nks = (K + 31) / 32;
  const int per = (nks + XW - 1) / XW;
  ks0 = wave * per;
  kcnt = max(0, min(per, nks - ks0));
}

// Weight fragments of column tile ct for this wave's k-steps, streamed into
// the wave's own LDS region by LDS-DMA (no registers held while they fly;
// only this wave reads them, after its own vmcnt wait).  Lane l fetches row
// l / 4 (through the paired-tile row map), chunk wswz(row, l % 4).  Only the
// wave's own k-steps are requested: a CU holds a bounded number of misses in
// flight, and repeated requests of one line use them up.  Chunks past K hold
// other weights: the activations there are zero.
__device__ __forceinline__ void dma_w(int epi, const bf16* W, int N, int K, int ldw, int ct,
                                      bf16* sw) {
  const int lane = tidx() & 63;
  const int wave = wave_id();
  int ks0, kcnt;
  wave_krange(K, wave, ks0, kcnt);
  const int base = tile_base(epi, ct);
  const int r = lane >> 2;
  const int row = paired(epi) ? base + (r & 7) + (r >> 3) * 32 : min(base + r, N - 1);
  const int c8 = wswz(r, lane & 3) * 8;
  const bf16* src = W + (long)row * ldw;
#pragma unroll
  for (int j = 0; j < XKS; ++j) {
    if (j >= kcnt) break;  // wave-uniform
    __builtin_amdgcn_global_load_lds((void*)(src + min((ks0 + j) * 32 + c8, K - 8)),
                                     (lds_ptr_t)(sw + j * XWSTEP), 16, 0, 0);
  }
}

// Norm gains of this wave's k range (at most XKS * 32 = 256 of them) into
// the wave's gain row: one DMA instruction, issued before the phase wait.
__device__ __forceinline__ void dma_gain(const bf16* norm_w, int K, bf16* gain) {
  const int lane = tidx() & 63, wave = wave_id();
  int ks0, kcnt;
  wave_krange(K, wave, ks0, kcnt);
  if (kcnt == 0) return;  // wave-uniform
  __builtin_amdgcn_global_load_lds((void*)(norm_w + min(ks0 * 32 + lane * 8, K - 8)),
                                   (lds_ptr_t)gain, 16, 0, 0);
}

// Activation fragments (rows 0..63, clamped to M - 1) of this wave's k-steps
// (only those: steps past the range are never requested); k past K reads as
// zero.
__device__ __forceinline__ void load_x(CPhase& P, GemmRegs& r, int t0, int t1) {
  const int lane = tidx() & 63;
  const int wave = wave_id();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  int ks0, kcnt;
  wave_krange(P.K, wave, ks0, kcnt);
  unsigned rows[4];
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) rows[tm] = (unsigned)min(tm * 16 + fr, P.M - 1);
  if (P.a_f32) {
    // fp32 A (the Euler state into action_in, K <= 32: one k-step, wave 0),
    // rounded to bf16 on the way in (only k-step 0 exists)
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) r.fx[0][tm] = bf16x8{};
    if (kcnt > 0) {
      const int k = ks0 * 32 + fk;
      // every load issued before any use (a use right after its load would
      // make each load a round trip of its own)
      f32x4 lo[4], hi[4];
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        const float* src = static_cast<const float*>(P.a) + (rows[tm] * (unsigned)P.lda + (unsigned)min(k, P.K - 8));
        lo[tm] = ldgf4(src);
        hi[tm] = ldgf4(src + 4);
      }
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        bf16x8 t;
#pragma unroll
        for (int i = 0; i < 4; ++i) { t[i] = f2bf(lo[tm][i]); t[4 + i] = f2bf(hi[tm][i]); }
        r.fx[0][tm] = k < P.K ? t : bf16x8{};
      }
    }
  } else {
    // fragment-major A: one contiguous 1 KB block per (k-step, row tile).
    // Rows past M and k past K are never written (the workspace is cleared
    // at set-up), so they read as zero and the loads need no select: a use
    // right after a load would make every load a round trip of its own.
#pragma unroll
    for (int j = 0; j < XKS; ++j) {
      if (j >= kcnt) break;  // wave-uniform: no request past the wave's range
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        if (tm < t0 || tm >= t1) continue;  // wave-uniform: another unit's rows
        r.fx[j][tm] = ldg8(static_cast<const bf16*>(P.a) + (((unsigned)(ks0 + j) * 4u + tm) * 64u + lane) * 8u);
      }
    }
  }
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) r.ss[tm] = 0.f;
  if (P.norm_w) {
    // per-row sums of squares of the raw activations (norm_x applies
    // 1 / rms and the gains once the waves' sums have met); the activations
    // landed first
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(wc_vm(0));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
#pragma unroll
    for (int j = 0; j < XKS; ++j) {
      if (j >= kcnt) continue;  // wave-uniform
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        if (tm < t0 || tm >= t1) continue;  // wave-uniform
        const bf16x8 x = r.fx[j][tm];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const bf16x2 xp = {x[e], x[e + 1]};
          r.ss[tm] = __builtin_amdgcn_fdot2_f32_bf16(xp, xp, r.ss[tm], false);
        }
      }
    }
  }
}

// Epilogue work item of thread tid in a unit: tile row ml, 4-column group
// gi, first packed column n; `on` false if the thread has none.
struct EpiItem {
  int ml, n, gi;
  bool on;
};

__device__ __forceinline__ bool vt_unit(CPhase& P, int ct) {
  return P.vt && tile_base(P.epi, ct) >= P.rope_cols;
}

__device__ __forceinline__ EpiItem epi_item(CPhase& P, int ct, int t0, int t1) {
  const int tid = tidx();
  EpiItem it{};
  const int base = tile_base(P.epi, ct);
  if (paired(P.epi)) {
    it.ml = tid >> 1;
    it.gi = tid & 1;
    it.on = tid < XBM * 2 && it.ml < P.M;
  } else {
    it.ml = tid >> 2;
    it.gi = tid & 3;
    it.on = tid < XBM * 4 && it.ml < P.M;
  }
  it.n = base + it.gi * 4;
  if (!paired(P.epi) && it.n >= P.N) it.on = false;
  if ((it.ml >> 4) < t0 || (it.ml >> 4) >= t1) it.on = false;  // another unit's rows
  return it;
}

// Operands of the epilogue item (addresses clamped into the tensors, so
// every thread loads; values of threads without an item are ignored).
__device__ __forceinline__ void epi_prefetch(CPhase& P, const EpiItem& it, EpiPre& e) {
  const int m = min(it.ml, P.M - 1);
  const int n = min(it.n, P.N - 4);
  if (P.epi == XE_STORE) {
    if (P.bias) e.b = ldg4(P.bias + n);
    if (P.bias_f32) e.u = ldgf4(P.bias_f32 + n);
    if (P.res) e.r = ldg4(P.res + frag_off(m, n));  // fragment-major
  } else if (P.epi == XE_ROPE) {
    const int pos = m % P.rope_period, d = n & 31;
    e.u = ldgf4(P.cos_t + pos * 32 + d);
    e.w = ldgf4(P.sin_t + pos * 32 + d);
  } else if (P.epi == XE_EULER) {
    e.u = ldgf4(P.x_in + ((unsigned)m * (unsigned)P.N + (unsigned)n));
  }
}

union XShared {
  struct {
    float part[XW][XBM * XPS];  // partial tiles of the waves
    float ss[XW][XBM];          // per-wave row sums of squares
    bf16 gain[XW][512];         // norm gains of each wave's k range (staged)
  } g;
  struct {
    float amax[XW][16];         // [key group][query]
    float asum[XW][16];
    float o[XW][64][16];        // partial O^T [key group][d][query]
    bf16 q[64 * 64];            // staged queries (rows swizzled as K)
    bf16 q_lo[64 * 64];         // their bf16 remainders (when P.q_lo)
  } a;
};

// Fused RMSNorm of a unit's activations, once the per-wave row sums of
// squares are in LDS: every element of the wave's fragments becomes
// bf16((x * (1 / rms)) * gain) in fp32 -- the single rounding of torch's bf16
// RMSNorm (the reference module's nn.RMSNorm, vla/action_expert_bf16.py:74-78),
// with 1 / rms = 1 / sqrt(sum / K + eps) and the waves' sums added in wave
// order.  The gains of the wave's k range were staged in LDS by dma_gain
// (landed: load_x waited for every load of the wave).  Rows past M are zero
// and stay zero.
__device__ __forceinline__ void norm_x(CPhase& P, GemmRegs& r, const XShared& sh, int t0,
                                       int t1) {
  const int lane = tidx() & 63, wave = wave_id();
  const int fr = lane & 15, G = lane >> 4;
  int ks0, kcnt;
  wave_krange(P.K, wave, ks0, kcnt);
  float rs[4];
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < XW; ++w) t += sh.g.ss[w][tm * 16 + fr];
    rs[tm] = 1.0f / sqrtf(t / (float)P.K + P.norm_eps);
  }
  const bf16* gain = sh.g.gain[wave];
#pragma unroll
  for (int j = 0; j < XKS; ++j) {
    if (j >= kcnt) break;  // wave-uniform
    const bf16x8 gv = *reinterpret_cast<const bf16x8*>(gain + j * 32 + G * 8);
#pragma unroll
    for (int tm = 0; tm < 4; ++tm) {
      if (tm < t0 || tm >= t1) continue;  // wave-uniform
      bf16x8 x = r.fx[j][tm];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = f2bf(__fmul_rn(__fmul_rn(bf2f(x[e]), rs[tm]), bf2f(gv[e])));
      r.fx[j][tm] = x;
    }
  }
}

__device__ __forceinline__ f32x4 sum_parts(const XShared& sh, int ml, int nl) {
  f32x4 t = *reinterpret_cast<const f32x4*>(&sh.g.part[0][ml * XPS + nl]);
#pragma unroll
  for (int w = 1; w < XW; ++w) t += *reinterpret_cast<const f32x4*>(&sh.g.part[w][ml * XPS + nl]);
  return t;
}

// The epilogue of one unit (partial tiles in LDS): sums the waves' tiles in
// wave order and stores through to memory.
__device__ void gemm_epilogue(CPhase& P, const EpiItem& it, const EpiPre& e,
                              const XShared& sh) {
  if (!it.on) return;
  const int m = it.ml, n = it.n;
  auto get = [&](int nl, float v[4]) {
    const f32x4 t = sum_parts(sh, m, nl);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = t[i];
  };
  if (P.epi == XE_STORE) {
    float v[4];
    get(it.gi * 4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (P.bias) v[i] += bf2f(e.b[i]);
      if (P.bias_f32) v[i] += e.u[i];
      v[i] = rbf(v[i]);
    }
    if (P.act == SVLA_ACT_SILU) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(silu_f(v[i]));
    }
    if (P.res) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(v[i] + bf2f(e.r[i]));
    }
    st4_wt(static_cast<bf16*>(P.c) + frag_off(m, n), v);  // fragment-major
  } else if (P.epi == XE_ROPE) {
    // rotate-half RoPE on the bf16 projection in fp32 (vla/text_encoder_bf16.py:92-104)
    float x1[4], x2[4], o1[4], o2[4];
    get(it.gi * 4, x1);
    get(8 + it.gi * 4, x2);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = rbf(x1[i]), b = rbf(x2[i]);
      o1[i] = __fsub_rn(__fmul_rn(a, e.u[i]), __fmul_rn(b, e.w[i]));
      o2[i] = __fadd_rn(__fmul_rn(b, e.u[i]), __fmul_rn(a, e.w[i]));
    }
    bf16* crow = static_cast<bf16*>(P.c) + (long)m * P.ldc;
    st4_wt(crow + n, o1);
    st4_wt(crow + n + 32, o2);
    if (P.c_lo) {
      // the reference scores the fp32 RoPE output (vla/text_encoder_bf16.py:
      // 92-104, 117-122): keep what bf16 drops (exact in fp32), so that the
      // attention takes Q . K^T with Q = hi + lo
      float l1[4], l2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        l1[i] = __fsub_rn(o1[i], rbf(o1[i]));
        l2[i] = __fsub_rn(o2[i], rbf(o2[i]));
      }
      bf16* lrow = P.c_lo + (long)m * P.ldc;
      st4_wt(lrow + n, l1);
      st4_wt(lrow + n + 32, l2);
    }
  } else if (P.epi == XE_SILU) {
    // bf16(silu(bf16(gate))) * bf16(up), output column (n / 64) * 32 + n % 64
    // (vla/text_encoder_bf16.py:130-131)
    float g[4], u[4], o[4];
    get(it.gi * 4, g);
    get(8 + it.gi * 4, u);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = rbf(silu_f(rbf(g[i]))) * rbf(u[i]);
    st4_wt(static_cast<bf16*>(P.c) + frag_off(m, (n >> 6) * 32 + (n & 63)), o);  // fragment-major
  } else {
    // Euler: x_out = x_in + dt * bf16(v) in fp32
    float v[4], o[4];
    get(it.gi * 4, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __fadd_rn(e.u[i], __fmul_rn(P.dt, rbf(v[i])));
    st2f_wt(P.x_out + (long)m * P.N + n, o[0], o[1]);
    st2f_wt(P.x_out + (long)m * P.N + n + 2, o[2], o[3]);
  }
}

// one V^T word: item = (sample b, key quad kq, tile column c)
__device__ __forceinline__ void vt_item(CPhase& P, int ct, const XShared& sh, int item) {
  const int c = item & 15, kq = (item >> 4) & 15, b = item >> 8;
  const int base = tile_base(P.epi, ct);
  const int col = (c < 8 ? base + c : base + 32 + (c - 8)) - P.rope_cols;
  float v[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int key = 4 * kq + i;
    float t = 0.f;
    if (key < P.chunk) {
      const int ml = b * P.chunk + key;
#pragma unroll
      for (int w = 0; w < XW; ++w) t += sh.g.part[w][ml * XPS + c];
      t = rbf(t);
    }
    v[i] = t;
  }
  st4_wt(P.vt + ((long)b * (P.N - P.rope_cols) + col) * XVTS + 4 * kq, v);
}

// V columns of a self layer's QKV projection, stored transposed: thread
// (tile column c, key quad kq, sample b) stores keys 4 kq .. 4 kq + 3 of
// column c as one 8-byte word of V^T[b][col][XVTS] (keys past the chunk: 0).
// V is stored as projected (no RoPE).
// (several row groups only at one sample: key = row, so a 4-key word lies in
// one row tile)
__device__ void vt_epilogue(CPhase& P, int ct, const XShared& sh, int t0, int t1) {
  const int nb = P.M / P.chunk;
  for (int item = tidx(); item < 256 * nb; item += XT) {
    const int tile = ((item >> 4) & 15) >> 2;  // row tile of key 4 kq at sample 0
    if (P.row_groups > 1 && (tile < t0 || tile >= t1)) continue;
    vt_item(P, ct, sh, item);
  }
}


__device__ __forceinline__ void gemm_mma(CPhase& P, const GemmRegs& r, const bf16* sw,
                                         f32x4 (&acc)[4], int t0, int t1) {
  const int lane = tidx() & 63, wave = wave_id();
  const int fr = lane & 15, G = lane >> 4;
  int ks0, kcnt;
  wave_krange(P.K, wave, ks0, kcnt);
#pragma unroll
  for (int j = 0; j < XKS; ++j) {
    if (j >= kcnt) break;  // wave-uniform
    const bf16x8 fw = *reinterpret_cast<const bf16x8*>(sw + j * XWSTEP + fr * 32 + wswz(fr, G) * 8);
#pragma unroll
    for (int tm = 0; tm < 4; ++tm)
      if (tm >= t0 && tm < t1)  // wave-uniform
        acc[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw, r.fx[j][tm], acc[tm], 0, 0, 0);
  }
}

// partial tile of this wave: element (row tm*16 + fr, columns 4*(lane/16) .. +3)
__device__ __forceinline__ void put_partial(const f32x4 (&acc)[4], XShared& sh) {
  const int lane = tidx() & 63, wave = wave_id();
  const int fr = lane & 15;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm)
    *reinterpret_cast<f32x4*>(&sh.g.part[wave][(tm * 16 + fr) * XPS + 4 * (lane >> 4)]) = acc[tm];
}

// ---- attention units -----------------------------------------------------------
// One (sample, head).  K rows, V^T rows and the queries are staged into LDS by
// LDS-DMA, each line requested once per CU (fragments loaded straight from
// memory by every wave would request the same lines several times, and a CU
// holds a bounded number of misses in flight).  K and V^T use the GEMM weight
// region (free during attention phases); 16-byte chunks are XOR-swizzled by
// row so the fragment reads of 16 rows spread over the banks.  With at most
// 64 keys a unit is one (sample, head) and wave w < 4 takes query tile w with
// every key; with more keys a unit is one (sample, head, 16-query tile) -- the
// softmax is VALU work, so it is spread over 4x the CUs -- and wave w takes
// keys 32 w .. 32 w + 31, the waves meeting in LDS for the exact softmax.

// 128-byte rows (K, queries; V^T of 64 keys): chunk c of row r at slot
// c ^ ((r >> 1) & 7); longer V^T rows (128 or 256 keys): c ^ (r & 15)
__device__ __forceinline__ int rswz8(int r, int c) { return c ^ ((r >> 1) & 7); }
__device__ __forceinline__ int vswz(int d, int c, int ldvt) {
  return ldvt <= 64 ? rswz8(d, c) : c ^ (d & 15);
}
constexpr int kAttnVt = XMAXK * 64;  // V^T offset in the staging region (bf16)
constexpr int kAttnKlo = XKW * 64;   // K remainders (at most XKW keys: self layers) (bf16)

// K (keys clamped to Lk - 1) and V^T (64 rows of ldvt keys; the writers zero
// the keys past Lk) of sample b, kv head g: 1 KB per DMA instruction, the
// instructions dealt round the waves
__device__ __forceinline__ void attn_stage_kv(CPhase& P, int b, int g, bf16* st) {
  const int lane = tidx() & 63, wave = wave_id();
  const bf16* kb = P.k + b * P.k_bs + g * 64;
  const int nki = (P.lk + 7) >> 3;
  for (int i = wave; i < nki; i += XW) {
    const int key = i * 8 + (lane >> 3);
    const int c = rswz8(key, lane & 7);
    __builtin_amdgcn_global_load_lds((void*)(kb + (unsigned)min(key, P.lk - 1) * (unsigned)P.ldk + c * 8),
                                     (lds_ptr_t)(st + i * 512), 16, 0, 0);
  }
  if (P.k_lo && P.lk <= XKW) {  // uniform; rows XKW.. of the K region are free then
    const bf16* kl = P.k_lo + b * P.k_bs + g * 64;
    for (int i = wave; i < nki; i += XW) {
      const int key = i * 8 + (lane >> 3);
      const int c = rswz8(key, lane & 7);
      __builtin_amdgcn_global_load_lds((void*)(kl + (unsigned)min(key, P.lk - 1) * (unsigned)P.ldk + c * 8),
                                       (lds_ptr_t)(st + kAttnKlo + i * 512), 16, 0, 0);
    }
  }
  const bf16* vb = P.vt_in + b * P.vt_bs + (long)g * 64 * P.ldvt;
  const int lg = 31 - __builtin_clz(P.ldvt);  // ldvt is 64, 128 or 256
  const int nvi = P.ldvt >> 3;                // 64 ldvt elements / 512 per instruction
  for (int i = wave; i < nvi; i += XW) {
    const int e = i * 512 + lane * 8;
    const int d = e >> lg, cs = (e & (P.ldvt - 1)) >> 3;
    __builtin_amdgcn_global_load_lds((void*)(vb + (unsigned)d * (unsigned)P.ldvt + vswz(d, cs, P.ldvt) * 8),
                                     (lds_ptr_t)(st + kAttnVt + i * 512), 16, 0, 0);
  }
}
// query rows r0 .. r0 + 8 n - 1 (clamped to chunk - 1) of sample b, head h
// into LDS rows 0 .. 8 n - 1: one instruction for each of waves 0 .. n - 1
__device__ __forceinline__ void attn_stage_q(CPhase& P, int b, int h, int r0, int n, bf16* lq,
                                             bf16* lq_lo) {
  const int lane = tidx() & 63, wave = wave_id();
  if (wave >= n) return;  // wave-uniform
  const int row = wave * 8 + (lane >> 3);
  const int c = rswz8(row, lane & 7);
  const unsigned off = (unsigned)(b * P.q_bs + h * 64) +
                       (unsigned)min(r0 + row, P.chunk - 1) * (unsigned)P.ldq + c * 8;
  __builtin_amdgcn_global_load_lds((void*)(P.q + off), (lds_ptr_t)(lq + wave * 512), 16, 0, 0);
  if (P.q_lo)  // uniform
    __builtin_amdgcn_global_load_lds((void*)(P.q_lo + off), (lds_ptr_t)(lq_lo + wave * 512), 16,
                                     0, 0);
}
__device__ __forceinline__ void attn_decode(CPhase& P, int unit, int& b, int& h, int& qt) {
  const int bh = unit / P.q_tiles;
  qt = unit - bh * P.q_tiles;
  b = bh / P.heads;
  h = bh - b * P.heads;
}
__device__ __forceinline__ void attn_unit_kv(CPhase& P, int unit, bf16* st) {
  int b, h, qt;
  attn_decode(P, unit, b, h, qt);
  attn_stage_kv(P, b, h * P.kv_heads / P.heads, st);
}

// Every key in one 64-key quarter (self-attention over one chunk): wave qt
// of 0..3 takes query tile qt with all keys, so maxima, sums and the output
// stay in the wave (the same sums as the quarter exchange, whose other
// quarters add nothing).
__device__ __forceinline__ void attn_solo(CPhase& P, int b, int h, int qt, int lane, XShared& sh,
                                          const bf16* lk, const bf16* lv) {
  constexpr int KT = XKW / 16, KS = XKW / 32;
  const int G = lane >> 4, col = lane & 15;
  const int Lq = P.chunk, Lk = P.lk, ldvt = P.ldvt;
  const int nkt = (Lk + 15) / 16;  // <= KT (uniform)
  const int r = qt * 16 + col, qc = min(r, Lq - 1);
  bf16x8 qf[2], ql[2];
#pragma unroll
  for (int ds = 0; ds < 2; ++ds) {
    qf[ds] = *reinterpret_cast<const bf16x8*>(sh.a.q + r * 64 + rswz8(r, ds * 4 + G) * 8);
    if (P.q_lo) ql[ds] = *reinterpret_cast<const bf16x8*>(sh.a.q_lo + r * 64 + rswz8(r, ds * 4 + G) * 8);
  }
  f32x4 s[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t >= nkt) continue;  // wave-uniform
    const int key = t * 16 + col;
#pragma unroll
    for (int ds = 0; ds < 2; ++ds) {
      const int o = key * 64 + rswz8(key, ds * 4 + G) * 8;
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(lk + o);
      if (P.k_lo) {  // uniform: K = hi + lo
        const bf16x8 kl = *reinterpret_cast<const bf16x8*>(lk + kAttnKlo + o);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qf[ds], s[t], 0, 0, 0);
      }
      if (P.q_lo)  // uniform: Q = hi + lo
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, ql[ds], s[t], 0, 0, 0);
      s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ds], s[t], 0, 0, 0);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = t * 16 + 4 * G + i;
      const bool vis = key < Lk && !(P.causal && key > qc);
      s[t][i] = vis ? s[t][i] * P.scale : -INFINITY;
      mx = fmaxf(mx, s[t][i]);
    }
  mx = xor32_max(xor16_max(mx));
  constexpr float kLog2e = 1.4426950408889634f;
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ev = s[t][i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((s[t][i] - mx) * kLog2e);
      s[t][i] = ev;
      sum += ev;
    }
  sum = xor32_sum(xor16_sum(sum));
  const float rl = 1.0f / sum;  // one division per query; P = e * (1 / l)
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (2 * ks >= nkt) continue;  // wave-uniform
    const int kk = 32 * ks + 4 * G;
    bf16x8 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pf[i] = f2bf(s[2 * ks][i] * rl);
      pf[4 + i] = f2bf(s[2 * ks + 1][i] * rl);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = dt * 16 + col;
      const bf16* row = lv + d * ldvt;
      const uint64_t lo = *reinterpret_cast<const uint64_t*>(row + vswz(d, kk >> 3, ldvt) * 8 + (kk & 7));
      const uint64_t hi =
          *reinterpret_cast<const uint64_t*>(row + vswz(d, (kk + 16) >> 3, ldvt) * 8 + (kk & 7));
      const u32x4 w4 = {(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w4), pf, o[dt], 0, 0, 0);
    }
  }
  if (r >= Lq) return;
  const int om = b * P.chunk + r;  // row of the fragment-major output
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = o[dt][i];
    st4_wt(P.o + frag_off(om, h * 64 + dt * 16 + 4 * G), v);
  }
}

// kv_staged: this unit's K and V^T DMA was issued already
__device__ void attn_unit(CPhase& P, int unit, XShared& sh, bf16* st, bool kv_staged) {
  const int lane = tidx() & 63;
  const int wave = wave_id();
  int b, h, qt;
  attn_decode(P, unit, b, h, qt);
  const int G = lane >> 4, col = lane & 15;
  const int Lq = P.chunk, Lk = P.lk, ldvt = P.ldvt;
  const bool solo = Lk <= XKW;  // uniform
  if (!kv_staged) attn_unit_kv(P, unit, st);
  if (solo) attn_stage_q(P, b, h, 0, 8, sh.a.q, sh.a.q_lo);
  else attn_stage_q(P, b, h, qt * 16, 2, sh.a.q, sh.a.q_lo);
  // every wave's DMA landed, then the staged rows are visible to all
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(wc_vm(0));
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  const bf16* lk = st;
  const bf16* lv = st + kAttnVt;
  if (solo) {
    if (wave < 4) attn_solo(P, b, h, wave, lane, sh, lk, lv);
    return;
  }
  // this wave's 32 keys against the unit's query tile
  constexpr int KT = XKG / 16;  // 2 key tiles, one 32-key step
  const int k0 = wave * XKG;
  const int nkt = min(KT, max(0, (Lk - k0 + 15) / 16));  // key tiles with keys (uniform)
  const int qc = min(qt * 16 + col, Lq - 1);
  bf16x8 qf[2], ql[2];
#pragma unroll
  for (int ds = 0; ds < 2; ++ds) {
    qf[ds] = *reinterpret_cast<const bf16x8*>(sh.a.q + col * 64 + rswz8(col, ds * 4 + G) * 8);
    if (P.q_lo) ql[ds] = *reinterpret_cast<const bf16x8*>(sh.a.q_lo + col * 64 + rswz8(col, ds * 4 + G) * 8);
  }
  // S^T tiles: s[t] lane holds scores of keys k0 + 16 t + 4 G + i, query col
  // (K remainders exist only up to XKW keys, the one-wave path: not here)
  f32x4 s[KT];
#pragma unroll
  for (int t = 0; t < KT; ++t) {
    s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (t >= nkt) continue;  // wave-uniform
    const int key = k0 + t * 16 + col;  // < XMAXK: inside the staged rows
#pragma unroll
    for (int ds = 0; ds < 2; ++ds) {
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(lk + key * 64 + rswz8(key, ds * 4 + G) * 8);
      if (P.q_lo)  // uniform: Q = hi + lo
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, ql[ds], s[t], 0, 0, 0);
      s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ds], s[t], 0, 0, 0);
    }
  }
  // exact softmax: the key groups' maxima and sums meet in LDS (keys past
  // Lk, including rows never staged, are masked before any use)
  float mx = -INFINITY;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = k0 + t * 16 + 4 * G + i;
      const bool vis = key < Lk && !(P.causal && key > qc);
      s[t][i] = vis ? s[t][i] * P.scale : -INFINITY;
      mx = fmaxf(mx, s[t][i]);
    }
  mx = xor32_max(xor16_max(mx));
  if (lane < 16) sh.a.amax[wave][lane] = mx;
  wg_sync_lds();
  float m = sh.a.amax[0][col];
#pragma unroll
  for (int j = 1; j < XW; ++j) m = fmaxf(m, sh.a.amax[j][col]);
  constexpr float kLog2e = 1.4426950408889634f;
  float sum = 0.f;
#pragma unroll
  for (int t = 0; t < KT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ev = s[t][i] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((s[t][i] - m) * kLog2e);
      s[t][i] = ev;
      sum += ev;
    }
  sum = xor32_sum(xor16_sum(sum));
  if (lane < 16) sh.a.asum[wave][lane] = sum;
  wg_sync_lds();
  float l = sh.a.asum[0][col];
#pragma unroll
  for (int j = 1; j < XW; ++j) l += sh.a.asum[j][col];
  const float rl = 1.0f / l;  // one division per query; P = e * (1 / l)
  // O^T = V^T . P^T over the wave's 32 keys; contraction index 8 G + j <->
  // key k0 + 16 (j / 4) + 4 G + j % 4 (both operands)
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (nkt > 0) {  // wave-uniform
    bf16x8 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pf[i] = f2bf(s[0][i] * rl);
      pf[4 + i] = f2bf(s[1][i] * rl);
    }
    const int kk = k0 + 4 * G;  // < ldvt here
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = dt * 16 + col;
      const bf16* row = lv + d * ldvt;
      const uint64_t lo = *reinterpret_cast<const uint64_t*>(row + vswz(d, kk >> 3, ldvt) * 8 + (kk & 7));
      const uint64_t hi =
          *reinterpret_cast<const uint64_t*>(row + vswz(d, (kk + 16) >> 3, ldvt) * 8 + (kk & 7));
      const u32x4 w4 = {(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, w4), pf, o[dt], 0, 0, 0);
    }
  }
  // partial O^T of this key group: lane holds O^T[dt*16 + 4G + i][col]
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) sh.a.o[wave][dt * 16 + 4 * G + i][col] = o[dt][i];
  wg_sync_lds();
  // wave dt < 4 sums d-tile dt over the key groups in order and stores it
  const int qi = qt * 16 + col;
  if (wave < 4 && qi < Lq) {
    const int dt = wave;
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = dt * 16 + 4 * G + i;
      float t = sh.a.o[0][d][col];
#pragma unroll
      for (int j = 1; j < XW; ++j) t += sh.a.o[j][d][col];
      r[i] = t;
    }
    st4_wt(P.o + frag_off(b * P.chunk + qi, h * 64 + dt * 16 + 4 * G), r);  // fragment-major
  }
}

// V^T of the cross layers' projected prefix V: unit (layer, sample, block of
// 64 columns); thread (column d, key quad) for 4 rounds of 64 keys.
__device__ void vt_unit_transpose(CPhase& P, int unit) {
  const int tid = tidx();
  const int per_layer = P.vt_blocks * (P.M / P.chunk);
  const int li = unit / per_layer, rem = unit - li * per_layer;
  const int b = rem / P.vt_blocks, blk = rem - b * P.vt_blocks;
  const int d = tid & 63, kq = tid >> 6;
  constexpr int kRound = XT / 64 * 4;  // keys per round
  const bf16* src = P.vt_src[li] + b * P.vt_src_bs + blk * 64 + d;
  bf16* dst = P.vt_dst[li] + b * P.vt_dst_bs + (long)(blk * 64 + d) * XMAXK;
  constexpr int kRounds = XMAXK / kRound;
  // every load issued before any use (a use right after its load would make
  // each load a round trip of its own)
  uint16_t hv[kRounds][4];
#pragma unroll
  for (int round = 0; round < kRounds; ++round)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = round * kRound + kq * 4 + i;
      hv[round][i] = ldg16(src + (long)min(key, P.vt_keys - 1) * P.vt_ldv);
    }
#pragma unroll
  for (int round = 0; round < kRounds; ++round) {
    const int key0 = round * kRound + kq * 4;
    uint64_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w |= (uint64_t)(key0 + i < P.vt_keys ? hv[round][i] : (uint16_t)0) << (16 * i);
    st8_wt(dst + key0, w);
  }
}

// ---- the persistent kernel -------------------------------------------------------
// Touch every 64-byte line of a phase's table entry with scalar loads, so the
// reads of its fields after the phase wait hit the scalar cache (a dependent
// chain of misses would cost a memory round trip per link).  The result only
// keeps the loads alive.
__device__ __forceinline__ unsigned touch_phase(CPhase* ph) {
  typedef const __attribute__((address_space(4))) unsigned cu32;
  cu32* w = reinterpret_cast<cu32*>(ph);
  unsigned t = 0;
#pragma unroll
  for (int i = 0; i < (int)((sizeof(XPhase) + 63) / 64); ++i) t ^= w[i * 16];
  return t;
}

// A workgroup that leaves because the launch gave up (a wait timed out, the
// team did not form) fills the action output (the last phase's Euler state)
// with NaN: a caller that never reads the status word -- a replayed graph,
// for one -- still gets an unmistakable result.  (A give-up also sets the
// status word, so such a chunk is reported failed whichever of its Euler
// units still wrote.)
__device__ void poison_actions(const XArgs& g) {
  CPhase& L = g.ph[g.n_ph - 1];
  if (L.kind != XK_GEMM || L.epi != XE_EULER || !L.x_out) return;  // uniform
  const int n2 = L.M * L.N / 2;  // N even (action_dim % 16 == 0)
  const float q = __builtin_nanf("");
  for (int i = tidx(); i < n2; i += XT) st2f_wt(L.x_out + 2 * i, q, q);
  __builtin_amdgcn_s_waitcnt(wc_vm(0));
}

// One-XCD team mode: workgroup 0, when it is not a member, watches that the
// team forms (enough workgroups landed on the team's XCD); if it does not
// within the spin limit, it sets XS_TEAM and poisons the output.
__device__ void team_watch(const XArgs& g) {
  __shared__ int s_fail;
  if (wave_id() == 0) {
    const unsigned* reg = g.cnt + (size_t)g.n_ph * kSub * kCntStride;
    bool fail = true;
    for (int n = 0; n < g.spin; ++n) {
      if (__builtin_amdgcn_readfirstlane(ld_agent(reg)) >= (unsigned)g.team_size ||
          __builtin_amdgcn_readfirstlane(ld_agent(g.status)) != 0u) {
        fail = false;  // formed, or a member already reported a failure
        break;
      }
    }
    if (fail && (tidx() & 63) == 0)
      __hip_atomic_store(g.status, (unsigned)XS_TEAM, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if ((tidx() & 63) == 0) s_fail = fail;
  }
  __syncthreads();
  if (s_fail) poison_actions(g);
}

__global__ __launch_bounds__(XT, 1) void expert_kernel(XArgs g) {
  __shared__ XShared sh;
  __shared__ __attribute__((aligned(1024))) bf16 s_w[XW][XKS * XWSTEP];  // per-wave weights
  __shared__ int s_rank;
  const int tid = threadIdx.x, wave = wave_id(), lane = tid & 63;
  // team: every workgroup, or those on XCD team_xcd (ranked on arrival)
  if (tid == 0) {
    int rank = blockIdx.x;
    if (g.team_xcd >= 0) {
      unsigned x;
      asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
      rank = -1;
      if ((int)(x & 15u) == g.team_xcd) {
        unsigned* reg = g.cnt + (size_t)g.n_ph * kSub * kCntStride;
        const unsigned r =
            __hip_atomic_fetch_add(reg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        rank = r < (unsigned)g.team_size ? (int)r : -1;
      }
    }
    s_rank = rank;
  }
  __syncthreads();
  const int rank = s_rank;
  if (rank < 0) {
    if (g.team_xcd >= 0 && blockIdx.x == 0) team_watch(g);
    return;
  }
  const int team = g.team_xcd >= 0 ? g.team_size : (int)gridDim.x;
  bool failed = false;  // this workgroup gave up (poisons the output on its way out)
  if (g.team_xcd >= 0) {
    if (wave == 0) {
      // every member registered before anyone relies on the team's size
      const unsigned* reg = g.cnt + (size_t)g.n_ph * kSub * kCntStride;
      bool ok = false;
      for (int n = 0; n < g.spin; ++n) {
        const unsigned rr = __builtin_amdgcn_readfirstlane(ld_agent(reg));
        if (rr >= (unsigned)team) { ok = true; break; }
        if (__builtin_amdgcn_readfirstlane(ld_agent(g.status)) != 0u) break;
      }
      if (!ok && lane == 0)
        __hip_atomic_store(g.status, (unsigned)XS_TEAM, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 0) s_rank = ok ? rank : -1;
    }
    __syncthreads();
    failed = s_rank < 0;
  }

  if (wave == 1) {
    const unsigned t = touch_phase(g.ph) ^ (g.n_ph > 1 ? touch_phase(g.ph + 1) : 0u);
    asm volatile("" ::"s"(t));
  }
  for (int p = 0; p < g.n_ph && !failed; ++p) {
    CPhase& P = g.ph[p];
    if (rank >= P.units) continue;
    const int tid = tidx(), lane = tid & 63;  // (not hoisted: see tidx)
    const int mine = (P.units - rank + team - 1) / team;
    GemmRegs r;
    bf16* sw = s_w[wave];
    // weights of the first unit (and the K / V^T of a cross-attention unit)
    // before the wait: they do not depend on it
    if (P.kind == XK_GEMM) {
      dma_w(P.epi, P.w, P.N, P.K, P.ldw, rank % P.col_tiles, sw);
      if (P.norm_w) dma_gain(P.norm_w, P.K, sh.g.gain[wave]);
    }
    else if (P.kind == XK_ATTN && P.kv_static)
      attn_unit_kv(P, rank, &s_w[0][0]);
    if (p > 0) {
      if (wave == 1 && p + 1 < g.n_ph) {
        // while wave 0 waits: the next phase's table entry into the scalar
        // cache (this one's was touched a phase ago)
        const unsigned t = touch_phase(g.ph + p + 1);
        asm volatile("" ::"s"(t));
      }
      if (wave == 0) {
        const bool ok = wait_phase(g, p - 1, (unsigned)g.ph[p - 1].units);
        if (lane == 0) s_rank = ok ? rank : -1;
      }
      __syncthreads();
      if (s_rank < 0) {
        failed = true;
        break;
      }
    }
    if (g.stamps && rank == 0 && tidx() == 0) g.stamps[2 * p] = __builtin_amdgcn_s_memrealtime();
    if (P.kind == XK_GEMM) {
      for (int j = 0; j < mine; ++j) {
        const int u = rank + j * team;
        const int ct = u % P.col_tiles, grp = u / P.col_tiles;
        const int t0 = grp * P.group_tiles, t1 = min(t0 + P.group_tiles, 4);
        const bool vt = vt_unit(P, ct);
        const EpiItem it = epi_item(P, ct, t0, t1);
        EpiPre e{};
        if (!vt) epi_prefetch(P, it, e);
        // one row group: the activations stay in registers for the phase's units
        const bool load = j == 0 || P.row_groups > 1;
        if (load) {
          load_x(P, r, t0, t1);
          if (P.norm_w) {
            // per-row sums of squares of the whole K range meet in LDS, then
            // every wave normalises its activation fragments
#pragma unroll
            for (int tm = 0; tm < 4; ++tm) {
              float t = r.ss[tm];
              t = xor32_sum(xor16_sum(t));
              if (lane < 16) sh.g.ss[wave][tm * 16 + lane] = t;
            }
            wg_sync_lds();
            norm_x(P, r, sh, t0, t1);
          }
        }
        f32x4 acc[4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) acc[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
        // this wave's weight DMA (issued first) and activations have landed
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_waitcnt(wc_vm(0));
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        gemm_mma(P, r, sw, acc, t0, t1);
        put_partial(acc, sh);
        wg_sync_lds();  // also: this wave's weight reads are done
        // the next unit's weights stream in during this unit's epilogue
        if (j + 1 < mine)
          dma_w(P.epi, P.w, P.N, P.K, P.ldw, (u + team) % P.col_tiles, sw);
        if (vt) vt_epilogue(P, ct, sh, t0, t1);
        else gemm_epilogue(P, it, e, sh);
        wg_sync_lds();  // partial tiles free for the next unit
      }
    } else if (P.kind == XK_ATTN) {
      for (int j = 0; j < mine; ++j) {
        attn_unit(P, rank + j * team, sh, &s_w[0][0], j == 0 && P.kv_static);
        wg_sync_lds();  // LDS free for the next unit
      }
    } else {
      for (int j = 0; j < mine; ++j) vt_unit_transpose(P, rank + j * team);
    }
    // every store of this workgroup acknowledged, then one arrival
    __builtin_amdgcn_s_waitcnt(wc_vm(0));
    __syncthreads();
    if (tid == 0) {
      __hip_atomic_fetch_add(g.cnt + ((size_t)p * kSub + (rank & (kSub - 1))) * kCntStride,
                             (unsigned)mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (g.stamps && rank == 0) g.stamps[2 * p + 1] = __builtin_amdgcn_s_memrealtime();
    }
  }
  if (failed) poison_actions(g);
}

__global__ void clear_u32_kernel(unsigned* p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = 0u;
}

// ---- host-side plan ------------------------------------------------------------
constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct Arena {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off += align_up(bytes);
    return o;
  }
};

struct Layout {
  size_t phases, counters, status, arena, total;
  int n_ph;
  size_t n_cnt_words;
};

int n_cross(const svla_expert_desc* d) {
  int n = 0;
  for (int l = 0; l < d->n_layers; ++l) n += d->layers[l].cross != 0;
  return n;
}

int count_phases(const svla_expert_desc* d) {
  return (n_cross(d) > 0 ? 1 : 0) + d->num_steps * (4 + 5 * d->n_layers);
}

bool desc_ok(const svla_expert_desc* d) {
  if (!d || d->batch <= 0 || d->chunk <= 0 || d->head_dim != 64) return false;
  if (d->batch * d->chunk > XBM || d->chunk > XVTS) return false;
  if (d->hidden % 16 || d->inter % 32 || d->action_dim % 16 || d->n_layers <= 0) return false;
  if (d->hidden > XKS * XW * 32 || d->inter > XKS * XW * 32 || d->action_dim > 32) return false;
  if (d->n_q_heads <= 0 || d->n_kv_heads <= 0 || d->n_q_heads % d->n_kv_heads) return false;
  if (d->n_q_heads * 64 > XKS * XW * 32) return false;
  if (d->num_steps <= 0 || d->prefix_len <= 0 || d->prefix_len > XMAXK) return false;
  if (!d->layers || !d->w_action_in || !d->w_time_in_a || !d->time_bias || !d->w_time_out ||
      !d->w_action_out || !d->rope_cos || !d->rope_sin)
    return false;
  if (n_cross(d) > kMaxCross) return false;
  for (int l = 0; l < d->n_layers; ++l) {
    const svla_expert_layer& L = d->layers[l];
    if (!L.w_qkv || !L.w_o || !L.w_gu || !L.w_down || !L.norm1 || !L.norm2) return false;
    if (L.cross && (!L.cross_k || !L.cross_v || d->ld_cross % 8)) return false;
  }
  return true;
}

// Builds the phase list (and, with base != nullptr, the buffer addresses).
// trace (optional): the workspace offset of the activation entering each
// layer of each Euler step, and of the last layer's output: (n_layers + 1)
// entries per step, step-major.  Fragment-major [64 rows][hidden] bf16.
size_t build(const svla_expert_desc* d, char* base, std::vector<XPhase>* out, Layout* lay,
             std::vector<size_t>* trace = nullptr) {
  const int M = d->batch * d->chunk, H = d->hidden, qd = d->n_q_heads * 64,
            kvd = d->n_kv_heads * 64, I = d->inter, A = d->action_dim;
  Layout L{};
  L.n_ph = count_phases(d);
  L.n_cnt_words = (size_t)(L.n_ph + 1) * kSub * kCntStride;
  Arena ar;
  L.phases = ar.take(sizeof(XPhase) * L.n_ph);
  L.counters = ar.take(L.n_cnt_words * 4);
  L.status = ar.take(4);
  L.arena = ar.off;
  size_t last = 0;  // offset of the buffer buf() returned last
  auto buf = [&](size_t bytes) -> char* {
    last = ar.take(bytes);
    return base ? base + last : nullptr;
  };
  // fragment-major activation of N columns (64 rows)
  auto fbuf = [&](int N) { return (bf16*)buf((size_t)((N + 31) / 32) * 4096); };
  auto gemm = [&](const void* a, int lda, const void* w, int N, int K, void* c, int ldc) {
    XPhase P{};
    P.kind = XK_GEMM;
    P.epi = XE_STORE;
    P.M = M; P.N = N; P.K = K;
    P.col_tiles = (N + XBN - 1) / XBN;
    P.units = P.col_tiles;
    P.a = a; P.lda = lda;
    P.w = static_cast<const bf16*>(w); P.ldw = K;
    P.c = c; P.ldc = ldc;
    P.norm_eps = d->rms_eps;
    P.chunk = d->chunk;
    return P;
  };
  std::vector<XPhase> ph;
  // V^T of every cross layer's projected prefix V: [sample][kv][256 keys]
  std::vector<bf16*> cross_vt(d->n_layers, nullptr);
  if (n_cross(d) > 0) {
    XPhase T{};
    T.kind = XK_VT;
    T.M = M; T.chunk = d->chunk;
    T.vt_blocks = kvd / 64;
    T.vt_ldv = d->ld_cross;
    T.vt_keys = d->prefix_len;
    T.vt_src_bs = (long)d->prefix_len * d->ld_cross;
    T.vt_dst_bs = (long)kvd * XMAXK;
    for (int l = 0; l < d->n_layers; ++l) {
      if (!d->layers[l].cross) continue;
      cross_vt[l] = (bf16*)buf((size_t)d->batch * kvd * XMAXK * 2);
      T.vt_src[T.n_vt] = static_cast<const bf16*>(d->layers[l].cross_v);
      T.vt_dst[T.n_vt] = cross_vt[l];
      ++T.n_vt;
    }
    T.units = T.n_vt * d->batch * T.vt_blocks;
    ph.push_back(T);
  }
  const float* x_prev = d->x_in;
  for (int s = 0; s < d->num_steps; ++s) {
    // action / time embedding (the time part of time_in precomputed per step)
    bf16* a_emb = fbuf(H);
    XPhase P = gemm(x_prev, A, d->w_action_in, H, A, a_emb, H);
    P.a_f32 = 1;
    P.bias = static_cast<const bf16*>(d->b_action_in);
    ph.push_back(P);
    bf16* h_t = fbuf(H);
    P = gemm(a_emb, H, d->w_time_in_a, H, H, h_t, H);
    P.bias_f32 = d->time_bias + (size_t)s * H;
    P.act = SVLA_ACT_SILU;
    ph.push_back(P);
    bf16* ex = fbuf(H);
    if (trace) trace->push_back(last);
    P = gemm(h_t, H, d->w_time_out, H, H, ex, H);
    P.bias = static_cast<const bf16*>(d->b_time_out);
    ph.push_back(P);
    for (int l = 0; l < d->n_layers; ++l) {
      const svla_expert_layer& Ly = d->layers[l];
      const int nq = Ly.cross ? qd : qd + 2 * kvd;  // projected columns
      const int nqk = Ly.cross ? qd : qd + kvd;     // stored row-major (Q | K)
      bf16* qk = (bf16*)buf((size_t)M * nqk * 2);
      bf16* qk_lo = (bf16*)buf((size_t)M * nqk * 2);  // remainders of the fp32 RoPE output
      bf16* vt = Ly.cross ? nullptr : (bf16*)buf((size_t)d->batch * kvd * XVTS * 2);
      P = gemm(ex, H, Ly.w_qkv, nq, H, qk, nqk);
      P.epi = XE_ROPE;
      P.norm_w = static_cast<const bf16*>(Ly.norm1);
      P.cos_t = d->rope_cos; P.sin_t = d->rope_sin;
      P.rope_cols = nqk;
      P.rope_period = d->chunk;
      P.vt = vt;
      P.c_lo = qk_lo;
      ph.push_back(P);
      bf16* att = fbuf(qd);
      XPhase T{};
      T.kind = XK_ATTN;
      T.M = M;
      // one unit per (sample, head) when one wave takes every key, else per
      // (sample, head, 16-query tile)
      T.q_tiles = (Ly.cross ? d->prefix_len : d->chunk) <= XKW ? 1 : (d->chunk + 15) / 16;
      T.units = d->batch * d->n_q_heads * T.q_tiles;
      T.heads = d->n_q_heads; T.kv_heads = d->n_kv_heads;
      T.chunk = d->chunk;
      T.scale = 0.125f;
      T.q = qk; T.ldq = nqk; T.q_bs = (long)d->chunk * nqk;
      T.q_lo = qk_lo;
      if (Ly.cross) {
        T.k = static_cast<const bf16*>(Ly.cross_k); T.ldk = d->ld_cross;
        T.k_bs = (long)d->prefix_len * d->ld_cross;
        T.vt_in = cross_vt[l]; T.ldvt = XMAXK; T.vt_bs = (long)kvd * XMAXK;
        T.lk = d->prefix_len;
        T.causal = 0;
        T.kv_static = 1;
      } else {
        T.k = qk + qd; T.ldk = nqk; T.k_bs = (long)d->chunk * nqk;
        T.k_lo = qk_lo + qd;  // chunk <= XKW: the one-wave path, which reads it
        T.vt_in = vt; T.ldvt = XVTS; T.vt_bs = (long)kvd * XVTS;
        T.lk = d->chunk;
        T.causal = 1;
      }
      T.o = att; T.ldo = qd; T.o_bs = (long)d->chunk * qd;
      ph.push_back(T);
      bf16* ex1 = fbuf(H);
      P = gemm(att, qd, Ly.w_o, H, qd, ex1, H);
      P.res = ex; P.ldr = H;
      ph.push_back(P);
      bf16* act = fbuf(I);
      P = gemm(ex1, H, Ly.w_gu, 2 * I, H, act, I);
      P.epi = XE_SILU;
      P.norm_w = static_cast<const bf16*>(Ly.norm2);
      ph.push_back(P);
      bf16* ex2 = fbuf(H);
      if (trace) trace->push_back(last);
      P = gemm(act, I, Ly.w_down, H, I, ex2, H);
      P.res = ex1; P.ldr = H;
      ph.push_back(P);
      ex = ex2;
    }
    float* x_next = s + 1 == d->num_steps ? d->x_out : (float*)buf((size_t)M * A * 4);
    P = gemm(ex, H, d->w_action_out, A, H, nullptr, 0);
    P.epi = XE_EULER;
    P.norm_w = static_cast<const bf16*>(d->norm_out);
    P.x_in = x_prev;
    P.x_out = x_next;
    P.dt = d->dt;
    ph.push_back(P);
    x_prev = x_next;
  }
  // Row groups: a phase with few column tiles also splits its row tiles over
  // units, so a unit reads only its rows' activations (the critical path of
  // a phase; the weights stream in before the phase wait).  Up to
  // kUnitTarget units (one per CU of an MI355X); several groups of a phase
  // writing V^T only at one sample (key = row there).
  constexpr int kUnitTarget = 256;
  const int nrt = (M + 15) / 16;
  for (XPhase& P : ph) {
    if (P.kind != XK_GEMM) continue;
    int rg = 1;
    while (rg * 2 <= nrt && P.col_tiles * rg * 2 <= kUnitTarget && (!P.vt || d->batch == 1)) rg *= 2;
    P.row_groups = rg;
    P.group_tiles = rg == 1 ? 4 : (nrt + rg - 1) / rg;
    P.units = P.col_tiles * rg;
  }
  L.total = ar.off;
  if (out) *out = std::move(ph);
  if (lay) *lay = L;
  return L.total;
}

}  // namespace

extern "C" {

long svla_expert_workspace_size(const svla_expert_desc* d) {
  if (!desc_ok(d)) return 0;
  return (long)build(d, nullptr, nullptr, nullptr);
}

long svla_expert_trace_offset(const svla_expert_desc* d, int step, int layer) {
  if (!desc_ok(d) || step < 0 || step >= d->num_steps || layer < 0 || layer > d->n_layers)
    return -1;
  std::vector<size_t> tr;
  build(d, nullptr, nullptr, nullptr, &tr);
  const size_t i = (size_t)step * (d->n_layers + 1) + layer;
  return i < tr.size() ? (long)tr[i] : -1;
}

int svla_expert_prepare(const svla_expert_desc* d, void* ws, long ws_bytes, int team_xcd,
                        svla_expert_plan* plan, svla_stream_t stream) {
  if (!desc_ok(d) || !ws || !plan || ((uintptr_t)ws % kAlign) || team_xcd > 7) return SVLA_EINVAL;
  if (!d->x_in || !d->x_out || ((uintptr_t)d->x_in & 15) || ((uintptr_t)d->x_out & 15))
    return SVLA_EINVAL;
  std::vector<XPhase> ph;
  Layout L{};
  if (ws_bytes < 0 || build(d, static_cast<char*>(ws), &ph, &L) > (size_t)ws_bytes)
    return SVLA_EINVAL;
  if ((int)ph.size() != L.n_ph || L.status != L.counters + L.n_cnt_words * 4) return SVLA_EINVAL;
  char* base = static_cast<char*>(ws);
  hipStream_t s = (hipStream_t)stream;
  // zero the whole workspace once: the padding rows and columns of the
  // fragment-major activations are never written and must read as zero
  hipLaunchKernelGGL(clear_u32_kernel, dim3(1024), dim3(256), 0, s, reinterpret_cast<unsigned*>(base),
                     (long)(L.total / 4));
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  e = hipMemcpyAsync(base + L.phases, ph.data(), sizeof(XPhase) * ph.size(),
                     hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return (int)e;
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return (int)e;
  int dev = 0, cus = 0;
  if ((e = hipGetDevice(&dev)) != hipSuccess) return (int)e;
  if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess)
    return (int)e;
  // a one-XCD team is an eighth of the CUs (MI355X: 8 XCDs of 32 CUs); the
  // kernel's own registration check catches a team that does not form
  if (team_xcd >= 0 && (cus % 8 || cus < 8)) return SVLA_EINVAL;
  std::memset(plan, 0, sizeof(*plan));
  plan->phases = base + L.phases;
  plan->n_phases = L.n_ph;
  plan->counters = reinterpret_cast<unsigned*>(base + L.counters);
  plan->counter_words = (long)L.n_cnt_words;
  plan->status = reinterpret_cast<unsigned*>(base + L.status);
  plan->grid = cus;
  plan->team_xcd = team_xcd < 0 ? -1 : team_xcd;
  plan->team_size = team_xcd < 0 ? cus : cus / 8;
  plan->spin_limit = kSpin;
  plan->stamps = nullptr;
  return SVLA_OK;
}

int svla_expert_run(const svla_expert_plan* plan, svla_stream_t stream) {
  if (!plan || !plan->phases || plan->n_phases <= 0 || plan->grid <= 0 || plan->spin_limit < 0)
    return SVLA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const long words = plan->counter_words + kAlign / 4;  // counters, then the status word
  hipLaunchKernelGGL(clear_u32_kernel, dim3(256), dim3(256), 0, s, plan->counters, words);
  SVLA_CHECK_LAUNCH();
  XArgs g;
  g.ph = (CPhase*)plan->phases;
  g.n_ph = plan->n_phases;
  g.cnt = plan->counters;
  g.status = plan->status;
  g.team_xcd = plan->team_xcd;
  g.team_size = plan->team_size;
  g.spin = plan->spin_limit;
  g.stamps = plan->stamps;
  hipLaunchKernelGGL(expert_kernel, dim3(plan->grid), dim3(XT), 0, s, g);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_expert_status(const svla_expert_plan* plan, int* status) {
  if (!plan || !plan->status || !status) return SVLA_EINVAL;
  unsigned v = 0;
  hipError_t e = hipMemcpy(&v, plan->status, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return (int)e;
  *status = (int)v;
  return SVLA_OK;
}

}  // extern "C"
