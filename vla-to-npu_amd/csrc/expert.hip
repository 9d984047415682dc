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
// Design (CDNA4, measured on MI355X with a microbenchmark of this build):
//  * One workgroup of 8 waves per CU.  A phase is split into UNITS (a
//    64-row x 16-column output tile of a GEMM, or one (sample, head) of an
//    attention); unit u of a phase runs on team rank u % team_size.
//  * Phases hand over through device-scope arrival counters: a workgroup
//    that finished its units of phase p waits for its stores to be
//    acknowledged (vmcnt = 0), then adds its unit count to one of 8
//    sub-counters of phase p (spread so that 256 arrivals do not queue on one
//    address: a grid barrier measured 4.0 us with one counter, 2.0 us with
//    8); a workgroup with units in phase p + 1 polls the 8 sub-counters (8
//    lanes, agent-scope atomic loads) until they sum to phase p's unit count.
//    Completion of phase p implies completion of every earlier phase (each of
//    its units waited for p - 1), so one wait per phase suffices.
//  * Every phase writes its output to a buffer that no other phase of the
//    launch writes (activation versions, not in-place updates), 256-byte
//    aligned, with write-through (agent-scope) stores.  No cache can then
//    hold a stale copy of data a phase reads: nobody reads an address before
//    the phase that writes it has completed, so the first read of a line by
//    an XCD misses its L2 and later reads by that XCD's CUs hit the fresh
//    line.  Activations are read with plain loads (L2-cached broadcast).
//  * Weights never depend on the previous phase: a workgroup issues the
//    weight loads of its first unit of a phase BEFORE it waits for the
//    phase's inputs (register prefetch), so the weight latency overlaps the
//    hand-off; further units of the same phase prefetch during the epilogue.
//  * GEMM units are the skinny kernel's: 8 waves split K, each wave holds its
//    k-range of the 64 activation rows in registers for the whole phase and
//    one 16x16x32 MFMA fragment of weights per k-step; the 8 partial tiles
//    meet in LDS.  The RMSNorm in front of a projection is fused (gain on the
//    way into the MFMAs, row sums of squares from the same fragments, 1/rms
//    in the epilogue).  Paired epilogues (RoPE pairs (d, d+32), SiLU(gate) *
//    up) use the 16-column tile of 8 columns + their partners.
//  * Attention units: one (sample, head) on 4 waves of 16 queries each; V is
//    staged transposed in LDS, scores are fp32, the softmax is computed
//    exactly (max, sum, divide) and the probabilities rounded to bf16 before
//    P.V, as the reference torch module does (vla/text_encoder_bf16.py:117-126).
//  * Every wait is bounded: past kSpin polls (or when another workgroup has
//    already given up) the workgroup sets the status word and leaves, so the
//    grid always drains.  The team is either every workgroup of the launch
//    or, optionally, the workgroups of one XCD (selected by the hardware
//    XCC_ID register); the write-through / write-once discipline keeps the
//    results correct whichever CUs take part.
#include <cstring>
#include <mutex>
#include <vector>

#include "svla_common.h"

namespace {

constexpr int XW = 8;              // waves per workgroup
constexpr int XT = XW * 64;        // threads per workgroup
constexpr int XKS = 4;             // 32-deep k-steps per wave and pass
constexpr int XPASS = 2;           // passes per unit: K <= XW * XKS * 32 * XPASS = 2048
constexpr int XBM = 64;            // rows per GEMM unit (4 MFMA row tiles)
constexpr int XBN = 16;            // columns per GEMM unit
constexpr int XPS = XBN + 4;       // padded LDS row of a partial tile (floats)
constexpr int XMAXQ = 64;          // attention: queries per sample
constexpr int XMAXK = 256;         // attention: keys per sample
constexpr int XVT = XMAXK + 8;     // padded LDS row of V^T (bf16)
constexpr int kSub = 8;            // sub-counters per phase
constexpr int kCntStride = 32;     // unsigned per sub-counter (128 bytes apart)
constexpr int kSpin = 1 << 22;     // polls before a wait gives up

enum XKind { XK_GEMM = 0, XK_ATTN = 1 };
enum XEpi { XE_STORE = 0, XE_ROPE = 1, XE_SILU = 2, XE_EULER = 3 };
enum XStat { XS_OK = 0, XS_TIMEOUT = 1, XS_TEAM = 2 };

struct XPhase {
  int kind, epi, act, a_f32;
  int M, N, K, units, col_tiles;
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
  const float* x_in;  // Euler: x_out[m, n] = x_in[m, n] + dt * bf16(v) (fp32, leading dim N)
  float* x_out;
  float dt;
  // attention: unit = sample * heads + head
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  int ldq, ldk, ldv, ldo;
  long q_bs, k_bs, v_bs, o_bs;
  int heads, kv_heads, lq, lk, causal;
  float scale;
};

struct XArgs {
  const XPhase* ph;
  int n_ph;
  unsigned* cnt;     // [n_ph + 1][kSub][kCntStride]; the last row is the team registration
  unsigned* status;  // XStat of the launch (0 = ok)
  int team_xcd;      // < 0: every workgroup; else the workgroups on this XCD
  int team_size;     // participants expected when team_xcd >= 0
};

// Loads through pointers read from the phase table: tell the compiler they
// are global (flat loads would also count on lgkmcnt and force full waits).
typedef const __attribute__((address_space(1))) bf16x8* gbf8p;
typedef const __attribute__((address_space(1))) f32x4* gf4p;
typedef const __attribute__((address_space(1))) bf16x4* gbf4p;
__device__ __forceinline__ bf16x8 ldg8(const bf16* p) { return *(gbf8p)(p); }
__device__ __forceinline__ bf16x4 ldg4(const bf16* p) { return *(gbf4p)(p); }
__device__ __forceinline__ f32x4 ldgf4(const float* p) { return *(gf4p)(p); }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ unsigned ld_agent(const unsigned* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// gfx9 s_waitcnt immediate: vmcnt split over bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8; the counters not named are left unconstrained
constexpr int wc_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int wc_lgkm0 = 15 | (3 << 14) | (7 << 4);

// LDS written by this wave visible to the whole workgroup (global memory
// operations in flight are not waited for)
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
// 4 bf16 (8 bytes) stored write-through
__device__ __forceinline__ void st4_wt(bf16* p, const float v[4]) {
  bf16x4 o;
  o[0] = f2bf(v[0]); o[1] = f2bf(v[1]); o[2] = f2bf(v[2]); o[3] = f2bf(v[3]);
  st8_wt(p, __builtin_bit_cast(uint64_t, o));
}
__device__ __forceinline__ void st2f_wt(float* p, float a, float b) {
  st8_wt(p, __builtin_bit_cast(uint64_t, u32x2{__builtin_bit_cast(uint32_t, a),
                                               __builtin_bit_cast(uint32_t, b)}));
}

// Thread 0 of wave 0's lanes 0..7 poll the 8 sub-counters of `row` until they
// sum to `target`; false when the wait gave up (status set).  Wave 0 only.
__device__ bool wait_phase(const XArgs& g, int row, unsigned target) {
  const int lane = threadIdx.x & 63;
  const unsigned* c = g.cnt + ((size_t)row * kSub + (lane & (kSub - 1))) * kCntStride;
  for (int n = 0;; ++n) {
    unsigned s = lane < kSub ? ld_agent(c) : 0u;
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    if (__builtin_amdgcn_readfirstlane(s) >= target) return true;
    const unsigned st = ld_agent(g.status);
    if (__builtin_amdgcn_readfirstlane(st) != 0u) return false;
    if (n >= kSpin) {
      if (lane == 0)
        __hip_atomic_store(g.status, (unsigned)XS_TIMEOUT, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
  }
}

// ---- GEMM units ---------------------------------------------------------------
struct GemmRegs {
  bf16x8 fw[XKS];     // weights of the current unit: this wave's k-steps
  bf16x8 fx[XKS][4];  // activations: this wave's k-steps x 4 row tiles
  float ss[4];        // norm: this lane's row sums of squares (rows tm*16 + fr)
};

__device__ __forceinline__ bool paired(int epi) { return epi == XE_ROPE || epi == XE_SILU; }

// first packed column of unit column tile ct (16-column tile; a paired tile
// holds 8 columns of a first half and their 8 partners 32 columns on)
__device__ __forceinline__ int tile_base(const XPhase& P, int ct) {
  const int n0 = ct * XBN;
  return paired(P.epi) ? (n0 >> 6) * 64 + ((n0 & 63) >> 4) * 8 : n0;
}

// This wave's k-steps: [ks0, ks0 + kcnt) of the nks = ceil(K / 32) steps,
// `per` (uniform) per wave, taken in passes of XKS.
__device__ __forceinline__ void wave_krange(int K, int wave, int& ks0, int& kcnt, int& per) {
  const int nks = (K + 31) / 32;
  per = (nks + XW - 1) / XW;
  ks0 = wave * per;
  kcnt = max(0, min(per, nks - ks0));
}
__device__ __forceinline__ int n_passes(int K) {
  const int per = ((K + 31) / 32 + XW - 1) / XW;
  return (per + XKS - 1) / XKS;
}

// Weight fragments of column tile ct for pass `pass` (this lane's row, this
// wave's k-steps); steps past the wave's range reload its last one (never
// used), so all XKS loads are issued unconditionally and fly together.
__device__ __forceinline__ void load_w(const XPhase& P, int ct, int pass, GemmRegs& r) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  int ks0, kcnt, per;
  wave_krange(P.K, wave, ks0, kcnt, per);
  const int nks = (P.K + 31) / 32;
  const int base = tile_base(P, ct);
  const int row = paired(P.epi) ? base + (fr & 7) + (fr >> 3) * 32 : min(base + fr, P.N - 1);
  const unsigned roff = (unsigned)row * (unsigned)P.ldw;
#pragma unroll
  for (int j = 0; j < XKS; ++j) {
    const int ks = min(ks0 + min(pass * XKS + j, max(kcnt - 1, 0)), nks - 1);
    r.fw[j] = ldg8(P.w + (roff + (unsigned)min(ks * 32 + fk, P.K - 8)));
  }
}

// Activation fragments of row block rb for pass `pass` (+ the fused norm:
// gain applied, row sums of squares accumulated); k past K reads as zero.
__device__ __forceinline__ void load_x(const XPhase& P, int rb, int pass, GemmRegs& r) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  int ks0, kcnt, per;
  wave_krange(P.K, wave, ks0, kcnt, per);
  const int nks = (P.K + 31) / 32;
  const int j0 = pass * XKS;
  unsigned rows[4];
#pragma unroll
  for (int tm = 0; tm < 4; ++tm) rows[tm] = (unsigned)min(rb * XBM + tm * 16 + fr, P.M - 1);
  if (P.a_f32) {
    // fp32 A (the Euler state into action_in, K <= 32: one k-step, wave 0),
    // rounded to bf16 on the way in
#pragma unroll
    for (int j = 0; j < XKS; ++j)
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) r.fx[j][tm] = bf16x8{};
    if (kcnt > 0 && pass == 0) {
      const int k = ks0 * 32 + fk;
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        const float* src = static_cast<const float*>(P.a) + (rows[tm] * (unsigned)P.lda + (unsigned)min(k, P.K - 8));
        const f32x4 lo = ldgf4(src);
        const f32x4 hi = ldgf4(src + 4);
        bf16x8 t;
#pragma unroll
        for (int i = 0; i < 4; ++i) { t[i] = f2bf(lo[i]); t[4 + i] = f2bf(hi[i]); }
        r.fx[0][tm] = k < P.K ? t : bf16x8{};
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < XKS; ++j) {
      const int k = min(ks0 + min(j0 + j, max(kcnt - 1, 0)), nks - 1) * 32 + fk;
      const int kc = min(k, P.K - 8);
#pragma unroll
      for (int tm = 0; tm < 4; ++tm) {
        const bf16x8 t = ldg8(static_cast<const bf16*>(P.a) + (rows[tm] * (unsigned)P.lda + (unsigned)kc));
        r.fx[j][tm] = k < P.K ? t : bf16x8{};
      }
    }
  }
  if (P.norm_w) {
#pragma unroll
    for (int j = 0; j < XKS; ++j) {
      if (j0 + j >= kcnt) continue;  // wave-uniform
      const int k = (ks0 + j0 + j) * 32 + fk;
      const bf16x8 gv = ldg8(P.norm_w + min(k, P.K - 8));
#pragma unroll
      for (int tm = 0; tm < 4; ++tm)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float xv = bf2f(r.fx[j][tm][e]);
          r.ss[tm] = __builtin_fmaf(xv, xv, r.ss[tm]);
          r.fx[j][tm][e] = f2bf(__fmul_rn(xv, bf2f(gv[e])));
        }
    }
  }
}

struct XShared {
  float part[XW][XBM * XPS];  // partial tiles of the 8 waves
  float ss[XW][XBM];          // per-wave row sums of squares
  float rs[XBM];              // row scale 1 / rms
  bf16 vt[XBM][XVT];          // attention: V^T of one head group, [d][key]
  int rank;
};

template <int ACT>
__device__ __forceinline__ float xact(float v) {
  if constexpr (ACT == SVLA_ACT_SILU) return silu_f(v);
  else if constexpr (ACT == SVLA_ACT_GELU_TANH) return gelu_tanh_f(v);
  else return v;
}

// The epilogue of one unit (partial tiles already in LDS): sums the 8 waves'
// tiles in wave order and stores through to memory.
__device__ void gemm_epilogue(const XPhase& P, int rb, int ct, XShared& sh) {
  const int tid = threadIdx.x;
  const int base = tile_base(P, ct);
  const bool pr = paired(P.epi);
  const int groups = pr ? XBM * 2 : XBM * (XBN / 4);
  if (tid >= groups) return;
  const int ml = pr ? tid >> 1 : tid >> 2;
  const int gi = pr ? tid & 1 : tid & 3;
  const int m = rb * XBM + ml;
  if (m >= P.M) return;
  auto sum4 = [&](int nl, float v[4]) {
    f32x4 t = *reinterpret_cast<const f32x4*>(&sh.part[0][ml * XPS + nl]);
#pragma unroll
    for (int w = 1; w < XW; ++w) t += *reinterpret_cast<const f32x4*>(&sh.part[w][ml * XPS + nl]);
    const float sc = P.norm_w ? sh.rs[ml] : 1.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = t[i] * sc;
  };
  if (P.epi == XE_STORE) {
    const int n = base + gi * 4;
    if (n >= P.N) return;
    float v[4];
    sum4(gi * 4, v);
    if (P.bias) {
      const bf16x4 b = ldg4(P.bias + n);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += bf2f(b[i]);
    }
    if (P.bias_f32) {
      const f32x4 b = ldgf4(P.bias_f32 + n);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] += b[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = rbf(v[i]);
    if (P.act == SVLA_ACT_SILU) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(xact<SVLA_ACT_SILU>(v[i]));
    }
    if (P.res) {
      const bf16x4 r = ldg4(P.res + (long)m * P.ldr + n);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(v[i] + bf2f(r[i]));
    }
    st4_wt(static_cast<bf16*>(P.c) + (long)m * P.ldc + n, v);
  } else if (P.epi == XE_ROPE) {
    // rotate-half RoPE on the bf16 projection in fp32 (vla/text_encoder_bf16.py:92-104);
    // columns past rope_cols (V) are stored as projected
    const int n = base + gi * 4;
    float x1[4], x2[4];
    sum4(gi * 4, x1);
    sum4(8 + gi * 4, x2);
    float o1[4], o2[4];
    if (n < P.rope_cols) {
      const int pos = m % P.rope_period, d = n & 63;
      const f32x4 c = ldgf4(P.cos_t + pos * 32 + d);
      const f32x4 s = ldgf4(P.sin_t + pos * 32 + d);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = rbf(x1[i]), b = rbf(x2[i]);
        o1[i] = __fsub_rn(__fmul_rn(a, c[i]), __fmul_rn(b, s[i]));
        o2[i] = __fadd_rn(__fmul_rn(b, c[i]), __fmul_rn(a, s[i]));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) { o1[i] = rbf(x1[i]); o2[i] = rbf(x2[i]); }
    }
    bf16* crow = static_cast<bf16*>(P.c) + (long)m * P.ldc;
    st4_wt(crow + n, o1);
    st4_wt(crow + n + 32, o2);
  } else if (P.epi == XE_SILU) {
    // bf16(silu(bf16(gate))) * bf16(up), output column (n / 64) * 32 + n % 64
    // (vla/text_encoder_bf16.py:130-131)
    const int n = base + gi * 4;
    float g[4], u[4], o[4];
    sum4(gi * 4, g);
    sum4(8 + gi * 4, u);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = rbf(silu_f(rbf(g[i]))) * rbf(u[i]);
    st4_wt(static_cast<bf16*>(P.c) + (long)m * P.ldc + (n >> 6) * 32 + (n & 63), o);
  } else {
    // Euler: x_out = x_in + dt * bf16(v) in fp32
    const int n = base + gi * 4;
    if (n >= P.N) return;
    float v[4];
    sum4(gi * 4, v);
    const f32x4 x = ldgf4(P.x_in + (long)m * P.N + n);
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __fadd_rn(x[i], __fmul_rn(P.dt, rbf(v[i])));
    st2f_wt(P.x_out + (long)m * P.N + n, o[0], o[1]);
    st2f_wt(P.x_out + (long)m * P.N + n + 2, o[2], o[3]);
  }
}

// acc += this pass's weight and activation fragments
__device__ __forceinline__ void gemm_mma(const XPhase& P, const GemmRegs& r, int pass, f32x4 (&acc)[4]) {
  const int wave = wave_id();
  int ks0, kcnt, per;
  wave_krange(P.K, wave, ks0, kcnt, per);
#pragma unroll
  for (int j = 0; j < XKS; ++j) {
    if (pass * XKS + j >= kcnt) break;  // wave-uniform
#pragma unroll
    for (int tm = 0; tm < 4; ++tm)
      acc[tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.fw[j], r.fx[j][tm], acc[tm], 0, 0, 0);
  }
}

// partial tile of this wave: element (row tm*16 + fr, columns 4*(lane/16) .. +3)
__device__ __forceinline__ void put_partial(const f32x4 (&acc)[4], XShared& sh) {
  const int lane = threadIdx.x & 63, wave = wave_id();
  const int fr = lane & 15;
#pragma unroll
  for (int tm = 0; tm < 4; ++tm)
    *reinterpret_cast<f32x4*>(&sh.part[wave][(tm * 16 + fr) * XPS + 4 * (lane >> 4)]) = acc[tm];
}

// ---- attention units -----------------------------------------------------------
// One (sample, head): queries on waves 0..3 (16 each), all 8 waves stage V^T.
__device__ void attn_unit(const XPhase& P, int unit, XShared& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
  const int b = unit / P.heads, h = unit - b * P.heads;
  const int g = h * P.kv_heads / P.heads;
  const bf16* kb = P.k + b * P.k_bs + g * 64;
  const bf16* vb = P.v + b * P.v_bs + g * 64;
  const bf16* qb = P.q + b * P.q_bs + h * 64;
  const int Lk = P.lk, Lq = P.lq;
  // V^T into LDS: [d][key], keys >= Lk zero
  for (int idx = tid; idx < XMAXK * 8; idx += XT) {
    const int key = idx >> 3, d8 = (idx & 7) * 8;
    bf16x8 val = bf16x8{};
    if (key < Lk) val = ldg8(vb + (long)key * P.ldv + d8);
#pragma unroll
    for (int j = 0; j < 8; ++j) sh.vt[d8 + j][key] = val[j];
  }
  wg_sync_lds();
  if (wave >= 4) return;
  const int G = lane >> 4, col = lane & 15;
  const int q0 = wave * 16;
  const int qi = q0 + col;
  const int qc = min(qi, Lq - 1);
  bf16x8 qf[2];
#pragma unroll
  for (int ds = 0; ds < 2; ++ds) qf[ds] = ldg8(qb + (long)qc * P.ldq + ds * 32 + G * 8);
  const int nkt = (Lk + 15) / 16;
  // S^T tiles: lane holds scores of keys kt*16 + 4G + i for query qi
  f32x4 s[XMAXK / 16];
#pragma unroll
  for (int kt = 0; kt < XMAXK / 16; ++kt) {
    s[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (kt >= nkt) continue;  // wave-uniform
    const int key = min(kt * 16 + col, Lk - 1);
#pragma unroll
    for (int ds = 0; ds < 2; ++ds) {
      const bf16x8 kf = ldg8(kb + (long)key * P.ldk + ds * 32 + G * 8);
      s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ds], s[kt], 0, 0, 0);
    }
  }
  // exact softmax in fp32 over the visible keys
  float mx = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < XMAXK / 16; ++kt) {
    if (kt >= nkt) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kt * 16 + 4 * G + i;
      const bool vis = key < Lk && !(P.causal && key > qc);
      s[kt][i] = vis ? s[kt][i] * P.scale : -INFINITY;
      mx = fmaxf(mx, s[kt][i]);
    }
  }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  float sum = 0.f;
#pragma unroll
  for (int kt = 0; kt < XMAXK / 16; ++kt) {
    if (kt >= nkt) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = s[kt][i] == -INFINITY ? 0.f : expf(s[kt][i] - mx);
      s[kt][i] = e;
      sum += e;
    }
  }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);
  const float inv = 1.0f / sum;
  // O^T = V^T . P^T over 32-key steps; contraction index 8G + j <-> key
  // 32 ks + 16 (j / 4) + 4 G + j % 4 (both operands)
  f32x4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < XMAXK / 32; ++ks) {
    if (2 * ks >= nkt) continue;  // wave-uniform
    bf16x8 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pf[i] = f2bf(s[2 * ks][i] / sum);
      pf[4 + i] = f2bf(s[2 * ks + 1][i] / sum);
    }
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int d = dt * 16 + col;
      const uint64_t lo = *reinterpret_cast<const uint64_t*>(&sh.vt[d][32 * ks + 4 * G]);
      const uint64_t hi = *reinterpret_cast<const uint64_t*>(&sh.vt[d][32 * ks + 16 + 4 * G]);
      const u32x4 w4 = {(uint32_t)lo, (uint32_t)(lo >> 32), (uint32_t)hi, (uint32_t)(hi >> 32)};
      const bf16x8 vf = __builtin_bit_cast(bf16x8, w4);
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[dt], 0, 0, 0);
    }
  }
  (void)inv;
  if (qi < Lq) {
    bf16* orow = P.o + b * P.o_bs + (long)qi * P.ldo + h * 64;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      float r[4] = {o[dt][0], o[dt][1], o[dt][2], o[dt][3]};
      st4_wt(orow + dt * 16 + 4 * G, r);
    }
  }
}

// ---- the persistent kernel -------------------------------------------------------
__global__ __launch_bounds__(XT, 1) void expert_kernel(XArgs g) {
  __shared__ XShared sh;
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
    sh.rank = rank;
  }
  __syncthreads();
  const int rank = sh.rank;
  if (rank < 0) return;
  const int team = g.team_xcd >= 0 ? g.team_size : (int)gridDim.x;
  if (g.team_xcd >= 0) {
    if (wave == 0) {
      // every member registered before anyone relies on the team's size
      const unsigned* reg = g.cnt + (size_t)g.n_ph * kSub * kCntStride;
      bool ok = false;
      for (int n = 0; n < kSpin; ++n) {
        const unsigned r = __builtin_amdgcn_readfirstlane(ld_agent(reg));
        if (r >= (unsigned)team) { ok = true; break; }
        if (__builtin_amdgcn_readfirstlane(ld_agent(g.status)) != 0u) break;
      }
      if (!ok && lane == 0)
        __hip_atomic_store(g.status, (unsigned)XS_TEAM, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 0) sh.rank = ok ? rank : -1;
    }
    __syncthreads();
    if (sh.rank < 0) return;
  }

  for (int p = 0; p < g.n_ph; ++p) {
    const XPhase& P = g.ph[p];
    const int units = P.units;
    if (rank >= units) continue;
    GemmRegs r;
    const int mine = (units - rank + team - 1) / team;
    const bool gemm = P.kind == XK_GEMM;
    // weights of the first unit before the wait (they do not depend on it)
    if (gemm) load_w(P, rank % P.col_tiles, 0, r);
    if (p > 0) {
      if (wave == 0) {
        const bool ok = wait_phase(g, p - 1, (unsigned)g.ph[p - 1].units);
        if (lane == 0) sh.rank = ok ? rank : -1;
      }
      __syncthreads();
      if (sh.rank < 0) return;
    }
    if (gemm) {
      const int npass = n_passes(P.K);
      int rb_loaded = -1;
      for (int j = 0; j < mine; ++j) {
        const int u = rank + j * team;
        const int rb = u / P.col_tiles, ct = u - rb * P.col_tiles;
        f32x4 acc[4];
#pragma unroll
        for (int tm = 0; tm < 4; ++tm) acc[tm] = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int pass = 0; pass < npass; ++pass) {
          if (pass > 0) load_w(P, ct, pass, r);
          // activations stay in registers across the units of a row block
          // when one pass covers K
          if (npass > 1 || rb != rb_loaded) {
            if (pass == 0) {
#pragma unroll
              for (int tm = 0; tm < 4; ++tm) r.ss[tm] = 0.f;
            }
            load_x(P, rb, pass, r);
            rb_loaded = rb;
          }
          gemm_mma(P, r, pass, acc);
        }
        // the next unit's first weights load during this unit's epilogue
        if (j + 1 < mine) load_w(P, (u + team) % P.col_tiles, 0, r);
        put_partial(acc, sh);
        if (P.norm_w) {
          // per-row sums of squares of the whole K range meet in LDS
#pragma unroll
          for (int tm = 0; tm < 4; ++tm) {
            float t = r.ss[tm];
            t += __shfl_xor(t, 16, 64);
            t += __shfl_xor(t, 32, 64);
            if (lane < 16) sh.ss[wave][tm * 16 + lane] = t;
          }
          wg_sync_lds();
          if (tid < XBM) {
            float t = 0.f;
#pragma unroll
            for (int w = 0; w < XW; ++w) t += sh.ss[w][tid];
            sh.rs[tid] = 1.0f / sqrtf(t / (float)P.K + P.norm_eps);
          }
        }
        wg_sync_lds();
        gemm_epilogue(P, rb, ct, sh);
        wg_sync_lds();  // partial tiles free for the next unit
      }
    } else {
      for (int j = 0; j < mine; ++j) {
        attn_unit(P, rank + j * team, sh);
        wg_sync_lds();  // V^T free for the next unit
      }
    }
    // every store of this workgroup acknowledged, then one arrival
    __builtin_amdgcn_s_waitcnt(wc_vm(0));
    __syncthreads();
    if (tid == 0)
      __hip_atomic_fetch_add(g.cnt + ((size_t)p * kSub + (rank & (kSub - 1))) * kCntStride,
                             (unsigned)mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
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

int count_phases(const svla_expert_desc* d) { return d->num_steps * (4 + 5 * d->n_layers); }

bool desc_ok(const svla_expert_desc* d) {
  if (!d || d->batch <= 0 || d->chunk <= 0 || d->chunk > XMAXQ || d->head_dim != 64) return false;
  if (d->hidden % 16 || d->inter % 32 || d->action_dim % 16 || d->n_layers <= 0) return false;
  if (d->hidden > XKS * XPASS * XW * 32 || d->inter > XKS * XPASS * XW * 32) return false;
  if (d->n_q_heads <= 0 || d->n_kv_heads <= 0 || d->n_q_heads % d->n_kv_heads) return false;
  if (d->n_q_heads * 64 > XKS * XPASS * XW * 32) return false;
  if (d->num_steps <= 0 || d->prefix_len <= 0 || d->prefix_len > XMAXK) return false;
  if (!d->layers || !d->w_action_in || !d->w_time_in_a || !d->time_bias || !d->w_time_out ||
      !d->w_action_out || !d->rope_cos || !d->rope_sin)
    return false;
  for (int l = 0; l < d->n_layers; ++l) {
    const svla_expert_layer& L = d->layers[l];
    if (!L.w_qkv || !L.w_o || !L.w_gu || !L.w_down || !L.norm1 || !L.norm2) return false;
    if (L.cross && (!L.cross_k || !L.cross_v)) return false;
  }
  return true;
}

// Builds the phase list (and, with base != nullptr, the buffer addresses).
size_t build(const svla_expert_desc* d, char* base, std::vector<XPhase>* out, Layout* lay) {
  const int M = d->batch * d->chunk, H = d->hidden, qd = d->n_q_heads * 64,
            kvd = d->n_kv_heads * 64, I = d->inter, A = d->action_dim;
  const int rbs = (M + XBM - 1) / XBM;
  Layout L{};
  L.n_ph = count_phases(d);
  L.n_cnt_words = (size_t)(L.n_ph + 1) * kSub * kCntStride;
  Arena ar;
  L.phases = ar.take(sizeof(XPhase) * L.n_ph);
  L.counters = ar.take(L.n_cnt_words * 4);
  L.status = ar.take(4);
  L.arena = ar.off;
  auto buf = [&](size_t bytes) -> char* {
    const size_t o = ar.take(bytes);
    return base ? base + o : nullptr;
  };
  auto gemm = [&](const void* a, int lda, const void* w, int N, int K, void* c, int ldc) {
    XPhase P{};
    P.kind = XK_GEMM;
    P.epi = XE_STORE;
    P.M = M; P.N = N; P.K = K;
    P.col_tiles = (N + XBN - 1) / XBN;
    P.units = rbs * P.col_tiles;
    P.a = a; P.lda = lda;
    P.w = static_cast<const bf16*>(w); P.ldw = K;
    P.c = c; P.ldc = ldc;
    P.norm_eps = d->rms_eps;
    return P;
  };
  std::vector<XPhase> ph;
  const float* x_prev = d->x_in;
  for (int s = 0; s < d->num_steps; ++s) {
    // action / time embedding (the time part of time_in precomputed per step)
    bf16* a_emb = (bf16*)buf((size_t)M * H * 2);
    XPhase P = gemm(x_prev, A, d->w_action_in, H, A, a_emb, H);
    P.a_f32 = 1;
    P.bias = static_cast<const bf16*>(d->b_action_in);
    ph.push_back(P);
    bf16* h_t = (bf16*)buf((size_t)M * H * 2);
    P = gemm(a_emb, H, d->w_time_in_a, H, H, h_t, H);
    P.bias_f32 = d->time_bias + (size_t)s * H;
    P.act = SVLA_ACT_SILU;
    ph.push_back(P);
    bf16* ex = (bf16*)buf((size_t)M * H * 2);
    P = gemm(h_t, H, d->w_time_out, H, H, ex, H);
    P.bias = static_cast<const bf16*>(d->b_time_out);
    ph.push_back(P);
    for (int l = 0; l < d->n_layers; ++l) {
      const svla_expert_layer& Ly = d->layers[l];
      const int nq = Ly.cross ? qd : qd + 2 * kvd;
      bf16* qkv = (bf16*)buf((size_t)M * nq * 2);
      P = gemm(ex, H, Ly.w_qkv, nq, H, qkv, nq);
      P.epi = XE_ROPE;
      P.norm_w = static_cast<const bf16*>(Ly.norm1);
      P.cos_t = d->rope_cos; P.sin_t = d->rope_sin;
      P.rope_cols = Ly.cross ? qd : qd + kvd;
      P.rope_period = d->chunk;
      ph.push_back(P);
      bf16* att = (bf16*)buf((size_t)M * qd * 2);
      XPhase T{};
      T.kind = XK_ATTN;
      T.units = d->batch * d->n_q_heads;
      T.heads = d->n_q_heads; T.kv_heads = d->n_kv_heads;
      T.lq = d->chunk;
      T.scale = 0.125f;
      T.q = qkv; T.ldq = nq; T.q_bs = (long)d->chunk * nq;
      if (Ly.cross) {
        T.k = static_cast<const bf16*>(Ly.cross_k); T.ldk = d->ld_cross;
        T.v = static_cast<const bf16*>(Ly.cross_v); T.ldv = d->ld_cross;
        T.k_bs = T.v_bs = (long)d->prefix_len * d->ld_cross;
        T.lk = d->prefix_len;
        T.causal = 0;
      } else {
        T.k = qkv + qd; T.ldk = nq;
        T.v = qkv + qd + kvd; T.ldv = nq;
        T.k_bs = T.v_bs = (long)d->chunk * nq;
        T.lk = d->chunk;
        T.causal = 1;
      }
      T.o = att; T.ldo = qd; T.o_bs = (long)d->chunk * qd;
      ph.push_back(T);
      bf16* ex1 = (bf16*)buf((size_t)M * H * 2);
      P = gemm(att, qd, Ly.w_o, H, qd, ex1, H);
      P.res = ex; P.ldr = H;
      ph.push_back(P);
      bf16* act = (bf16*)buf((size_t)M * I * 2);
      P = gemm(ex1, H, Ly.w_gu, 2 * I, H, act, I);
      P.epi = XE_SILU;
      P.norm_w = static_cast<const bf16*>(Ly.norm2);
      ph.push_back(P);
      bf16* ex2 = (bf16*)buf((size_t)M * H * 2);
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

int svla_expert_prepare(const svla_expert_desc* d, void* ws, long ws_bytes, int team_xcd,
                        svla_expert_plan* plan, svla_stream_t stream) {
  if (!desc_ok(d) || !ws || !plan || ((uintptr_t)ws % kAlign) || team_xcd > 7) return SVLA_EINVAL;
  if (!d->x_in || !d->x_out || ((uintptr_t)d->x_in & 15) || ((uintptr_t)d->x_out & 15))
    return SVLA_EINVAL;
  std::vector<XPhase> ph;
  Layout L{};
  if (ws_bytes < 0 || build(d, static_cast<char*>(ws), &ph, &L) > (size_t)ws_bytes) return SVLA_EINVAL;
  char* base = static_cast<char*>(ws);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipMemcpyAsync(base + L.phases, ph.data(), sizeof(XPhase) * ph.size(),
                                hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return (int)e;
  e = hipStreamSynchronize(s);
  if (e != hipSuccess) return (int)e;
  int dev = 0, cus = 0;
  if ((e = hipGetDevice(&dev)) != hipSuccess) return (int)e;
  if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess)
    return (int)e;
  std::memset(plan, 0, sizeof(*plan));
  plan->phases = base + L.phases;
  plan->n_phases = L.n_ph;
  plan->counters = reinterpret_cast<unsigned*>(base + L.counters);
  plan->counter_words = (long)L.n_cnt_words;
  plan->status = reinterpret_cast<unsigned*>(base + L.status);
  plan->grid = cus;
  plan->team_xcd = team_xcd < 0 ? -1 : team_xcd;
  plan->team_size = team_xcd < 0 ? cus : cus / 8;
  return SVLA_OK;
}

int svla_expert_run(const svla_expert_plan* plan, svla_stream_t stream) {
  if (!plan || !plan->phases || plan->n_phases <= 0 || plan->grid <= 0) return SVLA_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  const long words = plan->counter_words + kAlign / 4;  // counters, then the status word
  hipLaunchKernelGGL(clear_u32_kernel, dim3(256), dim3(256), 0, s, plan->counters, words);
  SVLA_CHECK_LAUNCH();
  XArgs g;
  g.ph = static_cast<const XPhase*>(plan->phases);
  g.n_ph = plan->n_phases;
  g.cnt = plan->counters;
  g.status = plan->status;
  g.team_xcd = plan->team_xcd;
  g.team_size = plan->team_size;
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
