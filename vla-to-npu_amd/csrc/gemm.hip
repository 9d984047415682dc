// bf16 MFMA GEMM for gfx950 with fused prologues and epilogues.
//
//   C[M, N] = epilogue(alpha * norm(A)[M, K] . W[N, K]^T)
//
// Replaces the Allo GEMM region (cc/gemm.py:44-77, instantiated e.g. at
// vla/text_encoder_bf16.py:174-225), the host-side K-chunk accumulation
// loops (vla/text_encoder_bf16.py:584-590, vla/connector_bf16.py:116-126),
// the RMSNorm in front of every projection (vla/text_encoder_bf16.py:398-404)
// and the elementwise kernels behind them (RoPE, SiLU*up, GELU, residual add).
//
// Design (CDNA4):
//  * 256 threads = 4 wave64s per workgroup, block tile BM x BN, K step 64.
//    Large problems use 256x256 tiles (each wave 128x128 with
//    v_mfma_f32_32x32x16_bf16: 64 FLOP per LDS byte) at one workgroup per CU;
//    mid-size problems 128x128 / 64x128 / 64x64 tiles.
//  * Skinny-M problems (the bs=1 prefix and expert: M = 50 .. 241 rows) use a
//    separate kernel: 64-row tiles whose K loop is split over the 4 waves of
//    the workgroup, MFMA operand fragments loaded straight from global memory
//    (A and W are both K-contiguous, so a fragment is one 16-byte load per
//    lane), the 4 partial tiles summed through LDS.  This gives split-K
//    parallelism without any cross-workgroup reduction, workspace or atomics.
//  * Global -> register prefetch of the next K tile while the current one is
//    consumed from LDS; LDS double buffer, one barrier per K step.  LDS rows are
//    padded by 16 bytes so the 16-byte operand reads of 8 consecutive rows hit
//    distinct bank groups.
//  * The WEIGHT tile is the MFMA A operand and the activation tile the B
//    operand, so every lane's accumulator holds runs of 4 consecutive output
//    COLUMNS of one row: the epilogues (bias, RoPE pairs (d, d+32), SiLU(gate)
//    * up pairs (gate/up interleaved in blocks of 32 rows, so the partner is
//    always 32 packed columns away), residual) are lane-local, and stores are
//    8-byte vectors.
//  * A-operand gathers: the pixel-shuffle of the connector and the im2col of
//    the patch embedding are folded into the A-tile addressing; optionally the
//    A rows are RMS-normalised on the fly (per-row statistics computed in a
//    prologue, the tile scaled when it is written to LDS), which removes every
//    standalone RMSNorm launch of the decoder / expert layers.
//  * Workgroup ids are remapped so consecutive tiles land on the same XCD
//    (the hardware deals workgroups round-robin over the 8 XCDs, each with its
//    own L2): neighbouring tiles share A rows in that XCD's L2.
#include <mutex>

#include "svla_common.h"

namespace {

enum AMode { A_DENSE = 0, A_PSHUF = 1, A_PATCH = 2 };
enum Epi { EPI_STORE = 0, EPI_ROPE = 1, EPI_SILU = 2, EPI_EULER = 3 };

struct GemmArgs {
  const bf16* a;
  long lda;
  // A_PSHUF: source [n_img, grid*grid, hidden], shuffle factor `scale`
  int g_grid, g_hidden, g_scale;
  // A_PATCH: images [n_img, chans, img, img], patch size
  int p_chans, p_img, p_patch;
  const bf16* b;
  long ldb;
  void* c;
  long ldc;
  int M, N, K;
  float alpha;
  const bf16* bias;
  const float* bias_f32;
  const bf16* res;
  long ldr;
  const bf16* rowadd;  // added after rounding: rowadd[(m % rowadd_period) * N + n]
  int rowadd_period;
  int out_f32;
  const float* rope_cos;
  const float* rope_sin;
  int rope_cols;
  int rope_period;
  bf16* c_lo;  // ROPE (optional): o - bf16(o) of every rotated column, layout of c
  float* x_f32;
  long ldx;
  bf16* x_bf16;
  long ldxb;
  float dt;
  // output row remap: row m is stored at (m / c_rpg) * c_gstride + m % c_rpg
  // (c_rpg == 0: identity).  Lets the connector write each sample's image
  // tokens straight into its slot of the [B, prefix_len, H] prefix buffer.
  int c_rpg;
  long c_gstride;
  // fused RMSNorm of the A rows: a = bf16((x * r) * w[k]), r = 1 / sqrt(mean(x^2) + eps)
  const bf16* norm_w;
  float norm_eps;
  // skinny split-K (gridDim.z > 1): fp32 partial tiles [tile][split][BM * BN]
  // and one arrival counter per output tile (zero between calls)
  float* ws;
  unsigned* ws_cnt;
  // persistent wide kernel: the tile grid (its launch grid is one workgroup per
  // CU); w_cn > 0: each XCD keeps w_cn column blocks (see xcd_tile), else the
  // grouped order of tile_coords
  int tiles_m, tiles_n, w_cn;
  // slab-blocked operands / output of the wide kernel: element (row, k) of a
  // blocked [rows, K] matrix sits at (k / 32) * rows * 32 + row * 32 + k % 32,
  // so the 16 rows x 32 columns an LDS-DMA instruction fetches are one
  // contiguous kilobyte (the row-major layout gives 16 separate 64-byte pieces)
  int a_blk, b_blk, c_blk;
};

__device__ __forceinline__ long crow(const GemmArgs& p, int m) {
  if (p.c_rpg <= 0) return m;
  const int g = m / p.c_rpg;
  return (long)g * p.c_gstride + (m - g * p.c_rpg);
}

template <int ACT>
__device__ __forceinline__ float apply_act(float v) {
  if constexpr (ACT == SVLA_ACT_GELU_TANH) return gelu_tanh_f(v);
  else if constexpr (ACT == SVLA_ACT_GELU_ERF) return gelu_erf_f(v);
  else if constexpr (ACT == SVLA_ACT_SILU) return silu_f(v);
  else return v;
}

__device__ __forceinline__ void store_bf16x4(bf16* dst, const float v[4]) {
  bf16x4 o;
  o[0] = f2bf(v[0]); o[1] = f2bf(v[1]); o[2] = f2bf(v[2]); o[3] = f2bf(v[3]);
  *reinterpret_cast<bf16x4*>(dst) = o;
}

__device__ __forceinline__ void load_bf16x4(const bf16* src, float v[4]) {
  bf16x4 t = *reinterpret_cast<const bf16x4*>(src);
  v[0] = bf2f(t[0]); v[1] = bf2f(t[1]); v[2] = bf2f(t[2]); v[3] = bf2f(t[3]);
}

// ---- epilogues: 4 consecutive (packed) columns of one row ------------------
// Split in two so that a kernel issues the loads of a whole column tile's
// output groups before its first store: epi_load_groups reads the optional
// operands (bias, residual, position addend, RoPE tables, Euler state) of G
// groups -- one uniform branch region per optional operand, holding that
// operand's loads for all G groups, so they are in flight together -- and
// epi_apply blends them in and stores one group.  (A residual may alias the
// output, so a load issued after an earlier group's store could not be
// hoisted above it; and a region per group and operand would end each one
// with a full vmcnt(0) drain: either way the loads would run one by one.)
struct EpiIn {
  f32x4 u, w;      // fp32 bias | RoPE cos, sin | Euler x
  bf16x4 b, r, a;  // bf16 bias, residual, row-periodic addend
};

// m, n: each group's (row, first column), clamped into range by the caller
template <int EPI, int G>
__device__ __forceinline__ void epi_load_groups(const GemmArgs& p, const int (&m)[G],
                                                const int (&n)[G], EpiIn (&e)[G]) {
  if constexpr (EPI == EPI_STORE) {
    if (p.bias) {
#pragma unroll
      for (int g = 0; g < G; ++g) e[g].b = *reinterpret_cast<const bf16x4*>(p.bias + n[g]);
    }
    if (p.bias_f32) {
#pragma unroll
      for (int g = 0; g < G; ++g) e[g].u = *reinterpret_cast<const f32x4*>(p.bias_f32 + n[g]);
    }
    if (p.res) {
#pragma unroll
      for (int g = 0; g < G; ++g)
        e[g].r = *reinterpret_cast<const bf16x4*>(p.res + (long)m[g] * p.ldr + n[g]);
    }
    if (p.rowadd) {  // patch embedding's position table
#pragma unroll
      for (int g = 0; g < G; ++g)
        e[g].a = *reinterpret_cast<const bf16x4*>(p.rowadd + (long)(m[g] % p.rowadd_period) * p.N + n[g]);
    }
  } else if constexpr (EPI == EPI_ROPE) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int pos = m[g] % p.rope_period;
      const int d = n[g] & 63;  // < 32: n is in the first half of its 64-column block
      e[g].u = *reinterpret_cast<const f32x4*>(p.rope_cos + pos * 32 + d);
      e[g].w = *reinterpret_cast<const f32x4*>(p.rope_sin + pos * 32 + d);
    }
  } else if constexpr (EPI == EPI_EULER) {
#pragma unroll
    for (int g = 0; g < G; ++g)
      e[g].u = *reinterpret_cast<const f32x4*>(p.x_f32 + (long)m[g] * p.ldx + n[g]);
  }
}

// v (x1) = this group's 4 accumulators (times alpha); x2 = the paired group
// 32 columns on (RoPE / SiLU epilogues only).
template <int EPI, int ACT>
__device__ __forceinline__ void epi_apply(const GemmArgs& p, int m, int n, float* v, float* x2,
                                          const EpiIn& e) {
  if constexpr (EPI == EPI_STORE) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (p.bias) v[i] += bf2f(e.b[i]);
      if (p.bias_f32) v[i] += e.u[i];
    }
    if (p.out_f32) {
      float* dst = reinterpret_cast<float*>(p.c) + crow(p, m) * p.ldc + n;
      *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = rbf(v[i]);
    if constexpr (ACT != SVLA_ACT_NONE) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(apply_act<ACT>(v[i]));
    }
    if (p.rowadd) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(v[i] + bf2f(e.a[i]));
    }
    if (p.res) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = rbf(v[i] + bf2f(e.r[i]));
    }
    store_bf16x4(reinterpret_cast<bf16*>(p.c) + crow(p, m) * p.ldc + n, v);
  } else if constexpr (EPI == EPI_ROPE) {
    // mirrors apply_rope on the bf16 projection (vla/text_encoder_bf16.py:92-104):
    // out1 = x1*cos - x2*sin, out2 = x2*cos + x1*sin in fp32, then bf16;
    // columns past rope_cols (V) are stored unrotated
    bf16* c = reinterpret_cast<bf16*>(p.c) + crow(p, m) * p.ldc;
    const bool rot = n < p.rope_cols;
    float o1[4], o2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x1 = rbf(v[i]), y2 = rbf(x2[i]);
      const float r1 = __fsub_rn(__fmul_rn(x1, e.u[i]), __fmul_rn(y2, e.w[i]));
      const float r2 = __fadd_rn(__fmul_rn(y2, e.u[i]), __fmul_rn(x1, e.w[i]));
      o1[i] = rot ? r1 : x1;
      o2[i] = rot ? r2 : y2;
    }
    store_bf16x4(c + n, o1);
    store_bf16x4(c + n + 32, o2);
    if (p.c_lo && rot) {
      // the reference scores the fp32 RoPE output: keep what bf16 drops
      // (exact in fp32), so the attention can take Q = hi + lo
      float l1[4], l2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        l1[i] = __fsub_rn(o1[i], rbf(o1[i]));
        l2[i] = __fsub_rn(o2[i], rbf(o2[i]));
      }
      bf16* cl = p.c_lo + crow(p, m) * p.ldc;
      store_bf16x4(cl + n, l1);
      store_bf16x4(cl + n + 32, l2);
    }
  } else if constexpr (EPI == EPI_SILU) {
    // gate at packed column n (first half of a 64-block), up at n + 32; output
    // column (n / 64) * 32 + n % 64; out = bf16(bf16(silu(bf16(g))) * bf16(u))
    // (nn.SiLU on the bf16 gate projection, then the bf16 hadamard product,
    // vla/text_encoder_bf16.py:130-131)
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = rbf(silu_f(rbf(v[i]))) * rbf(x2[i]);
    const int nout = (n >> 6) * 32 + (n & 63);
    store_bf16x4(reinterpret_cast<bf16*>(p.c) + crow(p, m) * p.ldc + nout, o);
  } else {
    // Euler step x <- x + dt * bf16(v) in fp32 (+ optional bf16 copy of x)
    float o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = __fadd_rn(e.u[i], __fmul_rn(p.dt, rbf(v[i])));
    *reinterpret_cast<f32x4*>(p.x_f32 + (long)m * p.ldx + n) = f32x4{o[0], o[1], o[2], o[3]};
    if (p.x_bf16) store_bf16x4(p.x_bf16 + (long)m * p.ldxb + n, o);
  }
}

// ---- A operand gather -------------------------------------------------------
// Address of A[m][k .. k+7] for an in-range (m, k); no bounds checks, so
// callers can clamp (m, k) and issue the load without a branch.
template <int AMODE>
__device__ __forceinline__ const bf16* a_ptr(const GemmArgs& p, int m, int k) {
  if constexpr (AMODE == A_DENSE) {
    return p.a + (long)m * p.lda + k;
  } else if constexpr (AMODE == A_PSHUF) {
    // out[i][t*(s*E) + u*E + c] = x[(s*(i/gs) + t)*grid + s*(i%gs) + u][c]
    // with gs = grid/s (the reshape/transpose chain of vla/vla.py:435)
    const int s = p.g_scale, E = p.g_hidden, grid = p.g_grid;
    const int gs = grid / s;
    const int per = gs * gs;
    const int img = m / per, i = m - img * per;
    const int hp = i / gs, wp = i - hp * gs;
    const int sE = s * E;
    const int t = k / sE, rem = k - t * sE;
    const int u = rem / E, c = rem - u * E;
    const long tok = (long)(s * hp + t) * grid + s * wp + u;
    return p.a + ((long)img * grid * grid + tok) * E + c;
  } else {
    // im2col of Conv2d(k = stride = P): row = img*G*G + pr*G + pc,
    // col = ch*P*P + ky*P + kx (the conv weight's [E, C, P, P] flattening)
    const int P = p.p_patch, H = p.p_img, G = H / P;
    const int per = G * G;
    const int img = m / per, tkn = m - img * per;
    const int pr = tkn / G, pc = tkn - pr * G;
    const int P2 = P * P;
    const int ch = k / P2, r = k - ch * P2;
    const int ky = r / P, kx = r - ky * P;
    return p.a + (((long)img * p.p_chans + ch) * H + pr * P + ky) * H + pc * P + kx;
  }
}

template <int AMODE>
__device__ __forceinline__ bf16x8 load_a(const GemmArgs& p, int m, int k) {
  if (m >= p.M || k >= p.K) return bf16x8{};
  return ld8(a_ptr<AMODE>(p, m, k));
}

constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // elements; +16 bytes of padding per row
constexpr int kNumXCD = 8;

// Maps the hardware workgroup id so that consecutive logical tiles share an
// XCD (the hardware deals workgroups round-robin over the 8 XCDs).
__device__ __forceinline__ int xcd_remap(int bid, int total) {
  const int per = total / kNumXCD;
  const int full = per * kNumXCD;
  if (bid >= full) return bid;
  return (bid % kNumXCD) * per + bid / kNumXCD;
}

// Logical tile -> (row block, column block) in groups of kGroupRows row
// blocks: consecutive tiles walk down a group's rows, then across its
// columns, so the workgroups that run together on one XCD cover a compact
// rows x columns patch and share both their A row panels and their weight
// column panels in that XCD's L2.  (Row-major order makes a concurrent set
// span every column block, i.e. the whole weight matrix, which does not fit.)
constexpr int kGroupRows = 8;
__device__ __forceinline__ void tile_coords(int t, int gm, int gn, int& tm, int& tn) {
  const int per_group = kGroupRows * gn;
  const int group = t / per_group;
  const int first = group * kGroupRows;
  const int rows = min(gm - first, kGroupRows);
  const int r = t - group * per_group;
  tm = first + r % rows;
  tn = r / rows;
}

// Persistent wide kernel, column-resident order (w_cn > 0): the XCDs form
// tiles_n / w_cn column groups, and XCD x keeps the w_cn column blocks of its
// group (their weight panels stay in its L2 for the whole launch) and walks
// its own contiguous range of row blocks, i-th tile of the XCD = row block
// i / w_cn of the range, column i % w_cn of the group.  The 32 workgroups an
// XCD runs at once then read ~32 / w_cn fresh A slices per K step and weight
// slices that hit; the grouped order fetches both panels of a new patch at
// every round.
__device__ __forceinline__ int xcd_rows(const GemmArgs& p, int x, int& first) {
  const int xg = kNumXCD * p.w_cn / p.tiles_n;  // XCDs per column group
  const int rows = (p.tiles_m + xg - 1) / xg;
  first = (x % xg) * rows;
  return max(0, min(rows, p.tiles_m - first));
}
__device__ __forceinline__ void xcd_tile(const GemmArgs& p, int x, int i, int& tm, int& tn) {
  const int xg = kNumXCD * p.w_cn / p.tiles_n;
  int first;
  xcd_rows(p, x, first);
  tm = first + i / p.w_cn;
  tn = (x / xg) * p.w_cn + i % p.w_cn;
}

// Fused RMSNorm (NORM), row scales: s_r[r] = 1 / rms of A row m0 + r, r < R,
// computed before a kernel's main loop so that every operand element can then
// be rounded once, bf16((x * r) * w[k]), exactly as the standalone RMSNorm
// (rmsnorm_kernel) rounds its output; the accumulators need no row scale.
// The sum of squares is formed in the standalone kernel's own order, so r and
// with it every operand element are bit-identical to its: there one wave64
// per row, lane l summing chunks l, l + 64, l + 128, l + 192 (8 bf16 each) by
// fused multiply-adds, then a butterfly over xor 32, 16, 8, 4, 2, 1.  Here 8
// threads per row: thread t plays lanes t + 8 i (i = 0..7), so the levels
// xor 32, 16, 8 are local adds and xor 4, 2, 1 are shuffles.  One extra pass
// over the tile's A rows: its first touch brings them into L2 for the main
// loop; every 8 loads of a row are 128 contiguous bytes.  Rows past M are
// clamped (their outputs are never stored).  K <= 2048.  The caller's barrier
// publishes s_r.
template <int R, int NT>
__device__ __forceinline__ void norm_rows(const GemmArgs& p, int m0, float* s_r) {
  constexpr int RPP = NT / 8;                // rows per pass
  constexpr int NP = (R + RPP - 1) / RPP;    // passes: rows per thread
  constexpr int PG = NP <= 3 ? NP : 2;       // passes whose loads are in flight together
  static_assert(NP % PG == 0, "pass groups");
  const int t = threadIdx.x & 7;
  const int nj = (p.K + 511) / 512;
#pragma unroll
  for (int p0 = 0; p0 < NP; p0 += PG) {
    const bf16* x[PG];
    float v[PG][8];  // pass p0 + pp, lane t + 8 i's sum
#pragma unroll
    for (int pp = 0; pp < PG; ++pp) {
      x[pp] = p.a + (long)min(m0 + (p0 + pp) * RPP + (int)(threadIdx.x >> 3), p.M - 1) * p.lda;
#pragma unroll
      for (int i = 0; i < 8; ++i) v[pp][i] = 0.f;
    }
    // every load of a round is issued unconditionally from a clamped address
    // (a load under a branch ends its region with a full vmcnt drain) and a
    // chunk past K contributes fma(0, 0, v) = v, as the standalone kernel's
    // skipped chunk does
    for (int j = 0; j < nj; ++j) {
      bf16x8 q[PG][8];
#pragma unroll
      for (int pp = 0; pp < PG; ++pp)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          q[pp][i] = ld8(x[pp] + min((t + 8 * i + 64 * j) * 8, p.K - 8));
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool in = (t + 8 * i + 64 * j) * 8 < p.K;
#pragma unroll
        for (int pp = 0; pp < PG; ++pp)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float f = in ? bf2f(q[pp][i][e]) : 0.f;
            v[pp][i] = __builtin_fmaf(f, f, v[pp][i]);
          }
      }
    }
#pragma unroll
    for (int pp = 0; pp < PG; ++pp) {
      // lane bits 5, 4, 3 are i's bits 2, 1, 0
      const float u0 = (v[pp][0] + v[pp][4]) + (v[pp][2] + v[pp][6]);
      const float u1 = (v[pp][1] + v[pp][5]) + (v[pp][3] + v[pp][7]);
      float s = u0 + u1;
      s += __shfl_xor(s, 4, 64);
      s += __shfl_xor(s, 2, 64);
      s += __shfl_xor(s, 1, 64);
      const int r = (p0 + pp) * RPP + (int)(threadIdx.x >> 3);
      if (t == 0 && (R % RPP == 0 || r < R)) s_r[r] = 1.0f / sqrtf(s / (float)p.K + p.norm_eps);
    }
  }
}

// bf16((x * r) * w): one operand fragment of a normalised row (scale r, gain w)
__device__ __forceinline__ void norm_frag(bf16x8& x, float r, const bf16x8& w) {
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = f2bf(__fmul_rn(__fmul_rn(bf2f(x[j]), r), bf2f(w[j])));
}

template <int BM, int BN, int WAVES_M, int WAVES_N, int MF, int AMODE, bool NORM, int EPI,
          int ACT>
__global__ __launch_bounds__(256, (BM >= 256 ? 1 : 2)) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / MF, TN = WN / MF;
  constexpr int KSTEP = MF == 32 ? 16 : 32;      // K per MFMA
  constexpr int KFRAG = 8;                        // bf16 per lane per operand
  constexpr int LG = 64 / MF;                     // lane groups along K
  constexpr int A_CH = BM * BK / 8 / 256;
  constexpr int B_CH = BN * BK / 8 / 256;
  constexpr int PAIR_T = 32 / MF;                 // tile offset of the +32 column partner
  using acc_t = typename std::conditional<MF == 32, f32x16, f32x4>::type;
  constexpr int ACC_N = MF == 32 ? 16 : 4;
  static_assert(WAVES_M * WAVES_N == 4, "4 waves");
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small");
  static_assert(LG * KFRAG == KSTEP, "operand layout");
  static_assert((EPI != EPI_ROPE && EPI != EPI_SILU) || WN % 64 == 0,
                "paired epilogues need 64-column aligned wave tiles");
  static_assert(!NORM || AMODE == A_DENSE, "row norm only for dense A");

  __shared__ __attribute__((aligned(16))) bf16 sA[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) bf16 sB[2][BN * LDS_STRIDE];
  __shared__ float s_rs[NORM ? BM : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int gn = gridDim.x;
  const int tile = xcd_remap(blockIdx.y * gn + blockIdx.x, gn * gridDim.y);
  int tm_idx, tn_idx;
  tile_coords(tile, gridDim.y, gn, tm_idx, tn_idx);
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int kt_begin = 0;
  const int kt_end = (p.K + BK - 1) / BK;

  // Fused RMSNorm (NORM): row scales first (norm_rows), then each A chunk is
  // rounded as bf16((x * r) * w) on its way into LDS.
  if constexpr (NORM) {
    norm_rows<BM, 256>(p, m0, s_rs);
    __syncthreads();
  }

  acc_t acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j)
#pragma unroll
      for (int e = 0; e < ACC_N; ++e) acc[i][j][e] = 0.f;

  bf16x8 ra[A_CH], rb[B_CH];
  bf16x8 rw;  // norm gain for this thread's A k-chunk (the same for all its chunks)
  bool kin = true;  // this thread's k-chunk lies inside K (its column is the same in A and B)

  // Every load is issued unconditionally from a clamped address (rows past
  // M / N only feed outputs that are never stored); chunks past K are zeroed
  // when they are written to LDS.  Loads under a branch would each end their
  // own region with a full vmcnt(0) drain and serialise the prefetch.
  auto gload = [&](int kt) __attribute__((always_inline)) {
    const int kb = kt * BK;
    const int k = kb + (tid & 7) * 8;  // c & 7 == tid & 7 for every chunk c
    kin = k < p.K;
    const int kc = min(k, p.K - 8);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * 256;
      ra[i] = ld8(a_ptr<AMODE>(p, min(m0 + (c >> 3), p.M - 1), kc));
    }
    if constexpr (NORM) rw = ld8(p.norm_w + kc);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * 256;
      rb[i] = ld8(p.b + (long)min(n0 + (c >> 3), p.N - 1) * p.ldb + kc);
    }
  };
  auto sstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * 256;
      bf16x8 v = kin ? ra[i] : bf16x8{};
      if constexpr (NORM) norm_frag(v, s_rs[c >> 3], rw);
      *reinterpret_cast<bf16x8*>(&sA[buf][(c >> 3) * LDS_STRIDE + (c & 7) * 8]) = v;
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<bf16x8*>(&sB[buf][(c >> 3) * LDS_STRIDE + (c & 7) * 8]) =
          kin ? rb[i] : bf16x8{};
    }
  };

  const int frag_row = lane % MF;
  const int frag_k = (lane / MF) * KFRAG;

  if (kt_begin < kt_end) {
    gload(kt_begin);
    sstore(0);
    __syncthreads();
    for (int kt = kt_begin; kt < kt_end; ++kt) {
      const int cur = (kt - kt_begin) & 1;
      if (kt + 1 < kt_end) gload(kt + 1);
#pragma unroll
      for (int ks = 0; ks < BK / KSTEP; ++ks) {
        bf16x8 fw[TN], fx[TM];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          fw[tn] = *reinterpret_cast<const bf16x8*>(
              &sB[cur][(wn * WN + tn * MF + frag_row) * LDS_STRIDE + ks * KSTEP + frag_k]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          fx[tm] = *reinterpret_cast<const bf16x8*>(
              &sA[cur][(wm * WM + tm * MF + frag_row) * LDS_STRIDE + ks * KSTEP + frag_k]);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm) {
            if constexpr (MF == 32)
              acc[tn][tm] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fw[tn], fx[tm], acc[tn][tm],
                                                                    0, 0, 0);
            else
              acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[tn], fx[tm], acc[tn][tm],
                                                                    0, 0, 0);
          }
      }
      if (kt + 1 < kt_end) sstore(cur ^ 1);
      __syncthreads();
    }
  }

  // ---- accumulator layout: acc[tn][tm][r] = C[m][n] with
  //   m = m0 + wm*WM + tm*MF + lane % MF
  //   n = n0 + wn*WN + tn*MF + run(r) + 4*(lane / MF) + r % 4
  //   run(r) = 8*(r/4) for MF = 32 (4 runs of 4 columns), 0 for MF = 16.
  constexpr int RUNS = ACC_N / 4;
  constexpr int RUN_STRIDE = MF == 32 ? 8 : 0;
  const int col_in = 4 * (lane / MF);

  // ---- epilogue, one column tile at a time: all loads, then all stores
  constexpr bool PAIRED = EPI == EPI_ROPE || EPI == EPI_SILU;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    // paired epilogues: the first half of each 64-column block pairs with the
    // tile 32 columns on
    if (PAIRED && ((tn * MF) & 63) >= 32) continue;
    constexpr int G = TM * RUNS;
    int gm[G], gn[G];
    EpiIn e[G];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int q = 0; q < RUNS; ++q) {
        gm[tm * RUNS + q] = min(m0 + wm * WM + tm * MF + (lane % MF), p.M - 1);
        gn[tm * RUNS + q] = min(n0 + wn * WN + tn * MF + q * RUN_STRIDE + col_in, p.N - 4);
      }
    epi_load_groups<EPI, G>(p, gm, gn, e);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int q = 0; q < RUNS; ++q) {
        const int m = m0 + wm * WM + tm * MF + (lane % MF);
        const int n = n0 + wn * WN + tn * MF + q * RUN_STRIDE + col_in;
        if (m >= p.M || n >= p.N) continue;
        float x1[4], x2[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x1[i] = acc[tn][tm][4 * q + i] * p.alpha;
          x2[i] = PAIRED ? acc[(tn + PAIR_T) % TN][tm][4 * q + i] * p.alpha : 0.f;
        }
        epi_apply<EPI, ACT>(p, m, n, x1, x2, e[tm * RUNS + q]);
      }
  }
}

// ---- pipelined GEMM (LDS DMA) ---------------------------------------------------
// BM x BN block tile (128x128: 2x2 waves of 64x64; 64x64: 4x1 waves of 16x64),
// K step 32, 4-stage ring of LDS buffers filled by global_load_lds_dwordx4
// (each instruction moves 64 lanes x 16 B straight into LDS, no register
// staging), so three K tiles are in flight while the fourth is multiplied.
// The stages are separate LDS variables and every DMA is issued
// unconditionally (addresses clamped into the tensors), which lets the
// compiler track each stage's DMA separately instead of draining all of them
// before every LDS read; the only waits are the explicit vmcnt before each
// barrier (two newer stages stay in flight).
// LDS layout of a stage: row r holds 4 chunks of 8 bf16; logical chunk g of
// row r sits in slot g ^ ((r >> 1) & 3), so the 16-byte fragment reads of 8
// consecutive rows fall in 8 distinct bank groups.
// A K that is not a multiple of 32 ends with one tail step whose fragments are
// loaded straight from global memory with zero fill past K.
constexpr int PBK = 32;

__device__ __forceinline__ int pswz(int r, int g) { return g ^ ((r >> 1) & 3); }

// Epilogue of the LDS-DMA pipelines (same lane layout as gemm_kernel with
// MF = 16), one column tile at a time: all loads, then all stores.
template <int BM, int BN, int EPI, int ACT, int TN, int TM>
__device__ __forceinline__ void pipe_epilogue(const GemmArgs& p, const f32x4 (&acc)[TN][TM],
                                              int m0, int n0, int wm, int wn, int fr, int g) {
  constexpr int WAVES_M = BM >= 128 ? 2 : 4, WAVES_N = 4 / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr bool PAIRED = EPI == EPI_ROPE || EPI == EPI_SILU;
  const int col_in = 4 * g;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    // paired epilogues: the first half of each 64-column block pairs with the
    // tile 32 columns on
    if (PAIRED && (tn & 3) >= 2) continue;
    const int n = n0 + wn * WN + tn * 16 + col_in;
    int gm[TM], gn[TM];
    EpiIn e[TM];
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      gm[tm] = min(m0 + wm * WM + tm * 16 + fr, p.M - 1);
      gn[tm] = min(n, p.N - 4);
    }
    epi_load_groups<EPI, TM>(p, gm, gn, e);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int m = m0 + wm * WM + tm * 16 + fr;
      if (m >= p.M || n >= p.N) continue;
      float x1[4], x2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x1[i] = acc[tn][tm][i] * p.alpha;
        x2[i] = PAIRED ? acc[(tn + 2) % TN][tm][i] * p.alpha : 0.f;
      }
      epi_apply<EPI, ACT>(p, m, n, x1, x2, e[tm]);
    }
  }
}

template <int BM, int BN, int AMODE, bool NORM, int EPI, int ACT>
__global__ __launch_bounds__(256, 2) void gemm_pipe_kernel(GemmArgs p) {
  constexpr int WAVES_M = BM >= 128 ? 2 : 4, WAVES_N = 4 / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;  // 16x16 MFMA tiles per wave
  constexpr int A_DMA = BM / 64, B_DMA = BN / 64;  // 1 KB (16-row) DMA blocks per wave per stage
  static_assert(TM >= 1 && TN >= 1 && A_DMA >= 1 && B_DMA >= 1, "tile shape");
  static_assert((EPI != EPI_ROPE && EPI != EPI_SILU) || WN % 64 == 0,
                "paired epilogues need 64-column wave tiles");
  __shared__ __attribute__((aligned(1024))) bf16 sA0[BM * PBK], sA1[BM * PBK],
      sA2[BM * PBK], sA3[BM * PBK];
  __shared__ __attribute__((aligned(1024))) bf16 sB0[BN * PBK], sB1[BN * PBK],
      sB2[BN * PBK], sB3[BN * PBK];
  __shared__ __attribute__((aligned(16))) bf16 s_gain[NORM ? 2048 : 8];  // norm gain (K <= 2048)
  __shared__ float s_r[NORM ? BM : 1];                                    // norm row scales

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int gn = gridDim.x;
  const int tile = xcd_remap(blockIdx.y * gn + blockIdx.x, gn * gridDim.y);
  int tm_idx, tn_idx;
  tile_coords(tile, gridDim.y, gn, tm_idx, tn_idx);
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int nk = p.K / PBK;  // full K steps (>= 1, checked by the launcher)


  // per-lane DMA source rows (fixed across K tiles): block b covers rows
  // 16b .. 16b+15, lane -> row 16b + lane/4, slot lane%4
  int a_row[A_DMA], a_slot[A_DMA], b_row[B_DMA], b_slot[B_DMA];
#pragma unroll
  for (int j = 0; j < A_DMA; ++j) {
    const int r = (wave * A_DMA + j) * 16 + (lane >> 2);
    a_row[j] = min(m0 + r, p.M - 1);
    a_slot[j] = pswz(r, lane & 3);
  }
#pragma unroll
  for (int j = 0; j < B_DMA; ++j) {
    const int r = (wave * B_DMA + j) * 16 + (lane >> 2);
    b_row[j] = min(n0 + r, p.N - 1);
    b_slot[j] = pswz(r, lane & 3);
  }

  auto issue = [&](auto SI, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(SI)::value;
    bf16* sa = S == 0 ? sA0 : S == 1 ? sA1 : S == 2 ? sA2 : sA3;
    bf16* sb = S == 0 ? sB0 : S == 1 ? sB1 : S == 2 ? sB2 : sB3;
    kt = min(kt, nk - 1);  // past the end: reload the last tile (never read)
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) {
      const int blk = wave * A_DMA + j;
      const int k = kt * PBK + a_slot[j] * 8;
      const bf16* ga;
      if constexpr (AMODE == A_DENSE) ga = p.a + (long)a_row[j] * p.lda + k;
      else {
        // gathers: load_a's address map
        if constexpr (AMODE == A_PSHUF) {
          const int s_ = p.g_scale, E = p.g_hidden, grid = p.g_grid, gs = grid / s_;
          const int per = gs * gs, mm = a_row[j];
          const int img = mm / per, i = mm - img * per, hp = i / gs, wp = i - hp * gs;
          const int sE = s_ * E, t = k / sE, rem = k - t * sE, u = rem / E, c = rem - u * E;
          ga = p.a + ((long)img * grid * grid + (long)(s_ * hp + t) * grid + s_ * wp + u) * E + c;
        } else {
          const int P = p.p_patch, H = p.p_img, G = H / P, per = G * G, mm = a_row[j];
          const int img = mm / per, tkn = mm - img * per, pr = tkn / G, pc = tkn - pr * G;
          const int P2 = P * P, ch = k / P2, r = k - ch * P2, ky = r / P, kx = r - ky * P;
          ga = p.a + (((long)img * p.p_chans + ch) * H + pr * P + ky) * H + pc * P + kx;
        }
      }
      __builtin_amdgcn_global_load_lds((void*)ga, (lds_ptr_t)(sa + blk * 512), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) {
      const int blk = wave * B_DMA + j;
      const bf16* gb = p.b + (long)b_row[j] * p.ldb + kt * PBK + b_slot[j] * 8;
      __builtin_amdgcn_global_load_lds((void*)gb, (lds_ptr_t)(sb + blk * 512), 16, 0, 0);
    }
  };

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, g = lane >> 4;
  // Fused RMSNorm (NORM): the gain vector is copied to LDS (the main loop
  // then issues no global loads besides its DMA: a plain load would force a
  // full vmcnt drain) and the row scales are formed (norm_rows) while the
  // first stages stream in; each A fragment (lane: row tm * 16 + fr, columns
  // g * 8 .. + 7 of a K step) is rounded as bf16((x * r) * w) on its way into
  // the MFMAs.
  float rsv[TM];  // row scale of the lane's fragment row in row tile tm
  auto norm_setup = [&]() __attribute__((always_inline)) {
    if constexpr (NORM) {
      for (int c = tid * 8; c < p.K; c += 256 * 8)
        *reinterpret_cast<bf16x8*>(&s_gain[c]) = ld8(p.norm_w + c);
      norm_rows<BM, 256>(p, m0, s_r);
      __syncthreads();
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) rsv[tm] = s_r[wm * WM + tm * 16 + fr];
    }
  };
  auto normalise = [&](bf16x8 (&fx)[TM], int k) {
    if constexpr (NORM) {
      const bf16x8 gw = *reinterpret_cast<const bf16x8*>(&s_gain[k]);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) norm_frag(fx[tm], rsv[tm], gw);
    }
  };
  auto mma = [&](const bf16x8 (&fw)[TN], const bf16x8 (&fx)[TM]) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[tn], fx[tm], acc[tn][tm], 0, 0, 0);
  };

  auto compute = [&](auto SI, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(SI)::value;
    const bf16* sa = S == 0 ? sA0 : S == 1 ? sA1 : S == 2 ? sA2 : sA3;
    const bf16* sb = S == 0 ? sB0 : S == 1 ? sB1 : S == 2 ? sB2 : sB3;
    bf16x8 fw[TN], fx[TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int r = wn * WN + tn * 16 + fr;
      fw[tn] = *reinterpret_cast<const bf16x8*>(&sb[r * PBK + pswz(r, g) * 8]);
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int r = wm * WM + tm * 16 + fr;
      fx[tm] = *reinterpret_cast<const bf16x8*>(&sa[r * PBK + pswz(r, g) * 8]);
    }
    normalise(fx, kt * PBK + g * 8);
    mma(fw, fx);
  };

  // Before each barrier: s_waitcnt vmcnt(N) lgkmcnt(0).  vmcnt: each stage is
  // A_DMA + B_DMA instructions per wave and two newer stages may stay in
  // flight, so the stage computed next has landed.  lgkmcnt(0): this wave's
  // LDS reads of the stage computed before the barrier have completed, since
  // the DMA issued right after the barrier refills that stage.  (Without it
  // the compiler defers the wait to the reads' first use, after the barrier
  // and the refill's issue; a refill that hits in L2 could then overwrite a
  // fragment before a busy LDS served the read: one wave's 16 rows of a tile
  // read the wrong K tile, rarely and timing-dependent, measured on MI355X.)
  // gfx9 encoding: vmcnt[3:0] in bits 3:0, expcnt = 7 in bits 6:4, lgkmcnt
  // in bits 11:8.
  constexpr int kWaitN = 2 * (A_DMA + B_DMA);
  static_assert(kWaitN <= 15, "vmcnt immediate");
  constexpr int kWait2 = 0x070 | kWaitN;
  auto sync_step = [&]() __attribute__((always_inline)) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(kWait2);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;

  issue(I0{}, 0);
  issue(I1{}, 1);
  issue(I2{}, 2);
  norm_setup();
  for (int kt = 0; kt < nk; kt += 4) {
    sync_step();
    issue(I3{}, kt + 3);
    compute(I0{}, kt);
    sync_step();
    issue(I0{}, kt + 4);
    if (kt + 1 < nk) compute(I1{}, kt + 1);
    sync_step();
    issue(I1{}, kt + 5);
    if (kt + 2 < nk) compute(I2{}, kt + 2);
    sync_step();
    issue(I2{}, kt + 6);
    if (kt + 3 < nk) compute(I3{}, kt + 3);
  }
  // drain the trailing (never read) DMA before the workgroup can exit
  __builtin_amdgcn_s_waitcnt(0);

  // K tail (K % 32 = 8, 16 or 24): fragments from global memory, zero past K
  if (nk * PBK < p.K) {
    const int k = nk * PBK + g * 8;
    bf16x8 fw[TN], fx[TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + wn * WN + tn * 16 + fr;
      fw[tn] = (k < p.K && n < p.N) ? ld8(p.b + (long)n * p.ldb + k) : bf16x8{};
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) fx[tm] = load_a<AMODE>(p, m0 + wm * WM + tm * 16 + fr, k);
    normalise(fx, min(k, p.K - 8));  // fx is zero past K whatever the gain
    mma(fw, fx);
  }
  pipe_epilogue<BM, BN, EPI, ACT>(p, acc, m0, n0, wm, wn, fr, g);
}

// ---- line-DMA pipeline: 64-wide K stages fetched as whole cache lines ------
// Same tiles, waves and epilogue as gemm_pipe_kernel, but each LDS stage holds
// a 64-element K slice and every DMA instruction fetches 8 rows x 128 bytes
// (8 lanes per row): whole cache lines.  A CU's L1 serves misses at a per-line
// rate, so the 16-row x 64-byte instructions of the 32-wide stages (each line
// half used per instruction) bring about half the bytes per second (measured
// on MI355X: 200 KB per CU in 6.1 us as 16 x 64 B, 3.1 us as 8 x 128 B).  Two
// stages (the same LDS as four 32-wide ones): the next stage streams in while
// the current one is consumed as two 32-wide MFMA K steps.  Row r holds its 8
// 16-byte chunks at slots chunk ^ ((r >> 1) & 7), so a fragment read of 16
// rows (16 lanes, one chunk) spreads over the banks.
constexpr int LBK = 64;
__device__ __forceinline__ int lswz(int r, int c) { return c ^ ((r >> 1) & 7); }

template <int BM, int BN, int AMODE, bool NORM, int EPI, int ACT>
__global__ __launch_bounds__(256, 2) void gemm_line_kernel(GemmArgs p) {
  constexpr int WAVES_M = BM >= 128 ? 2 : 4, WAVES_N = 4 / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;          // 16x16 MFMA tiles per wave
  constexpr int A_DMA = BM / 32, B_DMA = BN / 32;    // 1 KB (8-row) DMA blocks per wave per stage
  static_assert(TM >= 1 && TN >= 1 && A_DMA >= 1 && B_DMA >= 1, "tile shape");
  static_assert((EPI != EPI_ROPE && EPI != EPI_SILU) || WN % 64 == 0,
                "paired epilogues need 64-column wave tiles");
  __shared__ __attribute__((aligned(1024))) bf16 sA0[BM * LBK], sA1[BM * LBK];
  __shared__ __attribute__((aligned(1024))) bf16 sB0[BN * LBK], sB1[BN * LBK];
  __shared__ __attribute__((aligned(16))) bf16 s_gain[NORM ? 2048 : 8];  // norm gain (K <= 2048)
  __shared__ float s_r[NORM ? BM : 1];                                    // norm row scales

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int gn = gridDim.x;
  const int tile = xcd_remap(blockIdx.y * gn + blockIdx.x, gn * gridDim.y);
  int tm_idx, tn_idx;
  tile_coords(tile, gridDim.y, gn, tm_idx, tn_idx);
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int nk = p.K / LBK;  // full 64-wide stages (>= 1, checked by the launcher)

  // per-lane DMA source rows (fixed across stages): block b covers rows
  // 8b .. 8b+7, lane -> row 8b + lane/8, LDS slot lane%8
  int a_row[A_DMA], a_chunk[A_DMA], b_row[B_DMA], b_chunk[B_DMA];
#pragma unroll
  for (int j = 0; j < A_DMA; ++j) {
    const int r = (wave * A_DMA + j) * 8 + (lane >> 3);
    a_row[j] = min(m0 + r, p.M - 1);
    a_chunk[j] = lswz(r, lane & 7);
  }
#pragma unroll
  for (int j = 0; j < B_DMA; ++j) {
    const int r = (wave * B_DMA + j) * 8 + (lane >> 3);
    b_row[j] = min(n0 + r, p.N - 1);
    b_chunk[j] = lswz(r, lane & 7);
  }

  auto issue = [&](auto SI, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(SI)::value;
    bf16* sa = S == 0 ? sA0 : sA1;
    bf16* sb = S == 0 ? sB0 : sB1;
    kt = min(kt, nk - 1);  // past the end: reload the last stage (never read)
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) {
      const int blk = wave * A_DMA + j;
      const int k = kt * LBK + a_chunk[j] * 8;
      const bf16* ga;
      if constexpr (AMODE == A_DENSE) ga = p.a + (long)a_row[j] * p.lda + k;
      else {
        // gathers: load_a's address map
        if constexpr (AMODE == A_PSHUF) {
          const int s_ = p.g_scale, E = p.g_hidden, grid = p.g_grid, gs = grid / s_;
          const int per = gs * gs, mm = a_row[j];
          const int img = mm / per, i = mm - img * per, hp = i / gs, wp = i - hp * gs;
          const int sE = s_ * E, t = k / sE, rem = k - t * sE, u = rem / E, c = rem - u * E;
          ga = p.a + ((long)img * grid * grid + (long)(s_ * hp + t) * grid + s_ * wp + u) * E + c;
        } else {
          const int P = p.p_patch, H = p.p_img, G = H / P, per = G * G, mm = a_row[j];
          const int img = mm / per, tkn = mm - img * per, pr = tkn / G, pc = tkn - pr * G;
          const int P2 = P * P, ch = k / P2, r = k - ch * P2, ky = r / P, kx = r - ky * P;
          ga = p.a + (((long)img * p.p_chans + ch) * H + pr * P + ky) * H + pc * P + kx;
        }
      }
      __builtin_amdgcn_global_load_lds((void*)ga, (lds_ptr_t)(sa + blk * 512), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) {
      const int blk = wave * B_DMA + j;
      const bf16* gb = p.b + (long)b_row[j] * p.ldb + kt * LBK + b_chunk[j] * 8;
      __builtin_amdgcn_global_load_lds((void*)gb, (lds_ptr_t)(sb + blk * 512), 16, 0, 0);
    }
  };

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int fr = lane & 15, g = lane >> 4;
  // fused RMSNorm as in gemm_pipe_kernel: gain to LDS and row scales while
  // the first stage streams in, bf16((x * r) * w) on the way into the MFMAs
  float rsv[TM];
  auto norm_setup = [&]() __attribute__((always_inline)) {
    if constexpr (NORM) {
      for (int c = tid * 8; c < p.K; c += 256 * 8)
        *reinterpret_cast<bf16x8*>(&s_gain[c]) = ld8(p.norm_w + c);
      norm_rows<BM, 256>(p, m0, s_r);
      __syncthreads();
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) rsv[tm] = s_r[wm * WM + tm * 16 + fr];
    }
  };
  auto normalise = [&](bf16x8 (&fx)[TM], int k) {
    if constexpr (NORM) {
      const bf16x8 gw = *reinterpret_cast<const bf16x8*>(&s_gain[k]);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) norm_frag(fx[tm], rsv[tm], gw);
    }
  };
  auto mma = [&](const bf16x8 (&fw)[TN], const bf16x8 (&fx)[TM]) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[tn], fx[tm], acc[tn][tm], 0, 0, 0);
  };

  // one stage = two 32-wide MFMA K steps (chunks 4h + g, h = 0, 1)
  auto compute = [&](auto SI, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(SI)::value;
    const bf16* sa = S == 0 ? sA0 : sA1;
    const bf16* sb = S == 0 ? sB0 : sB1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      bf16x8 fw[TN], fx[TM];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int r = wn * WN + tn * 16 + fr;
        fw[tn] = *reinterpret_cast<const bf16x8*>(&sb[r * LBK + lswz(r, 4 * h + g) * 8]);
      }
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) {
        const int r = wm * WM + tm * 16 + fr;
        fx[tm] = *reinterpret_cast<const bf16x8*>(&sa[r * LBK + lswz(r, 4 * h + g) * 8]);
      }
      normalise(fx, kt * LBK + h * 32 + g * 8);
      mma(fw, fx);
    }
  };

  // Before each barrier: s_waitcnt vmcnt(0) lgkmcnt(0): the stage computed
  // next has landed (it is the only one in flight), and this wave's LDS reads
  // of the stage computed before the barrier have completed, since the DMA
  // issued right after the barrier refills that stage.  gfx9 encoding.
  constexpr int kWait0 = 0x070;
  auto sync_step = [&]() __attribute__((always_inline)) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(kWait0);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  issue(I0{}, 0);
  norm_setup();
  for (int kt = 0; kt < nk; kt += 2) {
    sync_step();
    issue(I1{}, kt + 1);
    compute(I0{}, kt);
    sync_step();
    issue(I0{}, kt + 2);
    if (kt + 1 < nk) compute(I1{}, kt + 1);
  }
  // drain the trailing (never read) DMA before the workgroup can exit
  __builtin_amdgcn_s_waitcnt(0);

  // K tail (K % 64 = 8 .. 56): 32-wide steps from global memory, zero past K
  for (int kb = nk * LBK; kb < p.K; kb += 32) {
    const int k = kb + g * 8;
    bf16x8 fw[TN], fx[TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + wn * WN + tn * 16 + fr;
      fw[tn] = (k < p.K && n < p.N) ? ld8(p.b + (long)n * p.ldb + k) : bf16x8{};
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) fx[tm] = load_a<AMODE>(p, m0 + wm * WM + tm * 16 + fr, k);
    normalise(fx, min(k, p.K - 8));  // fx is zero past K whatever the gain
    mma(fw, fx);
  }
  pipe_epilogue<BM, BN, EPI, ACT>(p, acc, m0, n0, wm, wn, fr, g);
}

// ---- small-tile GEMM: BM x BN block tile, 4-stage line-DMA ring -------------
// For mid-size problems whose 64-row tiles leave most of the chip idle or need
// a cross-workgroup K split (the batch-1 prefix, M = 241: 32 x 32 tiles give
// 8 x 30 = 240 workgroups for N = 960), and tile shapes that put about one
// tile on each CU (96 x 96 on the batch-1 ViT's 3072 x 768 outputs: 256
// tiles).  Each workgroup streams 64-wide K stages of its BM A rows and BN
// weight rows as whole cache lines (the line kernel's LDS layout and swizzle)
// through a 4-stage ring, three stages in flight.  The 4 waves split the tile
// two ways and K two ways: wave w owns rows (BM / 2) (w & 1) .. + BM / 2 - 1
// and every column of the tile, and computes the 32-wide half (w >> 1) of
// each stage, so each activation fragment of a stage is read from LDS once
// and each weight fragment twice (once per row half).  The two K halves meet
// in LDS at the end; waves 0 and 1 run the epilogue (the same
// lane layout as the pipelines: 4 consecutive columns of one row per lane).
// The fused RMSNorm works as in the line kernel (row scales first, each A
// fragment rounded as bf16((x * r) * w) on the way into the MFMAs).
constexpr int SNS = 4;  // ring stages

template <int BM, int BN, int AMODE, bool NORM, int EPI, int ACT>
__global__ __launch_bounds__(256, (BM * BN <= 2048 ? 2 : 1)) void gemm_small_kernel(GemmArgs p) {
  constexpr int TM = BM / 32;          // 16-row MFMA tiles per wave
  constexpr int TN = BN / 16;          // 16-column MFMA tiles per wave
  constexpr int A_DMA = BM / 32;       // 1 KB (8-row) DMA blocks per wave per stage
  constexpr int B_DMA = BN / 32;
  constexpr bool PAIRED = EPI == EPI_ROPE || EPI == EPI_SILU;
  static_assert(BM % 32 == 0 && BN % 32 == 0 && BM <= 96 && BN <= 96, "tile shape");
  static_assert(!PAIRED || BN == 64, "paired epilogues need 64-column tiles");
  __shared__ __attribute__((aligned(1024))) bf16 sA0[BM * LBK], sA1[BM * LBK],
      sA2[BM * LBK], sA3[BM * LBK];
  __shared__ __attribute__((aligned(1024))) bf16 sB0[BN * LBK], sB1[BN * LBK],
      sB2[BN * LBK], sB3[BN * LBK];
  __shared__ __attribute__((aligned(16))) bf16 s_gain[NORM ? 2048 : 8];  // K <= 2048
  __shared__ float s_r[NORM ? BM : 1];                                      // norm row scales
  __shared__ __attribute__((aligned(16))) float s_red[2][TM * TN * 4][64];  // K-half 1's tiles

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, kg = wave >> 1;
  const int gn = gridDim.x;
  const int tile = xcd_remap(blockIdx.y * gn + blockIdx.x, gn * gridDim.y);
  int tm_idx, tn_idx;
  tile_coords(tile, gridDim.y, gn, tm_idx, tn_idx);
  const int m0 = tm_idx * BM, n0 = tn_idx * BN;
  const int nk = p.K / LBK;  // full 64-wide stages (>= 1, checked by the launcher)

  // DMA rows: block b covers rows 8b .. 8b + 7, wave w issues blocks
  // w * X_DMA + j; lane -> row lane / 8, chunk lane % 8 at slot lswz(row, chunk)
  int a_row[A_DMA], a_chunk[A_DMA], b_row[B_DMA], b_chunk[B_DMA];
#pragma unroll
  for (int j = 0; j < A_DMA; ++j) {
    const int r = (wave * A_DMA + j) * 8 + (lane >> 3);
    a_row[j] = min(m0 + r, p.M - 1);
    a_chunk[j] = lswz(r, lane & 7);
  }
#pragma unroll
  for (int j = 0; j < B_DMA; ++j) {
    const int r = (wave * B_DMA + j) * 8 + (lane >> 3);
    b_row[j] = min(n0 + r, p.N - 1);
    b_chunk[j] = lswz(r, lane & 7);
  }
  auto issue = [&](auto SI, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(SI)::value;
    bf16* sa = S == 0 ? sA0 : S == 1 ? sA1 : S == 2 ? sA2 : sA3;
    bf16* sb = S == 0 ? sB0 : S == 1 ? sB1 : S == 2 ? sB2 : sB3;
    kt = min(kt, nk - 1);  // past the end: reload the last stage (never read)
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) {
      const bf16* ga = a_ptr<AMODE>(p, a_row[j], kt * LBK + a_chunk[j] * 8);
      __builtin_amdgcn_global_load_lds((void*)ga, (lds_ptr_t)(sa + (wave * A_DMA + j) * 512), 16, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) {
      const bf16* gb = p.b + (long)b_row[j] * p.ldb + kt * LBK + b_chunk[j] * 8;
      __builtin_amdgcn_global_load_lds((void*)gb, (lds_ptr_t)(sb + (wave * B_DMA + j) * 512), 16, 0, 0);
    }
  };

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane & 15, g = lane >> 4;
  const int arow0 = wm * (BM / 2) + fr;  // the lane's A fragment row in row tile 0
  // fused RMSNorm as in gemm_pipe_kernel: gain to LDS and row scales while
  // the first stages stream in, bf16((x * r) * w) on the way into the MFMAs
  float rsv[TM];
  auto norm_setup = [&]() __attribute__((always_inline)) {
    if constexpr (NORM) {
      for (int c = tid * 8; c < p.K; c += 256 * 8)
        *reinterpret_cast<bf16x8*>(&s_gain[c]) = ld8(p.norm_w + c);
      norm_rows<BM, 256>(p, m0, s_r);
      __syncthreads();
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) rsv[tm] = s_r[arow0 + tm * 16];
    }
  };
  auto step = [&](const bf16x8 (&fw)[TN], bf16x8 (&fx)[TM], int k) __attribute__((always_inline)) {
    if constexpr (NORM) {
      const bf16x8 gw = *reinterpret_cast<const bf16x8*>(&s_gain[k]);
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) norm_frag(fx[tm], rsv[tm], gw);
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[tn], fx[tm], acc[tn][tm], 0, 0, 0);
  };
  // this wave's 32-wide half kg of a stage: chunks 4 kg + g
  auto compute = [&](auto SI, int kt) __attribute__((always_inline)) {
    constexpr int S = decltype(SI)::value;
    const bf16* sa = S == 0 ? sA0 : S == 1 ? sA1 : S == 2 ? sA2 : sA3;
    const bf16* sb = S == 0 ? sB0 : S == 1 ? sB1 : S == 2 ? sB2 : sB3;
    const int c = 4 * kg + g;
    bf16x8 fw[TN], fx[TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int r = tn * 16 + fr;
      fw[tn] = *reinterpret_cast<const bf16x8*>(&sb[r * LBK + lswz(r, c) * 8]);
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) {
      const int r = arow0 + tm * 16;
      fx[tm] = *reinterpret_cast<const bf16x8*>(&sa[r * LBK + lswz(r, c) * 8]);
    }
    step(fw, fx, kt * LBK + c * 8);
  };

  // Before each barrier: vmcnt(2 * D) lgkmcnt(0), D = DMA instructions per
  // wave per stage: the stage computed next has landed (the two issued after
  // it may stay in flight), and this wave's LDS reads of the stage computed
  // before the barrier have completed, since the DMA issued right after the
  // barrier refills that stage.  gfx9 encoding, expcnt unconstrained.
  constexpr int kWait = 0x070 | (2 * (A_DMA + B_DMA));
  static_assert(2 * (A_DMA + B_DMA) < 16, "vmcnt field");
  auto sync_step = [&]() __attribute__((always_inline)) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(kWait);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  issue(I0{}, 0);
  issue(I1{}, 1);
  issue(I2{}, 2);
  norm_setup();
  for (int kt = 0; kt < nk; kt += SNS) {
    sync_step();
    issue(I3{}, kt + 3);
    compute(I0{}, kt);
    sync_step();
    issue(I0{}, kt + 4);
    if (kt + 1 < nk) compute(I1{}, kt + 1);
    sync_step();
    issue(I1{}, kt + 5);
    if (kt + 2 < nk) compute(I2{}, kt + 2);
    sync_step();
    issue(I2{}, kt + 6);
    if (kt + 3 < nk) compute(I3{}, kt + 3);
  }
  // drain the trailing (never read) DMA before the workgroup exits
  __builtin_amdgcn_s_waitcnt(0);

  // K tail (K % 64 = 8 .. 56): 32-wide steps from global memory, zero past K,
  // step t taken by the waves of K half t % 2
  for (int kb = nk * LBK + kg * 32; kb < p.K; kb += 64) {
    const int k = kb + g * 8;
    bf16x8 fw[TN], fx[TM];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + tn * 16 + fr;
      fw[tn] = (k < p.K && n < p.N) ? ld8(p.b + (long)n * p.ldb + k) : bf16x8{};
    }
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) fx[tm] = load_a<AMODE>(p, m0 + arow0 + tm * 16, k);
    step(fw, fx, min(k, p.K - 8));  // fx is zero past K whatever the gain
  }

  // the two K halves meet: waves 2, 3 hand their tiles to 0, 1
  if (kg == 1) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
#pragma unroll
        for (int i = 0; i < 4; ++i) s_red[wm][(tn * TM + tm) * 4 + i][lane] = acc[tn][tm][i];
  }
  __syncthreads();
  if (kg == 1) return;
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int tm = 0; tm < TM; ++tm)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[tn][tm][i] += s_red[wm][(tn * TM + tm) * 4 + i][lane];

  // epilogue: lane holds columns n0 + 16 tn + 4 g .. + 3 of rows m0 + arow0 +
  // 16 tm; paired epilogues (RoPE / SiLU) combine tile tn < 2 with tile tn + 2
  // (32 columns on), so only those groups load operands and store
  constexpr int G = PAIRED ? TN / 2 : TN;
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int m = m0 + arow0 + tm * 16;
    const float sc = p.alpha;
    int gm[G], gnn[G];
    EpiIn e[G];
#pragma unroll
    for (int t = 0; t < G; ++t) {
      gm[t] = min(m, p.M - 1);
      gnn[t] = min(n0 + t * 16 + 4 * g, p.N - 4);
    }
    epi_load_groups<EPI, G>(p, gm, gnn, e);
#pragma unroll
    for (int t = 0; t < G; ++t) {
      const int n = n0 + t * 16 + 4 * g;
      if (m >= p.M || n >= p.N) continue;
      float x1[4], x2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        x1[i] = acc[t][tm][i] * sc;
        x2[i] = PAIRED ? acc[(t + G) % TN][tm][i] * sc : 0.f;
      }
      epi_apply<EPI, ACT>(p, m, n, x1, x2, e[t]);
    }
  }
}

// ---- wide GEMM: 256 x 256 block tile, one workgroup per CU -------------------
// For the big-M problems (the batched ViT, M = 98304 rows at batch 32).  Each
// of the 4 waves owns a 128 x 128 output tile (8 x 8 MFMA 16x16x32 tiles, 256
// fp32 accumulators per lane, kept in AGPRs), which halves the LDS bytes read
// per MFMA FLOP relative to a 64 x 64 wave tile: 16 fragment reads feed 64
// MFMAs per K step.  Operands stream through a 5-stage ring of LDS buffers
// (K step 32, 32 KB per stage, 160 KB in total) filled by global_load_lds.
// The barrier of step s guarantees stage s + 1 is in LDS, so the fragments of
// step s + 1 are read into a second register set while the MFMAs of step s
// run and no LDS latency is exposed; the DMA and fragment reads are spread
// between the MFMAs.  One barrier per K step, four stages of DMA in flight;
// the epilogue stages its output through the ring.  Same LDS row swizzle and
// accumulator layout as gemm_pipe_kernel.
//
// The MFMAs are issued through inline asm with the accumulator tied to an
// AGPR operand: with the builtin, the register allocator shuffles AGPR-resident
// loop accumulators with v_accvgpr_mov copies every iteration (measured: more
// than half of the MFMA rate lost).  The asm is opaque to the hazard
// recognizer, so the kernel inserts the wait states itself, before the
// epilogue reads results.  A tile's first K step takes srcC = 0, so the
// accumulators are never zeroed by VALU writes.
constexpr int WBM = 256, WBN = 256, WBK = 32;
constexpr int W_DMA = 4;  // 1 KB DMA blocks per wave per operand per stage
constexpr int W_STAGES = 5;                    // LDS ring depth
constexpr int W_STAGE = (WBM + WBN) * WBK;     // bf16 elements per stage (32 KB)
constexpr int WTM = 8, WTN = 8;  // wave tile 128 x 128 = 8 x 8 MFMA tiles

// s_waitcnt immediate (gfx9 encoding): vmcnt split over bits 3:0 and 15:14,
// expcnt bits 6:4 (7 = no wait), lgkmcnt bits 11:8 (15 = no wait)
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8);
}

// Calls f(std::integral_constant<int, i>{}) for i = 0 .. N - 1 (compile-time
// indices where a #pragma unroll is not honoured).
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ void mfma_agpr(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// The first K step of a tile: srcC is the inline constant 0, so the
// accumulators need no zeroing pass (256 VALU writes per wave and tile).
__device__ __forceinline__ void mfma_agpr_first(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, 0" : "=a"(acc) : "v"(a), "v"(b));
}

// Redefines every accumulator (no instruction emitted): uses of acc after this
// point depend on it, and volatile asm statements keep their relative order,
// so reads cannot move above (and writes cannot move below) the neighbouring
// s_nop wait states, which the compiler does not know the inline MFMAs need.
template <int N1, int N2>
__device__ __forceinline__ void pin_accumulators(f32x4 (&acc)[N1][N2]) {
#pragma unroll
  for (int i = 0; i < N1; ++i)
#pragma unroll
    for (int j = 0; j < N2; ++j) asm volatile("" : "+a"(acc[i][j]));
}

// Per-column addend of the wide epilogue, for the 8 MFMA column tiles of a
// 128-wide wave tile at column wn0, in two parts: the bf16 bias pieces are
// loaded early (wide_bias_raw) and only read in the epilogue (wide_addend,
// which adds the fp32 bias): loads return in order, so consuming a load
// right away would wait for every DMA issued before it, i.e. drain the ring.
__device__ __forceinline__ void wide_bias_raw(const GemmArgs& p, int wn0, int g,
                                              bf16x4 (&braw)[WTN]) {
#pragma unroll
  for (int tn = 0; tn < WTN; ++tn)
    braw[tn] = p.bias ? *reinterpret_cast<const bf16x4*>(p.bias + min(wn0 + tn * 16 + 4 * g, p.N - 4))
                      : bf16x4{};
}
__device__ __forceinline__ void wide_addend(const GemmArgs& p, int wn0, int g,
                                            const bf16x4 (&braw)[WTN], f32x4 (&cb)[WTN]) {
#pragma unroll
  for (int tn = 0; tn < WTN; ++tn)
#pragma unroll
    for (int i = 0; i < 4; ++i) cb[tn][i] = bf2f(braw[tn][i]);
  if (p.bias_f32) {
#pragma unroll
    for (int tn = 0; tn < WTN; ++tn)
      cb[tn] += *reinterpret_cast<const f32x4*>(p.bias_f32 + min(wn0 + tn * 16 + 4 * g, p.N - 4));
  }
}

// Epilogue of a 128 x 128 wave tile (accumulators in AGPRs, MFMA layout),
// staged through LDS so that every global store writes whole 128-byte lines.
// In the MFMA layout a lane holds C[m][n .. n+3] for 16 different rows per
// instruction, i.e. 32-byte pieces of 16 lines, which the memory side writes
// back as partial lines (measured: ~5x slower than line-sized stores and 1.3x
// the bytes).  Per 32-row chunk of the wave tile:
//  phase 1 (MFMA layout): v = bf16(act(bf16(alpha * acc + addend))) into the
//  wave's 8 KB staging buffer `st` (row r: 32 slots of 4 columns, chunk c in
//  slot c ^ ((r & 7) << 2), so the 16 rows x 4 chunks of one write fall on
//  distinct banks pairwise);
//  phase 2 (row layout): 16 lanes read a 256-byte row (one 16-byte read each:
//  the swizzle keeps bit 0, so slots 2j, 2j + 1 stay adjacent), add the
//  residual (RES) and store it.
// The staging buffer is private to the wave, whose LDS operations complete
// in order, so no barrier is needed.
// RES (p.res is set): all 8 residual pieces of a chunk (8 rows x 16 bytes
// per lane) are loaded together, one memory round trip per chunk (the
// epilogue of the ViT O and down projections is bound by these round trips:
// 16-19 us per tile with two per chunk).  Holding them any earlier (across
// phase 1 or the previous chunk) costs registers that the last K round then
// spills.
// Without a residual the stores are streaming (non-temporal): those outputs
// are fresh tensors far larger than the caches (the ViT QKV and MLP
// activations: 0.45 / 0.6 GB at batch 32), where they measured 6-8% faster;
// in-place residual updates keep ordinary stores (the residual stream is
// re-read right away).
// bf16 rounding of two values with one conversion (v_cvt_pk_bf16_f32, round
// to nearest even like the compiler's own), back to fp32 by a shift and a
// mask: rbf(a), rbf(b).  Written as asm because the compiler splits a
// two-element conversion whose halves are used separately into two
// single-element conversions.
__device__ __forceinline__ void rbf_pair(float a, float b, float& ra, float& rb) {
  unsigned u;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(u) : "v"(a), "v"(b));
  ra = __uint_as_float(u << 16);
  rb = __uint_as_float(u & 0xffff0000u);
}

template <int ACT, bool RES>
__device__ __forceinline__ void wide_epilogue(const GemmArgs& p, f32x4 (&acc)[WTN][WTM],
                                              const bf16x4 (&braw)[WTN], bf16* st, int wm0,
                                              int wn0, int lane) {
  const int fr = lane & 15, g = lane >> 4;
  f32x4 cb[WTN];
  wide_addend(p, wn0, g, braw, cb);
  auto st_addr = [&](int r, int chunk) __attribute__((always_inline)) {
    return st + r * 128 + ((chunk ^ ((r & 7) << 2)) << 2);
  };
  const float alpha = p.alpha;
  const int j = lane & 15;
  const int ncol = wn0 + 8 * j;
  // phase-2 piece q (0..7) of chunk c: row c * 32 + 4 q + lane / 16, columns ncol .. ncol + 7
  // phase-2 batch: pieces (rows) whose loads are in flight together
  constexpr int NB = RES ? 8 : 4;
  // A wave tile inside the matrix (every tile when M and N are multiples of
  // 256) stores without checks through running pointers: the lane's rows are
  // wm0 + lane / 16 + 4 i for i = 0 .. 31 in store order, so each store is
  // one pointer increment (per-store row arithmetic and bounds checks were
  // most of the epilogue's instructions).  Ragged tiles take a rolled,
  // checked loop.
  const bool full = wm0 + 128 <= p.M && wn0 + 128 <= p.N;
  bf16* const cbase = reinterpret_cast<bf16*>(p.c);
  const int r0 = wm0 + (lane >> 4);
  bf16* cp = p.c_blk ? cbase + (long)(ncol >> 5) * p.M * WBK + (long)r0 * WBK + (ncol & 31)
                     : cbase + (long)r0 * p.ldc + ncol;
  const long cstep = 4 * (p.c_blk ? (long)WBK : (long)p.ldc);
  const bf16* rp = RES && full ? p.res + (long)r0 * p.ldr + ncol : nullptr;
  const long rstep = 4 * (long)p.ldr;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
#pragma unroll
    for (int tn = 0; tn < WTN; ++tn) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int tm = 2 * c + h;
        bf16x4 o;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __builtin_fmaf(acc[tn][tm][i], alpha, cb[tn][i]);
        if constexpr (ACT != SVLA_ACT_NONE) {
          // the activation's input rounded to bf16 two at a time
          float x[4];
          rbf_pair(v[0], v[1], x[0], x[1]);
          rbf_pair(v[2], v[3], x[2], x[3]);
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = f2bf(apply_act<ACT>(x[i]));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = f2bf(v[i]);
        }
        *reinterpret_cast<bf16x4*>(st_addr(h * 16 + fr, tn * 4 + g)) = o;
      }
    }
    // keep the next chunk's accumulator reads below this chunk's LDS writes
    // (otherwise the scheduler hoists all 256 AGPR reads up front and runs
    // out of VGPRs)
    if (c + 1 < 4) {
      asm volatile("" ::: "memory");
#pragma unroll
      for (int tn = 0; tn < WTN; ++tn) {
        asm volatile("" : "+a"(acc[tn][2 * c + 2]));
        asm volatile("" : "+a"(acc[tn][2 * c + 3]));
      }
    }
    if (full) {
#pragma unroll
      for (int b0 = 0; b0 < 8; b0 += NB) {
        bf16x8 v[NB], rsb[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
          v[b] = *reinterpret_cast<const bf16x8*>(st_addr((b0 + b) * 4 + (lane >> 4), 2 * j));
        if constexpr (RES) {
#pragma unroll
          for (int b = 0; b < NB; ++b) {
            rsb[b] = ld8(rp);
            rp += rstep;
          }
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
          bf16x8 o = v[b];
          if constexpr (RES) {
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = f2bf(bf2f(o[i]) + bf2f(rsb[b][i]));
            st8(cp, o);
          } else {
            __builtin_nontemporal_store(o, reinterpret_cast<bf16x8*>(cp));
          }
          cp += cstep;
        }
      }
    } else {
#pragma unroll 1
      for (int q = 0; q < 8; ++q) {
        const int r = q * 4 + (lane >> 4);
        const int m = wm0 + c * 32 + r;
        if (m >= p.M || ncol >= p.N) continue;  // ncol < N: all 8 columns (N % 8 == 0)
        bf16x8 o = *reinterpret_cast<const bf16x8*>(st_addr(r, 2 * j));
        if constexpr (RES) {
          const bf16x8 rv = ld8(p.res + (long)m * p.ldr + ncol);
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = f2bf(bf2f(o[i]) + bf2f(rv[i]));
        }
        st8(p.c_blk ? cbase + (long)(ncol >> 5) * p.M * WBK + (long)m * WBK + (ncol & 31)
                    : cbase + (long)m * p.ldc + ncol,
            o);
      }
    }
  }
}

// RES: the output is p.c + p.res (a separate instantiation: the residual
// epilogue's registers would otherwise be reserved, and the last K round
// spill for them, in the kernels that have none)
//
// Ring: W_STAGES = 5 stages of one K tile each ([A 256 x 32 | B 256 x 32],
// 32 KB), 160 KB in all.  K tile j of the workgroup's stream (its tiles' K
// tiles back to back) lives in stage j % 5; at step j (MFMAs on K tile j,
// whose fragments are already in registers) stage j % 5 is free and takes K
// tile j + 5, so four K tiles are in flight while one is read: a DMA has
// four steps to land (the K loop is bound by DMA latency: with three steps
// it ran 20-35% below the same loop without DMA, measured on MI355X).  The
// last step of a tile skips its refill, which leaves that stage free for the
// epilogue's staging; the first step of the next tile issues the skipped K
// tile together with its own refill.
template <int AMODE, bool NORM, int EPI, int ACT, bool RES>
__global__ __launch_bounds__(256, 1) void gemm_wide_kernel(GemmArgs p) {
  static_assert(AMODE == A_DENSE && !NORM && EPI == EPI_STORE, "wide tile: plain dense GEMM");
  __shared__ __attribute__((aligned(1024))) bf16 sRing[W_STAGES * W_STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int nk = p.K / WBK;  // K % (4 * WBK) == 0 and K >= 8 * WBK (checked by the launcher)
  const int T = p.tiles_m * p.tiles_n, G = gridDim.x;
  // workgroup b takes logical tiles slot(b), slot(b) + G, ...; slot() gives
  // the workgroups of one XCD consecutive logical tiles, and tile_coords turns
  // those into a compact patch of row and column blocks (shared panels in
  // that XCD's L2)
  // (column-resident order: workgroup b is member b / 8 of XCD b % 8, which
  // is where the dispatcher places it, and takes the XCD's tiles b / 8,
  // b / 8 + G / 8, ...; the host checks that every member has one)
  const int xcd = blockIdx.x % kNumXCD;
  int L, Lstep, Lend;
  if (p.w_cn > 0) {
    int first;
    L = blockIdx.x / kNumXCD;
    Lstep = G / kNumXCD;
    Lend = xcd_rows(p, xcd, first) * p.w_cn;
  } else {
    L = xcd_remap(blockIdx.x, G);
    Lstep = G;
    Lend = T;
  }
  auto origin = [&](int l, int& m0_, int& n0_) __attribute__((always_inline)) {
    int tm_idx, tn_idx;
    if (p.w_cn > 0) xcd_tile(p, xcd, l, tm_idx, tn_idx);
    else tile_coords(l, p.tiles_m, p.tiles_n, tm_idx, tn_idx);
    m0_ = tm_idx * WBM;
    n0_ = tn_idx * WBN;
  };
  int m0, n0;
  origin(L, m0, n0);

  // per-lane DMA sources: block b = wave * W_DMA + j covers rows 16b .. 16b+15;
  // lane -> row 16b + lane / 4, LDS slot lane % 4 holding logical chunk
  // pswz(row, slot).  Rows past M / N are clamped (their results are dropped).
  // row and K-step strides of A and W (elements): row-major, or slab-blocked
  const long a_rs = p.a_blk ? WBK : p.lda, a_ks = p.a_blk ? (long)p.M * WBK : WBK;
  const long b_rs = p.b_blk ? WBK : p.ldb, b_ks = p.b_blk ? (long)p.N * WBK : WBK;
  const bf16* a_src[W_DMA];
  const bf16* b_src[W_DMA];
  auto set_src = [&](int m0_, int n0_) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < W_DMA; ++j) {
      const int r = (wave * W_DMA + j) * 16 + (lane >> 2);
      const int g = pswz(r, lane & 3);
      a_src[j] = p.a + (long)min(m0_ + r, p.M - 1) * a_rs + g * 8;
      b_src[j] = p.b + (long)min(n0_ + r, p.N - 1) * b_rs + g * 8;
    }
  };
  set_src(m0, n0);

  // DMA j of a stage: j < W_DMA -> A block, else B block j - W_DMA; kt is a
  // K tile of the tile whose sources are set
  auto issue_one = [&](int s, int j, int kt) __attribute__((always_inline)) {
    bf16* st = sRing + s * W_STAGE;
    if (j < W_DMA)
      __builtin_amdgcn_global_load_lds((void*)(a_src[j] + kt * a_ks),
                                       (lds_ptr_t)(st + (wave * W_DMA + j) * 512), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((void*)(b_src[j - W_DMA] + kt * b_ks),
                                       (lds_ptr_t)(st + WBM * WBK + (wave * W_DMA + j - W_DMA) * 512),
                                       16, 0, 0);
  };

  // accumulators: defined by each tile's first K step (srcC = 0), so they are
  // never zeroed
  f32x4 acc[WTN][WTM];

  // fragment f of a stage: f < WTN -> weight tile f, else activation tile f - WTN
  const int fr = lane & 15, g = lane >> 4;
  const int frag_off = fr * WBK + pswz(fr, g) * 8;  // pswz depends on fr only
  bf16x8 fw[2][WTN], fx[2][WTM];
  auto read_one = [&](int s, auto RI, int f) __attribute__((always_inline)) {
    constexpr int R = decltype(RI)::value;
    const bf16* sa = sRing + s * W_STAGE;
    const bf16* sb = sa + WBM * WBK;
    if (f < WTN)
      fw[R][f] = *reinterpret_cast<const bf16x8*>(&sb[(wn * 128 + f * 16) * WBK + frag_off]);
    else
      fx[R][f - WTN] =
          *reinterpret_cast<const bf16x8*>(&sa[(wm * 128 + (f - WTN) * 16) * WBK + frag_off]);
  };

  // each stage is 2 * W_DMA DMA instructions per wave
  constexpr int kStageVm = 2 * W_DMA;
  constexpr int kWaitPrologue = waitcnt_imm(4 * kStageVm, 15);  // stage 0 landed
  constexpr int kWaitStep = waitcnt_imm(3 * kStageVm, 0);       // next stage landed, own reads done
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  auto nxt = [](int s) __attribute__((always_inline)) { return s == W_STAGES - 1 ? 0 : s + 1; };

  // One step of the ring (stage s holds the K tile whose fragments are in
  // register set R): wait until stage s + 1 is in LDS for every wave and
  // every wave holds its stage-s fragments, then, between the first 32 of the
  // 64 MFMAs: refill stage s with K tile `kt` (REFILL; one DMA every 4
  // MFMAs) and read stage s + 1's fragments into the other register set (one
  // every 2 MFMAs), so the reads have landed by the next step.  EXTRA (the
  // first step of a tile): extra_kt >= 0 also issues that K tile into stage
  // `extra_s` right after the barrier.  (In vmcnt terms every VMEM instruction issued
  // after a stage's DMA counts, stores included; the waits stay
  // conservative.)  The last step of a tile reads nothing: the next tile's
  // first fragments are read after the epilogue, so they are not live
  // across it.
  auto step = [&](auto RC, int s, int kt, auto READ, auto REFILL, auto EXTRA, int extra_s,
                  int extra_kt) __attribute__((always_inline)) {
    constexpr int R = decltype(RC)::value;
    using RN = std::integral_constant<int, 1 - R>;
    const int sn = nxt(s);
    __builtin_amdgcn_s_waitcnt(kWaitStep);
    __builtin_amdgcn_s_barrier();
    if constexpr (decltype(EXTRA)::value) {
      if (extra_kt >= 0) {
#pragma unroll
        for (int j = 0; j < 2 * W_DMA; ++j) issue_one(extra_s, j, extra_kt);
      }
    }
#pragma unroll
    for (int i = 0; i < WTN * WTM; ++i) {
      if constexpr (decltype(EXTRA)::value)  // the tile's first step
        mfma_agpr_first(acc[i / WTM][i % WTM], fw[R][i / WTM], fx[R][i % WTM]);
      else
        mfma_agpr(acc[i / WTM][i % WTM], fw[R][i / WTM], fx[R][i % WTM]);
      if constexpr (decltype(REFILL)::value)
        if (i < 32 && i % 4 == 0) issue_one(s, i / 4, kt);
      if constexpr (decltype(READ)::value)
        if (i < 32 && i % 2 == 1) read_one(sn, RN{}, i / 2);
    }
  };
  using Y = std::true_type;
  using N = std::false_type;

  // prologue of the first tile: K tiles 0 .. 4 into stages 0 .. 4
#pragma unroll
  for (int s = 0; s < W_STAGES; ++s) {
#pragma unroll
    for (int j = 0; j < 2 * W_DMA; ++j) issue_one(s, j, s);
  }
  __builtin_amdgcn_s_waitcnt(kWaitPrologue);
  __builtin_amdgcn_s_barrier();
#pragma unroll
  for (int f = 0; f < WTN + WTM; ++f) read_one(0, I0{}, f);

  int s0 = 0;          // stage of the current tile's K tile 0
  int pend_kt = -1;    // K tile 4 of this tile, deferred by the previous tile's last step
  for (;;) {
    const int wm0 = m0 + wm * 128, wn0 = n0 + wn * 128;
    int s = s0;
    // steps 0 .. nk - 7 refill with this tile's K tiles 5 .. nk - 2; the
    // first also issues a deferred K tile 4 into the stage after s0's + 3
    const int ps = s0 == 0 ? W_STAGES - 1 : s0 - 1;  // (s0 + 4) % 5
    step(I0{}, s, 5, Y{}, Y{}, Y{}, ps, pend_kt);
    s = nxt(s);
    step(I1{}, s, 6, Y{}, Y{}, N{}, 0, 0);
    s = nxt(s);
    for (int kt = 2; kt + 6 < nk; kt += 2) {
      step(I0{}, s, kt + 5, Y{}, Y{}, N{}, 0, 0);
      s = nxt(s);
      step(I1{}, s, kt + 6, Y{}, Y{}, N{}, 0, 0);
      s = nxt(s);
    }
    // the epilogue's bf16 bias, loaded before the next tile's DMA so that
    // waiting for it does not wait for that DMA
    bf16x4 braw[WTN];
    wide_bias_raw(p, wn0, g, braw);
    // the last 6 steps: the first refills this tile's K tile nk - 1, the next
    // four the next tile's K tiles 0 .. 3 (or, after the last tile, reload
    // this tile's last K tile, never read); the last refills nothing
    const int L_next = L + Lstep;
    const bool has_next = L_next < Lend;
    step(I0{}, s, nk - 1, Y{}, Y{}, N{}, 0, 0);
    s = nxt(s);
    int mn0 = m0, nn0 = n0;
    if (has_next) {
      origin(L_next, mn0, nn0);
      set_src(mn0, nn0);
    }
    step(I1{}, s, has_next ? 0 : nk - 1, Y{}, Y{}, N{}, 0, 0);
    s = nxt(s);
    step(I0{}, s, has_next ? 1 : nk - 1, Y{}, Y{}, N{}, 0, 0);
    s = nxt(s);
    step(I1{}, s, has_next ? 2 : nk - 1, Y{}, Y{}, N{}, 0, 0);
    s = nxt(s);
    step(I0{}, s, has_next ? 3 : nk - 1, Y{}, Y{}, N{}, 0, 0);
    s = nxt(s);
    step(I1{}, s, 0, N{}, N{}, N{}, 0, 0);
    // let the last MFMAs retire before their accumulators are read
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    pin_accumulators(acc);

    // stage s held K tile nk - 1 (its fragments were read at the previous
    // step, before this step's barrier) and takes no DMA until the next
    // tile's first step: the epilogue stages through it, 8 KB per wave
    wide_epilogue<ACT, RES>(p, acc, braw, sRing + s * W_STAGE + wave * (32 * 128), wm0, wn0, lane);
    if (!has_next) break;
    L = L_next;
    m0 = mn0;
    n0 = nn0;
    s0 = nxt(s);   // the next tile's K tile 0
    pend_kt = 4;   // goes into stage s, after the next step's barrier
    static_for<0, WTN + WTM>([&](auto F) { read_one(s0, I0{}, decltype(F)::value); });
  }
  // drain the trailing (never read) DMA and the stores before exit
  __builtin_amdgcn_s_waitcnt(0);
}

// ---- skinny-M GEMM ----------------------------------------------------------
// One workgroup = 64 rows x BN columns, 8 waves.  The waves split the K loop
// (in steps of 32) and each accumulates the whole tile with 16x16x32 MFMAs
// whose operand fragments come straight from global memory.  Problems this
// small are latency-bound, so each wave issues the loads of up to KR k-steps
// at once before any MFMA.  The optional RMSNorm of the A rows forms the row
// scales first (norm_rows, over the whole K whatever the split) and rounds
// each A fragment as bf16((x * r) * w) on its way into the MFMAs.  The 8
// partial tiles are summed through LDS and all 512 threads run the epilogue.
//
// Split-K over workgroups (gridDim.z = S > 1, for long-K problems whose grid
// is far smaller than the chip): workgroup z covers k-steps
// [z * kps, (z + 1) * kps) and writes its fp32 tile to the workspace; the last of the S
// workgroups of a tile to arrive (device-scope counter) sums the S partials in
// split order, runs the epilogue and resets the counter.  No workgroup ever
// waits for another.
constexpr int SK_WAVES = 8;

template <int BN, int AMODE, bool NORM, int EPI, int ACT>
__global__ __launch_bounds__(SK_WAVES * 64) void skinny_kernel(GemmArgs p) {
  constexpr int BM = 64, TM = BM / 16, TN = BN / 16;
  constexpr int PS = BN + 4;  // padded LDS row of a partial tile (floats)
  constexpr int NT = SK_WAVES * 64;
  // k-steps whose loads are in flight together (bounded by the 256-VGPR budget
  // of 8 waves per workgroup); 8 waves x 4 steps cover K <= 1024 in one round
  constexpr int KR = BN <= 32 && AMODE == A_DENSE && !NORM ? 8 : 4;
  constexpr int PSZ = BM * BN;  // one split's workspace partial
  // Paired epilogues (RoPE / SiLU) combine packed column n with n + 32 of the
  // same 64-column block.  A 64-wide tile holds both halves; a 16-wide tile
  // (P16) takes 8 columns of a first half and their 8 partners, loading the
  // weight rows through that map (each lane reads its own row anyway): tile t
  // covers columns pbase + 0..7 and pbase + 32 + 0..7, pbase = 64 (t / 4) +
  // 8 (t % 4), held at tile columns 0..7 and 8..15.
  constexpr bool PAIRED = EPI == EPI_ROPE || EPI == EPI_SILU;
  constexpr bool P16 = PAIRED && BN == 16;
  static_assert(!PAIRED || BN % 64 == 0 || P16, "paired epilogue");
  static_assert(!NORM || AMODE == A_DENSE, "row norm only for dense A");
  __shared__ __attribute__((aligned(16))) float s_part[SK_WAVES][BM * PS];
  __shared__ float s_rs[NORM ? BM : 1];            // norm row scales
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  // first packed column of the tile's logical columns (P16: see above)
  const int nbase = P16 ? (n0 >> 6) * 64 + ((n0 & 63) >> 4) * 8 : n0;
  const int nkf = p.K / 32;  // full k-steps; a K % 32 tail is one extra step
  const int S = gridDim.z, z = blockIdx.z;
  const int kps = (nkf + S - 1) / S;  // k-steps of one split
  const int kb = min(nkf, z * kps), ke = min(nkf, kb + kps);
  // each wave takes whole rounds of KR k-steps (trailing waves may idle), so
  // only the last round of the last busy wave reloads a step to fill up
  const int rounds = (ke - kb + SK_WAVES * KR - 1) / (SK_WAVES * KR);
  const int per = rounds * KR;
  const int ks0 = kb + wave * per, ks1 = min(ke, ks0 + per);
  const int fr = lane & 15, fk = (lane >> 4) * 8;

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Operand rows are clamped into the tensors (rows past M / N only feed
  // outputs that are never stored) and k-steps past this wave's range reload
  // its last step: every load of a round is issued unconditionally, so the
  // whole round is in flight at once (a load under a branch would end its
  // region with a full vmcnt(0) drain and serialise the round).
  int a_rows[TM], b_rows[TN];
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) a_rows[tm] = min(m0 + tm * 16 + fr, p.M - 1);
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
    b_rows[tn] = P16 ? nbase + (fr & 7) + (fr >> 3) * 32 : min(n0 + tn * 16 + fr, p.N - 1);

  bf16x8 fw[KR][TN], fx[KR][TM], fg[KR];
  auto load_step = [&](int r, int k) __attribute__((always_inline)) {
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) fw[r][tn] = ld8(p.b + (long)b_rows[tn] * p.ldb + k);
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) fx[r][tm] = ld8(a_ptr<AMODE>(p, a_rows[tm], k));
    if constexpr (NORM) fg[r] = ld8(p.norm_w + k);
  };
  auto load_round = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < KR; ++r) load_step(r, min(base + r, ks1 - 1) * 32 + fk);
  };
  float rsv[TM];  // norm: row scale of row tm * 16 + fr
  if constexpr (NORM) {
    norm_rows<BM, NT>(p, m0, s_rs);
    __syncthreads();
#pragma unroll
    for (int tm = 0; tm < TM; ++tm) rsv[tm] = s_rs[tm * 16 + fr];
  }
  auto mma_step = [&](int r) __attribute__((always_inline)) {
    if constexpr (NORM) {
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) norm_frag(fx[r][tm], rsv[tm], fg[r]);
    }
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
#pragma unroll
      for (int tm = 0; tm < TM; ++tm)
        acc[tn][tm] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[r][tn], fx[r][tm], acc[tn][tm], 0, 0, 0);
  };
  auto mma_round = [&](int base) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < KR; ++r)
      if (base + r < ks1) mma_step(r);  // wave-uniform; only MFMAs under the branch
  };

  if (ks0 < ks1) {
    load_round(ks0);
    mma_round(ks0);
    for (int base = ks0 + KR; base < ks1; base += KR) {
      load_round(base);
      mma_round(base);
    }
  }
  // K tail (K % 32 = 8, 16 or 24): the last wave of the last split adds one
  // zero-filled step
  if (nkf * 32 < p.K && wave == SK_WAVES - 1 && z == S - 1) {
    const int k = nkf * 32 + fk;
    const bool kin = k < p.K;
    load_step(0, min(k, p.K - 8));
    if (!kin) {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) fw[0][tn] = bf16x8{};
#pragma unroll
      for (int tm = 0; tm < TM; ++tm) fx[0][tm] = bf16x8{};
    }
    mma_step(0);
  }

  // partial tile: element (m_l, n_l) at s_part[wave][m_l * PS + n_l]
#pragma unroll
  for (int tm = 0; tm < TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < TN; ++tn)
      *reinterpret_cast<f32x4*>(&s_part[wave][(tm * 16 + fr) * PS + tn * 16 + 4 * (lane >> 4)]) =
          acc[tn][tm];
  __syncthreads();

  auto wave_sum4 = [&](int ml, int nl) __attribute__((always_inline)) {
    f32x4 t = *reinterpret_cast<const f32x4*>(&s_part[0][ml * PS + nl]);
#pragma unroll
    for (int w = 1; w < SK_WAVES; ++w)
      t += *reinterpret_cast<const f32x4*>(&s_part[w][ml * PS + nl]);
    return t;
  };
  constexpr int G4 = BM * BN / 4;  // 4-column groups of the tile
  if (S > 1) {
    const int tile = blockIdx.y * gridDim.x + blockIdx.x;
    float* wt = p.ws + (long)tile * S * PSZ;
    // The partials are written and read with device-scope accesses, which
    // go through to the memory side instead of staying in one XCD's L2, and
    // every store is acknowledged (vmcnt = 0) before the barrier that
    // precedes this tile's counter increment: a workgroup that sees the
    // count reach S - 1 therefore reads every split's finished partial.
    // (A device-scope release/acquire fence pair orders the same way but
    // writes back and invalidates the whole L2 of each XCD: up to 5 us per
    // call at these sizes, measured on MI355X.)
    for (int u = tid; u < G4; u += NT) {
      const int ml = u / (BN / 4), nl = (u - ml * (BN / 4)) * 4;
      const f32x4 v = wave_sum4(ml, nl);
      float* d = wt + (long)z * PSZ + ml * BN + nl;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __hip_atomic_store(d + i, v[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (tid == 0)
      s_last = __hip_atomic_fetch_add(p.ws_cnt + tile, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(S - 1);
    __syncthreads();
    if (!s_last) return;
    // the total goes to wave 0's slot; the epilogue below then reads slot 0
    // only (sum in split order: the result does not depend on arrival order)
    for (int u = tid; u < G4; u += NT) {
      const int ml = u / (BN / 4), nl = (u - ml * (BN / 4)) * 4;
      f32x4 t = {0.f, 0.f, 0.f, 0.f};
      for (int zz = 0; zz < S; ++zz) {
        const float* q = wt + (long)zz * PSZ + ml * BN + nl;
#pragma unroll
        for (int i = 0; i < 4; ++i)
          t[i] += __hip_atomic_load(q + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      *reinterpret_cast<f32x4*>(&s_part[0][ml * PS + nl]) = t;
    }
    if (tid == 0)  // ready for the next call
      __hip_atomic_store(p.ws_cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
  }
  auto sum4 = [&](int ml, int nl, float v[4]) __attribute__((always_inline)) {
    const f32x4 t = S > 1 ? *reinterpret_cast<const f32x4*>(&s_part[0][ml * PS + nl])
                          : wave_sum4(ml, nl);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = t[i] * p.alpha;
  };
  // every thread handles ITER output groups: all their loads, then all stores
  // units per row: 4-column groups (paired: of the first half of each 64-block,
  // or of tile columns 0..7 for P16); the partner sits POFF tile columns on
  constexpr int UPR = P16 ? 2 : PAIRED ? BN / 64 * 8 : BN / 4;
  constexpr int POFF = P16 ? 8 : 32;
  // (a 16-column tile has 256 units: threads past them load in-tile unit 0
  // and store nothing)
  constexpr int UNITS = BM * UPR, ITER = (UNITS + NT - 1) / NT;
  static_assert(UNITS % NT == 0 || UNITS < NT, "epilogue units");
  int ml[ITER], nl[ITER], gm[ITER], gn[ITER];
  EpiIn e[ITER];
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int u = UNITS < NT && tid >= UNITS ? 0 : tid + it * NT;
    ml[it] = u / UPR;
    const int r = u - ml[it] * UPR;
    nl[it] = PAIRED && !P16 ? (r >> 3) * 64 + (r & 7) * 4 : r * 4;
    gm[it] = min(m0 + ml[it], p.M - 1);
    gn[it] = min(nbase + nl[it], p.N - 4);
  }
  epi_load_groups<EPI, ITER>(p, gm, gn, e);
#pragma unroll
  for (int it = 0; it < ITER; ++it) {
    const int m = m0 + ml[it], n = nbase + nl[it];
    if (m >= p.M || n >= p.N || (UNITS < NT && tid >= UNITS)) continue;
    float x1[4], x2[4];
    sum4(ml[it], nl[it], x1);
    if constexpr (PAIRED) sum4(ml[it], nl[it] + POFF, x2);
    epi_apply<EPI, ACT>(p, m, n, x1, x2, e[it]);
  }
}

// Row-major [rows, k] (leading dimension ldx) -> slab-blocked [k / 32][rows][32]:
// one thread per 16-byte piece, reading along rows and writing along slabs.
__global__ __launch_bounds__(256) void slab_block_kernel(const bf16* __restrict__ x, long ldx,
                                                         bf16* __restrict__ out, int rows, int k) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;  // piece index, slab-major
  const int per_slab_row = WBK / 8;
  const long per_slab = (long)rows * per_slab_row;
  if (i >= per_slab * (k / WBK)) return;
  const int slab = (int)(i / per_slab);
  const long rem = i - (long)slab * per_slab;
  const int r = (int)(rem / per_slab_row), q = (int)(rem - (long)r * per_slab_row);
  st8(out + i * 8, ld8(x + (long)r * ldx + slab * WBK + q * 8));
}

// ---- launch ---------------------------------------------------------------
enum TileId { T256 = 0, T128 = 1, T64x128 = 2, T64 = 3, S64 = 4, S32 = 5, T128S = 6,
              P128 = 7, W256 = 8, P64 = 9, P128x64 = 10, P64x128 = 11, S16 = 12, L128 = 13,
              L128x64 = 14, L64x128 = 15, L64 = 16, N32 = 17, N32x64 = 18, N96 = 19,
              NUM_TILES = 20 };

// Launches tile configuration t; SVLA_EINVAL for a tile / epilogue pair that
// has no kernel (the 128x64 pipeline, the 32-column skinny tile and the 32x32
// small tile have no paired RoPE / SiLU epilogue, the wide tile only the plain
// dense store), so a
// forced or mis-routed choice fails loudly instead of leaving C unwritten.
template <int AMODE, bool NORM, int EPI, int ACT>
int launch_tile(TileId t, dim3 grid, const GemmArgs& p, hipStream_t s) {
  switch (t) {
    case T256:
      hipLaunchKernelGGL((gemm_kernel<256, 256, 2, 2, 32, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case T128:
      hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2, 32, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case T64x128:
      hipLaunchKernelGGL((gemm_kernel<64, 128, 2, 2, 16, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case T64:
      hipLaunchKernelGGL((gemm_kernel<64, 64, 4, 1, 16, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case T128S:
      hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2, 16, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case S64:
      hipLaunchKernelGGL((skinny_kernel<64, AMODE, NORM, EPI, ACT>), grid, dim3(SK_WAVES * 64), 0, s, p);
      break;
    case P128:
      hipLaunchKernelGGL((gemm_pipe_kernel<128, 128, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case P64:
      hipLaunchKernelGGL((gemm_pipe_kernel<64, 64, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case P128x64:
      if constexpr (EPI != EPI_ROPE && EPI != EPI_SILU)
        hipLaunchKernelGGL((gemm_pipe_kernel<128, 64, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      else
        return SVLA_EINVAL;
      break;
    case P64x128:
      hipLaunchKernelGGL((gemm_pipe_kernel<64, 128, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case W256:
      if constexpr (AMODE == A_DENSE && !NORM && EPI == EPI_STORE) {
        if (p.res)
          hipLaunchKernelGGL((gemm_wide_kernel<AMODE, NORM, EPI, ACT, true>), grid, dim3(256), 0, s, p);
        else
          hipLaunchKernelGGL((gemm_wide_kernel<AMODE, NORM, EPI, ACT, false>), grid, dim3(256), 0, s, p);
      } else {
        return SVLA_EINVAL;
      }
      break;
    case S16:
      hipLaunchKernelGGL((skinny_kernel<16, AMODE, NORM, EPI, ACT>), grid, dim3(SK_WAVES * 64), 0, s, p);
      break;
    case L128:
      hipLaunchKernelGGL((gemm_line_kernel<128, 128, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case L128x64:
      if constexpr (EPI != EPI_ROPE && EPI != EPI_SILU)
        hipLaunchKernelGGL((gemm_line_kernel<128, 64, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      else
        return SVLA_EINVAL;
      break;
    case L64x128:
      hipLaunchKernelGGL((gemm_line_kernel<64, 128, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case L64:
      hipLaunchKernelGGL((gemm_line_kernel<64, 64, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case S32:
      if constexpr (EPI != EPI_ROPE && EPI != EPI_SILU)
        hipLaunchKernelGGL((skinny_kernel<32, AMODE, NORM, EPI, ACT>), grid, dim3(SK_WAVES * 64), 0, s, p);
      else
        return SVLA_EINVAL;
      break;
    case N32:
      if constexpr (EPI != EPI_ROPE && EPI != EPI_SILU)
        hipLaunchKernelGGL((gemm_small_kernel<32, 32, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      else
        return SVLA_EINVAL;
      break;
    case N32x64:
      hipLaunchKernelGGL((gemm_small_kernel<32, 64, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      break;
    case N96:
      if constexpr (EPI != EPI_ROPE && EPI != EPI_SILU)
        hipLaunchKernelGGL((gemm_small_kernel<96, 96, AMODE, NORM, EPI, ACT>), grid, dim3(256), 0, s, p);
      else
        return SVLA_EINVAL;
      break;
    default:
      return SVLA_EINVAL;
  }
  return 0;
}

constexpr int kNumCU = 256;

// Column blocks per XCD of the wide kernel's column-resident order (xcd_tile),
// or 0 for the grouped order: the fewest column groups whose weight panels
// (w_cn x 256 rows x K) fit kXcdWeightBytes of an XCD's 4 MB L2, with a tile
// for every workgroup of every XCD.  (ViT up-projection 98304x3072x768: 6
// column blocks, 2.4 MB, per XCD; O 98304x768x768: all 3; the QKV and down
// projections' panels do not fit.)
constexpr long kXcdWeightBytes = 2560L * 1024;
int wide_cols_per_xcd(int tiles_m, int tiles_n, int K, int grid) {
  if (grid % kNumXCD) return 0;
  const int members = grid / kNumXCD;
  for (int groups = 1; groups <= kNumXCD; groups *= 2) {
    if (tiles_n % groups) continue;
    const int cn = tiles_n / groups;
    if ((long)cn * WBN * K * 2 > kXcdWeightBytes) continue;
    const int xg = kNumXCD / groups;
    const int rows = (tiles_m + xg - 1) / xg;
    if ((tiles_m - (xg - 1) * rows) * cn < members) continue;  // the last XCD of a group
    return cn;
  }
  return 0;
}
constexpr int kSkinnyMaxM = 256;

struct TileCfg {
  TileId id;
  int bm, bn;
};

// Tuning override (svla_gemm_set_tile): -1 = automatic choice.  Strict: the
// forced tile is used as given, with no substitution for problems it cannot
// serve (those calls then fail with SVLA_EINVAL).
int g_force_tile = -1;
bool g_force_strict = false;

TileCfg tile_dims(TileId id) {
  switch (id) {
    case T256: return {T256, 256, 256};
    case T128: return {T128, 128, 128};
    case T128S: return {T128S, 128, 128};
    case P128: return {P128, 128, 128};
    case W256: return {W256, 256, 256};
    case P64: return {P64, 64, 64};
    case P128x64: return {P128x64, 128, 64};
    case P64x128: return {P64x128, 64, 128};
    case T64x128: return {T64x128, 64, 128};
    case T64: return {T64, 64, 64};
    case S64: return {S64, 64, 64};
    case S16: return {S16, 64, 16};
    case L128: return {L128, 128, 128};
    case L128x64: return {L128x64, 128, 64};
    case L64x128: return {L64x128, 64, 128};
    case L64: return {L64, 64, 64};
    case N32: return {N32, 32, 32};
    case N32x64: return {N32x64, 32, 64};
    case N96: return {N96, 96, 96};
    default: return {S32, 64, 32};
  }
}

// `plain`: dense A, no fused norm, plain store epilogue (the wide kernel's scope)
TileCfg pick_tile(int M, int N, int K, int epi, bool plain, bool wide_rows_ok, bool dense) {
  auto tiles = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  const bool paired = epi == EPI_ROPE || epi == EPI_SILU;
  const bool pipe_ok = K >= PBK;  // the pipelined kernels need one full K step
  // whole 4-step rounds and at least 8 K steps; 16-byte row stores (N, ldc,
  // ldr multiples of 8)
  const bool wide_ok = plain && K % (4 * WBK) == 0 && K >= 8 * WBK && wide_rows_ok;
  if (g_force_tile >= 0 && g_force_strict) return tile_dims((TileId)g_force_tile);
  if (g_force_tile >= 0 && !(paired && g_force_tile == S32)) {
    if (g_force_tile == W256 && !wide_ok) return pipe_ok ? tile_dims(P128) : tile_dims(T128);
    if (g_force_tile == P128 && !pipe_ok) return tile_dims(T128);
    if (g_force_tile == P64 && !pipe_ok) return tile_dims(T64);
    if ((g_force_tile == P128x64 || g_force_tile == P64x128) && !pipe_ok) return tile_dims(T64);
    if (g_force_tile == P128x64 && paired) return tile_dims(P64);  // paired needs 64-wide wave tiles
    const bool line_ok = K >= LBK;
    if ((g_force_tile == L128 || g_force_tile == L64x128) && !line_ok) return pipe_ok ? tile_dims(P128) : tile_dims(T128);
    if ((g_force_tile == L64 || g_force_tile == L128x64) && !line_ok) return pipe_ok ? tile_dims(P64) : tile_dims(T64);
    if (g_force_tile == L128x64 && paired) return tile_dims(L64);
    const bool small = g_force_tile == N32 || g_force_tile == N32x64 || g_force_tile == N96;
    if (small && !line_ok) return pipe_ok ? tile_dims(P64) : tile_dims(T64);
    if (g_force_tile == N32 && paired) return tile_dims(N32x64);
    if (g_force_tile == N96 && paired) return tile_dims(N32x64);
    return tile_dims((TileId)g_force_tile);
  }
  // 32-row small tiles (gemm_small_kernel) for dense problems up to 512 rows
  // while the grid stays within two workgroups per CU, measured on MI355X with
  // graph replay: the batch-1 prefix (241 rows) down 241x960x2560 14.1 ->
  // 7.7 us (the 32-column skinny tile needed a 2-way K split), O 241x960x960
  // 7.6 -> 5.0, cross K/V 241x320x320 5.2 -> 3.7, norm + QKV + RoPE
  // 241x1600x960 9.7 -> 7.3 (32 x 64); 482 rows: down 15.3 -> 9.3, norm + QKV
  // + RoPE 9.8 -> 9.0; 50 rows: O 50x720x960 6.6 -> 4.6, down 50x720x2048
  // 8.5 -> 6.3.  Not for paired epilogues up to 128 rows (norm + QKV + RoPE
  // 50x1600x720: 6.2 us on the 16-column skinny tile, 6.5 here), nor past 512
  // tiles (norm + gate|up 241x5120x960: 12.0 on the 64x64 line tile, 13.2
  // here; expert O 1600x720x960: 9.9 vs 10.5), nor for the gathers (connector
  // 192x960x12288: 40.2 vs 47.7, patch embedding 18.8 vs 23.3).
  // 96 x 96 small tiles for long-K problems of one such tile per CU, measured
  // on MI355X with graph replay: the batch-1 ViT down projection 3072x768x3072
  // 31.7 -> 27.4 us (256 tiles; its 64x64 line tile runs 576); short K loses
  // (ViT O 3072x768x768: 12.1 -> 13.5, QKV 19.1 -> 32.1), and so do the
  // paired / 64-column variants on every engine shape measured
  if (dense && !paired && K >= 2048 && M >= 2048 && tiles(96, 96) <= kNumCU)
    return tile_dims(N96);
  if (dense && M <= 512 && K >= LBK) {
    if (!paired && tiles(32, 32) <= 2 * kNumCU) return tile_dims(N32);
    if (paired && M > 128 && tiles(32, 64) <= 2 * kNumCU) return tile_dims(N32x64);
  }
  if (M <= kSkinnyMaxM) {
    // measured on MI355X (batch-1 expert and prefix shapes): each workgroup
    // pulls the whole A k-range, so narrower tiles spread the weight bytes
    // over more CUs at little extra cost while the grid still fits the chip.
    // 16 columns beat 32 / 64: expert O 50x720x960 7.6 -> 6.5 us; down
    // 50x720x2048 with 4 splits 9.3 -> 8.4; prefix O 241x960x960 8.4 -> 7.2;
    // paired (8 columns + their partners, bit-identical results) expert
    // norm + QKV + RoPE 50x1600x720 7.7 -> 6.2, norm + gate|up 50x4096x720
    // 7.7 -> 6.4.  Not past one tile per CU (prefix norm + QKV 241x1600x960:
    // 11.6 -> 15.0 us), nor for long K on grids over half the chip, where the
    // 32-column tile's split wins (prefix down 241x960x2560: 13.5 vs 14.0 us).
    // Paired problems past that go to the 64x64 LDS-DMA pipeline (prefix
    // norm + gate|up 241x5120x960: 21.5 -> 11.8 us on the 64-column skinny
    // tile; norm + QKV + RoPE 241x1600x960: 12.0 -> 10.1 us).
    const long t16 = tiles(64, 16);
    if (paired) {
      if (t16 <= kNumCU) return {S16, 64, 16};
      // past one 16-column tile per CU: the 64x64 line-DMA tile, measured on
      // MI355X (prefix norm + QKV + RoPE 241x1600x960: 11.1 us on the 64x64
      // LDS-DMA pipeline, 10.0 on the line tile)
      if (K >= LBK) return tile_dims(L64);
      return pipe_ok ? tile_dims(P64) : TileCfg{S64, 64, 64};
    }
    if (t16 <= kNumCU / 2 || (K < 1536 && t16 <= kNumCU)) return {S16, 64, 16};
    if (tiles(64, 64) < kNumCU / 2) return {S32, 64, 32};
    return {S64, 64, 64};
  }
  // measured on MI355X: 128x128 tiles win once the grid has ~4 waves of
  // workgroups; below that the 64x64 tile's larger grid wins
  // measured on MI355X (M = 98304, N = 3072): with its LDS-staged epilogue the
  // wide tile beats the 128x128 pipeline from K = 512 (K = 768 + GELU: 675 vs
  // 752 us; K = 3072: 1603 vs 2285 us) and loses below (K = 256: 465 vs 430)
  if (wide_ok && K >= 512 && tiles(WBM, WBN) >= 2 * kNumCU) return tile_dims(W256);
  const bool line_ok = K >= LBK;
  // dense A from M = 4096 (the batch-32 prefix, 7712 rows; its RMSNorm runs
  // on its own there), measured on MI355X with graph replay: the 128x128
  // line-DMA tile beats the register-staged 128x128 kernel and the other
  // pipelines on every prefix GEMM -- down 7712x960x2560 47.2 us, O
  // 7712x960x960 25.3, QKV + RoPE 7712x1600x960 43.8 (46.7 on 64x128), gate|up
  // + SiLU 7712x5120x960 93.4 (116.4 register-staged); a grid under one
  // 128x128 tile per CU takes the 64x64 line tile (the cross K/V projection
  // 7712x320x320: 9.4 -> 7.6 us).
  // The gathers from M = 4096 (the batch-32 patch embedding 98304x768x768
  // and pixel-shuffle connector 6144x960x12288), measured on MI355X with
  // graph replay: the register-staged 128x128 kernel -- patch 311 -> 219 us,
  // connector 310 -> 211 us against the 64x64 line tile the M >= 3072 rule
  // below would take (the 128x128 LDS-DMA pipeline: 235 / 210 us)
  if (!dense && M >= 4096) return tile_dims(T128);
  if (dense && M >= 4096) {
    if (!line_ok) return tile_dims(T128);
    if (tiles(128, 128) < kNumCU) return tile_dims(L64);
    return tile_dims(L128);
  }
  // from M = 3072 (the batch-1 ViT, 3 images), measured on MI355X, line-DMA
  // tiles: up 3072x3072x768 + GELU 38.0 -> 27.8 us (128x64), QKV
  // 3072x2304x768 22.9 -> 18.8 (128x128), down 3072x768x3072 35.8 -> 29.9 and
  // O 3072x768x768 14.0 -> 11.2 (64x64)
  if (M >= 3072 && line_ok && !paired) {
    if (N >= 3072) return tile_dims(L128x64);
    if (N >= 2048) return tile_dims(L128);
    return tile_dims(L64);
  }
  // from M = 3072 (the batch-1 ViT, 3 images) too, measured on MI355X: up
  // 3072x3072x768 + GELU 38.1 -> 35.0 us, down 3072x768x3072 42.7 -> 34.1 us,
  // QKV and O within 0.4 us
  if (M >= 3072 || tiles(128, 128) >= 4 * kNumCU) return pipe_ok ? tile_dims(P128) : tile_dims(T128);
  // mid-size (the batched expert, M = 1600), measured on MI355X: with at least
  // one 128x128 tile per CU the 32x32-MFMA register-staged 128x128 kernel wins
  // (gate|up 1600x4096x720: 19 us vs 34 us on 64x64); below that the 64x64
  // LDS-DMA pipeline's larger grid wins
  if (tiles(128, 128) >= kNumCU) return tile_dims(T128);
  if (!pipe_ok) return tile_dims(T64);
  // paired epilogues below one 128x128 tile per CU, measured on MI355X (the
  // expert at batch 32, M = 1600): the 64x64 line-DMA tile -- norm + QKV +
  // RoPE 1600x1600x720 19.3 -> 14.5 us, norm + Q + RoPE 1600x960x720 12.2 ->
  // 11.1
  if (paired && line_ok) return tile_dims(L64);
  // below that, measured on MI355X: when the 64x64 grid would put one or two
  // workgroups on each CU (256-512 tiles, uneven), a 128x64 / 64x128 tile
  // halves the grid to about one per CU (expert at batch 32, M = 1600: O
  // 12.5 -> 10.9 us, down 19.3 -> 16.9 us, Q + RoPE 12.1 -> 11.0 us; M =
  // 1928, K = 2560: 25.4 -> 22.4 us); with fewer tiles, or more (the batch-1
  // ViT's 576), 64x64 stays ahead.  Paired epilogues need 64-wide wave tiles:
  // 64x128, or 128x128 for large paired grids (QKV + RoPE 1600 x 720:
  // 17.7 -> 15.2 us).
  // Re-measured with the current kernels (graph replay, M = 1600): the
  // 128x64 tile still wins for long K (down, K = 2048: 17.8 vs 19.9 us) but
  // not for short K (time MLP 1600x720x720: 10.3 vs 9.4 us on 64x64; O,
  // K = 960: 11.0 vs 10.6).
  const long t64 = tiles(64, 64);
  if (t64 >= kNumCU && t64 <= 2 * kNumCU && (paired || K > 1024))
    return tile_dims(paired ? P64x128 : P128x64);
  if (paired && t64 > 2 * kNumCU && tiles(128, 128) >= kNumCU / 2) return tile_dims(P128);
  return tile_dims(P64);
}

// ---- skinny split-K --------------------------------------------------------
// Workspace: one per device, allocated on the first split call that is not
// being captured into a graph and kept for the life of the process (a split
// call on a capturing stream before that runs unsplit).  All split calls on a
// device share it, so such calls on different streams must not overlap in
// time; calls on one stream, and replays of graphs captured from them, are
// ordered.  svla_gemm_set_split(1) turns splitting off.
constexpr size_t kWsFloats = (size_t)4 << 20;  // 16 MB of fp32 partial tiles
constexpr int kWsTiles = 4096;                 // arrival counters
constexpr int kMaxDevices = 64;
struct SplitWs {
  float* part;
  unsigned* cnt;
};
SplitWs g_ws[kMaxDevices];
std::mutex g_ws_mu;
int g_force_split = -1;  // svla_gemm_set_split: -1 = automatic

const SplitWs* split_ws(hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  SplitWs& w = g_ws[dev];
  if (w.part) return &w;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
  float* part = nullptr;
  unsigned* cnt = nullptr;
  if (hipMalloc(&part, kWsFloats * sizeof(float)) != hipSuccess) return nullptr;
  if (hipMalloc(&cnt, kWsTiles * sizeof(unsigned)) != hipSuccess ||
      hipMemset(cnt, 0, kWsTiles * sizeof(unsigned)) != hipSuccess) {
    (void)hipFree(part);
    if (cnt) (void)hipFree(cnt);
    return nullptr;
  }
  w.part = part;
  w.cnt = cnt;
  return &w;
}

// ---- allocation-free split-K scratch (svla_linear_scratch_bf16) ------------
// A static device array stands in for the allocated workspace: kScratchFloats
// fp32 partial-tile slots, then kScratchTiles arrival counters (4 MB + 4 KB).
// Every device the library runs on holds its own copy from module load until
// the process ends.  In host code `scratch` names a host-side stand-in, not a
// device address: its address on each device is resolved once, with that
// device current, by hipGetSymbolAddress, and only that pointer is passed to
// kernels.  The counters are cleared when the address is resolved; each split
// call's last workgroup returns its tile's counter to zero.
constexpr size_t kScratchFloats = (size_t)1 << 20;
constexpr int kScratchTiles = 1024;
static __device__ __align__(256) float scratch[kScratchFloats + kScratchTiles];

__global__ void fill_u32_kernel(unsigned* p, int n, unsigned v) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

struct ScratchDev {
  SplitWs ws;
  bool ready;
};
ScratchDev g_scr[kMaxDevices];

// This device's scratch (resolved and cleared on stream s at the first call
// per device), or nullptr with *err set.
const SplitWs* scratch_ws(hipStream_t s, hipError_t* err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_ws_mu);
  ScratchDev& d = g_scr[dev];
  if (!d.ready) {
    void* ptr = nullptr;
    *err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (*err != hipSuccess || !ptr) return nullptr;
    float* base = static_cast<float*>(ptr);
    unsigned* cnt = reinterpret_cast<unsigned*>(base + kScratchFloats);
    hipLaunchKernelGGL(fill_u32_kernel, dim3((kScratchTiles + 255) / 256), dim3(256), 0, s, cnt,
                       kScratchTiles, 0u);
    *err = hipGetLastError();
    if (*err != hipSuccess) return nullptr;
    d.ws.part = base;
    d.ws.cnt = cnt;
    d.ready = true;
  }
  return &d.ws;
}

// Number of K splits for a skinny grid of `tiles` workgroups.  Measured on
// MI355X (bs=1 expert, prefix and connector shapes): a split costs ~1-2 us of
// partial stores, counter round trip and partial loads, which only long K
// repays -- K = 2048 at 23 tiles: 12.7 -> 10.2 us (S = 4); K = 2560 at 120
// tiles: 17.5 -> 14.3 us (S = 2); K = 12288 at 90 tiles: 69 -> 40 us (S = 2);
// K <= 960 always lost.  So: K >= 1536, at most one workgroup per CU, and at
// least 16 k-steps of 32 per split.
int pick_split(int tiles, int K, int bm, int bn) {
  const int nkf = K / 32;
  int S;
  if (g_force_split >= 1) {
    S = g_force_split;
  } else {
    if (K < 1536) return 1;
    S = min(kNumCU / tiles, nkf / 16);
  }
  S = min(S, max(1, nkf));
  // workspace capacity
  // (a partial is the fp32 tile)
  while (S > 1 && ((size_t)tiles * S * bm * bn > kWsFloats || tiles > kWsTiles)) --S;
  return max(S, 1);
}

template <int AMODE, bool NORM>
int dispatch(const GemmArgs& p, int epi, int act, TileId t, dim3 grid, hipStream_t s) {
  int rc;
  switch (epi) {
    case EPI_ROPE: rc = launch_tile<AMODE, NORM, EPI_ROPE, 0>(t, grid, p, s); break;
    case EPI_SILU: rc = launch_tile<AMODE, NORM, EPI_SILU, 0>(t, grid, p, s); break;
    case EPI_EULER: rc = launch_tile<AMODE, NORM, EPI_EULER, 0>(t, grid, p, s); break;
    default:
      switch (act) {
        case SVLA_ACT_GELU_TANH: rc = launch_tile<AMODE, NORM, EPI_STORE, SVLA_ACT_GELU_TANH>(t, grid, p, s); break;
        case SVLA_ACT_GELU_ERF: rc = launch_tile<AMODE, NORM, EPI_STORE, SVLA_ACT_GELU_ERF>(t, grid, p, s); break;
        case SVLA_ACT_SILU: rc = launch_tile<AMODE, NORM, EPI_STORE, SVLA_ACT_SILU>(t, grid, p, s); break;
        default: rc = launch_tile<AMODE, NORM, EPI_STORE, SVLA_ACT_NONE>(t, grid, p, s);
      }
  }
  if (rc) return rc;
  SVLA_CHECK_LAUNCH();
  return 0;
}

// Where the split-K partials of skinny problems go: the allocated per-device
// workspace (svla_linear_bf16 and the other entry points) or the static
// scratch array (svla_linear_scratch_bf16).
enum WsKind { WS_ALLOCATED = 0, WS_SCRATCH = 1 };

template <int AMODE>
int run_gemm(GemmArgs& p, int epi, int act, hipStream_t s, WsKind wk = WS_ALLOCATED) {
  if (p.M < 0 || p.N <= 0 || p.K <= 0) return SVLA_EINVAL;
  if (p.M == 0) return 0;
  if (p.K % 8 || p.N % 4 || p.ldb % 8 || p.ldc % 4) return SVLA_EINVAL;
  if (AMODE == A_DENSE && (p.lda % 8 || !svla_aligned16(p.a))) return SVLA_EINVAL;
  if (!svla_aligned16(p.b) || !svla_aligned16(p.c)) return SVLA_EINVAL;
  if (p.res && (p.ldr % 4)) return SVLA_EINVAL;
  if ((epi == EPI_ROPE || epi == EPI_SILU) && p.N % 64) return SVLA_EINVAL;
  if (epi == EPI_ROPE && (p.rope_cols % 64 || p.rope_period <= 0)) return SVLA_EINVAL;
  if (AMODE != A_DENSE && act) return SVLA_EINVAL;
  if (p.norm_w && (AMODE != A_DENSE || !svla_aligned16(p.norm_w))) return SVLA_EINVAL;

  const bool plain =
      AMODE == A_DENSE && !p.norm_w && epi == EPI_STORE && !p.rowadd && p.c_rpg <= 0;
  const bool wide_rows_ok = !p.out_f32 && p.N % 8 == 0 && p.ldc % 8 == 0 &&
                            (!p.res || (p.ldr % 8 == 0 && svla_aligned16(p.res)));
  const TileCfg t = pick_tile(p.M, p.N, p.K, epi, plain, wide_rows_ok, AMODE == A_DENSE);
  if (p.norm_w && p.K > 2048) return SVLA_EINVAL;  // the gain vector is staged in LDS (<= 2048)
  // a pipelined kernel needs one full K stage, the wide one whole 4-step
  // rounds of at least 8 steps (a strictly forced tile may violate either:
  // refused here, before any launch)
  const bool pipe = t.id == P128 || t.id == P64 || t.id == P128x64 || t.id == P64x128;
  const bool line = t.id == L128 || t.id == L64 || t.id == L128x64 || t.id == L64x128 ||
                    t.id == N32 || t.id == N32x64 || t.id == N96;
  if ((pipe && p.K < PBK) || (line && p.K < LBK)) return SVLA_EINVAL;
  if (t.id == W256 && !(plain && p.K % (4 * WBK) == 0 && p.K >= 8 * WBK && wide_rows_ok))
    return SVLA_EINVAL;
  const int gm = (p.M + t.bm - 1) / t.bm, gn = (p.N + t.bn - 1) / t.bn;
  dim3 grid(gn, gm, 1);
  if (t.id == W256) {  // persistent: one workgroup per CU walks the tiles
    p.tiles_m = gm;
    p.tiles_n = gn;
    grid = dim3(min(gm * gn, kNumCU), 1, 1);
    p.w_cn = wide_cols_per_xcd(gm, gn, p.K, (int)grid.x);
  }
  if (t.id == S32 || t.id == S64 || t.id == S16) {
    const int S = pick_split(gm * gn, p.K, t.bm, t.bn);
    const SplitWs* w = nullptr;
    if (S > 1 && wk == WS_SCRATCH) {
      // the same split as the allocated workspace would take, or an error:
      // the results stay bit-identical to svla_linear_bf16's
      if ((size_t)gm * gn * S * (t.bm * t.bn + t.bm) > kScratchFloats || gm * gn > kScratchTiles)
        return SVLA_ENOSPC;
      hipError_t e = hipSuccess;
      w = scratch_ws(s, &e);
      if (!w) return e != hipSuccess ? (int)e : SVLA_EINVAL;
    } else if (S > 1) {
      w = split_ws(s);
    }
    if (w) {
      p.ws = w->part;
      p.ws_cnt = w->cnt;
      grid.z = S;
    }
  }
  if constexpr (AMODE == A_DENSE) {
    if (p.norm_w) return dispatch<AMODE, true>(p, epi, act, t.id, grid, s);
  }
  return dispatch<AMODE, false>(p, epi, act, t.id, grid, s);
}

GemmArgs base_args(const void* a, long lda, const void* w, long ldw, void* c, long ldc, int m,
                   int n, int k) {
  GemmArgs p{};
  p.a = static_cast<const bf16*>(a);
  p.lda = lda;
  p.b = static_cast<const bf16*>(w);
  p.ldb = ldw;
  p.c = c;
  p.ldc = ldc;
  p.M = m;
  p.N = n;
  p.K = k;
  p.alpha = 1.0f;
  return p;
}

}  // namespace

extern "C" {

int svla_version(void) { return 200; }

int svla_gemm_set_tile(int tile) {
  const bool strict = tile >= 0 && (tile & SVLA_TILE_STRICT);
  if (strict) tile &= ~SVLA_TILE_STRICT;
  if (tile < -1 || tile >= NUM_TILES) return SVLA_EINVAL;
  g_force_tile = tile;
  g_force_strict = strict;
  return SVLA_OK;
}

int svla_gemm_tile_choice(int m, int n, int k, int act) {
  if (m <= 0 || n <= 0 || k <= 0 || act < 0 || act > SVLA_ACT_SILU) return SVLA_EINVAL;
  (void)act;  // the choice depends on the epilogue kind, not on the activation
  return (int)pick_tile(m, n, k, EPI_STORE, true, n % 8 == 0, true).id;
}

int svla_gemm_set_split(int splits) {
  if (splits < -1 || splits == 0 || splits > 64) return SVLA_EINVAL;
  g_force_split = splits;
  return SVLA_OK;
}

int svla_linear_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                     const float* bias_f32, const void* res, int ldr, void* c, int ldc, int m,
                     int n, int k, float alpha, int act, int out_f32, const void* norm_w,
                     float norm_eps, svla_stream_t stream) {
  if (act < 0 || act > SVLA_ACT_SILU) return SVLA_EINVAL;
  if (out_f32 && (act || res)) return SVLA_EINVAL;
  if (bias_f32 && !svla_aligned16(bias_f32)) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w, ldw, c, ldc, m, n, k);
  p.alpha = alpha;
  p.bias = static_cast<const bf16*>(bias);
  p.bias_f32 = bias_f32;
  p.res = static_cast<const bf16*>(res);
  p.ldr = ldr;
  p.out_f32 = out_f32;
  p.norm_w = static_cast<const bf16*>(norm_w);
  p.norm_eps = norm_eps;
  return run_gemm<A_DENSE>(p, EPI_STORE, act, (hipStream_t)stream);
}

int svla_linear_scratch_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                             const float* bias_f32, const void* res, int ldr, void* c, int ldc,
                             int m, int n, int k, float alpha, int act, int out_f32,
                             const void* norm_w, float norm_eps, svla_stream_t stream) {
  if (act < 0 || act > SVLA_ACT_SILU) return SVLA_EINVAL;
  if (out_f32 && (act || res)) return SVLA_EINVAL;
  if (bias_f32 && !svla_aligned16(bias_f32)) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w, ldw, c, ldc, m, n, k);
  p.alpha = alpha;
  p.bias = static_cast<const bf16*>(bias);
  p.bias_f32 = bias_f32;
  p.res = static_cast<const bf16*>(res);
  p.ldr = ldr;
  p.out_f32 = out_f32;
  p.norm_w = static_cast<const bf16*>(norm_w);
  p.norm_eps = norm_eps;
  return run_gemm<A_DENSE>(p, EPI_STORE, act, (hipStream_t)stream, WS_SCRATCH);
}

int svla_init(void) {
  if (!split_ws(nullptr)) return hipErrorOutOfMemory;
  hipError_t e = hipSuccess;
  if (!scratch_ws(nullptr, &e)) return e != hipSuccess ? (int)e : SVLA_EINVAL;
  return (int)hipDeviceSynchronize();
}

int svla_linear_wide_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                          const float* bias_f32, const void* res, int ldr, void* c, int ldc, int m,
                          int n, int k, float alpha, int act, int layout, svla_stream_t stream) {
  if (act < 0 || act > SVLA_ACT_SILU || (layout & ~7)) return SVLA_EINVAL;
  if (m <= 0 || m % WBM || n % WBN || k % (4 * WBK) || k < 8 * WBK) return SVLA_EINVAL;
  if ((long)m * k > (1L << 31) || (long)n * k > (1L << 31)) return SVLA_EINVAL;
  if (bias_f32 && !svla_aligned16(bias_f32)) return SVLA_EINVAL;
  if (res && ((layout & SVLA_LAYOUT_C_BLOCKED) || ldr % 8 || !svla_aligned16(res))) return SVLA_EINVAL;
  GemmArgs p = base_args(a, (layout & SVLA_LAYOUT_A_BLOCKED) ? k : lda, w,
                         (layout & SVLA_LAYOUT_W_BLOCKED) ? k : ldw, c,
                         (layout & SVLA_LAYOUT_C_BLOCKED) ? n : ldc, m, n, k);
  if (p.lda % 8 || p.ldb % 8 || p.ldc % 8 || !svla_aligned16(a) || !svla_aligned16(w) ||
      !svla_aligned16(c))
    return SVLA_EINVAL;
  p.alpha = alpha;
  p.bias = static_cast<const bf16*>(bias);
  p.bias_f32 = bias_f32;
  p.res = static_cast<const bf16*>(res);
  p.ldr = ldr;
  p.a_blk = (layout & SVLA_LAYOUT_A_BLOCKED) != 0;
  p.b_blk = (layout & SVLA_LAYOUT_W_BLOCKED) != 0;
  p.c_blk = (layout & SVLA_LAYOUT_C_BLOCKED) != 0;
  p.tiles_m = m / WBM;
  p.tiles_n = n / WBN;
  const dim3 grid(min(p.tiles_m * p.tiles_n, kNumCU), 1, 1);
  p.w_cn = wide_cols_per_xcd(p.tiles_m, p.tiles_n, k, (int)grid.x);
  return dispatch<A_DENSE, false>(p, EPI_STORE, act, W256, grid, (hipStream_t)stream);
}

int svla_slab_block_bf16(const void* x, int ldx, void* out, int rows, int k, svla_stream_t stream) {
  if (rows <= 0 || k <= 0 || k % WBK || ldx < k) return SVLA_EINVAL;
  const long total = (long)rows * k / 8;  // 16-byte pieces
  hipLaunchKernelGGL(slab_block_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const bf16*>(x), (long)ldx,
                     static_cast<bf16*>(out), rows, k);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_linear_rope_lo_bf16(const void* a, int lda, const void* w, int ldw, void* c,
                             void* c_lo, int ldc, int m, int n, int k, int rope_cols, int seq_len,
                             const float* cos_t, const float* sin_t, const void* norm_w,
                             float norm_eps, svla_stream_t stream) {
  if (!cos_t || !sin_t || rope_cols > n) return SVLA_EINVAL;
  if (!svla_aligned16(cos_t) || !svla_aligned16(sin_t)) return SVLA_EINVAL;
  if (c_lo && ((uintptr_t)c_lo & 7)) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w, ldw, c, ldc, m, n, k);
  p.rope_cos = cos_t;
  p.rope_sin = sin_t;
  p.rope_cols = rope_cols;
  p.rope_period = seq_len;
  p.c_lo = static_cast<bf16*>(c_lo);
  p.norm_w = static_cast<const bf16*>(norm_w);
  p.norm_eps = norm_eps;
  return run_gemm<A_DENSE>(p, EPI_ROPE, 0, (hipStream_t)stream);
}

int svla_linear_rope_bf16(const void* a, int lda, const void* w, int ldw, void* c, int ldc,
                          int m, int n, int k, int rope_cols, int seq_len, const float* cos_t,
                          const float* sin_t, const void* norm_w, float norm_eps,
                          svla_stream_t stream) {
  return svla_linear_rope_lo_bf16(a, lda, w, ldw, c, nullptr, ldc, m, n, k, rope_cols, seq_len,
                                  cos_t, sin_t, norm_w, norm_eps, stream);
}

int svla_linear_silu_mul_bf16(const void* a, int lda, const void* w_gu, int ldw, void* out,
                              int ldo, int m, int inter, int k, const void* norm_w,
                              float norm_eps, svla_stream_t stream) {
  if (inter % 32) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w_gu, ldw, out, ldo, m, 2 * inter, k);
  p.norm_w = static_cast<const bf16*>(norm_w);
  p.norm_eps = norm_eps;
  return run_gemm<A_DENSE>(p, EPI_SILU, 0, (hipStream_t)stream);
}

int svla_patch_embed_bf16(const void* images, const void* w, const void* bias, const void* pos,
                          void* out, int ldo, int n_img, int chans, int image, int patch,
                          int embed, svla_stream_t stream) {
  if (patch % 8 || image % patch || !svla_aligned16(images)) return SVLA_EINVAL;
  if (pos && !svla_aligned16(pos)) return SVLA_EINVAL;
  const int G = image / patch;
  const int K = chans * patch * patch;
  GemmArgs p = base_args(images, 0, w, K, out, ldo, n_img * G * G, embed, K);
  p.p_chans = chans;
  p.p_img = image;
  p.p_patch = patch;
  p.bias = static_cast<const bf16*>(bias);
  p.rowadd = static_cast<const bf16*>(pos);
  p.rowadd_period = G * G;
  return run_gemm<A_PATCH>(p, EPI_STORE, 0, (hipStream_t)stream);
}

int svla_connector_bf16(const void* x, const void* w, int ldw, void* out, int ldo, int n_img,
                        int grid, int hidden, int scale, int n_out, int rows_per_sample,
                        int sample_stride, svla_stream_t stream) {
  if (hidden % 8 || grid % scale || !svla_aligned16(x)) return SVLA_EINVAL;
  if (rows_per_sample < 0 || (rows_per_sample > 0 && sample_stride < rows_per_sample))
    return SVLA_EINVAL;
  const int gs = grid / scale;
  const int K = hidden * scale * scale;
  GemmArgs p = base_args(x, 0, w, ldw, out, ldo, n_img * gs * gs, n_out, K);
  p.g_grid = grid;
  p.g_hidden = hidden;
  p.g_scale = scale;
  p.c_rpg = rows_per_sample;
  p.c_gstride = sample_stride;
  return run_gemm<A_PSHUF>(p, EPI_STORE, 0, (hipStream_t)stream);
}

int svla_action_out_euler(const void* a, int lda, const void* w, int ldw, float* x_f32,
                          int ldx, void* x_bf16, int ldxb, int m, int n, int k,
                          const void* norm_w, float norm_eps, float dt, svla_stream_t stream) {
  if (!x_f32 || ldx % 4 || (x_bf16 && ldxb % 4)) return SVLA_EINVAL;
  // c is unused by the Euler epilogue but must satisfy the alignment check
  GemmArgs p = base_args(a, lda, w, ldw, x_f32, 4, m, n, k);
  p.x_f32 = x_f32;
  p.ldx = ldx;
  p.x_bf16 = static_cast<bf16*>(x_bf16);
  p.ldxb = ldxb;
  p.dt = dt;
  p.norm_w = static_cast<const bf16*>(norm_w);
  p.norm_eps = norm_eps;
  return run_gemm<A_DENSE>(p, EPI_EULER, 0, (hipStream_t)stream);
}

}  // extern "C"
