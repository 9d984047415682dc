// bf16 MFMA GEMM for gfx950 with fused epilogues.
//
//   C[M, N] = epilogue(alpha * A[M, K] . W[N, K]^T)
//
// Replaces the Allo GEMM region (cc/gemm.py:44-77, instantiated e.g. at
// vla/text_encoder_bf16.py:174-225) and the host-side K-chunk accumulation
// loops (vla/text_encoder_bf16.py:584-590, vla/connector_bf16.py:116-126).
//
// Design (CDNA4):
//  * 256 threads = 4 wave64s per workgroup; block tile BM x BN, K step 64.
//  * Global -> register prefetch of the next K tile while the current one is
//    consumed from LDS; LDS double buffer, one barrier per K step.  LDS rows are
//    padded by 16 bytes so the 16-byte MFMA operand reads of 8 consecutive rows
//    hit 8 distinct 4-bank groups.
//  * v_mfma_f32_16x16x32_bf16 with the WEIGHT tile as the A operand and the
//    activation tile as the B operand, so each lane's accumulator holds 4
//    consecutive output COLUMNS of one row: epilogues (bias, RoPE pairs
//    (d, d+32), SiLU(gate)*up pairs, residual) are lane-local and stores are
//    8-byte vectors.
//  * The A operand can be gathered: the pixel-shuffle of the connector and the
//    im2col of the patch embedding are folded into the A-tile addressing, so
//    neither is ever materialised in HBM.
//  * Small-M shapes (bs=1 prefix / expert) use split-K over an fp32 workspace
//    plus a reduce kernel that applies the same epilogue (deterministic, no
//    atomics, no memset -> safe under HIP graph capture).
#include "svla_common.h"

namespace {

enum AMode { A_DENSE = 0, A_PSHUF = 1, A_PATCH = 2 };
enum Epi { EPI_STORE = 0, EPI_ROPE = 1, EPI_SILU = 2, EPI_EULER = 3, EPI_PARTIAL = 4 };

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
  int act;
  int out_f32;
  const float* rope_cos;
  const float* rope_sin;
  int rope_cols;
  int rope_period;
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
  // split-K
  float* ws;
  long ws_bytes;
  int splits;
  int kt_per_split;
};

__device__ __forceinline__ long crow(const GemmArgs& p, int m) {
  if (p.c_rpg <= 0) return m;
  const int g = m / p.c_rpg;
  return (long)g * p.c_gstride + (m - g * p.c_rpg);
}

__device__ __forceinline__ float apply_act(int act, float v) {
  switch (act) {
    case SVLA_ACT_GELU_TANH: return gelu_tanh_f(v);
    case SVLA_ACT_GELU_ERF: return gelu_erf_f(v);
    case SVLA_ACT_SILU: return silu_f(v);
    default: return v;
  }
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

// ---- epilogues: each handles 4 consecutive columns of one row -------------
// v already includes alpha.  ACT is a compile-time activation (SVLA_ACT_*).
template <int ACT>
__device__ __forceinline__ void epi_store(const GemmArgs& p, int m, int n, float v[4]) {
  if (p.bias) {
    float b[4];
    load_bf16x4(p.bias + n, b);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += b[i];
  }
  if (p.bias_f32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] += p.bias_f32[n + i];
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
    for (int i = 0; i < 4; ++i) v[i] = rbf(apply_act(ACT, v[i]));
  }
  if (p.rowadd) {
    float r[4];
    load_bf16x4(p.rowadd + (long)(m % p.rowadd_period) * p.N + n, r);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = rbf(v[i] + r[i]);
  }
  if (p.res) {
    float r[4];
    load_bf16x4(p.res + (long)m * p.ldr + n, r);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = rbf(v[i] + r[i]);
  }
  store_bf16x4(reinterpret_cast<bf16*>(p.c) + crow(p, m) * p.ldc + n, v);
}

// RoPE pair: x1 at columns n1..n1+3 (head dims d..d+3 < 32), x2 at n1+32.
// Mirrors apply_rope on the bf16 projection (vla/text_encoder_bf16.py:92-104):
// out1 = x1*cos - x2*sin, out2 = x2*cos + x1*sin in fp32, then bf16.
__device__ __forceinline__ void epi_rope(const GemmArgs& p, int m, int n1, float x1[4],
                                         float x2[4]) {
  bf16* c = reinterpret_cast<bf16*>(p.c) + crow(p, m) * p.ldc;
#pragma unroll
  for (int i = 0; i < 4; ++i) { x1[i] = rbf(x1[i]); x2[i] = rbf(x2[i]); }
  if (n1 < p.rope_cols) {
    const int pos = m % p.rope_period;
    const int d = n1 & 63;
    const float* ct = p.rope_cos + pos * 32 + d;
    const float* st = p.rope_sin + pos * 32 + d;
    float o1[4], o2[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float cs = ct[i], sn = st[i];
      o1[i] = __fsub_rn(__fmul_rn(x1[i], cs), __fmul_rn(x2[i], sn));
      o2[i] = __fadd_rn(__fmul_rn(x2[i], cs), __fmul_rn(x1[i], sn));
    }
    store_bf16x4(c + n1, o1);
    store_bf16x4(c + n1 + 32, o2);
  } else {
    store_bf16x4(c + n1, x1);
    store_bf16x4(c + n1 + 32, x2);
  }
}

// gated MLP: out = bf16(bf16(silu(bf16(g))) * bf16(u))  (nn.SiLU on the bf16
// gate projection, then the bf16 hadamard product, vla/text_encoder_bf16.py:130-131)
__device__ __forceinline__ void epi_silu(const GemmArgs& p, int m, int nout, float g[4],
                                         float u[4]) {
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = rbf(silu_f(rbf(g[i]))) * rbf(u[i]);
  store_bf16x4(reinterpret_cast<bf16*>(p.c) + crow(p, m) * p.ldc + nout, o);
}

// Euler step x <- x + dt * bf16(v) in fp32 (+ optional bf16 copy of x).
__device__ __forceinline__ void epi_euler(const GemmArgs& p, int m, int n, float v[4]) {
  float* x = p.x_f32 + (long)m * p.ldx + n;
  float o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[i] = __fadd_rn(x[i], __fmul_rn(p.dt, rbf(v[i])));
    x[i] = o[i];
  }
  if (p.x_bf16) store_bf16x4(p.x_bf16 + (long)m * p.ldxb + n, o);
}

// ---- A operand gather -------------------------------------------------------
template <int AMODE>
__device__ __forceinline__ bf16x8 load_a(const GemmArgs& p, int m, int k) {
  if (m >= p.M || k >= p.K) return bf16x8{};
  const bf16* src;
  if constexpr (AMODE == A_DENSE) {
    src = p.a + (long)m * p.lda + k;
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
    src = p.a + ((long)img * grid * grid + tok) * E + c;
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
    src = p.a + (((long)img * p.p_chans + ch) * H + pr * P + ky) * H + pc * P + kx;
  }
  return ld8(src);
}

constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // elements; +16 bytes of padding per row

template <int BM, int BN, int WAVES_M, int WAVES_N, int AMODE, int EPI, int ACT = SVLA_ACT_NONE>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p) {
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_CH = BM * BK / 8 / 256;
  constexpr int B_CH = BN * BK / 8 / 256;
  static_assert(WAVES_M * WAVES_N == 4, "4 waves");
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small");
  static_assert(EPI != EPI_ROPE || WN % 64 == 0, "RoPE needs whole heads per wave");
  static_assert(EPI != EPI_SILU || TN % 2 == 0, "SiLU pairs gate/up subtiles");

  __shared__ __attribute__((aligned(16))) bf16 sA[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) bf16 sB[2][BN * LDS_STRIDE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int nk_total = (p.K + BK - 1) / BK;
  int kt_begin = 0, kt_end = nk_total;
  if constexpr (EPI == EPI_PARTIAL) {
    kt_begin = blockIdx.z * p.kt_per_split;
    kt_end = min(nk_total, kt_begin + p.kt_per_split);
  }

  f32x4 acc[TN][TM];
#pragma unroll
  for (int i = 0; i < TN; ++i)
#pragma unroll
    for (int j = 0; j < TM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  bf16x8 ra[A_CH], rb[B_CH];

  auto gload = [&](int kt) {
    const int kb = kt * BK;
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 3, kc = c & 7;
      ra[i] = load_a<AMODE>(p, m0 + row, kb + kc * 8);
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * 256;
      const int row = c >> 3, kc = c & 7;
      const int n = n0 + row, k = kb + kc * 8;
      rb[i] = (n < p.N && k < p.K) ? ld8(p.b + (long)n * p.ldb + k) : bf16x8{};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<bf16x8*>(&sA[buf][(c >> 3) * LDS_STRIDE + (c & 7) * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int c = tid + i * 256;
      *reinterpret_cast<bf16x8*>(&sB[buf][(c >> 3) * LDS_STRIDE + (c & 7) * 8]) = rb[i];
    }
  };

  const int frag_row = lane & 15;
  const int frag_k = (lane >> 4) * 8;

  if (kt_begin < kt_end) {
    gload(kt_begin);
    sstore(0);
    __syncthreads();
    for (int kt = kt_begin; kt < kt_end; ++kt) {
      const int cur = (kt - kt_begin) & 1;
      if (kt + 1 < kt_end) gload(kt + 1);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        bf16x8 fw[TN], fx[TM];
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
          fw[tn] = *reinterpret_cast<const bf16x8*>(
              &sB[cur][(wn * WN + tn * 16 + frag_row) * LDS_STRIDE + ks * 32 + frag_k]);
#pragma unroll
        for (int tm = 0; tm < TM; ++tm)
          fx[tm] = *reinterpret_cast<const bf16x8*>(
              &sA[cur][(wm * WM + tm * 16 + frag_row) * LDS_STRIDE + ks * 32 + frag_k]);
#pragma unroll
        for (int tn = 0; tn < TN; ++tn)
#pragma unroll
          for (int tm = 0; tm < TM; ++tm)
            acc[tn][tm] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fw[tn], fx[tm], acc[tn][tm],
                                                                  0, 0, 0);
      }
      if (kt + 1 < kt_end) sstore(cur ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue: acc[tn][tm][i] = C[m][n], m = row base + (lane & 15),
  //      n = col base + 4*(lane >> 4) + i
  const int col_in = 4 * (lane >> 4);
#pragma unroll
  for (int tm = 0; tm < TM; ++tm) {
    const int m = m0 + wm * WM + tm * 16 + (lane & 15);
    if (m >= p.M) continue;
    if constexpr (EPI == EPI_PARTIAL) {
      float* w = p.ws + ((long)blockIdx.z * p.M + m) * p.N;
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int n = n0 + wn * WN + tn * 16 + col_in;
        if (n < p.N) {
          const f32x4 a = acc[tn][tm];
          *reinterpret_cast<f32x4*>(w + n) =
              f32x4{a[0] * p.alpha, a[1] * p.alpha, a[2] * p.alpha, a[3] * p.alpha};
        }
      }
    } else if constexpr (EPI == EPI_ROPE) {
#pragma unroll
      for (int tb = 0; tb < TN; tb += 4) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int n1 = n0 + wn * WN + (tb + h) * 16 + col_in;
          if (n1 < p.N) {
            float x1[4], x2[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              x1[i] = acc[tb + h][tm][i] * p.alpha;
              x2[i] = acc[tb + h + 2][tm][i] * p.alpha;
            }
            epi_rope(p, m, n1, x1, x2);
          }
        }
      }
    } else if constexpr (EPI == EPI_SILU) {
#pragma unroll
      for (int tn = 0; tn < TN; tn += 2) {
        const int ng = n0 + wn * WN + tn * 16;  // gate block start (multiple of 32)
        if (ng < p.N) {
          float g[4], u[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            g[i] = acc[tn][tm][i] * p.alpha;
            u[i] = acc[tn + 1][tm][i] * p.alpha;
          }
          epi_silu(p, m, ng / 2 + col_in, g, u);
        }
      }
    } else {
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const int n = n0 + wn * WN + tn * 16 + col_in;
        if (n < p.N) {
          float v[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = acc[tn][tm][i] * p.alpha;
          if constexpr (EPI == EPI_EULER)
            epi_euler(p, m, n, v);
          else
            epi_store<ACT>(p, m, n, v);
        }
      }
    }
  }
}

// Split-K reduction + epilogue.  One thread per epilogue unit.
template <int EPI, int ACT = SVLA_ACT_NONE>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs p) {
  const long unit = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long MN = (long)p.M * p.N;
  auto sum4 = [&](int m, int n, float v[4]) {
    v[0] = v[1] = v[2] = v[3] = 0.f;
    for (int s = 0; s < p.splits; ++s) {
      const f32x4 t = *reinterpret_cast<const f32x4*>(p.ws + s * MN + (long)m * p.N + n);
      v[0] += t[0]; v[1] += t[1]; v[2] += t[2]; v[3] += t[3];
    }
  };
  if constexpr (EPI == EPI_ROPE) {
    // units: (m, 64-block b, q in 0..7) -> columns b*64 + 4q and +32
    const int per_row = p.N / 64 * 8;
    if (unit >= (long)p.M * per_row) return;
    const int m = unit / per_row, r = unit - (long)m * per_row;
    const int n1 = (r >> 3) * 64 + (r & 7) * 4;
    float x1[4], x2[4];
    sum4(m, n1, x1);
    sum4(m, n1 + 32, x2);
    epi_rope(p, m, n1, x1, x2);
  } else if constexpr (EPI == EPI_SILU) {
    // units: (m, 32-block b, q in 0..3) -> gate b*32 + 4q, up +16, out b*16 + 4q
    const int per_row = p.N / 32 * 4;
    if (unit >= (long)p.M * per_row) return;
    const int m = unit / per_row, r = unit - (long)m * per_row;
    const int ng = (r >> 2) * 32 + (r & 3) * 4;
    float g[4], u[4];
    sum4(m, ng, g);
    sum4(m, ng + 16, u);
    epi_silu(p, m, (r >> 2) * 16 + (r & 3) * 4, g, u);
  } else {
    const int per_row = p.N / 4;
    if (unit >= (long)p.M * per_row) return;
    const int m = unit / per_row, n = (unit - (long)m * per_row) * 4;
    float v[4];
    sum4(m, n, v);
    epi_store<ACT>(p, m, n, v);
  }
}

// ---- launch ---------------------------------------------------------------
struct TileCfg {
  int bm, bn;
};

template <int AMODE, int EPI, int ACT = SVLA_ACT_NONE>
int launch_cfg(const TileCfg& t, dim3 grid, GemmArgs& p, hipStream_t s) {
  if (t.bm == 128)
    hipLaunchKernelGGL((gemm_kernel<128, 128, 2, 2, AMODE, EPI, ACT>), grid, dim3(256), 0, s, p);
  else if (t.bm == 64 && t.bn == 128)
    hipLaunchKernelGGL((gemm_kernel<64, 128, 2, 2, AMODE, EPI, ACT>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gemm_kernel<64, 64, 4, 1, AMODE, EPI, ACT>), grid, dim3(256), 0, s, p);
  SVLA_CHECK_LAUNCH();
  return 0;
}

template <int EPI>
void launch_reduce(int act, int blocks, GemmArgs& p, hipStream_t s) {
  switch (act) {
    case SVLA_ACT_GELU_TANH:
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI, SVLA_ACT_GELU_TANH>), dim3(blocks), dim3(256), 0, s, p);
      break;
    case SVLA_ACT_GELU_ERF:
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI, SVLA_ACT_GELU_ERF>), dim3(blocks), dim3(256), 0, s, p);
      break;
    case SVLA_ACT_SILU:
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI, SVLA_ACT_SILU>), dim3(blocks), dim3(256), 0, s, p);
      break;
    default:
      hipLaunchKernelGGL((splitk_reduce_kernel<EPI, SVLA_ACT_NONE>), dim3(blocks), dim3(256), 0, s, p);
  }
}

constexpr int kNumCU = 256;

TileCfg pick_tile(int M, int N) {
  auto tiles = [&](int bm, int bn) { return (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
  if (M >= 512 && tiles(128, 128) >= kNumCU) return {128, 128};
  if (M >= 128 && tiles(64, 128) >= kNumCU / 2) return {64, 128};
  return {64, 64};
}

template <int AMODE>
int run_gemm(GemmArgs& p, int epi, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0 || p.K <= 0) return p.M == 0 ? 0 : SVLA_EINVAL;
  if (p.K % 8 || p.N % 4 || p.ldb % 8 || p.ldc % 4) return SVLA_EINVAL;
  if (AMODE == A_DENSE && (p.lda % 8 || !svla_aligned16(p.a))) return SVLA_EINVAL;
  if (!svla_aligned16(p.b) || !svla_aligned16(p.c)) return SVLA_EINVAL;
  if (p.res && (p.ldr % 4)) return SVLA_EINVAL;
  if (epi == EPI_ROPE && (p.N % 64 || p.rope_cols % 64 || p.rope_period <= 0)) return SVLA_EINVAL;
  if (epi == EPI_SILU && p.N % 32) return SVLA_EINVAL;
  if (AMODE != A_DENSE && p.act) return SVLA_EINVAL;

  TileCfg t = pick_tile(p.M, p.N);
  const int gm = (p.M + t.bm - 1) / t.bm, gn = (p.N + t.bn - 1) / t.bn;
  const int nk = (p.K + BK - 1) / BK;
  // split-K when the tile grid leaves most CUs idle and the K loop is long;
  // the fp32 partials [splits, M, N] must fit the caller's workspace
  int splits = 1;
  const long tiles = (long)gm * gn;
  if (epi != EPI_EULER && p.ws && tiles < kNumCU && nk >= 8) {
    int want = (int)((2 * kNumCU + tiles - 1) / tiles);
    want = min(want, nk / 4);
    want = min(want, 16);
    const long per_split = (long)p.M * p.N * 4;
    while (want > 1 && want * per_split > p.ws_bytes) --want;
    splits = max(1, want);
  }
  if (splits > 1) {
    const int per = (nk + splits - 1) / splits;
    splits = (nk + per - 1) / per;
    p.splits = splits;
    p.kt_per_split = per;
    dim3 grid(gn, gm, splits);
    int rc = launch_cfg<AMODE, EPI_PARTIAL>(t, grid, p, s);
    if (rc) return rc;
    long units;
    if (epi == EPI_ROPE) units = (long)p.M * (p.N / 64) * 8;
    else if (epi == EPI_SILU) units = (long)p.M * (p.N / 32) * 4;
    else units = (long)p.M * (p.N / 4);
    const int blocks = (int)((units + 255) / 256);
    if (epi == EPI_ROPE)
      hipLaunchKernelGGL(splitk_reduce_kernel<EPI_ROPE>, dim3(blocks), dim3(256), 0, s, p);
    else if (epi == EPI_SILU)
      hipLaunchKernelGGL(splitk_reduce_kernel<EPI_SILU>, dim3(blocks), dim3(256), 0, s, p);
    else
      launch_reduce<EPI_STORE>(p.act, blocks, p, s);
    SVLA_CHECK_LAUNCH();
    return 0;
  }
  dim3 grid(gn, gm, 1);
  if constexpr (AMODE == A_DENSE) {
    switch (epi) {
      case EPI_ROPE: return launch_cfg<AMODE, EPI_ROPE>(t, grid, p, s);
      case EPI_SILU: return launch_cfg<AMODE, EPI_SILU>(t, grid, p, s);
      case EPI_EULER: return launch_cfg<AMODE, EPI_EULER>(t, grid, p, s);
      default:
        switch (p.act) {
          case SVLA_ACT_GELU_TANH: return launch_cfg<AMODE, EPI_STORE, SVLA_ACT_GELU_TANH>(t, grid, p, s);
          case SVLA_ACT_GELU_ERF: return launch_cfg<AMODE, EPI_STORE, SVLA_ACT_GELU_ERF>(t, grid, p, s);
          case SVLA_ACT_SILU: return launch_cfg<AMODE, EPI_STORE, SVLA_ACT_SILU>(t, grid, p, s);
          default: return launch_cfg<AMODE, EPI_STORE>(t, grid, p, s);
        }
    }
  } else {
    if (epi != EPI_STORE) return SVLA_EINVAL;
    return launch_cfg<AMODE, EPI_STORE>(t, grid, p, s);
  }
}

GemmArgs base_args(const void* a, long lda, const void* w, long ldw, void* c, long ldc, int m,
                   int n, int k, float* ws, long ws_bytes) {
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
  p.ws = ws;
  p.ws_bytes = ws ? ws_bytes : 0;
  return p;
}

}  // namespace

extern "C" {

int svla_version(void) { return 100; }

int svla_linear_bf16(const void* a, int lda, const void* w, int ldw, const void* bias,
                     const float* bias_f32, const void* res, int ldr, void* c, int ldc, int m,
                     int n, int k, float alpha, int act, int out_f32, float* ws, long ws_bytes,
                     svla_stream_t stream) {
  if (act < 0 || act > SVLA_ACT_SILU) return SVLA_EINVAL;
  if (out_f32 && (act || res)) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w, ldw, c, ldc, m, n, k, ws, ws_bytes);
  p.alpha = alpha;
  p.bias = static_cast<const bf16*>(bias);
  p.bias_f32 = bias_f32;
  p.res = static_cast<const bf16*>(res);
  p.ldr = ldr;
  p.act = act;
  p.out_f32 = out_f32;
  return run_gemm<A_DENSE>(p, EPI_STORE, (hipStream_t)stream);
}

int svla_linear_rope_bf16(const void* a, int lda, const void* w, int ldw, void* c, int ldc,
                          int m, int n, int k, int rope_cols, int seq_len, const float* cos_t,
                          const float* sin_t, float* ws, long ws_bytes, svla_stream_t stream) {
  if (!cos_t || !sin_t || rope_cols > n) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w, ldw, c, ldc, m, n, k, ws, ws_bytes);
  p.rope_cos = cos_t;
  p.rope_sin = sin_t;
  p.rope_cols = rope_cols;
  p.rope_period = seq_len;
  return run_gemm<A_DENSE>(p, EPI_ROPE, (hipStream_t)stream);
}

int svla_linear_silu_mul_bf16(const void* a, int lda, const void* w_gu, int ldw, void* out,
                              int ldo, int m, int inter, int k, float* ws, long ws_bytes,
                              svla_stream_t stream) {
  if (inter % 16) return SVLA_EINVAL;
  GemmArgs p = base_args(a, lda, w_gu, ldw, out, ldo, m, 2 * inter, k, ws, ws_bytes);
  return run_gemm<A_DENSE>(p, EPI_SILU, (hipStream_t)stream);
}

int svla_patch_embed_bf16(const void* images, const void* w, const void* bias, const void* pos,
                          void* out, int ldo, int n_img, int chans, int image, int patch,
                          int embed, float* ws, long ws_bytes, svla_stream_t stream) {
  if (patch % 8 || image % patch || !svla_aligned16(images)) return SVLA_EINVAL;
  const int G = image / patch;
  const int K = chans * patch * patch;
  GemmArgs p = base_args(images, 0, w, K, out, ldo, n_img * G * G, embed, K, ws, ws_bytes);
  p.p_chans = chans;
  p.p_img = image;
  p.p_patch = patch;
  p.bias = static_cast<const bf16*>(bias);
  p.rowadd = static_cast<const bf16*>(pos);
  p.rowadd_period = G * G;
  if (pos && !svla_aligned16(pos)) return SVLA_EINVAL;
  return run_gemm<A_PATCH>(p, EPI_STORE, (hipStream_t)stream);
}

int svla_connector_bf16(const void* x, const void* w, int ldw, void* out, int ldo, int n_img,
                        int grid, int hidden, int scale, int n_out, int rows_per_sample,
                        int sample_stride, float* ws, long ws_bytes, svla_stream_t stream) {
  if (hidden % 8 || grid % scale || !svla_aligned16(x)) return SVLA_EINVAL;
  if (rows_per_sample < 0 || (rows_per_sample > 0 && sample_stride < rows_per_sample))
    return SVLA_EINVAL;
  const int gs = grid / scale;
  const int K = hidden * scale * scale;
  GemmArgs p = base_args(x, 0, w, ldw, out, ldo, n_img * gs * gs, n_out, K, ws, ws_bytes);
  p.g_grid = grid;
  p.g_hidden = hidden;
  p.g_scale = scale;
  p.c_rpg = rows_per_sample;
  p.c_gstride = sample_stride;
  return run_gemm<A_PSHUF>(p, EPI_STORE, (hipStream_t)stream);
}

int svla_action_out_euler(const void* a, int lda, const void* w, int ldw, float* x_f32,
                          int ldx, void* x_bf16, int ldxb, int m, int n, int k, float dt,
                          svla_stream_t stream) {
  if (!x_f32 || ldx % 4 || (x_bf16 && ldxb % 4)) return SVLA_EINVAL;
  // c is unused by the Euler epilogue but must satisfy the alignment check
  GemmArgs p = base_args(a, lda, w, ldw, x_f32, 4, m, n, k, nullptr, 0);
  p.x_f32 = x_f32;
  p.ldx = ldx;
  p.x_bf16 = static_cast<bf16*>(x_bf16);
  p.ldxb = ldxb;
  p.dt = dt;
  return run_gemm<A_DENSE>(p, EPI_EULER, (hipStream_t)stream);
}

}  // extern "C"
