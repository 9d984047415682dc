// Row normalisations (bandwidth-bound): one wave64 per row, 16-byte loads,
// the row kept in registers (cols <= 2048), fp32 statistics with shuffle
// reductions, one bf16 rounding of the output.
//
// RMSNorm replaces rms_norm_960_bf16 / rms_norm_bf16 (cc/bf16/rms_norm_960_bf16.cc:18-62,
// cc/bf16_old/rms_norm_bf16.cc:16-64) and mirrors torch 2.10's nn.RMSNorm on
// bf16 input: fp32 math x * rsqrt(mean(x^2) + eps) * w, one rounding.
// LayerNorm replaces layer_norm_bf16 + its bias kernel
// (cc/bf16_old/layer_norm_bf16.cc:16-70; vla/vision_block_bf16.py:101-127).
#include "svla_common.h"

namespace {

constexpr int MAXC = 4;  // 16-byte chunks per lane: cols <= 4 * 8 * 64 = 2048

// (The GEMMs' fused norm, norm_rows in gemm.hip, reproduces this kernel's
// sum of squares operation by operation: change both together.)
__global__ __launch_bounds__(256) void rmsnorm_kernel(const bf16* __restrict__ x, long ldx,
                                                      const bf16* __restrict__ w,
                                                      bf16* __restrict__ y, long ldy, int rows,
                                                      int cols, float eps) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const bf16* xr = x + row * ldx;
  // every load (row and gain) issued up front from a clamped address: a load
  // under a branch would end its region with a full wait, one round trip each
  bf16x8 v[MAXC], wv[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = min((lane + i * 64) * 8, cols - 8);
    v[i] = ld8(xr + c);
    wv[i] = ld8(w + c);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    if ((lane + i * 64) * 8 < cols) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float f = bf2f(v[i][j]);
        ss = __builtin_fmaf(f, f, ss);
      }
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / (float)cols + eps);
  bf16* yr = y + row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = (lane + i * 64) * 8;
    if (c < cols) {
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j) o[j] = f2bf(__fmul_rn(__fmul_rn(bf2f(v[i][j]), r), bf2f(wv[i][j])));
      st8(yr + c, o);
    }
  }
}

// Sum over the LPR lanes of each row group (LPR = 64: the whole wave; 32:
// each half separately).
template <int LPR>
__device__ __forceinline__ float row_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, SVLA_WAVE);
  return v;
}

// BLK: y is slab-blocked, element (row, c) at (c / 32) * rows * 32 + row * 32 +
// c % 32 (the A layout the 256x256 GEMM streams as contiguous kilobytes); each
// lane's 16-byte chunk stays inside one 64-byte slab row.
// RPW rows per wave: 2 for cols <= 1024, a 32-lane half per row, so that every
// lane holds chunks of a 768-wide row and, slab-blocked, the two halves' stores
// of one instruction fill whole 128-byte lines (rows 2j and 2j + 1 of a slab
// are adjacent); 1 (the whole wave) for wider rows.
template <bool BLK, int RPW>
__global__ __launch_bounds__(256) void layernorm_kernel(const bf16* __restrict__ x, long ldx,
                                                        const bf16* __restrict__ gmm,
                                                        const bf16* __restrict__ bta,
                                                        bf16* __restrict__ y, long ldy, int rows,
                                                        int cols, float eps) {
  constexpr int LPR = 64 / RPW;  // lanes per row
  const int lane = threadIdx.x & 63, sub = lane % LPR;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (row0 >= rows) return;  // wave-uniform
  // a second row past the end loads the last row (all lanes take part in the
  // shuffles) and stores nothing
  const int row = row0 + lane / LPR;
  const bool live = row < rows;
  const bf16* xr = x + (long)min(row, rows - 1) * ldx;
  // every load (row, gamma, beta) issued up front from a clamped address: a
  // load under a branch would end its region with a full wait
  const bf16* bsrc = bta ? bta : gmm;
  bf16x8 v[MAXC], gv[MAXC], bv[MAXC];
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = min((sub + i * LPR) * 8, cols - 8);
    v[i] = ld8(xr + c);
    gv[i] = ld8(gmm + c);
    bv[i] = ld8(bsrc + c);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    if ((sub + i * LPR) * 8 < cols) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s += bf2f(v[i][j]);
    }
  }
  const float mean = row_sum<LPR>(s) / (float)cols;
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = (sub + i * LPR) * 8;
    if (c < cols) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float d = bf2f(v[i][j]) - mean;
        ss += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(row_sum<LPR>(ss) / (float)cols + eps);
  if (!live) return;
  bf16* yr = y + (long)row * ldy;
#pragma unroll
  for (int i = 0; i < MAXC; ++i) {
    const int c = (sub + i * LPR) * 8;
    if (c < cols) {
      bf16x8 o;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        o[j] = f2bf((bf2f(v[i][j]) - mean) * rstd * bf2f(gv[i][j]) + (bta ? bf2f(bv[i][j]) : 0.f));
      if constexpr (BLK)
        st8(y + (long)(c >> 5) * rows * 32 + (long)row * 32 + (c & 31), o);
      else
        st8(yr + c, o);
    }
  }
}

template <bool BLK>
void launch_layernorm(const void* x, int ldx, const void* gamma, const void* beta, void* y,
                      long ldy, int rows, int cols, float eps, hipStream_t stream) {
  const int rpw = cols <= 4 * 8 * 32 ? 2 : 1;
  const dim3 grid((rows + 4 * rpw - 1) / (4 * rpw));
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, stream, static_cast<const bf16*>(x), (long)ldx,
                       static_cast<const bf16*>(gamma), static_cast<const bf16*>(beta),
                       static_cast<bf16*>(y), ldy, rows, cols, eps);
  };
  if (rpw == 2) args(layernorm_kernel<BLK, 2>);
  else args(layernorm_kernel<BLK, 1>);
}

bool norm_args_ok(const void* x, int ldx, const void* y, int ldy, int cols) {
  return cols > 0 && cols % 8 == 0 && cols <= MAXC * 512 && ldx % 8 == 0 && ldy % 8 == 0 &&
         ldx >= cols && ldy >= cols && svla_aligned16(x) && svla_aligned16(y);
}

}  // namespace

extern "C" int svla_rmsnorm_bf16(const void* x, int ldx, const void* w, void* y, int ldy,
                                 int rows, int cols, float eps, svla_stream_t stream) {
  if (!norm_args_ok(x, ldx, y, ldy, cols) || !svla_aligned16(w) || rows < 0) return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((rows + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const bf16*>(x), (long)ldx, static_cast<const bf16*>(w),
                     static_cast<bf16*>(y), (long)ldy, rows, cols, eps);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

extern "C" int svla_layernorm_bf16(const void* x, int ldx, const void* gamma, const void* beta,
                                   void* y, int ldy, int rows, int cols, float eps,
                                   svla_stream_t stream) {
  if (!norm_args_ok(x, ldx, y, ldy, cols) || !svla_aligned16(gamma) || rows < 0)
    return SVLA_EINVAL;
  if (beta && !svla_aligned16(beta)) return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  launch_layernorm<false>(x, ldx, gamma, beta, y, ldy, rows, cols, eps, (hipStream_t)stream);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

extern "C" int svla_layernorm_blocked_bf16(const void* x, int ldx, const void* gamma,
                                           const void* beta, void* y, int rows, int cols,
                                           float eps, svla_stream_t stream) {
  if (cols % 32 || !norm_args_ok(x, ldx, y, cols, cols) || !svla_aligned16(gamma) || rows < 0)
    return SVLA_EINVAL;
  if (beta && !svla_aligned16(beta)) return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  launch_layernorm<true>(x, ldx, gamma, beta, y, 0L, rows, cols, eps, (hipStream_t)stream);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}
