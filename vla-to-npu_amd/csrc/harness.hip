// Kernels behind the remaining per-kernel harness entry points: the fp32
// (cc/float/*) and "new" bf16 (cc/bf16_new/*) variants of the elementwise,
// norm and softmax kernels, the bf16 add (cc/bf16_old/add_32_32_bf16.cc), the
// fp32 patch convolution (cc/float/conv.cc) and sine / cosine
// (cc/float/sine.cc, cosine.cc, cc/bf16_new/sine_bf16.cc, cosine_bf16.cc).
//
// Every kernel computes in fp32 and, for bf16 outputs, rounds where the
// torch reference of the matching harness test rounds:
//  * ops on bf16 tensors in the "new" tests (e.g. rms_norm/test_rms_norm_bf16_new.py:25-33,
//    layer_norm/test_layer_bf16_new.py:25-34) round after every torch op;
//  * the fp32 tests and the old bf16 tests (reference computed in fp32 and
//    cast once) round once.
// These are bandwidth-bound single-pass kernels (16-byte loads where the
// layout allows, one wave per row for the row-wise ones).
#include "svla_common.h"

namespace {

template <typename T>
__device__ __forceinline__ float to_f(T v) {
  if constexpr (sizeof(T) == 4) return v;
  else return bf2f(v);
}
template <typename T>
__device__ __forceinline__ T from_f(float v) {
  if constexpr (sizeof(T) == 4) return v;
  else return f2bf(v);
}

__device__ __forceinline__ float unary_op(int op, float v) {
  switch (op) {
    case SVLA_OP_SILU: return silu_f(v);
    case SVLA_OP_GELU_TANH: return gelu_tanh_f(v);
    case SVLA_OP_GELU_ERF: return gelu_erf_f(v);
    case SVLA_OP_SIN: return sinf(v);
    default: return cosf(v);
  }
}

template <typename T>
__global__ __launch_bounds__(256) void unary_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                    long n, int op) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    y[i] = from_f<T>(unary_op(op, to_f(x[i])));
}

__global__ __launch_bounds__(256) void add_kernel(const bf16* __restrict__ x,
                                                  const bf16* __restrict__ y,
                                                  bf16* __restrict__ o, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    o[i] = f2bf(bf2f(x[i]) + bf2f(y[i]));
}

int grid_for(long n) {
  const long b = (n + 255) / 256;
  return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

// One wave per row, row kept in registers (cols <= 64 * 32 = 2048).
//  kind SVLA_NORM_RMS:      y = x * rsqrt(mean(x^2) + eps) * w            (nn.RMSNorm)
//  kind SVLA_NORM_RMS_ADD:  y = x / (||x|| / sqrt(cols) + eps) * w        (the harness RMSNorm
//                           module, rms_norm/test_rms.py:25-33)
//  kind SVLA_NORM_LAYER:    y = (x - mean) / sqrt(var + eps) * w (+ b)    (biased variance)
// ROUND_OPS (bf16 only): round after every step the torch bf16 reference takes.
constexpr int RMAX = 32;

template <typename T, bool ROUND_OPS>
__global__ __launch_bounds__(256) void row_norm_kernel(const T* __restrict__ x, long ldx,
                                                       const T* __restrict__ w,
                                                       const T* __restrict__ b, T* __restrict__ y,
                                                       long ldy, int rows, int cols, float eps,
                                                       int kind) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  auto rnd = [](float v) { return ROUND_OPS ? rbf(v) : v; };
  const T* xr = x + row * ldx;
  float v[RMAX];
  float s = 0.f, ss = 0.f;
#pragma unroll
  for (int i = 0; i < RMAX; ++i) {
    const int c = lane + i * 64;
    v[i] = c < cols ? to_f(xr[c]) : 0.f;
    s += v[i];
    ss += v[i] * v[i];
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  const float n = (float)cols;
  T* yr = y + row * ldy;
  if (kind == SVLA_NORM_LAYER) {
    const float mean = s / n;
    float dv = 0.f;
#pragma unroll
    for (int i = 0; i < RMAX; ++i) {
      const int c = lane + i * 64;
      const float d = c < cols ? v[i] - mean : 0.f;
      dv += d * d;
    }
    const float var = wave_sum(dv) / n;
    const float mean_r = rnd(mean);
    const float den = rnd(sqrtf(rnd(rnd(var) + eps)));
#pragma unroll
    for (int i = 0; i < RMAX; ++i) {
      const int c = lane + i * 64;
      if (c < cols) {
        float o = rnd(rnd(rnd(v[i] - mean_r) / den) * to_f(w[c]));
        if (b) o = rnd(o + to_f(b[c]));
        yr[c] = from_f<T>(o);
      }
    }
  } else if (kind == SVLA_NORM_RMS_ADD) {
    const float den = rnd(rnd(rnd(sqrtf(ss)) / sqrtf(n)) + eps);
#pragma unroll
    for (int i = 0; i < RMAX; ++i) {
      const int c = lane + i * 64;
      if (c < cols) yr[c] = from_f<T>(rnd(rnd(v[i] / den) * to_f(w[c])));
    }
  } else {
    const float r = 1.0f / sqrtf(ss / n + eps);
#pragma unroll
    for (int i = 0; i < RMAX; ++i) {
      const int c = lane + i * 64;
      if (c < cols) yr[c] = from_f<T>(__fmul_rn(__fmul_rn(v[i], r), to_f(w[c])));
    }
  }
}

// Row softmax with an optional causal limit: row r sees keys c <= row_start +
// r / row_div (row_start < 0: no mask).  One wave per row.
template <bool IN_F32, bool OUT_F32>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const void* __restrict__ s, long lds,
                                                           void* __restrict__ p, long ldp,
                                                           int rows, int cols, int row_start,
                                                           int row_div) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  auto ld = [&](int c) -> float {
    if constexpr (IN_F32) return static_cast<const float*>(s)[(long)row * lds + c];
    else return bf2f(static_cast<const bf16*>(s)[(long)row * lds + c]);
  };
  const int limit = row_start >= 0 ? row_start + row / row_div : cols;
  float mx = -INFINITY;
  for (int c = lane; c < cols; c += 64)
    if (c <= limit) mx = fmaxf(mx, ld(c));
  mx = wave_max(mx);
  float sum = 0.f;
  for (int c = lane; c < cols; c += 64)
    if (c <= limit) sum += expf(ld(c) - mx);
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  for (int c = lane; c < cols; c += 64) {
    const float e = c <= limit ? expf(ld(c) - mx) * inv : 0.f;
    if constexpr (OUT_F32) static_cast<float*>(p)[(long)row * ldp + c] = e;
    else static_cast<bf16*>(p)[(long)row * ldp + c] = f2bf(e);
  }
}

// Conv2d(k = stride = patch, no padding) in fp32, output [img * G_h * G_w, E]
// with the patches in row-major grid order: one thread per output element.
__global__ __launch_bounds__(256) void conv_patch_kernel(const float* __restrict__ img,
                                                         const float* __restrict__ kern,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ out, int n, int C,
                                                         int H, int W, int P, int E) {
  const int gh = H / P, gw = W / P;
  const long total = (long)n * gh * gw * E;
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int e = idx % E;
  const long t = idx / E;
  const int pc = t % gw, pr = (t / gw) % gh, im = t / ((long)gw * gh);
  float acc = bias ? bias[e] : 0.f;
  for (int c = 0; c < C; ++c) {
    const float* ip = img + (((long)im * C + c) * H + pr * P) * W + pc * P;
    const float* kp = kern + ((long)e * C + c) * P * P;
    for (int ky = 0; ky < P; ++ky)
      for (int kx = 0; kx < P; ++kx) acc = __builtin_fmaf(ip[ky * W + kx], kp[ky * P + kx], acc);
  }
  out[idx] = acc;
}

}  // namespace

extern "C" {

int svla_unary_f32(const float* x, float* y, long n, int op, svla_stream_t stream) {
  if (n < 0 || op < 0 || op > SVLA_OP_COS) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  hipLaunchKernelGGL(unary_kernel<float>, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream, x,
                     y, n, op);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_unary_bf16(const void* x, void* y, long n, int op, svla_stream_t stream) {
  if (n < 0 || op < 0 || op > SVLA_OP_COS) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  hipLaunchKernelGGL(unary_kernel<bf16>, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const bf16*>(x), static_cast<bf16*>(y), n, op);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_add_bf16(const void* x, const void* y, void* out, long n, svla_stream_t stream) {
  if (n < 0) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  hipLaunchKernelGGL(add_kernel, dim3(grid_for(n)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const bf16*>(x), static_cast<const bf16*>(y),
                     static_cast<bf16*>(out), n);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_row_norm(const void* x, int ldx, const void* w, const void* b, void* y, int ldy, int rows,
                  int cols, float eps, int kind, int is_f32, int round_ops,
                  svla_stream_t stream) {
  if (rows < 0 || cols <= 0 || cols > RMAX * 64 || ldx < cols || ldy < cols || !w) return SVLA_EINVAL;
  if (kind < SVLA_NORM_RMS || kind > SVLA_NORM_LAYER || (b && kind != SVLA_NORM_LAYER))
    return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  dim3 g((rows + 3) / 4), blk(256);
  hipStream_t st = (hipStream_t)stream;
  if (is_f32) {
    hipLaunchKernelGGL((row_norm_kernel<float, false>), g, blk, 0, st, static_cast<const float*>(x),
                       (long)ldx, static_cast<const float*>(w), static_cast<const float*>(b),
                       static_cast<float*>(y), (long)ldy, rows, cols, eps, kind);
  } else if (round_ops) {
    hipLaunchKernelGGL((row_norm_kernel<bf16, true>), g, blk, 0, st, static_cast<const bf16*>(x),
                       (long)ldx, static_cast<const bf16*>(w), static_cast<const bf16*>(b),
                       static_cast<bf16*>(y), (long)ldy, rows, cols, eps, kind);
  } else {
    hipLaunchKernelGGL((row_norm_kernel<bf16, false>), g, blk, 0, st, static_cast<const bf16*>(x),
                       (long)ldx, static_cast<const bf16*>(w), static_cast<const bf16*>(b),
                       static_cast<bf16*>(y), (long)ldy, rows, cols, eps, kind);
  }
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_softmax_rows(const void* s, int lds, void* p, int ldp, int rows, int cols, int row_start,
                      int row_div, int in_f32, int out_f32, svla_stream_t stream) {
  if (rows < 0 || cols <= 0 || lds < cols || ldp < cols || row_div <= 0) return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  dim3 g((rows + 3) / 4), b(256);
  hipStream_t st = (hipStream_t)stream;
  if (in_f32 && out_f32)
    hipLaunchKernelGGL((softmax_rows_kernel<true, true>), g, b, 0, st, s, (long)lds, p, (long)ldp, rows, cols, row_start, row_div);
  else if (in_f32)
    hipLaunchKernelGGL((softmax_rows_kernel<true, false>), g, b, 0, st, s, (long)lds, p, (long)ldp, rows, cols, row_start, row_div);
  else if (out_f32)
    hipLaunchKernelGGL((softmax_rows_kernel<false, true>), g, b, 0, st, s, (long)lds, p, (long)ldp, rows, cols, row_start, row_div);
  else
    hipLaunchKernelGGL((softmax_rows_kernel<false, false>), g, b, 0, st, s, (long)lds, p, (long)ldp, rows, cols, row_start, row_div);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_conv_patch_f32(const float* images, const float* kernel, const float* bias, float* out,
                        int n_img, int chans, int height, int width, int patch, int embed,
                        svla_stream_t stream) {
  if (n_img < 0 || chans <= 0 || patch <= 0 || embed <= 0 || height % patch || width % patch)
    return SVLA_EINVAL;
  const long total = (long)n_img * (height / patch) * (width / patch) * embed;
  if (total == 0) return SVLA_OK;
  hipLaunchKernelGGL(conv_patch_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, images, kernel, bias, out, n_img, chans, height, width,
                     patch, embed);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

}  // extern "C"
