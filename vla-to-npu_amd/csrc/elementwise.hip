// Bandwidth-bound elementwise, softmax-harness and utility kernels.
//
// silu / gelu / silu_mul: the reference's silu_{128,160,256}_bf16
// (cc/bf16/silu_160_bf16.cc:124), silu_bf16 (cc/bf16_old/silu_bf16.cc:192),
// gelu_bf16 (cc/bf16_old/gelu_bf16.cc:83) and the numpy hadamard
// (vla/text_encoder_bf16.py:581), computed exactly in fp32 instead of the AIE
// kernels' polynomial / LUT approximations (the parity target is torch).
// Softmax: masked_softmax_128_bf16 (cc/bf16/masked_softmax_128_bf16.cc:251),
// softmax_bf16_* (cc/bf16_old/v2_softmax_bf16.cc:552-663) and
// softmax_float32_seq1024 (cc/float/v1_softmax_float.cc:117), one wave per row.
#include "svla_common.h"

namespace {

template <typename F>
__global__ __launch_bounds__(256) void map8_kernel(const bf16* __restrict__ x, bf16* __restrict__ y,
                                                   long n8, F f) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
       i += (long)gridDim.x * blockDim.x) {
    const bf16x8 v = ld8(x + i * 8);
    bf16x8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = f2bf(f(bf2f(v[j])));
    st8(y + i * 8, o);
  }
}

template <typename F>
__global__ void map1_kernel(const bf16* __restrict__ x, bf16* __restrict__ y, long start, long n,
                            F f) {
  const long i = start + (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = f2bf(f(bf2f(x[i])));
}

struct SiluOp {
  __device__ float operator()(float v) const { return silu_f(v); }
};
struct GeluTanhOp {
  __device__ float operator()(float v) const { return gelu_tanh_f(v); }
};
struct GeluErfOp {
  __device__ float operator()(float v) const { return gelu_erf_f(v); }
};

int grid_for(long n8) {
  long b = (n8 + 255) / 256;
  return (int)(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

template <typename F>
int run_map(const void* x, void* y, long n, F f, hipStream_t s) {
  if (n < 0) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  const bf16* xi = static_cast<const bf16*>(x);
  bf16* yo = static_cast<bf16*>(y);
  long n8 = 0;
  if (svla_aligned16(x) && svla_aligned16(y)) {
    n8 = n / 8;
    if (n8) hipLaunchKernelGGL(map8_kernel<F>, dim3(grid_for(n8)), dim3(256), 0, s, xi, yo, n8, f);
  }
  const long rest = n - n8 * 8;
  if (rest)
    hipLaunchKernelGGL(map1_kernel<F>, dim3((rest + 255) / 256), dim3(256), 0, s, xi, yo, n8 * 8,
                       n, f);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

__global__ void silu_mul_kernel(const bf16* __restrict__ g, const bf16* __restrict__ u,
                                bf16* __restrict__ o, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    o[i] = f2bf(rbf(silu_f(bf2f(g[i]))) * bf2f(u[i]));
}

// one wave per row; row_start >= 0 enables the causal mask at global row
// row_start + r (keys c > row masked); row_start < 0: no mask.
template <bool IN_F32, bool OUT_F32>
__global__ __launch_bounds__(256) void softmax_kernel(const void* __restrict__ s, void* __restrict__ p,
                                                      int rows, int cols, int row_start) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  auto ld = [&](int c) -> float {
    if constexpr (IN_F32) return static_cast<const float*>(s)[(long)row * cols + c];
    else return bf2f(static_cast<const bf16*>(s)[(long)row * cols + c]);
  };
  const int limit = row_start >= 0 ? row_start + row : cols;  // last visible column
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
    if constexpr (OUT_F32) static_cast<float*>(p)[(long)row * cols + c] = e;
    else static_cast<bf16*>(p)[(long)row * cols + c] = f2bf(e);
  }
}

// RoPE on heads of 64: y[r][h*64 + d] rotate-half at position pos_offset + r.
template <bool IN_F32, bool OUT_F32>
__global__ void rope_kernel(const void* __restrict__ x, long ldx, void* __restrict__ y, long ldy,
                            int rows, int heads, const float* __restrict__ ct,
                            const float* __restrict__ st, int pos_offset) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;  // (row, head, d<32)
  if (idx >= (long)rows * heads * 32) return;
  const int d = idx & 31;
  const long rh = idx >> 5;
  const int hh = rh % heads;
  const int r = rh / heads;
  const long xo = (long)r * ldx + hh * 64 + d, yo = (long)r * ldy + hh * 64 + d;
  float x1, x2;
  if constexpr (IN_F32) {
    x1 = static_cast<const float*>(x)[xo];
    x2 = static_cast<const float*>(x)[xo + 32];
  } else {
    x1 = bf2f(static_cast<const bf16*>(x)[xo]);
    x2 = bf2f(static_cast<const bf16*>(x)[xo + 32]);
  }
  const int pos = pos_offset + r;
  const float c = ct[pos * 32 + d], s = st[pos * 32 + d];
  const float o1 = __fsub_rn(__fmul_rn(x1, c), __fmul_rn(x2, s));
  const float o2 = __fadd_rn(__fmul_rn(x2, c), __fmul_rn(x1, s));
  if constexpr (OUT_F32) {
    static_cast<float*>(y)[yo] = o1;
    static_cast<float*>(y)[yo + 32] = o2;
  } else {
    static_cast<bf16*>(y)[yo] = f2bf(o1);
    static_cast<bf16*>(y)[yo + 32] = f2bf(o2);
  }
}

// angle = pos / theta^(2k/D): the timescale is formed in fp32 exactly as
// apply_rope does (theta ** ((2/D) * k), vla/text_encoder_bf16.py:80-84).
__global__ void rope_table_kernel(float* ct, float* st, int max_pos, int half, float theta,
                                  float two_over_d) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= max_pos * half) return;
  const int pos = idx / half, k = idx % half;
  const float ts = powf(theta, two_over_d * (float)k);
  const float ang = (float)pos / ts;
  ct[idx] = cosf(ang);
  st[idx] = sinf(ang);
}

__global__ void transpose_kernel(const bf16* __restrict__ w, long ldw, bf16* __restrict__ o,
                                 int K, int N) {
  __shared__ bf16 tile[32][33];
  const int k0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: 8 rows per pass
  for (int r = ty; r < 32; r += 8) {
    const int k = k0 + r, n = n0 + tx;
    tile[r][tx] = (k < K && n < N) ? w[(long)k * ldw + n] : f2bf(0.f);
  }
  __syncthreads();
  for (int r = ty; r < 32; r += 8) {
    const int n = n0 + r, k = k0 + tx;
    if (n < N && k < K) o[(long)n * K + k] = tile[tx][r];
  }
}

// packed row p: block b = p / 32; even blocks are gate rows, odd blocks up rows
// (gate column j and up column j are always 32 packed rows apart)
__global__ void pack_gate_up_kernel(const bf16* __restrict__ wg, const bf16* __restrict__ wu,
                                    bf16* __restrict__ o, int K, int inter) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= 2L * inter * K) return;
  const int k = idx % K;
  const int prow = idx / K;
  const int blk = prow >> 5, within = prow & 31;
  const int j = (blk >> 1) * 32 + within;
  const bf16* src = (blk & 1) ? wu : wg;
  o[idx] = src[(long)k * inter + j];
}

// ids outside [0, vocab) produce a zero row instead of an out-of-bounds read
__global__ void embed_kernel(const int64_t* __restrict__ ids, const bf16* __restrict__ table,
                             long vocab, int hidden, float scale, bf16* __restrict__ out,
                             long ldo, long out_bs, long n_tokens, int per_sample) {
  const long r = blockIdx.x;
  if (r >= n_tokens) return;
  const int64_t id = ids[r];
  const bool ok = id >= 0 && id < vocab;
  bf16* dst = out + (r / per_sample) * out_bs + (r % per_sample) * ldo;
  const bf16* src = table + (ok ? id : 0) * hidden;
  for (int c = threadIdx.x; c < hidden; c += blockDim.x)
    dst[c] = f2bf(ok ? bf2f(src[c]) * scale : 0.f);
}

__global__ void time_embedding_kernel(double t, int dim, double min_p, double max_p, bf16* out) {
  const int half = dim / 2;
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= half) return;
  // fraction = linspace(0, 1, half); period = min * (max/min)^fraction
  const double frac = half > 1 ? (double)j / (double)(half - 1) : 0.0;
  const double period = min_p * pow(max_p / min_p, frac);
  const double x = (1.0 / period) * 2.0 * 3.141592653589793 * t;
  out[j] = f2bf((float)sin(x));
  out[half + j] = f2bf((float)cos(x));
}

__global__ void f32_to_bf16_kernel(const float* __restrict__ x, bf16* __restrict__ y, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long)gridDim.x * blockDim.x)
    y[i] = f2bf(x[i]);
}

}  // namespace

extern "C" {

int svla_silu_bf16(const void* x, void* y, long n, svla_stream_t stream) {
  return run_map(x, y, n, SiluOp{}, (hipStream_t)stream);
}

int svla_gelu_bf16(const void* x, void* y, long n, int kind, svla_stream_t stream) {
  if (kind == SVLA_ACT_GELU_TANH) return run_map(x, y, n, GeluTanhOp{}, (hipStream_t)stream);
  if (kind == SVLA_ACT_GELU_ERF) return run_map(x, y, n, GeluErfOp{}, (hipStream_t)stream);
  return SVLA_EINVAL;
}

int svla_silu_mul_bf16(const void* gate, const void* up, void* out, long n, svla_stream_t stream) {
  if (n < 0) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for((n + 7) / 8)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const bf16*>(gate),
                     static_cast<const bf16*>(up), static_cast<bf16*>(out), n);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_masked_softmax_bf16(const void* s, int row_start, void* p, int rows, int cols,
                             svla_stream_t stream) {
  if (rows < 0 || cols <= 0 || row_start < 0) return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  hipLaunchKernelGGL((softmax_kernel<false, false>), dim3((rows + 3) / 4), dim3(256), 0,
                     (hipStream_t)stream, s, p, rows, cols, row_start);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_softmax(const void* s, void* p, int rows, int cols, int in_f32, int out_f32,
                 svla_stream_t stream) {
  if (rows < 0 || cols <= 0) return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  dim3 g((rows + 3) / 4), b(256);
  hipStream_t st = (hipStream_t)stream;
  if (in_f32 && out_f32) hipLaunchKernelGGL((softmax_kernel<true, true>), g, b, 0, st, s, p, rows, cols, -1);
  else if (in_f32) hipLaunchKernelGGL((softmax_kernel<true, false>), g, b, 0, st, s, p, rows, cols, -1);
  else if (out_f32) hipLaunchKernelGGL((softmax_kernel<false, true>), g, b, 0, st, s, p, rows, cols, -1);
  else hipLaunchKernelGGL((softmax_kernel<false, false>), g, b, 0, st, s, p, rows, cols, -1);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_rope(const void* x, int ldx, void* y, int ldy, int rows, int heads, const float* cos_t,
              const float* sin_t, int pos_offset, int in_f32, int out_f32, svla_stream_t stream) {
  if (rows < 0 || heads <= 0 || pos_offset < 0 || ldx < heads * 64 || ldy < heads * 64)
    return SVLA_EINVAL;
  if (rows == 0) return SVLA_OK;
  const long n = (long)rows * heads * 32;
  dim3 g((n + 255) / 256), b(256);
  hipStream_t st = (hipStream_t)stream;
  if (in_f32 && out_f32)
    hipLaunchKernelGGL((rope_kernel<true, true>), g, b, 0, st, x, (long)ldx, y, (long)ldy, rows, heads, cos_t, sin_t, pos_offset);
  else if (in_f32)
    hipLaunchKernelGGL((rope_kernel<true, false>), g, b, 0, st, x, (long)ldx, y, (long)ldy, rows, heads, cos_t, sin_t, pos_offset);
  else if (out_f32)
    hipLaunchKernelGGL((rope_kernel<false, true>), g, b, 0, st, x, (long)ldx, y, (long)ldy, rows, heads, cos_t, sin_t, pos_offset);
  else
    hipLaunchKernelGGL((rope_kernel<false, false>), g, b, 0, st, x, (long)ldx, y, (long)ldy, rows, heads, cos_t, sin_t, pos_offset);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_rope_table(float* cos_t, float* sin_t, int max_pos, int head_dim, float theta,
                    svla_stream_t stream) {
  if (max_pos <= 0 || head_dim <= 0 || head_dim % 2) return SVLA_EINVAL;
  const int half = head_dim / 2;
  const int n = max_pos * half;
  hipLaunchKernelGGL(rope_table_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                     cos_t, sin_t, max_pos, half, theta, 2.0f / (float)head_dim);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_pack_weight_bf16(const void* w_kn, int ldw, void* out_nk, int k, int n,
                          svla_stream_t stream) {
  if (k <= 0 || n <= 0 || ldw < n) return SVLA_EINVAL;
  dim3 g((n + 31) / 32, (k + 31) / 32);
  hipLaunchKernelGGL(transpose_kernel, g, dim3(256), 0, (hipStream_t)stream,
                     static_cast<const bf16*>(w_kn), (long)ldw, static_cast<bf16*>(out_nk), k, n);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_pack_gate_up_bf16(const void* w_gate, const void* w_up, void* out, int k, int inter,
                           svla_stream_t stream) {
  if (k <= 0 || inter <= 0 || inter % 32) return SVLA_EINVAL;
  const long n = 2L * inter * k;
  hipLaunchKernelGGL(pack_gate_up_kernel, dim3((n + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const bf16*>(w_gate),
                     static_cast<const bf16*>(w_up), static_cast<bf16*>(out), k, inter);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_embed_bf16(const int64_t* ids, const void* table, long vocab, int hidden, float scale,
                    void* out, int ldo, long out_bs, long n_tokens, int per_sample,
                    svla_stream_t stream) {
  if (hidden <= 0 || vocab <= 0 || n_tokens < 0 || per_sample <= 0 || ldo < hidden)
    return SVLA_EINVAL;
  if (n_tokens == 0) return SVLA_OK;
  hipLaunchKernelGGL(embed_kernel, dim3(n_tokens), dim3(256), 0, (hipStream_t)stream, ids,
                     static_cast<const bf16*>(table), vocab, hidden, scale, static_cast<bf16*>(out),
                     (long)ldo, out_bs, n_tokens, per_sample);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_time_embedding_bf16(double t, int dim, double min_period, double max_period, void* out,
                             svla_stream_t stream) {
  if (dim <= 0 || dim % 2 || min_period <= 0 || max_period <= 0) return SVLA_EINVAL;
  hipLaunchKernelGGL(time_embedding_kernel, dim3((dim / 2 + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, t, dim, min_period, max_period, static_cast<bf16*>(out));
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

int svla_f32_to_bf16(const float* x, void* y, long n, svla_stream_t stream) {
  if (n < 0) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_for((n + 7) / 8)), dim3(256), 0,
                     (hipStream_t)stream, x, static_cast<bf16*>(y), n);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}

}  // extern "C"
