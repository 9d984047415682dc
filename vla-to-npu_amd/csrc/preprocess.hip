// Camera image pre-processing for the vision encoder, on gfx950.
//
// uint8 HWC frames (any size, RGB) -> bf16 CHW [3, S, S] in [-1, 1]: the frame
// is resized to (rh, rw) = round((H, W) * min(S / H, S / W)) (aspect ratio
// kept) with bilinear interpolation (half-pixel centres, per-axis scale
// in / out, edge-clamped: torch's interpolate(size=(rh, rw), mode="bilinear",
// align_corners=False) without antialiasing), placed at the top-left and the
// rest padded with black; then
// x -> x / 255 * 2 - 1.  This is the "resize/normalize to [-1, 1]" step in
// front of the pipeline's patch embedding (the reference feeds random images
// straight into it, vla/vla.py:306, 396-408).
//
// One thread per output pixel, writing its 3 channel planes; reads hit the
// 4 neighbouring source pixels (L2-resident for a frame).  Bandwidth kernel:
// 3 * S * S * 2 bytes written per frame (1.5 MB at S = 512).
#include "svla_common.h"

namespace {

__global__ __launch_bounds__(256) void image_kernel(const uint8_t* __restrict__ src, long src_bs,
                                                    int h, int w, int rh, int rw, float sy_scale,
                                                    float sx_scale,
                                                    bf16* __restrict__ dst, int S, int n) {
  const int img = blockIdx.y;
  const long pix = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (img >= n || pix >= (long)S * S) return;
  const int y = (int)(pix / S), x = (int)(pix - (long)y * S);
  const uint8_t* s = src + img * src_bs;
  float rgb[3] = {0.f, 0.f, 0.f};  // padding: black
  if (y < rh && x < rw) {
    // source coordinate of the output pixel centre (half-pixel convention)
    const float sy = fmaxf((y + 0.5f) * sy_scale - 0.5f, 0.f);
    const float sx = fmaxf((x + 0.5f) * sx_scale - 0.5f, 0.f);
    const int y0 = min((int)sy, h - 1), x0 = min((int)sx, w - 1);
    const int y1 = min(y0 + 1, h - 1), x1 = min(x0 + 1, w - 1);
    const float fy = sy - (float)y0, fx = sx - (float)x0;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
      const float p00 = s[((long)y0 * w + x0) * 3 + c], p01 = s[((long)y0 * w + x1) * 3 + c];
      const float p10 = s[((long)y1 * w + x0) * 3 + c], p11 = s[((long)y1 * w + x1) * 3 + c];
      const float top = p00 + (p01 - p00) * fx;
      const float bot = p10 + (p11 - p10) * fx;
      rgb[c] = top + (bot - top) * fy;
    }
  }
  bf16* d = dst + (long)img * 3 * S * S + pix;
#pragma unroll
  for (int c = 0; c < 3; ++c) d[(long)c * S * S] = f2bf(rgb[c] * (2.0f / 255.0f) - 1.0f);
}

}  // namespace

extern "C" int svla_image_to_bf16(const uint8_t* src, long src_bs, int n, int h, int w, void* dst,
                                  int out_size, svla_stream_t stream) {
  if (n < 0 || h <= 0 || w <= 0 || out_size <= 0 || src_bs < (long)h * w * 3) return SVLA_EINVAL;
  if (n == 0) return SVLA_OK;
  const float scale = fminf((float)out_size / (float)h, (float)out_size / (float)w);
  const int rh = max(1, min(out_size, (int)(h * scale + 0.5f)));
  const int rw = max(1, min(out_size, (int)(w * scale + 0.5f)));
  const long pixels = (long)out_size * out_size;
  dim3 grid((unsigned)((pixels + 255) / 256), (unsigned)n);
  hipLaunchKernelGGL(image_kernel, grid, dim3(256), 0, (hipStream_t)stream, src, src_bs, h, w, rh,
                     rw, (float)h / (float)rh, (float)w / (float)rw, static_cast<bf16*>(dst),
                     out_size, n);
  SVLA_CHECK_LAUNCH();
  return SVLA_OK;
}
