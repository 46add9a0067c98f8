// The image stages either side of the two networks, on the GPU, each with
// the reference's CPU arithmetic so the bytes and floats are identical:
//  - OpenCV's 8-bit bilinear resize (src/image.rs:33-142);
//  - the detector's input tensor from a page (src/det.rs:195-289);
//  - the recogniser's input tensor from a crop (src/rec.rs:10-43);
//  - the perspective text crop with bicubic sampling (src/crop.rs:1-127).
// Inputs and outputs are device memory, HWC. Every table a thread needs (a
// resize tap, a normalisation) is computed in the thread from the same
// integer and IEEE f32 / f64 operations the CPU performs, so no call
// allocates or uploads anything beyond its arguments.
#include "kernels.hpp"

namespace ppocr {

struct Tap {
  int near_i, far_i, near_w, far_w;
};

// Output coordinate d of a src -> dst resize: OpenCV's source position
// (d + 0.5) * scale - 0.5 rounded to f32, each 1/2048 weight rounded on its
// own, taps past an edge on the edge.
__device__ __forceinline__ Tap tap_at(int src, int dst, int d) {
  const double scale = 1.0 / ((double)dst / (double)src);
  const float f = (float)(((double)d + 0.5) * scale - 0.5);
  const float fl = floorf(f);
  const float a = f - fl;
  const int s = (int)fl, last = src - 1;
  Tap t;
  t.near_i = min(max(s, 0), last);
  t.far_i = min(max(s + 1, 0), last);
  t.near_w = (int)rintf((1.0f - a) * 2048.0f);
  t.far_w = (int)rintf(a * 2048.0f);
  return t;
}

// One output value from its four source values (near / far row, near / far
// column): horizontal products kept whole, then 4 bits off each row before
// its weight, 16 after, the sum rounded by 2 bits.
__device__ __forceinline__ int resize_mix(int nn, int nf, int fn, int ff, const Tap &tx, const Tap &ty) {
  const int a = nn * tx.near_w + nf * tx.far_w;
  const int b = fn * tx.near_w + ff * tx.far_w;
  const int v = (((a >> 4) * ty.near_w) >> 16) + (((b >> 4) * ty.far_w) >> 16);
  return min(max((v + 2) >> 2, 0), 255);
}

// Channel c of output pixel (x, y) of a resize of `src`.
__device__ __forceinline__ int resize_at(const uint8_t *src, int sw, const Tap &tx, const Tap &ty, int c) {
  const uint8_t *rn = src + (long)ty.near_i * sw * 3, *rf = src + (long)ty.far_i * sw * 3;
  return resize_mix(rn[tx.near_i * 3 + c], rn[tx.far_i * 3 + c], rf[tx.near_i * 3 + c], rf[tx.far_i * 3 + c],
                    tx, ty);
}

__global__ __launch_bounds__(256) void resize_kernel(const uint8_t *src, int sw, int sh, uint8_t *dst, int dw,
                                                     int dh) {
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long)dw * dh) return;
  const int y = (int)(g / dw), x = (int)(g - (long)y * dw);
  const Tap tx = tap_at(sw, dw, x), ty = tap_at(sh, dh, y);
#pragma unroll
  for (int c = 0; c < 3; c++) dst[g * 3 + c] = (uint8_t)resize_at(src, sw, tx, ty, c);
}

// The detector input: resized, x = v * (1/255 as f32), (x - mean) / std in
// f64, rounded once to f32.
__global__ __launch_bounds__(256) void det_input_kernel(const uint8_t *src, int sw, int sh, float *out, int dw,
                                                        int dh, double m0, double m1, double m2, double s0,
                                                        double s1, double s2) {
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long)dw * dh) return;
  const int y = (int)(g / dw), x = (int)(g - (long)y * dw);
  const Tap tx = tap_at(sw, dw, x), ty = tap_at(sh, dh, y);
  const float scale = (float)(1.0 / 255.0);
  const double mean[3] = {m0, m1, m2}, sd[3] = {s0, s1, s2};
#pragma unroll
  for (int c = 0; c < 3; c++) {
    const float v = (float)resize_at(src, sw, tx, ty, c) * scale;
    out[g * 3 + c] = (float)(((double)v - mean[c]) / sd[c]);
  }
}

// The recogniser input: 48 rows of `width`; the crop resized to rw columns
// and scaled to [-1, 1] in f32, zeros right of it.
__global__ __launch_bounds__(256) void rec_input_kernel(const uint8_t *src, int sw, int sh, float *out, int width,
                                                        int rw) {
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= 48L * width) return;
  const int y = (int)(g / width), x = (int)(g - (long)y * width);
  if (x >= rw) {
#pragma unroll
    for (int c = 0; c < 3; c++) out[g * 3 + c] = 0.0f;
    return;
  }
  const Tap tx = tap_at(sw, rw, x), ty = tap_at(sh, 48, y);
#pragma unroll
  for (int c = 0; c < 3; c++) out[g * 3 + c] = ((float)resize_at(src, sw, tx, ty, c) / 255.0f - 0.5f) / 0.5f;
}

// Keys' cubic weights, a = -0.75, in OpenCV's factoring.
__device__ __forceinline__ void cubic(float t, float *w) {
  const float A = -0.75f;
  w[0] = ((A * (t + 1.0f) - 5.0f * A) * (t + 1.0f) + 8.0f * A) * (t + 1.0f) - 4.0f * A;
  w[1] = ((A + 2.0f) * t - (A + 3.0f)) * t * t + 1.0f;
  w[2] = ((A + 2.0f) * (1.0f - t) - (A + 3.0f)) * (1.0f - t) * (1.0f - t) + 1.0f;
  w[3] = 1.0f - w[0] - w[1] - w[2];
}

// Pixel (x, y) of a crop rectangle: its source point through the
// projective map m (f64, then f32), the 4 x 4 bicubic window with edge pixels
// repeated, each row of four summed before the rows, rounded to 8 bits.
__device__ __forceinline__ void crop_pixel(const uint8_t *img, int iw, int ih, const CropMap &m, int x, int y,
                                           int v[3]) {
  const double xf = x, yf = y;
  double w = m.v[6] * xf + m.v[7] * yf + m.v[8];
  w = w == 0.0 ? 0.0 : 1.0 / w;
  const float sx = (float)((m.v[0] * xf + m.v[1] * yf + m.v[2]) * w);
  const float sy = (float)((m.v[3] * xf + m.v[4] * yf + m.v[5]) * w);
  const float fx = floorf(sx), fy = floorf(sy);
  float wx[4], wy[4];
  cubic(sx - fx, wx);
  cubic(sy - fy, wy);
  // The window's corner as an integer: a NaN reads as 0 and anything far
  // outside the image lands on its edge, as a saturating conversion does.
  const float kFar = 1073741824.0f;
  const long ix = (long)(isnan(fx) ? 0.0f : fminf(fmaxf(fx, -kFar), kFar)) - 1;
  const long iy = (long)(isnan(fy) ? 0.0f : fminf(fmaxf(fy, -kFar), kFar)) - 1;
  long col[4];
#pragma unroll
  for (int i = 0; i < 4; i++) col[i] = min(max(ix + i, 0L), (long)iw - 1) * 3;
  float acc[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint8_t *row = img + min(max(iy + j, 0L), (long)ih - 1) * iw * 3;
    float line[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int c = 0; c < 3; c++) line[c] += (float)row[col[i] + c] * wx[i];
#pragma unroll
    for (int c = 0; c < 3; c++) acc[c] += line[c] * wy[j];
  }
#pragma unroll
  for (int c = 0; c < 3; c++) v[c] = (int)fminf(fmaxf(rintf(acc[c]), 0.0f), 255.0f);
}

// One crop pixel (x, y) of the width x height rectangle, written turned a
// quarter counter-clockwise when `turn`.
__global__ __launch_bounds__(256) void crop_kernel(const uint8_t *img, int iw, int ih, CropMap m, uint8_t *out,
                                                   int width, int height, int turn) {
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= (long)width * height) return;
  const int y = (int)(g / width), x = (int)(g - (long)y * width);
  int v[3];
  crop_pixel(img, iw, ih, m, x, y, v);
  const long at = turn ? ((long)(width - 1 - x) * height + y) : g;
#pragma unroll
  for (int c = 0; c < 3; c++) out[at * 3 + c] = (uint8_t)v[c];
}

// The recogniser inputs of up to kCropLines crops in one launch, without the
// crops in memory: line blockIdx.y, output pixel (x, y) of its 48 x width
// tensor takes the four crop pixels its resize taps name, each computed as
// crop_kernel computes it (through the turn when the crop is turned), then
// the resize and the [-1, 1] scaling of rec_input_kernel: the same values
// as crop_text then rec_input.
__global__ __launch_bounds__(256) void crop_rec_kernel(const uint8_t *img, int iw, int ih, CropLines b) {
  const CropLine &L = b.l[blockIdx.y];
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= 48L * L.width) return;
  const int y = (int)(g / L.width), x = (int)(g - (long)y * L.width);
  float *o = L.out + g * 3;
  if (x >= L.rw) {
#pragma unroll
    for (int c = 0; c < 3; c++) o[c] = 0.0f;
    return;
  }
  const int sw = L.turn ? L.ch : L.cw, sh = L.turn ? L.cw : L.ch;  // the crop image's sides
  const Tap tx = tap_at(sw, L.rw, x), ty = tap_at(sh, 48, y);
  // Crop image pixel (cx, cy) is rectangle pixel (cw - 1 - cy, cx) when turned.
  auto px = [&](int cx, int cy, int v[3]) {
    if (L.turn)
      crop_pixel(img, iw, ih, L.m, L.cw - 1 - cy, cx, v);
    else
      crop_pixel(img, iw, ih, L.m, cx, cy, v);
  };
  int nn[3], nf[3], fn[3], ff[3];
  px(tx.near_i, ty.near_i, nn);
  px(tx.far_i, ty.near_i, nf);
  px(tx.near_i, ty.far_i, fn);
  px(tx.far_i, ty.far_i, ff);
#pragma unroll
  for (int c = 0; c < 3; c++)
    o[c] = ((float)resize_mix(nn[c], nf[c], fn[c], ff[c], tx, ty) / 255.0f - 0.5f) / 0.5f;
}

static unsigned blocks(long n) { return (unsigned)((n + 255) / 256); }

hipError_t launch_resize(const uint8_t *src, int sw, int sh, uint8_t *dst, int dw, int dh, hipStream_t s) {
  hipLaunchKernelGGL(resize_kernel, dim3(blocks((long)dw * dh)), dim3(256), 0, s, src, sw, sh, dst, dw, dh);
  return hipGetLastError();
}

hipError_t launch_det_input(const uint8_t *src, int sw, int sh, float *out, int dw, int dh, const double *mean,
                            const double *sd, hipStream_t s) {
  hipLaunchKernelGGL(det_input_kernel, dim3(blocks((long)dw * dh)), dim3(256), 0, s, src, sw, sh, out, dw, dh,
                     mean[0], mean[1], mean[2], sd[0], sd[1], sd[2]);
  return hipGetLastError();
}

hipError_t launch_rec_input(const uint8_t *src, int sw, int sh, float *out, int width, int rw, hipStream_t s) {
  hipLaunchKernelGGL(rec_input_kernel, dim3(blocks(48L * width)), dim3(256), 0, s, src, sw, sh, out, width, rw);
  return hipGetLastError();
}

hipError_t launch_crop_rec(const uint8_t *img, int iw, int ih, const CropLines &b, hipStream_t s) {
  if (b.n <= 0 || b.n > kCropLines) return hipErrorInvalidValue;
  int widest = 0;
  for (int i = 0; i < b.n; i++) widest = max(widest, b.l[i].width);
  hipLaunchKernelGGL(crop_rec_kernel, dim3(blocks(48L * widest), (unsigned)b.n), dim3(256), 0, s, img, iw, ih, b);
  return hipGetLastError();
}

hipError_t launch_crop(const uint8_t *img, int iw, int ih, const CropMap &m, uint8_t *out, int width, int height,
                       bool turn, hipStream_t s) {
  hipLaunchKernelGGL(crop_kernel, dim3(blocks((long)width * height)), dim3(256), 0, s, img, iw, ih, m, out, width,
                     height, turn ? 1 : 0);
  return hipGetLastError();
}

}  // namespace ppocr
