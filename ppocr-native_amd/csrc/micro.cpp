// The ppocr_hip_* entry points of include/ppocr_hip.h on device pointers:
// the engine's elementwise and reduction layers as single kernels (the ones
// the model launches for those layers), the DB threshold, and the image
// stages either side of the networks (resize, detector and recogniser
// inputs, text crop).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <mutex>
#include <vector>

#include "kernels.hpp"
#include "ppocr_hip.h"

namespace {

using namespace ppocr;

int code(hipError_t e) { return e == hipSuccess ? 0 : int(e); }

EltArgs flat(int mode, const float *a, const float *b, float *y, size_t n, int act) {
  EltArgs e{};
  e.mode = mode;
  e.lanes = 1;
  e.oh = 1, e.ow = 1, e.c = int(n);
  e.iw = 1, e.sh = 1, e.sw = 1;
  e.a = a, e.b = b, e.y = y;
  e.act = act;
  return e;
}

// The channel mean's workspace (f64 partial rows) and counters: one of each
// per device, grown on demand and kept. The counters are zeroed when they
// are allocated and every launch leaves them zero; calls that overlap on one
// device would share both.
struct MeanWork {
  float *work = nullptr;
  size_t floats = 0;
  int *count = nullptr;
  size_t counters = 0;
};
std::mutex g_mu;
std::vector<MeanWork> g_mean;

hipError_t mean_work_for(size_t floats, size_t counters, float **work, int **count) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_mean.size() <= size_t(dev)) g_mean.resize(dev + 1);
  MeanWork &m = g_mean[dev];
  if (m.floats < floats || m.counters < counters) {
    e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
  }
  if (m.floats < floats) {
    if (m.work) hipFree(m.work);
    m.work = nullptr, m.floats = 0;
    e = hipMalloc(&m.work, std::max<size_t>(floats, 4) * sizeof(float));
    if (e != hipSuccess) return e;
    m.floats = floats;
  }
  if (m.counters < counters) {
    if (m.count) hipFree(m.count);
    m.count = nullptr, m.counters = 0;
    e = hipMalloc(&m.count, counters * sizeof(int));
    if (e != hipSuccess) return e;
    e = hipMemset(m.count, 0, counters * sizeof(int));
    if (e != hipSuccess) return e;
    m.counters = counters;
  }
  *work = m.work;
  *count = m.count;
  return hipSuccess;
}

// The channel mean without allocation (ppocr_hip_channel_mean_noalloc): its
// partial rows and counters live in `scratch`, a file-scope device array
// each GPU holds until the process ends. On the host, `scratch` names a
// host-side stand-in, never the device memory: each device's address comes
// from hipGetSymbolAddress, once per device, with that device current, and
// only that address is passed on.
constexpr int kNoAllocMaxChannels = 4096;
constexpr size_t kNoAllocPartials = size_t(64) * kNoAllocMaxChannels;  // doubles: 64 chunks x channels
constexpr size_t kNoAllocCounters = 1024;                              // ints after the partial rows
static __device__ __align__(256) double scratch[kNoAllocPartials + kNoAllocCounters / 2];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
double *g_scratch[kMaxDevices];

__global__ void zero_ints(int *p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// This device's `scratch`, its counters zeroed (on `s`) the first time
// (each call also zeroes the counters it uses).
hipError_t scratch_on_device(double **out, hipStream_t s) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    int *counters = reinterpret_cast<int *>(static_cast<double *>(p) + kNoAllocPartials);
    hipLaunchKernelGGL(zero_ints, dim3((kNoAllocCounters + 255) / 256), dim3(256), 0, s, counters,
                       int(kNoAllocCounters));
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    g_scratch[dev] = static_cast<double *>(p);
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

}  // namespace

// The crop's size, before any turn: the longer of each pair of opposite
// sides, truncated (src/crop.rs:85-86; side lengths in f32).
static void crop_size(const float *q, size_t *w, size_t *h) {
  auto d = [&](int a, int b) {
    const float dx = q[2 * a] - q[2 * b], dy = q[2 * a + 1] - q[2 * b + 1];
    return std::sqrt(dx * dx + dy * dy);
  };
  *w = size_t(std::fmax(d(0, 1), d(2, 3)));
  *h = size_t(std::fmax(d(0, 3), d(1, 2)));
}

// The projective map sending the width x height rectangle's corners to the
// quad: eight linear equations in f64, Gaussian elimination with partial
// pivoting (ties to the lower row), src/crop.rs:7-53.
static ppocr::CropMap rect_to_quad(double width, double height, const float *q) {
  double m[8][9];
  const double from[4][2] = {{0, 0}, {width, 0}, {width, height}, {0, height}};
  for (int i = 0; i < 4; i++) {
    const double x = from[i][0], y = from[i][1], u = double(q[2 * i]), v = double(q[2 * i + 1]);
    const double r0[9] = {x, y, 1.0, 0.0, 0.0, 0.0, -x * u, -y * u, u};
    const double r1[9] = {0.0, 0.0, 0.0, x, y, 1.0, -x * v, -y * v, v};
    std::copy(r0, r0 + 9, m[i]);
    std::copy(r1, r1 + 9, m[i + 4]);
  }
  for (int col = 0; col < 8; col++) {
    int piv = col;
    for (int r = col + 1; r < 8; r++)
      if (std::fabs(m[r][col]) >= std::fabs(m[piv][col])) piv = r;
    std::swap(m[col], m[piv]);
    const double p = m[col][col];
    if (p == 0.0) continue;
    double prow[9];
    std::copy(m[col], m[col] + 9, prow);
    for (int r = 0; r < 8; r++) {
      const double f = m[r][col] / p;
      if (r == col || f == 0.0) continue;
      for (int k = col; k < 9; k++) m[r][k] -= f * prow[k];
    }
  }
  ppocr::CropMap out;
  for (int i = 0; i < 8; i++) out.v[i] = m[i][i] == 0.0 ? 0.0 : m[i][8] / m[i][i];
  out.v[8] = 1.0;
  return out;
}

// Largest image side the image stages take (keeps every index in 32 bits).
static const size_t kMaxSide = 1 << 15;

extern "C" {

int ppocr_hip_add(const float *a, const float *b, float *y, size_t n, int act, void *stream) {
  if (n == 0) return 0;
  if (act < 0 || act > 7 || n > size_t(1) << 40) return int(hipErrorInvalidValue);
  return code(launch_eltwise(flat(ELT_ADD, a, b, y, n, act), hipStream_t(stream)));
}

int ppocr_hip_mul(const float *a, const float *b, float *y, size_t n, void *stream) {
  if (n == 0) return 0;
  return code(launch_eltwise(flat(ELT_MUL, a, b, y, n, 0), hipStream_t(stream)));
}

int ppocr_hip_activation(const float *x, float *y, size_t n, int act, void *stream) {
  if (n == 0) return 0;
  if (act < 0 || act > 7) return int(hipErrorInvalidValue);
  return code(launch_eltwise(flat(ELT_ACT, x, nullptr, y, n, act), hipStream_t(stream)));
}

int ppocr_hip_copy_lds(const float *x, float *y, size_t n, void *stream) {
  if (n == 0) return 0;
  return code(launch_copy_lds(x, y, long(n), hipStream_t(stream)));
}

int ppocr_hip_channel_mean(const float *x, float *y, size_t pixels, size_t c, void *stream) {
  if (pixels == 0 || c == 0 || pixels > 0x7fffffff || c > 0x7fffffff) return int(hipErrorInvalidValue);
  const MeanShape m = mean_shape(true, int(pixels), int(c), 1, 0, false);
  MeanJob j{};
  j.x = x, j.pixels = int(pixels), j.c = int(c), j.lanes = 1;
  j.y = y;
  hipError_t e = mean_work_for(m.floats, m.count_n, &j.work, &j.count);
  if (e != hipSuccess) return code(e);
  return code(launch_mean_group(&j, 1, hipStream_t(stream)));
}

int ppocr_hip_channel_mean_noalloc(const float *x, float *y, size_t pixels, size_t c, void *stream, char *err,
                                   size_t err_len) {
  auto fail = [&](int code_, const char *msg) {
    if (err && err_len) snprintf(err, err_len, "%s", msg);
    return code_;
  };
  if (pixels == 0 || c == 0 || pixels > 0x7fffffff)
    return fail(int(hipErrorInvalidValue), "channel mean: pixels and channels must be positive");
  if (c > size_t(kNoAllocMaxChannels)) {
    char m[160];
    snprintf(m, sizeof m, "channel mean without allocation: %zu channels, over the %d its scratch holds", c,
             kNoAllocMaxChannels);
    return fail(int(hipErrorInvalidValue), m);
  }
  const MeanShape m = mean_shape(true, int(pixels), int(c), 1, 0, false);
  if (m.floats > 2 * kNoAllocPartials || m.count_n > kNoAllocCounters)
    return fail(int(hipErrorInvalidValue), "channel mean without allocation: shape exceeds its scratch");
  double *sc = nullptr;
  hipError_t e = scratch_on_device(&sc, hipStream_t(stream));
  if (e != hipSuccess) return fail(int(e), hipGetErrorString(e));
  MeanJob j{};
  j.x = x, j.pixels = int(pixels), j.c = int(c), j.lanes = 1;
  j.y = y;
  j.work = reinterpret_cast<float *>(sc);
  j.count = reinterpret_cast<int *>(sc + kNoAllocPartials);
  // The kernel leaves its counters at zero, but a call that overlapped
  // another or was cut short may not have: every call starts them at zero
  // on its own stream (a fill kernel, so the call stays capturable).
  if (m.count_n) {
    hipLaunchKernelGGL(zero_ints, dim3(unsigned((m.count_n + 255) / 256)), dim3(256), 0, hipStream_t(stream),
                       j.count, int(m.count_n));
    e = hipGetLastError();
    if (e != hipSuccess) return fail(int(e), hipGetErrorString(e));
  }
  e = launch_mean_group(&j, 1, hipStream_t(stream));
  if (e != hipSuccess) return fail(int(e), hipGetErrorString(e));
  return 0;
}

int ppocr_hip_channel_mul(const float *x, const float *g, float *y, size_t pixels, size_t c,
                          void *stream) {
  if (pixels == 0 || c == 0) return int(hipErrorInvalidValue);
  EltArgs e{};
  e.mode = ELT_CHANNELMUL;
  e.lanes = 1;
  e.oh = 1, e.ow = int(pixels), e.c = int(c);
  e.iw = 1, e.sh = 1, e.sw = 1;
  e.a = x, e.g = g, e.y = y;
  return code(launch_eltwise(e, hipStream_t(stream)));
}

int ppocr_hip_layer_norm(const float *x, const float *w, float *y, size_t rows, size_t c,
                         void *stream) {
  if (rows == 0 || c == 0) return int(hipErrorInvalidValue);
  return code(launch_layernorm(x, 0, w, int(rows), int(c), 1, y, 0, hipStream_t(stream)));
}

int ppocr_hip_row_argmax(const float *x, float *y, size_t rows, size_t cols, void *stream) {
  if (rows == 0 || cols == 0 || rows > 0x7fffffff || cols > 0x7fffffff) return int(hipErrorInvalidValue);
  return code(launch_row_argmax(x, y, int(rows), int(cols), hipStream_t(stream)));
}

int ppocr_hip_db_mask(const float *prob, uint8_t *mask, size_t n, float thresh, void *stream) {
  if (n == 0) return 0;
  if (!prob || !mask || n > (size_t)1 << 40) return int(hipErrorInvalidValue);
  return code(launch_db_mask(prob, mask, long(n), thresh, hipStream_t(stream)));
}

// ------------------------------------------------------------ image stages

int ppocr_hip_resize_linear(const uint8_t *src, size_t sw, size_t sh, uint8_t *dst, size_t dw, size_t dh,
                            void *stream) {
  if (!sw || !sh || !dw || !dh || !src || !dst || sw > kMaxSide || sh > kMaxSide || dw > kMaxSide || dh > kMaxSide)
    return int(hipErrorInvalidValue);
  return code(launch_resize(src, int(sw), int(sh), dst, int(dw), int(dh), hipStream_t(stream)));
}

int ppocr_hip_det_input(const uint8_t *page, size_t w, size_t h, float *out, size_t ow, size_t oh,
                        const double *mean, const double *std, void *stream) {
  if (!w || !h || !ow || !oh || !page || !out || !mean || !std || w > kMaxSide || h > kMaxSide || ow > kMaxSide ||
      oh > kMaxSide)
    return int(hipErrorInvalidValue);
  return code(launch_det_input(page, int(w), int(h), out, int(ow), int(oh), mean, std, hipStream_t(stream)));
}

size_t ppocr_rec_width(size_t w, size_t h, size_t *resized_w) {
  if (!w || !h) return 0;
  const double height = 48.0, r = double(w) / double(h);
  const double ratio = std::max(320.0 / height, r);
  const size_t width = size_t(height * ratio);
  const double fitted = std::ceil(height * r);
  if (resized_w) *resized_w = fitted > double(width) ? width : size_t(fitted);
  return width;
}

int ppocr_hip_rec_input(const uint8_t *crop, size_t w, size_t h, float *out, size_t out_cap, size_t *width,
                        void *stream) {
  size_t rw = 0;
  const size_t wd = ppocr_rec_width(w, h, &rw);
  if (width) *width = wd;
  if (!wd || !crop || !out || w > kMaxSide || h > kMaxSide || wd > kMaxSide || rw == 0) return int(hipErrorInvalidValue);
  if (48 * wd * 3 > out_cap) return int(hipErrorInvalidValue);
  return code(launch_rec_input(crop, int(w), int(h), out, int(wd), int(rw), hipStream_t(stream)));
}

size_t ppocr_rec_width_fit(size_t w, size_t h, size_t max_width, size_t *resized_w) {
  size_t rw = 0;
  const size_t width = ppocr_rec_width(w, h, &rw);
  if (width && max_width && width > max_width) {
    if (resized_w) *resized_w = max_width;
    return max_width;
  }
  if (resized_w) *resized_w = rw;
  return width;
}

int ppocr_hip_rec_input_fit(const uint8_t *crop, size_t w, size_t h, size_t max_width, float *out,
                            size_t out_cap, size_t *width, void *stream) {
  size_t rw = 0;
  const size_t wd = ppocr_rec_width_fit(w, h, max_width, &rw);
  if (width) *width = wd;
  if (!wd || !crop || !out || w > kMaxSide || h > kMaxSide || wd > kMaxSide || rw == 0) return int(hipErrorInvalidValue);
  if (48 * wd * 3 > out_cap) return int(hipErrorInvalidValue);
  return code(launch_rec_input(crop, int(w), int(h), out, int(wd), int(rw), hipStream_t(stream)));
}

int ppocr_hip_crop_rec_inputs(const uint8_t *page, size_t w, size_t h, const float *quads, size_t n,
                              size_t max_width, float *const *outs, const size_t *out_caps, size_t *widths,
                              void *stream) {
  if (!page || !w || !h || w > kMaxSide || h > kMaxSide || (n && (!quads || !outs || !out_caps)))
    return int(hipErrorInvalidValue);
  CropLines b{};
  for (size_t i = 0; i < n; i++) {
    const float *q = quads + 8 * i;
    size_t cw, ch;
    crop_size(q, &cw, &ch);
    const bool turn = cw && double(ch) / double(cw) >= 1.5;
    const size_t iw = turn ? ch : cw, ih = turn ? cw : ch;
    size_t rw = 0;
    const size_t wd = ppocr_rec_width_fit(iw, ih, max_width, &rw);
    if (widths) widths[i] = wd;
    if (!wd || !rw || cw > kMaxSide || ch > kMaxSide || wd > kMaxSide || !outs[i] || 48 * wd * 3 > out_caps[i])
      return int(hipErrorInvalidValue);
    CropLine &l = b.l[b.n++];
    l.m = rect_to_quad(double(cw), double(ch), q);
    l.out = outs[i];
    l.cw = int(cw), l.ch = int(ch), l.turn = turn ? 1 : 0, l.width = int(wd), l.rw = int(rw);
    if (b.n == kCropLines || i + 1 == n) {
      const int rc = code(launch_crop_rec(page, int(w), int(h), b, hipStream_t(stream)));
      if (rc) return rc;
      b.n = 0;
    }
  }
  return 0;
}

int ppocr_crop_size(const float *quad, size_t *width, size_t *height) {
  if (!quad) return 1;
  size_t w, h;
  crop_size(quad, &w, &h);
  const bool turn = double(h) / double(w) >= 1.5;
  if (width) *width = turn ? h : w;
  if (height) *height = turn ? w : h;
  return 0;
}

int ppocr_hip_crop_text(const uint8_t *page, size_t w, size_t h, const float *quad, uint8_t *out, size_t out_cap,
                        size_t *out_w, size_t *out_h, void *stream) {
  if (!page || !quad || !w || !h || w > kMaxSide || h > kMaxSide) return int(hipErrorInvalidValue);
  size_t cw, ch;
  crop_size(quad, &cw, &ch);
  const bool turn = double(ch) / double(cw) >= 1.5;
  if (out_w) *out_w = turn ? ch : cw;
  if (out_h) *out_h = turn ? cw : ch;
  if (cw * ch == 0) return 0;
  if (!out || cw > kMaxSide || ch > kMaxSide || cw * ch * 3 > out_cap) return int(hipErrorInvalidValue);
  const CropMap m = rect_to_quad(double(cw), double(ch), quad);
  return code(launch_crop(page, int(w), int(h), m, out, int(cw), int(ch), turn, hipStream_t(stream)));
}

}  // extern "C"
