// The engine's elementwise and reduction layers as single kernels on device
// pointers: the ppocr_hip_* entry points of include/ppocr_hip.h. They launch
// the kernels the model uses for the same layers.
#include <hip/hip_runtime.h>

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

// The channel mean's f64 partial sums: one buffer per device, grown on
// demand and kept; calls that overlap on one device would share it.
std::mutex g_mu;
std::vector<std::pair<double *, size_t>> g_partial;

double *partial_for(size_t doubles, hipError_t *err) {
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_partial.size() <= size_t(dev)) g_partial.resize(dev + 1, {nullptr, 0});
  auto &slot = g_partial[dev];
  if (slot.second < doubles) {
    if (slot.first) {
      hipDeviceSynchronize();
      hipFree(slot.first);
    }
    slot = {nullptr, 0};
    void *p = nullptr;
    *err = hipMalloc(&p, doubles * sizeof(double));
    if (*err != hipSuccess) return nullptr;
    slot = {static_cast<double *>(p), doubles};
  }
  return slot.first;
}

}  // namespace

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

int ppocr_hip_channel_mean(const float *x, float *y, size_t pixels, size_t c, void *stream) {
  if (pixels == 0 || c == 0 || pixels > 0x7fffffff || c > 0x7fffffff) return int(hipErrorInvalidValue);
  hipError_t e;
  double *part = partial_for(mean_partial_doubles(int(pixels), int(c), 1), &e);
  if (!part) return code(e);
  return code(launch_mean(x, 0, int(pixels), int(c), 1, part, nullptr, y, 0, hipStream_t(stream)));
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

}  // extern "C"
