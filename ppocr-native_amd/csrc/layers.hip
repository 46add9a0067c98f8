// The memory-bound layers: depthwise convolution, elementwise modes, pooling,
// channel mean with the squeeze-and-excite that follows, layer norm,
// attention, the CTC choice over logits, and the narrow transposed conv.
//
// Wherever the engine's CPU path fixes an order that a GPU thread can keep
// without losing coalescing, the kernel keeps it, so that the result is the
// CPU's bits for the same input: depthwise taps from the bias in row-major
// order (src/engine/kernels/depthwise.rs:93-217), average-pool taps summed in
// row-major order (src/engine/layers.rs:443-463), layer norm's sequential f32
// sums (layers.rs:467-479), attention's scores, 8-lane softmax and weighted
// sums (layers.rs:494-522, 273-294), and the squeeze-and-excite 1x1 layers'
// sums of one pixel (bias last, src/engine/kernels/pointwise.rs:135-185).
// Channel means sum in f64 as the CPU does (layers.rs:391-406), in another
// order.
#include "act.hpp"
#include "kernels.hpp"

namespace ppocr {

typedef float f32x4 __attribute__((ext_vector_type(4)));

static inline unsigned blocks_for(long n, int per) {
  long b = (n + per - 1) / per;
  return (unsigned)(b < 1 ? 1 : b);
}

// ------------------------------------------------------------ depthwise

// Thread: DX horizontally neighbouring outputs of V channels. Taps go from
// the bias, row by row, each one fused multiply-add, padding skipped.
template <int V, int DX>
__global__ __launch_bounds__(256) void dwconv_kernel(DwArgs a) {
  typedef typename std::conditional<V == 4, f32x4, float>::type T;
  const int cv = a.c / V;
  const int runs = (a.ow + DX - 1) / DX;
  long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
  long total = (long)a.lanes * a.oh * runs * cv;
  if (g >= total) return;
  int ch = (int)(g % cv) * V;
  long t = g / cv;
  int run = (int)(t % runs);
  t /= runs;
  int oy = (int)(t % a.oh);
  int ln = (int)(t / a.oh);
  int ox0 = run * DX;
  const float *x = a.x + (long)ln * a.x_lane_stride;
  T bias;
  if constexpr (V == 4) {
    bias = a.bias ? *reinterpret_cast<const f32x4 *>(a.bias + ch) : f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
    bias = a.bias ? a.bias[ch] : 0.0f;
  }
  T acc[DX];
#pragma unroll
  for (int o = 0; o < DX; o++) acc[o] = bias;
  for (int ky = 0; ky < a.kh; ky++) {
    int iy = oy * a.sh + ky - a.pt;
    if (iy < 0 || iy >= a.ih) continue;
    const float *row = x + (long)iy * a.iw * a.c + ch;
    for (int kx = 0; kx < a.kw; kx++) {
      T wv = *reinterpret_cast<const T *>(a.w + (long)(ky * a.kw + kx) * a.c + ch);
#pragma unroll
      for (int o = 0; o < DX; o++) {
        int ix = (ox0 + o) * a.sw + kx - a.pl;
        if (ix < 0 || ix >= a.iw) continue;
        T xv = *reinterpret_cast<const T *>(row + (long)ix * a.c);
        if constexpr (V == 4) {
          acc[o].x = fmaf(wv.x, xv.x, acc[o].x);
          acc[o].y = fmaf(wv.y, xv.y, acc[o].y);
          acc[o].z = fmaf(wv.z, xv.z, acc[o].z);
          acc[o].w = fmaf(wv.w, xv.w, acc[o].w);
        } else {
          acc[o] = fmaf(wv, xv, acc[o]);
        }
      }
    }
  }
  float *y = a.y + (long)ln * a.y_lane_stride + ((long)oy * a.ow) * a.c + ch;
#pragma unroll
  for (int o = 0; o < DX; o++) {
    if (ox0 + o >= a.ow) break;
    T v = acc[o];
    if constexpr (V == 4) {
      v.x = act(v.x, a.act);
      v.y = act(v.y, a.act);
      v.z = act(v.z, a.act);
      v.w = act(v.w, a.act);
    } else {
      v = act(v, a.act);
    }
    *reinterpret_cast<T *>(y + (long)(ox0 + o) * a.c) = v;
  }
}

hipError_t launch_dwconv(const DwArgs &a, hipStream_t s) {
  constexpr int DX = 4;
  auto aligned = [](const void *p) { return p == nullptr || (uintptr_t(p) & 15) == 0; };
  bool vec = a.c % 4 == 0 && aligned(a.x) && aligned(a.y) && aligned(a.w) && aligned(a.bias) &&
             a.x_lane_stride % 4 == 0 && a.y_lane_stride % 4 == 0;
  long runs = (a.ow + DX - 1) / DX;
  long total = (long)a.lanes * a.oh * runs * (vec ? a.c / 4 : a.c);
  if (vec)
    hipLaunchKernelGGL((dwconv_kernel<4, DX>), dim3(blocks_for(total, 256)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((dwconv_kernel<1, DX>), dim3(blocks_for(total, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ------------------------------------------------------------ elementwise

template <int V>
__device__ __forceinline__ void vload(float (&v)[V], const float *p) {
  if constexpr (V == 4) {
    f32x4 t = *reinterpret_cast<const f32x4 *>(p);
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    v[0] = *p;
  }
}

template <int V>
__device__ __forceinline__ void vstore(float *p, const float (&v)[V]) {
  if constexpr (V == 4) {
    *reinterpret_cast<f32x4 *>(p) = f32x4{v[0], v[1], v[2], v[3]};
  } else {
    *p = v[0];
  }
}

template <int V>
__global__ __launch_bounds__(256) void eltwise_kernel(EltArgs a) {
  const long per = (long)a.oh * a.ow * a.c;
  const long nv = (long)a.lanes * per / V;
  for (long g = (long)blockIdx.x * blockDim.x + threadIdx.x; g < nv;
       g += (long)gridDim.x * blockDim.x) {
    long e = g * V;
    int ln = (int)(e / per);
    long off = e - (long)ln * per;
    int ch = (int)(off % a.c);
    long pix = off / a.c;
    const float *A = a.a + (long)ln * a.a_lane_stride;
    float v[V], u[V], gt[V];
    switch (a.mode) {
      case ELT_ADD:
        vload<V>(v, A + off);
        vload<V>(u, a.b + (long)ln * a.b_lane_stride + off);
#pragma unroll
        for (int k = 0; k < V; k++) v[k] = v[k] + u[k];
        break;
      case ELT_MUL:
        vload<V>(v, A + off);
        vload<V>(u, a.b + (long)ln * a.b_lane_stride + off);
#pragma unroll
        for (int k = 0; k < V; k++) v[k] = v[k] * u[k];
        break;
      case ELT_ACT:
        vload<V>(v, A + off);
        break;
      case ELT_CHANNELMUL:
        vload<V>(v, A + off);
        vload<V>(gt, a.g + (long)ln * a.g_lane_stride + ch);
#pragma unroll
        for (int k = 0; k < V; k++) v[k] = v[k] * gt[k];
        break;
      case ELT_RESGATE:
        vload<V>(v, A + off);
        vload<V>(gt, a.g + (long)ln * a.g_lane_stride + ch);
#pragma unroll
        for (int k = 0; k < V; k++) v[k] = v[k] + v[k] * gt[k];
        break;
      case ELT_CONCAT:
        if (ch < a.ca) vload<V>(v, A + pix * a.ca + ch);
        else vload<V>(v, a.b + (long)ln * a.b_lane_stride + pix * a.cb + (ch - a.ca));
        break;
      default: {  // the upsampling modes
        int oy = (int)(pix / a.ow), ox = (int)(pix - (long)oy * a.ow);
        vload<V>(v, A + ((long)(oy / a.sh) * a.iw + ox / a.sw) * a.c + ch);
        if (a.mode == ELT_UPSAMPLEADD) {
          vload<V>(u, a.b + (long)ln * a.b_lane_stride + off);
#pragma unroll
          for (int k = 0; k < V; k++) v[k] = u[k] + v[k];
        } else if (a.mode == ELT_UPSAMPLEADD_RESGATE) {
          vload<V>(u, a.b + (long)ln * a.b_lane_stride + off);
          vload<V>(gt, a.g + (long)ln * a.g_lane_stride + ch);
#pragma unroll
          for (int k = 0; k < V; k++) v[k] = (u[k] + u[k] * gt[k]) + v[k];
        }
      }
    }
    if (a.act != ACT_NONE) {
#pragma unroll
      for (int k = 0; k < V; k++) v[k] = act(v[k], a.act);
    }
    vstore<V>(a.y + (long)ln * a.y_lane_stride + off, v);
  }
}

hipError_t launch_eltwise(const EltArgs &a, hipStream_t s) {
  long n = (long)a.lanes * a.oh * a.ow * a.c;
  bool vec = a.c % 4 == 0 && (a.mode != ELT_CONCAT || (a.ca % 4 == 0 && a.cb % 4 == 0));
  if (a.mode == ELT_ADD || a.mode == ELT_MUL || a.mode == ELT_ACT) vec = n % 4 == 0;
  if (vec && (a.a_lane_stride % 4 || a.b_lane_stride % 4 || a.y_lane_stride % 4)) vec = false;
  long nv = vec ? n / 4 : n;
  unsigned blocks = blocks_for(nv, 256);
  if (blocks > 65536u * 4) blocks = 65536u * 4;
  if (vec) hipLaunchKernelGGL(eltwise_kernel<4>, dim3(blocks), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(eltwise_kernel<1>, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ------------------------------------------------------------ pooling

// Max: the window cut at the bottom and right edges, seeded with its first
// tap, each later tap kept only when greater (src/engine/conv.rs:404-440).
// Average: whole windows, taps summed from zero in row-major order, then
// divided (src/engine/layers.rs:443-463).
__global__ __launch_bounds__(256) void pool_kernel(PoolArgs a) {
  long per = (long)a.oh * a.ow * a.c;
  long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long)a.lanes * per) return;
  int ln = (int)(g / per);
  long off = g - (long)ln * per;
  int ch = (int)(off % a.c);
  long pix = off / a.c;
  int oy = (int)(pix / a.ow), ox = (int)(pix - (long)oy * a.ow);
  const float *x = a.x + (long)ln * a.x_lane_stride;
  float accv = 0.0f;
  bool seeded = false;
  for (int ky = 0; ky < a.kh; ky++) {
    int iy = oy * a.sh + ky;
    if (iy >= a.ih) continue;
    for (int kx = 0; kx < a.kw; kx++) {
      int ix = ox * a.sw + kx;
      if (ix >= a.iw) continue;
      float v = x[((long)iy * a.iw + ix) * a.c + ch];
      if (a.avg) {
        accv = accv + v;
      } else if (!seeded || v > accv) {
        accv = v;
      }
      seeded = true;
    }
  }
  if (a.avg) accv = accv / (float)(a.kh * a.kw);
  a.y[(long)ln * a.y_lane_stride + off] = accv;
}

hipError_t launch_pool(const PoolArgs &a, hipStream_t s) {
  long n = (long)a.lanes * a.oh * a.ow * a.c;
  hipLaunchKernelGGL(pool_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ------------------------------------------------------------ mean and SE

// Pass 1: a block sums a run of `chunk` pixels of one lane for every channel
// in f64; threads split into `rows` pixel strides of `c` channels, joined in
// a fixed order in LDS.
__global__ __launch_bounds__(256) void mean_partial(const float *x, long x_lane_stride, int pixels,
                                                   int c, int chunk, int chunks, double *partial) {
  __shared__ double sums[256];
  int ln = blockIdx.y, run = blockIdx.x;
  const float *xl = x + (long)ln * x_lane_stride;
  int p0 = run * chunk, p1 = min(p0 + chunk, pixels);
  double *out = partial + ((long)ln * chunks + run) * c;
  for (int c0 = 0; c0 < c; c0 += 256) {
    int cw = min(256, c - c0);
    int rows = 256 / cw;
    int t = threadIdx.x;
    int ch = t % cw, r = t / cw;
    double s = 0.0;
    if (r < rows) {
      for (int p = p0 + r; p < p1; p += rows) s += (double)xl[(long)p * c + c0 + ch];
    }
    sums[t] = s;
    __syncthreads();
    if (t < cw) {
      double tot = 0.0;
      for (int k = 0; k < rows; k++) tot += sums[k * cw + t];
      out[c0 + t] = tot;
    }
    __syncthreads();
  }
}

// Pass 2: one block per lane joins the partials in order and divides; with
// an SE, then the two 1x1 layers of one pixel, each output from zero with a
// fused multiply-add per input in order, then its bias, then its activation.
__global__ __launch_bounds__(256) void mean_finish(const double *partial, int pixels, int c,
                                                  int chunks, SeArgs se, int has_se, float *y,
                                                  long y_lane_stride) {
  extern __shared__ float smem[];
  float *mean = smem;         // c
  float *hid = smem + c;      // mid
  int ln = blockIdx.x;
  const double *pl = partial + (long)ln * chunks * c;
  for (int ch = threadIdx.x; ch < c; ch += blockDim.x) {
    double s = 0.0;
    for (int r = 0; r < chunks; r++) s += pl[(long)r * c + ch];
    mean[ch] = (float)(s / (double)pixels);
  }
  __syncthreads();
  float *yl = y + (long)ln * y_lane_stride;
  if (!has_se) {
    for (int ch = threadIdx.x; ch < c; ch += blockDim.x) yl[ch] = mean[ch];
    return;
  }
  for (int j = threadIdx.x; j < se.mid; j += blockDim.x) {
    float acc = 0.0f;
    for (int i = 0; i < c; i++) acc = fmaf(se.w1[(long)i * se.mid + j], mean[i], acc);
    if (se.b1) acc = acc + se.b1[j];
    hid[j] = act(acc, se.act1);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < se.cout; j += blockDim.x) {
    float acc = 0.0f;
    for (int i = 0; i < se.mid; i++) acc = fmaf(se.w2[(long)i * se.cout + j], hid[i], acc);
    if (se.b2) acc = acc + se.b2[j];
    yl[j] = act(acc, se.act2);
  }
}

static int mean_chunk(int pixels) {
  int chunk = (pixels + 255) / 256;
  return chunk < 16 ? 16 : chunk;
}

size_t mean_partial_doubles(int pixels, int c, int lanes) {
  int chunk = mean_chunk(pixels);
  int chunks = (pixels + chunk - 1) / chunk;
  return (size_t)lanes * chunks * c;
}

hipError_t launch_mean(const float *x, long x_lane_stride, int pixels, int c, int lanes,
                       double *partial, const SeArgs *se, float *y, long y_lane_stride,
                       hipStream_t s) {
  int chunk = mean_chunk(pixels);
  int chunks = (pixels + chunk - 1) / chunk;
  hipLaunchKernelGGL(mean_partial, dim3(chunks, lanes), dim3(256), 0, s, x, x_lane_stride, pixels,
                     c, chunk, chunks, partial);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  SeArgs none{};
  size_t shm = (size_t)(c + (se ? se->mid : 0)) * sizeof(float);
  hipLaunchKernelGGL(mean_finish, dim3(lanes), dim3(256), shm, s, partial, pixels, c, chunks,
                     se ? *se : none, se ? 1 : 0, y, y_lane_stride);
  return hipGetLastError();
}

// ------------------------------------------------------------ layer norm

// A block of 64 threads takes 64 rows through LDS with coalesced loads and
// stores; each thread then normalises its row with sequential f32 sums.
__global__ __launch_bounds__(64) void layernorm_kernel(const float *x, long x_lane_stride,
                                                      const float *w, int rows, int c, int lanes,
                                                      float *y, long y_lane_stride) {
  extern __shared__ float tile[];  // 64 rows of c + 1
  const int stride = c + 1;
  long total = (long)rows * lanes;
  long r0 = (long)blockIdx.x * 64;
  int nr = (int)min((long)64, total - r0);
  for (int e = threadIdx.x; e < nr * c; e += 64) {
    int rr = e / c, k = e - rr * c;
    long row = r0 + rr;
    int ln = (int)(row / rows);
    long rl = row - (long)ln * rows;
    tile[rr * stride + k] = x[(long)ln * x_lane_stride + rl * c + k];
  }
  __syncthreads();
  if ((int)threadIdx.x < nr) {
    float *v = tile + threadIdx.x * stride;
    float s = 0.0f;
    for (int i = 0; i < c; i++) s = s + v[i];
    float mean = s / (float)c;
    float q = 0.0f;
    for (int i = 0; i < c; i++) {
      float d = v[i] - mean;
      q = q + d * d;
    }
    float var = q / (float)c;
    float r = sqrtf(var + w[2 * c]);
    for (int i = 0; i < c; i++) v[i] = (v[i] - mean) / r * w[i] + w[c + i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < nr * c; e += 64) {
    int rr = e / c, k = e - rr * c;
    long row = r0 + rr;
    int ln = (int)(row / rows);
    long rl = row - (long)ln * rows;
    y[(long)ln * y_lane_stride + rl * c + k] = tile[rr * stride + k];
  }
}

hipError_t launch_layernorm(const float *x, long x_lane_stride, const float *w, int rows, int c,
                            int lanes, float *y, long y_lane_stride, hipStream_t s) {
  long total = (long)rows * lanes;
  size_t shm = (size_t)64 * (c + 1) * sizeof(float);
  if (shm > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(layernorm_kernel, dim3(blocks_for(total, 64)), dim3(64), shm, s, x,
                     x_lane_stride, w, rows, c, lanes, y, y_lane_stride);
  return hipGetLastError();
}

// ------------------------------------------------------------ attention

// One block per (lane, head): K and V of the head in LDS, one thread per
// query (looping when t exceeds the block). Scores from zero with a fused
// multiply-add per head dimension against the pre-scaled query, an 8-lane
// softmax, then each output from zero with a fused multiply-add per key.
__global__ __launch_bounds__(128) void attention_kernel(const float *x, long x_lane_stride,
                                                       float scale, int t, int c, int heads,
                                                       float *y, long y_lane_stride,
                                                       float *gscores) {
  extern __shared__ float sm[];
  const int hd = c / heads;
  const int ln = blockIdx.x / heads, h = blockIdx.x % heads;
  float *ks = sm;                 // t * hd
  float *vs = ks + t * hd;        // t * hd
  // blockDim.x score rows of t + 1: in LDS, or for long lines in global memory.
  float *sc = gscores ? gscores + (long)blockIdx.x * blockDim.x * (t + 1) : vs + t * hd;
  const float *xl = x + (long)ln * x_lane_stride;
  for (int e = threadIdx.x; e < t * hd; e += blockDim.x) {
    int j = e / hd, d = e - j * hd;
    ks[e] = xl[(long)j * 3 * c + c + h * hd + d];
    vs[e] = xl[(long)j * 3 * c + 2 * c + h * hd + d];
  }
  __syncthreads();
  float *row = sc + threadIdx.x * (t + 1);
  for (int s = threadIdx.x; s < t; s += blockDim.x) {
    float q[64];
    for (int d = 0; d < hd; d++) q[d] = xl[(long)s * 3 * c + h * hd + d] * scale;
    for (int j = 0; j < t; j++) {
      float acc = 0.0f;
      for (int d = 0; d < hd; d++) acc = fmaf(ks[j * hd + d], q[d], acc);
      row[j] = acc;
    }
    // Softmax of the row in 8 lanes (src/engine/layers.rs:273-294).
    int body = t / 8 * 8;
    float lanes_[8];
    for (int l = 0; l < 8; l++) lanes_[l] = -__builtin_inff();
    for (int j = 0; j < body; j++) {
      float v = row[j];
      lanes_[j & 7] = v > lanes_[j & 7] ? v : lanes_[j & 7];
    }
    float mx = -__builtin_inff();
    for (int l = 0; l < 8; l++) mx = fmaxf(mx, lanes_[l]);
    for (int j = body; j < t; j++) mx = fmaxf(mx, row[j]);
    float sums[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < body; j++) {
      float e = exp_neg(row[j] - mx);
      row[j] = e;
      sums[j & 7] = sums[j & 7] + e;
    }
    float sum = 0.0f;
    for (int l = 0; l < 8; l++) sum = sum + sums[l];
    for (int j = body; j < t; j++) {
      float e = exp_neg(row[j] - mx);
      row[j] = e;
      sum = sum + e;
    }
    float r = 1.0f / sum;
    for (int j = 0; j < t; j++) row[j] = row[j] * r;
    float *out = y + (long)ln * y_lane_stride + (long)s * c + h * hd;
    for (int d = 0; d < hd; d++) {
      float acc = 0.0f;
      for (int j = 0; j < t; j++) acc = fmaf(vs[j * hd + d], row[j], acc);
      out[d] = acc;
    }
  }
}

static int attention_threads(int t) { return t < 128 ? ((t + 63) / 64) * 64 : 128; }

static bool attention_in_lds(int t, int hd) {
  size_t shm = ((size_t)2 * t * hd + (size_t)attention_threads(t) * (t + 1)) * sizeof(float);
  return shm <= 64 * 1024;
}

size_t attention_scratch_floats(int t, int c, int heads, int lanes) {
  int hd = c / heads;
  if (attention_in_lds(t, hd)) return 0;
  return (size_t)lanes * heads * attention_threads(t) * (t + 1);
}

hipError_t launch_attention(const float *x, long x_lane_stride, float scale, int t, int c,
                            int heads, int lanes, float *y, long y_lane_stride, float *scratch,
                            hipStream_t s) {
  int hd = c / heads;
  if (hd > 64 || heads <= 0 || c % heads) return hipErrorInvalidValue;
  int threads = attention_threads(t);
  bool lds = attention_in_lds(t, hd);
  if (!lds && !scratch) return hipErrorInvalidValue;
  size_t shm = ((size_t)2 * t * hd + (lds ? (size_t)threads * (t + 1) : 0)) * sizeof(float);
  if (shm > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(attention_kernel, dim3(lanes * heads), dim3(threads), shm, s, x,
                     x_lane_stride, scale, t, c, heads, y, y_lane_stride, lds ? nullptr : scratch);
  return hipGetLastError();
}

// ------------------------------------------------------------ CTC choice

struct Best {
  float m, s, b;
};

__device__ __forceinline__ Best best_join(Best x, Best y) {
  const float ninf = -__builtin_inff();
  Best r;
  r.m = x.m > y.m ? x.m : y.m;
  float sx = x.m == ninf ? 0.0f : x.s * exp_neg(x.m - r.m);
  float sy = y.m == ninf ? 0.0f : y.s * exp_neg(y.m - r.m);
  r.s = sx + sy;
  r.b = x.m > y.m ? x.b : (y.m > x.m ? y.b : fminf(x.b, y.b));
  return r;
}

// One block per row: each thread keeps a running (max, sum, first column)
// over columns tid, tid + 256, ...; the block joins them in a fixed order.
__global__ __launch_bounds__(256) void row_argmax_kernel(const float *x, float *y, int cols) {
  __shared__ Best part[4];
  const float *row = x + (long)blockIdx.x * cols;
  Best st{-__builtin_inff(), 0.0f, __builtin_inff()};
  int col = threadIdx.x;
  for (; col + 768 < cols; col += 1024) {
    float v0 = row[col], v1 = row[col + 256], v2 = row[col + 512], v3 = row[col + 768];
    float vs[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      float v = vs[k];
      if (v > st.m) {
        st.s = st.s * exp_neg(st.m - v) + 1.0f;
        st.m = v;
        st.b = (float)(col + 256 * k);
      } else {
        st.s = st.s + exp_neg(v - st.m);
      }
    }
  }
  for (; col < cols; col += 256) {
    float v = row[col];
    if (v > st.m) {
      st.s = st.s * exp_neg(st.m - v) + 1.0f;
      st.m = v;
      st.b = (float)col;
    } else {
      st.s = st.s + exp_neg(v - st.m);
    }
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    Best o{__shfl_xor(st.m, d, 64), __shfl_xor(st.s, d, 64), __shfl_xor(st.b, d, 64)};
    st = best_join(st, o);
  }
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = st;
  __syncthreads();
  if (threadIdx.x == 0) {
    Best r = part[0];
    for (int k = 1; k < 4; k++) r = best_join(r, part[k]);
    y[2 * (long)blockIdx.x] = r.b;
    y[2 * (long)blockIdx.x + 1] = 1.0f / r.s;
  }
}

hipError_t launch_row_argmax(const float *x, float *y, int rows, int cols, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(row_argmax_kernel, dim3(rows), dim3(256), 0, s, x, y, cols);
  return hipGetLastError();
}

// ------------------------------------------------------------ narrow convT

// One thread per input pixel: its kh*kw*oc (<= 16) outputs, each a fused
// multiply-add per input channel in order, then the activation. The bias
// comes first or last as the engine's pointwise call over one input row
// puts it (src/engine/layers.rs:658-679, kernels/pointwise.rs:135-185):
// first for a 16-column block except the row's last iw % 4 pixels, else
// last.
__global__ __launch_bounds__(256) void convt_small_kernel(ConvtArgs a) {
  long per = (long)a.ih * a.iw;
  long g = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (g >= (long)a.lanes * per) return;
  int ln = (int)(g / per);
  long pix = g - (long)ln * per;
  int iy = (int)(pix / a.iw), ix = (int)(pix - (long)iy * a.iw);
  const int cols = a.kh * a.kw * a.oc;
  const bool first = a.bias && cols == 16 && ix < a.iw / 4 * 4;
  const float *xp = a.x + (long)ln * a.x_lane_stride + pix * a.ic;
  float acc[16];
#pragma unroll
  for (int n = 0; n < 16; n++) acc[n] = first && n < cols ? a.bias[n] : 0.0f;
  for (int i = 0; i < a.ic; i++) {
    float v = xp[i];
#pragma unroll
    for (int n = 0; n < 16; n++)
      if (n < cols) acc[n] = fmaf(a.w[(long)i * cols + n], v, acc[n]);
  }
  float *yl = a.y + (long)ln * a.y_lane_stride;
  const long ow = (long)a.iw * a.kw;
#pragma unroll
  for (int n = 0; n < 16; n++) {
    if (n >= cols) break;
    float v = acc[n];
    if (a.bias && !first) v = v + a.bias[n];
    v = act(v, a.act);
    int tap = n / a.oc, o = n - tap * a.oc;
    int ky = tap / a.kw, kx = tap - ky * a.kw;
    yl[((long)(iy * a.kh + ky) * ow + (long)ix * a.kw + kx) * a.oc + o] = v;
  }
}

hipError_t launch_convt_small(const ConvtArgs &a, hipStream_t s) {
  if (a.kh * a.kw * a.oc > 16) return hipErrorInvalidValue;
  long n = (long)a.lanes * a.ih * a.iw;
  hipLaunchKernelGGL(convt_small_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace ppocr
