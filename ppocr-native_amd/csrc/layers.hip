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
#include <algorithm>

#include "act.hpp"
#include "kernels.hpp"

namespace ppocr {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// LDS a workgroup may use on gfx950 (kernels above 64 KiB raise their limit).
static const size_t kMaxLds = 160 * 1024;

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

// The same arithmetic with the window's size K and stride S known at compile
// time: each kernel row's input segment ((DX - 1) * S + K pixels of four
// channels) is loaded once, every load of the row issued before the first
// multiply-add; taps outside the image are skipped, as in the engine.
// Threads of a block of the depthwise kernel that also sums its outputs.
constexpr int kDwMeanThreads = 256;

template <int K, int S, int DX, bool MEAN, int TB = 256>
__global__ __launch_bounds__(MEAN ? TB : 256) void dwconv_fixed(DwArgs a) {
  constexpr int SPAN = (DX - 1) * S + K;
  const int cv = a.c / 4;
  const int runs = (a.ow + DX - 1) / DX;
  int ch, run, oy, ln, bx = 0;
  bool live;
  if constexpr (MEAN) {
    // Block = R runs of one lane x every channel group, so that the block
    // can sum its outputs per channel (dw_mean_blocks blocks per lane).
    // Blocks numbered XCD by XCD over the whole grid (xcd_tile); a block's
    // sums go to the slot of the rows it computed, so the join order stays.
    const int R = TB / cv;
    const int r = threadIdx.x / cv;
    ch = (threadIdx.x - r * cv) * 4;
    const int nbx = (int)gridDim.x;
    const int lin = xcd_tile((int)(blockIdx.y * gridDim.x + blockIdx.x), (int)(gridDim.x * gridDim.y));
    bx = lin % nbx;
    const int rg = bx * R + r;
    ln = lin / nbx;
    live = r < R && rg < a.oh * runs;
    oy = rg / runs;
    run = rg - oy * runs;
  } else {
    // Blocks numbered XCD by XCD (xcd_tile): neighbouring output rows, which
    // read the same input rows, meet in one L2.
    const long g = (long)xcd_tile((int)blockIdx.x, (int)gridDim.x) * blockDim.x + threadIdx.x;
    const long total = (long)a.lanes * a.oh * runs * cv;
    if (g >= total) return;
    ch = (int)(g % cv) * 4;
    long t = g / cv;
    run = (int)(t % runs);
    t /= runs;
    oy = (int)(t % a.oh);
    ln = (int)(t / a.oh);
    live = true;
  }
  double sum[4] = {0.0, 0.0, 0.0, 0.0};
  if (live) {
    const int ox0 = run * DX;
    const float *x = a.x + (long)ln * a.x_lane_stride + ch;
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc[DX];
    f32x4 bias = a.bias ? *reinterpret_cast<const f32x4 *>(a.bias + ch) : zero;
#pragma unroll
    for (int o = 0; o < DX; o++) acc[o] = bias;
    const int left = ox0 * S - a.pl;
    bool in[SPAN];
#pragma unroll
    for (int i = 0; i < SPAN; i++) in[i] = left + i >= 0 && left + i < a.iw;
    // 3 x 3 windows: every row's loads are unconditional (a row outside the
    // image reads the nearest one, whose taps are then skipped), so that the
    // compiler issues all three rows' loads before the first multiply-add
    // (one wait instead of three, 119 registers). Wider windows would need
    // 256 registers that way: their rows load in turn.
    constexpr bool kAllRows = K == 3;
#pragma unroll
    for (int ky = 0; ky < K; ky++) {
      const int iy = oy * a.sh + ky - a.pt;
      const bool row_in = iy >= 0 && iy < a.ih;
      if (!kAllRows && !row_in) continue;
      const float *row = x + (long)min(max(iy, 0), a.ih - 1) * a.iw * a.c;
      f32x4 seg[SPAN], wk[K];
#pragma unroll
      for (int i = 0; i < SPAN; i++) seg[i] = in[i] ? *reinterpret_cast<const f32x4 *>(row + (long)(left + i) * a.c) : zero;
#pragma unroll
      for (int kx = 0; kx < K; kx++) wk[kx] = *reinterpret_cast<const f32x4 *>(a.w + (long)(ky * K + kx) * a.c + ch);
#pragma unroll
      for (int kx = 0; kx < K; kx++) {
#pragma unroll
        for (int o = 0; o < DX; o++) {
          const int i = o * S + kx;
          if (row_in && in[i]) {
            acc[o].x = fmaf(wk[kx].x, seg[i].x, acc[o].x);
            acc[o].y = fmaf(wk[kx].y, seg[i].y, acc[o].y);
            acc[o].z = fmaf(wk[kx].z, seg[i].z, acc[o].z);
            acc[o].w = fmaf(wk[kx].w, seg[i].w, acc[o].w);
          }
        }
      }
    }
    float *y = a.y + (long)ln * a.y_lane_stride + ((long)oy * a.ow) * a.c + ch;
#pragma unroll
    for (int o = 0; o < DX; o++) {
      if (ox0 + o >= a.ow) break;
      f32x4 v = acc[o];
      v.x = act(v.x, a.act);
      v.y = act(v.y, a.act);
      v.z = act(v.z, a.act);
      v.w = act(v.w, a.act);
      *reinterpret_cast<f32x4 *>(y + (long)(ox0 + o) * a.c) = v;
      if constexpr (MEAN) {
        sum[0] += (double)v.x;
        sum[1] += (double)v.y;
        sum[2] += (double)v.z;
        sum[3] += (double)v.w;
      }
    }
  }
  if constexpr (MEAN) {
    // The block's f64 sums per channel, its runs joined in order.
    __shared__ double red[TB * 4];
#pragma unroll
    for (int k = 0; k < 4; k++) red[threadIdx.x * 4 + k] = sum[k];
    __syncthreads();
    const int R = TB / cv;
    if ((int)threadIdx.x < cv) {
      double tot[4] = {0.0, 0.0, 0.0, 0.0};
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int k = 0; k < 4; k++) tot[k] += red[(r * cv + threadIdx.x) * 4 + k];
      double *out = a.mean_part + ((long)ln * gridDim.x + bx) * a.c + threadIdx.x * 4;
#pragma unroll
      for (int k = 0; k < 4; k++) out[k] = tot[k];
    }
  }
}

template <typename F>
static hipError_t launch_fixed(F kernel, dim3 grid, dim3 block, const DwArgs &a, hipStream_t s) {
  hipLaunchKernelGGL(kernel, grid, block, 0, s, a);
  return hipGetLastError();
}

static constexpr int kDwRun = 4;  // outputs per thread along a row

// Outputs per thread along a row: four, or one when the layer is small (a
// few thread-rows of float4 per SIMD), so that its threads fill the GPU.
// With the channel sums the block count is the count of partial rows the
// mean joins, so those layers keep four (one output a thread in blocks four
// times as wide, to keep that count, ran slower: fewer blocks than CUs).
static int dw_run(const DwArgs &a) {
  return (long)a.lanes * a.oh * a.ow * (a.c / 4) < (1L << 18) && !a.mean_part ? 1 : kDwRun;
}

// The fixed-window variants: (kernel, stride) pairs with a template, the
// height-only strides (the recogniser's (2, 1) stages) run as stride 1.
static int dw_fixed_kind(const DwArgs &a) {
  if (a.kh != a.kw) return 0;
  const int k = a.kh;
  if (a.sh == a.sw) {
    if (k == 3 && a.sw == 1) return 31;
    if (k == 3 && a.sw == 2) return 32;
    if (k == 5 && a.sw == 1) return 51;
    if (k == 5 && a.sw == 2) return 52;
    if (k == 7 && a.sw == 1) return 71;
  } else if (a.sw == 1) {
    if (k == 3) return 31;
    if (k == 5) return 51;
  }
  return 0;
}

// ------------------------------------------------------- depthwise on tiles

// The depthwise convolution on output tiles of TR rows x TW columns x 4 * CG
// channels of one lane (TR, TW chosen on the host so that a tile has at most
// 256 / CG pixels): the tile's input window (the tile plus its halo, all its
// rows and columns, zero outside the image) and the taps' weights go into LDS
// by direct loads, all of them in flight at once, then each thread computes
// one output pixel of four channels from LDS. The same arithmetic as
// dwconv_fixed: from the bias, taps row by row, one fused multiply-add each,
// taps outside the image skipped (not multiplied by zero, which could turn a
// -0 sum into +0). Where dwconv_fixed makes each thread wait for K rows of
// loads in turn and gives small maps few threads, a tile waits for one round
// of loads and every output has its own thread.
//
// With MEAN the tile also sums its outputs per channel in f64 (pixels in
// thread order) into the partial row of its spatial tile: row (lane, tile)
// of dw_mean_blocks(a) rows per lane, the channels of the tile's group.
constexpr int kDwTileThreads = 256;

struct DwTile {
  int cg, tr, tw, tiles_x, tiles_y;
};

__device__ __attribute__((aligned(16))) float kDwZeros[4];

// Input rows and columns a tile's window covers.
__host__ __device__ inline int dw_tile_rows(const DwArgs &a, int tr) { return (tr - 1) * a.sh + a.kh; }
__host__ __device__ inline int dw_tile_cols(const DwArgs &a, int tw) { return (tw - 1) * a.sw + a.kw; }

template <int K, int S, int CG, bool MEAN>
__global__ __launch_bounds__(kDwTileThreads) void dwconv_tile(DwArgs a, DwTile tt) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int groups = a.c / (4 * CG);
  const int per_lane = tt.tiles_y * tt.tiles_x;
  // Blocks numbered XCD by XCD: neighbouring tiles of one channel group,
  // which share halo rows, meet in one L2.
  int b = xcd_tile((int)blockIdx.x, (int)gridDim.x);
  const int tx = b % tt.tiles_x;
  b /= tt.tiles_x;
  const int ty = b % tt.tiles_y;
  b /= tt.tiles_y;
  const int gi = b % groups, ln = b / groups;
  const int oy0 = ty * tt.tr, ox0 = tx * tt.tw, c0 = gi * 4 * CG;
  const int IR = dw_tile_rows(a, tt.tr), IC = dw_tile_cols(a, tt.tw);
  const int iy0 = oy0 * a.sh - a.pt, ix0 = ox0 * S - a.pl;
  const int win = IR * IC * CG;  // float4s of the window
  constexpr int WA = (K * K * CG + 63) / 64 * 64;  // float4s of the weights' area (whole loads)
  float *W = lds;                          // K * K taps x CG float4
  float *X = lds + WA * 4;                 // IR x IC pixels x CG float4 (rounded up to whole loads)
  const float *xl = a.x + (long)ln * a.x_lane_stride + c0;
  // Direct loads: float4 u of an area from src(u), 64 per instruction, the
  // instructions dealt over the waves.
  for (int q = wave; q * 64 < K * K * CG; q += 4) {
    const int u = q * 64 + lane;
    const int tap = u / CG, g = u - tap * CG;
    const float *p = u < K * K * CG ? a.w + (long)tap * a.c + c0 + 4 * g : kDwZeros;
    __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(W + q * 256), 16, 0, 0);
  }
  for (int q = wave; q * 64 < win; q += 4) {
    const int u = q * 64 + lane;
    const int pix = u / CG, g = u - pix * CG;
    const int r = pix / IC, col = pix - r * IC;
    const int iy = iy0 + r, ix = ix0 + col;
    const float *p = u < win && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw
                         ? xl + ((long)iy * a.iw + ix) * a.c + 4 * g
                         : kDwZeros;
    __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(X + q * 256), 16, 0, 0);
  }
  const int g = tid % CG, px = tid / CG;
  const int r = px / tt.tw, col = px - r * tt.tw;
  const int oy = oy0 + r, ox = ox0 + col;
  const bool live = r < tt.tr && oy < a.oh && ox < a.ow;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc = a.bias && live ? *reinterpret_cast<const f32x4 *>(a.bias + c0 + 4 * g) : zero;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  double sum[4] = {0.0, 0.0, 0.0, 0.0};
  if (live) {
    const int ry = r * a.sh, cx = col * S;
#pragma unroll
    for (int ky = 0; ky < K; ky++) {
      const int iy = iy0 + ry + ky;
      if (iy < 0 || iy >= a.ih) continue;
      const float *xr = X + ((ry + ky) * IC + cx) * CG * 4 + 4 * g;
#pragma unroll
      for (int kx = 0; kx < K; kx++) {
        const int ix = ix0 + cx + kx;
        if (ix < 0 || ix >= a.iw) continue;
        const f32x4 wv = *reinterpret_cast<const f32x4 *>(W + (ky * K + kx) * CG * 4 + 4 * g);
        const f32x4 xv = *reinterpret_cast<const f32x4 *>(xr + kx * CG * 4);
        acc.x = fmaf(wv.x, xv.x, acc.x);
        acc.y = fmaf(wv.y, xv.y, acc.y);
        acc.z = fmaf(wv.z, xv.z, acc.z);
        acc.w = fmaf(wv.w, xv.w, acc.w);
      }
    }
    f32x4 v = acc;
    v.x = act(v.x, a.act);
    v.y = act(v.y, a.act);
    v.z = act(v.z, a.act);
    v.w = act(v.w, a.act);
    *reinterpret_cast<f32x4 *>(a.y + (long)ln * a.y_lane_stride + ((long)oy * a.ow + ox) * a.c + c0 + 4 * g) = v;
    if constexpr (MEAN) sum[0] = v.x, sum[1] = v.y, sum[2] = v.z, sum[3] = v.w;
  }
  if constexpr (MEAN) {
    // The tile's f64 sums per channel, its pixels added in thread order.
    __syncthreads();  // every wave is done with the window: reuse it
    double *red = reinterpret_cast<double *>(X);
#pragma unroll
    for (int k = 0; k < 4; k++) red[tid * 4 + k] = sum[k];
    __syncthreads();
    if (tid < 4 * CG) {
      const int gg = tid / 4, k = tid % 4;
      double tot = 0.0;
      for (int pp = 0; pp < kDwTileThreads / CG; pp++) tot += red[(pp * CG + gg) * 4 + k];
      a.mean_part[((long)ln * per_lane + ty * tt.tiles_x + tx) * a.c + c0 + tid] = tot;
    }
  }
}

// The tiling of a layer, or cg = 0 when the tiled kernel does not take it.
// It takes channels a multiple of 16, the compiled windows, within the LDS
// bound, and of those the layers where it ran faster than dwconv_fixed in
// the detector's and the recogniser's graphs: 7 x 7 windows (the detector's
// 60 x 60 x 192 12.6 -> 9.4 us, 30 x 30 x 384 12.0 -> 8.3 us), 5 x 5 windows
// of at most 180K output float4s (times the stride), where few long-latency
// threads leave the GPU idle (60 x 60 x 192 8.0 -> 6.7 us, stride 2 to 30 x
// 30 x 192 9.3 -> 6.6 us), and 3 x 3 windows of one image without channel
// sums (the detector's three: its graph 508 -> 505 us). On the recogniser's
// sixteen lines and on the fused block's 3 x 3 with sums, dwconv_fixed's
// four outputs a thread reusing their loaded rows win (recogniser 413 ->
// 419 us, fused block 42.4 -> 47.9 us when tiled).
static DwTile dw_tile_of(const DwArgs &a, bool sums) {
  DwTile t{};
  const bool kind = a.kh == a.kw && (a.kh == 3 || a.kh == 5 || a.kh == 7) && (a.sw == 1 || (a.sw == 2 && a.kh != 7));
  if (!kind || a.c % 16 != 0 || a.sh < 1 || a.sh > 2) return t;
  const long work = (long)a.lanes * a.oh * a.ow * (a.c / 4) * a.sw;
  const bool one_image_3x3 = a.kh == 3 && a.lanes == 1 && !sums;
  if (!(a.kh == 7 || (a.kh == 5 && work <= 180L * 1024) || one_image_3x3)) return t;
  const int cg = a.c % 32 == 0 ? 8 : 4;
  const int pix = kDwTileThreads / cg;
  const int nx = (a.ow + pix - 1) / pix;
  const int tw = (a.ow + nx - 1) / nx;
  const int tr = std::max(1, std::min(pix / tw, a.oh));
  const size_t win = size_t(dw_tile_rows(a, tr)) * dw_tile_cols(a, tw) * cg;
  const size_t floats = (size_t(a.kh) * a.kw * cg + 63) / 64 * 64 * 4 + (win + 63) / 64 * 64 * 4;
  if (floats * sizeof(float) > 64 * 1024) return t;
  t.cg = cg, t.tr = tr, t.tw = tw, t.tiles_x = nx, t.tiles_y = (a.oh + tr - 1) / tr;
  return t;
}

static size_t dw_tile_lds(const DwArgs &a, const DwTile &t) {
  const size_t win = size_t(dw_tile_rows(a, t.tr)) * dw_tile_cols(a, t.tw) * t.cg;
  const size_t wa = (size_t(a.kh) * a.kw * t.cg + 63) / 64 * 64 * 4;
  size_t floats = wa + (win + 63) / 64 * 64 * 4;
  if (a.mean_part) floats = std::max(floats, wa + kDwTileThreads * 4 * 2);
  return floats * sizeof(float);
}

template <int CG, bool MEAN>
static hipError_t go_dw_tile(const DwArgs &a, const DwTile &t, hipStream_t s) {
  const long blocks = (long)a.lanes * (a.c / (4 * CG)) * t.tiles_y * t.tiles_x;
  if (blocks < 1 || blocks > 0x7fffffffL) return hipErrorInvalidValue;
  const dim3 grid((unsigned)blocks), block(kDwTileThreads);
  const size_t lds = dw_tile_lds(a, t);
  const int kind = a.kh * 10 + a.sw;
#define PPOCR_DW_TILE(KK, SS) \
  if (kind == KK * 10 + SS) { hipLaunchKernelGGL((dwconv_tile<KK, SS, CG, MEAN>), grid, block, lds, s, a, t); return hipGetLastError(); }
  PPOCR_DW_TILE(3, 1) PPOCR_DW_TILE(3, 2) PPOCR_DW_TILE(5, 1) PPOCR_DW_TILE(5, 2) PPOCR_DW_TILE(7, 1)
#undef PPOCR_DW_TILE
  return hipErrorInvalidValue;
}

static hipError_t launch_dw_tile(const DwArgs &a, const DwTile &t, hipStream_t s) {
  if (a.mean_part) return t.cg == 8 ? go_dw_tile<8, true>(a, t, s) : go_dw_tile<4, true>(a, t, s);
  return t.cg == 8 ? go_dw_tile<8, false>(a, t, s) : go_dw_tile<4, false>(a, t, s);
}

// ------------------------------------------- depthwise, then a 1x1, on tiles

// A depthwise layer and the 1x1 convolution that alone reads its output, in
// one launch. A workgroup takes a tile of TR x TW output pixels of one lane
// (at most P = 16 * RB: the MFMA rows) and every channel. The tile's input
// window (zero outside the image), the depthwise taps and bias, and the
// residual rows go into LDS by direct loads, all in flight together with
// the 1x1's weights (from the MFMA operand packing straight into B
// registers) and its bias. Each thread then computes depthwise outputs
// (pixel, channel quad) from LDS in dwconv_fixed's arithmetic (from the
// bias, taps row by row, one fused multiply-add each, taps outside the image
// skipped) into rows of c + 4 floats, and wave w multiplies every row block
// by column blocks w, w + 4, ... on v_mfma_f32_16x16x4_f32 (input group q of
// 16 channels, lane group g supplying channels 16q + 4g + e to step e). The
// products (plus the bias) go back to LDS over the spent window, and every
// thread finishes float4s of output rows: activation, residual, second
// activation, one coalesced store. Loops over pixels run rolled, so each
// activation is compiled once.
constexpr int kDwPwKq = 8;  // channel groups of 16 a workgroup holds: c <= 128

struct DwPwLds {
  int x, a, r, total;  // float offsets of the window / products, the depthwise rows, the residual
};

__host__ __device__ inline DwPwLds dwpw_lds(const DwArgs &d, int n, int tr, int tw, int p, bool res) {
  DwPwLds l;
  l.x = ((d.kh * d.kw + 1) * (d.c / 4) + 63) / 64 * 256;  // taps and bias, whole loads
  const int win = (dw_tile_rows(d, tr) * dw_tile_cols(d, tw) * (d.c / 4) + 63) / 64 * 256;
  const int prod = p * ((n + 15) / 16 * 16 + 4);
  l.a = l.x + (std::max(win, prod) + 63) / 64 * 64;
  l.r = l.a + (p * (d.c + 4) + 63) / 64 * 64;
  l.total = l.r + (res ? (p * (n / 4) + 63) / 64 * 256 : 0);
  return l;
}

// An activation of four values, dispatched once for the four (the common
// codes fold to their own few instructions).
__device__ __forceinline__ f32x4 act4(f32x4 v, int a) {
  switch (a) {
    case ACT_NONE: return v;
    case ACT_RELU: return f32x4{act(v.x, ACT_RELU), act(v.y, ACT_RELU), act(v.z, ACT_RELU), act(v.w, ACT_RELU)};
    case ACT_HARDSWISH:
      return f32x4{act(v.x, ACT_HARDSWISH), act(v.y, ACT_HARDSWISH), act(v.z, ACT_HARDSWISH), act(v.w, ACT_HARDSWISH)};
    default: return f32x4{act(v.x, a), act(v.y, a), act(v.z, a), act(v.w, a)};
  }
}

// The 1x1's products over KQ groups of 16 channels: wave-uniform, every
// column block of the wave (blocks past the last are computed and dropped),
// no branch inside the chain.
template <int KQ, int RB, int NBW>
__device__ __forceinline__ void dwpw_mfma(f32x4 (&acc)[RB][NBW], const float *A, int AS,
                                          const f32x4 (&bw)[NBW][kDwPwKq], int li, int lg) {
#pragma unroll
  for (int q = 0; q < KQ; q++) {
    f32x4 af[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) af[rb] = *reinterpret_cast<const f32x4 *>(A + (16 * rb + li) * AS + 16 * q + 4 * lg);
#pragma unroll
    for (int e = 0; e < 4; e++)
#pragma unroll
      for (int jj = 0; jj < NBW; jj++)
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
          acc[rb][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[rb][e], bw[jj][q][e], acc[rb][jj], 0, 0, 0);
  }
}

template <int K, int S, int RB, int NBW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void dwpw_tile(DwPwArgs a, DwTile tt) {
  constexpr int P = 16 * RB;
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const DwArgs &d = a.d;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, lg = lane >> 4;
  const int C = d.c, C4 = C / 4, KQ = C / 16, N = a.n, N4 = N / 4, NB = (N + 15) / 16;
  const int AS = C + 4, ON = NB * 16 + 4;
  // Tiles numbered XCD by XCD: neighbours, which share halo rows, meet in one L2.
  int b = xcd_tile((int)blockIdx.x, (int)gridDim.x);
  const int tx = b % tt.tiles_x;
  b /= tt.tiles_x;
  const int ty = b % tt.tiles_y, ln = b / tt.tiles_y;
  const int oy0 = ty * tt.tr, ox0 = tx * tt.tw;
  const int IC = dw_tile_cols(d, tt.tw);
  const int iy0 = oy0 * d.sh - d.pt, ix0 = ox0 * S - d.pl;
  const int wq = (K * K + 1) * C4, win = dw_tile_rows(d, tt.tr) * IC * C4;
  const DwPwLds L = dwpw_lds(d, N, tt.tr, tt.tw, P, a.res != nullptr);
  float *W = lds;          // taps [K * K][C], then the bias [C]
  float *X = lds + L.x;    // the window; later the products, rows of ON
  float *A = lds + L.a;    // the depthwise rows, AS apart
  float *R = lds + L.r;    // the residual rows, N apart
  // Output pixel p of the tile: its place in the lane's map, or -1 past the
  // tile or the map.
  auto out_at = [&](int p) {
    const int r = p / tt.tw, col = p - r * tt.tw;
    const int oy = oy0 + r, ox = ox0 + col;
    return r < tt.tr && oy < d.oh && ox < d.ow ? oy * d.ow + ox : -1;
  };
  const float *xl = d.x + (long)ln * d.x_lane_stride;
  for (int q = wave; q * 64 < wq; q += 4) {
    const int u = q * 64 + lane;
    const int tap = u / C4, g = u - tap * C4;
    const float *p = u >= wq ? kDwZeros
                     : tap < K * K ? d.w + (long)tap * C + 4 * g
                                   : (d.bias ? d.bias + 4 * g : kDwZeros);
    __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(W + q * 256), 16, 0, 0);
  }
  for (int q = wave; q * 64 < win; q += 4) {
    const int u = q * 64 + lane;
    const int pix = u / C4, g = u - pix * C4;
    const int r = pix / IC, col = pix - r * IC;
    const int iy = iy0 + r, ix = ix0 + col;
    const float *p = u < win && iy >= 0 && iy < d.ih && ix >= 0 && ix < d.iw
                         ? xl + ((long)iy * d.iw + ix) * C + 4 * g
                         : kDwZeros;
    __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(X + q * 256), 16, 0, 0);
  }
  if (a.res) {
    const float *rl = a.res + (long)ln * a.res_lane_stride;
    for (int q = wave; q * 64 < P * N4; q += 4) {
      const int u = q * 64 + lane, p = u / N4, c4 = u - p * N4;
      const int at = u < P * N4 ? out_at(p) : -1;
      const float *src = at >= 0 ? rl + (long)at * N + 4 * c4 : kDwZeros;
      __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(R + q * 256), 16, 0, 0);
    }
  }
  // The 1x1's B operands and bias, in flight beside the window. Every load
  // is unconditional (indices clamped; the operands past the last column
  // block or channel group are never used), so that none waits at a branch.
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  f32x4 bw[NBW][kDwPwKq];
  float pb[NBW];
  const float *bsrc = a.pw_b ? a.pw_b : a.pw;
#pragma unroll
  for (int jj = 0; jj < NBW; jj++) {
    const int j = min(wave + 4 * jj, NB - 1);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(a.pw) + (long)j * KQ * 64 + lane;
#pragma unroll
    for (int q = 0; q < kDwPwKq; q++) bw[jj][q] = src[min(q, KQ - 1) * 64];
    pb[jj] = bsrc[min(16 * j + li, N - 1)];
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // Thread t takes channel quad g = t % C4 of pixels t / C4, t / C4 + slots,
  // ... (slots = 256 / C4; threads past slots * C4 rest), so that a 3 x 3
  // window's taps and the bias stay in its registers.
  const int slots = 256 / C4, g = tid % C4, p0 = tid / C4;
  constexpr int KR = K <= 3 ? K * K : 1;
  f32x4 wk[KR];
  const f32x4 bias4 = *reinterpret_cast<const f32x4 *>(W + K * K * C + 4 * g);
  if constexpr (K <= 3) {
#pragma unroll
    for (int k = 0; k < KR; k++) wk[k] = *reinterpret_cast<const f32x4 *>(W + k * C + 4 * g);
  }
#pragma unroll 1
  for (int p = p0; p0 < slots && p < P; p += slots) {
    f32x4 v = zero;
    if (out_at(p) >= 0) {
      const int r = p / tt.tw, col = p - r * tt.tw;
      const int ry = r * d.sh, cx = col * S;
      f32x4 acc = bias4;
      // Every tap's operands are read (the window holds zeros outside the
      // image); a tap outside the image leaves the sum as it is, by select,
      // so that the reads issue together and no lane branches.
      auto row = [&](int ky) {
        const int iy = iy0 + ry + ky;
        const bool in_y = iy >= 0 && iy < d.ih;
        const float *xr = X + ((ry + ky) * IC + cx) * C + 4 * g;
#pragma unroll
        for (int kx = 0; kx < K; kx++) {
          const int ix = ix0 + cx + kx;
          const bool in = in_y && ix >= 0 && ix < d.iw;
          f32x4 wv;
          if constexpr (K <= 3) wv = wk[ky * K + kx];
          else wv = *reinterpret_cast<const f32x4 *>(W + (ky * K + kx) * C + 4 * g);
          const f32x4 xv = *reinterpret_cast<const f32x4 *>(xr + kx * C);
          const f32x4 t = {fmaf(wv.x, xv.x, acc.x), fmaf(wv.y, xv.y, acc.y), fmaf(wv.z, xv.z, acc.z),
                           fmaf(wv.w, xv.w, acc.w)};
          acc = in ? t : acc;
        }
      };
      // A 3 x 3 window's rows unrolled; wider windows row by row, their taps
      // from LDS (all their operands at once would take more registers than
      // two waves a SIMD have).
      if constexpr (K <= 3) {
#pragma unroll
        for (int ky = 0; ky < K; ky++) row(ky);
      } else {
#pragma unroll 1
        for (int ky = 0; ky < K; ky++) row(ky);
      }
      v = act4(acc, d.act);
    }
    *reinterpret_cast<f32x4 *>(A + p * AS + 4 * g) = v;
  }
  __syncthreads();  // the depthwise rows are whole; the window is spent

  f32x4 acc[RB][NBW];
#pragma unroll
  for (int rb = 0; rb < RB; rb++)
#pragma unroll
    for (int jj = 0; jj < NBW; jj++) acc[rb][jj] = zero;
  switch (KQ) {
    case 1: dwpw_mfma<1>(acc, A, AS, bw, li, lg); break;
    case 2: dwpw_mfma<2>(acc, A, AS, bw, li, lg); break;
    case 3: dwpw_mfma<3>(acc, A, AS, bw, li, lg); break;
    case 4: dwpw_mfma<4>(acc, A, AS, bw, li, lg); break;
    case 5: dwpw_mfma<5>(acc, A, AS, bw, li, lg); break;
    case 6: dwpw_mfma<6>(acc, A, AS, bw, li, lg); break;
    case 7: dwpw_mfma<7>(acc, A, AS, bw, li, lg); break;
    default: dwpw_mfma<8>(acc, A, AS, bw, li, lg); break;
  }
#pragma unroll
  for (int jj = 0; jj < NBW; jj++) {
    const int j = wave + 4 * jj;
    if (j >= NB) continue;
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
      for (int r = 0; r < 4; r++)
        X[(16 * rb + 4 * lg + r) * ON + 16 * j + li] = a.pw_b ? acc[rb][jj][r] + pb[jj] : acc[rb][jj][r];
  }
  __syncthreads();
  float *yl = a.y + (long)ln * a.y_lane_stride;
#pragma unroll 1
  for (int u = tid; u < P * N4; u += 256) {
    const int p = u / N4, c4 = u - p * N4;
    const int at = out_at(p);
    if (at < 0) continue;
    f32x4 v = act4(*reinterpret_cast<const f32x4 *>(X + p * ON + 4 * c4), a.pw_act);
    if (a.res) v = act4(v + *reinterpret_cast<const f32x4 *>(R + p * N + 4 * c4), a.act2);
    *reinterpret_cast<f32x4 *>(yl + (long)at * N + 4 * c4) = v;
  }
}

static bool dwpw_shape_ok(const DwArgs &d, int n) {
  return d.kh == d.kw && (d.kh == 3 || d.kh == 5) && (d.sw == 1 || d.sw == 2) && (d.sh == 1 || d.sh == 2) &&
         d.c % 16 == 0 && d.c >= 16 && d.c <= 16 * kDwPwKq && n >= 4 && n <= 192 && n % 4 == 0 &&
         d.lanes >= 1 && d.oh >= 1 && d.ow >= 1;
}

// The tile of a fused layer: P = 64, 32 or 16 pixels as 8 x 8, 4 x 8 or
// 4 x 4 (narrower maps take whole rows), the largest whose LDS stays within
// 64 KiB (two workgroups a CU or more) and that still gives 256 tiles or
// more (measured against 512 and 1024 tiles and against 128-pixel tiles:
// each slower); rb = 0 when the fused kernel does not take the layer. Up to
// 192 output channels (three column blocks a wave): the recogniser's
// 128 -> 256 block fused on four took 20.4 us against 16.4 for its two
// launches.
static DwTile dwpw_tile_of(const DwArgs &d, int n, bool res, int &rb) {
  DwTile t{};
  rb = 0;
  if (!dwpw_shape_ok(d, n)) return t;
  for (int p : {64, 32, 16}) {
    int tw = p == 16 ? 4 : 8, tr = p / tw;
    if (d.ow < tw) tw = d.ow, tr = p / tw;
    if (d.oh < tr) tr = d.oh, tw = std::min(d.ow, p / tr);
    const long tiles = long(d.lanes) * ((d.oh + tr - 1) / tr) * ((d.ow + tw - 1) / tw);
    if (size_t(dwpw_lds(d, n, tr, tw, p, res).total) * 4 > 64 * 1024) continue;
    t = DwTile{0, tr, tw, (d.ow + tw - 1) / tw, (d.oh + tr - 1) / tr};
    rb = p / 16;
    if (tiles >= 256) break;
  }
  return t;
}

bool dwpw_supported(const DwArgs &d, int n, bool res) {
  int rb;
  dwpw_tile_of(d, n, res, rb);
  return rb > 0;
}

template <int K, int S, int RB>
static hipError_t go_dwpw(const DwPwArgs &a, const DwTile &t, size_t lds, dim3 grid, hipStream_t s) {
  const int nbw = ((a.n + 15) / 16 + 3) / 4;
  switch (nbw) {
    case 1: hipLaunchKernelGGL((dwpw_tile<K, S, RB, 1>), grid, dim3(256), lds, s, a, t); break;
    case 2: hipLaunchKernelGGL((dwpw_tile<K, S, RB, 2>), grid, dim3(256), lds, s, a, t); break;
    case 3: hipLaunchKernelGGL((dwpw_tile<K, S, RB, 3>), grid, dim3(256), lds, s, a, t); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dwpw(const DwPwArgs &a, hipStream_t s) {
  const DwArgs &d = a.d;
  int rb;
  const DwTile t = dwpw_tile_of(d, a.n, a.res != nullptr, rb);
  if (!rb || !a.pw || !a.y) return hipErrorInvalidValue;
  const long blocks = long(d.lanes) * t.tiles_y * t.tiles_x;
  if (blocks < 1 || blocks > 0x7fffffffL) return hipErrorInvalidValue;
  const size_t lds = size_t(dwpw_lds(d, a.n, t.tr, t.tw, 16 * rb, a.res != nullptr).total) * 4;
  const dim3 grid((unsigned)blocks);
  const int kind = d.kh * 100 + d.sw * 10 + rb;
#define PPOCR_DWPW(KK, SS, RR) \
  if (kind == KK * 100 + SS * 10 + RR) return go_dwpw<KK, SS, RR>(a, t, lds, grid, s);
  PPOCR_DWPW(3, 1, 4) PPOCR_DWPW(3, 1, 2) PPOCR_DWPW(3, 1, 1)
  PPOCR_DWPW(3, 2, 4) PPOCR_DWPW(3, 2, 2) PPOCR_DWPW(3, 2, 1)
  PPOCR_DWPW(5, 1, 4) PPOCR_DWPW(5, 1, 2) PPOCR_DWPW(5, 1, 1)
  PPOCR_DWPW(5, 2, 4) PPOCR_DWPW(5, 2, 2) PPOCR_DWPW(5, 2, 1)
#undef PPOCR_DWPW
  return hipErrorInvalidValue;
}

bool dw_mean_supported(const DwArgs &a) { return a.c % 4 == 0 && a.c <= 1024 && dw_fixed_kind(a) != 0; }

int dw_mean_blocks(const DwArgs &a) {
  const DwTile t = dw_tile_of(a, true);
  if (t.cg) return t.tiles_y * t.tiles_x;  // one partial row per spatial tile
  const int cv = a.c / 4, R = kDwMeanThreads / cv;
  const int runs = (a.ow + kDwRun - 1) / kDwRun;  // the run with the sums (dw_run)
  return (a.oh * runs + R - 1) / R;
}

template <bool MEAN, int DX, int TB>
static hipError_t launch_dw_fixed(int kind, dim3 grid, const DwArgs &a, hipStream_t s) {
  const dim3 block(MEAN ? TB : 256);
  switch (kind) {
    case 31: return launch_fixed(dwconv_fixed<3, 1, DX, MEAN, TB>, grid, block, a, s);
    case 32: return launch_fixed(dwconv_fixed<3, 2, DX, MEAN, TB>, grid, block, a, s);
    case 51: return launch_fixed(dwconv_fixed<5, 1, DX, MEAN, TB>, grid, block, a, s);
    case 52: return launch_fixed(dwconv_fixed<5, 2, DX, MEAN, TB>, grid, block, a, s);
    case 71: return launch_fixed(dwconv_fixed<7, 1, DX, MEAN, TB>, grid, block, a, s);
  }
  return hipErrorInvalidValue;
}

template <bool MEAN>
static hipError_t launch_dw_fixed(int kind, dim3 grid, const DwArgs &a, hipStream_t s) {
  if (MEAN) return launch_dw_fixed<true, kDwRun, kDwMeanThreads>(kind, grid, a, s);
  return dw_run(a) == 1 ? launch_dw_fixed<false, 1, 256>(kind, grid, a, s)
                        : launch_dw_fixed<false, kDwRun, 256>(kind, grid, a, s);
}

hipError_t launch_dwconv(const DwArgs &a, hipStream_t s) {
  const int DX = dw_run(a);
  auto aligned = [](const void *p) { return p == nullptr || (uintptr_t(p) & 15) == 0; };
  bool vec = a.c % 4 == 0 && aligned(a.x) && aligned(a.y) && aligned(a.w) && aligned(a.bias) &&
             a.x_lane_stride % 4 == 0 && a.y_lane_stride % 4 == 0;
  const DwTile t = dw_tile_of(a, a.mean_part != nullptr);
  if (vec && t.cg) return launch_dw_tile(a, t, s);
  const int kind = dw_fixed_kind(a);
  if (a.mean_part) {
    // With the channel sums: only the fixed variants, one grid row per lane.
    if (!vec || !dw_mean_supported(a) || a.lanes > 65535) return hipErrorInvalidValue;
    return launch_dw_fixed<true>(kind, dim3(dw_mean_blocks(a), a.lanes), a, s);
  }
  long runs = (a.ow + DX - 1) / DX;
  long total = (long)a.lanes * a.oh * runs * (vec ? a.c / 4 : a.c);
  dim3 grid(blocks_for(total, 256));
  if (vec && kind) return launch_dw_fixed<false>(kind, grid, a, s);
  if (vec && DX == 1)
    hipLaunchKernelGGL((dwconv_kernel<4, 1>), grid, dim3(256), 0, s, a);
  else if (vec)
    hipLaunchKernelGGL((dwconv_kernel<4, kDwRun>), grid, dim3(256), 0, s, a);
  else if (DX == 1)
    hipLaunchKernelGGL((dwconv_kernel<1, 1>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((dwconv_kernel<1, kDwRun>), grid, dim3(256), 0, s, a);
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
__global__ __launch_bounds__(256) void eltwise_kernel(Group<EltArgs> grp) {
  const int prob = group_problem(grp);
  const EltArgs &a = grp.a[prob];
  const long blk = (long)blockIdx.x - grp.first[prob], nblk = grp.first[prob + 1] - grp.first[prob];
  const long per = (long)a.oh * a.ow * a.c;
  const long nv = (long)a.lanes * per / V;
  for (long g = blk * blockDim.x + threadIdx.x; g < nv; g += nblk * blockDim.x) {
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

// The upsample-add chain, four channels a thread over the finest map: the
// thread forms its pixel's value at every level from the coarsest source
// down, in each level the operations of the separate upsample-add (the
// gated addend, then the upsampled value added, then the activation), and
// stores level k where its pixel is the top-left one of its 2^k x 2^k block
// (so each level's element is written once, with the bits its own launch
// would give).
template <int L>
__global__ __launch_bounds__(256) void upadd_chain_kernel(ChainArgs a) {
  const int cq = a.c / 4;
  const long per = (long)a.h[0] * a.w[0] * cq, total = per * a.lanes;
  const int top_w = a.w[L - 1] / 2;
  for (long e = (long)blockIdx.x * 256 + threadIdx.x; e < total; e += (long)gridDim.x * 256) {
    const int ln = (int)(e / per);
    const long r = e - (long)ln * per;
    const int q = (int)(r % cq);
    const long pix = r / cq;
    const int y = (int)(pix / a.w[0]), x = (int)(pix - (long)y * a.w[0]), ch = 4 * q;
    f32x4 v = *reinterpret_cast<const f32x4 *>(a.top + (long)ln * a.top_lane_stride +
                                              ((long)(y >> L) * top_w + (x >> L)) * a.c + ch);
    // Every level's addend and gate first, all in flight together (none is
    // a level's output; loaded after a level's store, each would wait for
    // it), the gates unconditionally (kDwZeros, never used, when a level
    // has none).
    f32x4 us[L], gs[L];
#pragma unroll
    for (int k = 0; k < L; k++) {
      const long o = ((long)(y >> k) * a.w[k] + (x >> k)) * a.c + ch;
      us[k] = *reinterpret_cast<const f32x4 *>(a.b[k] + (long)ln * a.b_lane_stride[k] + o);
      gs[k] = *reinterpret_cast<const f32x4 *>(a.g[k] ? a.g[k] + (long)ln * a.g_lane_stride[k] + ch : kDwZeros);
    }
#pragma unroll
    for (int k = L - 1; k >= 0; k--) {
      const long o = ((long)(y >> k) * a.w[k] + (x >> k)) * a.c + ch;
      f32x4 u = us[k];
      if (a.g[k]) {
        const f32x4 g = gs[k];
#pragma unroll
        for (int i = 0; i < 4; i++) u[i] = u[i] + u[i] * g[i];
      }
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = u[i] + v[i];
      if (a.act[k] != ACT_NONE) {
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = act(v[i], a.act[k]);
      }
      if (((y | x) & ((1 << k) - 1)) == 0)
        *reinterpret_cast<f32x4 *>(a.y[k] + (long)ln * a.y_lane_stride[k] + o) = v;
    }
  }
}

bool upadd_chain_supported(const ChainArgs &a) {
  if (a.levels < 2 || a.levels > kChainMax || a.c % 4 || a.lanes < 1) return false;
  auto a16 = [](const void *p) { return (uintptr_t(p) & 15) == 0; };
  if (!a16(a.top) || a.top_lane_stride % 4) return false;
  for (int k = 0; k < a.levels; k++) {
    if (a.h[k] < 1 || a.w[k] < 1 || a.h[k] % 2 || a.w[k] % 2) return false;
    if (k + 1 < a.levels && (a.h[k] != 2 * a.h[k + 1] || a.w[k] != 2 * a.w[k + 1])) return false;
    if (!a16(a.b[k]) || !a16(a.y[k]) || (a.g[k] && !a16(a.g[k]))) return false;
    if (a.b_lane_stride[k] % 4 || a.y_lane_stride[k] % 4 || (a.g[k] && a.g_lane_stride[k] % 4)) return false;
  }
  return true;
}

hipError_t launch_upadd_chain(const ChainArgs &a, hipStream_t s) {
  if (!upadd_chain_supported(a)) return hipErrorInvalidValue;
  const long total = (long)a.lanes * a.h[0] * a.w[0] * (a.c / 4);
  const unsigned blocks = (unsigned)std::min<long>((total + 255) / 256, 65536L * 4);
  if (a.levels == 2) hipLaunchKernelGGL(upadd_chain_kernel<2>, dim3(blocks), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(upadd_chain_kernel<3>, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError();
}

bool eltwise_vec(const EltArgs &a) {
  bool vec = a.c % 4 == 0 && (a.mode != ELT_CONCAT || (a.ca % 4 == 0 && a.cb % 4 == 0));
  // Flat modes need whole vectors inside each lane's tensor.
  if (a.mode == ELT_ADD || a.mode == ELT_MUL || a.mode == ELT_ACT)
    vec = ((long)a.oh * a.ow * a.c) % 4 == 0;
  auto a16 = [](const void *p) { return p == nullptr || (uintptr_t(p) & 15) == 0; };
  if (!a16(a.a) || !a16(a.b) || !a16(a.g) || !a16(a.y)) vec = false;
  if (vec && (a.a_lane_stride % 4 || a.b_lane_stride % 4 || a.y_lane_stride % 4)) vec = false;
  return vec;
}

hipError_t launch_eltwise_group(const EltArgs *as, int n, hipStream_t s) {
  if (n < 1 || n > kGroupMax) return hipErrorInvalidValue;
  const bool vec = eltwise_vec(as[0]);
  Group<EltArgs> grp{};
  grp.n = n;
  long blocks = 0;
  for (int p = 0; p < n; p++) {
    if (eltwise_vec(as[p]) != vec) return hipErrorInvalidValue;
    const long e = (long)as[p].lanes * as[p].oh * as[p].ow * as[p].c;
    long b = blocks_for(vec ? e / 4 : e, 256);
    if (b > 65536L * 4) b = 65536L * 4;
    grp.first[p] = (int)blocks;
    blocks += b;
    grp.a[p] = as[p];
  }
  grp.first[n] = (int)blocks;
  if (vec) hipLaunchKernelGGL(eltwise_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, s, grp);
  else hipLaunchKernelGGL(eltwise_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, s, grp);
  return hipGetLastError();
}

hipError_t launch_eltwise(const EltArgs &a, hipStream_t s) { return launch_eltwise_group(&a, 1, s); }

// ------------------------------------------------------------ pooling

// Max: the window cut at the bottom and right edges, seeded with its first
// tap, each later tap kept only when greater (src/engine/conv.rs:404-440).
// Average: whole windows, taps summed from zero in row-major order, then
// divided (src/engine/layers.rs:443-463).
template <int V>
__global__ __launch_bounds__(256) void pool_kernel(PoolArgs a) {
  const int cv = a.c / V;
  long per = (long)a.oh * a.ow * cv;
  // Blocks numbered XCD by XCD (xcd_tile): neighbouring output rows, which
  // read the same input rows, meet in one L2.
  long g = (long)xcd_tile((int)blockIdx.x, (int)gridDim.x) * blockDim.x + threadIdx.x;
  if (g >= (long)a.lanes * per) return;
  int ln = (int)(g / per);
  long off = g - (long)ln * per;
  int ch = (int)(off % cv) * V;
  long pix = off / cv;
  int oy = (int)(pix / a.ow), ox = (int)(pix - (long)oy * a.ow);
  const float *x = a.x + (long)ln * a.x_lane_stride;
  float accv[V];
#pragma unroll
  for (int k = 0; k < V; k++) accv[k] = 0.0f;
  bool seeded = false;
  for (int ky = 0; ky < a.kh; ky++) {
    int iy = oy * a.sh + ky;
    if (iy >= a.ih) continue;
    for (int kx = 0; kx < a.kw; kx++) {
      int ix = ox * a.sw + kx;
      if (ix >= a.iw) continue;
      float v[V];
      vload<V>(v, x + ((long)iy * a.iw + ix) * a.c + ch);
#pragma unroll
      for (int k = 0; k < V; k++) {
        if (a.avg) {
          accv[k] = accv[k] + v[k];
        } else if (!seeded || v[k] > accv[k]) {
          accv[k] = v[k];
        }
      }
      seeded = true;
    }
  }
  if (a.avg) {
#pragma unroll
    for (int k = 0; k < V; k++) accv[k] = accv[k] / (float)(a.kh * a.kw);
  }
  vstore<V>(a.y + (long)ln * a.y_lane_stride + pix * a.c + ch, accv);
}

hipError_t launch_pool(const PoolArgs &a, hipStream_t s) {
  const bool v4 = a.c % 4 == 0 && a.x_lane_stride % 4 == 0 && a.y_lane_stride % 4 == 0 &&
                  (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
  long n = (long)a.lanes * a.oh * a.ow * (v4 ? a.c / 4 : a.c);
  if (v4)
    hipLaunchKernelGGL(pool_kernel<4>, dim3(blocks_for(n, 256)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(pool_kernel<1>, dim3(blocks_for(n, 256)), dim3(256), 0, s, a);
  return hipGetLastError();
}

// ------------------------------------------------------------ mean and SE

// One launch per channel mean (up to kGroupMax of them in one grid):
//
//  1. Sum: with an input x, workgroup (lane, chunk k, slice s) sums a run of
//     pixels of the slice's 32 channels in f64, each thread a fixed stride of
//     pixels, joined in LDS in thread order. With one chunk per lane that is
//     the whole sum; else it is stored as the chunk's partial row and the
//     workgroup counts itself in on the slice's counter.
//  2. Join: the last workgroup of a slice to count in (or, when a depthwise
//     convolution wrote the partial rows, every workgroup: one per slice)
//     adds the lane's partial rows of its channels, row by row in a fixed
//     split over the threads, joined in thread order, and divides by the
//     pixels. Which workgroup is last does not change the order, so the
//     result is the same on every run.
//  3. SE: the last slice of a lane to count in runs both 1x1 layers of the
//     squeeze-and-excite on the lane's means, each output from zero, inputs
//     in order, fused multiply-adds for outputs below outputs / 8 * 8 and a
//     separate product and sum past them, then the bias, then the activation
//     (the engine's one-pixel 1x1 rule, src/engine/kernels/pointwise.rs:
//     135-185), each thread streaming its outputs' weights from global
//     memory into registers, many loads in flight.
//
// Counters go back to zero as soon as the last workgroup has read them, so
// the next launch (or graph replay) finds them cleared. What workgroups hand
// each other within the launch (partial rows, means) is stored and loaded as
// device-scope atomics, which stay coherent across the XCDs' L2s; a
// workgroup waits for its stores to complete before it counts in. (An
// agent-scope fence instead writes the whole L2 back, and those writebacks
// queue up: measured about 75 ns a workgroup.)
//
// The mean divides an f64 sum by the pixel count and rounds once to f32, as
// the engine does (src/engine/layers.rs:391-406); the f64 sum runs in
// another order.

constexpr int kMeanSlice = 32;    // channels a summing workgroup covers
constexpr int kMeanStrides = 8;   // loads in flight per thread while summing
constexpr int kMeanMaxChunks = 64;
// LDS floats for a layer's m inputs: read 64 at a time, one iteration
// (up to 128 inputs) ahead, so up to 255 past the last (never used).
__host__ __device__ inline int se_in_floats(int m) { return ((m + 127) & ~127) + 128; }

// One 1x1 layer over one pixel: out_j = act(sum_i in_i * w[i][j] + bias_j)
// for j < n, inputs `in` (m floats in LDS, readable as se_in_floats says).
// The weights are packed in groups of four inputs, each output's four
// weights together: w[((i / 4) * n + j) * 4 + i % 4], zero past m. Each
// thread keeps NO outputs' sums (j = t + 256 o) and loads its outputs'
// weights, a 16-byte group at a time, from global memory straight into a
// rotating queue of QD groups in registers: the loads of a wave complete in
// the order they were issued, so each group's multiply-adds wait for that
// group alone while the next QD - 1 are in flight. `pre` runs after the
// first QD loads have gone out (in every wave, those without outputs too,
// which then return): the caller's wait for the layer's inputs overlaps
// their latency. The inputs come from LDS 64 to a register and are
// broadcast one at a time (readlane). Every sum runs from zero over the
// inputs in order; FUSED: every output is below n / 8 * 8 (the engine's
// fused columns); else each output picks fused or separate product and
// sum. Outputs go to `out` (LDS or global memory).
template <int NO, bool FUSED, typename Pre>
__device__ __forceinline__ void se_layer_n(const float *w, const float *bias, int m, int n, int code,
                                           const float *in, float *out, Pre pre) {
  // Groups in flight: 32 registers of weights. Queues of 16 / NO and
  // 32 / NO groups measured slower on the SEs of both networks: their
  // registers cost the summing workgroups occupancy (the kernel's register
  // count is the deepest queue's), and the layers' own loads gained nothing
  // from the depth.
  constexpr int QD = 8 / NO;
  constexpr int IT = QD > 16 ? QD : 16;   // groups per iteration, a multiple of QD and of 16
  constexpr int XR = IT / 16;             // input registers per iteration
  const int t = threadIdx.x, lane = t & 63;
  if (__builtin_amdgcn_readfirstlane(t >> 6) * 64 >= n) {
    pre();
    return;
  }
  const int groups = (m + 3) / 4, fused_end = n / 8 * 8;
  const f32x4 *wv = reinterpret_cast<const f32x4 *>(w);
  bool has[NO], fz[NO];
  int col[NO];
#pragma unroll
  for (int o = 0; o < NO; o++) {
    const int j = t + 256 * o;
    has[o] = j < n, fz[o] = j < fused_end, col[o] = j < n ? j : n - 1;
  }
  float acc[NO];
#pragma unroll
  for (int o = 0; o < NO; o++) acc[o] = 0.0f;
  // Queue slot s holds group g with g % QD == s; past the last group the
  // loads repeat the last one (never used).
  f32x4 q[QD][NO];
#pragma unroll
  for (int s = 0; s < QD; s++) {
    const f32x4 *row = wv + (long)min(s, groups - 1) * n;
#pragma unroll
    for (int o = 0; o < NO; o++) q[s][o] = row[col[o]];
  }
  pre();
  float xr[XR];
#pragma unroll
  for (int k = 0; k < XR; k++) xr[k] = in[64 * k + lane];
  auto iteration = [&](int g0, auto tail_c) {
    constexpr bool TAIL = decltype(tail_c)::value;
    float xn[XR];  // the next iteration's inputs
#pragma unroll
    for (int k = 0; k < XR; k++) xn[k] = in[4 * (g0 + IT) + 64 * k + lane];
#pragma unroll
    for (int s = 0; s < IT; s++) {
      const int slot = s % QD;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        if (TAIL && 4 * (g0 + s) + e >= m) continue;
        const float x = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xr[s / 16]), (4 * s + e) & 63));
#pragma unroll
        for (int o = 0; o < NO; o++) {
          const float wgt = q[slot][o][e];
          acc[o] = FUSED || fz[o] ? fmaf(wgt, x, acc[o]) : acc[o] + x * wgt;
        }
      }
      const f32x4 *row = wv + (long)min(g0 + s + QD, groups - 1) * n;
#pragma unroll
      for (int o = 0; o < NO; o++) q[slot][o] = row[col[o]];
    }
#pragma unroll
    for (int k = 0; k < XR; k++) xr[k] = xn[k];
  };
  const int full = m / (4 * IT);  // iterations whose inputs are all below m
  for (int it = 0; it < full; it++) iteration(it * IT, std::false_type{});
  if (4 * IT * full < m) iteration(full * IT, std::true_type{});
#pragma unroll
  for (int o = 0; o < NO; o++) {
    if (has[o]) {
      float v = acc[o];
      if (bias) v = v + bias[t + 256 * o];
      out[t + 256 * o] = act(v, code);
    }
  }
}

template <typename Pre>
__device__ __forceinline__ void se_layer(const float *w, const float *bias, int m, int n, int code,
                                         const float *in, float *out, Pre pre) {
  const bool fused = n % 8 == 0;
  if (n <= 256) {
    if (fused) se_layer_n<1, true>(w, bias, m, n, code, in, out, pre);
    else se_layer_n<1, false>(w, bias, m, n, code, in, out, pre);
  } else if (n <= 512) {
    if (fused) se_layer_n<2, true>(w, bias, m, n, code, in, out, pre);
    else se_layer_n<2, false>(w, bias, m, n, code, in, out, pre);
  } else {
    if (fused) se_layer_n<4, true>(w, bias, m, n, code, in, out, pre);
    else se_layer_n<4, false>(w, bias, m, n, code, in, out, pre);
  }
}

// Whether this workgroup is the last of `of` to count in on `*cnt` (then the
// counter is zero again). What the workgroups exchange within a launch is
// stored and loaded as device-scope atomics (coherent across the XCDs'
// L2s without writing the L2s back), so waiting for this workgroup's stores
// to complete before the count is enough for the last one to see them all.
__device__ __forceinline__ bool count_in(int *cnt, int of, int *flag) {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int last = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == of - 1;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  return *flag != 0;
}

template <typename T>
__device__ __forceinline__ void put_shared(T *p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T get_shared(const T *p) {
  return __hip_atomic_load(const_cast<T *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// SE: some job of the group has a squeeze-and-excite (the layers' register
// queues are compiled in only then).
template <int V, bool SE>
__global__ __launch_bounds__(256) void mean_se(Group<MeanJob> grp) {
  extern __shared__ __attribute__((aligned(16))) float dyn[];
  __shared__ double red[256 * V];
  __shared__ int flag;
  const int prob = group_problem(grp);
  const MeanJob &j = grp.a[prob];
  const int cs = grp.x[prob], S = grp.y[prob];
  const int c = j.c, P = j.chunks, t = threadIdx.x;
  const int K = j.x ? P : 1;
  const int blk = (int)blockIdx.x - grp.first[prob];
  const int per_lane = S * K;
  const int ln = blk / per_lane, r = blk - ln * per_lane;
  const int k = r / S, s = r - k * S;
  const int c0 = s * cs, cw = min(cs, c - c0);
  const MeanShape sh = mean_shape(j.x != nullptr, j.pixels, c, j.lanes, j.x ? 0 : P, j.has_se != 0);
  double *pl = reinterpret_cast<double *>(j.work) + (long)ln * P * c;
  int *cnt = j.count;  // [lanes] for the SE, then [lanes][S] for the slices
  double tot = 0.0;  // threads below cw: the channel's sum
  bool join = true;
  if (j.x) {
    const int chunk = (j.pixels + K - 1) / K;
    const int p0 = k * chunk, p1 = min(p0 + chunk, j.pixels);
    const float *xl = j.x + (long)ln * j.x_lane_stride;
    if constexpr (V == 4) {
      constexpr int NQ = kMeanSlice / 4, R = 256 / NQ;
      const int q = t % NQ, rr = t / NQ, ch = c0 + 4 * q;
      double a0 = 0.0, a1 = 0.0, a2 = 0.0, a3 = 0.0;
      if (4 * q < cw) {
        // kMeanStrides loads in flight; past the chunk they read zeros.
        for (int p = p0 + rr; p < p1; p += kMeanStrides * R) {
          f32x4 v[kMeanStrides];
#pragma unroll
          for (int u = 0; u < kMeanStrides; u++)
            v[u] = p + u * R < p1 ? *reinterpret_cast<const f32x4 *>(xl + (long)(p + u * R) * c + ch)
                                  : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int u = 0; u < kMeanStrides; u++) a0 += (double)v[u].x, a1 += (double)v[u].y, a2 += (double)v[u].z, a3 += (double)v[u].w;
        }
      }
      red[4 * t] = a0, red[4 * t + 1] = a1, red[4 * t + 2] = a2, red[4 * t + 3] = a3;
      __syncthreads();
      if (t < cw)
        for (int x = 0; x < R; x++) tot += red[(x * NQ + t / 4) * 4 + (t & 3)];
    } else {
      constexpr int R = 256 / kMeanSlice;
      const int cl = t % kMeanSlice, rr = t / kMeanSlice;
      double a = 0.0;
      if (cl < cw) {
        for (int p = p0 + rr; p < p1; p += kMeanStrides * R) {
          float v[kMeanStrides];
#pragma unroll
          for (int u = 0; u < kMeanStrides; u++) v[u] = p + u * R < p1 ? xl[(long)(p + u * R) * c + c0 + cl] : 0.0f;
#pragma unroll
          for (int u = 0; u < kMeanStrides; u++) a += (double)v[u];
        }
      }
      red[t] = a;
      __syncthreads();
      if (t < cw)
        for (int x = 0; x < R; x++) tot += red[x * kMeanSlice + t];
    }
    if (K == 1) {
      join = false;
    } else {
      if (t < cw) put_shared(pl + (long)k * c + c0 + t, tot);
      if (!count_in(cnt + j.lanes + ln * S + s, K, &flag)) return;
    }
  }
  if (join) {
    // Rows another workgroup of this launch wrote are read as device-scope
    // atomics; a depthwise convolution's rows come from the launch before.
    const int J = 256 / cs, cl = t % cs, jj = t / cs;
    double a = 0.0;
    if (cl < cw) {
      const double *p = pl + c0 + cl;
      for (int rr = jj; rr < P; rr += 16 * J) {
        double v[16];
        if (j.x) {
#pragma unroll
          for (int u = 0; u < 16; u++) v[u] = rr + u * J < P ? get_shared(p + (long)(rr + u * J) * c) : 0.0;
        } else {
#pragma unroll
          for (int u = 0; u < 16; u++) v[u] = rr + u * J < P ? p[(long)(rr + u * J) * c] : 0.0;
        }
#pragma unroll
        for (int u = 0; u < 16; u++) a += v[u];
      }
    }
    __syncthreads();  // the sum phase's join may still read red
    red[t] = a;
    __syncthreads();
    tot = 0.0;
    if (t < cw)
      for (int x = 0; x < J; x++) tot += red[x * cs + t];
  }
  const float mean = (float)(tot / (double)j.pixels);
  float *yl = j.y + (long)ln * j.y_lane_stride;
  if (!SE || !j.has_se) {
    if (t < cw) yl[c0 + t] = mean;
    return;
  }
  // The layers read their inputs sixteen at a time: room for 16 past each.
  float *in = dyn;                                   // c floats
  float *hid = dyn + se_in_floats(c);                // mid floats
  const float *means = nullptr;
  if (S > 1) {
    float *mw = j.work + sh.means_off + (long)ln * c;
    if (t < cw) put_shared(mw + c0 + t, mean);
    if (!count_in(cnt + ln, S, &flag)) return;
    means = mw;
  } else if (t < cw) {
    in[t] = mean;
  }
  if constexpr (SE) {
    const SeArgs &se = j.se;
    // Each layer's first weights go out before the wait for its inputs: the
    // lane's means (read from the other workgroups' stores, their loads
    // issued first so that the wait covers them alone), then the first
    // layer's outputs (published by the barrier).
    float mv[4];  // c <= 1024
    if (means) {
#pragma unroll
      for (int k = 0; k < 4; k++) mv[k] = t + 256 * k < c ? get_shared(means + t + 256 * k) : 0.0f;
    }
    se_layer(se.w1, se.b1, c, se.mid, se.act1, in, hid, [&] {
      if (means) {
#pragma unroll
        for (int k = 0; k < 4; k++)
          if (t + 256 * k < c) in[t + 256 * k] = mv[k];
      }
      __syncthreads();
    });
    se_layer(se.w2, se.b2, se.mid, se.cout, se.act2, hid, yl, [] { __syncthreads(); });
  }
}

__host__ __device__ MeanShape mean_shape(bool has_x, int pixels, int c, int lanes, int dw_rows, bool has_se) {
  MeanShape m{};
  if (has_x) {
    m.cs = kMeanSlice;
    int k = (pixels + 255) / 256;
    m.k = k < 1 ? 1 : (k > kMeanMaxChunks ? kMeanMaxChunks : k);
  } else {
    // Join slices when the partial rows come from a depthwise convolution:
    // the widest whose rows leave each thread at most sixteen loads.
    int cs = 4;
    for (int w = 32; w >= 8; w /= 2)
      if ((dw_rows + 256 / w - 1) / (256 / w) <= 16) {
        cs = w;
        break;
      }
    m.cs = cs;
    m.k = 1;
  }
  m.S = (c + m.cs - 1) / m.cs;
  const size_t rows = has_x ? (m.k > 1 ? size_t(m.k) : 0) : size_t(dw_rows);
  m.means_off = 2 * size_t(lanes) * rows * size_t(c);
  m.floats = m.means_off + (has_se && m.S > 1 ? size_t(lanes) * c : 0);
  // Counters: [lanes] for the SE, then [lanes][S] for the slices.
  m.count_n = has_x && m.k > 1 ? size_t(lanes) * (1 + m.S) : (has_se ? size_t(lanes) : 0);
  return m;
}

bool se_supported(int c, int mid, int cout) {
  return c >= 1 && mid >= 1 && cout >= 1 && c <= 1024 && mid <= 1024 && cout <= 1024;
}

hipError_t launch_mean_group(const MeanJob *jobs, int n, hipStream_t s) {
  if (n < 1 || n > kGroupMax) return hipErrorInvalidValue;
  Group<MeanJob> g{};
  long blocks = 0;
  size_t shm = 0;
  bool vec = true, any_se = false;
  for (int p = 0; p < n; p++) {
    const MeanJob &j = jobs[p];
    any_se = any_se || j.has_se;
    if (j.lanes < 1 || j.c < 1 || j.pixels < 1 || !j.work || !j.y) return hipErrorInvalidValue;
    if (!j.x && j.chunks < 1) return hipErrorInvalidValue;
    if ((reinterpret_cast<uintptr_t>(j.work) & 15) != 0) return hipErrorInvalidValue;
    const MeanShape m = mean_shape(j.x != nullptr, j.pixels, j.c, j.lanes, j.x ? 0 : j.chunks, j.has_se != 0);
    if (m.count_n && !j.count) return hipErrorInvalidValue;
    MeanJob jj = j;
    if (j.x) {
      jj.chunks = m.k;
      vec = vec && j.c % 4 == 0 && (reinterpret_cast<uintptr_t>(j.x) & 15) == 0 && j.x_lane_stride % 4 == 0;
    }
    if (j.has_se) {
      const SeArgs &se = j.se;
      if (!se.w1 || !se.w2 || !se_supported(j.c, se.mid, se.cout)) return hipErrorInvalidValue;
      if (((reinterpret_cast<uintptr_t>(se.w1) | reinterpret_cast<uintptr_t>(se.w2)) & 15) != 0)
        return hipErrorInvalidValue;
      const size_t in = size_t(se_in_floats(j.c)) + size_t(se_in_floats(se.mid));
      shm = std::max(shm, in * sizeof(float));
    }
    g.first[p] = (int)blocks;
    g.x[p] = m.cs;
    g.y[p] = m.S;
    g.a[p] = jj;
    blocks += long(j.lanes) * m.S * m.k;
    if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
  }
  g.n = n;
  g.first[n] = (int)blocks;
  const dim3 grid((unsigned)blocks);
  if (vec && any_se)
    hipLaunchKernelGGL((mean_se<4, true>), grid, dim3(256), shm, s, g);
  else if (vec)
    hipLaunchKernelGGL((mean_se<4, false>), grid, dim3(256), shm, s, g);
  else if (any_se)
    hipLaunchKernelGGL((mean_se<1, true>), grid, dim3(256), shm, s, g);
  else
    hipLaunchKernelGGL((mean_se<1, false>), grid, dim3(256), shm, s, g);
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

// Blocks of 256 threads over kLnRows rows: first one thread per row with the
// row in registers (MAXV float4s: the loads of a row are independent and all
// in flight at once) runs the two sums in sequence as the CPU's do and keeps
// the row's mean and root in LDS; then the whole block writes the outputs,
// four values a thread at a time, each (x - mean) / root * gamma + beta.
constexpr int kLnRows = 16;

template <int MAXV>
__global__ __launch_bounds__(256) void layernorm_rows(const float *x, long x_lane_stride,
                                                     const float *w, int rows, int c, int lanes,
                                                     float *y, long y_lane_stride) {
  __shared__ float stat[2 * kLnRows];
  const long total = (long)rows * lanes;
  const long r0 = (long)blockIdx.x * kLnRows;
  const int nv = c / 4, tid = threadIdx.x;
  auto row_ptr = [&](long row, const float *base, long stride) {
    const int ln = (int)(row / rows);
    return base + (long)ln * stride + (row - (long)ln * rows) * c;
  };
  if (tid < kLnRows && r0 + tid < total) {
    const f32x4 *xr = reinterpret_cast<const f32x4 *>(row_ptr(r0 + tid, x, x_lane_stride));
    f32x4 v[MAXV];
#pragma unroll
    for (int k = 0; k < MAXV; k++)
      if (k < nv) v[k] = xr[k];
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXV; k++)
      if (k < nv) s = (((s + v[k].x) + v[k].y) + v[k].z) + v[k].w;
    const float mean = s / (float)c;
    float q = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXV; k++) {
      if (k < nv) {
        float d0 = v[k].x - mean, d1 = v[k].y - mean, d2 = v[k].z - mean, d3 = v[k].w - mean;
        q = q + d0 * d0;
        q = q + d1 * d1;
        q = q + d2 * d2;
        q = q + d3 * d3;
      }
    }
    stat[2 * tid] = mean;
    stat[2 * tid + 1] = sqrtf(q / (float)c + w[2 * c]);
  }
  __syncthreads();
  const f32x4 *g4 = reinterpret_cast<const f32x4 *>(w);
  const f32x4 *b4 = reinterpret_cast<const f32x4 *>(w + c);
  for (int e = tid; e < kLnRows * nv; e += 256) {
    const int rr = e / nv, k = e - rr * nv;
    if (r0 + rr >= total) break;
    const f32x4 xv = reinterpret_cast<const f32x4 *>(row_ptr(r0 + rr, x, x_lane_stride))[k];
    const float mean = stat[2 * rr], r = stat[2 * rr + 1];
    const f32x4 g = g4[k], bb = b4[k];
    f32x4 o;
    o.x = (xv.x - mean) / r * g.x + bb.x;
    o.y = (xv.y - mean) / r * g.y + bb.y;
    o.z = (xv.z - mean) / r * g.z + bb.z;
    o.w = (xv.w - mean) / r * g.w + bb.w;
    reinterpret_cast<f32x4 *>(const_cast<float *>(row_ptr(r0 + rr, y, y_lane_stride)))[k] = o;
  }
}

hipError_t launch_layernorm(const float *x, long x_lane_stride, const float *w, int rows, int c,
                            int lanes, float *y, long y_lane_stride, hipStream_t s) {
  long total = (long)rows * lanes;
  auto a16 = [](const void *p) { return (uintptr_t(p) & 15) == 0; };
  if (c % 4 == 0 && c <= 128 && a16(x) && a16(y) && a16(w) && a16(w + c) &&
      x_lane_stride % 4 == 0 && y_lane_stride % 4 == 0) {
    hipLaunchKernelGGL(layernorm_rows<32>, dim3(blocks_for(total, kLnRows)), dim3(256), 0, s, x,
                       x_lane_stride, w, rows, c, lanes, y, y_lane_stride);
    return hipGetLastError();
  }
  size_t shm = (size_t)64 * (c + 1) * sizeof(float);
  if (shm > 64 * 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(layernorm_kernel, dim3(blocks_for(total, 64)), dim3(64), shm, s, x,
                     x_lane_stride, w, rows, c, lanes, y, y_lane_stride);
  return hipGetLastError();
}

// ------------------------------------------------------------ attention

// One block of 256 threads per (lane, head), in three phases that keep the
// engine's order for every value (src/engine/layers.rs:494-522, 273-294):
//  1. each score from zero, a fused multiply-add per head dimension against
//     the pre-scaled query; threads take (query, key) pairs;
//  2. softmax per row in 8 lanes: thread (row, l) keeps lane l (keys j with
//     j % 8 == l below the last whole group of 8); the row's maximum and sum
//     then join the lanes in order, the tail one key at a time;
//  3. each output from zero, a fused multiply-add per key in order against
//     the rounded probability; threads take (query, dimension) pairs.
// Q, K and V of the head sit in LDS; the t x t scores too, or for long lines
// in global scratch.
template <int HDV, int NT>
__global__ __launch_bounds__(NT) void attention_kernel(const float *x, long x_lane_stride,
                                                      float scale, int t, int c, int heads,
                                                      float *y, long y_lane_stride,
                                                      float *gscores) {
  extern __shared__ float sm[];
  const int hd = c / heads;
  const int ln = blockIdx.x / heads, h = blockIdx.x % heads;
  const int tid = threadIdx.x, nt = blockDim.x;
  const int ts = t + 1;  // score row stride
  float *qs = sm;                  // t * hd, pre-scaled
  float *ks = qs + t * hd;         // t * hd
  float *vs = ks + t * hd;         // t * hd
  float *lane_max = vs + t * hd;   // t * 8
  float *lane_sum = lane_max + t * 8;  // t * 8
  float *rinv = lane_sum + t * 8;      // t: row maximum, then 1 / sum
  float *rmax = rinv + t;              // t
  float *sc = gscores ? gscores + (long)blockIdx.x * t * ts : rmax + t;
  const float *xl = x + (long)ln * x_lane_stride;
  for (int e = tid; e < t * hd; e += nt) {
    int j = e / hd, d = e - j * hd;
    const float *px = xl + (long)j * 3 * c + h * hd + d;
    qs[e] = px[0] * scale;
    ks[e] = px[c];
    vs[e] = px[2 * c];
  }
  __syncthreads();
  const int fused = t / 8 * 8;  // keys past it multiply and add separately
  for (int e = tid; e < t * t; e += nt) {
    int s = e / t, j = e - s * t;
    const float *q = qs + s * hd, *k = ks + j * hd;
    float qv[HDV], kv[HDV];
#pragma unroll
    for (int d = 0; d < HDV; d++) {
      qv[d] = d < hd ? q[d] : 0.0f;
      kv[d] = d < hd ? k[d] : 0.0f;
    }
    float acc = 0.0f;
    if (j < fused) {
#pragma unroll
      for (int d = 0; d < HDV; d++)
        if (d < hd) acc = fmaf(kv[d], qv[d], acc);
    } else {
#pragma unroll
      for (int d = 0; d < HDV; d++)
        if (d < hd) acc = acc + qv[d] * kv[d];
    }
    sc[s * ts + j] = acc;
  }
  __syncthreads();
  const int body = t / 8 * 8;
  const float ninf = -__builtin_inff();
  for (int e = tid; e < t * 8; e += nt) {
    int s = e >> 3, l = e & 7;
    const float *row = sc + s * ts;
    float m = ninf;
    for (int j = l; j < body; j += 8) m = row[j] > m ? row[j] : m;
    lane_max[e] = m;
  }
  __syncthreads();
  for (int s = tid; s < t; s += nt) {
    const float *row = sc + s * ts;
    float m = ninf;
    for (int l = 0; l < 8; l++) m = fmaxf(m, lane_max[s * 8 + l]);
    for (int j = body; j < t; j++) m = fmaxf(m, row[j]);
    rmax[s] = m;
  }
  __syncthreads();
  for (int e = tid; e < t * 8; e += nt) {
    int s = e >> 3, l = e & 7;
    float *row = sc + s * ts;
    const float m = rmax[s];
    float sum = 0.0f;
    for (int j = l; j < body; j += 8) {
      float ex = exp_neg(row[j] - m);
      row[j] = ex;
      sum = sum + ex;
    }
    lane_sum[e] = sum;
  }
  __syncthreads();
  for (int s = tid; s < t; s += nt) {
    float *row = sc + s * ts;
    const float m = rmax[s];
    float sum = 0.0f;
    for (int l = 0; l < 8; l++) sum = sum + lane_sum[s * 8 + l];
    for (int j = body; j < t; j++) {
      float ex = exp_neg(row[j] - m);
      row[j] = ex;
      sum = sum + ex;
    }
    rinv[s] = 1.0f / sum;
  }
  __syncthreads();
  for (int e = tid; e < t * t; e += nt) {
    int s = e / t, j = e - s * t;
    sc[s * ts + j] = sc[s * ts + j] * rinv[s];
  }
  __syncthreads();
  float *yl = y + (long)ln * y_lane_stride + h * hd;
  for (int e = tid; e < t * hd; e += nt) {
    int s = e / hd, d = e - s * hd;
    const float *p = sc + s * ts;
    const float *v = vs + d;
    float acc = 0.0f;
    int j = 0;
    for (; j + 8 <= t; j += 8) {
      float vv[8], pp[8];
#pragma unroll
      for (int u = 0; u < 8; u++) vv[u] = v[(j + u) * hd], pp[u] = p[j + u];
#pragma unroll
      for (int u = 0; u < 8; u++) acc = fmaf(vv[u], pp[u], acc);
    }
    for (; j < t; j++) acc = fmaf(v[j * hd], p[j], acc);
    yl[(long)s * c + d] = acc;
  }
}

// The same three phases for a run of TQ query rows of one (lane, head):
// blocks of 256 threads over (lane, head, run), so that a batch of short
// lines still fills the GPU. K and V of the head (every row), the run's
// pre-scaled queries and its scores sit in LDS with rows padded to HDV
// floats, read as float4: a score's query and key rows as HDV / 4 vector
// reads, an output thread's four dimensions of V per key as one. Every
// value keeps the order above (the products and sums of a score over
// d < hd only, each output's keys in order).
template <int HDV>
__global__ __launch_bounds__(256) void attention_rows(const float *x, long x_lane_stride, float scale, int t,
                                                      int c, int heads, int runs, float *y, long y_lane_stride) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int hd = c / heads;
  const int tq = (t + runs - 1) / runs;
  const int blk = blockIdx.x;
  const int run = blk % runs, lh = blk / runs;
  const int ln = lh / heads, h = lh % heads;
  const int q0 = run * tq, nq = min(tq, t - q0);
  if (nq <= 0) return;
  const int tid = threadIdx.x, ts = t + 1;
  float *ks = sm;                      // t x HDV
  float *vs = ks + t * HDV;            // t x HDV
  float *qs = vs + t * HDV;            // tq x HDV, pre-scaled
  float *sc = qs + tq * HDV;           // tq x ts
  float *lane_max = sc + tq * ts;      // tq x 8
  float *lane_sum = lane_max + tq * 8; // tq x 8
  float *rmax = lane_sum + tq * 8;     // tq
  float *rinv = rmax + tq;             // tq
  const float *xl = x + (long)ln * x_lane_stride + h * hd;
  for (int e = tid; e < t * HDV; e += 256) {
    const int j = e / HDV, d = e - j * HDV;
    const float *px = xl + (long)j * 3 * c + d;
    ks[e] = d < hd ? px[c] : 0.0f;
    vs[e] = d < hd ? px[2 * c] : 0.0f;
  }
  for (int e = tid; e < nq * HDV; e += 256) {
    const int s = e / HDV, d = e - s * HDV;
    qs[e] = d < hd ? xl[(long)(q0 + s) * 3 * c + d] * scale : 0.0f;
  }
  __syncthreads();
  const int fused = t / 8 * 8;  // keys past it multiply and add separately
  for (int e = tid; e < nq * t; e += 256) {
    const int s = e / t, j = e - s * t;
    f32x4 qv[HDV / 4], kv[HDV / 4];
#pragma unroll
    for (int u = 0; u < HDV / 4; u++) {
      qv[u] = *reinterpret_cast<const f32x4 *>(qs + s * HDV + 4 * u);
      kv[u] = *reinterpret_cast<const f32x4 *>(ks + j * HDV + 4 * u);
    }
    float acc = 0.0f;
    if (j < fused) {
#pragma unroll
      for (int d = 0; d < HDV; d++)
        if (d < hd) acc = fmaf(kv[d / 4][d % 4], qv[d / 4][d % 4], acc);
    } else {
#pragma unroll
      for (int d = 0; d < HDV; d++)
        if (d < hd) acc = acc + qv[d / 4][d % 4] * kv[d / 4][d % 4];
    }
    sc[s * ts + j] = acc;
  }
  __syncthreads();
  const int body = t / 8 * 8;
  const float ninf = -__builtin_inff();
  for (int e = tid; e < nq * 8; e += 256) {
    const int s = e >> 3, l = e & 7;
    const float *row = sc + s * ts;
    float m = ninf;
    for (int j = l; j < body; j += 8) m = row[j] > m ? row[j] : m;
    lane_max[e] = m;
  }
  __syncthreads();
  for (int s = tid; s < nq; s += 256) {
    const float *row = sc + s * ts;
    float m = ninf;
    for (int l = 0; l < 8; l++) m = fmaxf(m, lane_max[s * 8 + l]);
    for (int j = body; j < t; j++) m = fmaxf(m, row[j]);
    rmax[s] = m;
  }
  __syncthreads();
  for (int e = tid; e < nq * 8; e += 256) {
    const int s = e >> 3, l = e & 7;
    float *row = sc + s * ts;
    const float m = rmax[s];
    float sum = 0.0f;
    for (int j = l; j < body; j += 8) {
      const float ex = exp_neg(row[j] - m);
      row[j] = ex;
      sum = sum + ex;
    }
    lane_sum[e] = sum;
  }
  __syncthreads();
  for (int s = tid; s < nq; s += 256) {
    float *row = sc + s * ts;
    const float m = rmax[s];
    float sum = 0.0f;
    for (int l = 0; l < 8; l++) sum = sum + lane_sum[s * 8 + l];
    for (int j = body; j < t; j++) {
      const float ex = exp_neg(row[j] - m);
      row[j] = ex;
      sum = sum + ex;
    }
    rinv[s] = 1.0f / sum;
  }
  __syncthreads();
  for (int e = tid; e < nq * t; e += 256) {
    const int s = e / t, j = e - s * t;
    sc[s * ts + j] = sc[s * ts + j] * rinv[s];
  }
  __syncthreads();
  float *yl = y + (long)ln * y_lane_stride + h * hd;
  for (int e = tid; e < nq * (HDV / 4); e += 256) {
    const int s = e / (HDV / 4), d4 = e - s * (HDV / 4);
    const float *p = sc + s * ts;
    const float *v = vs + 4 * d4;
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < t; j++) {
      const f32x4 vv = *reinterpret_cast<const f32x4 *>(v + j * HDV);
      const float pp = p[j];
      acc.x = fmaf(vv.x, pp, acc.x);
      acc.y = fmaf(vv.y, pp, acc.y);
      acc.z = fmaf(vv.z, pp, acc.z);
      acc.w = fmaf(vv.w, pp, acc.w);
    }
    float *o = yl + (long)(q0 + s) * c + 4 * d4;
#pragma unroll
    for (int k = 0; k < 4; k++)
      if (4 * d4 + k < hd) o[k] = acc[k];
  }
}

static size_t attention_rows_floats(int t, int hdv, int runs) {
  const size_t tq = (size_t)(t + runs - 1) / runs;
  return (size_t)2 * t * hdv + tq * hdv + tq * (t + 1) + tq * 18;
}

static size_t attention_lds_floats(int t, int hd, bool scores) {
  return (size_t)3 * t * hd + (size_t)t * 18 + (scores ? (size_t)t * (t + 1) : 0);
}

// gfx950 has 160 KiB of LDS per CU; a kernel may use it all once allowed to.

static bool attention_in_lds(int t, int hd) {
  return attention_lds_floats(t, hd, true) * sizeof(float) <= kMaxLds;
}

size_t attention_scratch_floats(int t, int c, int heads, int lanes) {
  int hd = c / heads;
  if (attention_in_lds(t, hd)) return 0;
  return (size_t)lanes * heads * t * (t + 1);
}

hipError_t launch_attention(const float *x, long x_lane_stride, float scale, int t, int c,
                            int heads, int lanes, float *y, long y_lane_stride, float *scratch,
                            hipStream_t s) {
  if (heads <= 0 || c % heads) return hipErrorInvalidValue;
  int hd = c / heads;
  if (hd > 64) return hipErrorInvalidValue;
  bool lds = attention_in_lds(t, hd);
  if (!lds && !scratch) return hipErrorInvalidValue;
  size_t shm = attention_lds_floats(t, hd, lds) * sizeof(float);
  if (shm > kMaxLds) return hipErrorInvalidValue;
  float *g = lds ? nullptr : scratch;
  auto go = [&](auto kernel, int nt) {
    // Allowed before any use beyond 64 KiB (and so before a graph capture
    // records such a launch).
    if (shm > 64 * 1024) {
      hipError_t e = allow_lds(reinterpret_cast<const void *>(kernel), int(kMaxLds));
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(lanes * heads), dim3(nt), shm, s, x, x_lane_stride, scale, t,
                       c, heads, y, y_lane_stride, g);
    return hipGetLastError();
  };
  // Lines whose K, V and a run's scores fit LDS: runs of query rows, enough
  // blocks for two per CU.
  const int hdv = hd <= 16 ? 16 : (hd <= 32 ? 32 : 64);
  const int runs = std::max(1, std::min(t, (512 + lanes * heads - 1) / (lanes * heads)));
  const size_t rshm = attention_rows_floats(t, hdv, runs) * sizeof(float);
  if (rshm <= 64 * 1024) {
    const long blocks = (long)lanes * heads * runs;
    if (hdv == 16)
      hipLaunchKernelGGL(attention_rows<16>, dim3((unsigned)blocks), dim3(256), rshm, s, x, x_lane_stride, scale, t,
                         c, heads, runs, y, y_lane_stride);
    else if (hdv == 32)
      hipLaunchKernelGGL(attention_rows<32>, dim3((unsigned)blocks), dim3(256), rshm, s, x, x_lane_stride, scale, t,
                         c, heads, runs, y, y_lane_stride);
    else
      hipLaunchKernelGGL(attention_rows<64>, dim3((unsigned)blocks), dim3(256), rshm, s, x, x_lane_stride, scale, t,
                         c, heads, runs, y, y_lane_stride);
    return hipGetLastError();
  }
  if (hd <= 16) return go(attention_kernel<16, 1024>, 1024);
  if (hd <= 32) return go(attention_kernel<32, 512>, 512);
  return go(attention_kernel<64, 256>, 256);
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

// Folds four values at columns c0 .. c0 + 3 into a running (max, sum, first
// column): their maximum first (the lowest column among equals) rescales the
// sum when it is a new maximum, then exp(v - max) of the four is added, with
// the hardware exp2 (within 1 ulp; the sum is a probability's denominator,
// held to a tolerance, while the argmax is exact).
__device__ __forceinline__ void best_fold4(Best &st, f32x4 v, int c0) {
  const float L = 1.44269504088896341f;  // log2(e)
  const float m4 = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
  if (m4 > st.m) {
    const int b = v[0] == m4 ? c0 : (v[1] == m4 ? c0 + 1 : (v[2] == m4 ? c0 + 2 : c0 + 3));
    st.s = st.m == -__builtin_inff() ? 0.0f : st.s * __builtin_amdgcn_exp2f((st.m - m4) * L);
    st.m = m4;
    st.b = (float)b;
  }
  const float c = st.m * L;
  st.s += __builtin_amdgcn_exp2f(fmaf(v[0], L, -c)) + __builtin_amdgcn_exp2f(fmaf(v[1], L, -c)) +
          (__builtin_amdgcn_exp2f(fmaf(v[2], L, -c)) + __builtin_amdgcn_exp2f(fmaf(v[3], L, -c)));
}

// One value at column c, as the engine's running update.
__device__ __forceinline__ void best_fold1(Best &st, float v, int c) {
  if (v > st.m) {
    st.s = st.m == -__builtin_inff() ? 1.0f : st.s * exp_neg(st.m - v) + 1.0f;
    st.m = v;
    st.b = (float)c;
  } else {
    st.s = st.s + exp_neg(v - st.m);
  }
}

// One block of 128 threads per row. The row's 16-byte aligned middle is read
// as float4 (columns 4t .. 4t+3 of every 512-float stride), four of them in
// flight per thread; the few columns before the first 16-byte boundary and
// after the last go one per thread. Each thread's columns arrive in
// increasing order, so its running state keeps the first maximum; the block
// joins the threads in a fixed order, ties to the lowest column.
constexpr int kArgmaxThreads = 128;

__global__ __launch_bounds__(kArgmaxThreads) void row_argmax_kernel(const float *x, float *y, int cols) {
  constexpr int T = kArgmaxThreads, U = 4;
  __shared__ Best part[T / 64];
  const float *row = x + (long)blockIdx.x * cols;
  const int tid = threadIdx.x;
  Best st{-__builtin_inff(), 0.0f, __builtin_inff()};
  const int head = min((int)((4 - (((uintptr_t)row >> 2) & 3)) & 3), cols);
  if (tid < head) best_fold1(st, row[tid], tid);
  const int nv = (cols - head) >> 2;
  const f32x4 *v4 = reinterpret_cast<const f32x4 *>(row + head);
  for (int base = 0; base < nv; base += U * T) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = base + tid + T * u;
      v[u] = i < nv ? v4[i] : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __builtin_amdgcn_sched_barrier(0);  // all four loads issue before the first use
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = base + tid + T * u;
      if (i < nv) best_fold4(st, v[u], head + 4 * i);
    }
  }
  const int t = head + 4 * nv + tid;
  if (t < cols) best_fold1(st, row[t], t);
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    Best o{__shfl_xor(st.m, d, 64), __shfl_xor(st.s, d, 64), __shfl_xor(st.b, d, 64)};
    st = best_join(st, o);
  }
  if ((tid & 63) == 0) part[tid >> 6] = st;
  __syncthreads();
  if (tid == 0) {
    Best r = part[0];
    for (int k = 1; k < T / 64; k++) r = best_join(r, part[k]);
    y[2 * (long)blockIdx.x] = r.b;
    y[2 * (long)blockIdx.x + 1] = 1.0f / r.s;
  }
}

hipError_t launch_row_argmax(const float *x, float *y, int rows, int cols, hipStream_t s) {
  if (rows <= 0 || cols <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(row_argmax_kernel, dim3(rows), dim3(kArgmaxThreads), 0, s, x, y, cols);
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
  const int fused = cols / 8 * 8;  // tail columns multiply and add separately
  for (int i = 0; i < a.ic; i++) {
    float v = xp[i];
#pragma unroll
    for (int n = 0; n < 16; n++) {
      if (n < fused) acc[n] = fmaf(a.w[(long)i * cols + n], v, acc[n]);
      else if (n < cols) acc[n] = acc[n] + v * a.w[(long)i * cols + n];
    }
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

// ------------------------------------------------------------ DB mask

// mask[i] = prob[i] > thresh, four pixels a thread (the DB threshold,
// src/det.rs:438, compared in f32).
__global__ __launch_bounds__(256) void db_mask_kernel(const float *prob, uint8_t *mask, long n, float thresh) {
  const long i = ((long)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 4 <= n && (reinterpret_cast<uintptr_t>(prob) & 15) == 0 && (reinterpret_cast<uintptr_t>(mask) & 3) == 0) {
    const f32x4 p = *reinterpret_cast<const f32x4 *>(prob + i);
    const uint32_t m = uint32_t(p.x > thresh) | uint32_t(p.y > thresh) << 8 | uint32_t(p.z > thresh) << 16 |
                       uint32_t(p.w > thresh) << 24;
    *reinterpret_cast<uint32_t *>(mask + i) = m;
    return;
  }
  for (long k = i; k < n && k < i + 4; k++) mask[k] = prob[k] > thresh;
}

hipError_t launch_db_mask(const float *prob, uint8_t *mask, long n, float thresh, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(db_mask_kernel, dim3(blocks_for((n + 3) / 4, 256)), dim3(256), 0, s, prob, mask, n, thresh);
  return hipGetLastError();
}

// A copy of n4 float4s through LDS by direct loads (global_load_lds, 16
// bytes a lane, 1024 float4s a block), the way the GEMM rings and the
// depthwise tiles load: the memory counters' calibration for such kernels.
__global__ __launch_bounds__(256) void copy_lds_kernel(const float *x, float *y, long n4) {
  __shared__ __attribute__((aligned(16))) float buf[1024 * 4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long base = (long)blockIdx.x * 1024;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int ins = q * 4 + wave;  // the wave's direct load: float4s 64 ins .. 64 ins + 63
    const long u = base + ins * 64 + lane;
    const float *p = u < n4 ? x + 4 * u : kDwZeros;
    __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(buf + ins * 256), 16, 0, 0);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const long u = base + q * 256 + tid;
    if (u < n4) reinterpret_cast<f32x4 *>(y)[u] = reinterpret_cast<const f32x4 *>(buf)[q * 256 + tid];
  }
}

hipError_t launch_copy_lds(const float *x, float *y, long n, hipStream_t s) {
  if (n <= 0 || n % 4 || (uintptr_t(x) & 15) || (uintptr_t(y) & 15)) return hipErrorInvalidValue;
  const long n4 = n / 4;
  hipLaunchKernelGGL(copy_lds_kernel, dim3(unsigned((n4 + 1023) / 1024)), dim3(256), 0, s, x, y, n4);
  return hipGetLastError();
}

// The DB threshold as row bitmasks (src/det.rs:438, compared in f32): one
// wave per 64-pixel word of a row, each lane one pixel, the wave's ballot
// the word (bit x % 64 of word x / 64; pixels past the width are 0). The
// map is `lanes` h x w maps, `lane_stride` floats apart; the words of a
// lane follow each other row by row.
__global__ __launch_bounds__(256) void db_bits_kernel(const float *map, long lane_stride, int w, int h, int words,
                                                       float thresh, unsigned long long *bits, long total) {
  const long word = (long)blockIdx.x * 4 + threadIdx.x / 64;
  if (word >= total) return;  // whole waves leave together
  const int lane = threadIdx.x % 64;
  const long row = word / words;
  const int x = int(word - row * words) * 64 + lane;
  const long ln = row / h;
  const float *src = map + ln * lane_stride + (row - ln * h) * w;
  const bool ink = x < w && src[x] > thresh;
  const unsigned long long b = __ballot(ink);
  if (lane == 0) bits[word] = b;
}

hipError_t launch_db_bits(const float *map, long lane_stride, int w, int h, int lanes, float thresh,
                          unsigned long long *bits, hipStream_t s) {
  if (w <= 0 || h <= 0 || lanes <= 0) return hipErrorInvalidValue;
  const int words = (w + 63) / 64;
  const long total = long(lanes) * h * words;
  hipLaunchKernelGGL(db_bits_kernel, dim3(unsigned((total + 3) / 4)), dim3(256), 0, s, map, lane_stride, w, h, words,
                     thresh, bits, total);
  return hipGetLastError();
}

}  // namespace ppocr
