// Layers computed directly on the vector ALUs, each output in the CPU
// engine's own summation order, so the results are bit-identical to it:
//  - conv_direct: a windowed convolution over few input channels (the RGB
//    stem), where an implicit GEMM would spend its time on index arithmetic;
//  - db_head: the detector head's two 2x2 stride-2 transposed convolutions,
//    the second narrow, in one pass, so the wide intermediate map never
//    reaches memory.
#include "act.hpp"
#include "kernels.hpp"

namespace ppocr {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Thread = one output pixel of one lane; block row blockIdx.y = a group of
// eight output channels, whose weights the block stages in LDS first (every
// thread of the block reads the same ones). Order per output
// (src/engine/kernels/dense.rs:38-147, conv.rs:146-236): the bias first
// (always for the RGB stem; otherwise for a multiple-of-16 width except the
// row's last ow % 4 pixels), taps [ky][kx], channels in order, a fused
// multiply-add for columns below oc / 8 * 8 and a separate multiply and add
// above; a bias not taken first is added last.
constexpr int kDirectTaps = 64;  // kh * kw * ic at most

// KH, KW, IC > 0: the window and channel count fixed at compile time, so the
// thread issues all of its patch's loads before the first multiply (the
// loads of a runtime loop would each wait for the previous sum). 0: any.
// Zeros for the unconditional loads of the direct kernels (at least IC
// floats).
__device__ __attribute__((aligned(16))) float kDirectZeros[4];

template <int KH, int KW, int IC>
__global__ __launch_bounds__(256) void conv_direct_kernel(DirectArgs a) {
  __shared__ __attribute__((aligned(16))) float ws[kDirectTaps * 8];
  constexpr bool FIXED = KH > 0;
  static_assert(IC <= 4, "kDirectZeros holds four floats");
  const int kh = FIXED ? KH : a.kh, kw = FIXED ? KW : a.kw, ic = FIXED ? IC : a.ic;
  const int j0 = blockIdx.y * 8;
  const int K = kh * kw * ic;
  // The bias of the group's eight columns, requested first and
  // unconditionally (a load under a per-lane condition would wait at once).
  float bk[8];
  const float *bsrc = a.bias ? a.bias : kDirectZeros;
#pragma unroll
  for (int k = 0; k < 8; k++) bk[k] = bsrc[a.bias ? min(j0 + k, a.oc - 1) : 0];
  for (int e = threadIdx.x; e < K * 8; e += 256) {
    const int r = e >> 3, k = e & 7;
    ws[e] = j0 + k < a.oc ? a.w[(long)r * a.oc + j0 + k] : 0.0f;
  }
  __syncthreads();
  const int per = a.oh * a.ow;
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= a.lanes * per) return;
  const int ln = g / per;
  const int rem = g - ln * per;
  const int oy = rem / a.ow, ox = rem - oy * a.ow;
  const float *x = a.x + (long)ln * a.x_lane_stride;
  const bool first = ox < a.first_end;
  float acc[8];
#pragma unroll
  for (int k = 0; k < 8; k++) acc[k] = (a.bias && first && j0 + k < a.oc) ? bk[k] : 0.0f;
  // Whether the group's eight columns all fuse is the same for the whole
  // block: branch once rather than select per column.
  const bool all_fused = j0 + 8 <= a.fused;
  auto tap_sum = [&](const float *tap, float v, int i) {
    const float4 w0 = *reinterpret_cast<const float4 *>(tap + i * 8);
    const float4 w1 = *reinterpret_cast<const float4 *>(tap + i * 8 + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
    if (all_fused) {
#pragma unroll
      for (int k = 0; k < 8; k++) acc[k] = fmaf(wv[k], v, acc[k]);
    } else {
#pragma unroll
      for (int k = 0; k < 8; k++) acc[k] = j0 + k < a.fused ? fmaf(wv[k], v, acc[k]) : acc[k] + v * wv[k];
    }
  };
  if constexpr (FIXED) {
    // Gather the patch (zeros where the window leaves the image, which are
    // then skipped, as the engine skips them), then sum in tap order.
    float patch[KH * KW * IC];
    bool in[KH * KW];
#pragma unroll
    for (int ky = 0; ky < KH; ky++) {
#pragma unroll
      for (int kx = 0; kx < KW; kx++) {
        const int iy = oy * a.sh + ky - a.pt, ix = ox * a.sw + kx - a.pl;
        const bool ok = iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
        in[ky * KW + kx] = ok;
        // Every load unconditional (outside the image: kDirectZeros), so
        // that the whole patch is in flight at once.
        const float *px = ok ? x + ((long)iy * a.iw + ix) * IC : kDirectZeros;
#pragma unroll
        for (int i = 0; i < IC; i++) patch[(ky * KW + kx) * IC + i] = px[i];
      }
    }
#pragma unroll
    for (int t = 0; t < KH * KW; t++) {
      if (!in[t]) continue;
#pragma unroll
      for (int i = 0; i < IC; i++) tap_sum(ws + t * IC * 8, patch[t * IC + i], i);
    }
  } else {
    for (int ky = 0; ky < kh; ky++) {
      const int iy = oy * a.sh + ky - a.pt;
      if (iy < 0 || iy >= a.ih) continue;
      for (int kx = 0; kx < kw; kx++) {
        const int ix = ox * a.sw + kx - a.pl;
        if (ix < 0 || ix >= a.iw) continue;
        const float *px = x + ((long)iy * a.iw + ix) * ic;
        for (int i = 0; i < ic; i++) tap_sum(ws + (ky * kw + kx) * ic * 8, px[i], i);
      }
    }
  }
  float *y = a.y + (long)ln * a.y_lane_stride + (long)rem * a.oc + j0;
#pragma unroll
  for (int k = 0; k < 8; k++) {
    if (j0 + k >= a.oc) break;
    float v = acc[k];
    if (a.bias && !first) v = v + bk[k];
    y[k] = act(v, a.act);
  }
}

bool direct_supported(int kh, int kw, int ic) { return kh * kw * ic <= kDirectTaps; }

// The RGB stem, 3x3 over 3 channels to OC (a multiple of 8): every output
// from its bias, every column fused (the stem rule, src/engine/conv.rs:
// 146-236). A block holds 256 / QS pixels; wave-uniform quarter (or half) q
// of the threads computes outputs q * OC / QS .. of every pixel, so that a
// small map still fills the GPU. The block's pixels x OC outputs are one run
// of memory (within a lane), written back from LDS as whole float4 rows.
template <int OC, int QS>
__global__ __launch_bounds__(256) void conv_stem_kernel(DirectArgs a) {
  constexpr int K = 27, PB = 256 / QS, OQ = OC / QS;
  static_assert(OQ % 4 == 0 && PB % 64 == 0, "float4 columns, whole waves per part");
  __shared__ __attribute__((aligned(16))) float ws[K * OC];
  __shared__ __attribute__((aligned(16))) float out[PB * OC];
  const int per = a.oh * a.ow, total = a.lanes * per;
  const int pl = threadIdx.x % PB, q = threadIdx.x / PB;
  // Blocks numbered XCD by XCD (xcd_tile): neighbouring output rows, which
  // read the same input rows, meet in one L2.
  const int g0 = xcd_tile((int)blockIdx.x, (int)gridDim.x) * PB, g = g0 + pl;
  // The pixel's patch is requested first, then every weight at once (a
  // rolled staging loop would wait out each load before the next), so that
  // both arrive in one round trip.
  float patch[K];
  bool in[9];
  if (g < total) {
    const int ln = g / per, rem = g - ln * per;
    const int oy = rem / a.ow, ox = rem - oy * a.ow;
    const float *x = a.x + (long)ln * a.x_lane_stride;
#pragma unroll
    for (int ky = 0; ky < 3; ky++) {
#pragma unroll
      for (int kx = 0; kx < 3; kx++) {
        const int iy = oy * a.sh + ky - a.pt, ix = ox * a.sw + kx - a.pl;
        const bool ok = iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
        in[ky * 3 + kx] = ok;
        const float *px = x + ((long)iy * a.iw + ix) * 3;
#pragma unroll
        for (int i = 0; i < 3; i++) patch[(ky * 3 + kx) * 3 + i] = ok ? px[i] : 0.0f;
      }
    }
  }
  // This part's biases, with the first loads (unconditional: a null bias
  // reads kDirectZeros, never used).
  float bq[OQ];
#pragma unroll
  for (int j = 0; j < OQ; j++) bq[j] = (a.bias ? a.bias : kDirectZeros)[a.bias ? q * OQ + j : 0];
  {
    constexpr int WN = (K * OC + 255) / 256;
    float wt[WN];
#pragma unroll
    for (int i = 0; i < WN; i++) wt[i] = a.w[min((int)threadIdx.x + 256 * i, K * OC - 1)];
#pragma unroll
    for (int i = 0; i < WN; i++)
      if ((int)threadIdx.x + 256 * i < K * OC) ws[threadIdx.x + 256 * i] = wt[i];
  }
  __syncthreads();
  if (g < total) {
    float acc[OQ];
#pragma unroll
    for (int j = 0; j < OQ; j++) acc[j] = a.bias ? bq[j] : 0.0f;
#pragma unroll
    for (int t = 0; t < 9; t++) {
      if (!in[t]) continue;
#pragma unroll
      for (int i = 0; i < 3; i++) {
        const float v = patch[t * 3 + i];
        const float *wr = ws + (t * 3 + i) * OC + q * OQ;
#pragma unroll
        for (int j = 0; j < OQ; j += 4) {
          const float4 w = *reinterpret_cast<const float4 *>(wr + j);
          acc[j] = fmaf(w.x, v, acc[j]);
          acc[j + 1] = fmaf(w.y, v, acc[j + 1]);
          acc[j + 2] = fmaf(w.z, v, acc[j + 2]);
          acc[j + 3] = fmaf(w.w, v, acc[j + 3]);
        }
      }
    }
    float *o = out + pl * OC + q * OQ;
#pragma unroll
    for (int j = 0; j < OQ; j += 4)
      *reinterpret_cast<float4 *>(o + j) =
          make_float4(act(acc[j], a.act), act(acc[j + 1], a.act), act(acc[j + 2], a.act), act(acc[j + 3], a.act));
  }
  __syncthreads();
  const int n = min(PB, total - g0);
  const int l0 = g0 / per, l1 = (g0 + n - 1) / per;
  if (l0 == l1) {
    float4 *dst = reinterpret_cast<float4 *>(a.y + (long)l0 * a.y_lane_stride + (long)(g0 - l0 * per) * OC);
    const float4 *src = reinterpret_cast<const float4 *>(out);
    for (int e = threadIdx.x; e < n * OC / 4; e += 256) dst[e] = src[e];
  } else {
    for (int e = threadIdx.x; e < n * OC; e += 256) {
      const int p = g0 + e / OC, ln = p / per, rem = p - ln * per;
      a.y[(long)ln * a.y_lane_stride + (long)rem * OC + e % OC] = out[e];
    }
  }
}

// A windowed convolution over a few channels per tap (IC a multiple of 4) to
// OC outputs (a multiple of 4): thread = one output pixel and all its
// outputs; the weights [k][oc] in LDS, read four columns at a time; the
// whole window loaded before the first sum. Order per output as the engine's
// vector dense kernel (src/engine/kernels/dense.rs:23-147): the bias first
// for pixels left of first_end, the taps [ky][kx] and their channels in
// order, a tap outside the image reading zeros, a fused multiply-add for
// columns below OC / 8 * 8 and a separate multiply and add above, a bias
// not taken first added last. The block's 256 pixels x OC outputs leave
// through LDS as whole float4 rows.
template <int KH, int KW, int IC, int OC>
__global__ __launch_bounds__(256) void conv_direct_pix(DirectArgs a) {
  static_assert(IC % 4 == 0 && OC % 4 == 0, "four channels at a time");
  constexpr int T = KH * KW, K = T * IC, FUSED = OC / 8 * 8;
  __shared__ __attribute__((aligned(16))) float ws[K * OC];
  __shared__ __attribute__((aligned(16))) float out[256 * OC];
  for (int e = threadIdx.x; e < K * OC; e += 256) ws[e] = a.w[e];
  __syncthreads();
  const int per = a.oh * a.ow, total = a.lanes * per;
  // Blocks numbered XCD by XCD (xcd_tile): neighbouring output rows, which
  // read the same input rows, meet in one L2.
  const int g0 = xcd_tile((int)blockIdx.x, (int)gridDim.x) * 256, g = g0 + threadIdx.x;
  if (g < total) {
    const int ln = g / per, rem = g - ln * per;
    const int oy = rem / a.ow, ox = rem - oy * a.ow;
    const float *x = a.x + (long)ln * a.x_lane_stride;
    // Tap t's IC channels, zeros outside the image.
    auto load = [&](int t, f32x4 *v) {
      const int ky = t / KW, kx = t - ky * KW;
      const int iy = oy * a.sh + ky - a.pt, ix = ox * a.sw + kx - a.pl;
      const bool ok = iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
      const f32x4 *px = reinterpret_cast<const f32x4 *>(x + ((long)iy * a.iw + ix) * IC);
#pragma unroll
      for (int q = 0; q < IC / 4; q++) v[q] = ok ? px[q] : f32x4{0.f, 0.f, 0.f, 0.f};
    };
    const bool early = ox < a.first_end;
    float acc[OC];
#pragma unroll
    for (int j = 0; j < OC; j++) acc[j] = a.bias && early ? a.bias[j] : 0.0f;
    // A runtime loop over the taps, the next tap's channels requested before
    // the current tap's sums (a fully unrolled window lets the compiler
    // hoist every weight read and product at once and spill them).
    f32x4 cur[IC / 4], nxt[IC / 4];
    load(0, cur);
#pragma unroll 1
    for (int t = 0; t < T; t++) {
      load(t + 1 < T ? t + 1 : t, nxt);
#pragma unroll
      for (int i = 0; i < IC; i++) {
        const float v = cur[i / 4][i % 4];
        const float *wr = ws + (t * IC + i) * OC;
#pragma unroll
        for (int j = 0; j < OC; j += 4) {
          const f32x4 w = *reinterpret_cast<const f32x4 *>(wr + j);
#pragma unroll
          for (int q = 0; q < 4; q++)
            acc[j + q] = j + q < FUSED ? fmaf(w[q], v, acc[j + q]) : acc[j + q] + w[q] * v;
        }
      }
#pragma unroll
      for (int q = 0; q < IC / 4; q++) cur[q] = nxt[q];
    }
    f32x4 *o = reinterpret_cast<f32x4 *>(out + threadIdx.x * OC);
#pragma unroll
    for (int j = 0; j < OC; j += 4) {
      float r[4];
#pragma unroll
      for (int q = 0; q < 4; q++) r[q] = act(a.bias && !early ? acc[j + q] + a.bias[j + q] : acc[j + q], a.act);
      o[j / 4] = f32x4{r[0], r[1], r[2], r[3]};
    }
  }
  __syncthreads();
  const int n = min(256, total - g0);
  const int l0 = g0 / per, l1 = (g0 + n - 1) / per;
  if (l0 == l1) {
    f32x4 *dst = reinterpret_cast<f32x4 *>(a.y + (long)l0 * a.y_lane_stride + (long)(g0 - l0 * per) * OC);
    const f32x4 *src = reinterpret_cast<const f32x4 *>(out);
    for (int e = threadIdx.x; e < n * OC / 4; e += 256) dst[e] = src[e];
  } else {
    for (int e = threadIdx.x; e < n * OC; e += 256) {
      const int p = g0 + e / OC, ln = p / per, rem = p - ln * per;
      a.y[(long)ln * a.y_lane_stride + (long)rem * OC + e % OC] = out[e];
    }
  }
}

// Measured on the detector's stem: 12 -> 24 beats the implicit GEMM (19.8
// against 28.6 us at 480 x 480); 24 -> 12, whose last four columns take a
// separate multiply and add, does not (23.6 against 21.9 us).
bool direct_pix_supported(int kh, int kw, int ic, int oc) { return kh == 2 && kw == 2 && ic == 12 && oc == 24; }

hipError_t launch_conv_direct(const DirectArgs &a, hipStream_t s) {
  const long n = (long)a.lanes * a.oh * a.ow;
  if (n <= 0 || a.oc <= 0) return hipSuccess;
  const unsigned nb = (unsigned)((n + 255) / 256);
  if (direct_pix_supported(a.kh, a.kw, a.ic, a.oc) && n <= 0x7fffff00L && a.fused == a.oc / 8 * 8 &&
      (reinterpret_cast<uintptr_t>(a.x) & 15) == 0 && a.x_lane_stride % 4 == 0 &&
      (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && a.y_lane_stride % 4 == 0) {
    hipLaunchKernelGGL((conv_direct_pix<2, 2, 12, 24>), dim3(nb), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  if (!direct_supported(a.kh, a.kw, a.ic) || n > 0x7fffff00L || (a.oc + 7) / 8 > 65535)
    return hipErrorInvalidValue;
  const bool stem = a.kh == 3 && a.kw == 3 && a.ic == 3 && a.first_end >= a.ow && a.fused >= a.oc &&
                    (reinterpret_cast<uintptr_t>(a.y) & 15) == 0 && a.y_lane_stride % 4 == 0;
  const unsigned blocks = (unsigned)((n + 255) / 256);
  // The stem: 256 pixels a block, each thread all outputs of one pixel; on a
  // map too small for that to fill the GPU (under two blocks a CU), 64
  // pixels a block with a quarter of the outputs a wave, or 128 for 24
  // outputs (halves of 12).
  if (stem) {
    const bool split = blocks < 512;
    const unsigned b64 = (unsigned)((n + 63) / 64), b128 = (unsigned)((n + 127) / 128);
    auto go = [&](auto kernel, unsigned nb) {
      hipLaunchKernelGGL(kernel, dim3(nb), dim3(256), 0, s, a);
      return hipGetLastError();
    };
    if (a.oc == 16) return split ? go(conv_stem_kernel<16, 4>, b64) : go(conv_stem_kernel<16, 1>, blocks);
    if (a.oc == 24) return split ? go(conv_stem_kernel<24, 2>, b128) : go(conv_stem_kernel<24, 1>, blocks);
    if (a.oc == 32) return split ? go(conv_stem_kernel<32, 4>, b64) : go(conv_stem_kernel<32, 1>, blocks);
    if (a.oc == 48) return split ? go(conv_stem_kernel<48, 4>, b64) : go(conv_stem_kernel<48, 1>, blocks);
  }
  dim3 grid(blocks, (a.oc + 7) / 8), block(256);
  if (a.kh == 3 && a.kw == 3 && a.ic == 3)
    hipLaunchKernelGGL((conv_direct_kernel<3, 3, 3>), grid, block, 0, s, a);
  else if (a.kh == 2 && a.kw == 2 && a.ic == 3)
    hipLaunchKernelGGL((conv_direct_kernel<2, 2, 3>), grid, block, 0, s, a);
  else if (a.kh == 3 && a.kw == 3 && a.ic == 1)
    hipLaunchKernelGGL((conv_direct_kernel<3, 3, 1>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((conv_direct_kernel<0, 0, 0>), grid, block, 0, s, a);
  return hipGetLastError();
}

// ---------------------------------------------------------------- stem block

// One workgroup per T x T tile of one lane's oh x ow maps. It computes s1
// over the tile plus two rows and columns (what the pool and the 2x2 layers
// read), the first 2x2 over the tile plus one row and column, then the max
// pool and the second 2x2 over the tile; s1 and the first 2x2's output never
// leave LDS. s1 and the pool in the CPU engine's order, bit for bit: s1 from
// its bias, taps [ky][kx] skipping those outside the input, channels in
// order, every column a fused multiply-add (the stem rule,
// src/engine/conv.rs:146-236), its weights wave-uniform scalar operands
// (the scalar cache); the pool seeded with its first tap, a later tap inside
// the map kept only when greater (conv.rs:404-440). The two 2x2 layers run
// on FP32 MFMA (sums in another order, within the MFMA tolerance), bias and
// activation after the products.
constexpr int kStemT = 14;
// The bias of a layer that has none: its sums start from, or add, nothing.
__device__ __attribute__((aligned(16))) float kStemNoBias[32];

// ACT: the activation of all three layers, fixed at compile time (a
// runtime choice per output would inline every activation's code).
template <int C1, int C2, int C3, int ACT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5))) void stem_block(StemArgs a) {
  constexpr int T = kStemT, R1 = T + 2, R2 = T + 1;
  // Pixels an odd number of float4s apart: a wave's float4 reads of
  // consecutive pixels fall in distinct banks.
  constexpr int P1 = (C1 / 4) % 2 ? C1 : C1 + 4, P2 = (C2 / 4) % 2 ? C2 : C2 + 4;
  static_assert(R1 * R1 == 256, "one s1 pixel per thread");
  static_assert(C1 % 8 == 0 && C2 % 4 == 0 && C3 % 4 == 0, "float4 channels, every stem column fused");
  // One LDS area: s1 until the first 2x2 has read it; then the first 2x2's
  // map (held in registers across the barrier) and the staged outputs. At
  // 29.6 KB, five workgroups share a CU.
  constexpr int F2 = R2 * R2 * P2, LDS_F = R1 * R1 * P1 > F2 + T * T * C3 ? R1 * R1 * P1 : F2 + T * T * C3;
  static_assert(F2 % 4 == 0, "staging on a float4 boundary");
  __shared__ __attribute__((aligned(16))) float lds[LDS_F];
  float *const m1 = lds, *const m2 = lds, *const st = lds + F2;
  const int tiles_x = (a.ow + T - 1) / T, tiles_y = (a.oh + T - 1) / T;
  // Tiles numbered XCD by XCD (xcd_tile): neighbours, which share input
  // rows, meet in one L2.
  int t = xcd_tile((int)blockIdx.x, (int)gridDim.x);
  const int tx = t % tiles_x;
  t /= tiles_x;
  const int ty = t % tiles_y;
  const int ln = t / tiles_y;
  const int y0 = ty * T, x0 = tx * T, tid = threadIdx.x;
  // Read through the constant address space: wave-uniform scalar loads.
  typedef const __attribute__((address_space(4))) float cfloat;
  cfloat *w1 = (cfloat *)a.w1;
  // The 2x2 layers on FP32 MFMA (v_mfma_f32_16x16x4f32): rows are the
  // map's pixels in row-major order of the region, 16 a row block, the
  // reduction index k = tap * C + channel, taps [ky][kx]. Lane (li, lg)
  // holds a row block's A at row li, k = 16s + 4lg + e (e = 0..3 in the four
  // MFMAs of step s: one float4 read from LDS), and B at column li for the
  // same k. The first layer's B (and bias) is requested before s1, the
  // second's after it, each well before its use. A tap outside the map
  // reads zeros.
  const int lane = tid & 63, wave = tid >> 6, li = lane & 15, lg = lane >> 4;
  constexpr int S2 = 4 * C1 / 16, S3 = 4 * C2 / 16, NB3 = (C3 + 15) / 16;
  static_assert(C2 <= 16 && 4 * C1 % 16 == 0 && 4 * C2 % 16 == 0, "one column block; whole steps");
  f32x4 bw2[S2], bw3[NB3][S3];
#pragma unroll
  for (int q = 0; q < S2; q++)
#pragma unroll
    for (int e = 0; e < 4; e++) bw2[q][e] = li < C2 ? a.w2[(16 * q + 4 * lg + e) * C2 + li] : 0.0f;
  const float bias2 = a.b2 && li < C2 ? a.b2[li] : 0.0f;
  float bias3[NB3];

  // s1: thread tid is pixel (y0 + tid / R1, x0 + tid % R1). All 27 input
  // values are requested before the first product (their latency, from
  // memory not yet cached, is the phase's longest wait).
  {
    const int Y = y0 + tid / R1, X = x0 + tid % R1;
    if (Y < a.oh && X < a.ow) {
      const float *x = a.x + (long)ln * a.x_lane_stride;
      float v[27];
      bool in[9];
#pragma unroll
      for (int k = 0; k < 9; k++) {
        const int iy = 2 * Y + k / 3 - 1, ix = 2 * X + k % 3 - 1;
        in[k] = iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
        const float *px = x + ((long)(in[k] ? iy : 0) * a.iw + (in[k] ? ix : 0)) * 3;
#pragma unroll
        for (int i = 0; i < 3; i++) v[k * 3 + i] = px[i];
      }
      // A missing bias reads zeros: every sum starts from +0 either way.
      cfloat *b = (cfloat *)(a.b1 ? a.b1 : kStemNoBias);
      float acc[C1];
#pragma unroll
      for (int j = 0; j < C1; j++) acc[j] = b[j];
#pragma unroll
      for (int k = 0; k < 9; k++) {
        if (!in[k]) continue;
#pragma unroll
        for (int i = 0; i < 3; i++) {
          cfloat *w = w1 + (k * 3 + i) * C1;
#pragma unroll
          for (int j = 0; j < C1; j++) acc[j] = fmaf(w[j], v[k * 3 + i], acc[j]);
        }
      }
      f32x4 *o = reinterpret_cast<f32x4 *>(m1 + tid * P1);
#pragma unroll
      for (int j = 0; j < C1; j += 4)
        o[j / 4] = f32x4{act(acc[j], ACT), act(acc[j + 1], ACT), act(acc[j + 2], ACT),
                         act(acc[j + 3], ACT)};
    }
  }
#pragma unroll
  for (int c = 0; c < NB3; c++) {
    const int n = 16 * c + li;
#pragma unroll
    for (int q = 0; q < S3; q++)
#pragma unroll
      for (int e = 0; e < 4; e++) bw3[c][q][e] = n < C3 ? a.w3[(16 * q + 4 * lg + e) * C3 + n] : 0.0f;
    bias3[c] = a.b3 && n < C3 ? a.b3[n] : 0.0f;
  }
  __syncthreads();

  // The first 2x2 over (T + 1) x (T + 1) pixels: a wave takes row blocks
  // two at a time (b and b + 4), two independent MFMA chains; its outputs
  // stay in registers until s1 is no longer read.
  constexpr int M2 = R2 * R2, MB2 = (M2 + 15) / 16;
  static_assert(MB2 <= 16, "two rounds of two row blocks a wave");
  f32x4 res[2][2];
  {
    constexpr int M = M2, S = S2;
#pragma unroll
    for (int it = 0; it < 2; it++) {
      const int b0 = wave + 8 * it;
      int sy[2], sx[2];
      bool live[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int m = (b0 + 4 * u) * 16 + li;
        sy[u] = m / R2, sx[u] = m - sy[u] * R2;
        live[u] = m < M && y0 + sy[u] < a.oh && x0 + sx[u] < a.ow;
      }
      f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
      for (int q = 0; q < S; q++) {
        const int k = 16 * q + 4 * lg, tap = k / C1, ch = k - tap * C1, ky = tap >> 1, kx = tap & 1;
        f32x4 v[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          v[u] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (live[u] && y0 + sy[u] + ky < a.oh && x0 + sx[u] + kx < a.ow)
            v[u] = *reinterpret_cast<const f32x4 *>(m1 + ((sy[u] + ky) * R1 + sx[u] + kx) * P1 + ch);
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int u = 0; u < 2; u++) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[u][e], bw2[q][e], acc[u], 0, 0, 0);
      }
      // acc[u][r]: row 4 lg + r of block b0 + 4u, column li.
#pragma unroll
      for (int u = 0; u < 2; u++)
#pragma unroll
        for (int r = 0; r < 4; r++) res[it][u][r] = act(acc[u][r] + bias2, ACT);
    }
  }
  // The pool over the tile, one pixel a thread.
  if (tid < T * T) {
    const int oy = tid / T, ox = tid % T, Y = y0 + oy, X = x0 + ox;
    if (Y < a.oh && X < a.ow) {
      f32x4 *dst = reinterpret_cast<f32x4 *>(a.pool + (long)ln * a.pool_lane_stride + ((long)Y * a.ow + X) * a.pool_px);
#pragma unroll
      for (int q = 0; q < C1 / 4; q++) {
        f32x4 m = reinterpret_cast<const f32x4 *>(m1 + (oy * R1 + ox) * P1)[q];
#pragma unroll
        for (int k = 1; k < 4; k++) {
          const int ky = k / 2, kx = k % 2;
          if (Y + ky >= a.oh || X + kx >= a.ow) continue;
          const f32x4 v = reinterpret_cast<const f32x4 *>(m1 + ((oy + ky) * R1 + ox + kx) * P1)[q];
#pragma unroll
          for (int e = 0; e < 4; e++) m[e] = v[e] > m[e] ? v[e] : m[e];
        }
        dst[q] = m;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 2; it++)
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int mo = (wave + 8 * it + 4 * u) * 16 + 4 * lg + r;
        if (mo < M2 && li < C2) m2[mo * P2 + li] = res[it][u][r];
      }
  __syncthreads();

  // The second 2x2 over the tile, its outputs staged in LDS past the first's
  // map, then stored as whole pixel rows.
  {
    constexpr int M = T * T, MB = (M + 15) / 16, S = S3, NB = NB3;
    for (int b = wave; b < MB; b += 4) {
      const int m = b * 16 + li, oy = m / T, ox = m - oy * T;
      const bool live = m < M && y0 + oy < a.oh && x0 + ox < a.ow;
      f32x4 acc[NB];
#pragma unroll
      for (int c = 0; c < NB; c++) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < S; q++) {
        const int k = 16 * q + 4 * lg, tap = k / C2, ch = k - tap * C2, ky = tap >> 1, kx = tap & 1;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (live && y0 + oy + ky < a.oh && x0 + ox + kx < a.ow)
          v = *reinterpret_cast<const f32x4 *>(m2 + ((oy + ky) * R2 + ox + kx) * P2 + ch);
#pragma unroll
        for (int e = 0; e < 4; e++)
#pragma unroll
          for (int c = 0; c < NB; c++) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(v[e], bw3[c][q][e], acc[c], 0, 0, 0);
      }
#pragma unroll
      for (int c = 0; c < NB; c++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int mo = b * 16 + 4 * lg + r, n = 16 * c + li;
          if (mo < M && n < C3) st[mo * C3 + n] = act(acc[c][r] + bias3[c], ACT);
        }
    }
  }
  __syncthreads();
  // Copy-out: each valid pixel's C3 outputs as C3 / 4 float4 stores.
  for (int e = tid; e < T * T * (C3 / 4); e += 256) {
    const int m = e / (C3 / 4), q = e - m * (C3 / 4), oy = m / T, ox = m - oy * T, Y = y0 + oy, X = x0 + ox;
    if (Y < a.oh && X < a.ow)
      reinterpret_cast<f32x4 *>(a.y + (long)ln * a.y_lane_stride + ((long)Y * a.ow + X) * a.y_px)[q] =
          reinterpret_cast<const f32x4 *>(st + m * C3)[q];
  }
}

bool stem_block_supported(int c1, int c2, int c3, int act1, int act2, int act3) {
  return c1 == 24 && c2 == 12 && c3 == 24 && act1 == act2 && act2 == act3 && (act1 == ACT_HARDSWISH || act1 == ACT_RELU);
}

hipError_t launch_stem_block(const StemArgs &a, hipStream_t s) {
  if (!stem_block_supported(a.c1, a.c2, a.c3, a.act1, a.act2, a.act3) || a.ih < 1 || a.iw < 1 || a.lanes < 0)
    return hipErrorInvalidValue;
  // s1 is the 3x3 stride-2 pad-1 map of the input; float4 stores.
  if (a.oh != (a.ih - 1) / 2 + 1 || a.ow != (a.iw - 1) / 2 + 1) return hipErrorInvalidValue;
  if ((reinterpret_cast<uintptr_t>(a.pool) & 15) || (reinterpret_cast<uintptr_t>(a.y) & 15) ||
      a.pool_lane_stride % 4 || a.y_lane_stride % 4 || a.pool_px % 4 || a.y_px % 4 || a.pool_px < a.c1 ||
      a.y_px < a.c3)
    return hipErrorInvalidValue;
  const long tiles = (long)a.lanes * ((a.oh + kStemT - 1) / kStemT) * ((a.ow + kStemT - 1) / kStemT);
  if (tiles == 0) return hipSuccess;
  if (tiles > 0x7fffffffL) return hipErrorInvalidValue;
  if (a.act1 == ACT_RELU)
    hipLaunchKernelGGL((stem_block<24, 12, 24, ACT_RELU>), dim3((unsigned)tiles), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((stem_block<24, 12, 24, ACT_HARDSWISH>), dim3((unsigned)tiles), dim3(256), 0, s, a);
  return hipGetLastError();
}

// Thread = one input pixel (iy, ix) of the first transposed convolution and
// one of its four taps (ky, kx) (one tap a workgroup, so the weights a wave
// reads are uniform: the first layer's from LDS as broadcasts, the second's
// scalar operands from the scalar cache; the four taps of
// a block of 256 pixels are workgroups i, i + 8, i + 16, i + 24, which run
// on one XCD and so read those pixels once from memory into its L2). It forms
// the OC1 values of intermediate pixel (2iy+ky, 2ix+kx) as the engine's
// pointwise call over one input row does (src/engine/layers.rs:600-680):
// the bias first for a multiple-of-16 column count except the row's last
// iw % 4 pixels, else last; fused multiply-adds below cols / 8 * 8. After
// the first activation the intermediate pixel gives its 2 x 2 outputs of
// the second convolution (four columns: bias last, separate multiply and
// add), then the second activation; the thread writes 2 rows x 2 columns of
// the final map. A1, A2: the activations when fixed at compile time (the
// DB head's ReLU and sigmoid), else -1 and read from the arguments.
constexpr int kHeadMaxIc = 128;

template <int A>
__device__ __forceinline__ float head_act(float v, int code) {
  if constexpr (A >= 0) return act(v, A);
  else return act(v, code);
}

template <int OC1, int A1, int A2>
__global__ __launch_bounds__(256) void db_head_kernel(HeadArgs a) {
  constexpr int COLS1 = 4 * OC1;
  // 4 * OC1 columns, a multiple of 8 for every supported OC1: all of them
  // fuse their multiply-adds (columns below cols / 8 * 8 do).
  static_assert(COLS1 % 8 == 0, "every first-layer column fuses");
  typedef const __attribute__((address_space(4))) float cfloat;
  const int blk = (int)blockIdx.x, tap = (blk >> 3) & 3, pb = (blk & 7) | ((blk >> 5) << 3);
  const int ky = tap >> 1, kx = tap & 1;
  const int n0 = (ky * 2 + kx) * OC1;  // the columns of tap (ky, kx)
  cfloat *w2 = (cfloat *)a.w2;
  // The tap's first-layer weights [ic][OC1] in LDS, read as broadcasts: read
  // from the scalar cache, each channel's weights were waited for just
  // before its multiply-adds.
  __shared__ __attribute__((aligned(16))) float w1[kHeadMaxIc * OC1];
  for (int e = threadIdx.x; e < a.ic * OC1; e += 256) {
    const int i = e / OC1;
    w1[e] = a.w1[(long)i * COLS1 + n0 + (e - i * OC1)];
  }
  __syncthreads();
  const int per = a.ih * a.iw;
  const int g = pb * 256 + threadIdx.x;
  if (g >= a.lanes * per) return;
  const int ln = g / per;
  const int pix = g - ln * per;
  const int iy = pix / a.iw, ix = pix - iy * a.iw;
  const bool first = COLS1 % 16 == 0 && ix < a.iw / 4 * 4;
  const float *xp = a.x + (long)ln * a.x_lane_stride + (long)pix * a.ic;
  float b1[OC1], t[OC1];
#pragma unroll
  for (int n = 0; n < OC1; n++) b1[n] = a.b1 ? ((cfloat *)a.b1)[n0 + n] : 0.0f;
#pragma unroll
  for (int n = 0; n < OC1; n++) t[n] = first ? b1[n] : 0.0f;
  // Channels in runs of eight: the next run's loads are issued before this
  // run's sums, so a thread waits for memory once per run, not per channel.
  float4 cur0 = *reinterpret_cast<const float4 *>(xp), cur1 = *reinterpret_cast<const float4 *>(xp + 4);
  for (int i0 = 0; i0 < a.ic; i0 += 8) {
    float4 nx0 = cur0, nx1 = cur1;
    if (i0 + 8 < a.ic) {
      nx0 = *reinterpret_cast<const float4 *>(xp + i0 + 8);
      nx1 = *reinterpret_cast<const float4 *>(xp + i0 + 12);
    }
    const float xv[8] = {cur0.x, cur0.y, cur0.z, cur0.w, cur1.x, cur1.y, cur1.z, cur1.w};
#pragma unroll
    for (int ii = 0; ii < 8; ii++) {
      const float *wr = w1 + (i0 + ii) * OC1;
#pragma unroll
      for (int n = 0; n < OC1; n++) t[n] = fmaf(wr[n], xv[ii], t[n]);
    }
    cur0 = nx0, cur1 = nx1;
  }
#pragma unroll
  for (int n = 0; n < OC1; n++) t[n] = head_act<A1>(a.b1 && !first ? t[n] + b1[n] : t[n], a.act1);
  // Second convolution, oc 1: four columns, tap (ky2, kx2) = column ky2 * 2 + kx2.
  float out[4];
#pragma unroll
  for (int c = 0; c < 4; c++) {
    float acc = 0.0f;
#pragma unroll
    for (int o = 0; o < OC1; o++) acc = acc + t[o] * w2[o * 4 + c];
    if (a.b2) acc = acc + ((cfloat *)a.b2)[c];
    out[c] = head_act<A2>(acc, a.act2);
  }
  const long ow = 4L * a.iw;
  float *y = a.y + (long)ln * a.y_lane_stride + (4L * iy + 2L * ky) * ow + 4L * ix + 2L * kx;
  *reinterpret_cast<float2 *>(y) = make_float2(out[0], out[1]);
  *reinterpret_cast<float2 *>(y + ow) = make_float2(out[2], out[3]);
}

bool head_supported(int ic, int oc1) {
  return ic > 0 && ic % 8 == 0 && ic <= kHeadMaxIc && (oc1 == 8 || oc1 == 16 || oc1 == 24 || oc1 == 32);
}

hipError_t launch_db_head(const HeadArgs &a, hipStream_t s) {
  const long n = (long)a.lanes * a.ih * a.iw;
  if (n <= 0) return hipSuccess;
  // The float4 loads need 16-byte aligned pixels, the float2 stores 8-byte ones.
  if (!head_supported(a.ic, a.oc1) || (reinterpret_cast<uintptr_t>(a.y) & 15) || (a.y_lane_stride & 3) ||
      (reinterpret_cast<uintptr_t>(a.x) & 15) || (a.x_lane_stride & 3) || n > 0x7fffff00L)
    return hipErrorInvalidValue;
  // Pixel blocks in groups of 8, each group's four taps: 32 workgroups.
  dim3 grid((unsigned)((n + 2047) / 2048 * 32)), block(256);
  const bool db = a.act1 == ACT_RELU && a.act2 == ACT_SIGMOID;
  switch (a.oc1) {
    case 8: hipLaunchKernelGGL((db_head_kernel<8, -1, -1>), grid, block, 0, s, a); break;
    case 16: hipLaunchKernelGGL((db_head_kernel<16, -1, -1>), grid, block, 0, s, a); break;
    case 24:
      if (db) hipLaunchKernelGGL((db_head_kernel<24, ACT_RELU, ACT_SIGMOID>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((db_head_kernel<24, -1, -1>), grid, block, 0, s, a);
      break;
    case 32: hipLaunchKernelGGL((db_head_kernel<32, -1, -1>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace ppocr
