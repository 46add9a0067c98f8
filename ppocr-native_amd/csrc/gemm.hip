// Dense convolution as an implicit matrix product on FP32 MFMA (gfx950).
//
// Row m of the product is an output pixel of some lane (lanes stacked along
// M), column n an output channel. The reduction follows the plan's weight
// order [kh][kw][ic + n2][oc] (src/engine/plan.rs:83-86, shaders/gemm.comp:
// 2-18): taps in [ky][kx] order, in each tap the channels of every source in
// turn (up to four sources, each possibly a nearest upsampling by 2^shift
// folded in), zero outside the image. It runs in chunks of BK:
//  - channel layout (all sources' channels a multiple of 4): each tap's
//    channels padded to whole chunks, read four channels at a time;
//  - flat layout (other channel counts, e.g. an RGB stem): the whole
//    reduction taps * channels padded to whole chunks, read one at a time.
// The host packs the weights in the same padded order, one row of the
// reduction per output column, so a chunk of weights is one aligned run.
//
// A workgroup is four waves over a BM x BN tile (BM = 4 * WM); each wave owns
// WM rows and all BN columns as (WM/16) x (BN/16) tiles of
// v_mfma_f32_16x16x4_f32. Within a chunk, lane l (group g = l / 16) supplies
// reduction indices g*BK/4 .. g*BK/4 + BK/4 - 1, one per MFMA step, so each
// lane reads its operands with vector LDS loads. Operands sit in two LDS
// buffers of rows of BK + 4 floats: while the MFMAs consume one chunk, the
// next chunk's global loads are in flight and then stored to the other
// buffer, one barrier per chunk.
//
// Epilogues: bias, activation, then optionally a residual add and a second
// activation (an Add folded in); a transposed convolution's spread store; or
// the CTC head's per-row (max, sum of exp, first argmax) over the tile's
// columns, merged across tiles by ctc_merge, so the logits never reach memory.
#include "act.hpp"
#include "kernels.hpp"

namespace ppocr {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <int N>
struct VecT;
template <>
struct VecT<1> { typedef float T; };
template <>
struct VecT<2> { typedef f32x2 T; };
template <>
struct VecT<4> { typedef f32x4 T; };

struct CtcState {
  float m, s, b;
};

__device__ __forceinline__ void ctc_push(CtcState &st, float v, float col) {
  if (v > st.m) {
    st.s = st.s * exp_neg(st.m - v) + 1.0f;
    st.m = v;
    st.b = col;
  } else {
    st.s += exp_neg(v - st.m);
  }
}

__device__ __forceinline__ CtcState ctc_join(CtcState x, CtcState y) {
  const float ninf = -__builtin_inff();
  CtcState r;
  r.m = x.m > y.m ? x.m : y.m;
  float sx = x.m == ninf ? 0.0f : x.s * exp_neg(x.m - r.m);
  float sy = y.m == ninf ? 0.0f : y.s * exp_neg(y.m - r.m);
  r.s = sx + sy;
  r.b = x.m > y.m ? x.b : (y.m > x.m ? y.b : fminf(x.b, y.b));
  return r;
}

// The source holding channel c of a tap's concatenation.
__device__ __forceinline__ ConvSrc pick_src(const ConvArgs &a, int c) {
  ConvSrc s = a.src[0];
  if (a.nsrc > 1 && c >= a.src[1].coff) s = a.src[1];
  if (a.nsrc > 2 && c >= a.src[2].coff) s = a.src[2];
  if (a.nsrc > 3 && c >= a.src[3].coff) s = a.src[3];
  return s;
}

template <int WM, int BN, int BK, bool VEC, bool PW, bool CTC>
__global__ __launch_bounds__(256) void conv_mfma(ConvArgs a) {
  constexpr int BM = 4 * WM;
  constexpr int S = BK + 4;
  constexpr int KS = BK / 4;
  constexpr int KW = KS >= 4 ? 4 : KS;  // floats per LDS operand read
  constexpr int KR = KS / KW;           // operand reads per chunk
  constexpr int MT = WM / 16, NT = BN / 16;
  constexpr int AV = VEC ? 4 : 1;
  constexpr int A_KV = BK / AV;
  constexpr int A_ELEMS = BM * A_KV;
  constexpr int A_PER = (A_ELEMS + 255) / 256;
  constexpr int B_KV = BK / 4;
  constexpr int B_ELEMS = BN * B_KV;
  constexpr int B_PER = (B_ELEMS + 255) / 256;
  typedef typename VecT<AV>::T AT;
  typedef typename VecT<KW>::T KT;

  __shared__ __attribute__((aligned(16))) float As[2][BM * S];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * S];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per_lane = a.oh * a.ow;
  const int M = a.lanes * per_lane;
  const int ntn = (a.n + BN - 1) / BN;
  const int tn = blockIdx.x % ntn, tm = blockIdx.x / ntn;
  const int m0 = tm * BM, n0 = tn * BN;
  if (m0 >= M) return;

  // Rows this thread stages, decomposed once.
  int a_row[A_PER], a_kv[A_PER], a_lane[A_PER], a_y[A_PER], a_x[A_PER];
  bool a_ok[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; i++) {
    int e = tid + 256 * i;
    a_row[i] = e / A_KV;
    a_kv[i] = e % A_KV;
    int m = m0 + a_row[i];
    a_ok[i] = e < A_ELEMS && m < M;
    int mm = a_ok[i] ? m : 0;
    a_lane[i] = mm / per_lane;
    int rem = mm - a_lane[i] * per_lane;
    if (PW) {
      a_y[i] = rem;
      a_x[i] = 0;
    } else {
      int oy = rem / a.ow, ox = rem - oy * a.ow;
      a_y[i] = oy * a.sh - a.pt;
      a_x[i] = ox * a.sw - a.pl;
    }
  }
  const float *b_ptr[B_PER];
  int b_off[B_PER];
  bool b_ok[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; i++) {
    int e = tid + 256 * i;
    b_ok[i] = e < B_ELEMS;
    int nn = e / B_KV, kv = e % B_KV;
    b_off[i] = nn * S + kv * 4;
    b_ptr[i] = a.wt + (long)(n0 + (b_ok[i] ? nn : 0)) * a.wt_k + kv * 4;
  }

  AT ra[A_PER];
  f32x4 rb[B_PER];

  auto load = [&](int q) {
    int tap = 0, cbase = 0;
    if (VEC) {
      tap = q / a.cpt;
      cbase = (q - tap * a.cpt) * BK;
    }
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      int t = tap, c;
      if (VEC) {
        c = cbase + a_kv[i] * AV;
      } else {
        int k = q * BK + a_kv[i];
        t = k / a.ctot;
        c = k - t * a.ctot;
      }
      AT v;
      if constexpr (AV == 4) v = f32x4{0.f, 0.f, 0.f, 0.f};
      else v = 0.0f;
      bool live = a_ok[i] && c < a.ctot && t < a.kh * a.kw;
      if (PW) {
        if (live) {
          const ConvSrc &src = a.src[0];
          v = *reinterpret_cast<const AT *>(src.p + (long)a_lane[i] * src.lane_stride +
                                            (long)a_y[i] * src.c + c);
          if (a.gate) v = v * *reinterpret_cast<const AT *>(a.gate + (long)a_lane[i] * a.gate_lane_stride + c);
        }
      } else {
        int ky = t / a.kw, kx = t - ky * a.kw;
        int iy = a_y[i] + ky, ix = a_x[i] + kx;
        live = live && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
        if (live) {
          const ConvSrc src = pick_src(a, c);
          int cl = c - src.coff;
          long pix = (long)(iy >> src.shift) * (a.iw >> src.shift) + (ix >> src.shift);
          v = *reinterpret_cast<const AT *>(src.p + (long)a_lane[i] * src.lane_stride + pix * src.c + cl);
          if (a.gate && src.coff == 0)
            v = v * *reinterpret_cast<const AT *>(a.gate + (long)a_lane[i] * a.gate_lane_stride + cl);
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      if (b_ok[i]) rb[i] = *reinterpret_cast<const f32x4 *>(b_ptr[i] + (long)q * BK);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; i++)
      if (tid + 256 * i < A_ELEMS) *reinterpret_cast<AT *>(&As[buf][a_row[i] * S + a_kv[i] * AV]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_PER; i++)
      if (b_ok[i]) *reinterpret_cast<f32x4 *>(&Bs[buf][b_off[i]]) = rb[i];
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int li = lane & 15, lg = lane >> 4;
  load(0);
  store(0);
  __syncthreads();
  for (int q = 0; q < a.chunks; q++) {
    const int cur = q & 1;
    if (q + 1 < a.chunks) load(q + 1);
#pragma unroll
    for (int r = 0; r < KR; r++) {
      KT av[MT], bv[NT];
#pragma unroll
      for (int i = 0; i < MT; i++)
        av[i] = *reinterpret_cast<const KT *>(&As[cur][(wave * WM + i * 16 + li) * S + lg * KS + r * KW]);
#pragma unroll
      for (int j = 0; j < NT; j++)
        bv[j] = *reinterpret_cast<const KT *>(&Bs[cur][(j * 16 + li) * S + lg * KS + r * KW]);
#pragma unroll
      for (int k = 0; k < KW; k++) {
#pragma unroll
        for (int i = 0; i < MT; i++) {
#pragma unroll
          for (int j = 0; j < NT; j++) {
            float x, w;
            if constexpr (KW == 1) {
              x = av[i];
              w = bv[j];
            } else {
              x = av[i][k];
              w = bv[j][k];
            }
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, w, acc[i][j], 0, 0, 0);
          }
        }
      }
    }
    if (q + 1 < a.chunks) store(cur ^ 1);
    __syncthreads();
  }

  if constexpr (CTC) {
    // Per row: the tile's (max, sum of exp, first column of the max).
#pragma unroll
    for (int i = 0; i < MT; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        int m = m0 + wave * WM + i * 16 + lg * 4 + r;
        CtcState st{-__builtin_inff(), 0.0f, __builtin_inff()};
#pragma unroll
        for (int j = 0; j < NT; j++) {
          int n = n0 + j * 16 + li;
          if (n < a.vocab) ctc_push(st, acc[i][j][r] + a.bias[n], (float)n);
        }
#pragma unroll
        for (int d = 1; d < 16; d <<= 1) {
          CtcState o;
          o.m = __shfl_xor(st.m, d, 64);
          o.s = __shfl_xor(st.s, d, 64);
          o.b = __shfl_xor(st.b, d, 64);
          st = ctc_join(st, o);
        }
        if (li == 0 && m < M) {
          float4 *p = reinterpret_cast<float4 *>(a.part) + (long)m * ntn + tn;
          *p = make_float4(st.m, st.s, st.b, 0.0f);
        }
      }
    }
    return;
  } else {
#pragma unroll
    for (int i = 0; i < MT; i++) {
#pragma unroll
      for (int r = 0; r < 4; r++) {
        int m = m0 + wave * WM + i * 16 + lg * 4 + r;
        if (m >= M) continue;
        int ln = m / per_lane, rem = m - ln * per_lane;
#pragma unroll
        for (int j = 0; j < NT; j++) {
          int n = n0 + j * 16 + li;
          if (n >= a.n) continue;
          float v = acc[i][j][r];
          if (a.bias) v = v + a.bias[n];
          v = act(v, a.act);
          if (a.res) v = act(v + a.res[(long)ln * a.res_lane_stride + (long)rem * a.n + n], a.act2);
          long at;
          if (a.mode == GEMM_SPREAD) {
            int iy = rem / a.iw, ix = rem - iy * a.iw;
            int tap = n / a.spread_oc, o = n - tap * a.spread_oc;
            int ky = tap / a.spread_kw, kx = tap - ky * a.spread_kw;
            int kh = a.n / (a.spread_kw * a.spread_oc);
            long ow = (long)a.iw * a.spread_kw;
            at = ((long)(iy * kh + ky) * ow + (long)ix * a.spread_kw + kx) * a.spread_oc + o;
          } else {
            at = (long)rem * a.n + n;
          }
          a.y[(long)ln * a.y_lane_stride + at] = v;
        }
      }
    }
  }
}

// One wave per row: join the row's tile partials, then y = (best, 1 / sum).
__global__ __launch_bounds__(256) void ctc_merge(const float4 *part, int rows, int ntiles,
                                                 float *y, long y_lane_stride, int rows_per_lane) {
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  CtcState st{-__builtin_inff(), 0.0f, __builtin_inff()};
  for (int t = lane; t < ntiles; t += 64) {
    float4 p = part[(long)row * ntiles + t];
    st = ctc_join(st, CtcState{p.x, p.y, p.z});
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    CtcState o;
    o.m = __shfl_xor(st.m, d, 64);
    o.s = __shfl_xor(st.s, d, 64);
    o.b = __shfl_xor(st.b, d, 64);
    st = ctc_join(st, o);
  }
  if (lane == 0) {
    int ln = row / rows_per_lane, t = row - ln * rows_per_lane;
    float *out = y + (long)ln * y_lane_stride + 2 * t;
    out[0] = st.b;
    out[1] = 1.0f / st.s;
  }
}

template <int WM, int BN, int BK, bool VEC, bool PW, bool CTC>
static hipError_t go(const ConvArgs &a, hipStream_t s) {
  long M = (long)a.lanes * a.oh * a.ow;
  long tiles = (M + 4 * WM - 1) / (4 * WM) * ((a.n + BN - 1) / BN);
  if (tiles <= 0 || tiles > 0x7fffffffL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((conv_mfma<WM, BN, BK, VEC, PW, CTC>), dim3((unsigned)tiles), dim3(256), 0, s,
                     a);
  return hipGetLastError();
}

#define PPOCR_TILES(BK, VEC, PW)                                              \
  if (t.wm == 32 && t.bn == 64) return go<32, 64, BK, VEC, PW, false>(a, s); \
  if (t.wm == 32 && t.bn == 32) return go<32, 32, BK, VEC, PW, false>(a, s); \
  if (t.wm == 32 && t.bn == 16) return go<32, 16, BK, VEC, PW, false>(a, s); \
  if (t.wm == 16 && t.bn == 64) return go<16, 64, BK, VEC, PW, false>(a, s);

#define PPOCR_TILES_SMALL(BK, VEC, PW)                                        \
  if (t.wm == 16 && t.bn == 64) return go<16, 64, BK, VEC, PW, false>(a, s); \
  if (t.wm == 16 && t.bn == 32) return go<16, 32, BK, VEC, PW, false>(a, s); \
  if (t.wm == 16 && t.bn == 16) return go<16, 16, BK, VEC, PW, false>(a, s);

bool gemm_tile_supported(const GemmTile &t) {
  if (t.bk == 64) return t.vec && t.wm == 16 && (t.bn == 16 || t.bn == 32 || t.bn == 64);
  bool tile = (t.wm == 32 && (t.bn == 16 || t.bn == 32 || t.bn == 64)) || (t.wm == 16 && t.bn == 64);
  if (!tile) return false;
  if (t.vec) return t.bk == 8 || t.bk == 16 || t.bk == 32;
  return !t.pointwise && (t.bk == 8 || t.bk == 16 || t.bk == 32);
}

hipError_t launch_conv(const ConvArgs &a, const GemmTile &t, hipStream_t s) {
  if (a.mode == GEMM_CTC) {
    if (!t.pointwise || !t.vec || t.bn != 64) return hipErrorInvalidValue;
    if (t.wm == 32 && t.bk == 8) return go<32, 64, 8, true, true, true>(a, s);
    if (t.wm == 32 && t.bk == 16) return go<32, 64, 16, true, true, true>(a, s);
    return hipErrorInvalidValue;
  }
  if (!gemm_tile_supported(t)) return hipErrorInvalidValue;
  if (t.vec && t.pointwise) {
    if (t.bk == 64) { PPOCR_TILES_SMALL(64, true, true) }
    if (t.bk == 32) { PPOCR_TILES(32, true, true) }
    if (t.bk == 16) { PPOCR_TILES(16, true, true) }
    if (t.bk == 8) { PPOCR_TILES(8, true, true) }
  } else if (t.vec) {
    if (t.bk == 64) { PPOCR_TILES_SMALL(64, true, false) }
    if (t.bk == 32) { PPOCR_TILES(32, true, false) }
    if (t.bk == 16) { PPOCR_TILES(16, true, false) }
    if (t.bk == 8) { PPOCR_TILES(8, true, false) }
  } else {
    if (t.bk == 32) { PPOCR_TILES(32, false, false) }
    if (t.bk == 16) { PPOCR_TILES(16, false, false) }
    if (t.bk == 8) { PPOCR_TILES(8, false, false) }
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ctc_merge(const float *part, int rows, int ntiles, float *y, long y_lane_stride,
                            int rows_per_lane, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(ctc_merge, dim3((rows + 3) / 4), dim3(256), 0, s,
                     reinterpret_cast<const float4 *>(part), rows, ntiles, y, y_lane_stride,
                     rows_per_lane);
  return hipGetLastError();
}

}  // namespace ppocr
