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
#include <algorithm>

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

// The two largest of two (largest, second) pairs.
__device__ __forceinline__ void top2(float a1, float a2, float b1, float b2, float &m1, float &m2) {
  m1 = fmaxf(a1, b1);
  m2 = a1 > b1 ? fmaxf(a2, b1) : (b1 > a1 ? fmaxf(b2, a1) : a1);
}

// The source holding channel c of a tap's concatenation.
__device__ __forceinline__ ConvSrc pick_src(const ConvArgs &a, int c) {
  ConvSrc s = a.src[0];
  if (a.nsrc > 1 && c >= a.src[1].coff) s = a.src[1];
  if (a.nsrc > 2 && c >= a.src[2].coff) s = a.src[2];
  if (a.nsrc > 3 && c >= a.src[3].coff) s = a.src[3];
  return s;
}

// How a tile's A operand (the input patch of each row) is read.
//  L_FLAT: any channel count, one float at a time over taps * channels.
//  L_SOURCES: up to four sources (upsampled by 2^shift), four channels at a
//    time; the source of each channel is looked up per chunk.
//  L_WINDOW: one source at full resolution, kh, kw <= 8: each staged element
//    keeps a base pointer at its window's corner and a mask of the window rows
//    and columns inside the image; a chunk adds a uniform offset.
//  L_POINTWISE: 1x1 over one source (also the transposed conv's and the CTC
//    head's input): base pointer plus a uniform channel offset.
enum { L_FLAT = 0, L_SOURCES = 1, L_WINDOW = 2, L_POINTWISE = 3 };

// The CTC head's epilogue for one wave's MT row blocks x NT column blocks
// (rows from m_first, 16 a block; columns from n0): per row, the tile's
// (max, sum of exp, first column of the max, second value). Each lane takes
// the maximum of its NT columns (the first among equals: its columns rise
// with j); the 16 lanes of the row then join the maximum, the sum of
// exp(v - max) (hardware exp2, within 1 ulp: the sum is a probability's
// denominator, held to a tolerance) and the lowest column holding the
// maximum.
template <int CTRL>
__device__ __forceinline__ float dpp16(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Joins of the 16 lanes of a DPP row that leave the same bits in every lane:
// pairs within quads, then mirrored quads (lane i <-> 7 - i), then mirrored
// halves (lane i <-> 15 - i).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp16<0xB1>(v));
  v = fmaxf(v, dpp16<0x4E>(v));
  v = fmaxf(v, dpp16<0x141>(v));
  return fmaxf(v, dpp16<0x140>(v));
}
__device__ __forceinline__ float row16_min(float v) {
  v = fminf(v, dpp16<0xB1>(v));
  v = fminf(v, dpp16<0x4E>(v));
  v = fminf(v, dpp16<0x141>(v));
  return fminf(v, dpp16<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v = v + dpp16<0xB1>(v);
  v = v + dpp16<0x4E>(v);
  v = v + dpp16<0x141>(v);
  return v + dpp16<0x140>(v);
}

// A CTC tile's per-row statistics from its logits (acc + bias, columns past
// the vocabulary -inf): per row the maximum, the sum of exp(v - max) by
// hardware exp2, the first column holding the maximum and the second value,
// each the same in the 16 lanes of the row's DPP row, handed to `use` with
// the row's block and index in it.
template <int MT, int NT, typename Use>
__device__ __forceinline__ void ctc_tile_rows(const f32x4 (&acc)[MT][NT], int n0, const float *bias, int vocab,
                                              int lane, Use use) {
  const int li = lane & 15;
  constexpr float L = 1.44269504088896341f;  // log2(e)
  float bn[NT];  // this lane's columns' bias, once for the tile's rows
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int n = n0 + j * 16 + li;
    bn[j] = n < vocab ? bias[n] : 0.0f;
  }
#pragma unroll
  for (int i = 0; i < MT; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float v[NT];
      float lm = -__builtin_inff(), lb = __builtin_inff(), ls = -__builtin_inff();
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const int n = n0 + j * 16 + li;
        v[j] = n < vocab ? acc[i][j][r] + bn[j] : -__builtin_inff();
        if (v[j] > lm)
          ls = lm, lm = v[j], lb = (float)n;
        else if (v[j] > ls)
          ls = v[j];
      }
      const float gm = row16_max(lm);
      // The tile's second value (the maximum again when two columns hold
      // it), for the near-tie check of ctc_merge.
      float g2 = row16_max(lm == gm ? ls : lm);
      const unsigned long long held = __ballot(lm == gm);
      if (__popcll((held >> (lane & 48)) & 0xffffull) >= 2) g2 = gm;
      const float c = gm * L;
      float sum = 0.0f;
#pragma unroll
      for (int j = 0; j < NT; j++) sum += __builtin_amdgcn_exp2f(fmaf(v[j], L, -c));
      sum = row16_sum(sum);
      const float b = row16_min(lm == gm ? lb : __builtin_inff());
      use(i, r, make_float4(gm, sum, b, g2));
    }
  }
}

// One tile's per-row partials (max, sum of exp, first column of the max,
// second value) to `part`, row m's tile tn at m * ntn + tn.
template <int MT, int NT>
__device__ __forceinline__ void ctc_rows(const f32x4 (&acc)[MT][NT], int m_first, int M, int n0, const float *bias,
                                         int vocab, float *part, int ntn, int tn, int lane) {
  const int li = lane & 15, lg = lane >> 4;
  ctc_tile_rows<MT, NT>(acc, n0, bias, vocab, lane, [&](int i, int r, float4 rec) {
    const int m = m_first + i * 16 + lg * 4 + r;
    if (li == 0 && m < M) reinterpret_cast<float4 *>(part)[(long)m * ntn + tn] = rec;
  });
}

// A run's partial of one row joined with its next tile's (`y`, columns
// after x's; y's maximum is finite): the greater maximum, the sums rescaled
// to it by hardware exp2 (the sum only makes the probability, held to
// 1e-5 relative; the tiles' own sums use it too), the first column of the
// maximum, and the second value of the two.
__device__ __forceinline__ float4 ctc_join_partial(float4 x, float4 y) {
  constexpr float L = 1.44269504088896341f;  // log2(e)
  float m1, m2;
  top2(x.x, x.w, y.x, y.w, m1, m2);
  const float b = x.x > y.x ? x.z : (y.x > x.x ? y.z : fminf(x.z, y.z));
  const float s = x.x > y.x ? x.y + y.y * __builtin_amdgcn_exp2f((y.x - x.x) * L)
                            : y.y + x.y * __builtin_amdgcn_exp2f((x.x - y.x) * L);
  return make_float4(m1, s, b, m2);
}

template <int WM, int BN, int BK, int LAY, bool CTC>
__global__ __launch_bounds__(256) void conv_mfma(ConvArgs a) {
  constexpr bool VEC = LAY != L_FLAT;
  constexpr bool FAST = LAY == L_WINDOW || LAY == L_POINTWISE;
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
  const int tile = a.xcd_rows ? xcd_tile(blockIdx.x, gridDim.x) : blockIdx.x;
  const int tn = tile % ntn, tm = tile / ntn;
  const int m0 = tm * BM, n0 = tn * BN;
  if (m0 >= M) return;

  // Rows this thread stages, decomposed once.
  int a_row[A_PER], a_kv[A_PER], a_lane[A_PER], a_y[A_PER], a_x[A_PER];
  bool a_ok[A_PER];
  const float *a_base[FAST ? A_PER : 1];
  const float *g_base[FAST ? A_PER : 1];
  unsigned a_mask[LAY == L_WINDOW ? A_PER : 1];
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
    if (LAY == L_POINTWISE) {
      a_y[i] = rem;
      a_x[i] = 0;
    } else {
      int oy = rem / a.ow, ox = rem - oy * a.ow;
      a_y[i] = oy * a.sh - a.pt;
      a_x[i] = ox * a.sw - a.pl;
    }
    if constexpr (FAST) {
      const ConvSrc &src = a.src[0];
      long pix = LAY == L_POINTWISE ? (long)a_y[i] : (long)a_y[i] * a.iw + a_x[i];
      a_base[i] = src.p + (long)a_lane[i] * src.lane_stride + pix * src.c + a_kv[i] * 4;
      g_base[i] = a.gate ? a.gate + (long)a_lane[i] * a.gate_lane_stride + a_kv[i] * 4 : nullptr;
    }
    if constexpr (LAY == L_WINDOW) {
      unsigned ym = 0, xm = 0;
      for (int k = 0; k < a.kh; k++) ym |= (unsigned)(a_y[i] + k >= 0 && a_y[i] + k < a.ih) << k;
      for (int k = 0; k < a.kw; k++) xm |= (unsigned)(a_x[i] + k >= 0 && a_x[i] + k < a.iw) << k;
      a_mask[i] = a_ok[i] ? ym | xm << 8 : 0u;
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

  // The chunk being loaded: tap (ky, kx), channel chunk cc of that tap.
  int ky = 0, kx = 0, cc = 0;
  auto advance = [&]() {
    if (++cc == a.cpt) {
      cc = 0;
      if (++kx == a.kw) kx = 0, ++ky;
    }
  };

  auto load = [&](int q) {
    if constexpr (FAST) {
      const int cb = cc * BK;
      const long off = LAY == L_WINDOW ? (long)(ky * a.iw + kx) * a.src[0].c + cb : (long)cb;
      const int climit = a.ctot - cb;  // staged channel offsets below this are real
#pragma unroll
      for (int i = 0; i < A_PER; i++) {
        bool live = a_kv[i] * 4 < climit;
        if (LAY == L_WINDOW) live = live && ((a_mask[i] >> ky) & (a_mask[i] >> (8 + kx)) & 1u);
        else live = live && a_ok[i];
        f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
        if (live) {
          v = *reinterpret_cast<const f32x4 *>(a_base[i] + off);
          if (a.gate) v = v * *reinterpret_cast<const f32x4 *>(g_base[i] + cb);
        }
        ra[i] = v;
      }
    } else {
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
        int tky = t / a.kw, tkx = t - tky * a.kw;
        int iy = a_y[i] + tky, ix = a_x[i] + tkx;
        live = live && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
        if (live) {
          const ConvSrc src = pick_src(a, c);
          int cl = c - src.coff;
          long pix = (long)(iy >> src.shift) * (a.iw >> src.shift) + (ix >> src.shift);
          v = *reinterpret_cast<const AT *>(src.p + (long)a_lane[i] * src.lane_stride + pix * src.c + cl);
          if (a.gate && src.coff == 0)
            v = v * *reinterpret_cast<const AT *>(a.gate + (long)a_lane[i] * a.gate_lane_stride + cl);
        }
        ra[i] = v;
      }
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
  advance();
  store(0);
  __syncthreads();
  for (int q = 0; q < a.chunks; q++) {
    const int cur = q & 1;
    if (q + 1 < a.chunks) {
      load(q + 1);
      advance();
    }
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
    ctc_rows<MT, NT>(acc, m0 + wave * WM, M, n0, a.bias, a.vocab, a.part, ntn, tn, lane);
    return;
  } else if (MT == 1 && BN <= 32 && a.pw_w) {
    // The folded 1x1: each wave's 16 pixels x BN activated outputs go to
    // LDS (the operand stages are free) and return as the A operand of a
    // 16 x 16 x 4 chain over those BN channels against the 1x1's weights,
    // up to 32 output columns; bias and activation, then its store. The
    // launch checks the conditions (one column tile, no residual).
    constexpr int TP = BN + 4;
    float *T = &As[0][0] + wave * 16 * TP;
    const int K2 = a.n, N2 = a.pw_n;
    float w2[BN / 4][2];
#pragma unroll
    for (int s4 = 0; s4 < BN / 4; s4++)
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) {
        const int k = 4 * s4 + lg, c = j2 * 16 + li;
        w2[s4][j2] = k < K2 && c < N2 ? a.pw_w[(long)k * N2 + c] : 0.0f;
      }
#pragma unroll
    for (int j = 0; j < NT; j++) {
      const int n = j * 16 + li;
      const float bv = a.bias && n < a.n ? a.bias[n] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float v = 0.0f;
        if (n < a.n) {
          v = acc[0][j][r];
          if (a.bias) v = v + bv;
          v = act(v, a.act);
        }
        T[(lg * 4 + r) * TP + n] = v;
      }
    }
    __syncthreads();
    f32x4 acc2[2];
    acc2[0] = acc2[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s4 = 0; s4 < BN / 4; s4++) {
      const float x = T[li * TP + 4 * s4 + lg];
#pragma unroll
      for (int j2 = 0; j2 < 2; j2++) acc2[j2] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, w2[s4][j2], acc2[j2], 0, 0, 0);
    }
#pragma unroll
    for (int j2 = 0; j2 < 2; j2++) {
      const int c = j2 * 16 + li;
      if (c >= N2) continue;
      const float b2 = a.pw_b ? a.pw_b[c] : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int m = m0 + wave * WM + lg * 4 + r;
        if (m >= M) continue;
        const int ln = m / per_lane, rem = m - ln * per_lane;
        float v = acc2[j2][r];
        if (a.pw_b) v = v + b2;
        a.y[(long)ln * a.y_lane_stride + (long)rem * N2 + c] = act(v, a.pw_act);
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


// A windowed convolution (kh, kw <= 3, stride 1 or 2, one to four sources,
// upsampled by 2^shift, channels a multiple of 4) on tiles of the output:
// 16 pixels wide by 4 * WR rows of one lane, BN output channels. For each
// block of CB input channels the workgroup stages in LDS the input patch its
// window covers (the tile plus the halo) and the block's weights for every
// tap, then runs all taps from there: each input element is fetched, and its
// source and position decoded, once per block instead of once per tap.
// Channel blocks are the packed weights' chunks (BK = CB), so the reduction
// order is channel block, tap, then the block's channels in MFMA steps (r, k)
// of four, lane group g supplying channel 16r + 4g + k (CB >= 16); bias,
// activation, residual and the second activation as in conv_mfma's epilogue. Wave w owns output rows
// w * WR .. w * WR + WR - 1 of the tile, one 16 x 16 MFMA row block each.
// Registers a thread of conv_patch holds for the next channel block: patch
// float4s (its channel group of every 256 / (CB / 4)-th pixel) and weight
// float4s (taps x its column pairs).
constexpr int kPatchPer = 6;
constexpr int kPatchPerR8W1 = 4;
constexpr int kWeightPer = 9;

// LDS layout of conv_patch. A ds_read_b128 on gfx950 (measured) serves lanes
// 32h..32h+31 in two cycles of 16 lanes split by the parity of lane bits
// 2..4, over 64 banks of 4 bytes; lanes of one cycle that read different
// addresses in one bank conflict. A fragment read's lane (li, lg) reads pixel
// (or column) li at channel quad lg + 4r, so one cycle holds each li once,
// from two lane groups whose quads differ by one. Rows of patch_row floats
// (a stride of 2 mod 4 quads on stride-1 tiles, odd quads on stride-2 tiles,
// whose pixels are two rows apart) and columns patch_col_stride floats apart
// (2 mod 4 quads) put every such read in distinct banks; a store of eight
// consecutive lanes (one pixel's or one (column, tap)'s eight quads) meets
// none either.
__host__ __device__ inline int patch_row(int cb, int stride) {
  return cb + (cb >= 16 && stride == 1 ? 8 : 4);
}
__host__ __device__ inline int patch_col_stride(int taps, int row, int cb) {
  const int ns = taps * row;
  return cb >= 16 ? ns + 4 * ((2 - ns / 4) & 3) : ns;
}

// R8 (BN = 32, 17 to 24 output channels): the second column block holds at
// most 8 real columns, which run on v_mfma_f32_4x4x1f32 instead of a 16 x 16
// block three quarters padding. That instruction makes 16 independent 4 x 4
// products: block b takes the A operand of lanes 4b..4b+3 and the B operand
// of the same lanes, and lane 4b + j keeps column j of rows 0..3 in its four
// accumulators. The A operand is the main block's own (lane l: pixel l % 16
// at reduction index set l / 16), so block b covers pixels 4(b % 4)..+3 over
// the reduction indices of lane group b / 4, against columns 16 + 4c..+3
// (c = 0, 1: two instructions); the four lane groups' partial sums are added
// at the end ((p0 + p1) + (p2 + p3), the same bits in every lane).
__device__ __attribute__((aligned(16))) float kPatchZeros[4];

template <int WR, int BN, int CB, bool R8>
__device__ __forceinline__ void conv_patch_body(const Group<ConvArgs> &grp) {
  // Each XCD takes a contiguous run of tiles (xcd_tile): neighbouring tiles
  // share halo rows and columns, which then meet in one L2.
  const int bid = xcd_tile((int)blockIdx.x, (int)gridDim.x);
  int prob = 0;
#pragma unroll
  for (int k = 1; k < kGroupMax; k++)
    if (k < grp.n && bid >= grp.first[k]) prob = k;
  const ConvArgs &a = grp.a[prob];
  const int tiles_x = grp.x[prob], tiles_y = grp.y[prob];
  const int S = patch_row(CB, a.sw);  // LDS row of one pixel / one (n, tap)
  constexpr int KS = CB / 4;       // channels per lane group per tap
  constexpr int KW = KS >= 4 ? 4 : KS;
  constexpr int KR = KS / KW;
  static_assert(!R8 || BN == 32, "the 8-column remainder follows one 16-column block");
  constexpr int NT = R8 ? 1 : BN / 16;  // 16 x 16 column blocks
  constexpr int TH = 4 * WR, TW = 16;
  constexpr int CQ = CB / 4;       // float4 groups per pixel
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int taps = a.kh * a.kw;
  const int PR = (TH - 1) * a.sh + a.kh, PC = (TW - 1) * a.sw + a.kw;
  float *P = lds;                      // PR * PC pixels x S
  float *Bs = lds + PR * PC * S;       // nr columns NS apart (taps x S), then one zero row of S
  const int NS = patch_col_stride(taps, S, CB);

  const int ntn = (a.n + BN - 1) / BN;
  int t = bid - grp.first[prob];
  const int tn = t % ntn;
  t /= ntn;
  const int tx0 = (t % tiles_x) * TW;
  t /= tiles_x;
  const int ty0 = (t % tiles_y) * TH;
  const int ln = t / tiles_y;
  const int n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int iy0 = ty0 * a.sh - a.pt, ix0 = tx0 * a.sw - a.pl;
  // Columns of this tile that exist: only their weights are staged. The MFMA
  // lanes of the others only feed output columns that are never stored: past
  // the first block they read the staged column li (the same banks as the
  // real lanes of the first block, none of this block's), else the zero row.
  const int nr = min(BN, a.n - n0);
  float *Z = Bs + nr * NS;
  if (tid < S) Z[tid] = 0.0f;
  int bbase[NT], bstep[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int n = j * 16 + li;
    const int nn = n < nr ? n : (j > 0 && li < nr ? li : -1);
    bbase[j] = nn >= 0 ? nn * NS : nr * NS;
    bstep[j] = nn >= 0 ? S : 0;
  }
  // The channel offset of lane group g's quad of read r within a pixel row.
  auto quad = [&](int g, int r) { return KW == 4 ? r * 16 + g * 4 : g * KS + r * KW; };

  f32x4 acc[WR][NT];
#pragma unroll
  for (int i = 0; i < WR; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // R8: the remainder's columns 16 + 4c + lane % 4 and their accumulators.
  constexpr int NR = R8 ? 2 : 0;
  int rbase[R8 ? 2 : 1], rstep[R8 ? 2 : 1];
  f32x4 accr[WR][R8 ? 2 : 1];
  if constexpr (R8) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int n = 16 + 4 * c + (lane & 3);
      const int nn = n < nr ? n : (n - 16 < nr ? n - 16 : -1);
      rbase[c] = nn >= 0 ? nn * NS : nr * NS;
      rstep[c] = nn >= 0 ? S : 0;
#pragma unroll
      for (int i = 0; i < WR; i++) accr[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // Each thread stages one channel group q of every (256 / CQ)-th patch
  // pixel (at most kPatchPer of them), walking the pixels without divisions,
  // and one or two (column, channel group) pairs of the weights across every
  // tap (at most kWeightPer float4). The next channel block's values are
  // fetched into registers while this block's MFMAs run, then stored to LDS
  // once every wave is done reading it.
  constexpr int PSTEP = 256 / CQ;
  const int q = tid % CQ, p0 = tid / CQ;
  const int sy = PSTEP / PC, sx = PSTEP - sy * PC;
  const int npx = PR * PC;
  constexpr int PAIRS = BN * CQ;
  constexpr int PPAIRS = (PAIRS + 255) / 256;
  // R8 on one row block a wave: its patch takes at most kPatchPerR8W1
  // float4s a thread (the launch checks), which keeps the registers of the
  // remainder within three waves per SIMD.
  constexpr int PP = R8 && WR == 1 ? kPatchPerR8W1 : kPatchPer;
  f32x4 rp[PP], rw[kWeightPer];
  // Every load of a block is unconditional (a pixel outside the image or a
  // channel past ctot reads kPatchZeros; past the taps, a weight load
  // repeats the first tap), so that none waits at a branch; the gate
  // multiplies the block's image pixels as they are stored.
  f32x4 rg;
  unsigned rlive = 0;  // which of rp hold image pixels
  bool rgated = false;
  auto fetch = [&](int cc) {
    const int c = cc * CB + q * 4;
    const bool live_c = c < a.ctot;
    const ConvSrc src = pick_src(a, live_c ? c : 0);
    const int cl = c - src.coff, sh = src.shift, sw_ = a.iw >> sh;
    const float *base = src.p + (long)ln * src.lane_stride + cl;
    rgated = a.gate && src.coff == 0;
    rg = *reinterpret_cast<const f32x4 *>(rgated ? a.gate + (long)ln * a.gate_lane_stride + cl : kPatchZeros);
    rlive = 0;
    int py = p0 / PC, px = p0 - (p0 / PC) * PC;
#pragma unroll
    for (int k = 0; k < PP; k++) {
      const int iy = iy0 + py, ix = ix0 + px;
      const bool in = p0 + k * PSTEP < npx && live_c && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
      rp[k] = *reinterpret_cast<const f32x4 *>(in ? base + ((long)(iy >> sh) * sw_ + (ix >> sh)) * src.c
                                                  : kPatchZeros);
      rlive |= (in ? 1u : 0u) << k;
      px += sx, py += sy;
      if (px >= PC) px -= PC, py++;
    }
    const long wstep = (long)a.cpt * CB;
#pragma unroll
    for (int u = 0; u < PPAIRS; u++) {
      const int pr = tid + 256 * u;
      const int n = pr / CQ, qq = pr - n * CQ;
      const bool real = pr < PAIRS && n < nr;
      const float *wsrc = a.wt + (long)(n0 + (real ? n : 0)) * a.wt_k + (long)cc * CB + qq * 4;
#pragma unroll
      for (int tp = 0; tp < kWeightPer / PPAIRS; tp++)
        rw[u * (kWeightPer / PPAIRS) + tp] = *reinterpret_cast<const f32x4 *>(wsrc + (tp < taps ? tp : 0) * wstep);
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int k = 0; k < PP; k++)
      if (p0 + k * PSTEP < npx) {
        f32x4 v = rp[k];
        if (rgated && (rlive >> k & 1u)) v = v * rg;
        *reinterpret_cast<f32x4 *>(P + (p0 + k * PSTEP) * S + q * 4) = v;
      }
#pragma unroll
    for (int u = 0; u < PPAIRS; u++) {
      const int pr = tid + 256 * u;
      const int n = pr / CQ, qq = pr - n * CQ;
#pragma unroll
      for (int tp = 0; tp < kWeightPer / PPAIRS; tp++)
        if (pr < PAIRS && n < nr && tp < taps)
          *reinterpret_cast<f32x4 *>(Bs + n * NS + tp * S + qq * 4) = rw[u * (kWeightPer / PPAIRS) + tp];
    }
  };
  // The bias of this thread's output columns, requested with the first block.
  const float *bsrc = a.bias ? a.bias : kPatchZeros;
  float bcol[NT], brem[R8 ? 2 : 1];
#pragma unroll
  for (int j = 0; j < NT; j++) bcol[j] = bsrc[a.bias ? min(n0 + j * 16 + li, a.n - 1) : 0];
  if constexpr (R8) {
#pragma unroll
    for (int c = 0; c < NR; c++) brem[c] = bsrc[a.bias ? min(n0 + 16 + 4 * c + (li & 3), a.n - 1) : 0];
  }
  fetch(0);
  for (int cc = 0; cc < a.cpt; cc++) {
    if (cc) __syncthreads();  // every wave is done with the previous block
    store();
    __syncthreads();
    if (cc + 1 < a.cpt) fetch(cc + 1);
    // The next block's loads stay ahead of this block's multiply-adds (the
    // compiler would otherwise sink them below, to their use).
    asm volatile("" ::: "memory");
    // One tap: the window offset (ky, kx) into the staged patch. A 3 x 3
    // window runs its nine taps unrolled.
    auto tap = [&](int tp, int ky, int kx) {
#pragma unroll
      for (int r = 0; r < KR; r++) {
        typedef typename VecT<KW>::T KT;
        KT av[WR], bv[NT];
#pragma unroll
        for (int i = 0; i < WR; i++) {
          const int ty = wave * WR + i;
          const int pix = (ty * a.sh + ky) * PC + li * a.sw + kx;
          av[i] = *reinterpret_cast<const KT *>(P + pix * S + quad(lg, r));
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
          bv[j] = *reinterpret_cast<const KT *>(Bs + bbase[j] + tp * bstep[j] + quad(lg, r));
        KT br[R8 ? 2 : 1];
        if constexpr (R8) {
#pragma unroll
          for (int c = 0; c < NR; c++)
            br[c] = *reinterpret_cast<const KT *>(Bs + rbase[c] + tp * rstep[c] + quad(lg, r));
        }
#pragma unroll
        for (int k = 0; k < KW; k++) {
#pragma unroll
          for (int i = 0; i < WR; i++) {
            float x;
            if constexpr (KW == 1) x = av[i];
            else x = av[i][k];
#pragma unroll
            for (int j = 0; j < NT; j++) {
              float w;
              if constexpr (KW == 1) w = bv[j];
              else w = bv[j][k];
              acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, w, acc[i][j], 0, 0, 0);
            }
            if constexpr (R8) {
#pragma unroll
              for (int c = 0; c < NR; c++) {
                float w;
                if constexpr (KW == 1) w = br[c];
                else w = br[c][k];
                accr[i][c] = __builtin_amdgcn_mfma_f32_4x4x1f32(x, w, accr[i][c], 0, 0, 0);
              }
            }
          }
        }
      }
    };
    if (a.kh == 3 && a.kw == 3) {
#pragma unroll
      for (int tp = 0; tp < 9; tp++) tap(tp, tp / 3, tp % 3);
    } else {
      for (int tp = 0; tp < taps; tp++) tap(tp, tp / a.kw, tp % a.kw);
    }
  }

#pragma unroll
  for (int i = 0; i < WR; i++) {
    const int oy = ty0 + wave * WR + i;
    if (oy >= a.oh) continue;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int ox = tx0 + lg * 4 + r;
      if (ox >= a.ow) continue;
      const long rem = (long)oy * a.ow + ox;
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const int n = n0 + j * 16 + li;
        if (n >= a.n) continue;
        float v = acc[i][j][r];
        if (a.bias) v = v + bcol[j];
        v = act(v, a.act);
        if (a.res) v = act(v + a.res[(long)ln * a.res_lane_stride + rem * a.n + n], a.act2);
        a.y[(long)ln * a.y_lane_stride + rem * a.n + n] = v;
      }
    }
  }
  if constexpr (R8) {
    // The lane groups' partial sums, added the same way in every lane; then
    // lane group g stores row g of each 4 x 4 block: pixel 4 * (li / 4) + g,
    // column n0 + 16 + 4c + li % 4.
#pragma unroll
    for (int i = 0; i < WR; i++) {
      const int oy = ty0 + wave * WR + i;
#pragma unroll
      for (int c = 0; c < NR; c++) {
        f32x4 v = accr[i][c];
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = v[e] + __shfl_xor(v[e], 16);
#pragma unroll
        for (int e = 0; e < 4; e++) v[e] = v[e] + __shfl_xor(v[e], 32);
        const int ox = tx0 + 4 * (li >> 2) + lg, n = n0 + 16 + 4 * c + (li & 3);
        if (oy >= a.oh || ox >= a.ow || n >= a.n) continue;
        const long rem = (long)oy * a.ow + ox;
        float u = lg == 0 ? v[0] : (lg == 1 ? v[1] : (lg == 2 ? v[2] : v[3]));
        if (a.bias) u = u + brem[c];
        u = act(u, a.act);
        if (a.res) u = act(u + a.res[(long)ln * a.res_lane_stride + rem * a.n + n], a.act2);
        a.y[(long)ln * a.y_lane_stride + rem * a.n + n] = u;
      }
    }
  }
}

template <int WR, int BN, int CB, bool R8>
__global__ __launch_bounds__(256) void conv_patch(Group<ConvArgs> grp) {
  conv_patch_body<WR, BN, CB, R8>(grp);
}

// One row block a wave and up to 32 columns, with or without the 8-column
// remainder: held to three waves per SIMD (the occupancy its LDS leaves room
// for; 64 columns would spill).
template <int BN, int CB, bool R8>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void conv_patch_w1(Group<ConvArgs> grp) {
  conv_patch_body<1, BN, CB, R8>(grp);
}

// One wave per row: join the row's tile partials, then y = (best, 1 / sum).
// The tiles also carry their second value: when the row's two largest
// values lie within `tie` of each other, the GPU's summation order could
// have decided the argmax, so the wave recomputes the logits of every column
// of every tile whose maximum is that close, in the CPU's order (the bias,
// then a fused multiply-add per input in order, src/engine/layers.rs:770-776),
// and takes the first column of their maximum.
//
// `tie` bounds how far the two orders can put two columns' logits apart:
// each order computes bias + sum of ci products with at most n = ci + 1
// roundings, so each lies within n u T of the exact sum (u = 2^-24, T =
// |bias| + sum |w_i x_i| <= bias_max + wsum_max * max |x_i|), the two orders
// within 2 n u T of each other, and two columns' differences within 4 n u T.
// The test takes twice that (8 n u T, which also covers an accumulation that
// rounds toward zero), so columns further below the maximum on the GPU are
// below it in the CPU's order too.
constexpr float kCtcUnit = 1.0f / 16777216.0f;  // 2^-24


__global__ __launch_bounds__(256) void ctc_merge(const float4 *part, int rows, int ntiles, float *y,
                                                 long y_lane_stride, int rows_per_lane, CtcExact ex) {
  int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  int lane = threadIdx.x & 63;
  if (row >= rows) return;
  CtcState st{-__builtin_inff(), 0.0f, __builtin_inff()};
  float m2 = -__builtin_inff();
  for (int t = lane; t < ntiles; t += 64) {
    float4 p = part[(long)row * ntiles + t];
    float n1, n2;
    top2(st.m, m2, p.x, p.w, n1, n2);
    m2 = n2;
    st = ctc_join(st, CtcState{p.x, p.y, p.z});
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    CtcState o;
    o.m = __shfl_xor(st.m, d, 64);
    o.s = __shfl_xor(st.s, d, 64);
    o.b = __shfl_xor(st.b, d, 64);
    const float o2 = __shfl_xor(m2, d, 64);
    float n1, n2;
    top2(st.m, m2, o.m, o2, n1, n2);
    m2 = n2;
    st = ctc_join(st, o);
  }
  // Every lane holds the row's joined values: the check is uniform.
  const int ln = row / rows_per_lane, tr = row - ln * rows_per_lane;
  float best = st.b;
  const float *x = ex.x + (long)ln * ex.x_lane_stride + (long)tr * ex.ci;
  float xm = 0.0f;  // max |x_i| of the row, the same in every lane
  for (int i = lane; i < ex.ci; i += 64) xm = fmaxf(xm, fabsf(x[i]));
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) xm = fmaxf(xm, __shfl_xor(xm, d, 64));
  const float terms = ex.bias_max + ex.wsum_max * xm;
  const float tie = fmaxf(8.0f * float(ex.ci + 1) * kCtcUnit * terms * 1.0001f, 1e-30f);
  if (ex.wt && st.m - m2 <= tie) {
    // The candidate tiles' logits again, each column's multiply-adds in
    // channel order from its bias: 64-column chunks of the candidate tiles,
    // four at a time so that each lane runs four independent chains. The
    // lane keeps the greatest logit (the lowest column among equal ones);
    // the wave joins the lanes once at the end, the same total order.
    float bm = -__builtin_inff(), bb = __builtin_inff();
    int c0s[4] = {0, 0, 0, 0}, c1s[4] = {0, 0, 0, 0}, nq = 0;
    auto run = [&]() {
      float v[4];
      const float *w[4];
      bool ok[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int col = c0s[k] + lane;
        ok[k] = k < nq && col < c1s[k];
        const int cc = ok[k] ? col : 0;  // a valid row to read; the value is dropped
        w[k] = ex.wt + (long)cc * ex.wt_k;
        v[k] = ex.bias[cc];
      }
      int i = 0;
      for (; i + 4 <= ex.ci; i += 4) {
        const float x0 = x[i], x1 = x[i + 1], x2 = x[i + 2], x3 = x[i + 3];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const float4 wv = *reinterpret_cast<const float4 *>(w[k] + i);
          v[k] = fmaf(wv.x, x0, v[k]);
          v[k] = fmaf(wv.y, x1, v[k]);
          v[k] = fmaf(wv.z, x2, v[k]);
          v[k] = fmaf(wv.w, x3, v[k]);
        }
      }
      for (; i < ex.ci; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = fmaf(w[k][i], x[i], v[k]);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const float cb = (float)(c0s[k] + lane);
        if (ok[k] && (v[k] > bm || (v[k] == bm && cb < bb))) bm = v[k], bb = cb;
      }
      nq = 0;
    };
    for (int t = 0; t < ntiles; t++) {
      if (part[(long)row * ntiles + t].x < st.m - tie) continue;
      const int c1 = min((t + 1) * ex.tile_n, ex.vocab);
      for (int c0 = t * ex.tile_n; c0 < c1; c0 += 64) {
        // A record over several tiles: only its tiles whose own maximum is close.
        if (ex.tmax && ex.tmax[(long)(c0 / 64) * rows + row] < st.m - tie) continue;
        c0s[nq] = c0, c1s[nq] = min(c0 + 64, c1), nq++;
        if (nq == 4) run();
      }
    }
    if (nq) run();
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const float ov = __shfl_xor(bm, d, 64), ob = __shfl_xor(bb, d, 64);
      if (ov > bm || (ov == bm && ob < bb)) bm = ov, bb = ob;
    }
    best = bb;
  }
  if (lane == 0) {
    float *yp = y + (long)ln * y_lane_stride + 2L * tr;
    yp[0] = best;
    yp[1] = 1.0f / st.s;
  }
}

// ------------------------------------------------------------ CTC, panels

// The CTC head's GEMM when the head's input is at most 128 wide. A
// workgroup keeps 128 rows (eight waves of 16) in its operand registers for
// the whole launch and walks a run of 64-column tiles: each tile's weights
// (enc_pack order: four column blocks, 4 KB per group of 16 inputs) come
// from global memory straight into one of two LDS stages (direct loads, the
// next tile's in flight while the MFMAs run on this one), and every wave
// reads its B fragments from there, one 16-byte read per lane per block and
// group. Each row's partials are joined over runs of kCtcRunTiles tiles
// (in column order, in registers) and go to ctc_merge as one record per row
// and run, a sixth of the per-tile records; a workgroup walks one run or
// more, as many as the row count needs for about kCtcTarget workgroups. The
// workgroups of one run of columns take one XCD's consecutive slots, so the
// run's weights meet in that XCD's L2. Reduction order: groups of 16 inputs
// in order, within a group four steps of one input per lane group.
// Measured on 1280 x 18385 x 120: 16-row waves, eight a workgroup (96
// VGPRs, four waves a SIMD with two workgroups a CU; four waves of 32 rows:
// 71.4 us at two waves a SIMD; of 64 rows: 86 us, their 230 VGPRs leave one
// wave a SIMD) and about 512 workgroups (256: 88 us, 1024: 74 us, with four
// waves of 32 rows).
constexpr int kCtcRows = 128;             // rows a workgroup
constexpr int kCtcWaves = 8;              // waves a workgroup, 128 / (16 * kCtcWaves) row blocks each
constexpr int kCtcTarget = 512;           // workgroups a launch aims at
constexpr int kCtcRunTiles = 6;           // 64-column tiles a partial record joins

template <int KQ>
__global__ __launch_bounds__(64 * kCtcWaves) void ctc_panel(CtcDirectArgs a, int row_tiles, int per_run, int runs,
                                                            int per_group) {
  constexpr int W = kCtcWaves, MT = kCtcRows / (16 * W), NT = 4, STAGE = NT * KQ * 64 * 4;  // floats
  constexpr int TPI = NT * KQ * 64 / (64 * W);  // direct loads a thread issues a tile
  extern __shared__ __attribute__((aligned(16))) float bs[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const int M = a.rows_per_lane * a.lanes;
  const int ntn = (a.vocab + 63) / 64, nb = (a.vocab + 15) / 16;
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int tm = tile % row_tiles, group = tile / row_tiles;
  const int t0 = group * per_group * per_run, t1 = min(ntn, t0 + per_group * per_run);
  const int m0 = tm * kCtcRows + wave * 16 * MT;
  if (t0 >= t1) return;

  // A tile's weights into stage `st`: 8 * KQ 16-byte groups a thread,
  // blocks past the vocabulary read the last block (their columns are
  // masked in the epilogue).
  auto issue = [&](int t, int st) {
    const f32x4 *src = reinterpret_cast<const f32x4 *>(a.wt);
#pragma unroll
    for (int i = 0; i < TPI; i++) {
      const int e = i * 64 * W + tid;  // 16-byte group of the tile
      const int blk = min(t * 4 + e / (KQ * 64), nb - 1);
      const f32x4 *p = src + (long)blk * KQ * 64 + e % (KQ * 64);
      __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(bs + st * STAGE + (i * 64 * W + wave * 64) * 4),
                                       16, 0, 0);
    }
  };
  issue(t0, 0);

  // This lane's rows (past the last row: the last row, never stored), zero
  // past the input width.
  f32x4 av[MT][KQ];
#pragma unroll
  for (int i = 0; i < MT; i++) {
    const int m = min(m0 + 16 * i + li, M - 1);
    const int ln = m / a.rows_per_lane;
    const float *row = a.x + ln * a.x_lane_stride + (long)(m - ln * a.rows_per_lane) * a.ci;
#pragma unroll
    for (int q = 0; q < KQ; q++) {
      const int k = 16 * q + 4 * lg;
      av[i][q] = k < a.ci ? *reinterpret_cast<const f32x4 *>(row + k) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }

  // The run's per-tile records of the workgroup's rows, joined at its end.
  float4 *recs = reinterpret_cast<float4 *>(bs + 2 * STAGE);
  for (int t = t0; t < t1; t++) {
    const int st = (t - t0) & 1;
    // Every wave is done with the other stage (the tile before last).
    ring_barrier();
    if (t + 1 < t1) {
      issue(t + 1, st ^ 1);
      ring_wait<TPI>();
    } else {
      ring_wait<0>();
    }
    ring_barrier();  // this tile's weights have landed, from every wave
    f32x4 acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 *bl = reinterpret_cast<const f32x4 *>(bs + st * STAGE) + lane;
#pragma unroll
    for (int q = 0; q < KQ; q++) {
      f32x4 bv[NT];
#pragma unroll
      for (int j = 0; j < NT; j++) bv[j] = bl[(j * KQ + q) * 64];
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
          for (int j = 0; j < NT; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][q][e], bv[j][e], acc[i][j], 0, 0, 0);
    }
    const int k = t % per_run;
    ctc_tile_rows<MT, NT>(acc, t * 64, a.bias, a.vocab, lane, [&](int i, int r, float4 rec) {
      const int row = wave * 16 * MT + i * 16 + lg * 4 + r;
      if (li == 0) recs[row * per_run + k] = rec;
      if (li == 0 && a.tmax && m0 + i * 16 + lg * 4 + r < M) a.tmax[(long)t * M + m0 + i * 16 + lg * 4 + r] = rec.x;
    });
    // A run's last tile: each row's records joined in column order, one
    // record out. (The next tile's stores wait behind its first barrier.)
    if (k == per_run - 1 || t + 1 == t1) {
      __syncthreads();
      const int m = tm * kCtcRows + tid;
      if (tid < kCtcRows && m < M) {
        float4 run_rec = recs[tid * per_run];
        for (int q = 1; q <= k; q++) run_rec = ctc_join_partial(run_rec, recs[tid * per_run + q]);
        reinterpret_cast<float4 *>(a.part)[(long)m * runs + t / per_run] = run_rec;
      }
    }
  }
}

bool ctc_direct_supported(int ci) { return ci > 0 && ci <= 128 && ci % 4 == 0; }

CtcRuns ctc_direct_runs(long rows, int vocab) {
  const int row_tiles = (int)((rows + kCtcRows - 1) / kCtcRows), ntn = (vocab + 63) / 64;
  CtcRuns r;
  // The records' grouping of tiles is fixed, so that a row's joins, and so
  // its bits, do not depend on how many rows the launch has; how many
  // records a workgroup walks is what follows the row count: about
  // kCtcTarget workgroups (two a CU, each holding two 32 KB stages).
  r.per_run = std::min(kCtcRunTiles, ntn);
  r.runs = (ntn + r.per_run - 1) / r.per_run;
  r.columns = 64 * r.per_run;
  r.per_group = std::max(1, int((long(row_tiles) * r.runs + kCtcTarget - 1) / kCtcTarget));
  return r;
}

hipError_t launch_ctc_direct(const CtcDirectArgs &a, hipStream_t s) {
  if (!ctc_direct_supported(a.ci) || a.x_lane_stride % 4 || a.vocab <= 0) return hipErrorInvalidValue;
  const long M = (long)a.rows_per_lane * a.lanes;
  if (M <= 0 || M >= (1L << 31)) return hipErrorInvalidValue;
  const int row_tiles = (int)((M + kCtcRows - 1) / kCtcRows);
  const CtcRuns r = ctc_direct_runs(M, a.vocab);
  const int per_run = r.per_run, runs = r.runs;
  const unsigned blocks = (unsigned)(row_tiles * ((runs + r.per_group - 1) / r.per_group));
  const int kq = enc_kpad(a.ci) / 16;
  // Two weight stages, then the run's per-tile records.
  const size_t shm = (size_t)2 * 4 * kq * 64 * 16 + size_t(kCtcRows) * per_run * 16;
  auto go = [&](auto kernel) {
    if (shm > 64 * 1024) {
      hipError_t e = allow_lds(reinterpret_cast<const void *>(kernel), int(shm));
      if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(64 * kCtcWaves), shm, s, a, row_tiles, per_run, runs, r.per_group);
    return hipGetLastError();
  };
  switch (kq) {
    case 2: return go(ctc_panel<2>);
    case 4: return go(ctc_panel<4>);
    default: return go(ctc_panel<8>);
  }
}

// ------------------------------------------------------------ pointwise ring

// A 1x1 convolution (one source, channels a multiple of 4, optional gate on
// the input channels) as a GEMM whose operand tiles travel from global memory
// straight into a ring of LDS stages (global_load_lds_dwordx4: no registers,
// no store instructions), so that several chunks of BK channels are in
// flight while the MFMAs run on the oldest one. On small maps the
// register-staged kernel above waits out one load round trip per chunk; here
// the round trips overlap.
//
// Tile: BM = 32 * MT rows (pixels) x BN = 32 * NT columns, four waves as a
// 2 x 2 grid, each 16 * MT x 16 * NT. A stage holds the tile's A rows then
// its B rows (the packed weights' rows), BK floats each, row-major, with the
// 16-byte group g of row r stored at slot g ^ ring_swz(r) so that an MFMA
// fragment read (ds_read_b128) meets no bank conflict. Measured on gfx950:
// such a read serves lanes 32h..32h+31 in two cycles of 16 lanes, split by
// the parity of lane bits 2..4, over 64 banks of 4 bytes; conflicts are
// counted within a cycle. A fragment read's lane (li, lg) wants row li at
// group 4r + lg, and one cycle holds each li once, with lg = 2h or 2h + 1
// as the parity of li's bits 2..3 says. A direct
// load writes 64 lanes x 16 bytes contiguously from a wave-uniform LDS
// address, so each lane loads whichever global group belongs at its slot.
// Rows past the matrix and channels past ctot read kRingZeros. A GEMM of
// fewer chunks than stages uses (and is given LDS for) only as many stages
// as it has chunks.
//
// Reduction order: chunks of BK channels in order; within a chunk the MFMA
// chain takes groups of four channels lane group by lane group. Bias,
// activation, residual and second activation as in conv_mfma's epilogue.
__device__ __attribute__((aligned(16))) float kRingZeros[4];

static const size_t kMaxLdsBytes = 160 * 1024;

// The chunk width of a windowed convolution on the ring: the packer lays each
// tap's channels out in chunks of this many floats.
constexpr int kRingBK = 32;

template <int BK>
__device__ __forceinline__ int ring_swz(int row) {
  // Two rows of 32 floats span the 64 banks (row & 1 picks the half), so the
  // slot must differ over the eight rows of one parity in a cycle: row / 2,
  // flipped in bit 0 where the cycle's lane group does (bits 2 and 3 of row).
  if constexpr (BK == 32) return ((row >> 1) & 7) ^ (((row >> 2) ^ (row >> 3)) & 1);
  else return row & 15;
}

// Whether the ring's epilogue can store whole rows four floats at a time:
// every row, lane and residual offset a multiple of four floats.
__host__ __device__ inline bool ring_rows_store(const ConvArgs &a) {
  return a.n % 4 == 0 && a.y_lane_stride % 4 == 0 && (!a.res || a.res_lane_stride % 4 == 0);
}

template <int MT, int NT, int ST, int BK>
struct RingShape {
  static constexpr int BM = 32 * MT, BN = 32 * NT;
  static constexpr int G = BK / 4;            // 16-byte groups per row
  static constexpr int RPI = 64 / G;          // rows one direct load fills
  static constexpr int STAGE = (BM + BN) * BK;  // floats per stage
  static constexpr int A_I = BM / (4 * RPI), B_I = BN / (4 * RPI);  // direct loads per wave per chunk
  static constexpr int L = A_I + B_I;
  static_assert(BM % (4 * RPI) == 0 && BN % (4 * RPI) == 0, "whole loads per wave");
  static_assert(L * (ST - 1) < 64, "pending loads must fit vmcnt");
};


template <int MT, int NT, int ST, int BK, bool GATE, bool WIN>
__global__ __launch_bounds__(256) void conv_ring(Group<ConvArgs> grp) {
  typedef RingShape<MT, NT, ST, BK> R;
  const int prob = group_problem(grp);
  const ConvArgs &a = grp.a[prob];
  const int gate_lanes = grp.x[prob], stages = grp.y[prob];
  const int blk = (int)blockIdx.x - grp.first[prob], nblk = grp.first[prob + 1] - grp.first[prob];
  constexpr int BM = R::BM, BN = R::BN, STAGE = R::STAGE, L = R::L, G = R::G, RPI = R::RPI;
  extern __shared__ __attribute__((aligned(16))) float ring[];
  float *gs = ring + stages * STAGE;  // gate rows of the lanes the tile touches

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int per_lane = a.oh * a.ow;
  const int M = a.lanes * per_lane;
  const int ntn = (a.n + BN - 1) / BN;
  const int tile = a.xcd_rows ? xcd_tile(blk, nblk) : blk;
  const int tn = tile % ntn, tm = tile / ntn;
  const int m0 = tm * BM, n0 = tn * BN;
  if (m0 >= M) return;
  const int chunks = WIN ? a.chunks : (a.ctot + BK - 1) / BK;
  const int KP = chunks * BK;

  // The residual rows of the outputs this thread stores go out first, into
  // registers, so that their latency runs beside the operands'; then the
  // gate rows (zero past ctot) by direct loads into LDS, ahead of the
  // chunks, so that waiting for the first chunk also waits for them.
  const int lane0 = m0 / per_lane;
  constexpr int RV = MT * NT;  // residual float4s per thread
  const bool rows_store = a.mode == GEMM_STORE && ring_rows_store(a);
  f32x4 rv[RV];
  if (rows_store && a.res) {
    constexpr int CV = BN / 4;
#pragma unroll
    for (int i = 0; i < RV; i++) {
      const int e = tid + 256 * i, row = e / CV, c4 = e - row * CV;
      const int m = m0 + row, n = n0 + c4 * 4;
      rv[i] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (m < M && n < a.n) {
        const int ln = m / per_lane, rem = m - ln * per_lane;
        rv[i] = *reinterpret_cast<const f32x4 *>(a.res + (long)ln * a.res_lane_stride + (long)rem * a.n + n);
      }
    }
  }
  if constexpr (GATE) {
    const int kv = KP / 4, gslots = gate_lanes * kv;
    for (int q = wave; q * 64 < gslots; q += 4) {
      const int u = q * 64 + lane, l = u / kv, k = (u - l * kv) * 4;
      const float *p = l < gate_lanes && k < a.ctot && lane0 + l < a.lanes
                           ? a.gate + (long)(lane0 + l) * a.gate_lane_stride + k
                           : kRingZeros;
      __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(gs + q * 256), 16, 0, 0);
    }
  }

  // The global row and group each lane fetches for each of its direct loads.
  const int lrow = lane / G, lslot = lane % G;
  // Pointwise: the row's pointer at its group. Windowed: the row's lane and
  // window corner (a row past the matrix sits far outside the image).
  const float *a_src[R::A_I];
  int a_k[R::A_I], a_ln[WIN ? R::A_I : 1], a_y[WIN ? R::A_I : 1], a_x[WIN ? R::A_I : 1];
#pragma unroll
  for (int i = 0; i < R::A_I; i++) {
    const int r = (i * 4 + wave) * RPI + lrow;
    const int m = m0 + r;
    const int g = lslot ^ ring_swz<BK>(r);
    a_k[i] = g * 4;
    const int ln = m / per_lane, px = m - ln * per_lane;
    if constexpr (WIN) {
      const int oy = px / a.ow, ox = px - oy * a.ow;
      a_ln[i] = ln;
      a_y[i] = m < M ? oy * a.sh - a.pt : -(1 << 20);
      a_x[i] = ox * a.sw - a.pl;
      a_src[i] = nullptr;
    } else {
      a_src[i] = m < M ? a.src[0].p + (long)ln * a.src[0].lane_stride + (long)px * a.ctot + g * 4 : nullptr;
    }
  }
  const float *b_src[R::B_I];
  int b_k[R::B_I];
#pragma unroll
  for (int i = 0; i < R::B_I; i++) {
    const int r = (i * 4 + wave) * RPI + lrow;
    const int n = n0 + r;
    const int g = lslot ^ ring_swz<BK>(r);
    b_k[i] = g * 4;
    b_src[i] = n < a.n ? a.wt + (long)n * a.wt_k + g * 4 : nullptr;
  }

  // The fields the loads test, read once: `a` lives in the kernel
  // arguments, which the compiler would otherwise read again for every
  // chunk (its direct loads write memory), waiting on each read.
  const int ctot = a.ctot, ih = a.ih, iw = a.iw, cpt = a.cpt, kw = a.kw;
  auto issue = [&](int q, int st) {
    const int k0 = q * BK;
    float *base = ring + st * STAGE;
    // Windowed: chunk q is channel block cc of tap (ky, kx).
    int ky = 0, kx = 0, cb = 0;
    if constexpr (WIN) {
      const int tap = q / cpt;
      cb = (q - tap * cpt) * BK;
      ky = tap / kw;
      kx = tap - ky * kw;
    }
#pragma unroll
    for (int i = 0; i < R::A_I; i++) {
      const float *p = kRingZeros;
      if constexpr (WIN) {
        const int c = cb + a_k[i], iy = a_y[i] + ky, ix = a_x[i] + kx;
        if (c < ctot && iy >= 0 && iy < ih && ix >= 0 && ix < iw) {
          const ConvSrc s = pick_src(a, c);
          const long pix = (long)(iy >> s.shift) * (iw >> s.shift) + (ix >> s.shift);
          p = s.p + (long)a_ln[i] * s.lane_stride + pix * s.c + (c - s.coff);
        }
      } else {
        if (a_src[i] && k0 + a_k[i] < ctot) p = a_src[i] + k0;
      }
      __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(base + (i * 4 + wave) * RPI * BK), 16, 0, 0);
    }
    // The packed rows are zero past each tap's channels.
#pragma unroll
    for (int i = 0; i < R::B_I; i++) {
      const float *p = b_src[i] && (WIN || k0 + b_k[i] < ctot) ? b_src[i] + k0 : kRingZeros;
      __builtin_amdgcn_global_load_lds((const void *)p, (lds_void *)(base + (BM + (i * 4 + wave) * RPI) * BK), 16,
                                       0, 0);
    }
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int li = lane & 15, lg = lane >> 4;
  int ar[MT], asw[MT], arel[MT];
#pragma unroll
  for (int i = 0; i < MT; i++) {
    ar[i] = wm * 16 * MT + i * 16 + li;
    asw[i] = ring_swz<BK>(ar[i]);
    const int m = min(m0 + ar[i], M - 1);
    arel[i] = min(m / per_lane - lane0, gate_lanes - 1);
  }
  int br[NT], bsw[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    br[j] = wn * 16 * NT + j * 16 + li;
    bsw[j] = ring_swz<BK>(br[j]);
    br[j] += BM;
  }

#pragma unroll
  for (int s = 0; s < ST - 1; s++)
    if (s < chunks) issue(s, s);


  for (int q = 0; q < chunks; q++) {
    // Chunk q is complete once no more than the later chunks' loads are
    // pending; the barrier then also frees the stage chunk q - 1 used.
    ring_wait_chunks<L, ST - 2>(min(ST - 2, chunks - 1 - q));
    ring_barrier();
    if (q + ST - 1 < chunks) issue(q + ST - 1, (q + ST - 1) % ST);
    const float *base = ring + (q % ST) * STAGE;
#pragma unroll
    for (int r = 0; r < BK / 16; r++) {
      const int g = r * 4 + lg;
      f32x4 av[MT], bv[NT];
#pragma unroll
      for (int i = 0; i < MT; i++) {
        av[i] = *reinterpret_cast<const f32x4 *>(base + ar[i] * BK + (g ^ asw[i]) * 4);
        if constexpr (GATE) av[i] = av[i] * *reinterpret_cast<const f32x4 *>(gs + arel[i] * KP + q * BK + g * 4);
      }
#pragma unroll
      for (int j = 0; j < NT; j++) bv[j] = *reinterpret_cast<const f32x4 *>(base + br[j] * BK + (g ^ bsw[j]) * 4);
#pragma unroll
      for (int k = 0; k < 4; k++)
#pragma unroll
        for (int i = 0; i < MT; i++)
#pragma unroll
          for (int j = 0; j < NT; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][k], bv[j][k], acc[i][j], 0, 0, 0);
    }
  }

  // Bias per column once; rows and columns past the matrix store nothing.
  float bias_v[NT];
  int col[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    col[j] = n0 + wn * 16 * NT + j * 16 + li;
    bias_v[j] = a.bias && col[j] < a.n ? a.bias[col[j]] : 0.0f;
  }
  if (a.mode == GEMM_STORE && ring_rows_store(a)) {
    // Through LDS: the tile, after bias and activation, row-major (rows
    // padded by 4 so that the four row groups of a store land in distinct
    // banks); then each thread stores four consecutive outputs of a row,
    // with the residual and second activation, so a wave writes whole rows.
    constexpr int TS = BN + 4;
    __syncthreads();  // every wave is done with the ring
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
          float v = acc[i][j][r];
          if (a.bias) v = v + bias_v[j];
          ring[(wm * 16 * MT + i * 16 + lg * 4 + r) * TS + wn * 16 * NT + j * 16 + li] = act(v, a.act);
        }
    __syncthreads();
    constexpr int CV = BN / 4;
    static_assert(BM * CV == 256 * RV, "one residual float4 per thread and store");
#pragma unroll
    for (int i = 0; i < RV; i++) {
      const int e = tid + 256 * i, row = e / CV, c4 = e - row * CV;
      const int m = m0 + row, n = n0 + c4 * 4;
      if (m >= M || n >= a.n) continue;
      const int ln = m / per_lane, rem = m - ln * per_lane;
      f32x4 v = *reinterpret_cast<const f32x4 *>(ring + row * TS + c4 * 4);
      if (a.res) {
        v.x = act(v.x + rv[i].x, a.act2);
        v.y = act(v.y + rv[i].y, a.act2);
        v.z = act(v.z + rv[i].z, a.act2);
        v.w = act(v.w + rv[i].w, a.act2);
      }
      *reinterpret_cast<f32x4 *>(a.y + (long)ln * a.y_lane_stride + (long)rem * a.n + n) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < MT; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int m = m0 + wm * 16 * MT + i * 16 + lg * 4 + r;
      const int ln = m / per_lane, rem = m - ln * per_lane;
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const int n = col[j];
        if (m < M && n < a.n) {
          float v = acc[i][j][r];
          if (a.bias) v = v + bias_v[j];
          v = act(v, a.act);
          if (a.res) v = act(v + a.res[(long)ln * a.res_lane_stride + (long)rem * a.n + n], a.act2);
          long at;
          if (a.mode == GEMM_SPREAD) {
            const int iy = rem / a.iw, ix = rem - iy * a.iw;
            const int tap = n / a.spread_oc, o = n - tap * a.spread_oc;
            const int ky = tap / a.spread_kw, kx = tap - ky * a.spread_kw;
            const int kh = a.n / (a.spread_kw * a.spread_oc);
            const long ow = (long)a.iw * a.spread_kw;
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

// Lanes whose gate rows a tile of bm rows can touch.
static int ring_gate_lanes(const ConvArgs &a, int bm) {
  const long per_lane = (long)a.oh * a.ow;
  return (int)std::min<long>(a.lanes, bm / per_lane + 2);
}

// Whether the ring runs a windowed convolution (implicit GEMM over taps).
static bool ring_window(const ConvArgs &a) { return a.kh != 1 || a.kw != 1 || a.nsrc != 1 || a.sh != 1 || a.sw != 1; }

static int ring_chunks(const ConvArgs &a, int bk) {
  return ring_window(a) ? a.chunks : (a.ctot + bk - 1) / bk;
}

// Stages a GEMM uses: its chunk count when below the ring's.
static int ring_stages(const ConvArgs &a, int st, int bk) { return std::min(st, ring_chunks(a, bk)); }

static size_t ring_lds(const ConvArgs &a, int mt, int nt, int st, int bk) {
  const int bm = 32 * mt, bn = 32 * nt, kp = ring_chunks(a, bk) * bk;
  size_t b = (size_t)ring_stages(a, st, bk) * (bm + bn) * bk * sizeof(float);
  if (a.mode == GEMM_STORE && ring_rows_store(a)) b = std::max(b, (size_t)bm * (bn + 4) * sizeof(float));
  // Gate rows by whole direct loads of 64 16-byte slots.
  if (a.gate) b += ((size_t)ring_gate_lanes(a, bm) * (kp / 4) + 63) / 64 * 64 * 16;
  return b;
}

template <int MT, int NT, int ST, int BK, bool GATE, bool WIN>
static hipError_t go_ring1(const ConvArgs *as, int n, hipStream_t s) {
  typedef RingShape<MT, NT, ST, BK> R;
  Group<ConvArgs> grp{};
  grp.n = n;
  long total = 0;
  size_t lds = 0;
  for (int p = 0; p < n; p++) {
    const ConvArgs &a = as[p];
    const long M = (long)a.lanes * a.oh * a.ow;
    const long tiles = (M + R::BM - 1) / R::BM * ((a.n + R::BN - 1) / R::BN);
    if (tiles <= 0) return hipErrorInvalidValue;
    grp.first[p] = (int)total;
    total += tiles;
    if (total > 0x7fffffffL) return hipErrorInvalidValue;
    grp.x[p] = ring_gate_lanes(a, R::BM);
    grp.y[p] = ring_stages(a, ST, BK);
    grp.a[p] = a;
    lds = std::max(lds, ring_lds(a, MT, NT, ST, BK));
  }
  grp.first[n] = (int)total;
  if (lds > kMaxLdsBytes) return hipErrorInvalidValue;
  if (lds > 64 * 1024) {
    hipError_t e = allow_lds(reinterpret_cast<const void *>(conv_ring<MT, NT, ST, BK, GATE, WIN>), (int)kMaxLdsBytes);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL((conv_ring<MT, NT, ST, BK, GATE, WIN>), dim3((unsigned)total), dim3(256), lds, s, grp);
  return hipGetLastError();
}

template <int MT, int NT, int ST, int BK>
static hipError_t go_ring(const ConvArgs *as, int n, hipStream_t s) {
  if (ring_window(as[0])) return go_ring1<MT, NT, ST, BK, false, true>(as, n, s);
  return as[0].gate ? go_ring1<MT, NT, ST, BK, true, false>(as, n, s)
                    : go_ring1<MT, NT, ST, BK, false, false>(as, n, s);
}

bool ring_supported(const ConvArgs &a) {
  if (a.mode != GEMM_STORE && a.mode != GEMM_SPREAD) return false;
  if (a.ctot % 4 != 0) return false;
  if (!ring_window(a))
    return a.nsrc == 1 && a.src[0].shift == 0 && a.ctot == a.src[0].c && a.oh == a.ih && a.ow == a.iw &&
           a.pt == 0 && a.pl == 0;
  // Windowed: GEMM_STORE, no gate, every source's channels a multiple of 4,
  // weights packed per tap in chunks of kRingBK.
  if (a.mode != GEMM_STORE || a.gate || a.nsrc < 1 || a.nsrc > 4) return false;
  for (int k = 0; k < a.nsrc; k++)
    if (a.src[k].c % 4 != 0 || a.src[k].coff % 4 != 0) return false;
  const int cpt = (a.ctot + kRingBK - 1) / kRingBK;
  return a.cpt == cpt && a.chunks == a.kh * a.kw * cpt && a.wt_k == (long)a.chunks * kRingBK;
}

bool ring_fits(const ConvArgs &a, const RingTile &t) {
  return ring_lds(a, t.mt, t.nt, t.st, t.bk) <= kMaxLdsBytes;
}

size_t ring_lds_bytes(const ConvArgs &a, const RingTile &t) { return ring_lds(a, t.mt, t.nt, t.st, t.bk); }

#define PPOCR_RING(MT, NT, ST, BK) \
  if (t.mt == MT && t.nt == NT && t.st == ST && t.bk == BK) return go_ring<MT, NT, ST, BK>(as, n, s);

// The tiles compiled (ring_tile in the model picks among them).
#define PPOCR_RING_TILES                                                                         \
  PPOCR_RING(1, 1, 2, 32) PPOCR_RING(1, 1, 3, 32) PPOCR_RING(1, 1, 4, 32) PPOCR_RING(1, 2, 2, 32) \
  PPOCR_RING(1, 2, 3, 32) PPOCR_RING(1, 2, 4, 32) PPOCR_RING(1, 3, 2, 32) PPOCR_RING(1, 3, 3, 32) \
  PPOCR_RING(1, 3, 4, 32)

hipError_t launch_conv_ring_group(const ConvArgs *as, int n, const RingTile &t, hipStream_t s) {
  if (n < 1 || n > kGroupMax) return hipErrorInvalidValue;
  for (int p = 0; p < n; p++)
    if (!ring_supported(as[p]) || !ring_fits(as[p], t) || ring_window(as[p]) != ring_window(as[0]) ||
        (as[p].gate != nullptr) != (as[0].gate != nullptr))
      return hipErrorInvalidValue;
  PPOCR_RING_TILES
  return hipErrorInvalidValue;
}

hipError_t launch_conv_ring(const ConvArgs &a, const RingTile &t, hipStream_t s) {
  return launch_conv_ring_group(&a, 1, t, s);
}

template <int WM, int BN, int BK, int LAY, bool CTC>
static hipError_t go(const ConvArgs &a, hipStream_t s) {
  long M = (long)a.lanes * a.oh * a.ow;
  long tiles = (M + 4 * WM - 1) / (4 * WM) * ((a.n + BN - 1) / BN);
  if (tiles <= 0 || tiles > 0x7fffffffL) return hipErrorInvalidValue;
  hipLaunchKernelGGL((conv_mfma<WM, BN, BK, LAY, CTC>), dim3((unsigned)tiles), dim3(256), 0, s,
                     a);
  return hipGetLastError();
}

#define PPOCR_TILES(BK, LAY)                                               \
  if (t.wm == 32 && t.bn == 64) return go<32, 64, BK, LAY, false>(a, s); \
  if (t.wm == 32 && t.bn == 32) return go<32, 32, BK, LAY, false>(a, s); \
  if (t.wm == 32 && t.bn == 16) return go<32, 16, BK, LAY, false>(a, s); \
  if (t.wm == 16 && t.bn == 64) return go<16, 64, BK, LAY, false>(a, s); \
  if (t.wm == 16 && t.bn == 32) return go<16, 32, BK, LAY, false>(a, s); \
  if (t.wm == 16 && t.bn == 16) return go<16, 16, BK, LAY, false>(a, s);

#define PPOCR_TILES_SMALL(BK, LAY)                                         \
  if (t.wm == 16 && t.bn == 64) return go<16, 64, BK, LAY, false>(a, s); \
  if (t.wm == 16 && t.bn == 32) return go<16, 32, BK, LAY, false>(a, s); \
  if (t.wm == 16 && t.bn == 16) return go<16, 16, BK, LAY, false>(a, s);

#define PPOCR_CHUNKS(LAY)                               \
  if (t.bk == 64) { PPOCR_TILES_SMALL(64, LAY) }        \
  if (t.bk == 32) { PPOCR_TILES(32, LAY) }              \
  if (t.bk == 16) { PPOCR_TILES(16, LAY) }              \
  if (t.bk == 8) { PPOCR_TILES(8, LAY) }

bool conv_pw_supported(const ConvArgs &a, const GemmTile &t) {
  // One tile's columns are every output column (a 16 x 16 x 4 chain over
  // them), 16-row MFMA blocks a wave, the LDS stages large enough to hold
  // four waves' 16 x (BN + 4) floats, no residual.
  return a.mode == GEMM_STORE && !a.res && t.wm == 16 && (t.bn == 16 || t.bn == 32) && a.n <= t.bn && t.bk >= 16 &&
         a.pw_n >= 1 && a.pw_n <= 32;
}

bool gemm_tile_supported(const GemmTile &t) {
  if (t.bk == 64) return t.vec && t.wm == 16 && (t.bn == 16 || t.bn == 32 || t.bn == 64);
  // One chunk per tap of 48 or 96 channels: windowed, 64-row tiles.
  if (t.bk == 48 || t.bk == 96)
    return t.vec && !t.pointwise && t.wm == 16 && (t.bn == 16 || t.bn == 32 || t.bn == 64);
  bool tile = (t.wm == 32 || t.wm == 16) && (t.bn == 16 || t.bn == 32 || t.bn == 64);
  if (!tile) return false;
  if (t.vec) return t.bk == 8 || t.bk == 16 || t.bk == 32;
  return !t.pointwise && (t.bk == 8 || t.bk == 16 || t.bk == 32);
}

hipError_t launch_conv(const ConvArgs &a, const GemmTile &t, hipStream_t s) {
  if (a.pw_w && !conv_pw_supported(a, t)) return hipErrorInvalidValue;
  if (a.mode == GEMM_CTC) {
    if (!t.pointwise || !t.vec || t.bn != 64) return hipErrorInvalidValue;
    if (t.wm == 32 && t.bk == 8) return go<32, 64, 8, L_POINTWISE, true>(a, s);
    if (t.wm == 32 && t.bk == 16) return go<32, 64, 16, L_POINTWISE, true>(a, s);
    return hipErrorInvalidValue;
  }
  if (!gemm_tile_supported(t)) return hipErrorInvalidValue;
  if (!t.vec) {
    if (t.bk == 32) { PPOCR_TILES(32, L_FLAT) }
    if (t.bk == 16) { PPOCR_TILES(16, L_FLAT) }
    if (t.bk == 8) { PPOCR_TILES(8, L_FLAT) }
  } else if (t.pointwise) {
    if (a.nsrc != 1 || a.src[0].shift != 0 || a.ctot != a.src[0].c) return hipErrorInvalidValue;
    PPOCR_CHUNKS(L_POINTWISE)
  } else if (a.nsrc == 1 && a.src[0].shift == 0 && a.kh <= 8 && a.kw <= 8) {
    if (t.bk == 96) { PPOCR_TILES_SMALL(96, L_WINDOW) }
    if (t.bk == 48) { PPOCR_TILES_SMALL(48, L_WINDOW) }
    PPOCR_CHUNKS(L_WINDOW)
  } else {
    if (t.bk == 96) { PPOCR_TILES_SMALL(96, L_SOURCES) }
    if (t.bk == 48) { PPOCR_TILES_SMALL(48, L_SOURCES) }
    PPOCR_CHUNKS(L_SOURCES)
  }
  return hipErrorInvalidValue;
}

bool patch_fits(int kh, int kw, int stride, int wr, int bk, int bn) {
  if (kh < 1 || kw < 1 || kh > 3 || kw > 3 || (stride != 1 && stride != 2) || (wr != 1 && wr != 2)) return false;
  if ((bk != 8 && bk != 16 && bk != 32) || (bn != 16 && bn != 32 && bn != 64)) return false;
  // What one thread holds for the next channel block must fit its registers.
  const int cq = bk / 4, pstep = 256 / cq, pairs = (bn * cq + 255) / 256;
  const int pr = (4 * wr - 1) * stride + kh, pc = 15 * stride + kw;
  if ((pr * pc + pstep - 1) / pstep > kPatchPer) return false;
  if (kWeightPer % pairs || kh * kw > kWeightPer / pairs) return false;
  const int row = patch_row(bk, stride);
  return (size_t(pr * pc + 1) * row + size_t(bn) * patch_col_stride(kh * kw, row, bk)) * sizeof(float) <= 160 * 1024;
}

bool patch_supported(const ConvArgs &a, int wr, int bk, int bn) {
  if (a.mode != GEMM_STORE || a.sh != a.sw) return false;
  for (int k = 0; k < a.nsrc; k++)
    if (a.src[k].c % 4 || a.src[k].coff % 4) return false;
  return patch_fits(a.kh, a.kw, a.sh, wr, bk, bn);
}

size_t patch_lds_bytes(const ConvArgs &a, int wr, int bk, int bn) {
  const size_t pr = size_t(4 * wr - 1) * a.sh + a.kh, pc = size_t(15) * a.sw + a.kw;
  const size_t nr = size_t(std::min(bn, a.n));  // staged columns; the zero row besides
  const int row = patch_row(bk, a.sw);
  return ((pr * pc + 1) * row + nr * patch_col_stride(a.kh * a.kw, row, bk)) * sizeof(float);
}

template <int WR, int BN, int CB, bool R8 = false>
static hipError_t go_patch(const ConvArgs *as, int n, hipStream_t s) {
  const void *kernel;
  if constexpr (WR == 1 && BN <= 32) kernel = reinterpret_cast<const void *>(conv_patch_w1<BN, CB, R8>);
  else kernel = reinterpret_cast<const void *>(conv_patch<WR, BN, CB, R8>);
  constexpr int TH = 4 * WR;
  Group<ConvArgs> grp{};
  grp.n = n;
  long blocks = 0;
  size_t shm = 0;
  for (int p = 0; p < n; p++) {
    const ConvArgs &a = as[p];
    const long tiles_x = (a.ow + 15) / 16, tiles_y = (a.oh + TH - 1) / TH;
    const long ntn = (a.n + BN - 1) / BN;
    const long nb = (long)a.lanes * tiles_y * tiles_x * ntn;
    if (nb <= 0) return hipErrorInvalidValue;
    grp.first[p] = (int)blocks;
    blocks += nb;
    if (blocks > 0x7fffffffL) return hipErrorInvalidValue;
    grp.x[p] = (int)tiles_x, grp.y[p] = (int)tiles_y;
    grp.a[p] = a;
    shm = std::max(shm, patch_lds_bytes(a, WR, CB, BN));
  }
  grp.first[n] = (int)blocks;
  if (shm > 160 * 1024) return hipErrorInvalidValue;
  if (shm > 64 * 1024) {
    hipError_t e = allow_lds(kernel, 160 * 1024);
    if (e != hipSuccess) return e;
  }
  if constexpr (WR == 1 && BN <= 32)
    hipLaunchKernelGGL((conv_patch_w1<BN, CB, R8>), dim3((unsigned)blocks), dim3(256), shm, s, grp);
  else
    hipLaunchKernelGGL((conv_patch<WR, BN, CB, R8>), dim3((unsigned)blocks), dim3(256), shm, s, grp);
  return hipGetLastError();
}

#define PPOCR_PATCH(WR, CB)                                        \
  if (bn == 16) return go_patch<WR, 16, CB>(as, n, s);           \
  if (bn == 32 && r8) return go_patch<WR, 32, CB, true>(as, n, s);        \
  if (bn == 32) return go_patch<WR, 32, CB>(as, n, s);           \
  if (bn == 64) return go_patch<WR, 64, CB>(as, n, s);

hipError_t launch_conv_patch(const ConvArgs &a, int wr, int bk, int bn, hipStream_t s) {
  return launch_conv_patch_group(&a, 1, wr, bk, bn, s);
}

hipError_t launch_conv_patch_group(const ConvArgs *as, int n, int wr, int bk, int bn, hipStream_t s) {
  if (n < 1 || n > kGroupMax) return hipErrorInvalidValue;
  // 17 to 24 columns on 32-column tiles: the 8-column remainder (R8); the
  // detector head's 3 x 3 (two row blocks a wave) went from 40 to 35 us, the
  // neck's group (one row block a wave, its patch within four float4s a
  // thread and the kernel held to three waves per SIMD) from 51 to 46 us.
  bool r8 = bn == 32;
  for (int p = 0; p < n; p++) {
    if (!patch_supported(as[p], wr, bk, bn)) return hipErrorInvalidValue;
    r8 = r8 && as[p].n > 16 && as[p].n <= 24;
    // One row block a wave: the patch within kPatchPerR8W1 float4s a thread.
    const int pr = 3 * as[p].sh + as[p].kh, pc = 15 * as[p].sw + as[p].kw;
    if (wr == 1 && (pr * pc + 256 / (bk / 4) - 1) / (256 / (bk / 4)) > kPatchPerR8W1) r8 = false;
  }
  if (wr == 2) {
    if (bk == 32) { PPOCR_PATCH(2, 32) }
    if (bk == 16) { PPOCR_PATCH(2, 16) }
    if (bk == 8) { PPOCR_PATCH(2, 8) }
  } else {
    if (bk == 32) { PPOCR_PATCH(1, 32) }
    if (bk == 16) { PPOCR_PATCH(1, 16) }
    if (bk == 8) { PPOCR_PATCH(1, 8) }
  }
  return hipErrorInvalidValue;
}

hipError_t launch_ctc_merge(const float *part, int rows, int ntiles, float *y, long y_lane_stride,
                            int rows_per_lane, const CtcExact &ex, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  // The recompute reads packed rows as float4.
  if (ex.wt && (ex.wt_k % 4 || (uintptr_t(ex.wt) & 15))) return hipErrorInvalidValue;
  hipLaunchKernelGGL(ctc_merge, dim3((rows + 3) / 4), dim3(256), 0, s,
                     reinterpret_cast<const float4 *>(part), rows, ntiles, y, y_lane_stride,
                     rows_per_lane, ex);
  return hipGetLastError();
}

}  // namespace ppocr
