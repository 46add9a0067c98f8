// The recogniser's transformer encoder in two launches per block:
//
//  enc_linear      LayerNorm of each input row, then a 1x1 layer (the block's
//                  q|k|v projection), bias, activation, residual; tiles of 16
//                  rows (time steps; the lanes' rows stacked);
//  enc_attn_block  multi-head attention of a run of query rows over the
//                  whole line, every head in one workgroup, the c -> c
//                  output projection, bias and residual, then (when the
//                  block's MLP follows) LayerNorm, fc1 with its activation,
//                  fc2, the residual, and the next LayerNorm when only it
//                  reads the sum;
//  enc_mlp         the MLP part alone, on tiles of 16 rows.
//
// The intermediate rows (normalised inputs, attention outputs, the summed
// rows, the MLP's hidden layer) stay in LDS. The GEMMs run on
// v_mfma_f32_16x16x4_f32 with the weights read straight into the B operand
// registers from an MFMA-order packing (enc_pack: one coalesced 1 KiB
// float4 load per wave per column block and 16 inputs), requested before
// the data they multiply is ready; the A operand is read from the LDS rows.
//
// LayerNorm (src/engine/layers.rs LayerNorm): mean and variance of the row,
// root = sqrt(var + eps), y = (x - mean) / root * gamma + beta; the two sums
// here are butterfly sums over 32 lanes (the CPU sums in sequence), so a
// row's statistics differ from the CPU's in the last bits. Attention keeps
// the engine's order for every score, softmax and output (the phases of
// attention_rows, src/engine/layers.rs:494-522).
#include <algorithm>

#include "act.hpp"
#include "kernels.hpp"

namespace ppocr {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kEncRows = 16;
constexpr size_t kEncMaxLds = 160 * 1024;  // gfx950: LDS per CU

int enc_kpad(int k) { return k <= 32 ? 32 : (k <= 64 ? 64 : (k <= 128 ? 128 : 256)); }

int enc_mlp_hpad(int hidden) { return hidden <= 128 ? 128 : 256; }

size_t enc_pack_floats(int kp, int n) { return (size_t)kp * ((n + 15) / 16 * 16); }

void enc_pack(const float *w, int k, int n, int kp, float *out) {
  const int kq = kp / 16, nb = (n + 15) / 16;
  for (int j = 0; j < nb; j++)
    for (int q = 0; q < kq; q++)
      for (int l = 0; l < 64; l++)
        for (int e = 0; e < 4; e++) {
          const int kk = 16 * q + 4 * (l >> 4) + e, nn = 16 * j + (l & 15);
          out[(((size_t)j * kq + q) * 64 + l) * 4 + e] = kk < k && nn < n ? w[(size_t)kk * n + nn] : 0.0f;
        }
}

namespace {

constexpr int kEncThreads = 512;  // eight waves: two a SIMD

// Row m of a batch is row m % rows of lane m / rows (32-bit: a launch takes
// fewer than 2^31 rows). A tile's 16 rows, split once into LDS by its first
// 16 threads, serve every later access.
struct TileRows {
  int lane[kEncRows], row[kEncRows];
};

__device__ __forceinline__ void split_rows(TileRows &tr, int rows, long M, long m0) {
  if (threadIdx.x < kEncRows) {
    const int m = (int)min(m0 + threadIdx.x, M - 1);
    const int ln = m / rows;
    tr.lane[threadIdx.x] = ln;
    tr.row[threadIdx.x] = m - ln * rows;
  }
}

__device__ __forceinline__ long row_off(const TileRows &tr, int r, long lane_stride, int width) {
  return tr.lane[r] * lane_stride + (long)tr.row[r] * width;
}

// The sum of v over each aligned group of 32 lanes, the same bits in every
// lane: butterflies by DPP (pairs within quads, mirrored quads, mirrored
// halves of 16) and one exchange between the two 16-lane rows.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float sum32(float v) {
  v = v + dpp<0xB1>(v);   // quad_perm [1, 0, 3, 2]: lane ^ 1
  v = v + dpp<0x4E>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2
  v = v + dpp<0x141>(v);  // row_half_mirror: lane i <-> 7 - i of 8
  v = v + dpp<0x140>(v);  // row_mirror: lane i <-> 15 - i of 16
  return v + __shfl_xor(v, 16, 32);
}

__device__ __attribute__((aligned(16))) float kEncZeros[4];

// A LayerNorm's parameters for the values one thread normalises in ln_tile
// (columns p, p + 32, ... of a row, p = thread % 32), read at a kernel's
// start. Every load is unconditional (indices clamped below k; a null `ln`
// reads zeros, never used), so that they arrive with the kernel's first
// loads: a load under a per-lane condition would wait at once, one round
// trip after another. `ln` holds gamma[k], beta[k], eps.
template <int KP>
struct LnRegs {
  float g[KP / 32], b[KP / 32], eps;
};

template <int KP>
__device__ __forceinline__ LnRegs<KP> ln_regs(const float *ln, int k) {
  LnRegs<KP> r;
  const int p = threadIdx.x % 32;
  const float *src = ln ? ln : kEncZeros;
#pragma unroll
  for (int u = 0; u < KP / 32; u++) {
    const int i = ln ? min(p + 32 * u, k - 1) : 0;
    r.g[u] = src[i];
    r.b[u] = src[ln ? k + i : 0];
  }
  r.eps = src[ln ? 2 * k : 0];
  return r;
}

// LayerNorm of the 16 rows of an LDS tile (row stride S, the first k of each
// row; the padding past k holds zeros and stays so), 32 threads a row with
// KP / 32 of its values each in registers; `lr` from ln_regs.
template <int KP, int S>
__device__ __forceinline__ void ln_tile(float *t, int k, const LnRegs<KP> &lr) {
  constexpr int P = kEncThreads / kEncRows, V = KP / P;
  static_assert(P == 32, "sum32 joins 32 lanes");
  const int tid = threadIdx.x, r = tid / P, p = tid % P;
  float *row = t + r * S;
  float x[V];
  float s = 0.0f;
#pragma unroll
  for (int u = 0; u < V; u++) {
    x[u] = row[p + P * u];
    s = s + x[u];
  }
  const float mean = sum32(s) / (float)k;
  float q = 0.0f;
#pragma unroll
  for (int u = 0; u < V; u++) {
    const float d = x[u] - mean;
    if (p + P * u < k) q = q + d * d;
  }
  const float root = sqrtf(sum32(q) / (float)k + lr.eps);
#pragma unroll
  for (int u = 0; u < V; u++) {
    const int i = p + P * u;
    if (i < k) row[i] = (x[u] - mean) / root * lr.g[u] + lr.b[u];
  }
}

// Rows m0 .. m0 + 15 of x (k floats each, k a multiple of 4) into an LDS tile
// of row stride S (and into t2 as well, if not null), zero past k and past
// the last row.
template <int KP, int S>
__device__ __forceinline__ void load_rows(float *t, const float *x, long stride, int rows, long M, long m0,
                                          int k, float *t2 = nullptr) {
  constexpr int V = KP / 4;
  for (int e = threadIdx.x; e < kEncRows * V; e += kEncThreads) {
    const int r = e / V, q = e - r * V;
    const long m = m0 + r;
    f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
    if (m < M && 4 * q < k) {
      const int ln = (int)m / rows;
      v = *reinterpret_cast<const f32x4 *>(x + ln * stride + (long)((int)m - ln * rows) * k + 4 * q);
    }
    *reinterpret_cast<f32x4 *>(t + r * S + 4 * q) = v;
    if (t2) *reinterpret_cast<f32x4 *>(t2 + r * S + 4 * q) = v;
  }
}

// The B operands of column block j of an enc_pack matrix (KQ groups of 16
// inputs), zero past the last block.
template <int KQ>
__device__ __forceinline__ void load_b(f32x4 (&b)[KQ], const float *wt, int j, int nb, int lane) {
  const f32x4 *p = reinterpret_cast<const f32x4 *>(wt) + (long)j * KQ * 64 + lane;
#pragma unroll
  for (int q = 0; q < KQ; q++) b[q] = j < nb ? p[q * 64] : f32x4{0.f, 0.f, 0.f, 0.f};
}

// acc += A (16 rows of an LDS tile, stride S) x B (one column block).
template <int KQ, int S>
__device__ __forceinline__ void mfma_rows(f32x4 &acc, const float *t, const f32x4 (&b)[KQ], int lane) {
  const int li = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int q = 0; q < KQ; q++) {
    const f32x4 a = *reinterpret_cast<const f32x4 *>(t + li * S + 16 * q + 4 * lg);
#pragma unroll
    for (int e = 0; e < 4; e++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[q][e], acc, 0, 0, 0);
  }
}

}  // namespace

// ------------------------------------------------------------- enc_linear

// Workgroup (x, y): rows 16x .. 16x + 15; wave w takes column block 8y + w.
template <int KP>
__global__ __launch_bounds__(kEncThreads) void enc_linear(EncLinArgs a) {
  constexpr int S = KP + 4, KQ = KP / 16;
  __shared__ __attribute__((aligned(16))) float xs[kEncRows * S];
  __shared__ TileRows tr;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const long M = (long)a.rows * a.lanes, m0 = (long)blockIdx.x * kEncRows;
  const int nb = (a.n + 15) / 16, j = blockIdx.y * 8 + w;
  f32x4 b[KQ];
  load_b<KQ>(b, a.wt, j, nb, lane);
  const LnRegs<KP> lr = ln_regs<KP>(a.ln, a.k);
  split_rows(tr, a.rows, M, m0);
  load_rows<KP, S>(xs, a.x, a.x_lane_stride, a.rows, M, m0, a.k);
  __syncthreads();
  if (a.ln) {
    ln_tile<KP, S>(xs, a.k, lr);
    __syncthreads();
  }
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  mfma_rows<KQ, S>(acc, xs, b, lane);
  const int li = lane & 15, lg = lane >> 4;
  const int col = 16 * j + li;
  if (col >= a.n) return;
  const float bias = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const long m = m0 + 4 * lg + r;
    if (m >= M) continue;
    float v = acc[r];
    if (a.bias) v = v + bias;
    v = act(v, a.act);
    if (a.res) v = act(v + a.res[row_off(tr, 4 * lg + r, a.res_lane_stride, a.n) + col], a.act2);
    a.y[row_off(tr, 4 * lg + r, a.y_lane_stride, a.n) + col] = v;
  }
}

bool enc_linear_supported(int k, int n) { return k > 0 && k % 4 == 0 && k <= 128 && n > 0; }

hipError_t launch_enc_linear(const EncLinArgs &a, hipStream_t s) {
  const long M = (long)a.rows * a.lanes;
  if (!enc_linear_supported(a.k, a.n) || a.x_lane_stride % 4 || M <= 0 || M >= (1L << 31))
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)((M + kEncRows - 1) / kEncRows), (unsigned)(((a.n + 15) / 16 + 7) / 8));
  switch (enc_kpad(a.k)) {
    case 32: hipLaunchKernelGGL(enc_linear<32>, grid, dim3(kEncThreads), 0, s, a); break;
    case 64: hipLaunchKernelGGL(enc_linear<64>, grid, dim3(kEncThreads), 0, s, a); break;
    default: hipLaunchKernelGGL(enc_linear<128>, grid, dim3(kEncThreads), 0, s, a); break;
  }
  return hipGetLastError();
}

// --------------------------------------------------------- enc_attn_block

// Tile b (workgroups renumbered XCD by XCD): lane b / runs, query rows
// tq * (b % runs) onward, every head:
// heads * tq <= 64 score rows (head, query), eight threads a row, thread p
// of a row taking keys j = p, p + 8, ... (the engine's softmax lanes).
// LDS: K and V of the line per head (rows padded to 16 floats), the run's
// pre-scaled queries, its probabilities, and the attention output rows (the
// projection's A tile).
constexpr int kAttnTq = 8;     // query rows a workgroup
constexpr int kAttnBody = 16;  // keys a softmax lane keeps: lines of fewer than 136 steps

struct AttnLds {
  int ks, vs, qs, sc, os, total;
};

// Floats from one head's K (or V) rows to the next: 8 more than the rows
// take, so that the heads' rows start in different LDS banks (the scatter of
// a key's channels to its heads, and the score reads of several heads, then
// spread over the banks); V starts 32 floats on for the same reason.
__host__ __device__ inline int attn_hs(int t) { return t * 16 + 8; }

// With the MLP (hp > 0) three tiles reuse regions whose data is spent: the
// hidden rows take K and V's place, the summed rows the probabilities', the
// normalised rows the attention outputs'.
__host__ __device__ inline AttnLds attn_lds(int t, int heads, int tq, int kp, int hp) {
  AttnLds l;
  l.ks = 0;
  l.vs = l.ks + heads * attn_hs(t) + 32;
  int end = l.vs + heads * attn_hs(t);
  if (hp && end < kEncRows * (hp + 4)) end = kEncRows * (hp + 4);
  l.qs = (end + 3) / 4 * 4;
  l.sc = l.qs + heads * tq * 16;
  int sc = heads * tq * (t + 1);
  if (hp && sc < kEncRows * (kp + 4)) sc = kEncRows * (kp + 4);
  l.os = (l.sc + sc + 3) / 4 * 4;
  l.total = l.os + kEncRows * (kp + 4);
  return l;
}

template <int KP, int HP>
__global__ __launch_bounds__(kEncThreads) void enc_attn_block(EncAttnArgs a, int tq) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  constexpr int S = KP + 4, KQ = KP / 16;
  const int t = a.t, c = a.c, heads = a.heads, hd = c / heads, c4 = c / 4;
  const int runs = (t + tq - 1) / tq;
  // The runs of one line on one XCD (each reads the line's K and V: they
  // then meet in that XCD's L2).
  const int tile = xcd_tile(blockIdx.x, gridDim.x);
  const int ln = tile / runs, q0 = (tile % runs) * tq, nq = min(tq, t - q0);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const AttnLds L = attn_lds(t, heads, tq, KP, HP);
  float *ks = sm + L.ks, *vs = sm + L.vs, *qs = sm + L.qs, *sc = sm + L.sc;
  float *os = sm + L.os;
  f32x4 b[KQ];
  load_b<KQ>(b, a.wt, w, (c + 15) / 16, lane);
  const int li = lane & 15, lg = lane >> 4, col = 16 * w + li;
  // The MLP's LayerNorm parameters, with the kernel's first loads.
  const LnRegs<KP> lr_in = ln_regs<KP>(HP ? a.ln : nullptr, c);
  const LnRegs<KP> lr_out = ln_regs<KP>(HP ? a.ln_out : nullptr, c);
  // Its biases: fc1's columns 16 (w + 8 jj) + li, fc2's column 16 w + li
  // (clamped; those past the layer are never used).
  float fb1[2], fb2;
  {
    const float *s1 = HP && a.b1 ? a.b1 : kEncZeros, *s2 = HP && a.b2 ? a.b2 : kEncZeros;
#pragma unroll
    for (int jj = 0; jj < 2; jj++) fb1[jj] = s1[HP && a.b1 ? min(16 * (w + 8 * jj) + li, a.hidden - 1) : 0];
    fb2 = s2[HP && a.b2 ? min(col, c - 1) : 0];
  }
  // This lane's residual and bias, for the projection's epilogue, loaded
  // unconditionally (rows and column clamped into the line; values past the
  // run or the width are never stored).
  float res[4];
  {
    const bool hr = a.res != nullptr;
    const float *rs = hr ? a.res + (long)ln * a.res_lane_stride : kEncZeros;
#pragma unroll
    for (int rr = 0; rr < 4; rr++) res[rr] = rs[hr ? (long)min(q0 + 4 * lg + rr, t - 1) * c + min(col, c - 1) : 0];
  }
  const float bias = (a.bias ? a.bias : kEncZeros)[a.bias ? min(col, c - 1) : 0];

  // K and V: thread (key slot, part) moves four channels of one of them for
  // keys slot, slot + per, ...; where each channel lands is worked out once.
  const float *xl = a.qkv + (long)ln * a.qkv_lane_stride;
  {
    const int parts = 2 * c4, per = kEncThreads / parts;
    const int slot = tid / parts, p = tid - slot * parts;
    if (slot < per) {
      const int v = p >= c4, ch = 4 * (p - v * c4);
      int off[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int h = (ch + u) / hd;
        off[u] = h * attn_hs(t) + ch + u - h * hd;
      }
      float *dst = v ? vs : ks;
      const float *src = xl + (v ? 2 * c : c) + ch;
      // Sixteen keys' loads in flight at a time (indices clamped to the
      // line, so that none waits on a branch), then their LDS stores.
      for (int j0 = slot; j0 < t; j0 += 16 * per) {
        f32x4 x[16];
#pragma unroll
        for (int i = 0; i < 16; i++)
          x[i] = *reinterpret_cast<const f32x4 *>(src + (long)min(j0 + i * per, t - 1) * 3 * c);
#pragma unroll
        for (int i = 0; i < 16; i++) {
          const int j = j0 + i * per;
          if (j < t) {
#pragma unroll
            for (int u = 0; u < 4; u++) dst[off[u] + j * 16] = x[i][u];
          }
        }
      }
    }
    const int qper = kEncThreads / c4, qslot = tid / c4, qp = tid - qslot * c4;
    if (qslot < qper) {
      const int ch = 4 * qp;
      int off[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int h = (ch + u) / hd;
        off[u] = h * tq * 16 + ch + u - h * hd;
      }
      for (int s = qslot; s < nq; s += qper) {
        const f32x4 x = *reinterpret_cast<const f32x4 *>(xl + (long)(q0 + s) * 3 * c + ch);
#pragma unroll
        for (int u = 0; u < 4; u++) qs[off[u] + s * 16] = x[u] * a.scale;
      }
    }
  }
  for (int e = tid; e < kEncRows * S; e += kEncThreads) os[e] = 0.0f;
  // Zeros past hd in the key and query rows: the score sums then run over
  // all 16 places, each extra term adding an exact zero.
  for (int e = tid; e < heads * (t + tq); e += kEncThreads) {
    const int hk = e / t;
    float *pad = e < heads * t ? ks + hk * attn_hs(t) + (e - hk * t) * 16 : qs + (e - heads * t) * 16;
    for (int d = hd; d < 16; d++) pad[d] = 0.0f;
  }
  __syncthreads();

  const int ts = t + 1, fused = t / 8 * 8, rows = heads * nq;
  const int r = tid >> 3, p8 = tid & 7;
  const int h = r < rows ? r / nq : 0, s = r - h * nq;
  const float ninf = -__builtin_inff();
  float *row = sc + r * ts;
  // One row (head, query) per eight consecutive lanes; lane p8 keeps keys
  // j = p8 + 8i below t / 8 * 8 (the engine's softmax lanes) in registers,
  // and the tail key t / 8 * 8 + p8 if there is one. The lanes of a row
  // exchange maxima and sums by shuffles, each joining them in the engine's
  // order, and store the row's probabilities for the outputs.
  if (r < rows) {
    f32x4 qv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) qv[u] = *reinterpret_cast<const f32x4 *>(qs + (h * tq + s) * 16 + 4 * u);
    const float *kb = ks + h * attn_hs(t) + p8 * 16;
    const int body = fused / 8, tail = t - fused;
    float sv[kAttnBody];
    // Scores: from zero, a fused multiply-add per head dimension in order
    // (the zero padding past hd adds nothing), four keys at a time (their
    // loads together, their sums interleaved).
#pragma unroll
    for (int i = 0; i < kAttnBody; i += 4) {
      if (i < body) {
        f32x4 kv[4][4];
#pragma unroll
        for (int k = 0; k < 4; k++)
#pragma unroll
          for (int u = 0; u < 4; u++)
            kv[k][u] = *reinterpret_cast<const f32x4 *>(kb + min(i + k, body - 1) * 128 + 4 * u);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int d = 0; d < 16; d++)
#pragma unroll
          for (int k = 0; k < 4; k++) acc[k] = fmaf(kv[k][d / 4][d % 4], qv[d / 4][d % 4], acc[k]);
#pragma unroll
        for (int k = 0; k < 4; k++) sv[i + k] = acc[k];
      }
    }
    // The tail key: products and sums separately.
    float tv = ninf;
    if (p8 < tail) {
      f32x4 kv[4];
#pragma unroll
      for (int u = 0; u < 4; u++) kv[u] = *reinterpret_cast<const f32x4 *>(kb + body * 128 + 4 * u);
      float acc = 0.0f;
#pragma unroll
      for (int d = 0; d < 16; d++) acc = acc + qv[d / 4][d % 4] * kv[d / 4][d % 4];
      tv = acc;
    }
    // The row's maximum: each lane's over its keys in order, the lanes in
    // order, then the tail keys in order.
    float ml = ninf;
#pragma unroll
    for (int i = 0; i < kAttnBody; i++)
      if (i < body) ml = sv[i] > ml ? sv[i] : ml;
    float m = ninf;
#pragma unroll
    for (int l = 0; l < 8; l++) m = fmaxf(m, __shfl(ml, l, 8));
#pragma unroll
    for (int l = 0; l < 7; l++)
      if (l < tail) m = fmaxf(m, __shfl(tv, l, 8));
    // Exponentials; each lane's sum in key order, the lanes' sums in order,
    // then the tail's exponentials in order.
    float sl = 0.0f;
#pragma unroll
    for (int i = 0; i < kAttnBody; i++)
      if (i < body) {
        sv[i] = exp_neg(sv[i] - m);
        sl = sl + sv[i];
      }
    const float te = p8 < tail ? exp_neg(tv - m) : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) sum = sum + __shfl(sl, l, 8);
#pragma unroll
    for (int l = 0; l < 7; l++)
      if (l < tail) sum = sum + __shfl(te, l, 8);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < kAttnBody; i++)
      if (i < body) row[p8 + 8 * i] = sv[i] * inv;
    if (p8 < tail) row[fused + p8] = te * inv;
  }
  __syncthreads();
  // Outputs: from zero, a fused multiply-add per key in order, two head
  // dimensions a thread (eight lanes a row), eight keys' loads at a time;
  // into the projection's A tile.
  if (r < rows && 2 * p8 < hd) {
    const float *v = vs + h * attn_hs(t) + 2 * p8;
    f32x2 acc = f32x2{0.f, 0.f};
    int j = 0;
    for (; j + 8 <= t; j += 8) {
      f32x2 vv[8];
      float pp[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        vv[u] = *reinterpret_cast<const f32x2 *>(v + (j + u) * 16);
        pp[u] = row[j + u];
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        acc.x = fmaf(vv[u].x, pp[u], acc.x);
        acc.y = fmaf(vv[u].y, pp[u], acc.y);
      }
    }
    for (; j < t; j++) {
      const f32x2 vv = *reinterpret_cast<const f32x2 *>(v + j * 16);
      const float pp = row[j];
      acc.x = fmaf(vv.x, pp, acc.x);
      acc.y = fmaf(vv.y, pp, acc.y);
    }
    os[s * S + h * hd + 2 * p8] = acc.x;
    if (2 * p8 + 1 < hd) os[s * S + h * hd + 2 * p8 + 1] = acc.y;
  }
  __syncthreads();

  // The projection: wave w takes column block w.
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  mfma_rows<KQ, S>(acc, os, b, lane);
  if constexpr (HP == 0) {
    if (col >= c) return;
#pragma unroll
    for (int rr = 0; rr < 4; rr++) {
      const int sq = 4 * lg + rr;
      if (sq >= nq) continue;
      float v = acc[rr];
      if (a.bias) v = v + bias;
      v = act(v, a.act);
      if (a.res) v = act(v + res[rr], a.act2);
      a.y[(long)ln * a.y_lane_stride + (long)(q0 + sq) * c + col] = v;
    }
  } else {
    // The MLP on the 16 rows (those past nq hold finite values never
    // stored): fc1's weights requested now, fc2's after the barrier.
    constexpr int SH = HP + 4, HQ = HP / 16;
    const int hidden = a.hidden, nb1 = (hidden + 15) / 16;
    float *zs = sm + L.sc, *ns = sm + L.os, *hs = sm + L.ks;
    f32x4 w1a[KQ], w1b[KQ];
    load_b<KQ>(w1a, a.w1, w, nb1, lane);
    load_b<KQ>(w1b, a.w1, w + 8, nb1, lane);
    __syncthreads();  // every wave's projection has read os
    f32x4 w2[HQ];
    load_b<HQ>(w2, a.w2, w, (c + 15) / 16, lane);
    if (col < KP) {
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        float v = 0.0f;
        if (col < c) {
          v = acc[rr];
          if (a.bias) v = v + bias;
          v = act(v, a.act);
          if (a.res) v = act(v + res[rr], a.act2);
        }
        zs[(4 * lg + rr) * S + col] = v;
        ns[(4 * lg + rr) * S + col] = v;
      }
    }
    const int pad = HP - 16 * nb1;
    for (int e = tid; e < kEncRows * pad; e += kEncThreads) hs[(e / pad) * SH + 16 * nb1 + e % pad] = 0.0f;
    __syncthreads();
    if (a.ln) {
      ln_tile<KP, S>(ns, c, lr_in);
      __syncthreads();
    }
    {
      f32x4 h0 = f32x4{0.f, 0.f, 0.f, 0.f}, h1 = h0;
      mfma_rows<KQ, S>(h0, ns, w1a, lane);
      mfma_rows<KQ, S>(h1, ns, w1b, lane);
#pragma unroll
      for (int jj = 0; jj < 2; jj++) {
        const int j = w + 8 * jj;
        if (j >= nb1) continue;
        const int hc = 16 * j + li;
        const f32x4 hv = jj ? h1 : h0;
        const float hb = fb1[jj];
#pragma unroll
        for (int rr = 0; rr < 4; rr++) {
          float v = hv[rr];
          if (a.b1) v = v + hb;
          hs[(4 * lg + rr) * SH + hc] = hc < hidden ? act(v, a.act1m) : 0.0f;
        }
      }
    }
    __syncthreads();
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
    mfma_rows<HQ, SH>(o, hs, w2, lane);
    // Each lane reads and rewrites its own (row, column) of zs.
    if (col < c) {
      const float ob = fb2;
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        float v = o[rr];
        if (a.b2) v = v + ob;
        v = act(v, a.act2m);
        float *z = zs + (4 * lg + rr) * S + col;
        *z = act(*z + v, a.act3m);
      }
    }
    __syncthreads();
    if (a.ln_out) {
      ln_tile<KP, S>(zs, c, lr_out);
      __syncthreads();
    }
    for (int e = tid; e < nq * c4; e += kEncThreads) {
      const int sq = e / c4, q = e - sq * c4;
      *reinterpret_cast<f32x4 *>(a.y + (long)ln * a.y_lane_stride + (long)(q0 + sq) * c + 4 * q) =
          *reinterpret_cast<const f32x4 *>(zs + sq * S + 4 * q);
    }
  }
}

// Query rows a workgroup: about one workgroup per CU (each loads its line's
// K and V), at most kAttnTq.
static int attn_tq(int t, int lanes) {
  const long q = ((long)t * lanes + 255) / 256;
  return (int)std::max(1L, std::min<long>(kAttnTq, q));
}

bool enc_attn_fits(int t, int c, int heads, int hidden) {
  // The row count per workgroup can reach kAttnTq.
  const int hp = hidden ? enc_mlp_hpad(hidden) : 0;
  return t / 8 <= kAttnBody &&
         (size_t)attn_lds(t, heads, kAttnTq, enc_kpad(c), hp).total * sizeof(float) <= kEncMaxLds;
}

bool enc_attn_supported(int c, int heads, int hidden) {
  return heads > 0 && heads * kAttnTq <= 64 && c % heads == 0 && c / heads <= 16 && c % 4 == 0 && c <= 128 &&
         hidden >= 0 && hidden <= 256;
}

hipError_t launch_enc_attn(const EncAttnArgs &a, hipStream_t s) {
  const int hidden = a.w1 ? a.hidden : 0;
  if (!enc_attn_supported(a.c, a.heads, hidden) || !enc_attn_fits(a.t, a.c, a.heads, hidden) ||
      a.qkv_lane_stride % 4 || (hidden && a.y_lane_stride % 4))
    return hipErrorInvalidValue;
  const int kp = enc_kpad(a.c), hp = hidden ? enc_mlp_hpad(hidden) : 0, tq = attn_tq(a.t, a.lanes);
  const size_t shm = (size_t)attn_lds(a.t, a.heads, tq, kp, hp).total * sizeof(float);
  const unsigned blocks = (unsigned)((long)a.lanes * ((a.t + tq - 1) / tq));
  auto go = [&](auto kernel) {
    // Allowed the whole LDS once, before any launch that needs over 64 KiB
    // (and so before a graph capture records one).
    hipError_t e = allow_lds(reinterpret_cast<const void *>(kernel), int(kEncMaxLds));
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(blocks), dim3(kEncThreads), shm, s, a, tq);
    return hipGetLastError();
  };
#define PPOCR_ENC_HP(KP)                                      \
  switch (hp) {                                              \
    case 0: return go(enc_attn_block<KP, 0>);                \
    case 128: return go(enc_attn_block<KP, 128>);            \
    default: return go(enc_attn_block<KP, 256>);             \
  }
  switch (kp) {
    case 32: PPOCR_ENC_HP(32)
    case 64: PPOCR_ENC_HP(64)
    default: PPOCR_ENC_HP(128)
  }
#undef PPOCR_ENC_HP
}

// ---------------------------------------------------------------- enc_mlp

// Workgroup x: rows 16x .. 16x + 15. Wave w takes fc1's column blocks w and
// w + 8 and fc2's block w; all their weights are requested at the start.
template <int KP, int HP>
__global__ __launch_bounds__(kEncThreads) void enc_mlp(EncMlpArgs a) {
  constexpr int S = KP + 4, SH = HP + 4, KQ = KP / 16, HQ = HP / 16;
  __shared__ __attribute__((aligned(16))) float zs[kEncRows * S];
  __shared__ __attribute__((aligned(16))) float ns[kEncRows * S];
  __shared__ __attribute__((aligned(16))) float hs[kEncRows * SH];
  __shared__ TileRows tr;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const long M = (long)a.rows * a.lanes, m0 = (long)blockIdx.x * kEncRows;
  const int c = a.c, hidden = a.hidden;
  const int nb1 = (hidden + 15) / 16, nb2 = (c + 15) / 16;
  f32x4 b0[KQ], b1[KQ], b2[HQ];
  load_b<KQ>(b0, a.w1, w, nb1, lane);
  load_b<KQ>(b1, a.w1, w + 8, nb1, lane);
  load_b<HQ>(b2, a.w2, w, nb2, lane);
  const LnRegs<KP> lr_in = ln_regs<KP>(a.ln, c), lr_out = ln_regs<KP>(a.ln_out, c);
  // The biases of fc1's columns 16 (w + 8 jj) + li and fc2's 16 w + li,
  // with the first loads (clamped; those past the layer are never used).
  float fb1[2], fb2;
  {
    const float *s1 = a.b1 ? a.b1 : kEncZeros, *s2 = a.b2 ? a.b2 : kEncZeros;
#pragma unroll
    for (int jj = 0; jj < 2; jj++) fb1[jj] = s1[a.b1 ? min(16 * (w + 8 * jj) + li, hidden - 1) : 0];
    fb2 = s2[a.b2 ? min(16 * w + li, c - 1) : 0];
  }
  split_rows(tr, a.rows, M, m0);
  load_rows<KP, S>(zs, a.x, a.x_lane_stride, a.rows, M, m0, c, ns);
  const int pad = HP - 16 * nb1;
  for (int e = tid; e < kEncRows * pad; e += kEncThreads) hs[(e / pad) * SH + 16 * nb1 + e % pad] = 0.0f;
  __syncthreads();
  if (a.ln) {
    ln_tile<KP, S>(ns, c, lr_in);
    __syncthreads();
  }
  {
    f32x4 acc0 = f32x4{0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
    mfma_rows<KQ, S>(acc0, ns, b0, lane);
    mfma_rows<KQ, S>(acc1, ns, b1, lane);
#pragma unroll
    for (int jj = 0; jj < 2; jj++) {
      const int j = w + 8 * jj;
      if (j >= nb1) continue;
      const int col = 16 * j + li;
      const f32x4 acc = jj ? acc1 : acc0;
      const float bias = fb1[jj];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float v = acc[r];
        if (a.b1) v = v + bias;
        hs[(4 * lg + r) * SH + col] = col < hidden ? act(v, a.act1) : 0.0f;
      }
    }
  }
  __syncthreads();
  f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
  mfma_rows<HQ, SH>(acc, hs, b2, lane);
  // Each lane reads and rewrites its own (row, column) of zs: no other
  // thread touches them until the barrier.
  const int col = 16 * w + li;
  if (col < c) {
    const float bias = fb2;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float v = acc[r];
      if (a.b2) v = v + bias;
      v = act(v, a.act2);
      float *z = zs + (4 * lg + r) * S + col;
      *z = a.residual ? act(*z + v, a.act3) : v;
    }
  }
  __syncthreads();
  if (a.ln_out) {
    ln_tile<KP, S>(zs, c, lr_out);
    __syncthreads();
  }
  const int c4 = c / 4;
  for (int e = tid; e < kEncRows * c4; e += kEncThreads) {
    const int r = e / c4, q = e - r * c4;
    const long m = m0 + r;
    if (m >= M) continue;
    *reinterpret_cast<f32x4 *>(a.y + row_off(tr, r, a.y_lane_stride, c) + 4 * q) =
        *reinterpret_cast<const f32x4 *>(zs + r * S + 4 * q);
  }
}

bool enc_mlp_supported(int c, int hidden) {
  return c > 0 && c % 4 == 0 && c <= 128 && hidden > 0 && hidden <= 256;
}

hipError_t launch_enc_mlp(const EncMlpArgs &a, hipStream_t s) {
  const long M = (long)a.rows * a.lanes;
  if (!enc_mlp_supported(a.c, a.hidden) || a.x_lane_stride % 4 || a.y_lane_stride % 4 || M <= 0 ||
      M >= (1L << 31))
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)((M + kEncRows - 1) / kEncRows));
  const int kp = enc_kpad(a.c), hp = enc_mlp_hpad(a.hidden);
  auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, dim3(kEncThreads), 0, s, a); };
  if (kp == 32)
    hp == 128 ? go(enc_mlp<32, 128>) : go(enc_mlp<32, 256>);
  else if (kp == 64)
    hp == 128 ? go(enc_mlp<64, 128>) : go(enc_mlp<64, 256>);
  else
    hp == 128 ? go(enc_mlp<128, 128>) : go(enc_mlp<128, 256>);
  return hipGetLastError();
}

}  // namespace ppocr
