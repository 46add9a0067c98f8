// Launch arguments and host launchers of the backend's HIP kernels.
//
// Tensors are NHWC f32. A launch covers every lane of a batch: lane `l` of a
// tensor starts `lane_stride` floats after lane 0. Launchers return a
// hipError_t from the launch (or hipErrorInvalidValue for shapes a kernel
// does not take); they never synchronise.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <mutex>
#include <set>
#include <tuple>

namespace ppocr {

// Lets `kernel` take up to `bytes` of dynamic LDS on the current device: the
// attribute is set once per device, kernel and size (several handles may
// launch from several threads, on several devices).
inline hipError_t allow_lds(const void *kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::tuple<int, const void *, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(dev, kernel, bytes);
  if (done.count(key)) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert(key);
  return e;
}

// ------------------------------------------------- direct-to-LDS load helpers

typedef __attribute__((address_space(3))) void lds_void;

// Wait until at most n of this wave's vector memory operations are pending.
template <int n>
__device__ __forceinline__ void ring_wait() {
  static_assert(n >= 0 && n < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}

// ring_wait<k * L>() for a runtime k in [0, KMAX].
template <int L, int KMAX>
__device__ __forceinline__ void ring_wait_chunks(int k) {
  if constexpr (KMAX > 0) {
    if (k >= KMAX) {
      ring_wait<KMAX * L>();
      return;
    }
    ring_wait_chunks<L, KMAX - 1>(k);
  } else {
    ring_wait<0>();
  }
}

// A workgroup barrier without the memory fence __syncthreads() adds (whose
// vmcnt(0) would wait out every chunk in flight): the direct loads a stage
// needs are waited for explicitly, and a wave's LDS reads of a stage have
// returned before its MFMAs, hence before it reaches the next barrier. The
// empty asm keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- GEMM conv

// One input of an implicit-GEMM convolution: `c` channels starting at channel
// `coff` of each tap's concatenation, `shift` > 0 when it is read as
// nearest-upsampled by 2^shift (an upsampling folded in).
struct ConvSrc {
  const float *p;
  long lane_stride;
  int c;
  int shift;
  int coff;
};

enum GemmMode : int { GEMM_STORE = 0, GEMM_SPREAD = 1, GEMM_CTC = 2 };

// Up to kGroupMax independent problems of one kernel in one launch (so that
// small layers which do not depend on each other fill the GPU together):
// workgroup b runs block b - first[p] of problem p, first[p] <= b <
// first[p + 1]; x and y carry two per-problem integers of the kernel.
constexpr int kGroupMax = 4;
template <typename A>
struct Group {
  int n;
  int first[kGroupMax + 1];
  int x[kGroupMax], y[kGroupMax];
  A a[kGroupMax];
};

// Workgroup i of a launch runs on XCD i % 8 (the dispatcher deals them round
// robin) and each XCD has its own L2. Renumber so that each XCD takes one
// contiguous run of tiles: neighbouring row tiles, which share input rows of
// a window (and, with several column tiles, the same A rows), then meet in
// the same L2 instead of each XCD fetching them from HBM. A bijection on
// [0, groups): the first groups % 8 XCDs take one tile more.
__device__ __forceinline__ int xcd_tile(int i, int groups) {
  const int per = (groups + 7) >> 3;
  const int tall = (groups & 7) ? (groups & 7) : 8;
  const int xcd = i & 7, local = i >> 3;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

// The problem of a grouped launch that workgroup blockIdx.x belongs to.
template <typename A>
__device__ __forceinline__ int group_problem(const Group<A> &g) {
  int p = 0;
#pragma unroll
  for (int k = 1; k < kGroupMax; k++)
    if (k < g.n && (int)blockIdx.x >= g.first[k]) p = k;
  return p;
}

struct ConvArgs {
  int lanes;
  int ih, iw, oh, ow;   // per-lane window image and output sizes
  int n;                // output columns (oc, or the spread/CTC columns)
  int kh, kw, sh, sw, pt, pl;
  int nsrc;
  ConvSrc src[4];
  int ctot;             // channels of a tap: the sources' sum
  int cpt;              // channel layout: chunks per tap, ceil(ctot / BK)
  int chunks;           // reduction chunks: kh * kw * cpt, or ceil(kh * kw * ctot / BK)
  const float *wt;      // packed weights [n_pad][chunks * BK], zero padded
  long wt_k;            // floats per packed weight row (chunks * BK)
  const float *bias;    // n values or null
  const float *gate;    // per-lane channel gate of source 0, or null
  long gate_lane_stride;
  const float *res;     // per-lane residual [m][n], or null
  long res_lane_stride;
  int act, act2;
  float *y;
  long y_lane_stride;
  int mode;             // GemmMode
  int spread_kw, spread_oc;  // GEMM_SPREAD: non-overlapping transposed conv
  float *part;          // GEMM_CTC: per row and column tile (max, sum, best)
  int vocab;
  int xcd_rows;         // 1: give each XCD a contiguous run of tiles (see xcd_tile)
  // A 1x1 convolution of this one's output folded into the epilogue (its
  // weights [n][pw_n] as the plan stores them, bias, activation): the tile's
  // activated outputs are its input and only its output is stored, pw_n
  // columns a pixel. Null pw_w: none.
  const float *pw_w, *pw_b;
  int pw_n, pw_act;
};

struct GemmTile {
  int wm, bn, bk;  // wave rows (4 waves per tile), tile columns, reduction chunk
  bool vec;        // channel layout, four channels at a time (else flat layout)
  bool pointwise;  // 1x1, stride 1, no padding, one source
};

// Tiles launch_conv has compiled: BK 8, 16, 32 with WM 32 (BN 16, 32, 64) or
// WM 16 (BN 64); BK 64 (channel layout) with WM 16 and BN 16, 32, 64.
bool gemm_tile_supported(const GemmTile &t);
// Whether launch_conv takes a.pw_w (a folded 1x1) on tile t.
bool conv_pw_supported(const ConvArgs &a, const GemmTile &t);
hipError_t launch_conv(const ConvArgs &a, const GemmTile &t, hipStream_t s);
// The 1x1 convolution (GEMM_STORE or GEMM_SPREAD, one source of ctot
// channels, a multiple of 4) with its operand chunks in an LDS ring fed by
// direct loads: tiles of 32 * mt rows x 32 * nt columns, st stages of bk
// channels (compiled: mt 1, nt 1 to 3, st 3 or 4, bk 32).
struct RingTile {
  int mt, nt, st, bk;
};
bool ring_supported(const ConvArgs &a);
bool ring_fits(const ConvArgs &a, const RingTile &t);
size_t ring_lds_bytes(const ConvArgs &a, const RingTile &t);  // dynamic LDS of one workgroup
hipError_t launch_conv_ring(const ConvArgs &a, const RingTile &t, hipStream_t s);
// n <= kGroupMax problems, each ring_supported with the same gate and window
// kind and ring_fits for t, as one launch.
hipError_t launch_conv_ring_group(const ConvArgs *a, int n, const RingTile &t, hipStream_t s);
// The halo-tile windowed convolution (GEMM_STORE, kh, kw <= 3, stride 1 or
// 2, channels a multiple of 4): output tiles 16 wide x 4 * wr rows, bn
// columns, channel blocks of bk (the packed weights' chunk).
bool patch_fits(int kh, int kw, int stride, int wr, int bk, int bn);
bool patch_supported(const ConvArgs &a, int wr, int bk, int bn);
size_t patch_lds_bytes(const ConvArgs &a, int wr, int bk, int bn);
hipError_t launch_conv_patch(const ConvArgs &a, int wr, int bk, int bn, hipStream_t s);
// n <= kGroupMax problems, each patch_supported for (wr, bk, bn), as one launch.
hipError_t launch_conv_patch_group(const ConvArgs *a, int n, int wr, int bk, int bn, hipStream_t s);

// CTC choice from the GEMM's per-tile partials: y[2m] = best, y[2m+1] = 1/sum.
// `ex` names the head's input rows and weights, for rows whose two largest
// logits are too close for the GPU's summation order to decide (wt null:
// no such check).
struct CtcExact {
  const float *x;      // the head's input: rows_per_lane rows of ci per lane
  long x_lane_stride;
  int ci;
  const float *wt;     // packed weights: column n's ci inputs at wt + n * wt_k
  long wt_k;
  const float *bias;   // per column
  int vocab;
  int tile_n;          // columns a partial record covers (a GEMM tile, or a run of tiles)
  const float *tmax;   // or per 64-column tile and row its maximum, tile t's row m at t * rows + m
  int tmax_n;          // tiles
  // Bounds of a column's terms for the near-tie test: the largest |bias| and
  // the largest sum of a column's |weights|.
  float bias_max, wsum_max;
};
hipError_t launch_ctc_merge(const float *part, int rows, int ntiles, float *y, long y_lane_stride,
                            int rows_per_lane, const CtcExact &ex, hipStream_t s);

// The CTC head's GEMM over an input at most 128 wide (a multiple of 4), its
// operands read straight into MFMA registers: the rows of x (ci floats,
// rows_per_lane of them per lane) against the weights in enc_pack order
// (kp = enc_kpad(ci), columns padded to 16), bias per column; per row and
// run of `columns` columns (ctc_direct_runs) a float4 partial (max, sum of
// exp, first column of the max, second value), row m's run k at
// part[m * runs + k], for launch_ctc_merge.
struct CtcDirectArgs {
  const float *x;
  long x_lane_stride;
  int rows_per_lane, lanes, ci;
  const float *wt, *bias;
  int vocab;
  float *part;
  float *tmax;  // optional: per 64-column tile and row its maximum, tile t's row m at t * rows + m
};
bool ctc_direct_supported(int ci);
struct CtcRuns {
  int per_run;  // 64-column tiles a workgroup walks
  int runs;     // runs over the columns: partial records per row
  int columns;  // columns a record covers (the last run's may be fewer)
  int per_group; // runs a workgroup walks
};
CtcRuns ctc_direct_runs(long rows, int vocab);
hipError_t launch_ctc_direct(const CtcDirectArgs &a, hipStream_t s);

// ---------------------------------------------------------------- depthwise

struct DwArgs {
  int lanes, ih, iw, c, oh, ow, kh, kw, sh, sw, pt, pl;
  const float *x;
  long x_lane_stride;
  const float *w;     // [kh][kw][c]
  const float *bias;  // c or null
  int act;
  float *y;
  long y_lane_stride;
  // When set: also the f64 sums of y per channel, one row of c per block,
  // dw_mean_blocks(a) blocks per lane ([lane][block][c]), for the channel
  // mean that reads y (joined by launch_mean_group with x null).
  double *mean_part;
};
hipError_t launch_dwconv(const DwArgs &a, hipStream_t s);
bool dw_mean_supported(const DwArgs &a);
int dw_mean_blocks(const DwArgs &a);

// A depthwise layer and the 1x1 convolution that alone reads its output, in
// one launch (the depthwise map never stored). d.y is unused.
struct DwPwArgs {
  DwArgs d;
  const float *pw;    // the 1x1's weights packed by enc_pack with kp = d.c
  const float *pw_b;  // its bias or null
  int n, pw_act;      // its output channels and activation
  const float *res;   // added after the activation, or null
  long res_lane_stride;
  int act2;           // applied after the residual
  float *y;
  long y_lane_stride;
};
bool dwpw_supported(const DwArgs &d, int n, bool res);
hipError_t launch_dwpw(const DwPwArgs &a, hipStream_t s);

// ---------------------------------------------------------------- elementwise

enum EltMode : int {
  ELT_ADD = 0,          // a + b
  ELT_CHANNELMUL = 1,   // a * g[c]
  ELT_UPSAMPLE = 2,     // a[oy / sh][ox / sw]
  ELT_UPSAMPLEADD = 3,  // b + a[oy / sh][ox / sw]
  ELT_CONCAT = 4,       // channels of a (ca) then of b (cb)
  ELT_RESGATE = 5,      // a + a * g[c]
  ELT_UPSAMPLEADD_RESGATE = 6,  // (b + b * g[c]) + a[oy / sh][ox / sw]
  ELT_MUL = 7,          // a * b
  ELT_ACT = 8,          // a
};

struct EltArgs {
  int mode, lanes;
  int oh, ow, c;        // output size
  int iw, sh, sw;       // upsampling source width and factors
  int ca, cb;           // concat channel counts
  const float *a; long a_lane_stride;
  const float *b; long b_lane_stride;
  const float *g; long g_lane_stride;
  int act;
  float *y; long y_lane_stride;
};
hipError_t launch_eltwise(const EltArgs &a, hipStream_t s);

// A chain of 2x nearest upsample-adds in one pass (a feature pyramid's
// top-down path): level k (0 the finest) is
//   y_k = act_k((b_k + b_k * g_k[c]) + y_{k+1}[oy / 2][ox / 2])
// (without a gate: b_k + y_{k+1}...), y_levels being `top`. Each level's map
// is h[k] x w[k] = 2 h[k+1] x 2 w[k+1]; top is (h / 2) x (w / 2) of the
// coarsest level. Every level's output is written.
constexpr int kChainMax = 3;
struct ChainArgs {
  int lanes, levels, c;
  int h[kChainMax], w[kChainMax];
  const float *top; long top_lane_stride;
  const float *b[kChainMax]; long b_lane_stride[kChainMax];
  const float *g[kChainMax]; long g_lane_stride[kChainMax];  // null: no gate
  int act[kChainMax];
  float *y[kChainMax]; long y_lane_stride[kChainMax];
};
bool upadd_chain_supported(const ChainArgs &a);
hipError_t launch_upadd_chain(const ChainArgs &a, hipStream_t s);
// Whether launch_eltwise takes four floats at a time (the same for every
// member of a grouped launch).
bool eltwise_vec(const EltArgs &a);
hipError_t launch_eltwise_group(const EltArgs *a, int n, hipStream_t s);

struct PoolArgs {
  int avg, lanes, ih, iw, c, oh, ow, kh, kw, sh, sw;
  const float *x; long x_lane_stride;
  float *y; long y_lane_stride;
};
hipError_t launch_pool(const PoolArgs &a, hipStream_t s);

// ---------------------------------------------------------------- reductions

// Channel mean of every lane, with the squeeze-and-excite that may follow it:
// y = act2(W2 act1(W1 mean + b1) + b2), two 1x1 convolutions of one pixel.
// `w1`, `w2` hold each layer's weights in groups of four inputs, an
// output's four weights together (se_pack), 16-byte aligned.
struct SeArgs {
  const float *w1, *b1; int mid, act1;
  const float *w2, *b2; int cout, act2;
};
// One channel mean (with its squeeze-and-excite when has_se). One launch:
// workgroups sum pixel chunks of channel slices in f64 (or, with x null,
// join the `chunks` partial rows per lane a depthwise convolution wrote to
// `work`); the last workgroup of a slice to finish joins the slice's partial
// rows in a fixed order, and with an SE the last slice of a lane to finish
// runs both 1x1 layers. `work` (mean_shape(...).floats floats, 16-byte
// aligned) holds the partial rows (with x null: the depthwise convolution's
// lanes * chunks * c doubles at its start) and the gathered means; `count`
// (count_n ints) must be zero before the first launch, and every launch
// leaves it zero again. Launches that share `work` or `count` must not
// overlap.
struct MeanJob {
  const float *x;
  long x_lane_stride;
  int pixels, c, lanes, chunks;
  float *work;
  int *count;
  SeArgs se;
  int has_se;
  float *y;
  long y_lane_stride;
};
// How a job is cut: slices of `cs` channels (S of them), `k` pixel chunks per
// lane (1 when the partial rows come from a depthwise convolution); the
// workspace's means start `means_off` floats in, and it holds `floats`; the
// job needs `count_n` counters.
struct MeanShape {
  int cs, S, k;
  size_t means_off, floats, count_n;
};
__host__ __device__ MeanShape mean_shape(bool has_x, int pixels, int c, int lanes, int dw_rows, bool has_se);
// Whether the SE layers' shapes are ones the kernel takes.
bool se_supported(int c, int mid, int cout);
// The packed form of a 1x1 layer's plan weights w[i * n + j] (m inputs, n
// outputs): out[((i / 4) * n + j) * 4 + i % 4], inputs past m zero;
// se_pack_floats(m, n) floats.
inline size_t se_pack_floats(int m, int n) { return size_t((m + 3) / 4) * 4 * size_t(n); }
inline void se_pack(const float *w, int m, int n, float *out) {
  for (int i = 0; i < (m + 3) / 4 * 4; i++)
    for (int j = 0; j < n; j++)
      out[(size_t(i / 4) * n + j) * 4 + i % 4] = i < m ? w[size_t(i) * n + j] : 0.0f;
}
hipError_t launch_mean_group(const MeanJob *j, int n, hipStream_t s);

hipError_t launch_layernorm(const float *x, long x_lane_stride, const float *w, int rows, int c,
                            int lanes, float *y, long y_lane_stride, hipStream_t s);

// Attention keeps K and V of a head in LDS; score rows go to LDS too unless
// the line is long, when they take attention_scratch_floats() floats of
// `scratch` (nonzero only then).
size_t attention_scratch_floats(int t, int c, int heads, int lanes);
hipError_t launch_attention(const float *x, long x_lane_stride, float scale, int t, int c,
                            int heads, int lanes, float *y, long y_lane_stride, float *scratch,
                            hipStream_t s);

// ------------------------------------------------------ transformer encoder

// The encoder's GEMM weights (k inputs x n outputs, input-major as in the
// plan) in MFMA operand order, inputs padded to kp (a multiple of 16): for
// column block j and input group q of 16, 64 float4s, lane l's holding
// W[16q + 4(l / 16) + e][16j + l % 16], e = 0..3, zero past k and n.
int enc_kpad(int k);            // kp of the 1x1 layers over the encoder's width
int enc_mlp_hpad(int hidden);   // kp of the MLP's fc2
size_t enc_pack_floats(int kp, int n);
void enc_pack(const float *w, int k, int n, int kp, float *out);

// Rows of `rows` per lane, each lane `*_lane_stride` floats after the last.
// y = act2(act(LN(x) W + bias) + res): LayerNorm when ln (gamma[k], beta[k],
// eps) is set, the residual when res is.
struct EncLinArgs {
  int rows, lanes, k, n;
  const float *x;
  long x_lane_stride;
  const float *ln;
  const float *wt, *bias;  // wt: enc_pack, kp = enc_kpad(k)
  int act, act2;
  const float *res;
  long res_lane_stride;
  float *y;
  long y_lane_stride;
};
bool enc_linear_supported(int k, int n);
hipError_t launch_enc_linear(const EncLinArgs &a, hipStream_t s);

// Attention of the lanes' t steps (rows of q | k | v, 3c floats), then
// z = act2(act(attention Wp + bias) + res) with the c x c projection Wp;
// when w1 is set, then y = act3m(z + act2m(act1m(LN(z) W1 + b1) W2 + b2))
// and LN_out(y) in its place when ln_out is set; else y = z.
struct EncAttnArgs {
  int t, lanes, c, heads;
  float scale;
  const float *qkv;
  long qkv_lane_stride;
  const float *wt, *bias;  // wt: enc_pack, kp = enc_kpad(c)
  int act, act2;
  const float *res;
  long res_lane_stride;
  int hidden;
  const float *ln;         // gamma[c], beta[c], eps
  const float *w1, *b1;    // w1: enc_pack, kp = enc_kpad(c)
  int act1m;
  const float *w2, *b2;    // w2: enc_pack, kp = enc_mlp_hpad(hidden)
  int act2m, act3m;
  const float *ln_out;
  float *y;
  long y_lane_stride;
};
// hidden: the MLP's width, 0 without it.
bool enc_attn_supported(int c, int heads, int hidden);
bool enc_attn_fits(int t, int c, int heads, int hidden);  // the line's K and V fit LDS
hipError_t launch_enc_attn(const EncAttnArgs &a, hipStream_t s);

// z = act3(x + act2(act1(LN(x) W1 + b1) W2 + b2)) (the residual when
// `residual`, else without x), then LN_out(z) in its place when ln_out is set.
struct EncMlpArgs {
  int rows, lanes, c, hidden;
  const float *x;
  long x_lane_stride;
  const float *ln;
  const float *w1, *b1;  // w1: enc_pack, kp = enc_kpad(c)
  int act1;
  const float *w2, *b2;  // w2: enc_pack, kp = enc_mlp_hpad(hidden)
  int act2, act3;
  int residual;
  const float *ln_out;
  float *y;
  long y_lane_stride;
};
bool enc_mlp_supported(int c, int hidden);
hipError_t launch_enc_mlp(const EncMlpArgs &a, hipStream_t s);

hipError_t launch_row_argmax(const float *x, float *y, int rows, int cols, hipStream_t s);

// Transposed convolution with few outputs per pixel (kh*kw*oc <= 16): one
// thread per input pixel, all its outputs.
struct ConvtArgs {
  int lanes, ih, iw, ic, oc, kh, kw;
  const float *x; long x_lane_stride;
  const float *w;     // [ic][kh][kw][oc]
  const float *bias;  // kh*kw*oc or null
  int act;
  float *y; long y_lane_stride;
};
hipError_t launch_convt_small(const ConvtArgs &a, hipStream_t s);

// ------------------------------------------------------- direct (VALU) layers

// A windowed convolution over one source, in the CPU engine's order: bias
// first for outputs ox < first_end, fused multiply-adds for channels below
// `fused`.
struct DirectArgs {
  int lanes, ih, iw, ic, oh, ow, oc, kh, kw, sh, sw, pt, pl;
  const float *x; long x_lane_stride;
  const float *w;     // [kh][kw][ic][oc]
  const float *bias;  // oc or null
  int act, first_end, fused;
  float *y; long y_lane_stride;
};
bool direct_supported(int kh, int kw, int ic);
// The window shapes the direct kernel also takes with four or more channels
// (each output pixel's outputs from one thread).
bool direct_pix_supported(int kh, int kw, int ic, int oc);
hipError_t launch_conv_direct(const DirectArgs &a, hipStream_t s);

// The detector's stem block in one pass: s1 = 3x3 stride-2 convolution of
// the RGB input (pad 1, 3 -> C1, the stem rule), then from s1 both a 2x2
// stride-1 max pool cut at the bottom and right edges (`pool`) and two 2x2
// stride-1 convolutions padded right and bottom, C1 -> C2 -> C3 (`y`), on
// MFMA with their biases added after the products. The s1 map and the first
// 2x2's map stay in LDS. The input is ih x iw; s1 is oh x ow, as are both
// outputs.
struct StemArgs {
  int lanes, ih, iw, oh, ow, c1, c2, c3;
  const float *x; long x_lane_stride;
  const float *w1, *b1; int act1;
  const float *w2, *b2; int act2;
  const float *w3, *b3; int act3;
  // Floats from one pixel to the next in each output: c1 and c3 for maps of
  // their own, c1 + c3 when y sits c1 floats into the pool's pixels (one
  // map of both, the next convolution's single source).
  float *pool; long pool_lane_stride; int pool_px;
  float *y; long y_lane_stride; int y_px;
};
// The stem block's kernels: C1 24, C2 12, C3 24, one activation, ReLU or
// hard swish, for all three layers.
bool stem_block_supported(int c1, int c2, int c3, int act1, int act2, int act3);
hipError_t launch_stem_block(const StemArgs &a, hipStream_t s);

// Two 2x2 stride-2 transposed convolutions in a row: ic -> oc1 (act1), then
// oc1 -> 1 (act2); y is the final map, (4 ih) x (4 iw).
struct HeadArgs {
  int lanes, ih, iw, ic, oc1;
  const float *x; long x_lane_stride;
  const float *w1, *b1;  // [ic][2][2][oc1], 4 * oc1 or null
  int act1;
  const float *w2, *b2;  // [oc1][2][2][1], 4 or null
  int act2;
  float *y; long y_lane_stride;
};
bool head_supported(int ic, int oc1);
hipError_t launch_db_head(const HeadArgs &a, hipStream_t s);

// mask[i] = prob[i] > thresh over n floats (bytes out).
hipError_t launch_db_mask(const float *prob, uint8_t *mask, long n, float thresh, hipStream_t s);
hipError_t launch_copy_lds(const float *x, float *y, long n, hipStream_t s);
hipError_t launch_db_bits(const float *map, long lane_stride, int w, int h, int lanes, float thresh,
                          unsigned long long *bits, hipStream_t s);

// ------------------------------------------------------------- image stages

// Device-memory image stages (HWC, 8-bit BGR in). See image.hip.
struct CropMap {
  double v[9];  // rectangle -> quad projective map, row major, v[8] = 1
};
hipError_t launch_resize(const uint8_t *src, int sw, int sh, uint8_t *dst, int dw, int dh, hipStream_t s);
hipError_t launch_det_input(const uint8_t *src, int sw, int sh, float *out, int dw, int dh, const double *mean,
                            const double *sd, hipStream_t s);
hipError_t launch_rec_input(const uint8_t *src, int sw, int sh, float *out, int width, int rw, hipStream_t s);
hipError_t launch_crop(const uint8_t *img, int iw, int ih, const CropMap &m, uint8_t *out, int width, int height,
                       bool turn, hipStream_t s);
// One line of a batched crop + recogniser input: the cw x ch rectangle's
// map, turned when `turn`, into a 48 x width tensor of which the first rw
// columns hold the resized crop.
struct CropLine {
  CropMap m;
  float *out;
  int cw, ch, turn, width, rw;
};
constexpr int kCropLines = 16;
struct CropLines {
  int n;
  CropLine l[kCropLines];
};
hipError_t launch_crop_rec(const uint8_t *img, int iw, int ih, const CropLines &b, hipStream_t s);

}  // namespace ppocr
