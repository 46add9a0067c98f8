// The GPU model: the HIP counterpart of the engine's `GpuModel`
// (src/engine/gpu/mod.rs:81-291) behind the C ABI of include/ppocr_hip.h.
//
// Load: parse and check the plan, refuse what the GPU does not run, upload
// the weights, build the steps (fusion), repack the weights of every step
// that runs as an implicit GEMM, set one lane at the stored size.
//
// Lanes: every image of a run. Lanes of equal size form a batch that every
// launch covers at once (lanes stacked along the GEMM rows, or a grid axis),
// so sixteen recogniser lines cost one launch per step, not sixteen. Each
// batch owns one device arena in which every materialised plan buffer has a
// home, reused by liveness as `Lane::arrange` does (src/engine/gpu/mod.rs:
// 297-388), each lane of a home `stride` floats after the previous one.
//
// Run: per batch, a pitched copy of the inputs to the device, the batch's
// launch list (built once per size configuration), pitched copies of the
// outputs back, all on the model's stream, then one synchronisation.
#include <hip/hip_runtime.h>
#include <string.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <fstream>
#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "plan.hpp"
#include "ppocr_hip.h"

namespace ppocr {

namespace {

std::string fmt(const char *f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

void put_err(const std::string &m, char *err, size_t len) {
  if (!err || !len) return;
  size_t n = std::min(m.size(), len - 1);
  memcpy(err, m.data(), n);
  err[n] = 0;
}

#define HIPTRY(call, what)                                                       \
  do {                                                                           \
    hipError_t e_ = (call);                                                      \
    if (e_ != hipSuccess) {                                                      \
      err = std::string(what) + ": " + hipGetErrorString(e_);                    \
      return false;                                                              \
    }                                                                            \
  } while (0)

size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

enum StepKind {
  S_GEMM, S_DW, S_ELT, S_POOL, S_MEAN, S_LN, S_ATTN, S_CTC, S_CONVT, S_DIRECT, S_HEAD,
  // The detector's stem block: RGB stem, its 2x2 max pool and two 2x2 layers.
  S_STEM,
  // The transformer encoder's fused steps: LayerNorm -> 1x1 (enc_linear),
  // attention -> 1x1 -> Add (enc_attn_block), LayerNorm -> 1x1 -> 1x1 -> Add
  // [-> LayerNorm] (enc_mlp), and the last two as one (enc_attn_block).
  S_ENC_LIN, S_ENC_ATTN, S_ENC_MLP, S_ENC_BLOCK
};

struct Source {
  size_t slot;
  int c, shift;
};

struct Step {
  StepKind kind;
  int op;
  int gate = -1;     // Channelmul folded into a convolution's first input
  int add = -1;      // Add folded into a convolution's output / of a residual gate
  int resgate = -1;  // Channelmul of a residual gate, x + x * g
  // S_GEMM, S_DW: a 1x1 convolution of this step's output folded into it
  // (the step then writes that 1x1's output, or on S_DW the sum of its
  // folded Add), or -1.
  int pw1 = -1;
  int fc1 = -1, fc2 = -1;  // squeeze-and-excite 1x1 layers after a Mean; an encoder step's 1x1 layers
  int ln_out = -1;         // S_ENC_MLP, S_ENC_BLOCK: the LayerNorm of its sum, written in its place
  int m_ln = -1, m_fc1 = -1, m_fc2 = -1, m_add = -1;  // S_ENC_BLOCK: its MLP's operations
  int head2 = -1;          // the narrow transposed convolution folded into S_HEAD
  int st2 = -1, st3 = -1, st_pool = -1;  // S_STEM: the two 2x2 layers and the pool
  // S_STEM: the pool's map also holds the second 2x2's channels after its
  // own (one map, the next convolution's single source); only the pool's
  // slot is written.
  bool st_joint = false;
  // S_ELT as an upsample-add chain: its levels' operations, finest first
  // (chain[0] == op), and each level's residual-gate channelmul or -1.
  std::vector<int> chain, chain_gate;
  bool dw_sums = false;    // S_DW: also sum its output per channel for the next step's mean
  bool patch = false;      // S_GEMM: a windowed convolution on halo tiles (conv_patch)
  bool ring = false;       // S_GEMM: a windowed convolution on the LDS ring (conv_ring)
  int mean_of_dw = -1;     // S_MEAN: the depthwise operation whose sums it joins
  int elt = 0;             // EltMode
  std::vector<Source> sources;
  // Implicit-GEMM steps
  GemmTile tile{};
  int gemm_n = 0, chunks = 0, ctot = 0, cpt = 0;
  size_t wt_off = 0, wt_k = 0;
  size_t se_w1 = 0, se_w2 = 0;  // S_MEAN with an SE: the 1x1 weights, 16-byte aligned in the packed arena
  float ctc_bias_max = 0, ctc_wsum_max = 0;  // S_CTC: the largest |bias| and sum of a column's |weights|
  size_t enc_w1 = 0, enc_w2 = 0, enc_w3 = 0;  // encoder steps: their 1x1 weights in enc_pack order
};

enum GroupKind { GK_NONE = 0, GK_RING, GK_PATCH, GK_MEAN, GK_ELT };

struct Launch {
  std::string name;
  int op;
  std::function<hipError_t(hipStream_t)> fn;
  // Launches of the same batch this one must follow: those that write what
  // it reads or reads what it writes (memory homes are reused, so an earlier
  // reader of a home must finish before a later writer), and the previous
  // launch of its own step.
  std::vector<int> deps;
  int step = -1;
  // Algorithmic work of the launch: floating-point operations of the layer,
  // and bytes it must move (each input and the weights read once, each
  // output written once), for roofline fractions.
  double flops = 0, bytes = 0;
  // Grouping: a launch of kind gk may run together with launches of the
  // same kind and key that neither depend on it nor it on them, as one
  // grouped launch (a grid over all their blocks). Its arguments:
  int gk = GK_NONE;
  long gkey = 0;
  ConvArgs conv{};   // GK_RING, GK_PATCH
  RingTile rt{};     // GK_RING
  int bk = 0, bn = 0;  // GK_PATCH
  MeanJob mean{};    // GK_MEAN
  EltArgs elt{};     // GK_ELT
  // A grouped launch: the launches of build order it runs, and the plan
  // operation each of them starts from.
  std::vector<int> members;
  std::vector<int> member_ops;
};

// A batch of lanes of one size.
struct Batch {
  size_t h = 0, w = 0;
  std::vector<size_t> lanes;  // model lane indices, in order
  Plan plan;
  std::vector<size_t> home;   // plan buffer -> home, or SIZE_MAX
  std::vector<size_t> home_floats, home_off;
  size_t ws_off = 0;          // workspace in the arena, floats
  std::vector<size_t> step_ws;  // each step's own workspace, floats past ws_off
  float *arena = nullptr;
  size_t arena_floats = 0;
  float *host_in = nullptr;   // pinned, lanes * in_len
  size_t host_in_cap = 0;
  std::vector<float *> host_out;
  std::vector<size_t> host_out_cap;
  size_t in_len = 0;
  std::vector<Launch> launches;

  // The DB threshold's row bitmasks of one output (when the model is set to
  // write them): in the arena after the workspace, and pinned on the host.
  size_t bits_off = 0, bits_w = 0, bits_h = 0, bits_wpr = 0;
  unsigned long long *host_bits = nullptr;
  size_t host_bits_cap = 0;

  float *dev(size_t slot) const { return arena + home_off[home[slot]]; }
  float *ws(size_t step) const { return arena + ws_off + step_ws[step]; }
  long stride(size_t slot) const { return long(home_floats[home[slot]]); }
};

}  // namespace

struct Model {
  int device = 0;
  std::string name;
  int integrated = 0;
  size_t device_bytes = 0;
  hipStream_t stream = nullptr;
  // Whether independent launches of one kind run as grouped launches (in a
  // topological order of the groups); homes are then reused only where that
  // adds no ordering the data lacks.
  static constexpr bool kGrouped = true;
  Plan plan;
  std::vector<float> weights;     // host copy of the plan's weights
  float *dweights = nullptr;      // the plan's weights on the device
  float *dpacked = nullptr;       // GEMM-packed weights
  std::vector<Step> steps;
  std::vector<std::unique_ptr<Batch>> batches;
  std::vector<std::pair<size_t, size_t>> lane_at;  // lane -> (batch, index in batch)
  std::vector<std::pair<size_t, size_t>> sizes;
  size_t active_batches = 0;
  // The launches of one run over every batch, captured as a HIP graph on the
  // second run after the lanes were arranged (the first runs them eagerly,
  // which also sets any kernel attribute outside the capture).
  bool use_graphs = true;
  int eager_runs = 0;
  // The output whose DB threshold each run also writes as row bitmasks
  // (-1: none), and that threshold.
  long db_output = -1;
  float db_thresh = 0.3f;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;

  ~Model();
  void drop_graph();
  bool enqueue(std::string &err);
  bool launch_all(std::string &err);
  void link(Batch &b) const;
  bool load(const uint8_t *bytes, size_t len, std::string &err);
  bool build_steps(std::string &err);
  bool pack(std::string &err);
  bool set_sizes(const size_t *hw, size_t n, std::string &err);
  size_t max_lanes() const;
  bool arrange(Batch &b, std::string &err);
  void build_launches(Batch &b);
  void account(Batch &b) const;
  void group(Batch &b) const;
  bool run(bool copy_in, bool copy_out, std::string &err, bool sync = true);
  bool set_db_mask(long output, float thresh, std::string &err);
  bool copy_out_all(std::string &err);
  std::vector<size_t> step_reads(const Step &s) const;
  int enc_hidden(const Step &s) const { return s.kind == S_ENC_BLOCK ? int(plan.ops[s.m_fc1].oc) : 0; }
  size_t step_writes(const Step &s) const;
  // The step's other outputs: S_STEM's pool, an upsample-add chain's
  // coarser levels.
  std::vector<size_t> step_writes_extra(const Step &s) const {
    std::vector<size_t> r;
    if (s.kind == S_STEM && !s.st_joint) r.push_back(plan.ops[s.st_pool].y);
    for (size_t k = 1; k < s.chain.size(); k++) r.push_back(plan.ops[s.chain[k]].y);
    return r;
  }
};

Model::~Model() {
  if (stream) hipStreamSynchronize(stream);
  drop_graph();
  for (auto &b : batches) {
    if (b->arena) hipFree(b->arena);
    if (b->host_in) hipHostFree(b->host_in);
    if (b->host_bits) hipHostFree(b->host_bits);
    for (float *p : b->host_out)
      if (p) hipHostFree(p);
  }
  if (dweights) hipFree(dweights);
  if (dpacked) hipFree(dpacked);
  if (stream) hipStreamDestroy(stream);
}

// ---------------------------------------------------------------- steps

std::vector<size_t> Model::step_reads(const Step &s) const {
  const Op &op = plan.ops[s.op];
  std::vector<size_t> r;
  switch (s.kind) {
    case S_GEMM:
      for (const Source &src : s.sources) r.push_back(src.slot);
      if (s.gate >= 0) r.push_back(plan.ops[s.gate].x2);
      if (s.add >= 0) {
        const Op &a = plan.ops[s.add];
        r.push_back(a.x == op.y ? a.x2 : a.x);
      }
      break;
    case S_ELT:
      if (!s.chain.empty()) {
        r.push_back(plan.ops[s.chain.back()].x);
        for (size_t k = 0; k < s.chain.size(); k++) {
          if (s.chain_gate[k] >= 0) {
            r.push_back(plan.ops[s.chain_gate[k]].x), r.push_back(plan.ops[s.chain_gate[k]].x2);
          } else {
            r.push_back(plan.ops[s.chain[k]].x2);
          }
        }
      } else if (s.elt == ELT_RESGATE) {
        r = {plan.ops[s.resgate].x, plan.ops[s.resgate].x2};
      } else if (s.elt == ELT_UPSAMPLEADD_RESGATE) {
        r = {op.x, plan.ops[s.resgate].x, plan.ops[s.resgate].x2};
      } else {
        r.push_back(op.x);
        size_t x2;
        if (op.has_second(&x2)) r.push_back(x2);
      }
      break;
    case S_DW:
      r.push_back(op.x);
      if (s.add >= 0) {  // the residual of its folded 1x1
        const Op &a = plan.ops[s.add];
        r.push_back(a.x == plan.ops[s.pw1].y ? a.x2 : a.x);
      }
      break;
    case S_ENC_LIN:
    case S_ENC_ATTN:
    case S_ENC_MLP:
    case S_ENC_BLOCK:
      // Its first operation's input, and a residual other than that input.
      r.push_back(op.x);
      if (s.add >= 0) {
        const Op &a = plan.ops[s.add];
        const size_t last = plan.ops[s.kind == S_ENC_MLP ? s.fc2 : s.fc1].y;
        const size_t res = a.x == last ? a.x2 : a.x;
        if (res != op.x) r.push_back(res);
      }
      break;
    default:
      r.push_back(op.x);
  }
  return r;
}

size_t Model::step_writes(const Step &s) const {
  if (s.kind == S_HEAD) return plan.ops[s.head2].y;
  if (s.pw1 >= 0) return s.add >= 0 ? plan.ops[s.add].y : plan.ops[s.pw1].y;
  if (s.kind == S_STEM) return s.st_joint ? plan.ops[s.st_pool].y : plan.ops[s.st3].y;
  if (s.kind == S_MEAN && s.fc2 >= 0) return plan.ops[s.fc2].y;
  if ((s.kind == S_ENC_MLP || s.kind == S_ENC_BLOCK) && s.ln_out >= 0) return plan.ops[s.ln_out].y;
  if (s.kind == S_ENC_BLOCK) return plan.ops[s.m_add].y;
  if ((s.kind == S_ENC_LIN || s.kind == S_ENC_ATTN) && s.add < 0) return plan.ops[s.fc1].y;
  if (s.kind == S_ELT && s.elt == ELT_UPSAMPLEADD_RESGATE) return plan.ops[s.op].y;
  if (s.add >= 0) return plan.ops[s.add].y;
  return plan.ops[s.op].y;
}

// The fusion rules. Each folded operation's output is never materialised.
//  - Mean, then two 1x1 layers of its single pixel, each read only by the
//    next: one squeeze-and-excite step (mean + both layers).
//  - Channelmul whose product only the Add after it reads, adding it to the
//    multiply's own input: x + x * g (src/engine/gpu/mod.rs:607-617); when
//    that sum only feeds an Upsampleadd's addend, it folds into that step.
//  - Channelmul only a convolution reads: the gate scales the convolution's
//    first input as it is staged (gpu/mod.rs:501-505).
//  - Nearest upsamplings by powers of two and channel concatenations that
//    only feed a convolution: up to four shifted sources (gpu/mod.rs:506-521,
//    535-605).
//  - An Add that is the only reader of a convolution's output: the
//    convolution's epilogue (gpu/mod.rs:522-526).
//  - A 1x1 convolution that is the only reader of the implicit-GEMM
//    convolution just before it: that convolution's epilogue (decided in
//    pack, once the convolution's tile is known).
//  - A 1x1 convolution (with its folded Add) that is the only reader of the
//    depthwise layer just before it, when that layer sums nothing for a
//    mean: one launch of both (dwpw_tile), the depthwise map never stored.
// The depthwise launch shape of an operation (pointers unset).
static DwArgs dw_shape(const Op &op) {
  DwArgs a{};
  a.lanes = 1;
  a.ih = int(op.ih), a.iw = int(op.iw), a.c = int(op.oc), a.oh = int(op.oh), a.ow = int(op.ow);
  a.kh = int(op.kh), a.kw = int(op.kw), a.sh = int(op.sh), a.sw = int(op.sw);
  a.pt = int(op.pt), a.pl = int(op.pl);
  return a;
}

// How a channel-mean step's launch is cut, for L lanes of the batch's plan.
static MeanShape mean_step_shape(const Step &s, const Plan &p, size_t L) {
  const Op &op = p.ops[size_t(s.op)];
  int rows = 0;
  if (s.mean_of_dw >= 0) {
    DwArgs d = dw_shape(p.ops[size_t(s.mean_of_dw)]);
    d.lanes = int(L);
    rows = dw_mean_blocks(d);
  }
  return mean_shape(s.mean_of_dw < 0, int(op.ih * op.iw), int(op.ic), int(L), rows, s.fc1 >= 0);
}

bool Model::build_steps(std::string &err) {
  const auto &ops = plan.ops;
  const size_t n = ops.size();
  std::vector<size_t> readers(plan.pool.size(), 0);
  std::vector<size_t> writer(plan.pool.size(), SIZE_MAX);
  for (size_t i = 0; i < n; i++) {
    readers[ops[i].x]++;
    size_t x2;
    if (ops[i].has_second(&x2)) readers[x2]++;
    if (writer[ops[i].y] != SIZE_MAX) {
      err = fmt("operation %zu writes buffer %zu again", i, ops[i].y);  // gpu/mod.rs:622-630
      return false;
    }
    writer[ops[i].y] = i;
  }
  for (size_t s : plan.out_slot) readers[s]++;

  for (size_t i = 0; i < n; i++) {  // gpu/mod.rs:633-649
    const Op &op = ops[i];
    if (op.kind == K_CTCHEAD) return err = fmt("operation %zu: the CTC head with probabilities", i), false;
    if (op.kind == K_ATTENTION && op.oc / op.n2 > 64)
      return err = fmt("operation %zu: attention heads too large", i), false;
  }

  auto residual_gate = [&](size_t m) {
    if (m + 1 >= n) return false;
    const Op &g = ops[m], &a = ops[m + 1];
    return g.kind == K_CHANNELMUL && g.fused == 0 && readers[g.y] == 1 && a.kind == K_ADD &&
           a.fused == 0 && a.x == g.x && a.x2 == g.y;
  };
  auto foldable = [&](size_t i, size_t slot) -> int {
    size_t p = writer[slot];
    if (p == SIZE_MAX || p >= i || readers[slot] != 1) return -1;
    const Op &o = ops[p];
    bool up = o.kind == K_UPSAMPLE && o.sh == o.sw && o.sh > 1 && (o.sh & (o.sh - 1)) == 0;
    return (o.kind == K_CONCATC || up) ? int(p) : -1;
  };
  std::function<void(size_t, size_t, int, int, std::vector<Source> &, std::vector<int> &)> expand =
      [&](size_t i, size_t slot, int ch, int shift, std::vector<Source> &srcs,
          std::vector<int> &producers) {
        int p = foldable(i, slot);
        if (p < 0) {
          srcs.push_back({slot, ch, shift});
          return;
        }
        producers.push_back(p);
        const Op &o = ops[p];
        if (o.kind == K_CONCATC) {
          expand(p, o.x, int(o.ic), shift, srcs, producers);
          expand(p, o.x2, int(o.n2), shift, srcs, producers);
        } else {
          int k = 0;
          while ((size_t(1) << k) < o.sh) k++;
          expand(p, o.x, ch, shift + k, srcs, producers);
        }
      };

  // Op k is a 1x1 convolution of one input, `from`, which nothing else reads.
  auto plain_1x1 = [&](size_t k, size_t from) {
    return k < n && ops[k].kind == K_CONV && ops[k].is_pointwise() && ops[k].x == from && ops[k].n2 == 0 &&
           readers[from] == 1;
  };
  // Op k adds `from` (which nothing else reads) and `other`.
  auto adds = [&](size_t k, size_t from, size_t other) {
    return k < n && ops[k].kind == K_ADD && readers[from] == 1 &&
           ((ops[k].x == from && ops[k].x2 == other) || (ops[k].x2 == from && ops[k].x == other));
  };
  // Op k adds `from` (which nothing else reads) to another buffer.
  auto add_after = [&](size_t k, size_t from) {
    return k < n && ops[k].kind == K_ADD && readers[from] == 1 && ((ops[k].x == from) != (ops[k].x2 == from));
  };

  // Operation i as the stem block's RGB stem: q = its two 2x2 layers (a
  // 2x2 stride-1 convolution padded right and bottom by one) and its pool.
  auto stem_block_at = [&](size_t i, int q[3]) {
    const Op &s1 = ops[i];
    if (!(s1.kh == 3 && s1.kw == 3 && s1.sh == 2 && s1.sw == 2 && s1.pt == 1 && s1.pl == 1 && s1.ic == 3 &&
          s1.n2 == 0 && readers[s1.y] == 2))
      return false;
    auto pad2x2 = [&](const Op &o, size_t from) {
      return o.kind == K_CONV && o.x == from && o.n2 == 0 && o.kh == 2 && o.kw == 2 && o.sh == 1 && o.sw == 1 &&
             o.pt == 0 && o.pl == 0 && o.oh == o.ih && o.ow == o.iw;
    };
    int c2 = -1, c3 = -1, pool = -1;
    for (size_t j = i + 1; j < n; j++) {
      const Op &o = ops[j];
      if (o.x == s1.y && pad2x2(o, s1.y)) c2 = int(j);
      if (o.x == s1.y && o.kind == K_MAXPOOL && o.kh == 2 && o.kw == 2 && o.sh == 1 && o.sw == 1 &&
          o.oh == o.ih && o.ow == o.iw)
        pool = int(j);
      if (c2 >= 0 && c3 < 0 && pad2x2(o, ops[size_t(c2)].y)) c3 = int(j);
    }
    if (c2 < 0 || c3 < 0 || pool < 0 || readers[ops[size_t(c2)].y] != 1) return false;
    const Op &o2 = ops[size_t(c2)], &o3 = ops[size_t(c3)];
    // An Add after the second 2x2 that only it feeds would fold into it.
    if (readers[o3.y] == 1 && size_t(c3) + 1 < n && ops[size_t(c3) + 1].kind == K_ADD &&
        (ops[size_t(c3) + 1].x == o3.y || ops[size_t(c3) + 1].x2 == o3.y))
      return false;
    if (!stem_block_supported(int(s1.oc), int(o2.oc), int(o3.oc), s1.fused, o2.fused, o3.fused)) return false;
    q[0] = c2, q[1] = c3, q[2] = pool;
    return true;
  };

  std::vector<bool> folded(n, false);
  std::vector<int> inside;
  steps.clear();
  for (size_t i = 0; i < n; i++) {
    if (folded[i]) continue;
    const Op &op = ops[i];
    Step s{};
    s.op = int(i);
    switch (op.kind) {
      case K_MEAN: {
        s.kind = S_MEAN;
        if (i + 2 < n && readers[op.y] == 1) {
          const Op &f1 = ops[i + 1], &f2 = ops[i + 2];
          if (f1.kind == K_CONV && f1.is_pointwise() && f1.x == op.y && f2.kind == K_CONV &&
              f2.is_pointwise() && f2.x == f1.y && readers[f1.y] == 1 && f1.n2 == 0 && f2.n2 == 0 &&
              se_supported(int(f1.ic), int(f1.oc), int(f2.oc))) {
            s.fc1 = int(i + 1), s.fc2 = int(i + 2);
            folded[i + 1] = folded[i + 2] = true;
          }
        }
        break;
      }
      case K_CHANNELMUL:
        s.kind = S_ELT;
        if (residual_gate(i)) {
          s.elt = ELT_RESGATE;
          s.resgate = int(i);
          s.add = int(i + 1);
          folded[i + 1] = true;
        } else {
          s.elt = ELT_CHANNELMUL;
        }
        break;
      case K_CONV: {
        s.kind = S_GEMM;
        size_t p = writer[op.x];
        if (p != SIZE_MAX && p < i && ops[p].kind == K_CHANNELMUL && readers[op.x] == 1 &&
            op.x != op.x2 && !residual_gate(p)) {
          s.gate = int(p);
          inside.push_back(int(p));
          s.sources.push_back({ops[p].x, int(op.ic), 0});
          if (op.n2) s.sources.push_back({op.x2, int(op.n2), 0});
        } else {
          std::vector<Source> srcs;
          std::vector<int> producers;
          expand(i, op.x, int(op.ic), 0, srcs, producers);
          if (op.n2) expand(i, op.x2, int(op.n2), 0, srcs, producers);
          bool plain = srcs.size() <= 2;
          for (auto &x : srcs) plain = plain && x.shift == 0;
          if (srcs.size() <= 4 && !plain) {
            s.sources = srcs;
            inside.insert(inside.end(), producers.begin(), producers.end());
          } else {
            s.sources.push_back({op.x, int(op.ic), 0});
            if (op.n2) s.sources.push_back({op.x2, int(op.n2), 0});
          }
        }
        if (readers[op.y] == 1 && i + 1 < n && ops[i + 1].kind == K_ADD &&
            ((ops[i + 1].x == op.y) != (ops[i + 1].x2 == op.y))) {
          s.add = int(i + 1);
          folded[i + 1] = true;
        }
        // A windowed convolution over a few channels that are not a multiple
        // of four (the RGB stem): computed directly.
        if (s.gate < 0 && s.add < 0 && op.n2 == 0 && s.sources.size() == 1 && s.sources[0].shift == 0 &&
            !op.is_pointwise() &&
            ((op.ic % 4 != 0 && direct_supported(int(op.kh), int(op.kw), int(op.ic))) ||
             direct_pix_supported(int(op.kh), int(op.kw), int(op.ic), int(op.oc))))
          s.kind = S_DIRECT;
        // The stem block: a 3x3 stride-2 RGB stem whose map only a 2x2 max
        // pool and a 2x2 layer read, that layer's map only a second 2x2
        // layer: one step, neither map stored.
        if (s.kind == S_DIRECT) {
          int q[3];
          if (stem_block_at(i, q)) {
            s.kind = S_STEM;
            s.st2 = q[0], s.st3 = q[1], s.st_pool = q[2];
            for (int k : q) folded[size_t(k)] = true;
          }
        }
        break;
      }
      case K_DWCONV: s.kind = S_DW; break;
      case K_ADD: s.kind = S_ELT, s.elt = ELT_ADD; break;
      case K_MAXPOOL: case K_AVGPOOL: s.kind = S_POOL; break;
      case K_CONCATC: s.kind = S_ELT, s.elt = ELT_CONCAT; break;
      case K_UPSAMPLE: s.kind = S_ELT, s.elt = ELT_UPSAMPLE; break;
      case K_UPSAMPLEADD: {
        s.kind = S_ELT, s.elt = ELT_UPSAMPLEADD;
        size_t a = writer[op.x2];
        if (readers[op.x2] == 1 && a != SIZE_MAX && a > 0 && a < i && residual_gate(a - 1)) {
          s.elt = ELT_UPSAMPLEADD_RESGATE;
          s.resgate = int(a - 1);
          inside.push_back(int(a - 1));
        }
        break;
      }
      case K_LAYERNORM: {
        // The encoder's pre-norm layers: LayerNorm -> 1x1 -> 1x1 -> Add of
        // the LayerNorm's input (the MLP and its residual), with the next
        // LayerNorm folded in when only it reads the sum; else LayerNorm ->
        // 1x1 (the q|k|v projection), with an Add after it folded in.
        s.kind = S_LN;
        const size_t c = op.oc;
        if (plain_1x1(i + 1, op.y) && ops[i + 1].ic == c && plain_1x1(i + 2, ops[i + 1].y) &&
            ops[i + 2].oc == c && adds(i + 3, ops[i + 2].y, op.x) &&
            enc_mlp_supported(int(c), int(ops[i + 1].oc))) {
          s.kind = S_ENC_MLP;
          s.fc1 = int(i + 1), s.fc2 = int(i + 2), s.add = int(i + 3);
          folded[i + 1] = folded[i + 2] = folded[i + 3] = true;
          const size_t z = ops[i + 3].y;
          if (i + 4 < n && ops[i + 4].kind == K_LAYERNORM && ops[i + 4].x == z && readers[z] == 1 &&
              ops[i + 4].oc == c) {
            s.ln_out = int(i + 4);
            folded[i + 4] = true;
          }
        } else if (plain_1x1(i + 1, op.y) && ops[i + 1].ic == c &&
                   enc_linear_supported(int(c), int(ops[i + 1].oc))) {
          s.kind = S_ENC_LIN;
          s.fc1 = int(i + 1);
          folded[i + 1] = true;
          if (add_after(i + 2, ops[i + 1].y)) s.add = int(i + 2), folded[i + 2] = true;
        }
        break;
      }
      case K_ATTENTION: {
        // Attention -> its c -> c output projection, with an Add after it.
        s.kind = S_ATTN;
        const size_t c = op.oc;
        if (plain_1x1(i + 1, op.y) && ops[i + 1].ic == c && ops[i + 1].oc == c &&
            enc_attn_supported(int(c), int(op.n2), 0)) {
          s.kind = S_ENC_ATTN;
          s.fc1 = int(i + 1);
          folded[i + 1] = true;
          if (add_after(i + 2, ops[i + 1].y)) s.add = int(i + 2), folded[i + 2] = true;
        }
        break;
      }
      case K_CTCARGMAX: s.kind = S_CTC; break;
      case K_CONVTRANSPOSE: {
        s.kind = op.kh * op.kw * op.oc <= 16 ? S_CONVT : S_GEMM;
        // The DB head: a 2x2 stride-2 transposed convolution whose output only
        // a second one to a single channel reads: one step, the intermediate
        // map never stored.
        auto two = [](const Op &o) { return o.kh == 2 && o.kw == 2 && o.sh == 2 && o.sw == 2; };
        if (s.kind == S_GEMM && i + 1 < n && readers[op.y] == 1) {
          const Op &o2 = ops[i + 1];
          if (o2.kind == K_CONVTRANSPOSE && o2.x == op.y && two(op) && two(o2) && o2.oc == 1 &&
              o2.ic == op.oc && head_supported(int(op.ic), int(op.oc))) {
            s.kind = S_HEAD;
            s.head2 = int(i + 1);
            folded[i + 1] = true;
          }
        }
        if (s.kind == S_GEMM) s.sources.push_back({op.x, int(op.ic), 0});
        break;
      }
      default:
        return err = fmt("operation %zu: %s is not supported on the GPU", i, kind_name(op.kind)), false;
    }
    steps.push_back(s);
  }
  steps.erase(std::remove_if(steps.begin(), steps.end(),
                             [&](const Step &s) {
                               return std::find(inside.begin(), inside.end(), s.op) != inside.end();
                             }),
              steps.end());
  // Attention -> projection -> Add, then the MLP of that sum when nothing
  // else reads the sum (its LayerNorm and its residual Add): one step, the
  // sum never stored.
  for (size_t k = 1; k < steps.size(); k++) {
    Step &a = steps[k - 1], &m = steps[k];
    if (a.kind != S_ENC_ATTN || a.add < 0 || m.kind != S_ENC_MLP) continue;
    const size_t z = ops[a.add].y;
    const Op &att = ops[a.op];
    if (ops[m.op].x != z || readers[z] != 2 ||
        !enc_attn_supported(int(att.oc), int(att.n2), int(ops[m.fc1].oc)))
      continue;
    a.kind = S_ENC_BLOCK;
    a.m_ln = m.op, a.m_fc1 = m.fc1, a.m_fc2 = m.fc2, a.m_add = m.add, a.ln_out = m.ln_out;
    steps.erase(steps.begin() + k);
  }
  // A stem block whose pool and second 2x2 only one convolution reads, as
  // its two sources in that order: both written as one map (pool channels,
  // then the 2x2's), the convolution's single source.
  for (Step &st : steps) {
    if (st.kind != S_STEM) continue;
    const size_t yp = ops[st.st_pool].y, y3 = ops[st.st3].y;
    if (readers[yp] != 1 || readers[y3] != 1) continue;
    for (Step &c : steps) {
      if (c.kind != S_GEMM || c.gate >= 0 || c.sources.size() != 2 || c.sources[0].slot != yp ||
          c.sources[1].slot != y3 || c.sources[0].shift || c.sources[1].shift)
        continue;
      c.sources = {{yp, c.sources[0].c + c.sources[1].c, 0}};
      st.st_joint = true;
    }
  }
  // Chains of 2x upsample-adds, each level's map the next one's upsampled
  // source (a feature pyramid's top-down sums): one step, in the finest
  // level's place, that writes every level (upadd_chain). Every other reader
  // of a coarser level must come after that place.
  {
    auto upadd = [&](const Step &t) {
      return t.kind == S_ELT && t.chain.empty() && (t.elt == ELT_UPSAMPLEADD || t.elt == ELT_UPSAMPLEADD_RESGATE) &&
             ops[t.op].sh == 2 && ops[t.op].sw == 2 && ops[t.op].oc % 4 == 0;
    };
    std::vector<int> prod(plan.pool.size(), -1);
    std::vector<std::vector<int>> rd(plan.pool.size());
    for (size_t k = 0; k < steps.size(); k++) {
      prod[step_writes(steps[k])] = int(k);
      for (size_t sl : step_reads(steps[k])) rd[sl].push_back(int(k));
    }
    std::vector<bool> drop(steps.size(), false);
    for (int f = int(steps.size()) - 1; f >= 0; f--) {
      if (drop[size_t(f)] || !upadd(steps[size_t(f)])) continue;
      std::vector<int> lv{f};
      while (lv.size() < size_t(kChainMax)) {
        const int q = prod[ops[steps[size_t(lv.back())].op].x];
        if (q < 0 || drop[size_t(q)] || !upadd(steps[size_t(q)]) || ops[steps[size_t(q)].op].oc != ops[steps[size_t(f)].op].oc)
          break;
        bool later = true;
        for (int r : rd[ops[steps[size_t(q)].op].y]) later = later && (r == lv.back() || r > f);
        if (!later) break;
        lv.push_back(q);
      }
      if (lv.size() < 2) continue;
      std::vector<int> ch, cg;
      for (int k : lv) ch.push_back(steps[size_t(k)].op), cg.push_back(steps[size_t(k)].resgate);
      steps[size_t(f)].chain = ch, steps[size_t(f)].chain_gate = cg;
      for (size_t k = 1; k < lv.size(); k++) drop[size_t(lv[k])] = true;
    }
    std::vector<Step> kept;
    for (size_t k = 0; k < steps.size(); k++)
      if (!drop[k]) kept.push_back(steps[k]);
    steps = kept;
  }
  // A channel mean right after the depthwise convolution that produces its
  // input: the depthwise kernel sums its outputs per channel as it stores
  // them, and the mean step only joins those sums (no second read).
  for (size_t k = 1; k < steps.size(); k++) {
    Step &d = steps[k - 1], &m = steps[k];
    if (d.kind != S_DW || m.kind != S_MEAN || ops[d.op].y != ops[m.op].x) continue;
    if (dw_mean_supported(dw_shape(ops[d.op]))) {
      d.dw_sums = true;
      m.mean_of_dw = d.op;
    }
  }
  return true;
}

// Choose each GEMM step's reduction chunk and tile, and repack its weights:
// Rows per wave of the halo tiles (tiles of 4 * wr rows): two when there is
// about a tile of 8 rows per CU or more and those tiles take no more rounds
// of the GPU's workgroup slots than tiles of 4 rows, counted in units of a
// 4-row tile's work; else one. A CU holds as many tiles as its 160 KiB of
// LDS takes, four at most (their registers). Measured on the detector: the
// four neck convolutions together (610 tiles of 8 rows, 1.2 rounds) run 7%
// faster on 4-row tiles, the head's (450) 13% slower.
static int patch_rows(long tiles4, long tiles8, bool fits2, size_t lds4, size_t lds8) {
  constexpr long kCUs = 256;  // MI355X
  auto slots = [](size_t lds) { return kCUs * std::max<long>(1, std::min<long>(4, long(160 * 1024 / std::max<size_t>(lds, 1)))); };
  const long s4 = slots(lds4), s8 = slots(lds8);
  const long r4 = (tiles4 + s4 - 1) / s4, r8 = 2 * ((tiles8 + s8 - 1) / s8);
  return fits2 && tiles8 >= 256 && r8 <= r4 ? 2 : 1;
}

// The LDS-ring GEMM's tile for an M x N product, from a sweep of tiles,
// stage counts and chunk widths over the detector's and recogniser's 1x1
// layers: 32-row tiles throughout (more workgroups per CU beat larger
// tiles); 96 columns when N is 96 and that leaves over one tile per CU,
// 64 when that leaves about three, else 32; three stages when tiles are
// plentiful (more of them fit a CU), else four.
static RingTile ring_tile(long M, int N) {
  auto tiles = [&](int n) { return (M + 31) / 32 * ((N + 32L * n - 1) / (32L * n)); };
  int nt = 1;
  if (N == 96 && tiles(3) >= 384)
    nt = 3;
  else if (N > 32 && (N <= 64 || tiles(2) >= 768))
    nt = 2;
  return RingTile{1, nt, tiles(nt) >= 512 ? 3 : 4, 32};
}

// Rounds of workgroups a ring launch of `tiles` tiles takes: a CU holds as
// many as its 160 KB of LDS and its 32 wave slots (eight workgroups of four
// waves) allow.
static long ring_rounds(long tiles, size_t lds) {
  constexpr long kCUs = 256;  // MI355X
  const long per_cu = std::max<long>(1, std::min<long>(8, long(160 * 1024 / std::max<size_t>(lds, 1))));
  return (tiles + kCUs * per_cu - 1) / (kCUs * per_cu);
}

// ring_tile for the launch of `as` (M rows in all), with two stages instead
// of three where that leaves room for enough workgroups a CU to run every
// tile in fewer rounds: a launch one round longer than it needs waits out
// its last workgroups with the GPU nearly idle (the fused block's gated
// 96 -> 96 1x1 over 160 x 160 pixels: 800 tiles, 768 at once with three
// stages, 1024 with two).
static RingTile ring_tile(const std::vector<ConvArgs> &as, long M) {
  RingTile t = ring_tile(M, as[0].n);
  if (t.st != 3) return t;
  long tiles = 0;
  size_t lds3 = 0, lds2 = 0;
  RingTile t2 = t;
  t2.st = 2;
  for (const ConvArgs &a : as) {
    tiles += (long(a.lanes) * a.oh * a.ow + 31) / 32 * ((a.n + 32L * t.nt - 1) / (32L * t.nt));
    lds3 = std::max(lds3, ring_lds_bytes(a, t));
    lds2 = std::max(lds2, ring_lds_bytes(a, t2));
  }
  return ring_rounds(tiles, lds2) < ring_rounds(tiles, lds3) ? t2 : t;
}

// row n of the packed matrix holds column n's reduction in the kernel's chunk
// order, zero where the padding of a chunk lies.
//  - channel layout (every source's channels a multiple of 4): per tap, the
//    tap's concatenated channels padded to cpt * BK;
//  - flat layout: taps * channels as one run padded to whole chunks.
// BK: the largest of 64, 32, 16, 8 that pads a tap's channels by at most an
// eighth, else the one that pads least: fewer chunks mean fewer load
// latencies in sequence, which is what small layers wait on.
bool Model::pack(std::string &err) {
  std::vector<float> packed;
  const auto &ops = plan.ops;
  for (Step &s : steps) {
    if (s.kind == S_MEAN && s.fc1 >= 0) {
      // The squeeze-and-excite's two 1x1 layers in the kernel's groups of
      // four inputs, each starting on a 256-byte boundary.
      const Op &f1 = ops[size_t(s.fc1)], &f2 = ops[size_t(s.fc2)];
      s.se_w1 = round_up(packed.size(), 64);
      packed.resize(s.se_w1 + se_pack_floats(int(f1.ic), int(f1.oc)), 0.0f);
      se_pack(weights.data() + f1.w0, int(f1.ic), int(f1.oc), packed.data() + s.se_w1);
      s.se_w2 = round_up(packed.size(), 64);
      packed.resize(s.se_w2 + se_pack_floats(int(f2.ic), int(f2.oc)), 0.0f);
      se_pack(weights.data() + f2.w0, int(f2.ic), int(f2.oc), packed.data() + s.se_w2);
      continue;
    }
    if (s.kind == S_ENC_LIN || s.kind == S_ENC_ATTN || s.kind == S_ENC_MLP || s.kind == S_ENC_BLOCK) {
      // The encoder's 1x1 layers in MFMA operand order.
      auto put = [&](const Op &f, int kp) {
        const size_t at = round_up(packed.size(), 64);
        packed.resize(at + enc_pack_floats(kp, int(f.oc)), 0.0f);
        enc_pack(weights.data() + f.w0, int(f.ic), int(f.oc), kp, packed.data() + at);
        return at;
      };
      const Op &f1 = ops[size_t(s.fc1)];
      if (s.kind == S_ENC_BLOCK) {
        const Op &g1 = ops[size_t(s.m_fc1)], &g2 = ops[size_t(s.m_fc2)];
        s.enc_w1 = put(f1, enc_kpad(int(f1.ic)));
        s.enc_w2 = put(g1, enc_kpad(int(g1.ic)));
        s.enc_w3 = put(g2, enc_mlp_hpad(int(g2.ic)));
      } else if (s.kind == S_ENC_MLP) {
        const Op &f2 = ops[size_t(s.fc2)];
        s.enc_w1 = put(f1, enc_kpad(int(f1.ic)));
        s.enc_w2 = put(f2, enc_mlp_hpad(int(f2.ic)));
      } else {
        s.enc_w1 = put(f1, enc_kpad(int(f1.ic)));
      }
      continue;
    }
    if (s.kind != S_GEMM && s.kind != S_CTC) continue;
    const Op &op = ops[s.op];
    int taps = 1, N;
    std::vector<Source> srcs = s.sources;
    if (s.kind == S_CTC) {
      srcs = {{op.x, int(op.ic), 0}};
      N = int(op.n2);
    } else if (op.kind == K_CONVTRANSPOSE) {
      N = int(op.kh * op.kw * op.oc);
    } else {
      taps = int(op.kh * op.kw);
      N = int(op.oc);
    }
    bool vec = true;
    int ctot = 0;
    for (auto &x : srcs) vec = vec && x.c % 4 == 0, ctot += x.c;
    bool pw = (op.kind != K_CONV || op.is_pointwise()) && srcs.size() == 1 && srcs[0].shift == 0 && vec;
    int bk, cpt = 0;
    if (vec) {
      int best = 0;
      double best_waste = 1e9;
      for (int cand : {64, 32, 16, 8}) {
        double waste = double((ctot + cand - 1) / cand * cand) / ctot - 1.0;
        if (waste <= 0.125) {
          best = cand;
          break;
        }
        if (waste < best_waste - 1e-12) best = cand, best_waste = waste;
      }
      bk = best;
      // A windowed convolution over 48 channels in all, or over 96 on a small
      // map: one chunk per tap, fewer load round trips in sequence (a large
      // map keeps chunks of 32: more waves per CU hide the loads better).
      bool shifted = false;
      for (auto &x : srcs) shifted = shifted || x.shift > 0;
      const size_t out_px = op.oh * op.ow;
      if (s.kind == S_GEMM && op.kind == K_CONV && !pw && !shifted &&
          (ctot == 48 || (ctot == 96 && out_px < 16384)))
        bk = ctot;
      // The CTC head has thousands of tiles and is throughput-bound: small
      // chunks keep the LDS footprint small and the occupancy high.
      if (s.kind == S_CTC) bk = 8;
      // A windowed convolution up to 3 x 3, stride 1 or 2: halo tiles (each
      // source pixel decoded once per channel block, not once per tap), whose
      // channel block (the chunk) is at most 32 and small enough that the
      // patch and the block's weights fit in LDS.
      // Measured on the detector: halo tiles win over upsampled sources and
      // on maps under 128 x 128; the implicit GEMM keeps large maps.
      const bool halo = shifted || out_px < 16384 || (op.kh == 3 && op.sh == 1);
      if (s.kind == S_GEMM && op.kind == K_CONV && !pw && op.kh <= 3 && op.kw <= 3 && op.sh == op.sw &&
          (op.sh == 1 || op.sh == 2) && halo) {
        const int bn0 = N <= 16 ? 16 : (N <= 32 ? 32 : 64);
        int pb = 0;
        double pw_best = 1e9;
        for (int cand : {32, 16, 8}) {
          if (!patch_fits(int(op.kh), int(op.kw), int(op.sh), 1, cand, bn0)) continue;
          double waste = double((ctot + cand - 1) / cand * cand) / ctot - 1.0;
          if (waste <= 0.125) {
            pb = cand;
            break;
          }
          if (waste < pw_best - 1e-12) pb = cand, pw_best = waste;
        }
        if (pb) s.patch = true, bk = pb;
      }
      // A windowed convolution that neither halo tiles nor the register-staged
      // implicit GEMM take well (a window wider than 3 or unequal strides)
      // and has no gate: the LDS ring, whose direct loads fetch each tap's
      // channels in chunks of 32. (On the stem's large maps the ring's
      // 32-row tiles re-read each tap's rows and the weights from L2 per
      // tile and lose to the 128-row implicit GEMM.)
      if (s.kind == S_GEMM && op.kind == K_CONV && !pw && !s.patch && s.gate < 0 &&
          (op.kh > 3 || op.kw > 3 || op.sh != op.sw || op.kh * op.kw == 1))
        s.ring = true, bk = 32;
      cpt = (ctot + bk - 1) / bk;
      s.chunks = taps * cpt;
    } else {
      int K = taps * ctot;
      bk = K <= 8 ? 8 : (K <= 16 ? 16 : 32);
      s.chunks = (K + bk - 1) / bk;
    }
    int bn = N <= 16 ? 16 : (N <= 32 ? 32 : 64);
    if (s.kind == S_CTC) bn = 64;
    int wm = bk >= 48 ? 16 : 32;
    s.tile = GemmTile{wm, bn, bk, vec, pw};
    if (!gemm_tile_supported(s.tile) && s.kind != S_CTC)
      return err = fmt("operation %d: no GEMM tile for this shape", s.op), false;
    s.gemm_n = N;
    s.ctot = ctot;
    s.cpt = cpt;
    s.wt_k = size_t(s.chunks) * bk;
    int n_pad = (N + bn - 1) / bn * bn;
    size_t start = round_up(packed.size(), 64);
    packed.resize(start + size_t(n_pad) * s.wt_k, 0.0f);
    s.wt_off = start;
    float *dst = packed.data() + start;
    const float *w = weights.data() + op.w0;
    for (int nn = 0; nn < N; nn++) {
      float *row = dst + size_t(nn) * s.wt_k;
      for (int tap = 0; tap < taps; tap++) {
        for (int c = 0; c < ctot; c++) {
          size_t kk = size_t(tap) * ctot + c;  // the plan's reduction index
          size_t k = vec ? size_t(tap) * cpt * bk + c : kk;
          row[k] = s.kind == S_CTC ? w[(size_t(nn) / 16) * op.ic * 16 + kk * 16 + nn % 16]
                                   : w[kk * N + nn];
        }
      }
    }
    if (s.kind == S_CTC) {
      double bm = 0, wm = 0;
      for (int nn = 0; nn < N; nn++) {
        double ws = 0;
        for (size_t k = 0; k < op.ic; k++) ws += std::fabs(double(w[(size_t(nn) / 16) * op.ic * 16 + k * 16 + nn % 16]));
        wm = std::max(wm, ws);
        if (op.b1) bm = std::max(bm, std::fabs(double(weights[op.b0 + size_t(nn)])));
      }
      // Rounded up to the next float.
      s.ctc_bias_max = std::nextafter(float(bm), INFINITY), s.ctc_wsum_max = std::nextafter(float(wm), INFINITY);
    }
    if (s.kind == S_CTC && ctc_direct_supported(int(op.ic))) {
      // The same weights in MFMA operand order for ctc_direct (the rows above
      // serve ctc_merge's exact recomputation of near ties): for column block
      // j and input group q of 16, lane l's four inputs 16q + 4(l / 16) + e of
      // column 16j + l % 16, from the plan's panels of 16 columns.
      const int ci = int(op.ic), kp = enc_kpad(ci), kq = kp / 16, nb = (N + 15) / 16;
      s.enc_w1 = round_up(packed.size(), 64);
      packed.resize(s.enc_w1 + enc_pack_floats(kp, N), 0.0f);
      float *o = packed.data() + s.enc_w1;
      for (int j = 0; j < nb; j++)
        for (int q = 0; q < kq; q++)
          for (int l = 0; l < 64; l++)
            for (int e = 0; e < 4; e++) {
              const int kk = 16 * q + 4 * (l >> 4) + e, nn = 16 * j + (l & 15);
              if (kk < ci && nn < N)
                o[(((size_t)j * kq + q) * 64 + l) * 4 + e] = w[(size_t(nn) / 16) * ci * 16 + size_t(kk) * 16 + nn % 16];
            }
    }
  }
  // Depthwise layers and the 1x1 convolution that alone reads each: one
  // step, the 1x1's weights packed in MFMA operand order over its c inputs.
  {
    const auto &ops = plan.ops;
    std::vector<size_t> readers(plan.pool.size(), 0);
    for (const Op &o : ops) {
      readers[o.x]++;
      size_t x2;
      if (o.has_second(&x2)) readers[x2]++;
    }
    for (size_t sl : plan.out_slot) readers[sl]++;
    for (size_t k = 0; k + 1 < steps.size(); k++) {
      Step &d = steps[k];
      const Step &c = steps[k + 1];
      const Op &dop = ops[size_t(d.op)], &co = ops[size_t(c.op)];
      if (d.kind != S_DW || d.dw_sums || d.pw1 >= 0 || c.kind != S_GEMM || c.patch || c.ring || c.pw1 >= 0) continue;
      if (co.kind != K_CONV || !co.is_pointwise() || co.n2 || co.x != dop.y || readers[dop.y] != 1) continue;
      if (c.gate >= 0 || c.sources.size() != 1 || c.sources[0].shift || !dwpw_supported(dw_shape(dop), int(co.oc), c.add >= 0))
        continue;
      const int ci = int(dop.oc), n = int(co.oc);
      d.enc_w1 = round_up(packed.size(), 64);
      packed.resize(d.enc_w1 + enc_pack_floats(ci, n), 0.0f);
      enc_pack(weights.data() + co.w0, ci, n, ci, packed.data() + d.enc_w1);
      d.pw1 = c.op;
      d.add = c.add;
      steps.erase(steps.begin() + long(k) + 1);
    }
  }
  if (packed.empty()) return true;
  HIPTRY(hipMalloc(&dpacked, packed.size() * sizeof(float)), "allocating packed weights");
  HIPTRY(hipMemcpy(dpacked, packed.data(), packed.size() * sizeof(float), hipMemcpyHostToDevice),
         "uploading packed weights");
  // A 1x1 convolution whose input only the implicit-GEMM convolution just
  // before it writes and nothing else reads: folded into that convolution's
  // epilogue, whose tile holds every output column of its pixels (16-row
  // MFMA blocks a wave); the 1x1's map is then the only one stored.
  {
    const auto &ops = plan.ops;
    std::vector<size_t> readers(plan.pool.size(), 0);
    for (const Op &o : ops) {
      readers[o.x]++;
      size_t x2;
      if (o.has_second(&x2)) readers[x2]++;
    }
    for (size_t sl : plan.out_slot) readers[sl]++;
    for (size_t k = 0; k + 1 < steps.size(); k++) {
      Step &g = steps[k];
      const Step &c = steps[k + 1];
      const Op &go = ops[size_t(g.op)], &co = ops[size_t(c.op)];
      if (g.kind != S_GEMM || c.kind != S_GEMM || g.patch || g.ring || g.add >= 0 || g.pw1 >= 0) continue;
      if (go.kind != K_CONV || co.kind != K_CONV || !co.is_pointwise() || co.n2 || co.x != go.y) continue;
      if (readers[go.y] != 1 || c.gate >= 0 || c.add >= 0 || c.sources.size() != 1 || c.sources[0].shift) continue;
      GemmTile t = g.tile;
      t.wm = 16;
      ConvArgs probe{};
      probe.mode = GEMM_STORE, probe.n = g.gemm_n, probe.pw_n = int(co.oc);
      if (!gemm_tile_supported(t) || !conv_pw_supported(probe, t)) continue;
      g.tile = t;
      g.pw1 = c.op;
      steps.erase(steps.begin() + long(k) + 1);
    }
  }
  return true;
}

bool Model::load(const uint8_t *bytes, size_t len, std::string &err) {
  if (!plan.parse(bytes, len, weights, err)) return false;
  if (!build_steps(err)) return false;
  HIPTRY(hipGetDevice(&device), "no GPU");
  hipDeviceProp_t prop;
  HIPTRY(hipGetDeviceProperties(&prop, device), "reading the GPU's properties");
  name = prop.name;
  if (name.empty()) name = prop.gcnArchName;
  integrated = prop.integrated;
  device_bytes = prop.totalGlobalMem;
  // The weights go up (on the null stream) before the model's stream is
  // created: HIP gives a process's streams its hardware queues in the order
  // they are first used, and a null stream first used after the streams of
  // several models that run at once (the page path: a detector and three
  // recognisers) slowed them (1.47 -> 1.80 ms a page, with eight queues).
  HIPTRY(hipMalloc(&dweights, std::max<size_t>(weights.size(), 1) * sizeof(float)),
         "allocating the weights");
  if (!weights.empty())
    HIPTRY(hipMemcpy(dweights, weights.data(), weights.size() * sizeof(float),
                     hipMemcpyHostToDevice),
           "uploading the weights");
  HIPTRY(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "creating a stream");
  if (!pack(err)) return false;
  size_t hw[2] = {plan.in_h, plan.in_w};
  return set_sizes(hw, 1, err);
}

// ---------------------------------------------------------------- memory

bool Model::arrange(Batch &b, std::string &err) {
  const Plan &p = b.plan;
  const size_t L = b.lanes.size();
  std::vector<size_t> last(p.pool.size(), 0);
  for (size_t i = 0; i < steps.size(); i++)
    for (size_t s : step_reads(steps[i])) last[s] = i;
  for (size_t s : p.out_slot) last[s] = SIZE_MAX;
  b.home.assign(p.pool.size(), SIZE_MAX);
  // Steps each step depends on through the data, transitively (the
  // launches' RAW edges). A freed home is reused only by a step that already
  // follows every reader of the home's last buffer: reuse then adds no
  // ordering the data does not, and independent steps stay independent.
  const size_t n = steps.size();
  std::vector<size_t> producer(p.pool.size(), SIZE_MAX);
  std::vector<std::vector<size_t>> slot_readers(p.pool.size());
  for (size_t i = 0; i < n; i++) {
    producer[step_writes(steps[i])] = i;
    for (size_t y2 : step_writes_extra(steps[i])) producer[y2] = i;
    for (size_t sl : step_reads(steps[i])) slot_readers[sl].push_back(i);
  }
  std::vector<std::vector<bool>> anc(n, std::vector<bool>(n, false));
  for (size_t i = 0; i < n; i++)
    for (size_t sl : step_reads(steps[i])) {
      const size_t w = producer[sl];
      if (w == SIZE_MAX || w >= i) continue;
      anc[i][w] = true;
      for (size_t k = 0; k < w; k++)
        if (anc[w][k]) anc[i][k] = true;
    }
  std::vector<size_t> sizes, freel;
  std::vector<std::vector<size_t>> held_by;  // per home: the readers of its last buffer
  // For step i: the smallest free home it may take that holds n floats,
  // else the largest it may take, grown; else a new home.
  auto place = [&](size_t need, size_t i) {
    need = round_up(std::max<size_t>(need, 1), 64);
    auto allowed = [&](size_t h) {
      if (!kGrouped) return true;
      for (size_t r : held_by[h])
        if (i == SIZE_MAX || !anc[i][r]) return false;
      return true;
    };
    int best = -1;
    for (size_t k = 0; k < freel.size(); k++)
      if (allowed(freel[k]) && sizes[freel[k]] >= need && (best < 0 || sizes[freel[k]] < sizes[freel[best]]))
        best = int(k);
    if (best < 0)
      for (size_t k = 0; k < freel.size(); k++)
        if (allowed(freel[k]) && (best < 0 || sizes[freel[k]] > sizes[freel[best]])) best = int(k);
    if (best >= 0) {
      size_t h = freel[best];
      freel.erase(freel.begin() + best);
      sizes[h] = std::max(sizes[h], need);
      return h;
    }
    sizes.push_back(need);
    held_by.emplace_back();
    return sizes.size() - 1;
  };
  b.home[p.in_slot] = place(p.pool[p.in_slot], SIZE_MAX);
  for (size_t i = 0; i < n; i++) {
    size_t y = step_writes(steps[i]);
    b.home[y] = place(p.pool[y] + (steps[i].st_joint ? p.pool[p.ops[steps[i].st3].y] : 0), i);
    for (size_t y2 : step_writes_extra(steps[i])) b.home[y2] = place(p.pool[y2], i);
    for (size_t sl : step_reads(steps[i]))
      if (last[sl] == i && std::find(freel.begin(), freel.end(), b.home[sl]) == freel.end()) {
        freel.push_back(b.home[sl]);
        held_by[b.home[sl]] = slot_readers[sl];
      }
  }
  b.home_floats = sizes;
  b.home_off.resize(sizes.size());
  size_t off = 0;
  for (size_t h = 0; h < sizes.size(); h++) {
    b.home_off[h] = off;
    off += round_up(sizes[h] * L, 64);
  }
  // Workspace: channel-mean partials (f64), CTC tile partials, attention
  // scores; each step its own region, so that steps which do not depend on
  // each other can run at the same time.
  size_t ws = 0;
  b.step_ws.assign(steps.size(), 0);
  for (size_t i = 0; i < steps.size(); i++) {
    const Step &s = steps[i];
    const Op &op = p.ops[s.op];
    size_t need = 0;
    if (s.kind == S_MEAN) {
      // Partial rows and gathered means, then the counters.
      const MeanShape m = mean_step_shape(s, p, L);
      need = round_up(m.floats, 4) + m.count_n;
    }
    if (s.kind == S_CTC) {
      size_t ntn = (s.gemm_n + s.tile.bn - 1) / s.tile.bn;
      need = L * op.iw * ntn * 4;
      if (ctc_direct_supported(int(op.ic))) {  // run records, then the per-tile maxima
        const CtcRuns r = ctc_direct_runs(long(L * op.iw), int(op.n2));
        need = std::max(need, L * op.iw * (size_t(r.runs) * 4 + (op.n2 + 63) / 64));
      }
    }
    if (s.kind == S_ATTN) need = attention_scratch_floats(int(op.iw), int(op.oc), int(op.n2), int(L));
    // Lines too long for the fused attention's LDS: attention rows, then the
    // projection over them.
    if ((s.kind == S_ENC_ATTN || s.kind == S_ENC_BLOCK) && !enc_attn_fits(int(op.iw), int(op.oc), int(op.n2), enc_hidden(s)))
      need = round_up(L * op.iw * op.oc, 64) * (s.kind == S_ENC_BLOCK ? 2 : 1) +
             attention_scratch_floats(int(op.iw), int(op.oc), int(op.n2), int(L));
    b.step_ws[i] = ws;
    ws += round_up(need, 64);
  }
  b.ws_off = off;
  off += round_up(std::max<size_t>(ws, 64), 64);
  b.bits_w = b.bits_h = b.bits_wpr = 0;
  if (db_output >= 0) {
    // The map: the last operation writing that output, one channel.
    const size_t slot = p.out_slot[size_t(db_output)];
    const Op *map = nullptr;
    for (const Op &o : p.ops)
      if (o.y == slot) map = &o;
    if (!map || map->oc != 1) return err = "the DB mask's output is not a one-channel map", false;
    b.bits_w = map->ow, b.bits_h = map->oh, b.bits_wpr = (map->ow + 63) / 64;
    b.bits_off = off;
    off += round_up(2 * L * b.bits_h * b.bits_wpr, 64);
  }
  if (off > b.arena_floats) {
    if (b.arena) {
      hipFree(b.arena);
      b.arena = nullptr;
      b.arena_floats = 0;
    }
    size_t want = off + off / 4;  // a quarter more for the next, slightly larger size
    HIPTRY(hipMalloc(&b.arena, want * sizeof(float)), fmt("allocating %zu bytes of device memory", want * 4).c_str());
    b.arena_floats = want;
  }
  b.in_len = p.in_h * p.in_w * p.in_c;
  if (b.host_in_cap < b.in_len * L) {
    if (b.host_in) hipHostFree(b.host_in);
    b.host_in = nullptr;
    b.host_in_cap = 0;
    size_t want = b.in_len * L + b.in_len * L / 4;
    HIPTRY(hipHostMalloc(&b.host_in, want * sizeof(float), hipHostMallocDefault), "allocating pinned input");
    b.host_in_cap = want;
  }
  b.host_out.resize(p.out_slot.size(), nullptr);
  b.host_out_cap.resize(p.out_slot.size(), 0);
  for (size_t k = 0; k < p.out_slot.size(); k++) {
    size_t need = p.out_n[k] * L;
    if (b.host_out_cap[k] < need) {
      if (b.host_out[k]) hipHostFree(b.host_out[k]);
      b.host_out[k] = nullptr;
      b.host_out_cap[k] = 0;
      size_t want = need + need / 4;
      HIPTRY(hipHostMalloc(&b.host_out[k], want * sizeof(float), hipHostMallocDefault), "allocating pinned output");
      b.host_out_cap[k] = want;
    }
  }
  const size_t bits_need = L * b.bits_h * b.bits_wpr;
  if (b.host_bits_cap < bits_need) {
    if (b.host_bits) hipHostFree(b.host_bits);
    b.host_bits = nullptr;
    b.host_bits_cap = 0;
    const size_t want = bits_need + bits_need / 4;
    HIPTRY(hipHostMalloc(&b.host_bits, want * sizeof(unsigned long long), hipHostMallocDefault),
           "allocating the pinned DB mask");
    b.host_bits_cap = want;
  }
  build_launches(b);
  // The channel means' counters start at zero (each launch leaves them so).
  for (const Launch &l : b.launches)
    if (l.gk == GK_MEAN) {
      const MeanJob &j = l.mean;
      const MeanShape m = mean_shape(j.x != nullptr, j.pixels, j.c, j.lanes, j.x ? 0 : j.chunks, j.has_se != 0);
      if (m.count_n)
        HIPTRY(hipMemsetAsync(j.count, 0, m.count_n * sizeof(int), stream), "clearing the channel mean counters");
    }
  account(b);
  group(b);
  return true;
}

void Model::build_launches(Batch &b) {
  b.launches.clear();
  const Plan &p = b.plan;
  const int L = int(b.lanes.size());
  const float *W = dweights;
  for (size_t si = 0; si < steps.size(); si++) {
    const Step &s = steps[si];
    const size_t first_launch = b.launches.size();
    const Op &op = p.ops[s.op];
    const size_t y = step_writes(s);
    float *Y = b.dev(y);
    const long ys = b.stride(y);
    const float *bias = op.b1 ? W + op.b0 : nullptr;
    switch (s.kind) {
      case S_GEMM: {
        ConvArgs a{};
        a.lanes = L;
        a.n = s.gemm_n;
        if (op.kind == K_CONVTRANSPOSE) {
          a.ih = int(op.ih), a.iw = int(op.iw), a.oh = int(op.ih), a.ow = int(op.iw);
          a.kh = a.kw = a.sh = a.sw = 1;
          a.mode = GEMM_SPREAD;
          a.spread_kw = int(op.kw), a.spread_oc = int(op.oc);
        } else {
          a.ih = int(op.ih), a.iw = int(op.iw), a.oh = int(op.oh), a.ow = int(op.ow);
          a.kh = int(op.kh), a.kw = int(op.kw), a.sh = int(op.sh), a.sw = int(op.sw);
          a.pt = int(op.pt), a.pl = int(op.pl);
          a.mode = GEMM_STORE;
        }
        a.nsrc = int(s.sources.size());
        int coff = 0;
        for (size_t k = 0; k < s.sources.size(); k++) {
          const Source &src = s.sources[k];
          a.src[k] = ConvSrc{b.dev(src.slot), b.stride(src.slot), src.c, src.shift, coff};
          coff += src.c;
        }
        a.ctot = s.ctot, a.cpt = s.cpt;
        a.chunks = s.chunks;
        a.wt = dpacked + s.wt_off;
        a.wt_k = long(s.wt_k);
        a.bias = bias;
        if (s.gate >= 0) {
          size_t g = p.ops[s.gate].x2;
          a.gate = b.dev(g), a.gate_lane_stride = b.stride(g);
        }
        a.act = op.fused;
        if (s.add >= 0) {
          const Op &ad = p.ops[s.add];
          size_t r = ad.x == op.y ? ad.x2 : ad.x;
          a.res = b.dev(r), a.res_lane_stride = b.stride(r);
          a.act2 = ad.fused;
        }
        a.y = Y, a.y_lane_stride = ys;
        if (s.pw1 >= 0) {
          const Op &q = p.ops[s.pw1];
          a.pw_w = W + q.w0, a.pw_b = q.b1 ? W + q.b0 : nullptr;
          a.pw_n = int(q.oc), a.pw_act = q.fused;
        }
        GemmTile t = s.tile;
        if (s.patch) {
          // Tiles of 8 rows (each wave two MFMA row blocks: half the LDS reads
          // per MFMA) when there is about one per CU or more, else of 4.
          const long ntn = (a.n + t.bn - 1) / t.bn;
          const long tiles8 = long(L) * ((a.oh + 7) / 8) * ((a.ow + 15) / 16) * ntn;
          const long tiles4 = long(L) * ((a.oh + 3) / 4) * ((a.ow + 15) / 16) * ntn;
          const int wr = patch_rows(tiles4, tiles8, patch_fits(a.kh, a.kw, a.sh, 2, t.bk, t.bn),
                                    patch_lds_bytes(a, 1, t.bk, t.bn), patch_lds_bytes(a, 2, t.bk, t.bn));
          const int bk = t.bk, bn = t.bn;
          b.launches.push_back({"conv_patch", s.op, [a, wr, bk, bn](hipStream_t st) {
                                  return launch_conv_patch(a, wr, bk, bn, st);
                                }});
          Launch &l = b.launches.back();
          l.gk = GK_PATCH, l.gkey = bk * 1000 + bn, l.conv = a, l.bk = bk, l.bn = bn;
          break;
        }
        long M = long(L) * a.oh * a.ow;
        a.xcd_rows = 1;
        if ((t.pointwise || s.ring) && ring_supported(a) && ring_fits(a, ring_tile({a}, M))) {
          const RingTile rt = ring_tile({a}, M);
          const char *nm = op.kind == K_CONVTRANSPOSE ? "convt_gemm" : (t.pointwise ? "pointwise_gemm" : "conv_gemm");
          b.launches.push_back({nm, s.op, [a, rt](hipStream_t st) { return launch_conv_ring(a, rt, st); }});
          Launch &l = b.launches.back();
          l.gk = GK_RING, l.gkey = (a.gate ? 1 : 0) + (s.ring ? 2 : 0), l.conv = a, l.rt = rt;
          break;
        }
        long tiles = (M + 127) / 128 * ((a.n + t.bn - 1) / t.bn);
        // Fewer than four tiles per CU of 128 rows: take 64-row tiles.
        if (tiles < 1024) t.wm = 16;
        const char *nm = op.kind == K_CONVTRANSPOSE ? "convt_gemm" : (t.pointwise ? "pointwise_gemm" : "conv_gemm");
        b.launches.push_back({nm, s.op, [a, t](hipStream_t st) { return launch_conv(a, t, st); }});
        if (s.pw1 >= 0) b.launches.back().member_ops = {s.op, s.pw1};
        break;
      }
      case S_CTC: {
        ConvArgs a{};
        a.lanes = L;
        a.ih = 1, a.iw = int(op.iw), a.oh = 1, a.ow = int(op.iw);
        a.n = s.gemm_n;
        a.kh = a.kw = a.sh = a.sw = 1;
        a.nsrc = 1;
        a.src[0] = ConvSrc{b.dev(op.x), b.stride(op.x), int(op.ic), 0, 0};
        a.ctot = s.ctot, a.cpt = s.cpt;
        a.chunks = s.chunks;
        a.wt = dpacked + s.wt_off;
        a.wt_k = long(s.wt_k);
        a.bias = W + op.b0;
        a.mode = GEMM_CTC;
        a.vocab = int(op.n2);
        float *part = b.ws(si);
        a.part = part;
        a.y = Y, a.y_lane_stride = ys;
        GemmTile t = s.tile;
        int ntn = (a.n + t.bn - 1) / t.bn, tile_n = t.bn;  // partial records per row, columns each
        int rows = L * int(op.iw), T = int(op.iw);
        float *tmax = nullptr;  // per-tile maxima after a run's records, for the near-tie recheck
        int tiles = 0;
        if (ctc_direct_supported(int(op.ic))) {
          const CtcRuns r = ctc_direct_runs(rows, a.vocab);
          tiles = (a.vocab + 63) / 64;
          tmax = part + size_t(rows) * r.runs * 4;
          const CtcDirectArgs d{a.src[0].p, a.src[0].lane_stride, T, L, int(op.ic), dpacked + s.enc_w1, a.bias,
                                a.vocab, part, tmax};
          b.launches.push_back({"ctc_gemm", s.op, [d](hipStream_t st) { return launch_ctc_direct(d, st); }});
          ntn = r.runs, tile_n = r.columns;
        } else {
          b.launches.push_back({"ctc_gemm", s.op, [a, t](hipStream_t st) { return launch_conv(a, t, st); }});
        }
        const CtcExact ex{a.src[0].p, a.src[0].lane_stride, int(op.ic), a.wt, a.wt_k, a.bias, a.vocab, tile_n,
                          tmax, tiles, s.ctc_bias_max, s.ctc_wsum_max};
        b.launches.push_back({"ctc_merge", s.op, [part, rows, ntn, Y, ys, T, ex](hipStream_t st) {
                                return launch_ctc_merge(part, rows, ntn, Y, ys, T, ex, st);
                              }});
        break;
      }
      case S_DW: {
        DwArgs a{L, int(op.ih), int(op.iw), int(op.oc), int(op.oh), int(op.ow), int(op.kh), int(op.kw),
                 int(op.sh), int(op.sw), int(op.pt), int(op.pl), b.dev(op.x), b.stride(op.x), W + op.w0,
                 bias, op.fused, Y, ys, nullptr};
        if (s.pw1 >= 0) {
          const Op &q = p.ops[s.pw1];
          DwPwArgs f{};
          f.d = a;
          f.d.y = nullptr;
          f.pw = dpacked + s.enc_w1, f.pw_b = q.b1 ? W + q.b0 : nullptr;
          f.n = int(q.oc), f.pw_act = q.fused;
          if (s.add >= 0) {
            const Op &ad = p.ops[s.add];
            const size_t r = ad.x == q.y ? ad.x2 : ad.x;
            f.res = b.dev(r), f.res_lane_stride = b.stride(r);
            f.act2 = ad.fused;
          }
          f.y = Y, f.y_lane_stride = ys;
          b.launches.push_back({"dwconv_pw", s.op, [f](hipStream_t st) { return launch_dwpw(f, st); }});
          b.launches.back().member_ops = {s.op, s.pw1};
          break;
        }
        // The sums go to the workspace of the mean step that follows.
        if (s.dw_sums) a.mean_part = reinterpret_cast<double *>(b.ws(si + 1));
        b.launches.push_back({"dwconv", s.op, [a](hipStream_t st) { return launch_dwconv(a, st); }});
        break;
      }
      case S_ELT: {
        if (!s.chain.empty()) {
          ChainArgs c{};
          c.lanes = L, c.levels = int(s.chain.size()), c.c = int(op.oc);
          const Op &top = p.ops[s.chain.back()];
          c.top = b.dev(top.x), c.top_lane_stride = b.stride(top.x);
          for (int k = 0; k < c.levels; k++) {
            const Op &o = p.ops[s.chain[k]];
            c.h[k] = int(o.oh), c.w[k] = int(o.ow), c.act[k] = o.fused;
            const size_t addend = s.chain_gate[k] >= 0 ? p.ops[s.chain_gate[k]].x : o.x2;
            c.b[k] = b.dev(addend), c.b_lane_stride[k] = b.stride(addend);
            if (s.chain_gate[k] >= 0) {
              const size_t g = p.ops[s.chain_gate[k]].x2;
              c.g[k] = b.dev(g), c.g_lane_stride[k] = b.stride(g);
            }
            c.y[k] = b.dev(o.y), c.y_lane_stride[k] = b.stride(o.y);
          }
          b.launches.push_back({"upsample_add_chain", s.op, [c](hipStream_t st) { return launch_upadd_chain(c, st); }});
          b.launches.back().member_ops.assign(s.chain.rbegin(), s.chain.rend());
          break;
        }
        EltArgs a{};
        a.mode = s.elt, a.lanes = L;
        a.oh = int(op.oh), a.ow = int(op.ow), a.c = int(op.oc);
        a.iw = int(op.iw), a.sh = int(std::max<size_t>(op.sh, 1)), a.sw = int(std::max<size_t>(op.sw, 1));
        a.act = op.fused;
        a.y = Y, a.y_lane_stride = ys;
        a.a = b.dev(op.x), a.a_lane_stride = b.stride(op.x);
        switch (s.elt) {
          case ELT_ADD: case ELT_UPSAMPLEADD:
            a.b = b.dev(op.x2), a.b_lane_stride = b.stride(op.x2);
            break;
          case ELT_CHANNELMUL:
            a.g = b.dev(op.x2), a.g_lane_stride = b.stride(op.x2);
            break;
          case ELT_CONCAT:
            a.b = b.dev(op.x2), a.b_lane_stride = b.stride(op.x2);
            a.ca = int(op.ic), a.cb = int(op.n2);
            break;
          case ELT_RESGATE: {
            const Op &cm = p.ops[s.resgate];
            a.a = b.dev(cm.x), a.a_lane_stride = b.stride(cm.x);
            a.g = b.dev(cm.x2), a.g_lane_stride = b.stride(cm.x2);
            a.act = p.ops[s.add].fused;
            break;
          }
          case ELT_UPSAMPLEADD_RESGATE: {
            const Op &cm = p.ops[s.resgate];
            a.b = b.dev(cm.x), a.b_lane_stride = b.stride(cm.x);
            a.g = b.dev(cm.x2), a.g_lane_stride = b.stride(cm.x2);
            break;
          }
          default: break;
        }
        static const char *names[] = {"add", "channel_mul", "upsample", "upsample_add", "concat",
                                      "residual_gate", "upsample_add_gate", "mul", "activation"};
        b.launches.push_back({names[s.elt], s.op, [a](hipStream_t st) { return launch_eltwise(a, st); }});
        b.launches.back().gk = GK_ELT, b.launches.back().gkey = eltwise_vec(a) ? 1 : 0, b.launches.back().elt = a;
        break;
      }
      case S_POOL: {
        PoolArgs a{op.kind == K_AVGPOOL, L, int(op.ih), int(op.iw), int(op.oc), int(op.oh), int(op.ow),
                   int(op.kh), int(op.kw), int(op.sh), int(op.sw), b.dev(op.x), b.stride(op.x), Y, ys};
        b.launches.push_back({op.kind == K_AVGPOOL ? "avgpool" : "maxpool", s.op,
                              [a](hipStream_t st) { return launch_pool(a, st); }});
        break;
      }
      case S_MEAN: {
        const bool se = s.fc1 >= 0;
        MeanJob j{};
        j.x = s.mean_of_dw >= 0 ? nullptr : b.dev(op.x);
        j.x_lane_stride = b.stride(op.x);
        j.pixels = int(op.ih * op.iw), j.c = int(op.ic), j.lanes = L;
        if (s.mean_of_dw >= 0) {
          DwArgs d = dw_shape(p.ops[s.mean_of_dw]);
          d.lanes = L;
          j.chunks = dw_mean_blocks(d);
        }
        j.work = b.ws(si);
        j.count = reinterpret_cast<int *>(b.ws(si) + round_up(mean_step_shape(s, p, L).floats, 4));
        if (se) {
          const Op &f1 = p.ops[s.fc1], &f2 = p.ops[s.fc2];
          j.se = SeArgs{dpacked + s.se_w1, f1.b1 ? W + f1.b0 : nullptr, int(f1.oc), f1.fused,
                        dpacked + s.se_w2, f2.b1 ? W + f2.b0 : nullptr, int(f2.oc), f2.fused};
          j.has_se = 1;
        }
        j.y = Y, j.y_lane_stride = ys;
        b.launches.push_back({se ? "se_squeeze" : "channel_mean", s.op,
                              [j](hipStream_t st) { return launch_mean_group(&j, 1, st); }});
        Launch &l = b.launches.back();
        l.gk = GK_MEAN;
        l.mean = j;
        break;
      }
      case S_LN: {
        const float *x = b.dev(op.x);
        long xs = b.stride(op.x);
        const float *w = W + op.w0;
        int rows = int(op.oh * op.ow), c = int(op.oc);
        b.launches.push_back({"layernorm", s.op, [=](hipStream_t st) {
                                return launch_layernorm(x, xs, w, rows, c, L, Y, ys, st);
                              }});
        break;
      }
      case S_ATTN: {
        const float *x = b.dev(op.x);
        long xs = b.stride(op.x);
        float scale = weights[op.w0];
        int t = int(op.iw), c = int(op.oc), heads = int(op.n2);
        float *scratch = b.ws(si);
        b.launches.push_back({"attention", s.op, [=](hipStream_t st) {
                                return launch_attention(x, xs, scale, t, c, heads, L, Y, ys, scratch, st);
                              }});
        break;
      }
      case S_ENC_LIN: {
        const Op &f = p.ops[s.fc1];
        EncLinArgs a{};
        a.rows = int(op.oh * op.ow), a.lanes = L, a.k = int(f.ic), a.n = int(f.oc);
        a.x = b.dev(op.x), a.x_lane_stride = b.stride(op.x);
        a.ln = W + op.w0;
        a.wt = dpacked + s.enc_w1, a.bias = f.b1 ? W + f.b0 : nullptr, a.act = f.fused;
        if (s.add >= 0) {
          const Op &ad = p.ops[s.add];
          const size_t r = ad.x == f.y ? ad.x2 : ad.x;
          a.res = b.dev(r), a.res_lane_stride = b.stride(r), a.act2 = ad.fused;
        }
        a.y = Y, a.y_lane_stride = ys;
        b.launches.push_back({"ln_linear", s.op, [a](hipStream_t st) { return launch_enc_linear(a, st); }});
        break;
      }
      case S_ENC_ATTN:
      case S_ENC_BLOCK: {
        const Op &f = p.ops[s.fc1];
        EncAttnArgs a{};
        a.t = int(op.iw), a.lanes = L, a.c = int(op.oc), a.heads = int(op.n2), a.scale = weights[op.w0];
        a.qkv = b.dev(op.x), a.qkv_lane_stride = b.stride(op.x);
        a.wt = dpacked + s.enc_w1, a.bias = f.b1 ? W + f.b0 : nullptr, a.act = f.fused;
        if (s.add >= 0) {
          const Op &ad = p.ops[s.add];
          const size_t r = ad.x == f.y ? ad.x2 : ad.x;
          a.res = b.dev(r), a.res_lane_stride = b.stride(r), a.act2 = ad.fused;
        }
        EncMlpArgs m{};  // the MLP part, for lines too long for one launch
        if (s.kind == S_ENC_BLOCK) {
          const Op &g1 = p.ops[s.m_fc1], &g2 = p.ops[s.m_fc2], &ln2 = p.ops[s.m_ln];
          a.hidden = int(g1.oc), a.ln = W + ln2.w0;
          a.w1 = dpacked + s.enc_w2, a.b1 = g1.b1 ? W + g1.b0 : nullptr, a.act1m = g1.fused;
          a.w2 = dpacked + s.enc_w3, a.b2 = g2.b1 ? W + g2.b0 : nullptr, a.act2m = g2.fused;
          a.act3m = p.ops[s.m_add].fused;
          a.ln_out = s.ln_out >= 0 ? W + p.ops[s.ln_out].w0 : nullptr;
          m.rows = a.t, m.lanes = L, m.c = a.c, m.hidden = a.hidden, m.ln = a.ln;
          m.b1 = a.b1, m.act1 = a.act1m, m.b2 = a.b2, m.act2 = a.act2m, m.act3 = a.act3m;
          m.residual = 1, m.ln_out = a.ln_out;
        }
        a.y = Y, a.y_lane_stride = ys;
        if (enc_attn_fits(a.t, a.c, a.heads, a.w1 ? a.hidden : 0)) {
          b.launches.push_back({s.kind == S_ENC_BLOCK ? "attention_block" : "attention_proj", s.op,
                                [a](hipStream_t st) { return launch_enc_attn(a, st); }});
          break;
        }
        // The attention rows into the workspace, then the projection (into
        // the workspace too when the MLP follows), then the MLP.
        float *rows = b.ws(si);
        float *sum = rows + round_up(size_t(L) * a.t * a.c, 64);
        float *scratch = s.kind == S_ENC_BLOCK ? sum + round_up(size_t(L) * a.t * a.c, 64) : sum;
        const long rs = long(a.t) * a.c;
        const float *x = a.qkv;
        const long xs = a.qkv_lane_stride;
        b.launches.push_back({"attention", s.op, [=](hipStream_t st) {
                                return launch_attention(x, xs, a.scale, a.t, a.c, a.heads, L, rows, rs, scratch, st);
                              }});
        EncLinArgs g{};
        g.rows = a.t, g.lanes = L, g.k = a.c, g.n = a.c;
        g.x = rows, g.x_lane_stride = rs;
        g.wt = a.wt, g.bias = a.bias, g.act = a.act, g.act2 = a.act2;
        g.res = a.res, g.res_lane_stride = a.res_lane_stride;
        g.y = s.kind == S_ENC_BLOCK ? sum : Y, g.y_lane_stride = s.kind == S_ENC_BLOCK ? rs : ys;
        b.launches.push_back({"ln_linear", s.fc1, [g](hipStream_t st) { return launch_enc_linear(g, st); }});
        if (s.kind == S_ENC_BLOCK) {
          m.x = sum, m.x_lane_stride = rs;
          m.w1 = a.w1, m.w2 = a.w2;
          m.y = Y, m.y_lane_stride = ys;
          b.launches.push_back({"ln_mlp", s.m_ln, [m](hipStream_t st) { return launch_enc_mlp(m, st); }});
        }
        break;
      }
      case S_ENC_MLP: {
        const Op &f1 = p.ops[s.fc1], &f2 = p.ops[s.fc2], &ad = p.ops[s.add];
        EncMlpArgs a{};
        a.rows = int(op.oh * op.ow), a.lanes = L, a.c = int(op.oc), a.hidden = int(f1.oc);
        a.x = b.dev(op.x), a.x_lane_stride = b.stride(op.x);
        a.ln = W + op.w0;
        a.w1 = dpacked + s.enc_w1, a.b1 = f1.b1 ? W + f1.b0 : nullptr, a.act1 = f1.fused;
        a.w2 = dpacked + s.enc_w2, a.b2 = f2.b1 ? W + f2.b0 : nullptr, a.act2 = f2.fused;
        a.act3 = ad.fused, a.residual = 1;
        a.ln_out = s.ln_out >= 0 ? W + p.ops[s.ln_out].w0 : nullptr;
        a.y = Y, a.y_lane_stride = ys;
        b.launches.push_back({"ln_mlp", s.op, [a](hipStream_t st) { return launch_enc_mlp(a, st); }});
        break;
      }
      case S_CONVT: {
        ConvtArgs a{L, int(op.ih), int(op.iw), int(op.ic), int(op.oc), int(op.kh), int(op.kw),
                    b.dev(op.x), b.stride(op.x), W + op.w0, bias, op.fused, Y, ys};
        b.launches.push_back({"convt_small", s.op, [a](hipStream_t st) { return launch_convt_small(a, st); }});
        break;
      }
      case S_DIRECT: {
        DirectArgs a{};
        a.lanes = L;
        a.ih = int(op.ih), a.iw = int(op.iw), a.ic = int(op.ic);
        a.oh = int(op.oh), a.ow = int(op.ow), a.oc = int(op.oc);
        a.kh = int(op.kh), a.kw = int(op.kw), a.sh = int(op.sh), a.sw = int(op.sw);
        a.pt = int(op.pt), a.pl = int(op.pl);
        a.x = b.dev(op.x), a.x_lane_stride = b.stride(op.x);
        a.w = W + op.w0, a.bias = bias, a.act = op.fused;
        // kernels/dense.rs:38-147 and conv.rs:146-236: the RGB stem always
        // starts from the bias; otherwise a multiple-of-16 width does, except
        // for the row's last ow % 4 pixels.
        const bool stem = op.ic == 3 && op.n2 == 0;
        a.first_end = stem ? a.ow : (op.oc % 16 == 0 ? a.ow - a.ow % 4 : 0);
        a.fused = int(op.oc / 8 * 8);
        a.y = Y, a.y_lane_stride = ys;
        b.launches.push_back({"conv_direct", s.op, [a](hipStream_t st) { return launch_conv_direct(a, st); }});
        break;
      }
      case S_STEM: {
        const Op &o2 = p.ops[s.st2], &o3 = p.ops[s.st3], &pl = p.ops[s.st_pool];
        StemArgs a{};
        a.lanes = L;
        a.ih = int(op.ih), a.iw = int(op.iw), a.oh = int(op.oh), a.ow = int(op.ow);
        a.c1 = int(op.oc), a.c2 = int(o2.oc), a.c3 = int(o3.oc);
        a.x = b.dev(op.x), a.x_lane_stride = b.stride(op.x);
        a.w1 = W + op.w0, a.b1 = bias, a.act1 = op.fused;
        a.w2 = W + o2.w0, a.b2 = o2.b1 ? W + o2.b0 : nullptr, a.act2 = o2.fused;
        a.w3 = W + o3.w0, a.b3 = o3.b1 ? W + o3.b0 : nullptr, a.act3 = o3.fused;
        a.pool = b.dev(pl.y), a.pool_lane_stride = b.stride(pl.y), a.pool_px = a.c1;
        a.y = Y, a.y_lane_stride = ys, a.y_px = a.c3;
        if (s.st_joint) a.y = a.pool + a.c1, a.y_lane_stride = a.pool_lane_stride, a.pool_px = a.y_px = a.c1 + a.c3;
        b.launches.push_back({"stem_block", s.op, [a](hipStream_t st) { return launch_stem_block(a, st); }});
        b.launches.back().member_ops = {s.op, s.st2, s.st3, s.st_pool};
        std::sort(b.launches.back().member_ops.begin(), b.launches.back().member_ops.end());
        break;
      }
      case S_HEAD: {
        const Op &o2 = p.ops[s.head2];
        HeadArgs a{};
        a.lanes = L;
        a.ih = int(op.ih), a.iw = int(op.iw), a.ic = int(op.ic), a.oc1 = int(op.oc);
        a.x = b.dev(op.x), a.x_lane_stride = b.stride(op.x);
        a.w1 = W + op.w0, a.b1 = bias, a.act1 = op.fused;
        a.w2 = W + o2.w0, a.b2 = o2.b1 ? W + o2.b0 : nullptr, a.act2 = o2.fused;
        a.y = Y, a.y_lane_stride = ys;
        b.launches.push_back({"db_head", s.op, [a](hipStream_t st) { return launch_db_head(a, st); }});
        break;
      }
    }
    for (size_t k = first_launch; k < b.launches.size(); k++) b.launches[k].step = int(si);
  }
  link(b);
}

// The dependencies between a batch's launches, from the memory each step
// reads and writes: its inputs' and output's homes (a home holds different
// buffers over a run, so a later writer waits for the earlier readers) and
// its own workspace region. A launch also follows the previous launch of its
// step. Independent launches of one kind may then share one grid (group).
void Model::link(Batch &b) const {
  const size_t H = b.home_floats.size();
  const size_t R = H + steps.size();
  std::vector<int> writer(R, -1);
  std::vector<std::vector<int>> readers(R);
  for (size_t j = 0; j < b.launches.size(); j++) {
    Launch &l = b.launches[j];
    const Step &s = steps[size_t(l.step)];
    std::vector<size_t> rd, wr;
    for (size_t slot : step_reads(s)) rd.push_back(b.home[slot]);
    wr.push_back(b.home[step_writes(s)]);
    for (size_t y2 : step_writes_extra(s)) wr.push_back(b.home[y2]);
    const size_t ws = H + size_t(l.step);
    if (s.kind == S_MEAN || s.kind == S_CTC || s.kind == S_ATTN || s.kind == S_ENC_ATTN || s.kind == S_ENC_BLOCK)
      rd.push_back(ws), wr.push_back(ws);
    if (s.kind == S_DW && s.dw_sums) wr.push_back(ws + 1);  // the next step's partial sums
    std::vector<int> deps;
    if (j > 0 && b.launches[j - 1].step == l.step) deps.push_back(int(j - 1));
    for (size_t r : rd)
      if (writer[r] >= 0) deps.push_back(writer[r]);
    for (size_t w : wr) {
      if (writer[w] >= 0) deps.push_back(writer[w]);
      deps.insert(deps.end(), readers[w].begin(), readers[w].end());
    }
    std::sort(deps.begin(), deps.end());
    deps.erase(std::unique(deps.begin(), deps.end()), deps.end());
    deps.erase(std::remove(deps.begin(), deps.end(), int(j)), deps.end());
    l.deps = deps;
    for (size_t r : rd) readers[r].push_back(int(j));
    for (size_t w : wr) writer[w] = int(j), readers[w].clear();
  }
}

// Independent launches of one kind as grouped launches. Kind by kind (the
// costliest first) and in build order, a groupable launch joins the first
// earlier group of its kind and key that has room, none of whose launches it
// depends on or depend on it, and whose growth keeps the order between
// groups acyclic. The groups then run in a
// topological order, among the ready ones the one built first. A grouped
// launch's work is its members' sum; it is named after its first member.
void Model::group(Batch &b) const {
  if (!kGrouped) return;
  const int n = int(b.launches.size());
  std::vector<std::vector<char>> reach(static_cast<size_t>(n), std::vector<char>(static_cast<size_t>(n), 0));
  for (int j = 0; j < n; j++)
    for (int d : b.launches[size_t(j)].deps) {
      reach[size_t(j)][size_t(d)] = 1;
      for (int k = 0; k < n; k++)
        if (reach[size_t(d)][size_t(k)]) reach[size_t(j)][size_t(k)] = 1;
    }
  const size_t N = size_t(n);
  std::vector<int> gid(N);
  std::vector<std::vector<int>> groups(N);
  for (int j = 0; j < n; j++) gid[size_t(j)] = j, groups[size_t(j)] = {j};
  // The groups in a topological order (empty if there is a cycle).
  auto order = [&]() {
    std::vector<int> indeg(N, 0), out_order;
    std::vector<std::vector<int>> out(N);
    for (int j = 0; j < n; j++)
      for (int d : b.launches[size_t(j)].deps) {
        const int a = gid[size_t(d)], c = gid[size_t(j)];
        if (a != c) out[size_t(a)].push_back(c), indeg[size_t(c)]++;
      }
    std::vector<int> ready;
    int live = 0;
    for (int g = 0; g < n; g++)
      if (!groups[size_t(g)].empty()) {
        live++;
        if (indeg[size_t(g)] == 0) ready.push_back(g);
      }
    while (!ready.empty()) {
      auto it = std::min_element(ready.begin(), ready.end());
      const int g = *it;
      ready.erase(it);
      out_order.push_back(g);
      for (int c : out[size_t(g)])
        if (--indeg[size_t(c)] == 0) ready.push_back(c);
    }
    if (int(out_order.size()) != live) out_order.clear();
    return out_order;
  };
  // The costliest kinds first, so that cheap merges do not order them.
  for (int kind : {GK_PATCH, GK_RING, GK_MEAN, GK_ELT})
  for (int j = 0; j < n; j++) {
    const Launch &l = b.launches[size_t(j)];
    if (l.gk != kind) continue;
    for (int g = 0; g < j; g++) {
      auto &G = groups[size_t(g)];
      if (G.empty() || int(G.size()) >= kGroupMax) continue;
      const Launch &f = b.launches[size_t(G[0])];
      if (f.gk != l.gk || f.gkey != l.gkey) continue;
      bool independent = true;
      for (int m : G) independent = independent && !reach[size_t(j)][size_t(m)] && !reach[size_t(m)][size_t(j)];
      if (!independent) continue;
      G.push_back(j);
      groups[size_t(j)].clear();
      gid[size_t(j)] = g;
      if (!order().empty()) break;
      G.pop_back();
      groups[size_t(j)] = {j};
      gid[size_t(j)] = j;
    }
  }
  const std::vector<int> seq = order();
  if (int(seq.size()) == n) return;  // nothing grouped
  std::vector<Launch> out;
  std::vector<int> at(N, -1);  // group -> index in out
  for (int g : seq) {
    std::vector<int> mem = groups[size_t(g)];
    at[size_t(g)] = int(out.size());
    if (mem.size() == 1) {
      out.push_back(b.launches[size_t(mem[0])]);
      out.back().members = mem;
      if (out.back().member_ops.empty()) out.back().member_ops = {out.back().op};
      continue;
    }
    Launch gl = b.launches[size_t(mem[0])];
    gl.members = mem;
    for (int m : mem) {
      const Launch &ml = b.launches[size_t(m)];
      if (ml.member_ops.empty()) gl.member_ops.push_back(ml.op);
      else gl.member_ops.insert(gl.member_ops.end(), ml.member_ops.begin(), ml.member_ops.end());
    }
    gl.flops = gl.bytes = 0;
    for (int m : mem) gl.flops += b.launches[size_t(m)].flops, gl.bytes += b.launches[size_t(m)].bytes;
    switch (gl.gk) {
      case GK_RING: {
        // Longest reductions first; one tile for all, chosen for their rows
        // together when they share a width, else the first one's.
        std::sort(mem.begin(), mem.end(), [&](int x, int y) {
          return b.launches[size_t(x)].conv.ctot * b.launches[size_t(x)].conv.kh * b.launches[size_t(x)].conv.kw >
                 b.launches[size_t(y)].conv.ctot * b.launches[size_t(y)].conv.kh * b.launches[size_t(y)].conv.kw;
        });
        std::vector<ConvArgs> as;
        long M = 0;
        bool same_n = true;
        for (int m : mem) {
          const ConvArgs &a = b.launches[size_t(m)].conv;
          as.push_back(a);
          M += long(a.lanes) * a.oh * a.ow;
          same_n = same_n && a.n == as[0].n;
        }
        RingTile t = same_n ? ring_tile(as, M) : gl.rt;
        for (const ConvArgs &a : as)
          if (!ring_fits(a, t)) t = gl.rt;
        gl.fn = [as, t](hipStream_t st) { return launch_conv_ring_group(as.data(), int(as.size()), t, st); };
        break;
      }
      case GK_PATCH: {
        std::vector<ConvArgs> as;
        long tiles8 = 0, tiles4 = 0;
        size_t lds4 = 0, lds8 = 0;
        bool fits2 = true;
        for (int m : mem) {
          const Launch &x = b.launches[size_t(m)];
          as.push_back(x.conv);
          const long cols = long(x.conv.lanes) * ((x.conv.ow + 15) / 16) * ((x.conv.n + x.bn - 1) / x.bn);
          tiles8 += cols * ((x.conv.oh + 7) / 8);
          tiles4 += cols * ((x.conv.oh + 3) / 4);
          fits2 = fits2 && patch_fits(x.conv.kh, x.conv.kw, x.conv.sh, 2, x.bk, x.bn);
          lds4 = std::max(lds4, patch_lds_bytes(x.conv, 1, x.bk, x.bn));
          lds8 = std::max(lds8, patch_lds_bytes(x.conv, 2, x.bk, x.bn));
        }
        const int wr = patch_rows(tiles4, tiles8, fits2, lds4, lds8), bk = gl.bk, bn = gl.bn;
        gl.fn = [as, wr, bk, bn](hipStream_t st) {
          return launch_conv_patch_group(as.data(), int(as.size()), wr, bk, bn, st);
        };
        break;
      }
      case GK_MEAN: {
        std::vector<MeanJob> js;
        for (int m : mem) js.push_back(b.launches[size_t(m)].mean);
        gl.fn = [js](hipStream_t st) { return launch_mean_group(js.data(), int(js.size()), st); };
        break;
      }
      case GK_ELT: {
        std::vector<EltArgs> es;
        for (int m : mem) es.push_back(b.launches[size_t(m)].elt);
        gl.fn = [es](hipStream_t st) { return launch_eltwise_group(es.data(), int(es.size()), st); };
        break;
      }
      default:
        break;
    }
    out.push_back(std::move(gl));
  }
  // Dependencies between the new launches, from their members'.
  for (Launch &l : out) {
    std::vector<int> deps;
    for (int m : l.members)
      for (int d : b.launches[size_t(m)].deps) {
        const int t = at[size_t(gid[size_t(d)])];
        if (t != int(&l - out.data())) deps.push_back(t);
      }
    std::sort(deps.begin(), deps.end());
    deps.erase(std::unique(deps.begin(), deps.end()), deps.end());
    l.deps = deps;
  }
  b.launches = std::move(out);
}

// Each launch's algorithmic work, in the order build_launches made them.
void Model::account(Batch &b) const {
  const Plan &p = b.plan;
  const double L = double(b.lanes.size()), F = 4.0;
  size_t li = 0;
  for (const Step &s : steps) {
    const Op &op = p.ops[s.op];
    const double in_px = double(op.ih) * op.iw, out_px = double(op.oh) * op.ow;
    Launch &l = b.launches[li++];
    switch (s.kind) {
      case S_GEMM: {
        double M, K = 0, N = s.gemm_n, in = 0;
        if (op.kind == K_CONVTRANSPOSE) {
          M = L * in_px, K = double(op.ic), in = M * K;
        } else {
          M = L * out_px;
          for (const Source &src : s.sources) {
            K += double(op.kh * op.kw) * src.c;
            in += L * double(op.ih >> src.shift) * double(op.iw >> src.shift) * src.c;
          }
          if (s.gate >= 0) in += L * op.ic;
          if (s.add >= 0) in += M * N;
        }
        l.flops = 2.0 * M * N * K;
        l.bytes = F * (in + M * N + K * N + (op.b1 ? N : 0));
        if (s.pw1 >= 0) {
          // The folded 1x1: its product, its weights, and its map stored in
          // place of this layer's.
          const Op &q = p.ops[size_t(s.pw1)];
          l.flops += 2.0 * M * double(q.oc) * N;
          l.bytes = F * (in + M * double(q.oc) + K * N + (op.b1 ? N : 0) + N * double(q.oc) + (q.b1 ? q.oc : 0));
        }
        break;
      }
      case S_CTC: {
        double M = L * op.iw, K = double(op.ic), N = double(op.n2);
        double ntn = double((s.gemm_n + s.tile.bn - 1) / s.tile.bn);
        if (ctc_direct_supported(int(op.ic))) ntn = ctc_direct_runs(long(M), int(op.n2)).runs;
        l.flops = 2.0 * M * N * K;
        l.bytes = F * (M * K + K * N + N + 2 * M);
        Launch &merge = b.launches[li++];
        merge.bytes = F * (M * ntn * 4 + 2 * M);
        break;
      }
      case S_DW:
        l.flops = 2.0 * L * out_px * op.oc * op.kh * op.kw;
        l.bytes = F * (L * in_px * op.ic + L * out_px * op.oc + double(op.kh * op.kw + 1) * op.oc);
        if (s.pw1 >= 0) {
          // The folded 1x1: its product, weights and residual, and its map
          // stored in place of the depthwise one.
          const Op &q = p.ops[size_t(s.pw1)];
          const double M = L * out_px, N = double(q.oc);
          l.flops += 2.0 * M * double(op.oc) * N;
          l.bytes = F * (L * in_px * op.ic + double(op.kh * op.kw + 1) * op.oc + double(op.oc) * N +
                         (q.b1 ? N : 0) + M * N * (s.add >= 0 ? 2 : 1));
        }
        break;
      case S_ELT: {
        double out = L * out_px * op.oc, src = L * in_px * op.ic;
        if (!s.chain.empty()) {
          const Op &top = p.ops[s.chain.back()];
          double f = L * double(top.ih) * top.iw * top.ic;
          for (size_t k = 0; k < s.chain.size(); k++) {
            const Op &o = p.ops[s.chain[k]];
            f += 2.0 * L * double(o.oh) * o.ow * o.oc + (s.chain_gate[k] >= 0 ? L * o.oc : 0.0);
          }
          l.bytes = F * f;
          break;
        }
        switch (s.elt) {
          case ELT_ADD: l.bytes = F * 3 * out; break;
          case ELT_CHANNELMUL: case ELT_RESGATE: l.bytes = F * (2 * out + L * op.oc); break;
          case ELT_UPSAMPLE: l.bytes = F * (src + out); break;
          case ELT_UPSAMPLEADD: l.bytes = F * (src + 2 * out); break;
          case ELT_UPSAMPLEADD_RESGATE: l.bytes = F * (src + 2 * out + L * op.oc); break;
          default: l.bytes = F * 2 * out;
        }
        break;
      }
      case S_POOL:
        l.bytes = F * L * (in_px * op.ic + out_px * op.oc);
        break;
      case S_MEAN:
        // Joining a depthwise step's sums reads none of the input again.
        l.bytes = F * L * ((s.mean_of_dw >= 0 ? 0.0 : in_px * op.ic) + op.oc);
        if (s.fc1 >= 0) {
          const Op &f1 = p.ops[s.fc1], &f2 = p.ops[s.fc2];
          l.flops = 2.0 * L * (double(f1.ic) * f1.oc + double(f2.ic) * f2.oc);
          l.bytes += F * (double(f1.w1 + f1.b1 + f2.w1 + f2.b1));
        }
        break;
      case S_LN:
        l.bytes = F * (2 * L * out_px * op.oc + op.w1);
        break;
      case S_ATTN: {
        double t = double(op.iw), hd = double(op.oc / op.n2);
        l.flops = L * op.n2 * t * t * hd * 4;
        l.bytes = F * L * t * (op.ic + op.oc);
        break;
      }
      case S_ENC_LIN: {
        const Op &f = p.ops[s.fc1];
        const double M = L * out_px, K = double(f.ic), N = double(f.oc);
        l.flops = 2.0 * M * N * K;
        l.bytes = F * (M * K + 2.0 * K + 1 + K * N + (f.b1 ? N : 0) + M * N * (s.add >= 0 ? 2 : 1));
        break;
      }
      case S_ENC_ATTN:
      case S_ENC_BLOCK: {
        const Op &f = p.ops[s.fc1];
        const double t = double(op.iw), c = double(op.oc), hd = c / double(op.n2), M = L * t;
        const double attn = L * op.n2 * t * t * hd * 4, proj = 2.0 * M * c * c;
        const double w = F * (c * c + (f.b1 ? c : 0)), res = F * M * c * (s.add >= 0 ? 2 : 1);
        double mlp_flops = 0, mlp_bytes = 0;  // the MLP after it, when merged
        if (s.kind == S_ENC_BLOCK) {
          const Op &g1 = p.ops[s.m_fc1], &g2 = p.ops[s.m_fc2];
          const double h = double(g1.oc);
          mlp_flops = 2.0 * M * c * h * 2;
          mlp_bytes = F * (2 * c + 1 + 2 * c * h + (g1.b1 ? h : 0) + (g2.b1 ? c : 0) + (s.ln_out >= 0 ? 2 * c + 1 : 0));
        }
        if (b.launches.size() > li && b.launches[li].op == s.fc1) {
          // Lines too long for one launch: attention rows to the workspace,
          // the projection, then the MLP.
          l.flops = attn, l.bytes = F * M * (op.ic + op.oc);
          Launch &g = b.launches[li++];
          g.flops = proj, g.bytes = F * M * c + w + res;
          if (s.kind == S_ENC_BLOCK) {
            Launch &m = b.launches[li++];
            m.flops = mlp_flops, m.bytes = mlp_bytes + F * 2 * M * c;
          }
        } else {
          l.flops = attn + proj + mlp_flops;
          l.bytes = F * M * op.ic + w + res + mlp_bytes;
        }
        break;
      }
      case S_ENC_MLP: {
        const Op &f1 = p.ops[s.fc1], &f2 = p.ops[s.fc2];
        const double M = L * out_px, c = double(op.oc), h = double(f1.oc);
        l.flops = 2.0 * M * c * h * 2;
        l.bytes = F * (2 * M * c + 2 * c + 1 + 2 * c * h + (f1.b1 ? h : 0) + (f2.b1 ? c : 0) +
                       (s.ln_out >= 0 ? 2 * c + 1 : 0));
        break;
      }
      case S_CONVT:
        l.flops = 2.0 * L * in_px * op.ic * op.kh * op.kw * op.oc;
        l.bytes = F * (L * in_px * op.ic + L * out_px * op.oc + op.w1 + op.b1);
        break;
      case S_DIRECT:
        l.flops = 2.0 * L * out_px * op.oc * op.kh * op.kw * op.ic;
        l.bytes = F * (L * in_px * op.ic + L * out_px * op.oc + op.w1 + op.b1);
        break;
      case S_STEM: {
        // Each layer's products; the input read and both outputs written once.
        const Op &o2 = p.ops[s.st2], &o3 = p.ops[s.st3];
        l.flops = 2.0 * L * out_px * (op.oc * 27.0 + 4.0 * o2.ic * o2.oc + 4.0 * o3.ic * o3.oc);
        l.bytes = F * (L * in_px * op.ic + L * out_px * (op.oc + o3.oc) + op.w1 + op.b1 + o2.w1 + o2.b1 +
                       o3.w1 + o3.b1);
        break;
      }
      case S_HEAD: {
        const Op &o2 = p.ops[s.head2];
        const double mid_px = out_px, fin_px = double(o2.oh) * o2.ow;
        l.flops = 2.0 * L * (in_px * op.ic * 4 * op.oc + mid_px * o2.ic * 4 * o2.oc);
        l.bytes = F * (L * in_px * op.ic + L * fin_px * o2.oc + op.w1 + op.b1 + o2.w1 + o2.b1);
        break;
      }
    }
  }
}

bool Model::set_sizes(const size_t *hw, size_t n, std::string &err) {
  HIPTRY(hipSetDevice(device), "selecting the GPU");
  std::vector<std::pair<size_t, size_t>> want;
  for (size_t i = 0; i < n; i++) want.push_back({hw[2 * i], hw[2 * i + 1]});
  if (want == sizes && !batches.empty() && !lane_at.empty()) return true;
  // Check every size on a copy of the plan first; lanes before the first
  // that fails stay valid, as src/engine/gpu/mod.rs:188-190 promises.
  size_t good = 0;
  std::string size_err;
  for (; good < n; good++) {
    Plan probe = plan;
    if (!probe.set_size(want[good].first, want[good].second, weights.size(), size_err)) break;
  }
  if (good < n) want.resize(good);
  // Batches: one per distinct size, in order of first appearance.
  std::vector<std::pair<size_t, size_t>> order;
  std::vector<std::pair<size_t, size_t>> at(want.size());
  std::vector<std::vector<size_t>> members;
  for (size_t i = 0; i < want.size(); i++) {
    auto it = std::find(order.begin(), order.end(), want[i]);
    size_t g = size_t(it - order.begin());
    if (it == order.end()) {
      order.push_back(want[i]);
      members.push_back({});
    }
    at[i] = {g, members[g].size()};
    members[g].push_back(i);
  }
  drop_graph();  // the lanes' memory moves: record the run again
  while (batches.size() < order.size()) batches.emplace_back(new Batch());
  lane_at.clear();
  sizes.clear();
  for (size_t g = 0; g < order.size(); g++) {
    Batch &b = *batches[g];
    b.h = order[g].first, b.w = order[g].second;
    b.lanes = members[g];
    b.plan = plan;
    std::string e;
    if (!b.plan.set_size(b.h, b.w, weights.size(), e)) return err = e, false;
    if (!arrange(b, err)) return false;
  }
  // Memory of batches no longer used is kept for later runs.
  lane_at = at;
  sizes = want;
  active_batches = order.size();
  if (good < n) return err = size_err, false;
  return true;
}

// The most lanes one run takes. The Vulkan backend is bounded by its
// descriptor budget (src/engine/gpu/mod.rs:184-186); this one by memory and
// by 32-bit element counts: lanes of the first lane's size (the load size
// before any), each holding every plan buffer at once plus a quarter more
// for the workspace (the arena reuses memory, so this over-counts), in 80 %
// of the device's memory, and few enough that the largest buffer's
// elements over all lanes still count in 31 bits.
size_t Model::max_lanes() const {
  const Plan &p = active_batches ? batches[0]->plan : plan;
  size_t floats = 0, largest = 1;
  for (size_t f : p.pool) floats += f, largest = std::max(largest, f);
  const size_t per_lane = std::max<size_t>(1, (floats + floats / 4 + p.in_h * p.in_w * p.in_c) * sizeof(float));
  const size_t by_memory = device_bytes / 10 * 8 / per_lane;
  const size_t by_count = size_t(0x7fffffff) / largest;
  return std::max<size_t>(1, std::min(by_memory, by_count));
}

void Model::drop_graph() {
  if (graph_exec) hipGraphExecDestroy(graph_exec);
  if (graph) hipGraphDestroy(graph);
  graph_exec = nullptr;
  graph = nullptr;
  eager_runs = 0;
}

// Enqueue every batch's launches once on the stream: eagerly the first time
// after the lanes were arranged, from the captured graph afterwards. A
// capture that fails leaves the model running eagerly.
bool Model::enqueue(std::string &err) {
  if (use_graphs && !graph_exec && eager_runs >= 1) {
    bool ok = hipStreamBeginCapture(stream, hipStreamCaptureModeRelaxed) == hipSuccess;
    std::string ignored;
    ok = ok && launch_all(ignored);
    hipGraph_t captured = nullptr;
    hipError_t end = hipStreamEndCapture(stream, &captured);
    ok = ok && end == hipSuccess && captured;
    if (ok && hipGraphInstantiate(&graph_exec, captured, nullptr, nullptr, 0) == hipSuccess) {
      graph = captured;
    } else {
      if (captured) hipGraphDestroy(captured);
      graph_exec = nullptr;
      use_graphs = false;
      (void)hipGetLastError();
    }
  }
  if (graph_exec) {
    HIPTRY(hipGraphLaunch(graph_exec, stream), "launching the run's graph");
    return true;
  }
  if (!launch_all(err)) return false;
  eager_runs++;
  return true;
}

// Every launch of the active batches, in order, on the model's stream.
bool Model::launch_all(std::string &err) {
  for (size_t g = 0; g < active_batches; g++)
    for (const Launch &l : batches[g]->launches) {
      hipError_t e = l.fn(stream);
      if (e != hipSuccess)
        return err = fmt("launching %s (operation %d): %s", l.name.c_str(), l.op, hipGetErrorString(e)), false;
    }
  return true;
}

bool Model::run(bool copy_in, bool copy_out, std::string &err, bool sync) {
  HIPTRY(hipSetDevice(device), "selecting the GPU");
  if (lane_at.empty()) return err = "no lanes are set", false;
  if (copy_in) {
    for (size_t g = 0; g < active_batches; g++) {
      Batch &b = *batches[g];
      const Plan &p = b.plan;
      HIPTRY(hipMemcpy2DAsync(b.dev(p.in_slot), b.stride(p.in_slot) * sizeof(float), b.host_in,
                              b.in_len * sizeof(float), b.in_len * sizeof(float), b.lanes.size(),
                              hipMemcpyHostToDevice, stream),
             "copying the input");
    }
  }
  if (!enqueue(err)) return false;
  // The DB threshold's bitmasks of the map, after the forward (outside the
  // captured graph: one launch per batch on the same stream).
  if (db_output >= 0)
    for (size_t g = 0; g < active_batches; g++) {
      Batch &b = *batches[g];
      const size_t slot = b.plan.out_slot[size_t(db_output)];
      HIPTRY(launch_db_bits(b.dev(slot), b.stride(slot), int(b.bits_w), int(b.bits_h), int(b.lanes.size()),
                            db_thresh, reinterpret_cast<unsigned long long *>(b.arena + b.bits_off), stream),
             "thresholding the map");
    }
  if (copy_out && !copy_out_all(err)) return false;
  if (sync) HIPTRY(hipStreamSynchronize(stream), "running the plan");
  return true;
}

// Every batch's outputs (and DB bitmasks) to the pinned host buffers, queued
// on the model's stream.
bool Model::copy_out_all(std::string &err) {
  for (size_t g = 0; g < active_batches; g++) {
    Batch &b = *batches[g];
    const Plan &p = b.plan;
    for (size_t k = 0; k < p.out_slot.size(); k++)
      HIPTRY(hipMemcpy2DAsync(b.host_out[k], p.out_n[k] * sizeof(float), b.dev(p.out_slot[k]),
                              b.stride(p.out_slot[k]) * sizeof(float), p.out_n[k] * sizeof(float),
                              b.lanes.size(), hipMemcpyDeviceToHost, stream),
             "copying the results");
    if (db_output >= 0)
      HIPTRY(hipMemcpyAsync(b.host_bits, b.arena + b.bits_off,
                            b.lanes.size() * b.bits_h * b.bits_wpr * sizeof(unsigned long long),
                            hipMemcpyDeviceToHost, stream),
             "copying the DB mask");
  }
  return true;
}

// From the next run on, also write output `output`'s DB threshold as row
// bitmasks (output < 0: stop). The lanes keep their sizes; their memory is
// arranged again for the bitmasks.
bool Model::set_db_mask(long output, float thresh, std::string &err) {
  HIPTRY(hipSetDevice(device), "selecting the GPU");
  if (output >= long(plan.out_slot.size())) return err = fmt("the plan has no output %ld", output), false;
  const long before = db_output;
  db_output = output < 0 ? -1 : output;
  db_thresh = thresh;
  if (before == db_output) return true;
  drop_graph();
  for (size_t g = 0; g < active_batches; g++)
    if (!arrange(*batches[g], err)) {
      db_output = before;
      return false;
    }
  return true;
}

}  // namespace ppocr

// ---------------------------------------------------------------- C ABI

struct ppocr_gpu_model {
  ppocr::Model m;
};

using ppocr::Batch;
using ppocr::put_err;

extern "C" {

int ppocr_gpu_load_bytes(const void *bytes, size_t len, ppocr_gpu_model **out, char *err,
                         size_t err_len) {
  if (!out) return put_err("no output handle", err, err_len), 1;
  *out = nullptr;
  std::unique_ptr<ppocr_gpu_model> h(new (std::nothrow) ppocr_gpu_model());
  if (!h) return put_err("out of memory", err, err_len), 1;
  std::string e;
  if (!h->m.load(static_cast<const uint8_t *>(bytes), len, e)) return put_err(e, err, err_len), 1;
  *out = h.release();
  return 0;
}

int ppocr_gpu_load(const char *plan_path, ppocr_gpu_model **out, char *err, size_t err_len) {
  if (out) *out = nullptr;
  std::ifstream f(plan_path ? plan_path : "", std::ios::binary);
  if (!f) return put_err(std::string("reading the plan: cannot open ") + (plan_path ? plan_path : "(null)"), err, err_len), 1;
  std::vector<char> bytes((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  return ppocr_gpu_load_bytes(bytes.data(), bytes.size(), out, err, err_len);
}

void ppocr_gpu_free(ppocr_gpu_model *model) { delete model; }

const char *ppocr_gpu_device(const ppocr_gpu_model *model) { return model ? model->m.name.c_str() : ""; }

int ppocr_gpu_integrated(const ppocr_gpu_model *model) { return model ? model->m.integrated : 0; }

int ppocr_gpu_set_sizes(ppocr_gpu_model *model, const size_t *hw, size_t n_lanes, char *err,
                        size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  if (n_lanes > ppocr_gpu_max_lanes(model))
    return put_err(ppocr::fmt("%zu lanes, more than the %zu a run takes", n_lanes, ppocr_gpu_max_lanes(model)), err, err_len), 1;
  std::string e;
  if (!model->m.set_sizes(hw, n_lanes, e)) return put_err(e, err, err_len), 1;
  return 0;
}

int ppocr_gpu_set_input_size(ppocr_gpu_model *model, size_t height, size_t width, char *err,
                             size_t err_len) {
  size_t hw[2] = {height, width};
  return ppocr_gpu_set_sizes(model, hw, 1, err, err_len);
}

size_t ppocr_gpu_max_lanes(const ppocr_gpu_model *model) { return model ? model->m.max_lanes() : 0; }

size_t ppocr_gpu_lanes(const ppocr_gpu_model *model) { return model ? model->m.lane_at.size() : 0; }

float *ppocr_gpu_lane_input(ppocr_gpu_model *model, size_t lane, size_t *len) {
  if (!model || lane >= model->m.lane_at.size()) return nullptr;
  auto [g, i] = model->m.lane_at[lane];
  Batch &b = *model->m.batches[g];
  if (len) *len = b.in_len;
  return b.host_in + i * b.in_len;
}

const float *ppocr_gpu_lane_output(const ppocr_gpu_model *model, size_t lane, size_t index,
                                   size_t *len) {
  if (!model || lane >= model->m.lane_at.size()) return nullptr;
  auto [g, i] = model->m.lane_at[lane];
  const Batch &b = *model->m.batches[g];
  if (index >= b.plan.out_slot.size()) return nullptr;
  size_t n = b.plan.out_n[index];
  if (len) *len = n;
  return b.host_out[index] + i * n;
}

int ppocr_gpu_set_db_mask(ppocr_gpu_model *model, long output, float thresh, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  std::string e;
  if (!model->m.set_db_mask(output, thresh, e)) return put_err(e, err, err_len), 1;
  return 0;
}

const uint64_t *ppocr_gpu_lane_db_mask(const ppocr_gpu_model *model, size_t lane, size_t *words_per_row,
                                       size_t *rows) {
  if (!model || model->m.db_output < 0 || lane >= model->m.lane_at.size()) return nullptr;
  auto [g, i] = model->m.lane_at[lane];
  const Batch &b = *model->m.batches[g];
  if (words_per_row) *words_per_row = b.bits_wpr;
  if (rows) *rows = b.bits_h;
  return reinterpret_cast<const uint64_t *>(b.host_bits + i * b.bits_h * b.bits_wpr);
}

size_t ppocr_gpu_output_count(const ppocr_gpu_model *model) {
  return model ? model->m.plan.out_slot.size() : 0;
}

int ppocr_gpu_run(ppocr_gpu_model *model, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  std::string e;
  if (!model->m.run(true, true, e)) return put_err(e, err, err_len), 1;
  return 0;
}

float *ppocr_gpu_lane_input_device(ppocr_gpu_model *model, size_t lane, size_t *len) {
  if (!model || lane >= model->m.lane_at.size()) return nullptr;
  auto [g, i] = model->m.lane_at[lane];
  Batch &b = *model->m.batches[g];
  if (len) *len = b.in_len;
  return b.dev(b.plan.in_slot) + i * b.stride(b.plan.in_slot);
}

int ppocr_gpu_run_device(ppocr_gpu_model *model, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  std::string e;
  if (!model->m.run(false, true, e)) return put_err(e, err, err_len), 1;
  return 0;
}

int ppocr_gpu_run_device_async(ppocr_gpu_model *model, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  std::string e;
  if (!model->m.run(false, true, e, false)) return put_err(e, err, err_len), 1;
  return 0;
}

int ppocr_gpu_wait(ppocr_gpu_model *model, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  hipSetDevice(model->m.device);
  const hipError_t r = hipStreamSynchronize(model->m.stream);
  if (r != hipSuccess) return put_err(std::string("running the plan: ") + hipGetErrorString(r), err, err_len), 1;
  return 0;
}

int ppocr_gpu_upload(ppocr_gpu_model *model, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  ppocr::Model &m = model->m;
  std::string e;
  hipSetDevice(m.device);
  for (size_t g = 0; g < m.active_batches; g++) {
    Batch &b = *m.batches[g];
    const ppocr::Plan &p = b.plan;
    hipError_t r = hipMemcpy2DAsync(b.dev(p.in_slot), b.stride(p.in_slot) * sizeof(float), b.host_in,
                                    b.in_len * sizeof(float), b.in_len * sizeof(float), b.lanes.size(),
                                    hipMemcpyHostToDevice, m.stream);
    if (r != hipSuccess) return put_err(std::string("copying the input: ") + hipGetErrorString(r), err, err_len), 1;
  }
  hipError_t r = hipStreamSynchronize(m.stream);
  if (r != hipSuccess) return put_err(std::string("copying the input: ") + hipGetErrorString(r), err, err_len), 1;
  return 0;
}

int ppocr_gpu_download(ppocr_gpu_model *model, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  ppocr::Model &m = model->m;
  hipSetDevice(m.device);
  std::string e;
  if (!m.copy_out_all(e)) return put_err(e, err, err_len), 1;
  hipError_t r = hipStreamSynchronize(m.stream);
  if (r != hipSuccess) return put_err(std::string("copying the results: ") + hipGetErrorString(r), err, err_len), 1;
  return 0;
}

int ppocr_gpu_run_resident(ppocr_gpu_model *model, int repeats, float *ms, char *err, size_t err_len) {
  if (!model) return put_err("no model", err, err_len), 1;
  ppocr::Model &m = model->m;
  hipSetDevice(m.device);
  if (m.lane_at.empty()) return put_err("no lanes are set", err, err_len), 1;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  if (ms) {
    hipEventCreate(&t0);
    hipEventCreate(&t1);
    hipEventRecord(t0, m.stream);
  }
  for (int r = 0; r < repeats; r++) {
    std::string e;
    if (!m.enqueue(e)) {
      if (t0) hipEventDestroy(t0), hipEventDestroy(t1);
      return put_err(e, err, err_len), 1;
    }
  }
  hipError_t e = hipSuccess;
  if (ms) {
    hipEventRecord(t1, m.stream);
    e = hipEventSynchronize(t1);
    if (e == hipSuccess) hipEventElapsedTime(ms, t0, t1);
    hipEventDestroy(t0);
    hipEventDestroy(t1);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(m.stream);
  if (e != hipSuccess) return put_err(std::string("running the plan: ") + hipGetErrorString(e), err, err_len), 1;
  return 0;
}

void *ppocr_gpu_stream(ppocr_gpu_model *model) { return model ? (void *)model->m.stream : nullptr; }

int ppocr_gpu_set_graphs(ppocr_gpu_model *model, int enable) {
  if (!model) return 1;
  model->m.drop_graph();
  model->m.use_graphs = enable != 0;
  return 0;
}

size_t ppocr_gpu_launch_count(const ppocr_gpu_model *model) {
  if (!model) return 0;
  size_t n = 0;
  for (size_t g = 0; g < model->m.active_batches; g++) n += model->m.batches[g]->launches.size();
  return n;
}

static const ppocr::Launch *launch_at(const ppocr_gpu_model *model, size_t i) {
  for (size_t g = 0; g < model->m.active_batches; g++) {
    const auto &ls = model->m.batches[g]->launches;
    if (i < ls.size()) return &ls[i];
    i -= ls.size();
  }
  return nullptr;
}

const char *ppocr_gpu_launch_name(const ppocr_gpu_model *model, size_t i, size_t *op) {
  if (!model) return nullptr;
  const ppocr::Launch *l = launch_at(model, i);
  if (!l) return nullptr;
  if (op) *op = size_t(l->op);
  return l->name.c_str();
}

size_t ppocr_gpu_launch_ops(const ppocr_gpu_model *model, size_t i, size_t *ops, size_t cap) {
  if (!model) return 0;
  const ppocr::Launch *l = launch_at(model, i);
  if (!l) return 0;
  const std::vector<int> one{l->op};
  const std::vector<int> &v = l->member_ops.empty() ? one : l->member_ops;
  for (size_t k = 0; k < v.size() && k < cap && ops; k++) ops[k] = size_t(v[k]);
  return v.size();
}

int ppocr_gpu_launch_work(const ppocr_gpu_model *model, size_t i, double *flops, double *bytes) {
  if (!model) return 1;
  const ppocr::Launch *l = launch_at(model, i);
  if (!l) return 1;
  if (flops) *flops = l->flops;
  if (bytes) *bytes = l->bytes;
  return 0;
}

int ppocr_gpu_profile_launches(ppocr_gpu_model *model, int repeats, float *ms, char *err, size_t err_len) {
  if (!model || !ms || repeats < 1) return put_err("bad arguments", err, err_len), 1;
  ppocr::Model &m = model->m;
  hipSetDevice(m.device);
  size_t n = ppocr_gpu_launch_count(model);
  hipEvent_t t0, t1;
  hipEventCreate(&t0);
  hipEventCreate(&t1);
  for (size_t i = 0; i < n; i++) {
    const ppocr::Launch *l = launch_at(model, i);
    hipEventRecord(t0, m.stream);
    for (int r = 0; r < repeats; r++) {
      hipError_t e = l->fn(m.stream);
      if (e != hipSuccess) {
        hipEventDestroy(t0), hipEventDestroy(t1);
        return put_err(ppocr::fmt("launching %s: %s", l->name.c_str(), hipGetErrorString(e)), err, err_len), 1;
      }
    }
    hipEventRecord(t1, m.stream);
    hipError_t e = hipEventSynchronize(t1);
    if (e != hipSuccess) {
      hipEventDestroy(t0), hipEventDestroy(t1);
      return put_err(std::string("profiling: ") + hipGetErrorString(e), err, err_len), 1;
    }
    float t = 0;
    hipEventElapsedTime(&t, t0, t1);
    ms[i] = t / repeats;
  }
  hipEventDestroy(t0);
  hipEventDestroy(t1);
  return 0;
}

}  // extern "C"
