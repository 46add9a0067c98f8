// The engine's PPOCRPL1 plan: reading, checking and sizing.
//
// Follows src/engine/plan.rs: the file layout (9-20), the 15 kinds and the
// folded activations (79-175, plus this backend's code 7, hard swish), the
// size rules (414-494), every consistency check (498-767), the subnormal
// flush and the refusal of non-finite weights (819-842), and the layer norm
// epsilon check (367-377). Nothing in a plan is trusted: after `parse` and
// every successful `set_size` the executor can index without re-checking.
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace ppocr {

enum Kind : int {
  K_CONV, K_DWCONV, K_ADD, K_MAXPOOL, K_AVGPOOL, K_CHANNELMUL, K_CONCATC, K_LAYERNORM,
  K_ATTENTION, K_MEAN, K_CTCHEAD, K_CTCARGMAX, K_UPSAMPLE, K_UPSAMPLEADD, K_CONVTRANSPOSE,
  K_COUNT
};
enum { FUSED_COUNT = 8 };

const char *kind_name(int kind);

struct Op {
  int kind = 0, fused = 0;
  size_t x = 0, x2 = 0, y = 0;
  size_t ih = 0, iw = 0, ic = 0, oh = 0, ow = 0, oc = 0;
  size_t kh = 0, kw = 0, sh = 0, sw = 0;
  long pt = 0, pb = 0, pl = 0, pr = 0;
  size_t n2 = 0;
  size_t w0 = 0, w1 = 0, b0 = 0, b1 = 0;

  size_t out_len() const { return oh * ow * oc; }
  size_t in_len() const { return ih * iw * ic; }
  bool has_second(size_t *slot) const;
  bool is_pointwise() const;
};

struct Plan {
  size_t in_slot = 0, in_h = 0, in_w = 0, in_c = 0;
  std::vector<size_t> out_slot, out_n;
  std::vector<Op> ops;
  std::vector<size_t> pool;  // floats each buffer holds at the current size

  // Read and check a plan file; fills `weights` (subnormals flushed).
  bool parse(const uint8_t *bytes, size_t len, std::vector<float> &weights, std::string &err);
  // Re-derive every shape for an input of height x width and check the
  // result; on error the plan keeps its previous size.
  bool set_size(size_t height, size_t width, size_t weight_floats, std::string &err);

 private:
  bool produced(size_t before, size_t slot, size_t *h, size_t *w, size_t *c) const;
  bool derive(size_t height, size_t width, std::string &err);
  bool check(size_t weight_floats, std::string &err) const;
};

}  // namespace ppocr
