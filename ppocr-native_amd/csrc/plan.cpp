// PPOCRPL1 reading and checking; see plan.hpp. Each rule cites the
// src/engine/plan.rs line it follows.
#include "plan.hpp"

#include <string.h>

#include <cstdarg>
#include <cstdio>
#include <limits>

namespace ppocr {

namespace {

const size_t OP_FIELDS = 20;                      // plan.rs:68
const size_t MAX_SCRATCH_FLOATS = size_t(1) << 30;  // plan.rs:73
const size_t MAX_WINDOW = size_t(1) << 16;          // plan.rs:77
const size_t SMAX = std::numeric_limits<size_t>::max();

std::string fmt(const char *f, ...) {
  char buf[256];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

bool shape_len(size_t a, size_t b, size_t c, size_t *out) {
  if (!a || !b || !c || a > SMAX / b) return false;
  size_t ab = a * b;
  if (ab > SMAX / c) return false;
  *out = ab * c;
  return true;
}

bool window(size_t n, long before, long after, size_t k, size_t s, size_t *out) {
  if (before < 0 || after < 0 || s == 0) return false;
  size_t span = n + size_t(before) + size_t(after);
  if (span < k) return false;
  *out = (span - k) / s + 1;
  return true;
}

}  // namespace

const char *kind_name(int kind) {
  static const char *names[K_COUNT] = {
      "Conv", "Dwconv", "Add", "Maxpool", "Avgpool", "Channelmul", "Concatc", "Layernorm",
      "Attention", "Mean", "Ctchead", "Ctcargmax", "Upsample", "Upsampleadd", "Convtranspose"};
  return kind >= 0 && kind < K_COUNT ? names[kind] : "?";
}

// plan.rs:251-257
bool Op::has_second(size_t *slot) const {
  bool binary = kind == K_ADD || kind == K_CHANNELMUL || kind == K_CONCATC ||
                kind == K_UPSAMPLEADD || (kind == K_CONV && n2 > 0);
  if (binary && slot) *slot = x2;
  return binary;
}

// plan.rs:260-264
bool Op::is_pointwise() const {
  return kind == K_CONV && kh == 1 && kw == 1 && sh == 1 && sw == 1 && pt == 0 && pb == 0 &&
         pl == 0 && pr == 0;
}

// plan.rs:403-408
bool Plan::produced(size_t before, size_t slot, size_t *h, size_t *w, size_t *c) const {
  for (size_t i = before; i-- > 0;) {
    if (ops[i].y == slot) {
      *h = ops[i].oh, *w = ops[i].ow, *c = ops[i].oc;
      return true;
    }
  }
  if (slot == in_slot) {
    *h = in_h, *w = in_w, *c = in_c;
    return true;
  }
  return false;
}

// plan.rs:414-494
bool Plan::derive(size_t height, size_t width, std::string &err) {
  in_h = height, in_w = width;
  for (size_t i = 0; i < ops.size(); i++) {
    Op &op = ops[i];
    size_t h, w, c;
    if (!produced(i, op.x, &h, &w, &c)) return err = fmt("op %zu reads a buffer nothing wrote", i), false;
    if (c != op.ic) return err = fmt("op %zu reads a tensor of another shape", i), false;
    size_t oh = 0, ow = 0;
    switch (op.kind) {
      case K_CONV: case K_DWCONV: case K_MAXPOOL: case K_AVGPOOL:
        if (!window(h, op.pt, op.pb, op.kh, op.sh, &oh) || !window(w, op.pl, op.pr, op.kw, op.sw, &ow))
          return err = fmt("op %zu has a window larger than its padded input", i), false;
        break;
      case K_UPSAMPLE: case K_UPSAMPLEADD:
        if ((op.sh && h > SMAX / op.sh) || (op.sw && w > SMAX / op.sw))
          return err = fmt("op %zu output size overflows", i), false;
        oh = h * op.sh, ow = w * op.sw;
        break;
      case K_CONVTRANSPOSE:
        if ((op.kh && h > SMAX / op.kh) || (op.kw && w > SMAX / op.kw))
          return err = fmt("op %zu output size overflows", i), false;
        oh = h * op.kh, ow = w * op.kw;
        break;
      case K_MEAN: oh = ow = 1; break;
      default: oh = h, ow = w;
    }
    bool has = true;
    size_t wh = oh, ww = ow, wc = op.oc;
    switch (op.kind) {
      case K_ADD: case K_UPSAMPLEADD: break;
      case K_CONCATC: wc = op.n2; break;
      case K_CHANNELMUL: wh = ww = 1; break;
      case K_CONV:
        if (op.n2 > 0) wh = h, ww = w, wc = op.n2;
        else has = false;
        break;
      default: has = false;
    }
    if (has) {
      size_t h2, w2, c2;
      if (!produced(i, op.x2, &h2, &w2, &c2) || h2 != wh || w2 != ww || c2 != wc)
        return err = fmt("op %zu reads a second tensor of another shape", i), false;
    }
    op.ih = h, op.iw = w, op.oh = oh, op.ow = ow;
  }
  std::fill(pool.begin(), pool.end(), 0);
  size_t image;
  if (!shape_len(height, width, in_c, &image)) return err = "input shape is zero or overflows", false;
  if (in_slot >= pool.size()) return err = fmt("buffer %zu does not exist", in_slot), false;
  pool[in_slot] = std::max(pool[in_slot], image);
  for (size_t i = 0; i < ops.size(); i++) {
    size_t n;
    if (!shape_len(ops[i].oh, ops[i].ow, ops[i].oc, &n))
      return err = fmt("op %zu output shape is zero or overflows", i), false;
    if (ops[i].y >= pool.size()) return err = fmt("buffer %zu does not exist", ops[i].y), false;
    pool[ops[i].y] = std::max(pool[ops[i].y], n);
  }
  for (size_t k = 0; k < out_slot.size(); k++) {
    size_t h, w, c;
    if (!produced(ops.size(), out_slot[k], &h, &w, &c))
      return err = fmt("output %zu is never written", k), false;
    out_n[k] = h * w * c;
  }
  return true;
}

// plan.rs:498-767
bool Plan::check(size_t weight_floats, std::string &err) const {
  for (size_t n : pool)
    if (n > MAX_SCRATCH_FLOATS)
      return err = fmt("a buffer wants %zu floats, ceiling is %zu", n, MAX_SCRATCH_FLOATS), false;
  size_t input_len;
  if (!shape_len(in_h, in_w, in_c, &input_len)) return err = "input shape is zero or overflows", false;
  if (in_slot >= pool.size() || pool[in_slot] < input_len)
    return err = "the input buffer is smaller than the image", false;
  for (size_t k = 0; k < out_slot.size(); k++)
    if (out_slot[k] >= pool.size() || pool[out_slot[k]] < out_n[k])
      return err = fmt("output %zu claims %zu elements, its buffer holds fewer", k, out_n[k]), false;
  for (size_t i = 0; i < ops.size(); i++) {
    const Op &op = ops[i];
    auto at = [&](const char *what) { return fmt("op %zu (%s) %s", i, kind_name(op.kind), what); };
    size_t in_len, out_len;
    if (!shape_len(op.ih, op.iw, op.ic, &in_len)) return err = at("input shape is zero or overflows"), false;
    if (!shape_len(op.oh, op.ow, op.oc, &out_len)) return err = at("output shape is zero or overflows"), false;
    switch (op.kind) {
      case K_CONV: case K_DWCONV: case K_AVGPOOL: case K_MAXPOOL: {
        size_t k4[4] = {op.kh, op.kw, op.sh, op.sw};
        long p4[4] = {op.pt, op.pb, op.pl, op.pr};
        for (int j = 0; j < 4; j++)
          if (k4[j] == 0 || k4[j] > MAX_WINDOW || p4[j] < 0 || size_t(p4[j]) > MAX_WINDOW)
            return err = at("has an unsupported kernel, stride or padding"), false;
        break;
      }
      case K_MEAN:
        if (op.oh != 1 || op.ow != 1 || op.ic != op.oc) return err = at("invalid channel mean"), false;
        break;
      case K_CONCATC:
        if (op.ih != op.oh || op.iw != op.ow || op.ic + op.n2 != op.oc)
          return err = at("invalid channel concatenation"), false;
        break;
      case K_CTCHEAD: case K_CTCARGMAX: {
        size_t vocab = op.kind == K_CTCHEAD ? op.oc : op.n2;
        size_t columns = (vocab + 15) / 16 * 16;
        if (op.ih != 1 || op.oh != 1 || op.iw != op.ow || vocab == 0 ||
            (op.kind == K_CTCARGMAX && op.oc != 2) || (op.ic && columns > SMAX / op.ic) ||
            columns * op.ic != op.w1 || op.b1 != columns)
          return err = at("invalid CTC head"), false;
        break;
      }
      case K_LAYERNORM:
        if (op.oc * 2 + 1 != op.w1) return err = at("needs gamma, beta and epsilon"), false;
        break;
      case K_ATTENTION:
        if (op.ih != 1 || op.oh != 1 || op.iw != op.ow || op.oc * 3 != op.ic || op.n2 == 0 ||
            op.oc % op.n2 != 0 || op.w1 != 1 || op.iw > MAX_SCRATCH_FLOATS / op.iw)
          return err = at("invalid attention shape"), false;
        break;
      case K_UPSAMPLE: case K_UPSAMPLEADD:
        if (op.ic != op.oc || op.sh == 0 || op.sw == 0 || op.ih * op.sh != op.oh || op.iw * op.sw != op.ow)
          return err = at("invalid upsampling"), false;
        break;
      case K_CONVTRANSPOSE: {
        size_t cols = op.kh * op.kw * op.oc;
        if (op.kh == 0 || op.kw == 0 || op.sh != op.kh || op.sw != op.kw || op.pt || op.pb || op.pl ||
            op.pr || op.ih * op.kh != op.oh || op.iw * op.kw != op.ow || cols * op.ic != op.w1 ||
            (op.b1 != 0 && op.b1 != cols))
          return err = at("invalid transposed convolution"), false;
        break;
      }
      default: break;
    }
    if ((op.kind == K_ADD || op.kind == K_CHANNELMUL || op.kind == K_LAYERNORM) &&
        (op.ih != op.oh || op.iw != op.ow || op.ic != op.oc))
      return err = at("elementwise input/output shapes differ"), false;
    if (op.kind == K_AVGPOOL &&
        (op.ic != op.oc || op.pt || op.pb || op.pl || op.pr || op.kh > op.ih || op.kw > op.iw ||
         op.oh != (op.ih - op.kh) / op.sh + 1 || op.ow != (op.iw - op.kw) / op.sw + 1))
      return err = at("average pool requires complete valid windows"), false;
    if (op.kind == K_MAXPOOL) {
      if (op.ic != op.oc || op.pt != 0 || op.pl != 0)
        return err = at("maxpool changes channels or requests unsupported padding"), false;
      if ((op.oh - 1) * op.sh >= op.ih || (op.ow - 1) * op.sw >= op.iw)
        return err = at("maxpool contains an empty output window"), false;
    }
    if (op.is_pointwise() && (op.ih != op.oh || op.iw != op.ow))
      return err = at("unit-stride pointwise changes spatial dimensions"), false;
    if (op.x >= pool.size() || pool[op.x] < in_len) return err = at("reads past its input buffer"), false;
    if (op.y >= pool.size() || pool[op.y] < out_len) return err = at("writes past its output buffer"), false;
    size_t s2 = 0;
    bool has2 = op.has_second(&s2);
    if (op.y == op.x || (has2 && s2 == op.y)) return err = at("writes the buffer it reads"), false;
    if (has2) {
      size_t need;
      switch (op.kind) {
        case K_ADD: case K_UPSAMPLEADD: need = out_len; break;
        case K_CONCATC: need = op.oh * op.ow * op.n2; break;
        case K_CONV: need = op.ih * op.iw * op.n2; break;
        default: need = op.oc;
      }
      if (s2 >= pool.size() || pool[s2] < need) return err = at("reads past its second input buffer"), false;
    }
    if (op.kind == K_CONV || op.kind == K_DWCONV) {
      size_t taps = op.kh * op.kw, want;
      if (op.n2 > 0 && (op.kind == K_DWCONV || op.is_pointwise()))
        return err = at("reads a second input it cannot"), false;
      if (op.kind == K_DWCONV) {
        if (op.ic != op.oc) return err = at("is depthwise but changes channel count"), false;
        want = taps * op.oc;
      } else {
        want = (op.ic + op.n2) * taps * op.oc;
      }
      if (op.w1 != want) return err = at("has weights the shape contradicts"), false;
      if (op.b1 != 0 && op.b1 != op.oc) return err = at("has a bias of the wrong length"), false;
    }
    bool weighted = op.kind == K_CONV || op.kind == K_DWCONV || op.kind == K_LAYERNORM ||
                    op.kind == K_ATTENTION || op.kind == K_CTCHEAD || op.kind == K_CTCARGMAX ||
                    op.kind == K_CONVTRANSPOSE;
    if (!weighted && (op.w1 || op.b1)) return err = at("has weights it does not use"), false;
    if (op.fused != 0 && !(op.kind == K_CONV || op.kind == K_DWCONV || op.kind == K_ADD ||
                           op.kind == K_CONVTRANSPOSE))
      return err = at("has an invalid folded activation"), false;
    size_t blocks[2][2] = {{op.w0, op.w1}, {op.b0, op.b1}};
    for (auto &b : blocks) {
      if (!b[1]) continue;
      if (b[0] > SMAX - b[1] || b[0] + b[1] > weight_floats)
        return err = at("has a weight block past the weights"), false;
    }
  }
  return true;
}

bool Plan::set_size(size_t height, size_t width, size_t weight_floats, std::string &err) {
  size_t oh = in_h, ow = in_w;
  if (derive(height, width, err) && check(weight_floats, err)) return true;
  std::string ignored;
  derive(oh, ow, ignored);
  return false;
}

// plan.rs:303-365, 819-842
bool Plan::parse(const uint8_t *bytes, size_t len, std::vector<float> &weights, std::string &err) {
  if (len < 8 || memcmp(bytes, "PPOCRPL1", 8) != 0)
    return err = "unsupported plan: not a ppocr-native plan", false;
  size_t at = 8;
  auto next = [&](size_t *v) {
    if (at + 4 > len) return false;
    uint32_t w;
    memcpy(&w, bytes + at, 4);
    at += 4;
    *v = w;
    return true;
  };
  const char *trunc = "invalid plan: the description is truncated";
  size_t nbuf, nout, nops;
  if (!next(&in_slot) || !next(&in_h) || !next(&in_w) || !next(&in_c) || !next(&nbuf) ||
      !next(&nout) || !next(&nops))
    return err = trunc, false;
  // A count past the file fails on the first missing word, before reserving.
  if (nout > (len - at) / 4 || nops > (len - at) / (4 * OP_FIELDS) + 1) return err = trunc, false;
  out_slot.assign(nout, 0);
  out_n.assign(nout, 0);
  for (size_t k = 0; k < nout; k++)
    if (!next(&out_slot[k])) return err = trunc, false;
  ops.assign(nops, Op());
  for (size_t i = 0; i < nops; i++) {
    size_t f[OP_FIELDS];
    for (size_t j = 0; j < OP_FIELDS; j++)
      if (!next(&f[j])) return err = trunc, false;
    if (f[0] >= K_COUNT) return err = fmt("unsupported plan: operation kind %zu is unknown", f[0]), false;
    if (f[1] >= FUSED_COUNT) return err = fmt("unsupported plan: activation %zu is unknown", f[1]), false;
    Op &op = ops[i];
    op.kind = int(f[0]), op.fused = int(f[1]);
    op.x = f[2], op.x2 = f[3], op.y = f[4], op.ic = f[5], op.oc = f[6];
    op.kh = f[7], op.kw = f[8], op.sh = f[9], op.sw = f[10];
    op.pt = long(f[11]), op.pb = long(f[12]), op.pl = long(f[13]), op.pr = long(f[14]);
    op.n2 = f[15], op.w0 = f[16], op.w1 = f[17], op.b0 = f[18], op.b1 = f[19];
  }
  if (nbuf == 0 || nbuf > nops + 1)
    return err = fmt("invalid plan: %zu buffers for %zu operations", nbuf, nops), false;
  pool.assign(nbuf, 0);
  size_t start = (at + 63) / 64 * 64;
  if (start > len) return err = "invalid plan: the plan ends before its weights", false;
  size_t raw = len - start;
  if (raw % 4) return err = fmt("invalid plan: the weights are %zu bytes, not a whole number of floats", raw), false;
  weights.resize(raw / 4);
  for (size_t i = 0; i < weights.size(); i++) {
    uint32_t b;
    memcpy(&b, bytes + start + 4 * i, 4);
    if ((b & 0x7f800000u) == 0) b &= 0x80000000u;  // subnormal to signed zero
    if ((b & 0x7f800000u) == 0x7f800000u)
      return err = fmt("invalid plan: the weights hold a non-finite value at float %zu", i), false;
    float v;
    memcpy(&v, &b, 4);
    weights[i] = v;
  }
  std::string e;
  if (!derive(in_h, in_w, e) || !check(weights.size(), e)) return err = "invalid plan: " + e, false;
  for (const Op &op : ops)
    if (op.kind == K_LAYERNORM && !(weights[op.w0 + 2 * op.oc] > 0.0f))
      return err = "invalid plan: layer normalization epsilon is not positive", false;
  return true;
}

}  // namespace ppocr
