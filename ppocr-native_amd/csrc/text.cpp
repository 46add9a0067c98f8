// Reading the recogniser's output: the class list of a model and the greedy
// CTC decode of its per-step (class, probability) output into text and a
// score, as RapidOCR computes them (src/rec.rs:45-161: Python's
// str.splitlines for the classes, numpy's pairwise f64 sum and Python's
// round to five decimals for the score).
#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

#include "post.hpp"

namespace ppocr {

// ------------------------------------------------------------ dictionary

// Decodes one UTF-8 code point at s[i] (the input is the model's character
// list, valid UTF-8); returns its length in bytes.
static size_t utf8_at(const std::string &s, size_t i, uint32_t *cp) {
  const unsigned char c = (unsigned char)s[i];
  size_t n = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 1;
  if (i + n > s.size()) n = 1;
  uint32_t v = n == 1 ? c : n == 2 ? (c & 0x1f) : n == 3 ? (c & 0x0f) : (c & 0x07);
  for (size_t k = 1; k < n; k++) v = v << 6 | ((unsigned char)s[i + k] & 0x3f);
  *cp = v;
  return n;
}

// Python's str.splitlines boundaries.
static bool line_break(uint32_t c) {
  return c == '\n' || c == '\r' || c == 0x0b || c == 0x0c || c == 0x1c || c == 0x1d || c == 0x1e ||
         c == 0x85 || c == 0x2028 || c == 0x2029;
}

Dictionary::Dictionary(const std::string &text) {
  classes.push_back("blank");
  size_t start = 0, i = 0;
  while (i < text.size()) {
    uint32_t cp;
    const size_t n = utf8_at(text, i, &cp);
    if (!line_break(cp)) {
      i += n;
      continue;
    }
    classes.push_back(text.substr(start, i - start));
    i += n;
    if (cp == '\r' && i < text.size() && text[i] == '\n') i++;  // "\r\n" is one break
    start = i;
  }
  if (start < text.size()) classes.push_back(text.substr(start));
  classes.push_back(" ");
}

// ------------------------------------------------------------ CTC decode

// numpy's float64 add.reduce: sequential below 8 values, eight running sums
// up to 128 values, and above that two halves split at a multiple of 8.
static double numpy_sum(const double *v, size_t n) {
  if (n < 8) {
    double s = 0.0;
    for (size_t i = 0; i < n; i++) s += v[i];
    return s;
  }
  if (n <= 128) {
    double r[8];
    for (int k = 0; k < 8; k++) r[k] = v[k];
    const size_t full = n - n % 8;
    for (size_t i = 8; i < full; i += 8)
      for (int k = 0; k < 8; k++) r[k] += v[i + k];
    double s = ((r[0] + r[1]) + (r[2] + r[3])) + ((r[4] + r[5]) + (r[6] + r[7]));
    for (size_t i = full; i < n; i++) s += v[i];
    return s;
  }
  const size_t half = n / 2 - (n / 2) % 8;
  return numpy_sum(v, half) + numpy_sum(v + half, n - half);
}

// Python's round(x, 5) of a value whose x * 1e5 is exact in f64.
static double round5(double x) { return std::nearbyint(x * 1e5) / 1e5; }

bool ctc_decode(const uint32_t *best, const float *prob, size_t steps, const Dictionary &dict,
                std::string &text, double &score) {
  text.clear();
  std::vector<double> kept;
  for (size_t t = 0; t < steps; t++) {
    const uint32_t c = best[t];
    if (c == 0 || (t > 0 && c == best[t - 1])) continue;
    if (c >= dict.size()) return false;
    text += dict.classes[c];
    kept.push_back(round5((double)prob[t]));
  }
  if (kept.empty()) {
    score = 0.0;
    return true;
  }
  score = round5(numpy_sum(kept.data(), kept.size()) / (double)kept.size());
  return true;
}

}  // namespace ppocr
