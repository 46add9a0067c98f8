// The C ABI of the host stages (include/ppocr_hip.h): the recogniser's text
// (text.cpp) and the detector's boxes (boxes.cpp), with their buffers and
// errors marshalled for C callers.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "post.hpp"
#include "ppocr_hip.h"

struct ppocr_dictionary {
  ppocr::Dictionary d;
};

namespace {

void say(char *err, size_t len, const char *msg) {
  if (!err || !len) return;
  std::snprintf(err, len, "%s", msg);
}

}  // namespace

extern "C" {

int ppocr_dictionary_load(const char *text, size_t len, ppocr_dictionary **out, char *err, size_t err_len) {
  if (!out || (!text && len)) return say(err, err_len, "null argument"), 1;
  *out = new ppocr_dictionary{ppocr::Dictionary(std::string(text ? text : "", len))};
  return 0;
}

void ppocr_dictionary_free(ppocr_dictionary *d) { delete d; }

size_t ppocr_dictionary_len(const ppocr_dictionary *d) { return d ? d->d.size() : 0; }

const char *ppocr_dictionary_class(const ppocr_dictionary *d, size_t index, size_t *len) {
  if (!d || index >= d->d.size()) return nullptr;
  if (len) *len = d->d.classes[index].size();
  return d->d.classes[index].c_str();
}

static int decode_out(const std::string &text, double score, char *out, size_t cap, size_t *out_len,
                      double *out_score, char *err, size_t err_len) {
  if (out_len) *out_len = text.size();
  if (out_score) *out_score = score;
  if (text.size() + 1 > cap || !out) return say(err, err_len, "text buffer too small"), 2;
  std::memcpy(out, text.data(), text.size());
  out[text.size()] = 0;
  return 0;
}

int ppocr_ctc_decode(const ppocr_dictionary *d, const uint32_t *best, const float *prob, size_t steps, char *text,
                     size_t text_cap, size_t *text_len, double *score, char *err, size_t err_len) {
  if (!d || (steps && (!best || !prob))) return say(err, err_len, "null argument"), 1;
  std::string t;
  double s = 0.0;
  if (!ppocr::ctc_decode(best, prob, steps, d->d, t, s)) return say(err, err_len, "a class is outside the dictionary"), 1;
  return decode_out(t, s, text, text_cap, text_len, score, err, err_len);
}

int ppocr_ctc_decode_pairs(const ppocr_dictionary *d, const float *pairs, size_t steps, char *text, size_t text_cap,
                           size_t *text_len, double *score, char *err, size_t err_len) {
  if (!d || (steps && !pairs)) return say(err, err_len, "null argument"), 1;
  std::vector<uint32_t> best(steps);
  std::vector<float> prob(steps);
  for (size_t t = 0; t < steps; t++) {
    const float c = pairs[2 * t];
    if (!(c >= 0.0f) || c != std::floor(c) || c >= 4294967296.0f)
      return say(err, err_len, "a class is not a whole number"), 1;
    best[t] = uint32_t(c), prob[t] = pairs[2 * t + 1];
  }
  return ppocr_ctc_decode(d, best.data(), prob.data(), steps, text, text_cap, text_len, score, err, err_len);
}

int ppocr_find_contours(const uint8_t *mask, size_t width, size_t height, int32_t *points, size_t points_cap,
                        size_t *lengths, size_t contours_cap, size_t *n_points, size_t *n_contours) {
  if (!mask && width * height) return 1;
  const ppocr::Contours c = ppocr::find_contours(mask, width, height);
  size_t total = 0;
  for (const auto &v : c) total += v.size();
  if (n_points) *n_points = total;
  if (n_contours) *n_contours = c.size();
  if (total > points_cap || c.size() > contours_cap || (total && !points) || (c.size() && !lengths)) return 2;
  size_t k = 0;
  for (size_t i = 0; i < c.size(); i++) {
    lengths[i] = c[i].size();
    for (const auto &p : c[i]) points[k++] = p.x, points[k++] = p.y;
  }
  return 0;
}

int ppocr_min_area_rect(const int32_t *points, size_t n, float *rect, float *corners) {
  if (n && !points) return 1;
  std::vector<ppocr::Point> pts(n);
  for (size_t i = 0; i < n; i++) pts[i] = {points[2 * i], points[2 * i + 1]};
  const ppocr::RotatedRect r = ppocr::min_area_rect(pts);
  if (rect) rect[0] = r.cx, rect[1] = r.cy, rect[2] = r.width, rect[3] = r.height, rect[4] = r.angle;
  if (corners) {
    const ppocr::Quad q = ppocr::box_points(r);
    for (int i = 0; i < 4; i++) corners[2 * i] = q[i][0], corners[2 * i + 1] = q[i][1];
  }
  return 0;
}

int ppocr_unclip(const float *quad, double ratio, int32_t *ring, size_t cap, size_t *n) {
  if (!quad) return 1;
  ppocr::Quad q;
  for (int i = 0; i < 4; i++) q[i] = {quad[2 * i], quad[2 * i + 1]};
  const std::vector<ppocr::Point> r = ppocr::unclip(q, ratio);
  if (n) *n = r.size();
  if (r.size() > cap || (r.size() && !ring)) return 2;
  for (size_t i = 0; i < r.size(); i++) ring[2 * i] = r[i].x, ring[2 * i + 1] = r[i].y;
  return 0;
}

int ppocr_db_boxes(const float *prob, const uint8_t *mask, size_t map_w, size_t map_h, size_t dest_w,
                   size_t dest_h, const ppocr_db_options *options, float *boxes, size_t boxes_cap, size_t *n_boxes,
                   char *err, size_t err_len) {
  if ((!prob && map_w * map_h) || !options) return say(err, err_len, "null argument"), 1;
  if (!map_w || !map_h || !dest_w || !dest_h) return say(err, err_len, "empty map or page"), 1;
  ppocr::DbOptions o;
  o.thresh = options->thresh, o.box_thresh = options->box_thresh;
  o.unclip_ratio = options->unclip_ratio, o.max_candidates = options->max_candidates;
  const std::vector<ppocr::Quad> b = ppocr::boxes_from_prob(prob, mask, map_w, map_h, dest_w, dest_h, o);
  if (n_boxes) *n_boxes = b.size();
  if (b.size() > boxes_cap || (b.size() && !boxes)) return say(err, err_len, "box buffer too small"), 2;
  for (size_t i = 0; i < b.size(); i++)
    for (int k = 0; k < 4; k++) boxes[8 * i + 2 * k] = b[i][k][0], boxes[8 * i + 2 * k + 1] = b[i][k][1];
  return 0;
}

int ppocr_db_boxes_bits(const float *prob, const uint64_t *bits, size_t words_per_row, size_t map_w, size_t map_h,
                        size_t dest_w, size_t dest_h, const ppocr_db_options *options, float *boxes,
                        size_t boxes_cap, size_t *n_boxes, char *err, size_t err_len) {
  if ((!prob || !bits) && map_w * map_h) return say(err, err_len, "null argument"), 1;
  if (!options) return say(err, err_len, "null argument"), 1;
  if (!map_w || !map_h || !dest_w || !dest_h) return say(err, err_len, "empty map or page"), 1;
  if (words_per_row < (map_w + 63) / 64) return say(err, err_len, "fewer bit words a row than the map is wide"), 1;
  ppocr::DbOptions o;
  o.thresh = options->thresh, o.box_thresh = options->box_thresh;
  o.unclip_ratio = options->unclip_ratio, o.max_candidates = options->max_candidates;
  const std::vector<ppocr::Quad> b =
      ppocr::boxes_from_bits(prob, bits, words_per_row, map_w, map_h, dest_w, dest_h, o);
  if (n_boxes) *n_boxes = b.size();
  if (b.size() > boxes_cap || (b.size() && !boxes)) return say(err, err_len, "box buffer too small"), 2;
  for (size_t i = 0; i < b.size(); i++)
    for (int k = 0; k < 4; k++) boxes[8 * i + 2 * k] = b[i][k][0], boxes[8 * i + 2 * k + 1] = b[i][k][1];
  return 0;
}

}  // extern "C"
