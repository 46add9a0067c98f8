// Host stages either side of the GPU model: CTC text decode (text.cpp) and
// the DB post-process, probability map to text boxes (boxes.cpp).
#pragma once
#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

namespace ppocr {

struct Point {
  int32_t x, y;
  bool operator==(const Point &o) const { return x == o.x && y == o.y; }
};
using Quad = std::array<std::array<float, 2>, 4>;  // [x, y] corners
using Contours = std::vector<std::vector<Point>>;

// cv2.RotatedRect: angle in degrees within [-90, 0), the direction of the
// side called width, y pointing down.
struct RotatedRect {
  float cx, cy, width, height, angle;
};

// The recogniser's classes: blank, the model's characters, a space.
struct Dictionary {
  std::vector<std::string> classes;
  explicit Dictionary(const std::string &character_list);
  size_t size() const { return classes.size(); }
};

// Greedy CTC decode of per-step best classes and probabilities; false when a
// class is outside the dictionary.
bool ctc_decode(const uint32_t *best, const float *prob, size_t steps, const Dictionary &dict,
                std::string &text, double &score);

Contours find_contours(const uint8_t *mask, size_t width, size_t height);
// The same from row bitmasks: bit x % 64 of word y * words_per_row + x / 64
// is pixel (x, y); bits past the width must be zero.
Contours find_contours_bits(const uint64_t *bits, size_t words_per_row, size_t width, size_t height);
// Row bitmasks of mask[i] != 0, or of prob[i] > thresh when mask is null.
std::vector<uint64_t> pack_rows(const uint8_t *mask, const float *prob, float thresh, size_t width, size_t height);
double contour_mean(const float *map, size_t width, size_t height, const std::vector<Point> &contour);
RotatedRect min_area_rect(const std::vector<Point> &points);
Quad box_points(const RotatedRect &r);
std::pair<Quad, float> mini_box(const std::vector<Point> &points);
std::vector<Point> unclip(const Quad &quad, double ratio);

struct DbOptions {
  float thresh = 0.3f;          // text where prob > thresh (f32 compare)
  double box_thresh = 0.5;      // least mean probability inside a region
  double unclip_ratio = 1.5;    // growth: area * ratio / perimeter
  size_t max_candidates = 1000; // regions considered, in contour order
};

struct Candidate {
  enum Kind { kSmall, kLowScore, kSmallAfterUnclip, kKept } kind;
  double score;
  Point corners[4];
};
Candidate contour_candidate(const float *prob, size_t map_w, size_t map_h, const std::vector<Point> &contour,
                            size_t dest_w, size_t dest_h, const DbOptions &o);
bool order_and_clip(const Point corners[4], size_t width, size_t height, Quad &out);
void sort_boxes(std::vector<Quad> &boxes);
// `mask` (map_w * map_h bytes, nonzero = text) may be null: then prob > thresh.
std::vector<Quad> boxes_from_prob(const float *prob, const uint8_t *mask, size_t map_w, size_t map_h,
                                  size_t dest_w, size_t dest_h, const DbOptions &o);
// The same with the threshold already taken, as row bitmasks (the GPU's).
std::vector<Quad> boxes_from_bits(const float *prob, const uint64_t *bits, size_t words_per_row, size_t map_w,
                                  size_t map_h, size_t dest_w, size_t dest_h, const DbOptions &o);

}  // namespace ppocr
