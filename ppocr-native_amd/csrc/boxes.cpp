// Text boxes out of the detector's probability map, on the host: the region
// borders of the thresholded map, each region's mean probability, its
// minimum-area rectangle, that rectangle grown by the unclip distance, and
// the boxes scaled to the page and put in reading order (RapidOCR's DB
// postprocess as the reference engine runs it, src/det.rs:291-452).
//
// The work is short and sequential per region, so it stays on the CPU (the
// threshold itself has a GPU kernel, db_mask in layers.hip). Every number it
// produces is the one the Python pipeline produces, to the bit; what fixes
// each piece of arithmetic is named where it is used:
//  - region borders: cv2.findContours(RETR_LIST, CHAIN_APPROX_SIMPLE), the
//    Suzuki-Abe border following (src/contour.rs:1-140);
//  - mean inside a border: cv2.fillPoly's even-odd spans (src/contour.rs:
//    142-199);
//  - minimum-area rectangle: cv2.convexHull's index order, cv2.minAreaRect's
//    f32 rotating calipers, cv2.boxPoints (src/geometry.rs:1-280);
//  - growth: shapely's area and length, pyclipper's round offset and the
//    union that tidies it (src/geometry.rs:282-435);
//  - scaling: numpy's f32 divide, multiply and round-half-even.
#include <unistd.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <functional>
#include <limits>
#include <mutex>
#include <numeric>
#include <thread>
#include <vector>

#include "post.hpp"

namespace ppocr {

namespace {

// A total order on f32 (the one Rust's total_cmp gives): -NaN, -inf, ...,
// -0, +0, ..., +inf, NaN.
bool f32_before(float a, float b) {
  int32_t ka, kb;
  std::memcpy(&ka, &a, 4);
  std::memcpy(&kb, &b, 4);
  ka ^= int32_t(uint32_t(ka >> 31) >> 1);
  kb ^= int32_t(uint32_t(kb >> 31) >> 1);
  return ka < kb;
}

int64_t turn(Point o, Point a, Point b) {  // > 0: a -> b turns left with y up
  return (int64_t(a.x) - o.x) * (int64_t(b.y) - o.y) - (int64_t(a.y) - o.y) * (int64_t(b.x) - o.x);
}

// ---------------------------------------------------------------- borders

// The eight neighbours, numbered clockwise on the screen (y down) from east.
constexpr int kNx[8] = {1, 1, 0, -1, -1, -1, 0, 1};
constexpr int kNy[8] = {0, 1, 1, 1, 0, -1, -1, -1};
constexpr int kEast = 0, kWest = 4;
int clockwise(int d, int k) { return (d + k) & 7; }
int counterclockwise(int d, int k) { return (d - k) & 7; }

// Suzuki-Abe border following with 8-connected regions over a copy of the
// mask framed by one pixel of paper. A pixel is paper, ink not yet on a
// border, on a border, or on a border whose east neighbour was found to be
// paper while the border was followed (that mark keeps a hole border from
// starting there again).
//
// The mask comes in as row bitmasks (bit x % 64 of word x / 64 of a row is
// pixel x; bits past the width are zero). A border can only start at ink
// with paper to its west (an outer border) or to its east (a hole border),
// and which pixels those are is fixed by the mask, since following a border
// only relabels ink. So the scan visits, in raster order, just the pixels
// where a row's bits change, and asks each the same two questions the full
// raster scan asks of every pixel: the same borders, in the same order.
class BorderTracer {
 public:
  BorderTracer(const uint64_t *bits, size_t words_per_row, size_t width, size_t height)
      : h_(height), pitch_(long(width) + 2), bits_(bits), wpr_(words_per_row),
        label_(size_t(pitch_) * (height + 2), kPaper) {
    // Eight pixels a table lookup: byte b of a word spreads to 8 labels.
    static const std::array<uint64_t, 256> spread = [] {
      std::array<uint64_t, 256> t{};
      for (int v = 0; v < 256; v++)
        for (int k = 0; k < 8; k++)
          if (v >> k & 1) t[size_t(v)] |= uint64_t(kInk) << (8 * k);
      return t;
    }();
    for (size_t y = 0; y < height; y++) {
      uint8_t *row = label_.data() + at(0, long(y));
      for (size_t k = 0; k < wpr_; k++) {
        uint64_t v = bits_[y * wpr_ + k];
        for (size_t b = 0; v; b++, v >>= 8) {
          const size_t x = 64 * k + 8 * b;
          if (!(v & 0xff)) continue;
          const uint64_t lanes = spread[v & 0xff];
          const size_t n = std::min<size_t>(8, width - x);
          std::memcpy(row + x, &lanes, n);
        }
      }
    }
    for (int d = 0; d < 8; d++) step_[d] = kNx[d] + long(kNy[d]) * pitch_;
  }

  // Every border, in cv2.findContours's list order: the reverse of the order
  // in which a raster scan meets them.
  Contours all() {
    Contours found;
    for (long y = 0; y < long(h_); y++) {
      const uint64_t *row = bits_ + size_t(y) * wpr_;
      for (size_t k = 0; k < wpr_; k++) {
        const uint64_t ink = row[k];
        if (!ink) continue;
        // West neighbours' bits (bit 63 of the word before), east ones' (bit
        // 0 of the word after); off the row is paper.
        const uint64_t west = ink << 1 | (k ? row[k - 1] >> 63 : 0);
        const uint64_t east = ink >> 1 | (k + 1 < wpr_ ? row[k + 1] << 63 : 0);
        for (uint64_t edge = ink & ~(west & east); edge; edge &= edge - 1) {
          const long p = at(long(64 * k) + __builtin_ctzll(edge), y);
          const uint8_t v = label_[p];
          if (v == kInk && label_[p - 1] == kPaper)
            found.push_back(follow(p, kWest));  // an outer border, paper to its west
          else if ((v == kInk || v == kTraced) && label_[p + 1] == kPaper)
            found.push_back(follow(p, kEast));  // a hole border, paper to its east
        }
      }
    }
    std::reverse(found.begin(), found.end());
    return found;
  }

 private:
  enum : uint8_t { kPaper = 0, kInk = 1, kTraced = 2, kTracedEastPaper = 3 };

  long at(long x, long y) const { return (y + 1) * pitch_ + x + 1; }
  Point point(long p) const { return Point{int32_t(p % pitch_) - 1, int32_t(p / pitch_) - 1}; }
  bool ink(long p) const { return label_[p] != kPaper; }

  // The border through `start`, whose neighbour in direction `paper` is
  // paper; its corners (CHAIN_APPROX_SIMPLE: the pixels where the step to
  // the next pixel changes direction), in the order the border is followed.
  std::vector<Point> follow(long start, int paper) {
    // The border's last pixel: the first ink clockwise from the paper side.
    int closing = -1;
    for (int k = 0; k < 8 && closing < 0; k++)
      if (ink(start + step_[clockwise(paper, k)])) closing = clockwise(paper, k);
    if (closing < 0) {  // a pixel on its own
      label_[start] = kTracedEastPaper;
      return {point(start)};
    }
    const long last = start + step_[closing];
    std::vector<Point> corners;
    long p = start;
    int came_from = closing;  // direction, seen from p, of the pixel before it
    int first = -1, prev = -1;  // the headings of the first step and of the step before
    for (;;) {
      // Counter-clockwise from the pixel before, the first ink neighbour.
      int go = came_from;
      bool east_paper = false;
      for (int k = 1; k <= 8; k++) {
        const int d = counterclockwise(came_from, k);
        if (ink(p + step_[d])) {
          go = d;
          break;
        }
        east_paper = east_paper || d == kEast;
      }
      if (east_paper)
        label_[p] = kTracedEastPaper;
      else if (label_[p] == kInk)
        label_[p] = kTraced;
      // CHAIN_APPROX_SIMPLE: a corner wherever the heading changes; the
      // first pixel's turn (from the last step) is settled at the end.
      if (first < 0)
        first = go;
      else if (go != prev)
        corners.push_back(point(p));
      prev = go;
      const long next = p + step_[go];
      if (p == last && next == start) break;
      came_from = clockwise(go, 4);
      p = next;
    }
    if (first != prev) corners.insert(corners.begin(), point(start));
    return corners;
  }

  size_t h_;
  long pitch_;
  const uint64_t *bits_;
  size_t wpr_;
  std::vector<uint8_t> label_;
  long step_[8];
};

// ---------------------------------------------------------------- hull

// The indices of the convex hull of integer points in cv2.convexHull's
// order: only the vertices (no point on an edge, each repeated point by its
// first index), counter-clockwise with y pointing up, starting from the
// greatest point by (x, y); and when those indices, read around the hull,
// rise at every step but one (or fall at every step but one), OpenCV
// starts them at their least (or greatest) index.
std::vector<size_t> hull_indices(const std::vector<Point> &p) {
  std::vector<size_t> s(p.size());
  std::iota(s.begin(), s.end(), size_t(0));
  std::stable_sort(s.begin(), s.end(),
                   [&](size_t a, size_t b) { return p[a].x < p[b].x || (p[a].x == p[b].x && p[a].y < p[b].y); });
  s.erase(std::unique(s.begin(), s.end(), [&](size_t a, size_t b) { return p[a] == p[b]; }), s.end());
  if (s.size() < 3) return std::vector<size_t>(s.rbegin(), s.rend());
  // Andrew's monotone chain: the top chain from the greatest point down to
  // the least, then the bottom chain back up, left turns only.
  std::vector<size_t> h;
  auto add = [&](size_t k, size_t keep) {
    while (h.size() > keep && turn(p[h[h.size() - 2]], p[h.back()], p[k]) <= 0) h.pop_back();
    h.push_back(k);
  };
  for (size_t i = s.size(); i-- > 0;) add(s[i], 1);
  const size_t top = h.size();
  for (size_t i = 1; i < s.size(); i++) add(s[i], top);
  h.pop_back();  // the greatest point again
  const size_t n = h.size();
  if (n < 3) return h;
  auto monotone_from = [&](size_t first, bool rising) {
    for (size_t k = 0; k + 1 < n; k++)
      if ((h[(first + k) % n] < h[(first + k + 1) % n]) != rising) return false;
    return true;
  };
  const size_t least = size_t(std::min_element(h.begin(), h.end()) - h.begin());
  const size_t most = size_t(std::max_element(h.begin(), h.end()) - h.begin());
  size_t first = 0;
  if (monotone_from(least, true))
    first = least;
  else if (monotone_from(most, false))
    first = most;
  std::rotate(h.begin(), h.begin() + long(first), h.end());
  return h;
}

// ---------------------------------------------------------------- rectangle

struct V2 {
  float x, y;
};

// v turned a quarter clockwise (with y up) k times.
V2 quarter(V2 v, int k) {
  switch (k & 3) {
    case 0: return v;
    case 1: return {v.y, -v.x};
    case 2: return {-v.x, -v.y};
    default: return {-v.y, v.x};
  }
}

// cv2.minAreaRect's rotating calipers, in f32, around the convex polygon
// `q` (at least three vertices, counter-clockwise with y up). Four calipers
// rest on the lowest, rightmost, highest and leftmost vertices (the first
// of equals); each step the one whose edge turns least rolls to its next
// vertex, and the rectangle of the least area so far (the later of equals)
// is kept as a corner and two side vectors.
struct Calipers {
  V2 corner, side_u, side_v;

  explicit Calipers(const std::vector<V2> &q) {
    const size_t n = q.size();
    std::vector<V2> edge(n);
    std::vector<float> inv_len(n);
    size_t rest[4] = {0, 0, 0, 0};  // lowest, rightmost, highest, leftmost
    for (size_t i = 0; i < n; i++) {
      const V2 a = q[i], b = q[(i + 1) % n];
      if (a.y < q[rest[0]].y) rest[0] = i;
      if (a.x > q[rest[1]].x) rest[1] = i;
      if (a.y > q[rest[2]].y) rest[2] = i;
      if (a.x < q[rest[3]].x) rest[3] = i;
      const double ex = double(b.x - a.x), ey = double(b.y - a.y);
      edge[i] = {float(ex), float(ey)};
      inv_len[i] = float(1.0 / std::sqrt(ex * ex + ey * ey));
    }
    float least = std::numeric_limits<float>::max();
    V2 dir{0.0f, 0.0f};
    float across = 0.0f, along = 0.0f;
    size_t at_left = 0, at_low = 0;
    for (size_t stepi = 0; stepi < n; stepi++) {
      int roll = 0;
      V2 t0 = quarter(edge[rest[0]], 0);
      for (int k = 1; k < 4; k++) {
        const V2 tk = quarter(edge[rest[k]], k);
        if (tk.y * t0.x - tk.x * t0.y < 0.0f) roll = k, t0 = tk;
      }
      const size_t e = rest[roll];
      dir = quarter(V2{edge[e].x * inv_len[e], edge[e].y * inv_len[e]}, roll);
      rest[roll] = (rest[roll] + 1) % n;
      const V2 lo = q[rest[0]], rt = q[rest[1]], hi = q[rest[2]], lf = q[rest[3]];
      const float w = (rt.x - lf.x) * dir.x + (rt.y - lf.y) * dir.y;
      const float h = (hi.y - lo.y) * dir.x - (hi.x - lo.x) * dir.y;
      if (w * h <= least) {
        least = w * h;
        best_dir_ = dir, across = w, along = h, at_left = rest[3], at_low = rest[0];
      }
    }
    // The corner where the side through the leftmost support meets the
    // side through the lowest one.
    const V2 d = best_dir_, n2{-d.y, d.x};
    const float c1 = d.x * q[at_left].x + q[at_left].y * d.y;
    const float c2 = n2.x * q[at_low].x + q[at_low].y * n2.y;
    const float inv = 1.0f / (d.x * n2.y - n2.x * d.y);
    corner = {(c1 * n2.y - c2 * d.y) * inv, (d.x * c2 - n2.x * c1) * inv};
    side_u = {d.x * across, d.y * across};
    side_v = {n2.x * along, n2.y * along};
  }

 private:
  V2 best_dir_{0.0f, 0.0f};
};

float f64_length(double x, double y) { return float(std::sqrt(x * x + y * y)); }

constexpr double kPi = 3.14159265358979323846;

// ---------------------------------------------------------------- offset

// Clipper's rounding of a coordinate: half away from zero.
int32_t clipper_int(double v) { return v < 0.0 ? int32_t(v - 0.5) : int32_t(v + 0.5); }

// What Clipper's union leaves of a convex ring: repeated and collinear
// points removed one at a time (the first found each time), and the ring
// started just after the last point of its first run at the least y.
std::vector<Point> clipper_clean(std::vector<Point> r) {
  for (bool dropped = true; dropped && r.size() >= 3;) {
    dropped = false;
    const size_t n = r.size();
    for (size_t i = 0; i < n; i++) {
      const Point before = r[(i + n - 1) % n], here = r[i], after = r[(i + 1) % n];
      if (here == after || turn(before, here, after) == 0) {
        r.erase(r.begin() + long(i));
        dropped = true;
        break;
      }
    }
  }
  if (r.empty()) return r;
  const int32_t top = std::min_element(r.begin(), r.end(), [](Point a, Point b) { return a.y < b.y; })->y;
  const size_t n = r.size();
  size_t end_of_run = n - 1;
  for (size_t i = 0; i < n; i++)
    if (r[i].y == top && r[(i + 1) % n].y != top) {
      end_of_run = i;
      break;
    }
  std::rotate(r.begin(), r.begin() + long((end_of_run + 1) % n), r.end());
  return r;
}

// pyclipper's ClipperOffset with round joins on a closed polygon: each
// vertex moves out along its edges' normals, and where the outline turns
// outwards an arc of steps around the vertex fills the join.
class RoundOffset {
 public:
  explicit RoundOffset(double delta) : d_(delta) {
    const double tol = std::min(0.25, std::fabs(delta) * 0.25);
    const double steps = std::min(kPi / std::acos(1.0 - tol / std::fabs(delta)), std::fabs(delta) * kPi);
    sin_ = std::sin(2.0 * kPi / steps), cos_ = std::cos(2.0 * kPi / steps);
    steps_per_rad_ = steps / (2.0 * kPi);
  }

  // `ring`: at least three distinct vertices, counter-clockwise with y up.
  std::vector<Point> grow(const std::vector<std::array<double, 2>> &ring) const {
    const size_t n = ring.size();
    std::vector<std::array<double, 2>> normal(n);
    for (size_t i = 0; i < n; i++) {
      const auto &a = ring[i], &b = ring[(i + 1) % n];
      const double dx = b[0] - a[0], dy = b[1] - a[1];
      const double inv = 1.0 / std::sqrt(dx * dx + dy * dy);
      normal[i] = {dy * inv, -dx * inv};
    }
    std::vector<Point> out;
    size_t prev = n - 1;  // the edge arriving at vertex j
    for (size_t j = 0; j < n; j++) {
      const auto &v = ring[j], &in = normal[prev], &on = normal[j];
      double s = in[0] * on[1] - on[0] * in[1];
      const double c = in[0] * on[0] + in[1] * on[1];
      if (std::fabs(s * d_) < 1.0) {
        if (c > 0.0) {  // almost straight on: one point, and the arriving edge stays
          out.push_back(moved(v, in));
          continue;
        }
      } else {
        s = std::max(-1.0, std::min(1.0, s));
      }
      if (s * d_ < 0.0) {  // turning inwards: both offsets and the vertex
        out.push_back(moved(v, in));
        out.push_back(Point{int32_t(v[0]), int32_t(v[1])});
        out.push_back(moved(v, on));
      } else {
        const int32_t arc = std::max<int32_t>(clipper_int(steps_per_rad_ * std::fabs(std::atan2(s, c))), 1);
        std::array<double, 2> r = in;
        for (int32_t k = 0; k < arc; k++) {
          out.push_back(moved(v, r));
          r = {r[0] * cos_ - sin_ * r[1], r[0] * sin_ + r[1] * cos_};
        }
        out.push_back(moved(v, on));
      }
      prev = j;
    }
    return out;
  }

 private:
  Point moved(const std::array<double, 2> &v, const std::array<double, 2> &dir) const {
    return Point{clipper_int(v[0] + dir[0] * d_), clipper_int(v[1] + dir[1] * d_)};
  }

  double d_, sin_, cos_, steps_per_rad_;
};

// ---------------------------------------------------------------- regions

constexpr float kThinnest = 3.0f;  // map pixels: a thinner region is noise

float f32_distance(const std::array<float, 2> &p, const std::array<float, 2> &q) {
  const float dx = p[0] - q[0], dy = p[1] - q[1];
  return std::sqrt(dx * dx + dy * dy);
}

}  // namespace

namespace {

// A few host threads for the regions' candidates. Each candidate depends
// on its own border and the map alone, and the results are gathered in
// region order, so the boxes never depend on how many threads ran them.
// The workers live for the process (the pool is never destroyed, so no
// join runs at exit); a process forked after they started runs the work
// on its calling thread alone.
class Workers {
 public:
  static Workers &get() {
    static Workers *w = new Workers();
    return *w;
  }

  // f(i) for every i below n, on the calling thread and the workers;
  // returns when all are done. One job runs at a time.
  void run(size_t n, const std::function<void(size_t)> &f) {
    if (n < 2 || threads_ == 0 || getpid() != pid_) {
      for (size_t i = 0; i < n; i++) f(i);
      return;
    }
    std::lock_guard<std::mutex> one(job_mu_);
    {
      std::lock_guard<std::mutex> g(mu_);
      job_ = &f, n_ = n, busy_ = threads_;
      next_.store(0);
      gen_++;
    }
    wake_.notify_all();
    drain();
    std::unique_lock<std::mutex> g(mu_);
    idle_.wait(g, [&] { return busy_ == 0; });
    job_ = nullptr;
  }

 private:
  Workers() : pid_(getpid()) {
    const unsigned hw = std::thread::hardware_concurrency();
    threads_ = hw > 2 ? std::min(4u, hw - 1) : 0;
    for (unsigned i = 0; i < threads_; i++) std::thread([this] { loop(); }).detach();
  }

  void drain() {
    for (size_t i = next_.fetch_add(1); i < n_; i = next_.fetch_add(1)) (*job_)(i);
  }

  void loop() {
    uint64_t seen = 0;
    std::unique_lock<std::mutex> g(mu_);
    for (;;) {
      wake_.wait(g, [&] { return gen_ != seen; });
      seen = gen_;
      g.unlock();
      drain();
      g.lock();
      if (--busy_ == 0) idle_.notify_one();
    }
  }

  const pid_t pid_;
  unsigned threads_ = 0;
  std::mutex job_mu_, mu_;
  std::condition_variable wake_, idle_;
  const std::function<void(size_t)> *job_ = nullptr;
  size_t n_ = 0;
  unsigned busy_ = 0;
  uint64_t gen_ = 0;
  std::atomic<size_t> next_{0};
};

}  // namespace

std::vector<uint64_t> pack_rows(const uint8_t *mask, const float *prob, float thresh, size_t width, size_t height) {
  const size_t wpr = (width + 63) / 64;
  std::vector<uint64_t> bits(wpr * height, 0);
  for (size_t y = 0; y < height; y++)
    for (size_t x = 0; x < width; x++) {
      const size_t i = y * width + x;
      if (mask ? mask[i] != 0 : prob[i] > thresh) bits[y * wpr + x / 64] |= uint64_t(1) << (x % 64);
    }
  return bits;
}

Contours find_contours_bits(const uint64_t *bits, size_t words_per_row, size_t width, size_t height) {
  return BorderTracer(bits, words_per_row, width, height).all();
}

Contours find_contours(const uint8_t *mask, size_t width, size_t height) {
  const std::vector<uint64_t> bits = pack_rows(mask, nullptr, 0.0f, width, height);
  return find_contours_bits(bits.data(), (width + 63) / 64, width, height);
}

double contour_mean(const float *map, size_t width, size_t height, const std::vector<Point> &c) {
  if (c.empty() || width == 0 || height == 0) return 0.0;
  int32_t xmin = c[0].x, xmax = c[0].x, ymin = c[0].y, ymax = c[0].y;
  for (const Point &p : c) {
    xmin = std::min(xmin, p.x), xmax = std::max(xmax, p.x);
    ymin = std::min(ymin, p.y), ymax = std::max(ymax, p.y);
  }
  const int32_t W = int32_t(width), H = int32_t(height);
  const int32_t x0 = std::clamp(xmin, 0, W - 1), x1 = std::clamp(xmax, 0, W - 1);
  const int32_t y0 = std::clamp(ymin, 0, H - 1), y1 = std::clamp(ymax, 0, H - 1);
  const size_t bw = size_t(x1 - x0 + 1);
  std::vector<uint8_t> inside(bw * size_t(y1 - y0 + 1), 0);
  auto set = [&](int64_t x, int64_t y) {
    if (x >= x0 && x <= x1 && y >= y0 && y <= y1) inside[size_t(y - y0) * bw + size_t(x - x0)] = 1;
  };
  // The outline: a border's corners are joined by rows, columns or
  // diagonals, drawn pixel by pixel. Edges that are not rows also go into
  // the table the spans are cut from, their upper end first.
  struct Edge {
    int64_t y_top, y_end, x_top, dx, dy;
  };
  std::vector<Edge> edges;
  const size_t n = c.size();
  for (size_t i = 0; i < n; i++) {
    const Point a = c[i], b = c[(i + 1) % n];
    const int64_t dx = int64_t(b.x) - a.x, dy = int64_t(b.y) - a.y;
    const int64_t len = std::max(dx < 0 ? -dx : dx, dy < 0 ? -dy : dy);
    const int64_t sx = (dx > 0) - (dx < 0), sy = (dy > 0) - (dy < 0);
    for (int64_t k = 0; k <= len; k++) set(a.x + sx * k, a.y + sy * k);
    if (dy > 0) edges.push_back({a.y, b.y, a.x, dx, dy});
    else if (dy < 0) edges.push_back({b.y, a.y, b.x, -dx, -dy});
  }
  // cv2.fillPoly's even-odd rule: on each row, the spans between pairs of
  // crossings (an edge crosses rows y_top <= y < y_end).
  std::vector<int64_t> cross;
  for (int64_t y = y0; y <= y1; y++) {
    cross.clear();
    for (const Edge &e : edges)
      if (e.y_top <= y && y < e.y_end) cross.push_back(e.x_top + (y - e.y_top) * e.dx / e.dy);
    std::sort(cross.begin(), cross.end());
    for (size_t k = 0; k + 1 < cross.size(); k += 2)
      for (int64_t x = cross[k]; x <= cross[k + 1]; x++) set(x, y);
  }
  double sum = 0.0;
  size_t count = 0;
  for (int32_t y = y0; y <= y1; y++) {
    const float *row = map + size_t(y) * width;
    const uint8_t *in = inside.data() + size_t(y - y0) * bw;
    for (int32_t x = x0; x <= x1; x++)
      if (in[x - x0]) sum += double(row[x]), count++;
  }
  return count ? sum / double(count) : 0.0;
}

RotatedRect min_area_rect(const std::vector<Point> &points) {
  std::vector<V2> q;
  for (size_t i : hull_indices(points)) q.push_back({float(points[i].x), float(points[i].y)});
  double angle = -kPi / 2;  // a point, or an upright segment
  RotatedRect r{};
  if (q.size() == 1) {
    r.cx = q[0].x, r.cy = q[0].y;
  } else if (q.size() == 2) {
    r.cx = (q[0].x + q[1].x) * 0.5f, r.cy = (q[0].y + q[1].y) * 0.5f;
    const double dx = double(q[0].x - q[1].x), dy = double(q[0].y - q[1].y);
    const float len = f64_length(dx, dy);
    if (dx == 0.0) {
      r.width = len;
    } else if (dy < 0.0) {
      angle = std::atan2(dy, dx);
      r.width = len;
    } else {
      if (dy > 0.0) angle = -std::atan2(dx, dy);
      r.height = len;
    }
  } else if (q.size() >= 3) {
    const Calipers k(q);
    r.cx = k.corner.x + (k.side_u.x + k.side_v.x) * 0.5f;
    r.cy = k.corner.y + (k.side_u.y + k.side_v.y) * 0.5f;
    const float lu = f64_length(double(k.side_u.x), double(k.side_u.y));
    const float lv = f64_length(double(k.side_v.x), double(k.side_v.y));
    if (k.side_u.x == 0.0f && k.side_u.y > 0.0f) {
      r.width = lu, r.height = lv;
    } else {
      angle = -std::atan2(double(k.side_u.x), double(k.side_u.y));
      r.width = lv, r.height = lu;
    }
  }
  r.angle = float(angle * 180.0 / kPi);
  return r;
}

Quad box_points(const RotatedRect &r) {
  // cv2.boxPoints: half the angle's sine and cosine in f32.
  const double rad = double(r.angle) * kPi / 180.0;
  const float hs = float(std::sin(rad)) * 0.5f, hc = float(std::cos(rad)) * 0.5f;
  const float x = r.cx, y = r.cy, w = r.width, h = r.height;
  return Quad{{{x - hs * h - hc * w, y + hc * h - hs * w},
               {x + hs * h - hc * w, y - hc * h - hs * w},
               {x + hs * h + hc * w, y - hc * h + hs * w},
               {x - hs * h + hc * w, y + hc * h + hs * w}}};
}

std::pair<Quad, float> mini_box(const std::vector<Point> &points) {
  const RotatedRect r = min_area_rect(points);
  Quad c = box_points(r);
  // RapidOCR's get_mini_boxes: corners by x (stable), then each side's two
  // by y: top-left, top-right, bottom-right, bottom-left.
  std::stable_sort(c.begin(), c.end(), [](const auto &a, const auto &b) { return f32_before(a[0], b[0]); });
  const bool left_swapped = !(c[1][1] > c[0][1]), right_swapped = !(c[3][1] > c[2][1]);
  const auto &top_left = left_swapped ? c[1] : c[0], &bottom_left = left_swapped ? c[0] : c[1];
  const auto &top_right = right_swapped ? c[3] : c[2], &bottom_right = right_swapped ? c[2] : c[3];
  return {Quad{top_left, top_right, bottom_right, bottom_left}, std::min(r.width, r.height)};
}

std::vector<Point> unclip(const Quad &quad, double ratio) {
  // shapely: the area (shoelace, x taken relative to the first corner) and
  // the perimeter of the f32 quad, in f64.
  double x[4], y[4];
  for (int i = 0; i < 4; i++) x[i] = double(quad[i][0]), y[i] = double(quad[i][1]);
  double twice = 0.0, perimeter = 0.0;
  for (int i = 1; i < 4; i++) twice += (x[i] - x[0]) * (y[i - 1] - y[(i + 1) % 4]);
  for (int i = 0; i < 4; i++) {
    const double dx = x[(i + 1) % 4] - x[i], dy = y[(i + 1) % 4] - y[i];
    perimeter += std::sqrt(dx * dx + dy * dy);
  }
  const double delta = std::fabs(twice / 2.0) * ratio / perimeter;
  // pyclipper takes integer corners (truncated), drops repeats and closes
  // the ring.
  std::vector<std::array<double, 2>> ring;
  for (int i = 0; i < 4; i++) {
    const std::array<double, 2> v = {std::trunc(double(quad[i][0])), std::trunc(double(quad[i][1]))};
    if (ring.empty() || ring.back() != v) ring.push_back(v);
  }
  while (ring.size() > 1 && ring.front() == ring.back()) ring.pop_back();
  if (ring.size() < 3) return {};
  if (std::fabs(delta) < 1e-20) {
    std::vector<Point> same;
    for (const auto &v : ring) same.push_back(Point{int32_t(v[0]), int32_t(v[1])});
    return clipper_clean(same);
  }
  double signed_twice = 0.0;
  for (size_t i = 0; i < ring.size(); i++) {
    const auto &a = ring[i], &b = ring[(i + 1) % ring.size()];
    signed_twice += a[0] * b[1] - b[0] * a[1];
  }
  if (signed_twice < 0.0) std::reverse(ring.begin(), ring.end());
  return clipper_clean(RoundOffset(delta).grow(ring));
}

Candidate contour_candidate(const float *prob, size_t map_w, size_t map_h, const std::vector<Point> &contour,
                            size_t dest_w, size_t dest_h, const DbOptions &o) {
  Candidate out{};
  const auto box = mini_box(contour);
  if (box.second < kThinnest) return out.kind = Candidate::kSmall, out;
  out.score = contour_mean(prob, map_w, map_h, contour);
  if (o.box_thresh > out.score) return out.kind = Candidate::kLowScore, out;
  const auto grown = mini_box(unclip(box.first, o.unclip_ratio));
  if (grown.second < kThinnest + 2.0f) return out.kind = Candidate::kSmallAfterUnclip, out;
  // To page pixels as numpy does on the f32 box: v / map * dest in f32,
  // rounded half to even, clipped to [0, dest].
  auto to_page = [](float v, size_t map, size_t dest) {
    const float d = float(dest);
    return int32_t(std::clamp(std::nearbyint(v / float(map) * d), 0.0f, d));
  };
  for (int i = 0; i < 4; i++)
    out.corners[i] = Point{to_page(grown.first[i][0], map_w, dest_w), to_page(grown.first[i][1], map_h, dest_h)};
  out.kind = Candidate::kKept;
  return out;
}

bool order_and_clip(const Point corners[4], size_t width, size_t height, Quad &out) {
  // RapidOCR's order_points_clockwise: the two leftmost corners (a stable
  // sort by x) top then bottom, the two rightmost likewise; clipped to the
  // page; kept when both sides from the top-left corner are over 3 pixels
  // (f32 lengths truncated).
  Point c[4] = {corners[0], corners[1], corners[2], corners[3]};
  std::stable_sort(c, c + 4, [](Point a, Point b) { return a.x < b.x; });
  const Point tl = c[1].y < c[0].y ? c[1] : c[0], bl = c[1].y < c[0].y ? c[0] : c[1];
  const Point tr = c[3].y < c[2].y ? c[3] : c[2], br = c[3].y < c[2].y ? c[2] : c[3];
  auto fit = [&](Point p) {
    return std::array<float, 2>{float(std::clamp<int32_t>(p.x, 0, int32_t(width) - 1)),
                                float(std::clamp<int32_t>(p.y, 0, int32_t(height) - 1))};
  };
  out = Quad{fit(tl), fit(tr), fit(br), fit(bl)};
  return int32_t(f32_distance(out[0], out[1])) > 3 && int32_t(f32_distance(out[0], out[3])) > 3;
}

void sort_boxes(std::vector<Quad> &boxes) {
  // Reading order: by the top-left corner's y; a new line wherever that y
  // grows by 10 or more from the box before; left to right on a line (both
  // sorts stable, f32 compared in total order).
  std::stable_sort(boxes.begin(), boxes.end(), [](const Quad &a, const Quad &b) { return f32_before(a[0][1], b[0][1]); });
  auto by_x = [](const Quad &a, const Quad &b) { return f32_before(a[0][0], b[0][0]); };
  size_t line_start = 0;
  for (size_t i = 1; i <= boxes.size(); i++)
    if (i == boxes.size() || boxes[i][0][1] - boxes[i - 1][0][1] >= 10.0f) {
      std::stable_sort(boxes.begin() + long(line_start), boxes.begin() + long(i), by_x);
      line_start = i;
    }
}

std::vector<Quad> boxes_from_prob(const float *prob, const uint8_t *mask, size_t map_w, size_t map_h,
                                  size_t dest_w, size_t dest_h, const DbOptions &o) {
  const std::vector<uint64_t> bits = pack_rows(mask, prob, o.thresh, map_w, map_h);
  return boxes_from_bits(prob, bits.data(), (map_w + 63) / 64, map_w, map_h, dest_w, dest_h, o);
}

std::vector<Quad> boxes_from_bits(const float *prob, const uint64_t *bits, size_t words_per_row, size_t map_w,
                                  size_t map_h, size_t dest_w, size_t dest_h, const DbOptions &o) {
  const Contours regions = find_contours_bits(bits, words_per_row, map_w, map_h);
  const size_t n = std::min(regions.size(), o.max_candidates);
  std::vector<Candidate> found(n);
  Workers::get().run(n, [&](size_t i) {
    found[i] = contour_candidate(prob, map_w, map_h, regions[i], dest_w, dest_h, o);
  });
  std::vector<Quad> boxes;
  for (const Candidate &c : found) {
    Quad q;
    if (c.kind == Candidate::kKept && order_and_clip(c.corners, dest_w, dest_h, q)) boxes.push_back(q);
  }
  sort_boxes(boxes);
  return boxes;
}

}  // namespace ppocr
