// The host stages on either side of the GPU model: reading text out of the
// recogniser's per-step (class, probability) output, and turning the
// detector's probability map into text boxes. Both are short, branchy and
// sequential per line or per region, so they run on the CPU; the map's
// threshold has a GPU kernel too (db_mask in layers.hip) for callers that
// download a bit mask instead of the map.
//
// Each stage reproduces, to the last bit, what the libraries RapidOCR builds
// on compute (the reference documents the exact arithmetic):
//  - CTC decode and its score: src/rec.rs:112-161 (numpy's pairwise f64 sum,
//    Python's round to five decimals);
//  - the class list: src/rec.rs:45-104 (str.splitlines);
//  - borders of a mask: src/contour.rs:1-140 (Suzuki-Abe border following,
//    cv2.findContours RETR_LIST / CHAIN_APPROX_SIMPLE);
//  - mean inside a border: src/contour.rs:142-199 (cv2.fillPoly even-odd);
//  - minimum-area rectangle: src/geometry.rs:1-280 (cv2.convexHull's order,
//    cv2.minAreaRect's f32 rotating calipers, cv2.boxPoints);
//  - growth of a box: src/geometry.rs:282-435 (pyclipper's round offset);
//  - the DB postprocess: src/det.rs:291-477.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "post.hpp"

namespace ppocr {

// f32 ordering that is total: -NaN < -inf < ... < -0 < +0 < ... < inf < NaN
// (the sort key the reference's ordering uses).
static bool total_less(float a, float b) {
  int32_t ia, ib;
  std::memcpy(&ia, &a, 4), std::memcpy(&ib, &b, 4);
  ia ^= (int32_t)((uint32_t)(ia >> 31) >> 1);
  ib ^= (int32_t)((uint32_t)(ib >> 31) >> 1);
  return ia < ib;
}

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

// ------------------------------------------------------------ contours

namespace {

// Neighbour k of a pixel, counter-clockwise on screen (y down) from east.
constexpr int kDx[8] = {1, 1, 0, -1, -1, -1, 0, 1};
constexpr int kDy[8] = {0, -1, -1, -1, 0, 1, 1, 1};
constexpr int kEast = 0, kWest = 4;

// Scan states; nonzero is foreground.
constexpr uint8_t kBack = 0, kFresh = 1, kOnBorder = 2, kOnBorderEastOpen = 3;

}  // namespace

Contours find_contours(const uint8_t *mask, size_t width, size_t height) {
  Contours out;
  const long W = (long)width + 2;
  // A frame of background pixels around the mask: no neighbour leaves it.
  std::vector<uint8_t> st((size_t)W * (height + 2), kBack);
  for (size_t y = 0; y < height; y++)
    for (size_t x = 0; x < width; x++) st[(y + 1) * W + x + 1] = mask[y * width + x] ? kFresh : kBack;
  long off[8];
  for (int k = 0; k < 8; k++) off[k] = kDx[k] + kDy[k] * W;
  auto pt = [&](long at) { return Point{int32_t(at % W) - 1, int32_t(at / W) - 1}; };

  std::vector<std::pair<long, int>> walk;  // pixel, direction of the step leaving it
  for (long y = 1; y <= (long)height; y++) {
    for (long x = 1; x <= (long)width; x++) {
      const long start = y * W + x;
      const uint8_t v = st[start];
      int from;
      if (v == kFresh && st[start - 1] == kBack)
        from = kWest;  // an outer border, entered from its left
      else if ((v == kFresh || v == kOnBorder) && st[start + 1] == kBack)
        from = kEast;  // a hole border, entered from its right
      else
        continue;
      // The border's last pixel: first foreground neighbour clockwise from
      // the background one that revealed it.
      int last_dir = -1;
      for (int k = 0; k < 8; k++) {
        const int d = (from + 8 - k) % 8;
        if (st[start + off[d]] != kBack) {
          last_dir = d;
          break;
        }
      }
      if (last_dir < 0) {  // a lone pixel
        st[start] = kOnBorderEastOpen;
        out.push_back({pt(start)});
        continue;
      }
      const long last = start + off[last_dir];
      walk.clear();
      long cur = start;
      int back = last_dir;
      for (;;) {
        bool east_open = false;
        int next_dir = back;
        for (int k = 1; k <= 8; k++) {
          const int d = (back + k) % 8;
          if (st[cur + off[d]] != kBack) {
            next_dir = d;
            break;
          }
          if (d == kEast) east_open = true;
        }
        if (east_open)
          st[cur] = kOnBorderEastOpen;
        else if (st[cur] == kFresh)
          st[cur] = kOnBorder;
        walk.push_back({cur, next_dir});
        const long next = cur + off[next_dir];
        if (next == start && cur == last) break;
        back = (next_dir + 4) % 8;
        cur = next;
      }
      // Corners: pixels where the step direction changes, from the first.
      const size_t n = walk.size();
      auto turn = [&](size_t i) { return walk[i].second != walk[(i + n - 1) % n].second; };
      size_t first = 0;
      while (first < n && !turn(first)) first++;
      if (first == n) first = 0;
      std::vector<Point> corners;
      for (size_t k = 0; k < n; k++) {
        const size_t i = (first + k) % n;
        if (turn(i)) corners.push_back(pt(walk[i].first));
      }
      out.push_back(std::move(corners));
    }
  }
  std::reverse(out.begin(), out.end());
  return out;
}

double contour_mean(const float *map, size_t width, size_t height, const std::vector<Point> &c) {
  if (c.empty() || width == 0 || height == 0) return 0.0;
  auto cx = [&](int32_t v) { return std::min<int32_t>(std::max<int32_t>(v, 0), int32_t(width) - 1); };
  auto cy = [&](int32_t v) { return std::min<int32_t>(std::max<int32_t>(v, 0), int32_t(height) - 1); };
  int32_t xmin = c[0].x, xmax = c[0].x, ymin = c[0].y, ymax = c[0].y;
  for (const Point &p : c) {
    xmin = std::min(xmin, p.x), xmax = std::max(xmax, p.x);
    ymin = std::min(ymin, p.y), ymax = std::max(ymax, p.y);
  }
  const int32_t x0 = cx(xmin), x1 = cx(xmax), y0 = cy(ymin), y1 = cy(ymax);
  const size_t w = size_t(x1 - x0 + 1), h = size_t(y1 - y0 + 1);
  std::vector<uint8_t> in(w * h, 0);
  auto mark = [&](int32_t x, int32_t y) {
    if (x >= x0 && x <= x1 && y >= y0 && y <= y1) in[size_t(y - y0) * w + size_t(x - x0)] = 1;
  };
  const size_t n = c.size();
  // The border itself (its edges run along rows, columns or diagonals).
  for (size_t i = 0; i < n; i++) {
    const Point a = c[i], b = c[(i + 1) % n];
    const int32_t dx = b.x - a.x, dy = b.y - a.y;
    const int32_t sx = (dx > 0) - (dx < 0), sy = (dy > 0) - (dy < 0);
    const int32_t steps = std::max(std::abs(dx), std::abs(dy));
    for (int32_t k = 0; k <= steps; k++) mark(a.x + sx * k, a.y + sy * k);
  }
  // Between crossings of each row, by the even-odd rule.
  std::vector<int32_t> xs;
  for (int32_t y = y0; y <= y1; y++) {
    xs.clear();
    for (size_t i = 0; i < n; i++) {
      Point lo = c[i], hi = c[(i + 1) % n];
      if (!(lo.y < hi.y)) std::swap(lo, hi);
      if (lo.y <= y && y < hi.y) xs.push_back(lo.x + (y - lo.y) * (hi.x - lo.x) / (hi.y - lo.y));
    }
    std::sort(xs.begin(), xs.end());
    for (size_t k = 0; k + 1 < xs.size(); k += 2)
      for (int32_t x = xs[k]; x <= xs[k + 1]; x++) mark(x, y);
  }
  double sum = 0.0;
  size_t count = 0;
  for (size_t r = 0; r < h; r++) {
    const float *row = map + (size_t(y0) + r) * width + size_t(x0);
    for (size_t k = 0; k < w; k++)
      if (in[r * w + k]) sum += (double)row[k], count++;
  }
  return count ? sum / (double)count : 0.0;
}

// ------------------------------------------------------------ rectangles

static int64_t cross(Point o, Point a, Point b) {
  const int64_t ux = int64_t(a.x) - o.x, uy = int64_t(a.y) - o.y;
  const int64_t vx = int64_t(b.x) - o.x, vy = int64_t(b.y) - o.y;
  return ux * vy - uy * vx;
}

// cv2.convexHull's indices in its order: Andrew's monotone chain
// counter-clockwise (y up) from the largest point by (x, y), collinear points
// dropped, the first of repeated points kept; then OpenCV's rotation that
// makes the indices one ascending or descending run when they can be.
static std::vector<size_t> hull_order(const std::vector<Point> &p) {
  std::vector<size_t> ord(p.size());
  for (size_t i = 0; i < p.size(); i++) ord[i] = i;
  auto less = [&](size_t a, size_t b) { return p[a].x != p[b].x ? p[a].x < p[b].x : p[a].y < p[b].y; };
  std::stable_sort(ord.begin(), ord.end(), less);
  ord.erase(std::unique(ord.begin(), ord.end(), [&](size_t a, size_t b) { return p[a] == p[b]; }), ord.end());
  if (ord.size() < 3) {
    std::reverse(ord.begin(), ord.end());
    return ord;
  }
  auto side = [&](auto first, auto last) {
    std::vector<size_t> h;
    for (auto it = first; it != last; ++it) {
      while (h.size() >= 2 && cross(p[h[h.size() - 2]], p[h.back()], p[*it]) <= 0) h.pop_back();
      h.push_back(*it);
    }
    h.pop_back();
    return h;
  };
  std::vector<size_t> lower = side(ord.begin(), ord.end());
  std::vector<size_t> hull = side(ord.rbegin(), ord.rend());
  hull.insert(hull.end(), lower.begin(), lower.end());
  const size_t n = hull.size();
  if (n < 3) return hull;
  size_t lo = 0, hi = 0, ascents = 0;
  for (size_t i = 1; i < n; i++) {
    ascents += hull[i - 1] < hull[i];
    if (ascents > 1 && ascents + 1 < i) break;
    if (hull[i] < hull[lo]) lo = i;
    if (hull[i] > hull[hi]) hi = i;
  }
  const size_t gap = lo > hi ? lo - hi : hi - lo;
  if ((gap == 1 || gap == n - 1) && (ascents <= 1 || ascents + 2 >= n)) {
    const bool up = (hi + 1) % n == lo;
    const size_t first = up ? lo : hi;
    std::vector<size_t> rot(n);
    for (size_t k = 0; k < n; k++) rot[k] = hull[(first + k) % n];
    bool run = true;
    for (size_t k = 0; k + 1 < n && run; k++) run = (rot[k] < rot[k + 1]) == up;
    if (first > 0 && run) return rot;
  }
  return hull;
}

struct Calipers {
  float corner[2], u[2], v[2];
};

// cv2.minAreaRect's rotating calipers in f32 over the hull in its order.
static Calipers calipers(const std::vector<std::array<float, 2>> &p) {
  const size_t n = p.size();
  std::vector<std::array<float, 2>> edge(n);
  std::vector<float> inv(n);
  size_t left = 0, bottom = 0, right = 0, top = 0;
  for (size_t i = 0; i < n; i++) {
    const auto &q = p[i], &r = p[(i + 1) % n];
    if (q[0] < p[left][0]) left = i;
    if (q[0] > p[right][0]) right = i;
    if (q[1] > p[top][1]) top = i;
    if (q[1] < p[bottom][1]) bottom = i;
    const double dx = double(r[0] - q[0]), dy = double(r[1] - q[1]);
    edge[i] = {float(dx), float(dy)};
    inv[i] = float(1.0 / std::sqrt(dx * dx + dy * dy));
  }
  size_t seq[4] = {bottom, right, top, left};
  float min_area = std::numeric_limits<float>::max();
  size_t best_l = 0, best_b = 0;
  float ba = 0, bw = 0, bb = 0, bh = 0;
  for (size_t it = 0; it < n; it++) {
    float t[4][2];
    {
      const auto &e0 = edge[seq[0]], &e1 = edge[seq[1]], &e2 = edge[seq[2]], &e3 = edge[seq[3]];
      t[0][0] = e0[0], t[0][1] = e0[1];
      t[1][0] = e1[1], t[1][1] = -e1[0];
      t[2][0] = -e2[0], t[2][1] = -e2[1];
      t[3][0] = -e3[1], t[3][1] = e3[0];
    }
    int main = 0;
    for (int i = 1; i < 4; i++)
      if (t[i][1] * t[main][0] + -t[i][0] * t[main][1] < 0.0f) main = i;
    const size_t k = seq[main];
    const float lx = edge[k][0] * inv[k], ly = edge[k][1] * inv[k];
    float a, b;
    switch (main) {
      case 0: a = lx, b = ly; break;
      case 1: a = ly, b = -lx; break;
      case 2: a = -lx, b = -ly; break;
      default: a = -ly, b = lx; break;
    }
    seq[main] = (seq[main] + 1) % n;
    const float width = (p[seq[1]][0] - p[seq[3]][0]) * a + (p[seq[1]][1] - p[seq[3]][1]) * b;
    const float height = -(p[seq[2]][0] - p[seq[0]][0]) * b + (p[seq[2]][1] - p[seq[0]][1]) * a;
    const float area = width * height;
    if (area <= min_area) {
      min_area = area;
      best_l = seq[3], ba = a, bw = width, bb = b, bh = height, best_b = seq[0];
    }
  }
  const float a1 = ba, b1 = bb, a2 = -bb, b2 = ba;
  const float c1 = a1 * p[best_l][0] + p[best_l][1] * b1;
  const float c2 = a2 * p[best_b][0] + p[best_b][1] * b2;
  const float idet = 1.0f / (a1 * b2 - a2 * b1);
  Calipers r;
  r.corner[0] = (c1 * b2 - c2 * b1) * idet;
  r.corner[1] = (a1 * c2 - a2 * c1) * idet;
  r.u[0] = a1 * bw, r.u[1] = b1 * bw;
  r.v[0] = a2 * bh, r.v[1] = b2 * bh;
  return r;
}

RotatedRect min_area_rect(const std::vector<Point> &points) {
  const std::vector<size_t> order = hull_order(points);
  std::vector<std::array<float, 2>> hull;
  for (size_t i : order) hull.push_back({float(points[i].x), float(points[i].y)});
  auto length = [](double dx, double dy) { return float(std::sqrt(dx * dx + dy * dy)); };
  const double kPi = 3.14159265358979323846;
  double angle = -kPi / 2;  // upright, a vertical segment and a point keep -90
  RotatedRect r{};
  if (hull.size() == 1) {
    r.cx = hull[0][0], r.cy = hull[0][1];
  } else if (hull.size() == 2) {
    const auto &p = hull[0], &q = hull[1];
    r.cx = (p[0] + q[0]) * 0.5f, r.cy = (p[1] + q[1]) * 0.5f;
    const double dx = double(p[0] - q[0]), dy = double(p[1] - q[1]);
    const float size = length(dx, dy);
    if (dx == 0.0) {
      r.width = size;
    } else if (dy < 0.0) {
      angle = std::atan2(dy, dx);
      r.width = size;
    } else {
      if (dy > 0.0) angle = -std::atan2(dx, dy);
      r.height = size;
    }
  } else if (hull.size() >= 3) {
    const Calipers c = calipers(hull);
    r.cx = c.corner[0] + (c.u[0] + c.v[0]) * 0.5f;
    r.cy = c.corner[1] + (c.u[1] + c.v[1]) * 0.5f;
    const float ul = length(double(c.u[0]), double(c.u[1])), vl = length(double(c.v[0]), double(c.v[1]));
    if (c.u[0] == 0.0f && c.u[1] > 0.0f) {
      r.width = ul, r.height = vl;
    } else {
      angle = -std::atan2(double(c.u[0]), double(c.u[1]));
      r.width = vl, r.height = ul;
    }
  }
  r.angle = float(angle * 180.0 / kPi);
  return r;
}

Quad box_points(const RotatedRect &r) {
  const double kPi = 3.14159265358979323846;
  const double rad = double(r.angle) * kPi / 180.0;
  const float a = float(std::sin(rad)) * 0.5f, b = float(std::cos(rad)) * 0.5f;
  const float cx = r.cx, cy = r.cy, w = r.width, h = r.height;
  Quad q;
  q[0] = {cx - a * h - b * w, cy + b * h - a * w};
  q[1] = {cx + a * h - b * w, cy - b * h - a * w};
  q[2] = {cx + a * h + b * w, cy - b * h + a * w};
  q[3] = {cx - a * h + b * w, cy + b * h + a * w};
  return q;
}

std::pair<Quad, float> mini_box(const std::vector<Point> &points) {
  const RotatedRect r = min_area_rect(points);
  Quad p = box_points(r);
  std::stable_sort(p.begin(), p.end(), [](const std::array<float, 2> &a, const std::array<float, 2> &b) {
    return total_less(a[0], b[0]);
  });
  std::array<float, 2> tl, bl, tr, br;
  if (p[1][1] > p[0][1]) tl = p[0], bl = p[1];
  else tl = p[1], bl = p[0];
  if (p[3][1] > p[2][1]) tr = p[2], br = p[3];
  else tr = p[3], br = p[2];
  return {Quad{tl, tr, br, bl}, std::min(r.width, r.height)};
}

// ------------------------------------------------------------ unclip

// Clipper's integer rounding: half away from zero by adding a half and
// truncating.
static int32_t clipper_round(double v) { return v < 0.0 ? int32_t(v - 0.5) : int32_t(v + 0.5); }

// Clipper's union of a convex ring with itself: repeated and collinear
// points dropped, the ring starting after the last point of its topmost run.
static std::vector<Point> clipper_tidy(std::vector<Point> ring) {
  while (ring.size() >= 3) {
    const size_t n = ring.size();
    size_t drop = n;
    for (size_t i = 0; i < n && drop == n; i++) {
      const Point prev = ring[(i + n - 1) % n], here = ring[i], next = ring[(i + 1) % n];
      if (here == next || cross(prev, here, next) == 0) drop = i;
    }
    if (drop == n) break;
    ring.erase(ring.begin() + drop);
  }
  const size_t n = ring.size();
  if (n == 0) return ring;
  int32_t top = ring[0].y;
  for (const Point &p : ring) top = std::min(top, p.y);
  size_t last = n - 1;
  for (size_t i = 0; i < n; i++)
    if (ring[i].y == top && ring[(i + 1) % n].y != top) {
      last = i;
      break;
    }
  std::rotate(ring.begin(), ring.begin() + (last + 1) % n, ring.end());
  return ring;
}

std::vector<Point> unclip(const Quad &quad, double ratio) {
  const double kPi = 3.14159265358979323846, kTau = 2.0 * kPi;
  // Shapely's area (shoelace relative to the first x) and perimeter.
  double p[4][2];
  for (int i = 0; i < 4; i++) p[i][0] = double(quad[i][0]), p[i][1] = double(quad[i][1]);
  double sum = 0.0;
  for (int i = 1; i < 4; i++) sum += (p[i][0] - p[0][0]) * (p[i - 1][1] - p[(i + 1) % 4][1]);
  double perim = 0.0;
  for (int i = 0; i < 4; i++) {
    const double dx = p[(i + 1) % 4][0] - p[i][0], dy = p[(i + 1) % 4][1] - p[i][1];
    perim += std::sqrt(dx * dx + dy * dy);
  }
  const double delta = std::fabs(sum / 2.0) * ratio / perim;
  // pyclipper truncates the corners to integers first.
  std::vector<std::array<double, 2>> ring;
  for (int i = 0; i < 4; i++) {
    const std::array<double, 2> q = {double(std::trunc(quad[i][0])), double(std::trunc(quad[i][1]))};
    if (ring.empty() || ring.back() != q) ring.push_back(q);
  }
  while (ring.size() > 1 && ring.front() == ring.back()) ring.pop_back();
  if (ring.size() < 3) return {};
  if (std::fabs(delta) < 1e-20) {
    std::vector<Point> r;
    for (auto &q : ring) r.push_back({int32_t(q[0]), int32_t(q[1])});
    return clipper_tidy(r);
  }
  double area2 = 0.0;
  for (size_t i = 0; i < ring.size(); i++) {
    const auto &a = ring[i], &b = ring[(i + 1) % ring.size()];
    area2 += a[0] * b[1] - b[0] * a[1];
  }
  if (area2 < 0.0) std::reverse(ring.begin(), ring.end());

  const double tol = std::min(0.25, std::fabs(delta) * 0.25);
  const double steps = std::min(kPi / std::acos(1.0 - tol / std::fabs(delta)), std::fabs(delta) * kPi);
  const double ssin = std::sin(kTau / steps), scos = std::cos(kTau / steps);
  const double per_rad = steps / kTau;
  const size_t n = ring.size();
  std::vector<std::array<double, 2>> nrm(n);
  for (size_t i = 0; i < n; i++) {
    const auto &a = ring[i], &b = ring[(i + 1) % n];
    const double dx = b[0] - a[0], dy = b[1] - a[1];
    const double inv = 1.0 / std::sqrt(dx * dx + dy * dy);
    nrm[i] = {dy * inv, -dx * inv};
  }
  auto at = [&](const std::array<double, 2> &q, const std::array<double, 2> &v) {
    return Point{clipper_round(q[0] + v[0] * delta), clipper_round(q[1] + v[1] * delta)};
  };
  std::vector<Point> out;
  size_t k = n - 1;
  for (size_t j = 0; j < n; j++) {
    const auto &q = ring[j], &nk = nrm[k], &nj = nrm[j];
    double sin_a = nk[0] * nj[1] - nj[0] * nk[1];
    const double cos_a = nk[0] * nj[0] + nk[1] * nj[1];
    if (std::fabs(sin_a * delta) < 1.0) {
      if (cos_a > 0.0) {  // nearly straight: one point, k stays
        out.push_back(at(q, nk));
        continue;
      }
    } else {
      sin_a = std::min(1.0, std::max(-1.0, sin_a));
    }
    if (sin_a * delta < 0.0) {
      out.push_back(at(q, nk));
      out.push_back({int32_t(q[0]), int32_t(q[1])});
      out.push_back(at(q, nj));
    } else {
      const int32_t turns = std::max<int32_t>(clipper_round(per_rad * std::fabs(std::atan2(sin_a, cos_a))), 1);
      std::array<double, 2> v = nk;
      for (int32_t s = 0; s < turns; s++) {
        out.push_back(at(q, v));
        v = {v[0] * scos - ssin * v[1], v[0] * ssin + v[1] * scos};
      }
      out.push_back(at(q, nj));
    }
    k = j;
  }
  return clipper_tidy(out);
}

// ------------------------------------------------------------ DB boxes

static constexpr float kMinSide = 3.0f;

Candidate contour_candidate(const float *prob, size_t map_w, size_t map_h, const std::vector<Point> &contour,
                            size_t dest_w, size_t dest_h, const DbOptions &o) {
  Candidate c{};
  const auto box = mini_box(contour);
  if (box.second < kMinSide) return c.kind = Candidate::kSmall, c;
  c.score = contour_mean(prob, map_w, map_h, contour);
  if (o.box_thresh > c.score) return c.kind = Candidate::kLowScore, c;
  const auto grown = mini_box(unclip(box.first, o.unclip_ratio));
  if (grown.second < kMinSide + 2.0f) return c.kind = Candidate::kSmallAfterUnclip, c;
  // numpy divides and multiplies the f32 box by the sizes in f32.
  auto scale = [](float v, size_t map, size_t dest) {
    const float d = float(dest);
    return int32_t(std::min(std::max(std::nearbyint(v / float(map) * d), 0.0f), d));
  };
  for (int i = 0; i < 4; i++)
    c.corners[i] = {scale(grown.first[i][0], map_w, dest_w), scale(grown.first[i][1], map_h, dest_h)};
  c.kind = Candidate::kKept;
  return c;
}

static float distance(const std::array<float, 2> &p, const std::array<float, 2> &q) {
  const float dx = p[0] - q[0], dy = p[1] - q[1];
  return std::sqrt(dx * dx + dy * dy);
}

bool order_and_clip(const Point corners[4], size_t width, size_t height, Quad &out) {
  Point s[4] = {corners[0], corners[1], corners[2], corners[3]};
  std::stable_sort(s, s + 4, [](const Point &a, const Point &b) { return a.x < b.x; });
  if (s[1].y < s[0].y) std::swap(s[0], s[1]);
  if (s[3].y < s[2].y) std::swap(s[2], s[3]);
  auto clip = [&](Point p) {
    return std::array<float, 2>{float(std::min<int32_t>(std::max<int32_t>(p.x, 0), int32_t(width) - 1)),
                                float(std::min<int32_t>(std::max<int32_t>(p.y, 0), int32_t(height) - 1))};
  };
  out = Quad{clip(s[0]), clip(s[2]), clip(s[3]), clip(s[1])};
  return int32_t(distance(out[0], out[1])) > 3 && int32_t(distance(out[0], out[3])) > 3;
}

void sort_boxes(std::vector<Quad> &boxes) {
  std::stable_sort(boxes.begin(), boxes.end(), [](const Quad &a, const Quad &b) { return total_less(a[0][1], b[0][1]); });
  struct Keyed {
    uint32_t line;
    float x;
    Quad q;
  };
  std::vector<Keyed> keyed;
  uint32_t line = 0;
  for (size_t i = 0; i < boxes.size(); i++) {
    if (i > 0 && boxes[i][0][1] - boxes[i - 1][0][1] >= 10.0f) line++;
    keyed.push_back({line, boxes[i][0][0], boxes[i]});
  }
  std::stable_sort(keyed.begin(), keyed.end(), [](const Keyed &a, const Keyed &b) {
    return a.line != b.line ? a.line < b.line : total_less(a.x, b.x);
  });
  for (size_t i = 0; i < boxes.size(); i++) boxes[i] = keyed[i].q;
}

std::vector<Quad> boxes_from_prob(const float *prob, const uint8_t *mask, size_t map_w, size_t map_h,
                                  size_t dest_w, size_t dest_h, const DbOptions &o) {
  std::vector<uint8_t> own;
  if (!mask) {
    own.resize(map_w * map_h);
    for (size_t i = 0; i < own.size(); i++) own[i] = prob[i] > o.thresh;
    mask = own.data();
  }
  const Contours contours = find_contours(mask, map_w, map_h);
  std::vector<Quad> boxes;
  const size_t m = std::min(contours.size(), o.max_candidates);
  for (size_t i = 0; i < m; i++) {
    const Candidate c = contour_candidate(prob, map_w, map_h, contours[i], dest_w, dest_h, o);
    Quad q;
    if (c.kind == Candidate::kKept && order_and_clip(c.corners, dest_w, dest_h, q)) boxes.push_back(q);
  }
  sort_boxes(boxes);
  return boxes;
}

}  // namespace ppocr

// ------------------------------------------------------------ C ABI

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

}  // extern "C"
