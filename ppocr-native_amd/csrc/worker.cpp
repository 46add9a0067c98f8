// ppocr_hip_worker: the worker's GPU call patterns over the C ABI alone
// (include/ppocr_hip.h), the way a host program binds the library.
//
// It follows src/bin/ppocr-native/ocr.rs:
//  - `Reader::new` with `gpu` (ocr.rs:131-187): both plans load on the GPU
//    or neither does, the same "no GPU (...)" message on failure, "running on
//    <device>" on success;
//  - `Detector::run` (ocr.rs:60-91): per page, set_input_size, the input,
//    run, output 0; a refused page is reported once with the same message;
//  - `recognise_all` / `read_on_gpu` (ocr.rs:436-530): lines in batches of up
//    to 16 lanes, one run per batch, each lane decoded with `ctc_decode`;
//  - `reorient` (ocr.rs:250-283, 588-612): a line at least 1.5 times as tall
//    as wide scoring under 0.90 is cropped again, turned half a turn and read
//    alone on one lane; the new reading is kept when it is not blank and
//    scores at least 0.05 more.
// The detector input is the page scaled so that its long side is at most
// `--limit` (960), both sides snapped to multiples of 32 (src/det.rs:10-27);
// crops are made on the GPU straight into the recogniser's lanes, at most
// `--max-width` (320) wide. RapidOCR's page fitting (`prepare_page`) and the
// text-score filter are left out. The CPU engine the reference falls back to
// is not part of this library: where the reference would run on the CPU,
// this worker stops with the reference's message.
//
// Pages are binary PPM (P6, 8-bit) files. Each page prints one JSON line:
//   {"page": "...", "lines": [{"quad": [x0, y0, ..., x3, y3], "text": "...",
//    "score": s}, ...], "reoriented": n, "ms": t}
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cctype>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "ppocr_hip.h"

namespace {

constexpr size_t kErr = 512;
constexpr size_t kRecHeight = 48;
// RapidOCR's DB options (src/det.rs:305-315): threshold, box threshold,
// unclip ratio, candidates.
constexpr ppocr_db_options kDb{0.3f, 0.5, 1.5, 1000};
constexpr double kVerticalAspect = 1.5;  // src/crop.rs:67
constexpr double kConfident = 0.90;      // ocr.rs:30
constexpr double kMinGain = 0.05;        // ocr.rs:31
const double kMean[3] = {0.485, 0.456, 0.406};
const double kStd[3] = {0.229, 0.224, 0.225};

struct Options {
  std::string det, rec, dict;
  size_t limit = 960, batch = 16, max_width = 320;
  bool gpu = false;
  std::vector<std::string> pages;
};

struct Line {
  float quad[8];
  std::string text;
  double score;
};

[[noreturn]] void die(const std::string &msg, int code = 1) {
  std::fprintf(stderr, "ppocr-native: %s\n", msg.c_str());
  std::exit(code);
}

bool read_file(const std::string &path, std::string &out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream s;
  s << f.rdbuf();
  out = s.str();
  return true;
}

// A binary PPM: "P6", width, height, maxval 255 (comments from '#' to the
// end of a line), one whitespace byte, then width * height * 3 bytes.
bool read_ppm(const std::string &path, std::vector<uint8_t> &rgb, size_t &w, size_t &h, std::string &err) {
  std::string b;
  if (!read_file(path, b)) return err = "cannot read " + path, false;
  size_t i = 0;
  auto field = [&](std::string &tok) {
    for (;;) {
      while (i < b.size() && std::isspace((unsigned char)b[i])) i++;
      if (i < b.size() && b[i] == '#') {
        while (i < b.size() && b[i] != '\n') i++;
        continue;
      }
      break;
    }
    size_t s = i;
    while (i < b.size() && !std::isspace((unsigned char)b[i])) i++;
    tok = b.substr(s, i - s);
    return !tok.empty();
  };
  std::string magic, ws, hs, ms;
  if (!field(magic) || magic != "P6" || !field(ws) || !field(hs) || !field(ms))
    return err = path + ": not a binary PPM (P6)", false;
  char *end = nullptr;
  w = std::strtoull(ws.c_str(), &end, 10);
  h = std::strtoull(hs.c_str(), &end, 10);
  if (ms != "255") return err = path + ": only 8-bit PPM pages", false;
  i++;  // the one whitespace byte after maxval
  if (w == 0 || h == 0 || w > 32768 || h > 32768 || b.size() < i + w * h * 3)
    return err = path + ": bad size or short data", false;
  rgb.assign(b.begin() + i, b.begin() + i + w * h * 3);
  return true;
}

int snap32(double x) { return int(std::nearbyint(x / 32.0)) * 32; }  // halves to even

// The detector input size for a page, src/det.rs:16-27 with the side fixed.
bool det_size(size_t width, size_t height, size_t limit, size_t &w, size_t &h) {
  const size_t lng = std::max(width, height);
  const double ratio = lng > limit ? double(limit) / double(lng) : 1.0;
  const int sw = snap32(double(size_t(double(width) * ratio)));
  const int sh = snap32(double(size_t(double(height) * ratio)));
  if (sw <= 0 || sh <= 0) return false;
  w = size_t(sw), h = size_t(sh);
  return true;
}

// `is_blank` (src/rec.rs:187-190): every character is Unicode White_Space
// or one of U+001C..U+001F.
bool is_blank(const std::string &s) {
  for (size_t i = 0; i < s.size();) {
    const unsigned char c = s[i];
    uint32_t cp;
    int n;
    if (c < 0x80) cp = c, n = 1;
    else if ((c >> 5) == 6) cp = c & 31, n = 2;
    else if ((c >> 4) == 14) cp = c & 15, n = 3;
    else cp = c & 7, n = 4;
    for (int k = 1; k < n && i + k < s.size(); k++) cp = (cp << 6) | (s[i + k] & 63);
    i += n;
    const bool ws = (cp >= 0x09 && cp <= 0x0d) || (cp >= 0x1c && cp <= 0x20) || cp == 0x85 || cp == 0xa0 ||
                    cp == 0x1680 || (cp >= 0x2000 && cp <= 0x200a) || cp == 0x2028 || cp == 0x2029 ||
                    cp == 0x202f || cp == 0x205f || cp == 0x3000;
    if (!ws) return false;
  }
  return true;
}

// `rereads` (ocr.rs:590-600).
bool rereads(const Line &l) {
  double mn[2] = {INFINITY, INFINITY}, mx[2] = {-INFINITY, -INFINITY};
  for (int p = 0; p < 4; p++)
    for (int a = 0; a < 2; a++) {
      mn[a] = std::min(mn[a], double(l.quad[2 * p + a]));
      mx[a] = std::max(mx[a], double(l.quad[2 * p + a]));
    }
  const double width = mx[0] - mn[0], height = mx[1] - mn[1];
  return width > 0.0 && height >= width * kVerticalAspect && l.score < kConfident;
}

std::string json_string(const std::string &s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') o += '\\', o += char(c);
    else if (c < 0x20) {
      char buf[8];
      std::snprintf(buf, sizeof buf, "\\u%04x", c);
      o += buf;
    } else o += char(c);
  }
  return o + "\"";
}

class Worker {
 public:
  explicit Worker(const Options &o) : o_(o) {}
  ~Worker() {
    if (page_) (void)hipFree(page_);
    if (crop_) (void)hipFree(crop_);
    if (det_) ppocr_gpu_free(det_);
    if (rec_) ppocr_gpu_free(rec_);
    if (dict_) ppocr_dictionary_free(dict_);
  }

  // `Reader::new` with `gpu`: both networks on the GPU, or the reference's
  // message and no worker.
  void load() {
    char err[kErr] = {0};
    std::string text;
    if (!read_file(o_.dict, text)) die("cannot read " + o_.dict);
    if (ppocr_dictionary_load(text.data(), text.size(), &dict_, err, kErr)) die(o_.dict + ": " + err);
    if (ppocr_gpu_load(o_.det.c_str(), &det_, err, kErr) || ppocr_gpu_load(o_.rec.c_str(), &rec_, err, kErr))
      die(std::string("no GPU (") + err + "); the CPU engine is not part of this library");
    // The detector's runs also write the map's DB threshold as row bitmasks.
    if (ppocr_gpu_set_db_mask(det_, 0, kDb.thresh, err, kErr)) die(std::string("DB mask: ") + err);
    std::fprintf(stderr, "ppocr-native: running on %s\n", ppocr_gpu_device(det_));
  }

  bool read(const std::string &path, std::string &json) {
    std::vector<uint8_t> rgb;
    size_t w = 0, h = 0;
    std::string err;
    if (!read_ppm(path, rgb, w, h, err)) return fail(err);
    const auto t0 = std::chrono::steady_clock::now();
    if (!upload(rgb, w, h)) return false;
    std::vector<Line> lines;
    int reoriented = 0;
    if (!detect(w, h, lines) || !recognise(w, h, lines) || !reorient(w, h, lines, reoriented)) return false;
    const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    std::ostringstream s;
    s.precision(9);
    s << "{\"page\": " << json_string(path) << ", \"lines\": [";
    for (size_t i = 0; i < lines.size(); i++) {
      s << (i ? ", " : "") << "{\"quad\": [";
      for (int k = 0; k < 8; k++) s << (k ? ", " : "") << lines[i].quad[k];
      s.precision(17);
      s << "], \"text\": " << json_string(lines[i].text) << ", \"score\": " << lines[i].score << "}";
      s.precision(9);
    }
    s << "], \"reoriented\": " << reoriented << ", \"ms\": " << ms << "}";
    json = s.str();
    return true;
  }

 private:
  bool fail(const std::string &msg) {
    std::fprintf(stderr, "ppocr-native: %s\n", msg.c_str());
    return false;
  }
  bool hip(hipError_t e, const char *what) {
    return e == hipSuccess ? true : fail(std::string(what) + ": " + hipGetErrorString(e));
  }
  void *stream(ppocr_gpu_model *m) { return ppocr_gpu_stream(m); }

  bool upload(const std::vector<uint8_t> &rgb, size_t w, size_t h) {
    if (rgb.size() > page_cap_) {
      if (page_) (void)hipFree(page_), page_ = nullptr;
      if (!hip(hipMalloc(&page_, rgb.size()), "allocating the page")) return false;
      page_cap_ = rgb.size();
    }
    return hip(hipMemcpy(page_, rgb.data(), rgb.size(), hipMemcpyHostToDevice), "uploading the page");
  }

  // `Detector::run` and `boxes_from_prob`: the page's boxes in reading order.
  bool detect(size_t width, size_t height, std::vector<Line> &lines) {
    size_t w, h;
    if (!det_size(width, height, o_.limit, w, h)) return true;  // no text on a page too thin
    char err[kErr] = {0};
    size_t n = 0;
    float *in = nullptr;
    if (ppocr_gpu_set_input_size(det_, h, w, err, kErr) ||
        !(in = ppocr_gpu_lane_input_device(det_, 0, &n)) || n != w * h * 3 ||
        ppocr_hip_det_input(page_, width, height, in, w, h, kMean, kStd, stream(det_)) ||
        ppocr_gpu_run_device(det_, err, kErr)) {
      if (!refused_) std::fprintf(stderr, "ppocr-native: the GPU refused a page (%s)\n", err);
      refused_ = true;
      return false;
    }
    size_t len = 0, wpr = 0, rows = 0;
    const float *prob = ppocr_gpu_lane_output(det_, 0, 0, &len);
    const uint64_t *bits = ppocr_gpu_lane_db_mask(det_, 0, &wpr, &rows);
    if (!prob || len != w * h || !bits || rows != h) return fail("the detector gave no map");
    std::vector<float> boxes(8 * 64);
    size_t nb = 0;
    for (;;) {
      const int rc = ppocr_db_boxes_bits(prob, bits, wpr, w, h, width, height, &kDb, boxes.data(),
                                         boxes.size() / 8, &nb, err, kErr);
      if (rc == 2) {
        boxes.resize(8 * nb);
        continue;
      }
      if (rc) return fail(std::string("boxes: ") + err);
      break;
    }
    for (size_t i = 0; i < nb; i++) {
      Line l{};
      std::memcpy(l.quad, &boxes[8 * i], sizeof l.quad);
      lines.push_back(l);
    }
    return true;
  }

  // Lane inputs for `quads` (n boxes of the page), made on the GPU from the
  // page, then one run; the lanes' texts and scores.
  bool run_lanes(size_t width, size_t height, const float *quads, size_t n, std::vector<Line *> out) {
    char err[kErr] = {0};
    std::vector<size_t> hw;
    for (size_t i = 0; i < n; i++) {
      size_t cw = 0, ch = 0, rw = 0;
      if (ppocr_crop_size(quads + 8 * i, &cw, &ch)) return fail("crop size");
      const size_t tw = ppocr_rec_width_fit(cw, ch, o_.max_width, &rw);
      if (tw == 0) return fail("an empty crop");
      hw.push_back(kRecHeight), hw.push_back(tw);
    }
    if (ppocr_gpu_set_sizes(rec_, hw.data(), n, err, kErr)) return fail(std::string("recogniser: ") + err);
    std::vector<float *> outs(n);
    std::vector<size_t> caps(n), got(n);
    for (size_t i = 0; i < n; i++)
      if (!(outs[i] = ppocr_gpu_lane_input_device(rec_, i, &caps[i]))) return fail("recogniser lane");
    if (ppocr_hip_crop_rec_inputs(page_, width, height, quads, n, o_.max_width, outs.data(), caps.data(),
                                  got.data(), stream(rec_)))
      return fail("recogniser inputs");
    if (ppocr_gpu_run_device(rec_, err, kErr)) return fail(std::string("recogniser: ") + err);
    for (size_t i = 0; i < n; i++)
      if (!decode(i, *out[i])) return false;
    return true;
  }

  // `recognise_all` on the GPU: batches of up to `batch` lanes.
  bool recognise(size_t width, size_t height, std::vector<Line> &lines) {
    for (size_t s = 0; s < lines.size(); s += o_.batch) {
      const size_t n = std::min(o_.batch, lines.size() - s);
      std::vector<float> quads(8 * n);
      std::vector<Line *> out;
      for (size_t i = 0; i < n; i++) {
        std::memcpy(&quads[8 * i], lines[s + i].quad, sizeof lines[s + i].quad);
        out.push_back(&lines[s + i]);
      }
      if (!run_lanes(width, height, quads.data(), n, out)) return false;
    }
    return true;
  }

  // `reorient`: the line's crop (`crop_text` on the GPU), turned half a
  // turn on the host (`rotate_half`: the pixels in reverse order), its
  // recogniser input made on the GPU and read alone on one lane.
  bool reorient(size_t width, size_t height, std::vector<Line> &lines, int &replaced) {
    char err[kErr] = {0};
    for (Line &l : lines) {
      if (!rereads(l)) continue;
      size_t cw = 0, ch = 0, rw = 0;
      if (ppocr_crop_size(l.quad, &cw, &ch)) return fail("crop size");
      const size_t bytes = cw * ch * 3;
      if (bytes > crop_cap_) {
        if (crop_) (void)hipFree(crop_), crop_ = nullptr;
        if (!hip(hipMalloc(&crop_, bytes), "allocating a crop")) return false;
        crop_cap_ = bytes;
      }
      hipStream_t st = hipStream_t(stream(rec_));
      size_t ow = 0, oh = 0;
      if (ppocr_hip_crop_text(page_, width, height, l.quad, crop_, crop_cap_, &ow, &oh, st) || ow != cw ||
          oh != ch)
        return fail("crop_text");
      std::vector<uint8_t> px(bytes);
      if (!hip(hipMemcpyAsync(px.data(), crop_, bytes, hipMemcpyDeviceToHost, st), "reading a crop") ||
          !hip(hipStreamSynchronize(st), "reading a crop"))
        return false;
      for (size_t i = 0, j = cw * ch - 1; i < j; i++, j--)
        for (int c = 0; c < 3; c++) std::swap(px[3 * i + c], px[3 * j + c]);
      if (!hip(hipMemcpyAsync(crop_, px.data(), bytes, hipMemcpyHostToDevice, st), "writing a crop") ||
          !hip(hipStreamSynchronize(st), "writing a crop"))
        return false;
      const size_t tw = ppocr_rec_width_fit(cw, ch, o_.max_width, &rw);
      if (tw == 0) continue;  // an empty crop reads as no text
      const size_t hw[2] = {kRecHeight, tw};
      if (ppocr_gpu_set_sizes(rec_, hw, 1, err, kErr)) return fail(std::string("recogniser: ") + err);
      size_t cap = 0, got = 0;
      float *in = ppocr_gpu_lane_input_device(rec_, 0, &cap);
      if (!in || ppocr_hip_rec_input_fit(crop_, cw, ch, o_.max_width, in, cap, &got, st) || got != tw)
        return fail("recogniser input");
      if (ppocr_gpu_run_device(rec_, err, kErr)) return fail(std::string("recogniser: ") + err);
      Line turned = l;
      if (!decode(0, turned)) return false;
      if (!is_blank(turned.text) && turned.score >= l.score + kMinGain) {
        l.text = turned.text, l.score = turned.score;
        replaced++;
      }
    }
    return true;
  }

  // Lane `lane`'s text and score from the last recogniser run.
  bool decode(size_t lane, Line &out) {
    char err[kErr] = {0};
    size_t len = 0, tl = 0;
    const float *pairs = ppocr_gpu_lane_output(rec_, lane, 0, &len);
    if (!pairs) return fail("recogniser output");
    int rc;
    while ((rc = ppocr_ctc_decode_pairs(dict_, pairs, len / 2, text_.data(), text_.size(), &tl, &out.score, err,
                                        kErr)) == 2)
      text_.resize(tl + 1);
    if (rc) return fail(std::string("ctc: ") + err);
    out.text.assign(text_.data(), tl);
    return true;
  }

  const Options &o_;
  ppocr_gpu_model *det_ = nullptr, *rec_ = nullptr;
  ppocr_dictionary *dict_ = nullptr;
  uint8_t *page_ = nullptr, *crop_ = nullptr;
  size_t page_cap_ = 0, crop_cap_ = 0;
  std::vector<char> text_ = std::vector<char>(4096);
  bool refused_ = false;
};

const char kUsage[] =
    "usage: ppocr_hip_worker --gpu --det DET.plan --rec REC.plan --dict characters.txt\n"
    "                        [--limit 960] [--batch 16] [--max-width 320] PAGE.ppm...\n";

}  // namespace

int main(int argc, char **argv) {
  Options o;
  for (int i = 1; i < argc; i++) {
    const std::string a = argv[i];
    auto value = [&]() -> std::string {
      if (i + 1 >= argc) die(a + " needs a value\n" + kUsage, 2);
      return argv[++i];
    };
    auto count = [&]() -> size_t {
      const std::string v = value();
      char *end = nullptr;
      const unsigned long long n = std::strtoull(v.c_str(), &end, 10);
      if (!*v.c_str() || *end || n == 0) die(a + ": a positive whole number, not " + v, 2);
      return size_t(n);
    };
    if (a == "--gpu") o.gpu = true;
    else if (a == "--det") o.det = value();
    else if (a == "--rec") o.rec = value();
    else if (a == "--dict") o.dict = value();
    else if (a == "--limit") o.limit = count();
    else if (a == "--batch") o.batch = count();
    else if (a == "--max-width") o.max_width = count();
    else if (a == "-h" || a == "--help") return std::fputs(kUsage, stdout), 0;
    else if (!a.empty() && a[0] == '-') die("unknown option " + a + "\n" + kUsage, 2);
    else o.pages.push_back(a);
  }
  if (o.det.empty() || o.rec.empty() || o.dict.empty()) die(std::string("--det, --rec and --dict are needed\n") + kUsage, 2);
  if (!o.gpu) die("this library reads on the GPU only: pass --gpu", 2);
  Worker w(o);
  w.load();
  int failed = 0;
  for (const std::string &p : o.pages) {
    std::string json;
    if (w.read(p, json)) std::printf("%s\n", json.c_str());
    else failed++;
    std::fflush(stdout);
  }
  return failed ? 1 : 0;
}
