/*
 * CPU oracle for the image stages either side of the detector and the
 * recogniser: the bilinear resize, the detector's input tensor, the
 * recogniser's input tensor and the perspective text crop. A restatement of
 * the reference's CPU arithmetic, pinned against the reference's golden
 * data (tests/golden/: OpenCV 5.0 and RapidOCR outputs).
 *
 * TEST INFRASTRUCTURE ONLY: the GPU kernels are compared against it; the product
 * library never links or calls it.
 *
 * Reference files (paths relative to the ppocr-native source tree):
 *   bilinear resize          src/image.rs:33-142
 *   detector input           src/det.rs:195-224
 *   recogniser input         src/rec.rs:10-43
 *   text crop                src/crop.rs:1-127, src/det.rs:398-402
 *   region borders           src/contour.rs:44-140
 *
 * Images are 8-bit, three channels, rows top to bottom (HWC).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* One output coordinate: source indices and weights in 1/2048 units. OpenCV
 * places output d at (d + 0.5) * scale - 0.5, rounded to f32; each weight is
 * rounded on its own; taps past an edge read the edge (image.rs:33-66). */
typedef struct {
    long near_i, far_i;
    int near_w, far_w;
} tap_t;

static tap_t tap_at(size_t src, size_t dst, size_t d) {
    double scale = 1.0 / ((double)dst / (double)src);
    float f = (float)(((double)d + 0.5) * scale - 0.5);
    float fl = floorf(f);
    float a = f - fl;
    long s = (long)fl, last = (long)src - 1;
    tap_t t;
    t.near_i = s < 0 ? 0 : (s > last ? last : s);
    t.far_i = s + 1 < 0 ? 0 : (s + 1 > last ? last : s + 1);
    t.near_w = (int)nearbyintf((1.0f - a) * 2048.0f);
    t.far_w = (int)nearbyintf(a * 2048.0f);
    return t;
}

/* cv2.resize INTER_LINEAR on 8 bits (image.rs:68-142): the horizontal pass
 * keeps full 1/2048 products; the vertical one drops 4 bits of each row,
 * weights, drops 16, adds, and rounds by two more. */
void oracle_resize_linear(const uint8_t *src, size_t sw, size_t sh, uint8_t *dst, size_t dw, size_t dh) {
    tap_t *xs = malloc(dw * sizeof(tap_t));
    int32_t *top = malloc(dw * 3 * sizeof(int32_t)), *bot = malloc(dw * 3 * sizeof(int32_t));
    for (size_t x = 0; x < dw; x++) xs[x] = tap_at(sw, dw, x);
    for (size_t y = 0; y < dh; y++) {
        tap_t ty = tap_at(sh, dh, y);
        const uint8_t *rn = src + (size_t)ty.near_i * sw * 3, *rf = src + (size_t)ty.far_i * sw * 3;
        for (size_t x = 0; x < dw; x++)
            for (int c = 0; c < 3; c++) {
                top[x * 3 + c] = (int32_t)rn[xs[x].near_i * 3 + c] * xs[x].near_w +
                                 (int32_t)rn[xs[x].far_i * 3 + c] * xs[x].far_w;
                bot[x * 3 + c] = (int32_t)rf[xs[x].near_i * 3 + c] * xs[x].near_w +
                                 (int32_t)rf[xs[x].far_i * 3 + c] * xs[x].far_w;
            }
        for (size_t k = 0; k < dw * 3; k++) {
            int32_t v = (((top[k] >> 4) * ty.near_w) >> 16) + (((bot[k] >> 4) * ty.far_w) >> 16);
            v = (v + 2) >> 2;
            dst[y * dw * 3 + k] = (uint8_t)(v < 0 ? 0 : (v > 255 ? 255 : v));
        }
    }
    free(xs), free(top), free(bot);
}

/* The detector input, HWC (det.rs:195-224, 228-289): resized, x = v * (1/255
 * as f32) in f32, then (x - mean) / std in f64, rounded once to f32. */
void oracle_det_input(const uint8_t *src, size_t sw, size_t sh, size_t dw, size_t dh, const double *mean,
                      const double *std, float *out) {
    uint8_t *r = malloc(dw * dh * 3);
    oracle_resize_linear(src, sw, sh, r, dw, dh);
    const float scale = (float)(1.0 / 255.0);
    for (size_t i = 0; i < dw * dh * 3; i++) {
        int c = (int)(i % 3);
        float x = (float)r[i] * scale;
        out[i] = (float)(((double)x - mean[c]) / std[c]);
    }
    free(r);
}

/* The recogniser's width for a w x h crop (rec.rs:19-31): the tensor width
 * 48 * max(320 / 48, w / h) truncated; the resized width 48 * w / h rounded
 * up, cut back to the tensor width. */
size_t oracle_rec_width(size_t w, size_t h, size_t *resized_w) {
    double ratio = 320.0 / 48.0 > (double)w / (double)h ? 320.0 / 48.0 : (double)w / (double)h;
    size_t width = (size_t)(48.0 * ratio);
    double fitted = ceil(48.0 * ((double)w / (double)h));
    *resized_w = fitted > (double)width ? width : (size_t)fitted;
    return width;
}

/* The width with the tensor capped at max_width (0: no cap): a crop wider
 * than the cap is resized to exactly max_width columns, any other keeps
 * rec.rs's widths. */
size_t oracle_rec_width_fit(size_t w, size_t h, size_t max_width, size_t *resized_w) {
    size_t width = oracle_rec_width(w, h, resized_w);
    if (max_width && width > max_width) {
        *resized_w = max_width;
        return max_width;
    }
    return width;
}

/* The recogniser input, HWC, 48 x width (rec.rs:19-43): resized to 48 rows
 * of resized_w, (v / 255 - 0.5) / 0.5 in f32, zeros to the right; the
 * widths of oracle_rec_width_fit. */
size_t oracle_rec_input_fit(const uint8_t *src, size_t w, size_t h, size_t max_width, float *out, size_t cap) {
    size_t rw;
    size_t width = oracle_rec_width_fit(w, h, max_width, &rw);
    if (48 * width * 3 > cap) return 0;
    uint8_t *r = malloc(rw * 48 * 3);
    oracle_resize_linear(src, w, h, r, rw, 48);
    memset(out, 0, 48 * width * 3 * sizeof(float));
    for (size_t y = 0; y < 48; y++)
        for (size_t x = 0; x < rw; x++)
            for (int c = 0; c < 3; c++)
                out[(y * width + x) * 3 + c] = ((float)r[(y * rw + x) * 3 + c] / 255.0f - 0.5f) / 0.5f;
    free(r);
    return width;
}

size_t oracle_rec_input(const uint8_t *src, size_t w, size_t h, float *out, size_t cap) {
    return oracle_rec_input_fit(src, w, h, 0, out, cap);
}

/* The projective map of the width x height rectangle's corners onto the
 * quad, by Gaussian elimination with partial pivoting (crop.rs:7-53). */
static void rect_to_quad(double width, double height, const float *q, double *out) {
    double m[8][9];
    const double from[4][2] = {{0, 0}, {width, 0}, {width, height}, {0, height}};
    for (int i = 0; i < 4; i++) {
        double x = from[i][0], y = from[i][1], u = (double)q[2 * i], v = (double)q[2 * i + 1];
        double a[9] = {x, y, 1.0, 0.0, 0.0, 0.0, -x * u, -y * u, u};
        double b[9] = {0.0, 0.0, 0.0, x, y, 1.0, -x * v, -y * v, v};
        memcpy(m[i], a, sizeof a), memcpy(m[i + 4], b, sizeof b);
    }
    for (int col = 0; col < 8; col++) {
        int piv = col; /* the last of equal largest magnitudes, as max_by keeps */
        for (int r = col + 1; r < 8; r++)
            if (!(fabs(m[r][col]) < fabs(m[piv][col]))) piv = r;
        double t[9];
        memcpy(t, m[col], sizeof t), memcpy(m[col], m[piv], sizeof t), memcpy(m[piv], t, sizeof t);
        double p = m[col][col];
        if (p == 0.0) continue;
        double prow[9];
        memcpy(prow, m[col], sizeof prow);
        for (int r = 0; r < 8; r++) {
            double f = m[r][col] / p;
            if (r != col && f != 0.0)
                for (int k = col; k < 9; k++) m[r][k] -= f * prow[k];
        }
    }
    for (int i = 0; i < 8; i++) out[i] = m[i][i] == 0.0 ? 0.0 : m[i][8] / m[i][i];
    out[8] = 1.0;
}

/* Keys' cubic weights, a = -0.75, in OpenCV's factoring (crop.rs:55-63). */
static void cubic(float t, float *w) {
    const float A = -0.75f;
    w[0] = ((A * (t + 1.0f) - 5.0f * A) * (t + 1.0f) + 8.0f * A) * (t + 1.0f) - 4.0f * A;
    w[1] = ((A + 2.0f) * t - (A + 3.0f)) * t * t + 1.0f;
    w[2] = ((A + 2.0f) * (1.0f - t) - (A + 3.0f)) * (1.0f - t) * (1.0f - t) + 1.0f;
    w[3] = 1.0f - w[0] - w[1] - w[2];
}

static float dist(const float *p, const float *q) {
    float dx = p[0] - q[0], dy = p[1] - q[1];
    return sqrtf(dx * dx + dy * dy);
}

/* The crop's size before any turn (crop.rs:84-87). */
void oracle_crop_size(const float *q, size_t *w, size_t *h) {
    float a = dist(q + 0, q + 2), b = dist(q + 4, q + 6), c = dist(q + 0, q + 6), d = dist(q + 2, q + 4);
    *w = (size_t)(a > b ? a : b);
    *h = (size_t)(c > d ? c : d);
}

/* get_rotate_crop_image (crop.rs:84-127): bicubic, edges repeated, each row
 * of four summed first; a quarter turn counter-clockwise when h / w >= 1.5.
 * Writes the crop (after any turn) and its size; 0 when cap is too small. */
int oracle_crop_text(const uint8_t *img, size_t iw, size_t ih, const float *q, uint8_t *out, size_t cap,
                     size_t *ow, size_t *oh) {
    size_t width, height;
    oracle_crop_size(q, &width, &height);
    if (width * height * 3 > cap) return 0;
    double m[9];
    rect_to_quad((double)width, (double)height, q, m);
    long lx = (long)iw - 1, ly = (long)ih - 1;
    int turn = (double)height / (double)width >= 1.5; /* a zero width turns too */
    for (size_t y = 0; y < height; y++)
        for (size_t x = 0; x < width; x++) {
            double xf = (double)x, yf = (double)y;
            double w = m[6] * xf + m[7] * yf + m[8];
            w = w == 0.0 ? 0.0 : 1.0 / w;
            float sx = (float)((m[0] * xf + m[1] * yf + m[2]) * w);
            float sy = (float)((m[3] * xf + m[4] * yf + m[5]) * w);
            float fx = floorf(sx), fy = floorf(sy), wx[4], wy[4];
            cubic(sx - fx, wx), cubic(sy - fy, wy);
            /* Saturating float -> integer: NaN is 0, the far outside an edge. */
            const float far = 1073741824.0f;
            long ix = (long)(isnan(fx) ? 0.0f : fminf(fmaxf(fx, -far), far)) - 1;
            long iy = (long)(isnan(fy) ? 0.0f : fminf(fmaxf(fy, -far), far)) - 1;
            float acc[3] = {0, 0, 0};
            for (int j = 0; j < 4; j++) {
                long r = iy + j < 0 ? 0 : (iy + j > ly ? ly : iy + j);
                float line[3] = {0, 0, 0};
                for (int i = 0; i < 4; i++) {
                    long cc = ix + i < 0 ? 0 : (ix + i > lx ? lx : ix + i);
                    const uint8_t *px = img + ((size_t)r * iw + (size_t)cc) * 3;
                    for (int c = 0; c < 3; c++) line[c] += (float)px[c] * wx[i];
                }
                for (int c = 0; c < 3; c++) acc[c] += line[c] * wy[j];
            }
            /* A quarter turn counter-clockwise: column x becomes row
             * width - 1 - x of a height-wide image (image.rs:145-155). */
            size_t at = turn ? ((width - 1 - x) * height + y) : (y * width + x);
            for (int c = 0; c < 3; c++) {
                float v = nearbyintf(acc[c]);
                out[at * 3 + c] = (uint8_t)(isnan(v) || v < 0.0f ? 0.0f : (v > 255.0f ? 255.0f : v));
            }
        }
    *ow = turn ? height : width;
    *oh = turn ? width : height;
    return 1;
}

/* Region borders of a binary mask (src/contour.rs:44-140): Suzuki and Abe's
 * border following over 8-connected foreground, every pixel visited in
 * raster order, outer borders (foreground with background to the west) and
 * hole borders (foreground, not marked east, with background to the east),
 * each followed counter-clockwise on screen from the first foreground
 * neighbour clockwise of the background pixel that revealed it, its pixels
 * marked (marked-east where the walk passed background to the east), and
 * reduced to the pixels where the step changes direction; the borders found
 * last listed first. Steps are numbered counter-clockwise on screen from
 * east, as the reference numbers them.
 *
 * Output: the corners of every border, x then y, one border after another
 * (pts), and each border's corner count (lens), in list order. Returns 0;
 * 1 when pts or lens is too small (n_pts and n_cont then hold the sizes
 * needed); 2 when out of memory. */
enum { BG = 0, UNSEEN = 1, MARKED = 2, MARKED_EAST = 3 };

int oracle_find_contours(const uint8_t *mask, size_t width, size_t height, int32_t *pts, size_t pts_cap,
                         size_t *lens, size_t lens_cap, size_t *n_pts, size_t *n_cont) {
    static const int sx[8] = {1, 1, 0, -1, -1, -1, 0, 1}, sy[8] = {0, -1, -1, -1, 0, 1, 1, 1};
    const int east = 0, west = 4;
    const long stride = (long)width + 2;
    uint8_t *state = calloc((size_t)stride * (height + 2), 1);
    size_t chain_cap = 1024, found_cap = 1024, nf = 0, found_pts_cap = 4096, nfp = 0;
    long *chain_at = malloc(chain_cap * sizeof(long));
    int *chain_dir = malloc(chain_cap * sizeof(int));
    size_t *found_len = malloc(found_cap * sizeof(size_t));
    int32_t *found_pts = malloc(found_pts_cap * 2 * sizeof(int32_t));
    int rc = 0;
    if (!state || !chain_at || !chain_dir || !found_len || !found_pts) {
        rc = 2;
        goto done;
    }
    for (size_t y = 0; y < height; y++)
        for (size_t x = 0; x < width; x++)
            state[(y + 1) * stride + x + 1] = mask[y * width + x] ? UNSEEN : BG;
    long off[8];
    for (int d = 0; d < 8; d++) off[d] = sx[d] + sy[d] * stride;
    for (size_t y = 1; y <= height; y++)
        for (size_t x = 1; x <= width; x++) {
            const long start = (long)y * stride + (long)x;
            const uint8_t here = state[start];
            int from;
            if (here == UNSEEN && state[start - 1] == BG)
                from = west;
            else if ((here == UNSEEN || here == MARKED) && state[start + 1] == BG)
                from = east;
            else
                continue;
            int last_dir = -1;
            for (int k = 0; k < 8 && last_dir < 0; k++) {
                const int d = (from + 8 - k) % 8;
                if (state[start + off[d]] != BG) last_dir = d;
            }
            size_t n = 0;
            if (last_dir < 0) {
                state[start] = MARKED_EAST;
                chain_at[0] = start, chain_dir[0] = 0, n = 1;
            } else {
                const long last = start + off[last_dir];
                long cur = start;
                int back = last_dir;
                for (;;) {
                    int east_bg = 0, next_dir = back;
                    for (int k = 1; k <= 8; k++) {
                        const int d = (back + k) % 8;
                        if (state[cur + off[d]] != BG) {
                            next_dir = d;
                            break;
                        }
                        if (d == east) east_bg = 1;
                    }
                    if (east_bg)
                        state[cur] = MARKED_EAST;
                    else if (state[cur] == UNSEEN)
                        state[cur] = MARKED;
                    if (n == chain_cap) {
                        chain_cap *= 2;
                        long *a = realloc(chain_at, chain_cap * sizeof(long));
                        int *b = realloc(chain_dir, chain_cap * sizeof(int));
                        if (a) chain_at = a;
                        if (b) chain_dir = b;
                        if (!a || !b) {
                            rc = 2;
                            goto done;
                        }
                    }
                    chain_at[n] = cur, chain_dir[n] = next_dir, n++;
                    const long next = cur + off[next_dir];
                    if (next == start && cur == last) break;
                    back = (next_dir + 4) % 8;
                    cur = next;
                }
            }
            /* The corners: a lone pixel is its own; else the pixels whose step
             * differs from the one before (cyclically), from the first such. */
            size_t first = 0, k = 0;
            int any = 0;
            if (last_dir >= 0)
                for (; first < n; first++)
                    if (chain_dir[first] != chain_dir[(first + n - 1) % n]) {
                        any = 1;
                        break;
                    }
            if (nf == found_cap) {
                found_cap *= 2;
                size_t *a = realloc(found_len, found_cap * sizeof(size_t));
                if (!a) {
                    rc = 2;
                    goto done;
                }
                found_len = a;
            }
            for (size_t i = 0; i < n; i++) {
                const size_t at = (first + i) % n;
                const int keep = last_dir < 0 ? 1 : (any && chain_dir[at] != chain_dir[(at + n - 1) % n]);
                if (!keep) continue;
                if (nfp == found_pts_cap) {
                    found_pts_cap *= 2;
                    int32_t *a = realloc(found_pts, found_pts_cap * 2 * sizeof(int32_t));
                    if (!a) {
                        rc = 2;
                        goto done;
                    }
                    found_pts = a;
                }
                found_pts[2 * nfp] = (int32_t)(chain_at[at] % stride) - 1;
                found_pts[2 * nfp + 1] = (int32_t)(chain_at[at] / stride) - 1;
                nfp++, k++;
            }
            found_len[nf++] = k;
        }
    *n_pts = nfp;
    *n_cont = nf;
    if (nfp > pts_cap || nf > lens_cap) {
        rc = 1;
        goto done;
    }
    /* List order: the last border found first. */
    {
        size_t end = nfp, o = 0;
        for (size_t c = nf; c-- > 0;) {
            const size_t begin = end - found_len[c];
            memcpy(pts + 2 * o, found_pts + 2 * begin, found_len[c] * 2 * sizeof(int32_t));
            o += found_len[c];
            lens[nf - 1 - c] = found_len[c];
            end = begin;
        }
    }
done:
    free(state);
    free(chain_at);
    free(chain_dir);
    free(found_len);
    free(found_pts);
    return rc;
}
