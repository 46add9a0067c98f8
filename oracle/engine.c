/*
 * CPU oracle: a restatement, in C, of ppocr-native's plan reader and of the
 * CPU engine's arithmetic, operation by operation, at its AVX2+FMA tier.
 *
 * TEST INFRASTRUCTURE ONLY. The GPU backend is compared against this file.
 * Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline may load
 * it; the product library never links or calls it.
 *
 * Reference files (paths relative to the ppocr-native source tree):
 *   plan layout and checks     src/engine/plan.rs:9-28, 296-842
 *   op dispatch                src/engine/mod.rs:1120-1233
 *   convolution / pooling      src/engine/conv.rs:42-79, 115-468
 *   other layers               src/engine/layers.rs:375-832
 *   exp / sigmoid              src/engine/kernels/activation.rs:10-60, 151-159
 *   GELU, swish, hard sigmoid  src/engine/layers.rs:20-72, 212-226
 *
 * Summation orders (tier 3): every convolution output starts from its bias
 * and adds weight*input with a fused multiply-add, taps in [ky][kx] order and
 * within a tap the channels of each source in order (kernels/dense.rs:38-147,
 * kernels/depthwise.rs:93-217). Two pointwise cases add the bias last instead
 * (kernels/pointwise.rs:135-185, 762): output widths that are not a multiple
 * of 16, and the last count % 4 pixels of each call of rows_per_group rows
 * (conv.rs:21-30). The channel mean sums in f64 (layers.rs:391-406); layer
 * norm sums in f32 with separate multiply and add (layers.rs:467-479);
 * softmax and the CTC head reduce in 8 lanes (layers.rs:247-294, 753-832).
 *
 * Extension: folded activation code 7 is hard swish,
 * x * clamp(x * (1/6) + 0.5, 0, 1), product and sum rounded separately.
 * The reference reads codes 0-6 only.
 *
 * Rows of a layer are shared between OpenMP threads; every output is
 * computed by one thread in a fixed order, so results do not depend on the
 * thread count.
 */
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { CONV, DWCONV, ADD, MAXPOOL, AVGPOOL, CHANNELMUL, CONCATC, LAYERNORM,
       ATTENTION, MEAN, CTCHEAD, CTCARGMAX, UPSAMPLE, UPSAMPLEADD, CONVTRANSPOSE,
       KIND_COUNT };
enum { F_NONE, F_RELU, F_SIGMOID, F_GELU, F_SWISH, F_HARDSIGMOID, F_HARDSIGMOIDFIFTH,
       F_HARDSWISH, FUSED_COUNT };

#define OP_FIELDS 20
#define MAX_SCRATCH_FLOATS ((size_t)1 << 30)
#define MAX_WINDOW ((size_t)1 << 16)
#define LANES 8
#define PANEL 16

typedef struct {
    int kind, fused;
    size_t x, x2, y, ih, iw, ic, oh, ow, oc, kh, kw, sh, sw;
    long pt, pb, pl, pr;
    size_t n2, w0, w1, b0, b1;
} op_t;

typedef struct oracle_model {
    size_t in_slot, in_h, in_w, in_c;
    size_t nbuf, nout, nops;
    size_t *out_slot, *out_n;
    op_t *ops;
    float *weights;
    size_t nweights;
    size_t *pool;      /* floats each buffer holds at the current size */
    float **bufs;      /* one allocation per plan buffer */
    size_t *cap;       /* floats allocated per buffer */
} oracle_model;

/* ---------------------------------------------------------------- errors */

static void fail(char *err, size_t len, const char *fmt, ...) {
    if (!err || !len) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, len, fmt, ap);
    va_end(ap);
}

/* ------------------------------------------------------------ arithmetic */

static inline float f_of(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t u_of(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* XNNPACK f32-vsigmoid p5 constants, kernels/activation.rs:10-21. */
#define EXP_MAGIC_BIAS f_of(0x4b40007fu)
#define LOG2E f_of(0x3fb8aa3bu)
#define MINUS_LN2 f_of(0xbf317218u)
#define EXP_C5 f_of(0x3c07cfceu)
#define EXP_C4 f_of(0x3d2b9d0du)
#define EXP_C3 f_of(0x3e2aad40u)
#define EXP_C2 f_of(0x3efffee3u)
#define EXP_C1 f_of(0x3f7ffffbu)
#define EXP_CUTOFF f_of(0xc2aeac4fu)
#define HARDSIGMOID_ALPHA f_of(0x3e2aaaadu)
#define ONE_SIXTH f_of(0x3e2aaaabu)

/* exp(z) for z <= 0 with the tier-3 one-FMA reduction; activation.rs:37-60. */
float oracle_exp_neg(float z) {
    float n = fmaf(z, LOG2E, EXP_MAGIC_BIAS);
    float s = f_of(u_of(n) << 23);
    n = n - EXP_MAGIC_BIAS;
    float t = fmaf(n, MINUS_LN2, z);
    float p = fmaf(fmaf(fmaf(fmaf(EXP_C5, t, EXP_C4), t, EXP_C3), t, EXP_C2), t, EXP_C1);
    if (z < EXP_CUTOFF) return 0.0f;
    return fmaf(t * s, p, s);
}

/* activation.rs:151-159 */
static inline float sigmoid_one(float x) {
    float e = oracle_exp_neg(f_of(u_of(x) | 0x80000000u));
    float f = e / (e + 1.0f);
    return (u_of(x) & 0x80000000u) ? f : 1.0f - f;
}

/* Rust's f32::clamp: NaN passes through, -0 stays. */
static inline float clampf(float v, float lo, float hi) {
    if (v < lo) v = lo;
    if (v > hi) v = hi;
    return v;
}

/* layers.rs:20-67 with FMA (tier 3's activation_avx2). */
static const uint32_t PHI_P[6] = {0x3ecc4228u, 0x3d0aa93cu, 0x3b9943c9u,
                                  0x39310738u, 0x36d52462u, 0x32c36a3cu};
static const uint32_t PHI_Q[5] = {0x3e80c788u, 0x3ceaaaeeu, 0x3af6ffc6u,
                                  0x389a737au, 0x35a0b9e3u};

static inline float gelu_one(float x) {
    float c = clampf(x, -5.5f, 5.5f);
    float s = c * c;
    float p = f_of(PHI_P[5]);
    for (int i = 4; i >= 0; i--) p = fmaf(p, s, f_of(PHI_P[i]));
    float q = f_of(PHI_Q[4]);
    for (int i = 3; i >= 0; i--) q = fmaf(q, s, f_of(PHI_Q[i]));
    q = fmaf(q, s, 1.0f);
    return x * clampf(fmaf(c, p / q, 0.5f), 0.0f, 1.0f);
}

float oracle_act(float v, int fused) {
    switch (fused) {
    case F_RELU: return clampf(v, 0.0f, INFINITY);
    case F_SIGMOID: return sigmoid_one(v);
    case F_GELU: return gelu_one(v);
    case F_SWISH: return v * sigmoid_one(v);
    case F_HARDSIGMOID: return clampf(v * HARDSIGMOID_ALPHA + 0.5f, 0.0f, 1.0f);
    case F_HARDSIGMOIDFIFTH: return clampf(v * 0.2f + 0.5f, 0.0f, 1.0f);
    case F_HARDSWISH: return v * clampf(v * ONE_SIXTH + 0.5f, 0.0f, 1.0f);
    default: return v;
    }
}

/* ------------------------------------------------------------ plan file */

static int shape_len(size_t a, size_t b, size_t c, size_t *out) {
    if (!a || !b || !c) return 0;
    if (a > SIZE_MAX / b) return 0;
    size_t ab = a * b;
    if (ab > SIZE_MAX / c) return 0;
    *out = ab * c;
    return 1;
}

static int second_of(const op_t *op, size_t *slot) {
    int binary = op->kind == ADD || op->kind == CHANNELMUL || op->kind == CONCATC ||
                 op->kind == UPSAMPLEADD || (op->kind == CONV && op->n2 > 0);
    if (binary) *slot = op->x2;
    return binary;
}

static int is_pointwise(const op_t *op) {
    return op->kind == CONV && op->kh == 1 && op->kw == 1 && op->sh == 1 && op->sw == 1 &&
           op->pt == 0 && op->pb == 0 && op->pl == 0 && op->pr == 0;
}

/* What `slot` holds when op `before` runs; plan.rs:403-408. */
static int produced(const oracle_model *m, size_t before, size_t slot, size_t *h, size_t *w,
                    size_t *c) {
    for (size_t i = before; i-- > 0;) {
        if (m->ops[i].y == slot) {
            *h = m->ops[i].oh; *w = m->ops[i].ow; *c = m->ops[i].oc;
            return 1;
        }
    }
    if (slot == m->in_slot) {
        *h = m->in_h; *w = m->in_w; *c = m->in_c;
        return 1;
    }
    return 0;
}

static int window_out(size_t n, long before, long after, size_t k, size_t s, size_t *out) {
    if (before < 0 || after < 0 || s == 0) return 0;
    size_t span = n + (size_t)before + (size_t)after;
    if (span < k) return 0;
    *out = (span - k) / s + 1;
    return 1;
}

/* plan.rs:414-494 */
static int derive_shapes(oracle_model *m, size_t height, size_t width, char *err, size_t el) {
    m->in_h = height;
    m->in_w = width;
    for (size_t i = 0; i < m->nops; i++) {
        op_t *op = &m->ops[i];
        size_t h, w, c;
        if (!produced(m, i, op->x, &h, &w, &c)) { fail(err, el, "op %zu reads a buffer nothing wrote", i); return 0; }
        if (c != op->ic) { fail(err, el, "op %zu reads a tensor of another shape", i); return 0; }
        size_t oh = 0, ow = 0;
        switch (op->kind) {
        case CONV: case DWCONV: case MAXPOOL: case AVGPOOL:
            if (!window_out(h, op->pt, op->pb, op->kh, op->sh, &oh) ||
                !window_out(w, op->pl, op->pr, op->kw, op->sw, &ow)) {
                fail(err, el, "op %zu has a window larger than its padded input", i); return 0;
            }
            break;
        case UPSAMPLE: case UPSAMPLEADD:
            if ((op->sh && h > SIZE_MAX / op->sh) || (op->sw && w > SIZE_MAX / op->sw)) { fail(err, el, "op %zu output size overflows", i); return 0; }
            oh = h * op->sh; ow = w * op->sw;
            break;
        case CONVTRANSPOSE:
            if ((op->kh && h > SIZE_MAX / op->kh) || (op->kw && w > SIZE_MAX / op->kw)) { fail(err, el, "op %zu output size overflows", i); return 0; }
            oh = h * op->kh; ow = w * op->kw;
            break;
        case MEAN: oh = 1; ow = 1; break;
        default: oh = h; ow = w; break;
        }
        int has2 = 1;
        size_t wh = oh, ww = ow, wc = op->oc;
        switch (op->kind) {
        case ADD: case UPSAMPLEADD: break;
        case CONCATC: wc = op->n2; break;
        case CHANNELMUL: wh = 1; ww = 1; break;
        case CONV: if (op->n2 > 0) { wh = h; ww = w; wc = op->n2; } else has2 = 0; break;
        default: has2 = 0;
        }
        if (has2) {
            size_t h2, w2, c2;
            if (!produced(m, i, op->x2, &h2, &w2, &c2) || h2 != wh || w2 != ww || c2 != wc) {
                fail(err, el, "op %zu reads a second tensor of another shape", i); return 0;
            }
        }
        op->ih = h; op->iw = w; op->oh = oh; op->ow = ow;
    }
    memset(m->pool, 0, m->nbuf * sizeof(size_t));
    size_t image;
    if (!shape_len(height, width, m->in_c, &image)) { fail(err, el, "input shape is zero or overflows"); return 0; }
    if (m->in_slot >= m->nbuf) { fail(err, el, "buffer %zu does not exist", m->in_slot); return 0; }
    if (m->pool[m->in_slot] < image) m->pool[m->in_slot] = image;
    for (size_t i = 0; i < m->nops; i++) {
        op_t *op = &m->ops[i];
        size_t n;
        if (!shape_len(op->oh, op->ow, op->oc, &n)) { fail(err, el, "op %zu output shape is zero or overflows", i); return 0; }
        if (op->y >= m->nbuf) { fail(err, el, "buffer %zu does not exist", op->y); return 0; }
        if (m->pool[op->y] < n) m->pool[op->y] = n;
    }
    for (size_t k = 0; k < m->nout; k++) {
        size_t h, w, c;
        if (!produced(m, m->nops, m->out_slot[k], &h, &w, &c)) { fail(err, el, "output %zu is never written", k); return 0; }
        m->out_n[k] = h * w * c;
    }
    return 1;
}

static int mul_ok(size_t a, size_t b, size_t *out) {
    if (a && b > SIZE_MAX / a) return 0;
    *out = a * b;
    return 1;
}

/* plan.rs:498-767 */
static int check_plan(const oracle_model *m, char *err, size_t el) {
    for (size_t s = 0; s < m->nbuf; s++)
        if (m->pool[s] > MAX_SCRATCH_FLOATS) { fail(err, el, "a buffer wants %zu floats, ceiling is %zu", m->pool[s], MAX_SCRATCH_FLOATS); return 0; }
    size_t input_len;
    if (!shape_len(m->in_h, m->in_w, m->in_c, &input_len)) { fail(err, el, "input shape is zero or overflows"); return 0; }
    if (m->in_slot >= m->nbuf || m->pool[m->in_slot] < input_len) { fail(err, el, "the input buffer is smaller than the image"); return 0; }
    for (size_t k = 0; k < m->nout; k++)
        if (m->out_slot[k] >= m->nbuf || m->pool[m->out_slot[k]] < m->out_n[k]) { fail(err, el, "output %zu claims more elements than its buffer", k); return 0; }
    for (size_t i = 0; i < m->nops; i++) {
        const op_t *op = &m->ops[i];
        size_t in_len, out_len;
        if (!shape_len(op->ih, op->iw, op->ic, &in_len)) { fail(err, el, "op %zu input shape is zero or overflows", i); return 0; }
        if (!shape_len(op->oh, op->ow, op->oc, &out_len)) { fail(err, el, "op %zu output shape is zero or overflows", i); return 0; }
        switch (op->kind) {
        case CONV: case DWCONV: case AVGPOOL: case MAXPOOL: {
            size_t k4[4] = {op->kh, op->kw, op->sh, op->sw};
            long p4[4] = {op->pt, op->pb, op->pl, op->pr};
            for (int j = 0; j < 4; j++) {
                if (k4[j] == 0 || k4[j] > MAX_WINDOW || p4[j] < 0 || (size_t)p4[j] > MAX_WINDOW) {
                    fail(err, el, "op %zu has an unsupported kernel, stride or padding", i); return 0;
                }
            }
            break;
        }
        case MEAN:
            if (op->oh != 1 || op->ow != 1 || op->ic != op->oc) { fail(err, el, "op %zu invalid channel mean", i); return 0; }
            break;
        case CONCATC:
            if (op->ih != op->oh || op->iw != op->ow || op->ic + op->n2 != op->oc) { fail(err, el, "op %zu invalid channel concatenation", i); return 0; }
            break;
        case CTCHEAD: case CTCARGMAX: {
            size_t vocab = op->kind == CTCHEAD ? op->oc : op->n2;
            size_t columns = (vocab + PANEL - 1) / PANEL * PANEL, wl;
            if (op->ih != 1 || op->oh != 1 || op->iw != op->ow || vocab == 0 ||
                (op->kind == CTCARGMAX && op->oc != 2) || !mul_ok(columns, op->ic, &wl) ||
                wl != op->w1 || op->b1 != columns) {
                fail(err, el, "op %zu invalid CTC head", i); return 0;
            }
            break;
        }
        case LAYERNORM:
            if (op->oc * 2 + 1 != op->w1) { fail(err, el, "op %zu needs gamma, beta and epsilon", i); return 0; }
            break;
        case ATTENTION:
            if (op->ih != 1 || op->oh != 1 || op->iw != op->ow || op->oc * 3 != op->ic || op->n2 == 0 ||
                op->oc % op->n2 != 0 || op->w1 != 1 || op->iw > MAX_SCRATCH_FLOATS / op->iw) {
                fail(err, el, "op %zu invalid attention shape", i); return 0;
            }
            break;
        case UPSAMPLE: case UPSAMPLEADD:
            if (op->ic != op->oc || op->sh == 0 || op->sw == 0 || op->ih * op->sh != op->oh || op->iw * op->sw != op->ow) {
                fail(err, el, "op %zu invalid upsampling", i); return 0;
            }
            break;
        case CONVTRANSPOSE: {
            size_t cols = op->kh * op->kw * op->oc;
            if (op->kh == 0 || op->kw == 0 || op->sh != op->kh || op->sw != op->kw || op->pt || op->pb ||
                op->pl || op->pr || op->ih * op->kh != op->oh || op->iw * op->kw != op->ow ||
                cols * op->ic != op->w1 || (op->b1 != 0 && op->b1 != cols)) {
                fail(err, el, "op %zu invalid transposed convolution", i); return 0;
            }
            break;
        }
        default: break;
        }
        if ((op->kind == ADD || op->kind == CHANNELMUL || op->kind == LAYERNORM) &&
            (op->ih != op->oh || op->iw != op->ow || op->ic != op->oc)) {
            fail(err, el, "op %zu elementwise input/output shapes differ", i); return 0;
        }
        if (op->kind == AVGPOOL &&
            (op->ic != op->oc || op->pt || op->pb || op->pl || op->pr || op->kh > op->ih || op->kw > op->iw ||
             op->oh != (op->ih - op->kh) / op->sh + 1 || op->ow != (op->iw - op->kw) / op->sw + 1)) {
            fail(err, el, "op %zu average pool requires complete valid windows", i); return 0;
        }
        if (op->kind == MAXPOOL) {
            if (op->ic != op->oc || op->pt != 0 || op->pl != 0) { fail(err, el, "op %zu maxpool changes channels or requests unsupported padding", i); return 0; }
            if ((op->oh - 1) * op->sh >= op->ih || (op->ow - 1) * op->sw >= op->iw) { fail(err, el, "op %zu maxpool contains an empty output window", i); return 0; }
        }
        if (is_pointwise(op) && (op->ih != op->oh || op->iw != op->ow)) { fail(err, el, "op %zu unit-stride pointwise changes spatial dimensions", i); return 0; }
        if (op->x >= m->nbuf || m->pool[op->x] < in_len) { fail(err, el, "op %zu reads past its input buffer", i); return 0; }
        if (op->y >= m->nbuf || m->pool[op->y] < out_len) { fail(err, el, "op %zu writes past its output buffer", i); return 0; }
        size_t s2;
        int has2 = second_of(op, &s2);
        if (op->y == op->x || (has2 && s2 == op->y)) { fail(err, el, "op %zu writes the buffer it reads", i); return 0; }
        if (has2) {
            size_t need;
            switch (op->kind) {
            case ADD: case UPSAMPLEADD: need = out_len; break;
            case CONCATC: need = op->oh * op->ow * op->n2; break;
            case CONV: need = op->ih * op->iw * op->n2; break;
            default: need = op->oc;
            }
            if (s2 >= m->nbuf || m->pool[s2] < need) { fail(err, el, "op %zu reads past its second input buffer", i); return 0; }
        }
        if (op->kind == CONV || op->kind == DWCONV) {
            size_t taps = op->kh * op->kw, want;
            if (op->n2 > 0 && (op->kind == DWCONV || is_pointwise(op))) { fail(err, el, "op %zu reads a second input it cannot", i); return 0; }
            if (op->kind == DWCONV) {
                if (op->ic != op->oc) { fail(err, el, "op %zu is depthwise but changes channel count", i); return 0; }
                want = taps * op->oc;
            } else {
                want = (op->ic + op->n2) * taps * op->oc;
            }
            if (op->w1 != want) { fail(err, el, "op %zu: %zu weights for a shape needing %zu", i, op->w1, want); return 0; }
            if (op->b1 != 0 && op->b1 != op->oc) { fail(err, el, "op %zu has a bias of the wrong length", i); return 0; }
        }
        int weighted = op->kind == CONV || op->kind == DWCONV || op->kind == LAYERNORM ||
                       op->kind == ATTENTION || op->kind == CTCHEAD || op->kind == CTCARGMAX ||
                       op->kind == CONVTRANSPOSE;
        if (!weighted && (op->w1 || op->b1)) { fail(err, el, "op %zu has weights it does not use", i); return 0; }
        if (op->fused != F_NONE && !(op->kind == CONV || op->kind == DWCONV || op->kind == ADD || op->kind == CONVTRANSPOSE)) {
            fail(err, el, "op %zu has an invalid folded activation", i); return 0;
        }
        size_t blocks[2][2] = {{op->w0, op->w1}, {op->b0, op->b1}};
        for (int b = 0; b < 2; b++) {
            if (!blocks[b][1]) continue;
            if (blocks[b][0] > SIZE_MAX - blocks[b][1] || blocks[b][0] + blocks[b][1] > m->nweights) {
                fail(err, el, "op %zu: a weight block reaches past the weights", i); return 0;
            }
        }
    }
    return 1;
}

static int alloc_buffers(oracle_model *m, char *err, size_t el) {
    for (size_t s = 0; s < m->nbuf; s++) {
        size_t need = m->pool[s] ? m->pool[s] : 1;
        if (m->cap[s] < need) {
            float *p = (float *)calloc(need, sizeof(float));
            if (!p) { fail(err, el, "cannot allocate %zu bytes of scratch", need * 4); return 0; }
            free(m->bufs[s]);
            m->bufs[s] = p;
            m->cap[s] = need;
        }
    }
    return 1;
}

void oracle_free(oracle_model *m) {
    if (!m) return;
    if (m->bufs)
        for (size_t s = 0; s < m->nbuf; s++) free(m->bufs[s]);
    free(m->bufs); free(m->cap); free(m->pool); free(m->ops);
    free(m->out_slot); free(m->out_n); free(m->weights);
    free(m);
}

int oracle_set_size(oracle_model *m, size_t height, size_t width, char *err, size_t el) {
    size_t oh = m->in_h, ow = m->in_w;
    if (!derive_shapes(m, height, width, err, el) || !check_plan(m, err, el)) {
        char scratch[8];
        derive_shapes(m, oh, ow, scratch, sizeof scratch);
        return 1;
    }
    if (!alloc_buffers(m, err, el)) {
        char scratch[8];
        derive_shapes(m, oh, ow, scratch, sizeof scratch);
        return 1;
    }
    return 0;
}

/* plan.rs:303-365 and 819-842 */
int oracle_load(const uint8_t *bytes, size_t len, oracle_model **out, char *err, size_t el) {
    *out = NULL;
    if (len < 8 || memcmp(bytes, "PPOCRPL1", 8) != 0) { fail(err, el, "unsupported plan: not a ppocr-native plan"); return 1; }
    size_t at = 8;
#define NEXT(dst)                                                                           \
    do {                                                                                    \
        if (at + 4 > len) { fail(err, el, "invalid plan: the description is truncated"); goto bad; } \
        uint32_t w_;                                                                        \
        memcpy(&w_, bytes + at, 4);                                                         \
        at += 4;                                                                            \
        (dst) = w_;                                                                         \
    } while (0)
    oracle_model *m = (oracle_model *)calloc(1, sizeof *m);
    size_t nbuf, nout, nops;
    NEXT(m->in_slot); NEXT(m->in_h); NEXT(m->in_w); NEXT(m->in_c);
    NEXT(nbuf); NEXT(nout); NEXT(nops);
    /* Counts are read item by item, so a count past the file fails on the
     * first missing word instead of allocating. */
    if (nout > (len - at) / 4 || nops > (len - at) / 4 / OP_FIELDS + 1) {
        fail(err, el, "invalid plan: the description is truncated"); goto bad;
    }
    m->nout = nout;
    m->out_slot = (size_t *)calloc(nout ? nout : 1, sizeof(size_t));
    m->out_n = (size_t *)calloc(nout ? nout : 1, sizeof(size_t));
    for (size_t k = 0; k < nout; k++) NEXT(m->out_slot[k]);
    m->ops = (op_t *)calloc(nops ? nops : 1, sizeof(op_t));
    m->nops = nops;
    for (size_t i = 0; i < nops; i++) {
        size_t f[OP_FIELDS];
        for (int j = 0; j < OP_FIELDS; j++) NEXT(f[j]);
        if (f[0] >= KIND_COUNT) { fail(err, el, "unsupported plan: operation kind %zu is unknown", f[0]); goto bad; }
        if (f[1] >= FUSED_COUNT) { fail(err, el, "unsupported plan: activation %zu is unknown", f[1]); goto bad; }
        op_t *op = &m->ops[i];
        op->kind = (int)f[0]; op->fused = (int)f[1];
        op->x = f[2]; op->x2 = f[3]; op->y = f[4]; op->ic = f[5]; op->oc = f[6];
        op->kh = f[7]; op->kw = f[8]; op->sh = f[9]; op->sw = f[10];
        op->pt = (long)f[11]; op->pb = (long)f[12]; op->pl = (long)f[13]; op->pr = (long)f[14];
        op->n2 = f[15]; op->w0 = f[16]; op->w1 = f[17]; op->b0 = f[18]; op->b1 = f[19];
    }
#undef NEXT
    if (nbuf == 0 || nbuf > nops + 1) { fail(err, el, "invalid plan: %zu buffers for %zu operations", nbuf, nops); goto bad; }
    m->nbuf = nbuf;
    size_t start = (at + 63) / 64 * 64;
    if (start > len) { fail(err, el, "invalid plan: the plan ends before its weights"); goto bad; }
    size_t raw = len - start;
    if (raw % 4) { fail(err, el, "invalid plan: the weights are %zu bytes, not a whole number of floats", raw); goto bad; }
    m->nweights = raw / 4;
    m->weights = (float *)malloc((m->nweights ? m->nweights : 1) * sizeof(float));
    for (size_t i = 0; i < m->nweights; i++) {
        uint32_t b;
        memcpy(&b, bytes + start + 4 * i, 4);
        if ((b & 0x7f800000u) == 0) b &= 0x80000000u; /* subnormal to signed zero */
        if ((b & 0x7f800000u) == 0x7f800000u) { fail(err, el, "invalid plan: the weights hold a non-finite value at float %zu", i); goto bad; }
        m->weights[i] = f_of(b);
    }
    m->pool = (size_t *)calloc(nbuf, sizeof(size_t));
    m->bufs = (float **)calloc(nbuf, sizeof(float *));
    m->cap = (size_t *)calloc(nbuf, sizeof(size_t));
    {
        char *e2 = err;
        size_t l2 = el;
        char tmp[256];
        if (!derive_shapes(m, m->in_h, m->in_w, tmp, sizeof tmp) || !check_plan(m, tmp, sizeof tmp)) {
            fail(e2, l2, "invalid plan: %s", tmp);
            goto bad;
        }
    }
    for (size_t i = 0; i < nops; i++) {
        const op_t *op = &m->ops[i];
        if (op->kind == LAYERNORM && !(m->weights[op->w0 + 2 * op->oc] > 0.0f)) {
            fail(err, el, "invalid plan: layer normalization epsilon is not positive"); goto bad;
        }
    }
    if (!alloc_buffers(m, err, el)) goto bad;
    *out = m;
    return 0;
bad:
    oracle_free(m);
    return 1;
}

/* ------------------------------------------------------------ accessors */

void oracle_input_shape(const oracle_model *m, size_t *hwc) {
    hwc[0] = m->in_h; hwc[1] = m->in_w; hwc[2] = m->in_c;
}
float *oracle_input(oracle_model *m) { return m->bufs[m->in_slot]; }
size_t oracle_output_count(const oracle_model *m) { return m->nout; }
const float *oracle_output(const oracle_model *m, size_t k, size_t *n) {
    *n = m->out_n[k];
    return m->bufs[m->out_slot[k]];
}
size_t oracle_op_count(const oracle_model *m) { return m->nops; }
/* kind, fused, ih, iw, ic, oh, ow, oc, kh, kw, sh, sw, n2, x, x2, y */
void oracle_op_info(const oracle_model *m, size_t i, size_t *f) {
    const op_t *op = &m->ops[i];
    size_t v[16] = {(size_t)op->kind, (size_t)op->fused, op->ih, op->iw, op->ic, op->oh, op->ow, op->oc,
                    op->kh, op->kw, op->sh, op->sw, op->n2, op->x, op->x2, op->y};
    memcpy(f, v, sizeof v);
}
size_t oracle_pool_floats(const oracle_model *m, size_t slot) { return m->pool[slot]; }
const float *oracle_buffer(const oracle_model *m, size_t slot) { return m->bufs[slot]; }

/* ------------------------------------------------------------ operations */

static int g_threads = 1;

/* Pointwise layer: conv.rs:128-143 and kernels/pointwise.rs. Calls of
 * rows_per_group rows; within a call, outputs of a multiple-of-16 width
 * start from the bias except the last count % 4 pixels, every other output
 * adds it last (pointwise.rs:46-130, 584-760). Columns below co / 8 * 8 sum
 * with fused multiply-adds; the rest multiply and add separately (the
 * scalar tail columns of pw_any and matvec_t, pointwise.rs:723-743,
 * matvec.rs:84-90). */
static void pointwise(const op_t *op, const float *x, float *y, const float *w, const float *b) {
    size_t ci = op->ic, co = op->oc;
    size_t rows = (48 + op->ow - 1) / op->ow;
    if (rows > op->oh) rows = op->oh;
    size_t groups = (op->oh + rows - 1) / rows;
    long gi;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (gi = 0; gi < (long)groups; gi++) {
        size_t first = (size_t)gi * rows;
        size_t nr = op->oh - first < rows ? op->oh - first : rows;
        size_t count = nr * op->ow;
        size_t bias_first = co % 16 == 0 ? count / 4 * 4 : 0;
        size_t fused = co / 8 * 8;
        /* Four pixels at a time, every output's chain in input order; the
         * innermost loops run across outputs (independent chains). */
        float *acc = (float *)malloc(4 * co * sizeof(float));
        for (size_t p0 = 0; p0 < count; p0 += 4) {
            size_t np = count - p0 < 4 ? count - p0 : 4;
            for (size_t q = 0; q < np; q++)
                for (size_t j = 0; j < co; j++) acc[q * co + j] = (b && p0 + q < bias_first) ? b[j] : 0.0f;
            for (size_t i = 0; i < ci; i++) {
                const float *wi = w + i * co;
                for (size_t q = 0; q < np; q++) {
                    const float xi = x[(first * op->ow + p0 + q) * ci + i];
                    float *a = acc + q * co;
                    for (size_t j = 0; j < fused; j++) a[j] = fmaf(wi[j], xi, a[j]);
                    for (size_t j = fused; j < co; j++) a[j] = a[j] + xi * wi[j];
                }
            }
            for (size_t q = 0; q < np; q++) {
                float *yp = y + (first * op->ow + p0 + q) * co;
                for (size_t j = 0; j < co; j++) {
                    float v = acc[q * co + j];
                    if (b && p0 + q >= bias_first) v = v + b[j];
                    yp[j] = oracle_act(v, op->fused);
                }
            }
        }
        free(acc);
    }
}

/* One tap's products into the accumulators: fused for the columns below
 * `fused`, multiply then add for the rest. */
static inline void tap_acc(float *acc, const float *tap, const float *px, size_t n, size_t co,
                           size_t fused) {
    for (size_t i = 0; i < n; i++) {
        const float *ti = tap + i * co;
        const float xi = px[i];
        for (size_t j = 0; j < fused; j++) acc[j] = fmaf(ti[j], xi, acc[j]);
        for (size_t j = fused; j < co; j++) acc[j] = acc[j] + xi * ti[j];
    }
}

/* Windowed dense convolution over one or two sources: kernels/dense.rs:38-147,
 * taps [ky][kx], then the channels of x and of x2. The bias comes first for a
 * multiple-of-16 width except the row's last ow % 4 pixels, else last;
 * columns below co / 8 * 8 use fused multiply-adds. The RGB stem (three
 * channels, one input, conv.rs:13-14, 146-236) starts every output from its
 * bias. */
static void conv_window(const op_t *op, const float *x, const float *x2, float *y, const float *w,
                        const float *b) {
    size_t ct = op->ic + op->n2, co = op->oc;
    size_t fused = co / 8 * 8;
    int stem = op->ic == 3 && op->n2 == 0;
    size_t first_end = stem ? op->ow : (co % 16 == 0 ? op->ow - op->ow % 4 : 0);
    long oy;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (oy = 0; oy < (long)op->oh; oy++) {
        float *acc = (float *)malloc(co * sizeof(float));
        for (size_t ox = 0; ox < op->ow; ox++) {
            int bias_first = ox < first_end;
            for (size_t j = 0; j < co; j++) acc[j] = (b && bias_first) ? b[j] : 0.0f;
            for (size_t ky = 0; ky < op->kh; ky++) {
                long iy = (long)oy * (long)op->sh + (long)ky - op->pt;
                if (iy < 0 || iy >= (long)op->ih) continue;
                for (size_t kx = 0; kx < op->kw; kx++) {
                    long ix = (long)ox * (long)op->sw + (long)kx - op->pl;
                    if (ix < 0 || ix >= (long)op->iw) continue;
                    const float *tap = w + (ky * op->kw + kx) * ct * co;
                    const float *p1 = x + ((size_t)iy * op->iw + (size_t)ix) * op->ic;
                    tap_acc(acc, tap, p1, op->ic, co, fused);
                    if (op->n2) {
                        const float *p2 = x2 + ((size_t)iy * op->iw + (size_t)ix) * op->n2;
                        tap_acc(acc, tap + op->ic * co, p2, op->n2, co, fused);
                    }
                }
            }
            float *yp = y + ((size_t)oy * op->ow + ox) * co;
            for (size_t j = 0; j < co; j++) {
                float v = (b && !bias_first) ? acc[j] + b[j] : acc[j];
                yp[j] = oracle_act(v, op->fused);
            }
        }
        free(acc);
    }
}

/* kernels/depthwise.rs:93-217: bias seed, taps row-major, padding skipped. */
static void depthwise(const op_t *op, const float *x, float *y, const float *w, const float *b) {
    size_t c = op->oc;
    long oy;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (oy = 0; oy < (long)op->oh; oy++) {
        for (size_t ox = 0; ox < op->ow; ox++) {
            /* Each channel from its bias, taps row-major; the innermost
             * loop runs across channels (independent chains). */
            float *yp = y + ((size_t)oy * op->ow + ox) * c;
            for (size_t ch = 0; ch < c; ch++) yp[ch] = b ? b[ch] : 0.0f;
            for (size_t ky = 0; ky < op->kh; ky++) {
                long iy = (long)oy * (long)op->sh + (long)ky - op->pt;
                if (iy < 0 || iy >= (long)op->ih) continue;
                for (size_t kx = 0; kx < op->kw; kx++) {
                    long ix = (long)ox * (long)op->sw + (long)kx - op->pl;
                    if (ix < 0 || ix >= (long)op->iw) continue;
                    const float *wt = w + (ky * op->kw + kx) * c;
                    const float *xt = x + ((size_t)iy * op->iw + (size_t)ix) * c;
                    for (size_t ch = 0; ch < c; ch++) yp[ch] = fmaf(wt[ch], xt[ch], yp[ch]);
                }
            }
            for (size_t ch = 0; ch < c; ch++) yp[ch] = oracle_act(yp[ch], op->fused);
        }
    }
}

/* conv.rs:404-440: the window cut at the bottom and right edges. */
static void maxpool(const op_t *op, const float *x, float *y) {
    size_t c = op->oc;
    for (size_t oy = 0; oy < op->oh; oy++)
        for (size_t ox = 0; ox < op->ow; ox++) {
            float *yp = y + (oy * op->ow + ox) * c;
            int seeded = 0;
            for (size_t ky = 0; ky < op->kh; ky++) {
                size_t iy = oy * op->sh + ky;
                if (iy >= op->ih) continue;
                for (size_t kx = 0; kx < op->kw; kx++) {
                    size_t ix = ox * op->sw + kx;
                    if (ix >= op->iw) continue;
                    const float *src = x + (iy * op->iw + ix) * c;
                    for (size_t ch = 0; ch < c; ch++) {
                        /* MAXPS keeps the first operand only when greater. */
                        if (!seeded || src[ch] > yp[ch]) yp[ch] = seeded ? src[ch] : src[ch];
                    }
                    seeded = 1;
                }
            }
        }
}

/* layers.rs:443-463 */
static void avgpool(const op_t *op, const float *x, float *y) {
    float divisor = (float)(op->kh * op->kw);
    for (size_t oy = 0; oy < op->oh; oy++)
        for (size_t ox = 0; ox < op->ow; ox++) {
            float *out = y + (oy * op->ow + ox) * op->oc;
            for (size_t ch = 0; ch < op->oc; ch++) out[ch] = 0.0f;
            for (size_t ky = 0; ky < op->kh; ky++)
                for (size_t kx = 0; kx < op->kw; kx++) {
                    const float *src = x + ((oy * op->sh + ky) * op->iw + ox * op->sw + kx) * op->ic;
                    for (size_t ch = 0; ch < op->oc; ch++) out[ch] += src[ch];
                }
            for (size_t ch = 0; ch < op->oc; ch++) out[ch] /= divisor;
        }
}

/* layers.rs:391-406: pixels summed in order in f64, then divided. */
static void channel_mean(const float *x, float *y, size_t pixels, size_t c) {
    double *sums = (double *)calloc(c, sizeof(double));
    for (size_t p = 0; p < pixels; p++)
        for (size_t ch = 0; ch < c; ch++) sums[ch] += (double)x[p * c + ch];
    for (size_t ch = 0; ch < c; ch++) y[ch] = (float)(sums[ch] / (double)pixels);
    free(sums);
}

/* layers.rs:467-479 */
static void layer_norm(const float *x, float *y, const float *w, size_t pixels, size_t c) {
    const float *gamma = w, *beta = w + c;
    float eps = w[2 * c];
    for (size_t p = 0; p < pixels; p++) {
        const float *v = x + p * c;
        float s = 0.0f;
        for (size_t i = 0; i < c; i++) s += v[i];
        float mean = s / (float)c;
        float q = 0.0f;
        for (size_t i = 0; i < c; i++) {
            float d = v[i] - mean;
            q += d * d;
        }
        float var = q / (float)c;
        float r = sqrtf(var + eps);
        for (size_t i = 0; i < c; i++) y[p * c + i] = (v[i] - mean) / r * gamma[i] + beta[i];
    }
}

static inline float max_lane(float a, float b) { return a > b ? a : b; }

/* Softmax of one row: layers.rs:273-294 with FMA exp. */
static void softmax_row(float *y, size_t n) {
    size_t body = n / LANES * LANES;
    float lanes[LANES];
    for (int l = 0; l < LANES; l++) lanes[l] = -INFINITY;
    for (size_t j = 0; j < body; j++) lanes[j % LANES] = max_lane(lanes[j % LANES], y[j]);
    float mx = -INFINITY;
    for (int l = 0; l < LANES; l++) mx = fmaxf(mx, lanes[l]);
    for (size_t j = body; j < n; j++) mx = fmaxf(mx, y[j]);
    float sums[LANES] = {0};
    for (size_t j = 0; j < body; j++) {
        y[j] = oracle_exp_neg(y[j] - mx);
        sums[j % LANES] += y[j];
    }
    float sum = 0.0f;
    for (int l = 0; l < LANES; l++) sum += sums[l];
    for (size_t j = body; j < n; j++) {
        y[j] = oracle_exp_neg(y[j] - mx);
        sum += y[j];
    }
    float r = 1.0f / sum;
    for (size_t j = 0; j < n; j++) y[j] *= r;
}

/* layers.rs:494-522: per head, S = (Q * scale) K^T from zero over the
 * head's dimensions (a pointwise product whose columns are the keys: fused
 * multiply-adds below t / 8 * 8 keys, multiply then add past them), softmax
 * per row, then S V from zero with FMA over the keys (its columns, the head
 * padded to a multiple of 8, are all fused). */
static void attention(const op_t *op, const float *x, float *y, float scale) {
    size_t t = op->iw, c = op->oc, heads = op->n2, hd = c / heads;
    long h;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (h = 0; h < (long)heads; h++) {
        float *q = (float *)malloc(t * hd * sizeof(float));
        float *scores = (float *)malloc(t * t * sizeof(float));
        for (size_t s = 0; s < t; s++)
            for (size_t d = 0; d < hd; d++) q[s * hd + d] = x[s * 3 * c + (size_t)h * hd + d] * scale;
        for (size_t s = 0; s < t; s++) {
            for (size_t j = 0; j < t; j++) {
                float acc = 0.0f;
                const float *k = x + j * 3 * c + c + (size_t)h * hd;
                if (j < t / 8 * 8)
                    for (size_t d = 0; d < hd; d++) acc = fmaf(k[d], q[s * hd + d], acc);
                else
                    for (size_t d = 0; d < hd; d++) acc = acc + q[s * hd + d] * k[d];
                scores[s * t + j] = acc;
            }
            softmax_row(scores + s * t, t);
        }
        for (size_t s = 0; s < t; s++)
            for (size_t d = 0; d < hd; d++) {
                float acc = 0.0f;
                for (size_t j = 0; j < t; j++)
                    acc = fmaf(x[j * 3 * c + 2 * c + (size_t)h * hd + d], scores[s * t + j], acc);
                y[s * c + (size_t)h * hd + d] = acc;
            }
        free(q);
        free(scores);
    }
}

/* The CTC head's per-pixel softmax state over 16-column panels, 8 lanes:
 * layers.rs:753-832. Lane l holds columns 16j + l and 16j + 8 + l. */
typedef struct { float m[LANES], sum[LANES], best[LANES]; } head_state;

static void head_init(head_state *s) {
    for (int l = 0; l < LANES; l++) { s->m[l] = -INFINITY; s->sum[l] = 0.0f; s->best[l] = 0.0f; }
}

static void head_panel(head_state *s, const float *logits16, size_t j) {
    for (int l = 0; l < LANES; l++) {
        float a0 = logits16[l], a1 = logits16[LANES + l], m = s->m[l];
        float top = max_lane(a0, a1);
        float grown = max_lane(m, top);
        float sum = s->sum[l] * oracle_exp_neg(m - grown);
        sum += oracle_exp_neg(a0 - grown);
        sum += oracle_exp_neg(a1 - grown);
        s->m[l] = grown;
        s->sum[l] = sum;
        if (top > m) s->best[l] = (float)(j * PANEL + (size_t)l + (a1 > a0 ? LANES : 0));
    }
}

static void head_finish(const head_state *s, float *best, float *max_out, float *r) {
    float mx = -INFINITY;
    for (int l = 0; l < LANES; l++) mx = fmaxf(mx, s->m[l]);
    float sum = 0.0f;
    for (int l = 0; l < LANES; l++) sum += s->sum[l] * oracle_exp_neg(s->m[l] - mx);
    float b = INFINITY;
    for (int l = 0; l < LANES; l++)
        if (s->m[l] == mx) b = fminf(b, s->best[l]);
    *best = b;
    *max_out = mx;
    *r = 1.0f / sum;
}

/* layers.rs:707-811: logits from the bias with FMA over ci per column. */
static void ctc_head(const op_t *op, const float *x, float *y, const float *w, const float *b, int probs) {
    size_t t = op->iw, ci = op->ic, vocab = probs ? op->oc : op->n2;
    size_t panels = (vocab + PANEL - 1) / PANEL;
    long p;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (p = 0; p < (long)t; p++) {
        head_state s;
        head_init(&s);
        const float *xp = x + (size_t)p * ci;
        for (size_t j = 0; j < panels; j++) {
            const float *panel = w + j * ci * PANEL;
            float logits[PANEL];
            for (size_t col = 0; col < PANEL; col++) logits[col] = b[j * PANEL + col];
            for (size_t i = 0; i < ci; i++)
                for (size_t col = 0; col < PANEL; col++)
                    logits[col] = fmaf(panel[i * PANEL + col], xp[i], logits[col]);
            head_panel(&s, logits, j);
            if (probs) {
                size_t n = vocab - j * PANEL < PANEL ? vocab - j * PANEL : PANEL;
                memcpy(y + (size_t)p * vocab + j * PANEL, logits, n * sizeof(float));
            }
        }
        float best, mx, r;
        head_finish(&s, &best, &mx, &r);
        if (probs) {
            for (size_t k = 0; k < vocab; k++) {
                float *v = y + (size_t)p * vocab + k;
                *v = oracle_exp_neg(*v - mx) * r;
            }
        } else {
            y[2 * p] = best;
            y[2 * p + 1] = r;
        }
    }
}

/* layers.rs:600-680: each input row's blocks by one pointwise call of iw
 * pixels (kernels/pointwise.rs bias rule: first for a multiple-of-16 column
 * count except the last iw % 4 pixels, else last), written to each pixel's
 * kh x kw output pixels, then the activation. */
static void conv_transpose(const op_t *op, const float *x, float *y, const float *w, const float *b) {
    size_t cols = op->kh * op->kw * op->oc, ci = op->ic;
    size_t bias_first = cols % 16 == 0 ? op->iw / 4 * 4 : 0;
    long iy;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (iy = 0; iy < (long)op->ih; iy++) {
        for (size_t ix = 0; ix < op->iw; ix++) {
            const float *xp = x + ((size_t)iy * op->iw + ix) * ci;
            for (size_t n = 0; n < cols; n++) {
                float acc = (b && ix < bias_first) ? b[n] : 0.0f;
                if (n < cols / 8 * 8)
                    for (size_t i = 0; i < ci; i++) acc = fmaf(w[i * cols + n], xp[i], acc);
                else
                    for (size_t i = 0; i < ci; i++) acc = acc + xp[i] * w[i * cols + n];
                if (b && ix >= bias_first) acc = acc + b[n];
                size_t tap = n / op->oc, o = n % op->oc;
                size_t ky = tap / op->kw, kx = tap % op->kw;
                size_t oy = (size_t)iy * op->kh + ky, ox = ix * op->kw + kx;
                y[(oy * op->ow + ox) * op->oc + o] = oracle_act(acc, op->fused);
            }
        }
    }
}

static void run_op(oracle_model *m, const op_t *op) {
    const float *x = m->bufs[op->x];
    const float *x2 = m->bufs[op->x2];
    float *y = m->bufs[op->y];
    const float *wt = op->w1 ? m->weights + op->w0 : NULL;
    const float *bs = op->b1 ? m->weights + op->b0 : NULL;
    size_t n = op->oh * op->ow * op->oc;
    switch (op->kind) {
    case CONV:
        if (is_pointwise(op)) pointwise(op, x, y, wt, bs);
        else conv_window(op, x, op->n2 ? x2 : NULL, y, wt, bs);
        break;
    case DWCONV: depthwise(op, x, y, wt, bs); break;
    case ADD:
        for (size_t i = 0; i < n; i++) y[i] = oracle_act(x[i] + x2[i], op->fused);
        break;
    case CHANNELMUL:
        for (size_t p = 0; p < op->oh * op->ow; p++)
            for (size_t ch = 0; ch < op->oc; ch++) y[p * op->oc + ch] = x[p * op->oc + ch] * x2[ch];
        break;
    case MAXPOOL: maxpool(op, x, y); break;
    case AVGPOOL: avgpool(op, x, y); break;
    case CONCATC:
        for (size_t p = 0; p < op->oh * op->ow; p++) {
            memcpy(y + p * op->oc, x + p * op->ic, op->ic * sizeof(float));
            memcpy(y + p * op->oc + op->ic, x2 + p * op->n2, op->n2 * sizeof(float));
        }
        break;
    case LAYERNORM: layer_norm(x, y, wt, op->oh * op->ow, op->oc); break;
    case ATTENTION: attention(op, x, y, wt[0]); break;
    case MEAN: channel_mean(x, y, op->ih * op->iw, op->ic); break;
    case CTCHEAD: ctc_head(op, x, y, wt, bs, 1); break;
    case CTCARGMAX: ctc_head(op, x, y, wt, bs, 0); break;
    case UPSAMPLE:
    case UPSAMPLEADD:
        for (size_t oy = 0; oy < op->oh; oy++)
            for (size_t ox = 0; ox < op->ow; ox++) {
                const float *src = x + ((oy / op->sh) * op->iw + ox / op->sw) * op->oc;
                float *dst = y + (oy * op->ow + ox) * op->oc;
                if (op->kind == UPSAMPLE) {
                    memcpy(dst, src, op->oc * sizeof(float));
                } else {
                    const float *add = x2 + (oy * op->ow + ox) * op->oc;
                    for (size_t ch = 0; ch < op->oc; ch++) dst[ch] = add[ch] + src[ch];
                }
            }
        break;
    case CONVTRANSPOSE: conv_transpose(op, x, y, wt, bs); break;
    }
}

/* Run the plan once over the input buffer. */
void oracle_run(oracle_model *m, int threads) {
    g_threads = threads > 0 ? threads : 1;
    for (size_t i = 0; i < m->nops; i++) run_op(m, &m->ops[i]);
}

/* Run the operations [first, last) only; the buffers they read must hold
 * what earlier operations wrote. */
void oracle_run_ops(oracle_model *m, size_t first, size_t last, int threads) {
    g_threads = threads > 0 ? threads : 1;
    for (size_t i = first; i < last && i < m->nops; i++) run_op(m, &m->ops[i]);
}

/* ------------------------------------------------- standalone layer forms */

/* y = x1 + x2, then the activation `fused`. */
void oracle_add(const float *a, const float *b, float *y, size_t n, int fused) {
    for (size_t i = 0; i < n; i++) y[i] = oracle_act(a[i] + b[i], fused);
}
/* y = x1 * x2, elementwise. */
void oracle_mul(const float *a, const float *b, float *y, size_t n) {
    for (size_t i = 0; i < n; i++) y[i] = a[i] * b[i];
}
/* y = act(x). */
void oracle_activation(const float *x, float *y, size_t n, int fused) {
    for (size_t i = 0; i < n; i++) y[i] = oracle_act(x[i], fused);
}
void oracle_channel_mean(const float *x, float *y, size_t pixels, size_t c) {
    channel_mean(x, y, pixels, c);
}
void oracle_channel_mul(const float *x, const float *g, float *y, size_t pixels, size_t c) {
    for (size_t p = 0; p < pixels; p++)
        for (size_t ch = 0; ch < c; ch++) y[p * c + ch] = x[p * c + ch] * g[ch];
}
void oracle_layer_norm(const float *x, const float *w, float *y, size_t rows, size_t c) {
    layer_norm(x, y, w, rows, c);
}
void oracle_softmax_row(float *y, size_t n) { softmax_row(y, n); }
/* Each row's first index of the maximum, as a float, and 1 / sum of
 * exp(logit - max), through the CTC head's lane state (a row of `cols`
 * values is taken in 16-column panels, padded with -1e30). */
void oracle_row_argmax(const float *x, float *y, size_t rows, size_t cols, int threads) {
    g_threads = threads > 0 ? threads : 1;
    long r;
#pragma omp parallel for schedule(static) num_threads(g_threads)
    for (r = 0; r < (long)rows; r++) {
        head_state s;
        head_init(&s);
        const float *row = x + (size_t)r * cols;
        for (size_t j = 0; j * PANEL < cols; j++) {
            float logits[PANEL];
            for (size_t k = 0; k < PANEL; k++) {
                size_t col = j * PANEL + k;
                logits[k] = col < cols ? row[col] : -1e30f;
            }
            head_panel(&s, logits, j);
        }
        float best, mx, rr;
        head_finish(&s, &best, &mx, &rr);
        y[2 * r] = best;
        y[2 * r + 1] = rr;
    }
}
int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
