/*
 * ppocr_hip: an MI355X (gfx950) backend for ppocr-native's inference engine.
 *
 * C ABI of the drop-in for the engine's GPU model (src/engine/gpu/mod.rs,
 * `GpuModel`). It reads the engine's own PPOCRPL1 plan files and runs them in
 * fp32 with hand-written HIP kernels. Every entry point returns 0 on success
 * or a nonzero code with a message in `err` (NUL-terminated, truncated to
 * `err_len`); none aborts the process. A model is used from one thread at a
 * time; different models may be used on different threads.
 */
#ifndef PPOCR_HIP_H
#define PPOCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ppocr_gpu_model ppocr_gpu_model;

/* Replaces `GpuModel::load` (src/engine/gpu/mod.rs:113-163): read and check a
 * plan, upload its weights, build the dispatch steps, and set one lane at the
 * plan's stored input size. */
int ppocr_gpu_load(const char *plan_path, ppocr_gpu_model **out, char *err, size_t err_len);

/* `GpuModel::load` from plan bytes already in memory (the same checks as
 * `Plan::parse`, src/engine/plan.rs:303-365). */
int ppocr_gpu_load_bytes(const void *bytes, size_t len, ppocr_gpu_model **out, char *err,
                         size_t err_len);

/* Replaces dropping a `GpuModel` (src/engine/gpu/vk.rs:564-574): waits for the
 * device, then frees every buffer. NULL is accepted. */
void ppocr_gpu_free(ppocr_gpu_model *model);

/* Replaces `GpuModel::device` (src/engine/gpu/mod.rs:166): the GPU's name;
 * valid for the model's lifetime. */
const char *ppocr_gpu_device(const ppocr_gpu_model *model);

/* Replaces `GpuModel::integrated` (src/engine/gpu/mod.rs:171): 1 when the GPU
 * shares the CPU's memory, else 0 (0 on MI355X). */
int ppocr_gpu_integrated(const ppocr_gpu_model *model);

/* Replaces `GpuModel::set_input_size` (src/engine/gpu/mod.rs:178): one lane of
 * `height` x `width`. On error the model keeps no lanes (set sizes again). */
int ppocr_gpu_set_input_size(ppocr_gpu_model *model, size_t height, size_t width, char *err,
                             size_t err_len);

/* Replaces `GpuModel::set_sizes` (src/engine/gpu/mod.rs:191-230): one lane per
 * (height, width) pair of `hw` (2 * n_lanes values). Lanes of equal size run
 * as one batch. On error only the first lanes that could be set stay valid
 * (`ppocr_gpu_lanes` says how many). */
int ppocr_gpu_set_sizes(ppocr_gpu_model *model, const size_t *hw, size_t n_lanes, char *err,
                        size_t err_len);

/* Replaces `GpuModel::max_lanes` (src/engine/gpu/mod.rs:184): the most lanes one
 * run takes, bounded by memory rather than descriptors: lanes of the first
 * lane's size whose buffers (all at once, plus a quarter) fit in 80 % of the
 * device's memory, and whose largest buffer over all lanes has fewer than
 * 2^31 elements. ppocr_gpu_set_sizes refuses more lanes with a message. */
size_t ppocr_gpu_max_lanes(const ppocr_gpu_model *model);

/* Lanes the next run computes (no reference counterpart: the Rust model keeps
 * it private as `active`, src/engine/gpu/mod.rs:92). */
size_t ppocr_gpu_lanes(const ppocr_gpu_model *model);

/* Replaces `GpuModel::lane_input_mut` / `input_mut` (src/engine/gpu/mod.rs:234-244):
 * lane `lane`'s image, HWC f32, `*len` floats, in pinned host memory owned by
 * the model; valid until the next set_sizes. NULL for a lane out of range. */
float *ppocr_gpu_lane_input(ppocr_gpu_model *model, size_t lane, size_t *len);

/* Replaces `GpuModel::lane_output` / `output` (src/engine/gpu/mod.rs:248-256):
 * result `index` of lane `lane` from the last run (detector: H*W
 * probabilities; argmax recogniser: [T][2] = best class as f32, probability). */
const float *ppocr_gpu_lane_output(const ppocr_gpu_model *model, size_t lane, size_t index,
                                   size_t *len);

/* Results a run produces per lane (`Model::output_count`,
 * src/engine/mod.rs:1236). */
size_t ppocr_gpu_output_count(const ppocr_gpu_model *model);

/* Replaces `GpuModel::run` (src/engine/gpu/mod.rs:259-290): copy every lane's
 * input to the device, run every step, copy the results back; synchronous. */
int ppocr_gpu_run(ppocr_gpu_model *model, char *err, size_t err_len);

/* --- Measurement entry points (no reference counterpart: the Vulkan path has
 * no timestamps, src/engine/gpu/vk.rs). ------------------------------------ */

/* Copy every lane's input to the device now (synchronous). */
int ppocr_gpu_upload(ppocr_gpu_model *model, char *err, size_t err_len);

/* Run every step `repeats` times on the inputs already on the device, without
 * host copies, and wait. With `ms` non-NULL, `*ms` receives the device time of
 * all repeats measured with HIP events on the model's stream. */
int ppocr_gpu_run_resident(ppocr_gpu_model *model, int repeats, float *ms, char *err,
                           size_t err_len);

/* Copy every lane's results back to the host now (synchronous). */
int ppocr_gpu_download(ppocr_gpu_model *model, char *err, size_t err_len);

/* The model's HIP stream, as a hipStream_t. */
void *ppocr_gpu_stream(ppocr_gpu_model *model);

/* Device-resident input, for a caller that prepares the input on the GPU
 * (no Vulkan counterpart: there the worker writes `lane_input_mut`'s mapped
 * memory on the CPU, ocr.rs:227). The device address of `lane`'s input
 * (`*len` floats, HWC, the layout of `ppocr_gpu_lane_input`), valid until
 * the next set_sizes; write it in order on `ppocr_gpu_stream`. */
float *ppocr_gpu_lane_input_device(ppocr_gpu_model *model, size_t lane, size_t *len);

/* `ppocr_gpu_run` without the host-to-device copy: the forward over the
 * device-resident inputs, then every lane's results to the host buffers of
 * `ppocr_gpu_lane_output`; synchronous. */
int ppocr_gpu_run_device(ppocr_gpu_model *model, char *err, size_t err_len);

/* The same, returning once the forward and the copies of the results are
 * queued on the model's stream; `ppocr_gpu_wait` then waits for them. The
 * host output buffers and the device inputs are in use until then. Lets one
 * thread keep several handles (a page's detector, several recogniser
 * batches) busy at once. */
int ppocr_gpu_run_device_async(ppocr_gpu_model *model, char *err, size_t err_len);
int ppocr_gpu_wait(ppocr_gpu_model *model, char *err, size_t err_len);

/* The DB threshold (src/det.rs:438, `prob > thresh` in f32) of output
 * `output`, a one-channel map, written by every later run as row bitmasks
 * beside the outputs: one launch on the GPU after the forward, 1/32 of the
 * map's bytes to the host instead of a pass over the map there. It replaces
 * the host-side threshold the reference's `boxes_from_prob` starts with
 * (src/det.rs:430-452); ppocr_db_boxes_bits takes the result. `output` < 0
 * stops it. The lanes keep their sizes (their memory is arranged again).
 * Returns 0, or 1 with a message. */
int ppocr_gpu_set_db_mask(ppocr_gpu_model *model, long output, float thresh, char *err, size_t err_len);

/* Lane `lane`'s bitmasks from the last run: `*rows` rows of `*words_per_row`
 * words, bit x % 64 of word x / 64 of a row set where the map exceeds the
 * threshold (bits past the width zero); valid until the next run or
 * set_sizes. NULL when no DB mask is set or the lane does not exist. */
const uint64_t *ppocr_gpu_lane_db_mask(const ppocr_gpu_model *model, size_t lane, size_t *words_per_row,
                                       size_t *rows);

/* Runs record their launches in a HIP graph from the second run after the
 * lanes were set, and replay it (default, `enable` 1); with 0 every run
 * launches each kernel itself. Returns 0, or 1 for a NULL model. */
int ppocr_gpu_set_graphs(ppocr_gpu_model *model, int enable);

/* Kernel launches one run makes, and launch `i`'s kernel name (valid for the
 * model's lifetime) and the plan operation it starts from. */
size_t ppocr_gpu_launch_count(const ppocr_gpu_model *model);
const char *ppocr_gpu_launch_name(const ppocr_gpu_model *model, size_t i, size_t *op);

/* The plan operations launch `i` runs: one, or for a grouped launch (layers
 * of one kind that do not depend on each other, run as one grid) each
 * member's. Writes up to `cap` of them to `ops` and returns how many there are. */
size_t ppocr_gpu_launch_ops(const ppocr_gpu_model *model, size_t i, size_t *ops, size_t cap);

/* Launch `i`'s algorithmic work for the lanes of its batch: `*flops` the
 * layer's floating-point operations, `*bytes` what it must move (inputs and
 * weights read once, outputs written once). Returns 0, or 1 for a bad index. */
int ppocr_gpu_launch_work(const ppocr_gpu_model *model, size_t i, double *flops, double *bytes);

/* Time each launch of one run separately: `ms` receives launch_count values,
 * each the mean over `repeats` back-to-back repeats of that launch alone. */
int ppocr_gpu_profile_launches(ppocr_gpu_model *model, int repeats, float *ms, char *err,
                               size_t err_len);

/* --- Layer kernels on device memory ----------------------------------------
 * The engine's elementwise and reduction layers as single kernels on device
 * pointers and a HIP stream (`stream` NULL = the default stream). They are
 * the same kernels the model launches for those layers. */

/* y = act(a + b): `Kind::Add` with its folded activation
 * (src/engine/conv.rs:75-79; `act` is a `Fused` code, 7 = hard swish). */
int ppocr_hip_add(const float *a, const float *b, float *y, size_t n, int act, void *stream);

/* y = a * b, elementwise (no reference op: the engine's products are the
 * channel gates of `Kind::Channelmul`). */
int ppocr_hip_mul(const float *a, const float *b, float *y, size_t n, void *stream);

/* y = act(x) for one folded activation code (src/engine/conv.rs:59-71). */
int ppocr_hip_activation(const float *x, float *y, size_t n, int act, void *stream);

/* Measurement helper, no counterpart in the reference: y = x over n floats
 * (n a multiple of 4, 16-byte aligned pointers) through LDS by direct
 * global-to-LDS loads, the load path of the GEMM rings and the depthwise
 * tiles; it calibrates the memory counters for kernels that load that way
 * (ppocr_hip_activation with code 0 is the plain vector-load copy). */
int ppocr_hip_copy_lds(const float *x, float *y, size_t n, void *stream);

/* `Kind::Mean` (src/engine/layers.rs:391-406): y[c] = mean over `pixels` of
 * x[p][c], summed in f64. */
int ppocr_hip_channel_mean(const float *x, float *y, size_t pixels, size_t c, void *stream);

/* `ppocr_hip_channel_mean` without any allocation: no counterpart in the
 * reference; for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). Its
 * partial sums and counters live in a device array of the library that each
 * GPU holds until the process ends (2 MiB and 4 KiB), so `c` is limited to
 * 4096 channels; larger shapes return nonzero with the reason in `err`.
 * Calls that overlap on one GPU share that array and race; calls in order
 * (one stream, or synchronised) do not. Each call zeroes the counters it
 * uses on its stream before its kernel, so one overlapped or aborted call
 * does not spoil the calls after it. Same kernel and same results, bit for
 * bit, as ppocr_hip_channel_mean. */
int ppocr_hip_channel_mean_noalloc(const float *x, float *y, size_t pixels, size_t c, void *stream, char *err,
                                   size_t err_len);

/* `Kind::Channelmul` (src/engine/kernels/elementwise.rs:178-200):
 * y[p][c] = x[p][c] * g[c]. */
int ppocr_hip_channel_mul(const float *x, const float *g, float *y, size_t pixels, size_t c,
                          void *stream);

/* `Kind::Layernorm` (src/engine/layers.rs:467-479) over `rows` rows of `c`;
 * `w` holds gamma[c], beta[c], eps. */
int ppocr_hip_layer_norm(const float *x, const float *w, float *y, size_t rows, size_t c,
                         void *stream);

/* The CTC choice over precomputed logits (src/engine/layers.rs:813-832,
 * shaders/ctc.comp): for each of `rows` rows of `cols` values, y[2r] = the
 * first column holding the maximum (as f32), y[2r+1] = 1 / sum exp(v - max). */
int ppocr_hip_row_argmax(const float *x, float *y, size_t rows, size_t cols, void *stream);

/* --- Host stages either side of the model ---------------------------------
 * CPU code in the same library: the recogniser's text from its [T][2]
 * output, and the detector's text boxes from its probability map. Each
 * reproduces the reference's results bit for bit. */

typedef struct ppocr_dictionary ppocr_dictionary;

/* Replaces `Dictionary::from_metadata` (src/rec.rs:53-79): classes = blank,
 * the lines of `text` split as Python's str.splitlines splits them, a space. */
int ppocr_dictionary_load(const char *text, size_t len, ppocr_dictionary **out, char *err, size_t err_len);
void ppocr_dictionary_free(ppocr_dictionary *d);
/* `Dictionary::len` (src/rec.rs:82-85). */
size_t ppocr_dictionary_len(const ppocr_dictionary *d);
/* `Dictionary::class` (src/rec.rs:93-96): UTF-8 bytes, `*len` of them; NULL
 * for an index out of range. */
const char *ppocr_dictionary_class(const ppocr_dictionary *d, size_t index, size_t *len);

/* Replaces `ctc_decode` (src/rec.rs:133-152): repeats collapse, blanks drop,
 * score = mean of the kept probabilities each rounded to 5 decimals (numpy's
 * pairwise f64 sum), rounded again; 0 when nothing is kept. `text` receives
 * UTF-8 and a NUL (returns 2 when `text_cap` is too small; `*text_len` then
 * says how many bytes the text needs, without the NUL). */
int ppocr_ctc_decode(const ppocr_dictionary *d, const uint32_t *best, const float *prob, size_t steps,
                     char *text, size_t text_cap, size_t *text_len, double *score, char *err, size_t err_len);
/* The same from the argmax recogniser's output as `ppocr_gpu_lane_output`
 * gives it: `steps` pairs (class as f32, probability). */
int ppocr_ctc_decode_pairs(const ppocr_dictionary *d, const float *pairs, size_t steps, char *text,
                           size_t text_cap, size_t *text_len, double *score, char *err, size_t err_len);

/* Replaces `find_contours` (src/contour.rs:44-140): the borders of the
 * nonzero pixels as cv2.findContours(RETR_LIST, CHAIN_APPROX_SIMPLE) returns
 * them. Writes the corners of all contours as (x, y) pairs into `points`
 * and each contour's corner count into `lengths`; returns 2 (with the needed
 * sizes in `*n_points` and `*n_contours`) when the buffers are too small. */
int ppocr_find_contours(const uint8_t *mask, size_t width, size_t height, int32_t *points, size_t points_cap,
                        size_t *lengths, size_t contours_cap, size_t *n_points, size_t *n_contours);

/* Replaces `min_area_rect` and `RotatedRect::points` (src/geometry.rs:
 * 207-261, 28-42): `rect` = centre x, y, width, height, angle (degrees);
 * `corners` = cv2.boxPoints, (x, y) x 4. Either may be NULL. */
int ppocr_min_area_rect(const int32_t *points, size_t n, float *rect, float *corners);

/* Replaces `unclip` (src/geometry.rs:320-410): the quad (x, y) x 4 grown by
 * area * ratio / perimeter with round joins, as pyclipper computes it;
 * `*n` points into `ring` (returns 2 when `cap` is too small). */
int ppocr_unclip(const float *quad, double ratio, int32_t *ring, size_t cap, size_t *n);

/* `DbOptions` (src/det.rs:291-321); RapidOCR's defaults are 0.3, 0.5, 1.5,
 * 1000. */
typedef struct ppocr_db_options {
  float thresh;
  double box_thresh;
  double unclip_ratio;
  size_t max_candidates;
} ppocr_db_options;

/* Replaces `boxes_from_prob` (src/det.rs:430-452): the text boxes of a
 * map_w x map_h probability map, in the pixels of a dest_w x dest_h page, in
 * reading order, each four (x, y) corners (f32) into `boxes` (8 floats a
 * box). `mask` (map_w * map_h bytes, nonzero = text) may come from
 * ppocr_hip_db_mask; NULL thresholds `prob` here. Returns 2 when `boxes_cap`
 * is too small (`*n_boxes` says how many there are). */
int ppocr_db_boxes(const float *prob, const uint8_t *mask, size_t map_w, size_t map_h, size_t dest_w,
                   size_t dest_h, const ppocr_db_options *options, float *boxes, size_t boxes_cap,
                   size_t *n_boxes, char *err, size_t err_len);

/* The same boxes (src/det.rs:430-452, the threshold at :438 already taken)
 * from the map and its threshold as row bitmasks: bit x % 64 of word
 * y * words_per_row + x / 64 is prob[y][x] > thresh, bits past map_w zero,
 * as ppocr_gpu_set_db_mask has the detector's run write them. The borders
 * are followed from the pixels where a row's bits change; `prob` is read
 * only inside the regions' bounding boxes. */
int ppocr_db_boxes_bits(const float *prob, const uint64_t *bits, size_t words_per_row, size_t map_w, size_t map_h,
                        size_t dest_w, size_t dest_h, const ppocr_db_options *options, float *boxes,
                        size_t boxes_cap, size_t *n_boxes, char *err, size_t err_len);

/* The DB threshold on the GPU (src/det.rs:438): mask[i] = prob[i] > thresh
 * (f32), n bytes, device pointers. */
int ppocr_hip_db_mask(const float *prob, uint8_t *mask, size_t n, float thresh, void *stream);

/* --- Image stages on the GPU ------------------------------------------------
 * Device pointers, 8-bit three-channel images with rows top to bottom (HWC,
 * as the worker decodes pages), sides up to 32768. Results are the
 * reference's CPU results, bit for bit. */

/* Replaces `resize_linear` (src/image.rs:68-142): cv2.resize INTER_LINEAR on
 * 8 bits, sw x sh -> dw x dh. */
int ppocr_hip_resize_linear(const uint8_t *src, size_t sw, size_t sh, uint8_t *dst, size_t dw, size_t dh,
                            void *stream);

/* Replaces `det_input_hwc` (src/det.rs:228-289): the page resized to ow x oh,
 * v * (1/255 as f32), then (x - mean[c]) / std[c] in f64, one f32 rounding;
 * HWC f32 into `out` (3 * ow * oh floats, e.g. the detector's input). */
int ppocr_hip_det_input(const uint8_t *page, size_t w, size_t h, float *out, size_t ow, size_t oh,
                        const double *mean, const double *std, void *stream);

/* The recogniser tensor width for a w x h crop and, in `*resized_w`, the
 * width the crop is resized to (src/rec.rs:20-31); 0 for an empty crop. */
size_t ppocr_rec_width(size_t w, size_t h, size_t *resized_w);

/* Replaces `rec_input` (src/rec.rs:19-43), HWC: 48 rows of
 * ppocr_rec_width(w, h) pixels, the crop resized to height 48 and scaled to
 * [-1, 1] in f32, zeros right of it. `out_cap` floats at `out`; `*width`
 * receives the tensor width. */
int ppocr_hip_rec_input(const uint8_t *crop, size_t w, size_t h, float *out, size_t out_cap, size_t *width,
                        void *stream);

/* The recogniser input with the tensor width capped at `max_width` (no
 * reference counterpart: the page pipeline's crops "resized to height 48
 * with padded width <= 320"): a crop whose `ppocr_rec_width` exceeds the cap
 * is resized to max_width x 48 (squeezed), any other gives exactly
 * `ppocr_hip_rec_input`'s tensor. `max_width` 0 means no cap. */
size_t ppocr_rec_width_fit(size_t w, size_t h, size_t max_width, size_t *resized_w);
int ppocr_hip_rec_input_fit(const uint8_t *crop, size_t w, size_t h, size_t max_width, float *out,
                            size_t out_cap, size_t *width, void *stream);

/* The recogniser inputs of n boxes of a page, 16 lines per launch, without
 * the crops in memory (no reference counterpart: the worker crops each box
 * and then makes its input, ocr.rs:472-477): quads n x (x, y) x 4 as
 * `ppocr_hip_crop_text` takes them; line i's 48 x widths[i] tensor (HWC,
 * `out_caps[i]` floats at the device address outs[i]) gets exactly what
 * `ppocr_hip_crop_text` followed by `ppocr_hip_rec_input_fit` with
 * `max_width` would write. */
int ppocr_hip_crop_rec_inputs(const uint8_t *page, size_t w, size_t h, const float *quads, size_t n,
                              size_t max_width, float *const *outs, const size_t *out_caps, size_t *widths,
                              void *stream);

/* The size `ppocr_hip_crop_text` gives a quad's crop, after any turn. */
int ppocr_crop_size(const float *quad, size_t *width, size_t *height);

/* Replaces `crop_text` (src/crop.rs:84-127): the quad (x, y) x 4, top-left,
 * top-right, bottom-right, bottom-left, mapped onto an upright rectangle and
 * sampled bicubically (edges repeated), turned a quarter counter-clockwise
 * when 1.5 times taller than wide. `*out_w` x `*out_h` pixels into `out`
 * (`out_cap` bytes). */
int ppocr_hip_crop_text(const uint8_t *page, size_t w, size_t h, const float *quad, uint8_t *out,
                        size_t out_cap, size_t *out_w, size_t *out_h, void *stream);

#ifdef __cplusplus
}
#endif

#endif
