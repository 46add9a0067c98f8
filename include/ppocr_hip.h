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
 * run takes. */
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

/* Runs record their launches in a HIP graph from the second run after the
 * lanes were set, and replay it (default, `enable` 1); with 0 every run
 * launches each kernel itself. Returns 0, or 1 for a NULL model. */
int ppocr_gpu_set_graphs(ppocr_gpu_model *model, int enable);

/* Kernel launches one run makes, and launch `i`'s kernel name (valid for the
 * model's lifetime) and the plan operation it starts from. */
size_t ppocr_gpu_launch_count(const ppocr_gpu_model *model);
const char *ppocr_gpu_launch_name(const ppocr_gpu_model *model, size_t i, size_t *op);

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

/* `Kind::Mean` (src/engine/layers.rs:391-406): y[c] = mean over `pixels` of
 * x[p][c], summed in f64. */
int ppocr_hip_channel_mean(const float *x, float *y, size_t pixels, size_t c, void *stream);

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

#ifdef __cplusplus
}
#endif

#endif
