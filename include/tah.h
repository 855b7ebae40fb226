/*
 * tah.h - C ABI of libtah_hip.so, the MI355X (gfx950) accelerator for tabicl-anywhere's in-context hot path.
 *
 * It is the native side of the reference's two accelerator plugin traits and its card handle:
 *
 *   fit::Attend          src/fit.rs:45-74       (attend, attend_fits, in_context)
 *   predict::AttendCached src/predict.rs:63-79   (attend, stage)
 *   gpu::Gpu / VramModel  src/gpu.rs:725-1019, src/gpu.rs:2033-2149 (new, work budget, load, attend_resident,
 *                                                                     in_context)
 *
 * Conventions (the reference's, src/gpu.rs:720-722, src/gpu.rs:887-889):
 *   - every function returns an int status; 0 is success;
 *   - TAH_E_BUDGET is the reference's io::ErrorKind::OutOfMemory (working-memory budget exceeded);
 *   - TAH_E_DEVICE is a HIP runtime failure ("graphics card: ..."); callers answer on the CPU instead;
 *   - TAH_E_DECLINED is the reference's Ok(None)/Ok(false): not offered for this shape, nothing was done;
 *   - tah_last_error() gives the message of the last failure on a device handle;
 *   - host buffers are caller-owned and borrowed for the duration of the call; functions taking host pointers
 *     block until their results are on the host. Functions suffixed _dev take device pointers and leave the
 *     work queued on the device handle's stream (tah_sync waits for it).
 *   - a device handle may be shared by threads; calls on it are serialised.
 *
 * Matrices are row-major; weight matrices are [out][in] as PyTorch stores them. Keys and values of a fitted
 * in-context layer stay in the reference's stored chunk layout (src/fit.rs:102-127, src/fit.rs:549-576):
 * chunks of `chunk` training rows, the last one short; a chunk of rc rows is
 *     f32:     [K: d][rc] f32  then [V: d][rc] f32
 *     i16/i8:  [2d scales] f32, then [K: d][rc] ints, then [V: d][rc] ints     (value = int * scale[coordinate])
 * and chunk ci starts at byte ci * record(d, chunk).
 */
#ifndef TAH_H
#define TAH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    TAH_OK = 0,
    TAH_E_ARG = 1,      /* invalid argument (io::ErrorKind::InvalidInput) */
    TAH_E_BUDGET = 2,   /* over the working-memory budget (io::ErrorKind::OutOfMemory) */
    TAH_E_DEVICE = 3,   /* HIP runtime error; answer on the CPU */
    TAH_E_DECLINED = 4, /* not offered for this shape; nothing was done */
    TAH_E_SINK = 5      /* the caller's layer sink returned non-zero; the fit stopped there */
};

/* Stored formats of in-context keys and values: the reference's Kv codes (src/fit.rs:102-127, Kv::from_code). */
enum { TAH_KV_F32 = 0, TAH_KV_I16 = 1, TAH_KV_I8 = 2 };

/* One pre-norm attention block, x += attn(norm1 x); x += l2(gelu(l1(norm2 x))) (src/model.rs:27-98).
 * ss_hidden is 0 for a block without the scalable softmax ("QASSMax", src/model.rs:14-24, src/nn.rs:97-152). */
typedef struct tah_block {
    int32_t d, heads, ff, ss_hidden;
    const float *n1w, *n1b, *n2w, *n2b; /* [d] each; absent layer-norm biases are passed as zeros */
    const float *in_w, *in_b;           /* [3d][d], [3d]: query, key, value projections stacked */
    const float *out_w, *out_b;         /* [d][d], [d] */
    const float *l1w, *l1b;             /* [ff][d], [ff] */
    const float *l2w, *l2b;             /* [d][ff], [d] */
    const float *b0w, *b0b;             /* scalable softmax base MLP: [ss_hidden][1], [ss_hidden] */
    const float *b2w, *b2b;             /* [d][ss_hidden], [d] */
    const float *q0w, *q0b;             /* query MLP shared by the heads: [ss_hidden][hd], [ss_hidden] */
    const float *q2w, *q2b;             /* [hd][ss_hidden], [hd] */
} tah_block;

/* The whole network's weights and sizes (src/model.rs:110-143, Model::load src/model.rs:202-272). The two target
 * tables are the reference's class_table form (src/model.rs:164-177): [max_classes][width] with the bias folded
 * in, or for a regression model (max_classes 0) the layer as [weight][bias], 2 x width. */
typedef struct tah_model_desc {
    int32_t e, d, group, inds, cls, max_classes;
    int32_t col_heads, row_heads, icl_heads;
    int32_t col_blocks, row_blocks, icl_layers;
    int32_t dec_hidden, outputs, rope_half;
    const float *in_w, *in_b;       /* [e][group], [e] */
    const tah_block *col_a1;        /* [col_blocks]: inducing points attend to cells (fitting only; may be NULL) */
    const tah_block *col_a2;        /* [col_blocks]: cells attend to the inducing points' keys and values */
    const float *col_ind;           /* [col_blocks][inds][e] (fitting only; may be NULL) */
    const float *col_y;             /* [max_classes][e] or [2][e] */
    const float *cls_tokens;        /* [cls][e] */
    const tah_block *row;           /* [row_blocks] */
    const float *rope_freqs;        /* [rope_half] */
    const float *out_lnw, *out_lnb; /* [e] */
    const tah_block *icl;           /* [icl_layers] */
    const float *icl_y;             /* [max_classes][d] or [2][d] */
    const float *lnw, *lnb;         /* [d] */
    const float *dec0w, *dec0b;     /* [dec_hidden][d], [dec_hidden] */
    const float *dec2w, *dec2b;     /* [outputs][dec_hidden], [outputs] */
} tah_model_desc;

typedef struct tah_dev tah_dev;         /* one GPU: its stream, working memory and last error (gpu::Gpu) */
typedef struct tah_weights tah_weights; /* a model's weights on the card (gpu::GpuWeights) */
typedef struct tah_model tah_model;     /* one fitted in-context problem held on the card (gpu::VramModel) */

/* Bytes of one stored chunk of rc rows: Kv::record, src/fit.rs:123-126. */
size_t tah_kv_record(int32_t kv_format, int32_t d, int32_t rc);

/* ---- device handle: Gpu::new, set_work_budget, work_budget, working, overdrawn, release (src/gpu.rs:925-1019) */
int tah_open(int32_t ordinal, tah_dev **out);
void tah_close(tah_dev *dev);
const char *tah_last_error(const tah_dev *dev);
int tah_device_name(const tah_dev *dev, char *buf, size_t len);
/* The working-memory budget (default 16 GiB): calls size their batches to it, and fail with TAH_E_BUDGET when
 * even one row or one feature group would not fit. */
int tah_set_work_budget(tah_dev *dev, size_t bytes);
size_t tah_work_budget(const tah_dev *dev);
int tah_working(const tah_dev *dev, size_t *now, size_t *peak);
size_t tah_overdrawn(const tah_dev *dev);
int tah_release(tah_dev *dev);
int tah_sync(tah_dev *dev);
/* The device handle's HIP stream (a hipStream_t), for callers that time or order work around _dev calls. A call may
   fork part of its work onto a second stream of the handle (the column and row stages of 768 rows or more, as two
   halves); it joins that stream back into this one before it returns, so that ordering on this stream orders all of
   the call's work (a graph captured on it takes the fork and the join with it). */
void *tah_stream(tah_dev *dev);

/* ---- weights: GpuWeights::new / bytes (src/gpu.rs:1838-2027). Copies every tensor the card uses. */
int tah_weights_upload(tah_dev *dev, const tah_model_desc *m, tah_weights **out);
size_t tah_weights_bytes(const tah_weights *w);
/* Frees the weights; valid after tah_close of their device (no call may be using them). */
void tah_weights_free(tah_weights *w);

/* ---- fitted model on the card: VramModel::model_bytes / load (src/gpu.rs:2064-2116), but from the bundle's own
 * chunk records as they are stored (n{j}_kv{l}), any of the three formats, no re-layout on the host.
 * layer_records[l] points at layer l's bytes (tah_kv_record summed over its chunks); scales is n{j}_scale,
 * [layers][d]. A layer of head width 64 is held once, as the tiles the card makes of its records (f32: split-fp16
 * images; i16: the codes with their dequantisation factors; i8: the codes as fp16 with the scales), which every
 * attention kernel reads; other head widths keep the records. tah_model_bytes (like Gpu::model_bytes, from the
 * weights' shape) counts what the layers are held as, and the scales; 0 without weights. */
size_t tah_model_bytes(const tah_weights *w, int32_t kv_format, int32_t rows, int32_t chunk);
int tah_model_load(tah_dev *dev, const tah_weights *w, int32_t kv_format, int32_t rows, int32_t chunk,
                   const uint8_t *const *layer_records, const float *scales, tah_model **out);
/* Frees the model; valid after tah_close of its device (no call may be using it). */
void tah_model_free(tah_model *m);

/* ---- prediction: AttendCached::attend (src/predict.rs:66, VramHandle src/gpu.rs:2648-2655): attention outputs
 * [nq][d] (before the output projection) of queries q [nq][d] (already scaled) over layer `layer` of `model`. */
int tah_attend_resident(tah_dev *dev, const tah_model *model, int32_t layer, const float *q, int32_t nq,
                        float *out);
int tah_attend_resident_dev(tah_dev *dev, const tah_model *model, int32_t layer, const float *q_dev, int32_t nq,
                            float *out_dev);

/* AttendCached::stage (src/predict.rs:70, Gpu::in_context src/gpu.rs:2140): the whole in-context stage of one
 * problem, row representations h [nq][d] to the first out_n decoder outputs [nq][out_n]. */
int tah_stage(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *h, int32_t nq,
              int32_t out_n, float *out);
int tah_stage_dev(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *h_dev, int32_t nq,
                  int32_t out_n, float *out_dev);

/* The same without allocating: for callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). It has no counterpart in the reference. Its working buffers come
 * from a static device array of TAH_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends); nq is at most
 * TAH_NOALLOC_MAX_ROWS, and a model whose buffers would not fit there is refused with TAH_E_ARG. Calls on one GPU
 * share the array: calls that overlap on one GPU (through two device handles) race. */
#define TAH_NOALLOC_MAX_ROWS 256
#define TAH_NOALLOC_SCRATCH_BYTES ((size_t)24 << 20)
int tah_stage_dev_noalloc(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *h_dev, int32_t nq,
                          int32_t out_n, float *out_dev);

/* ---- the column and row stages, and AttendCached::rows (src/predict.rs:74-78, Gpu::predict src/gpu.rs:2146) --
 *
 * tah_model_set_columns: gives the fitted member's column cache (col_kv, [features][digits][col_blocks][2][e][inds],
 * src/fit.rs:6-7) to a model on the card, as VramModel holds it. */
int tah_model_set_columns(tah_dev *dev, tah_model *model, const tah_weights *w, const float *col_kv, int32_t features,
                          int32_t digits);
/* Card bytes tah_model_set_columns adds to a model of these weights: the column cache and the key/value images of
 * the column blocks it makes from it (a part of Gpu::model_bytes, src/gpu.rs:2064-2068, for a member whose column
 * cache the card holds). */
size_t tah_columns_bytes(const tah_weights *w, int32_t features, int32_t digits);
/* Card bytes a loaded model holds now: what tah_model_bytes counted at load plus what tah_model_set_columns added
 * (VramModel's size as the VRAM tier accounts it, src/gpu.rs:2495-2611). */
size_t tah_model_held_bytes(const tah_model *m);
/* The column stage at prediction (embed, src/predict.rs:282-353): x [n][features] (already normalised) to tokens
 * [n][cls + features][e], class tokens first. */
int tah_embed(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x, int32_t n, float *tok);
/* The row stage (represent, src/predict.rs:356-372): tokens [n][tokens][e] to row representations [n][d]. */
int tah_represent(tah_dev *dev, const tah_weights *w, const float *tok, int32_t n, int32_t tokens, float *rep);
/* AttendCached::rows: all three stages, x [n][features] to the first out_n decoder outputs [n][out_n], for a member
 * with one in-context problem. Rows are processed in sub-batches that fit the working-memory budget. */
int tah_predict_rows(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x, int32_t n,
                     int32_t out_n, float *out);
int tah_predict_rows_dev(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x_dev, int32_t n,
                         int32_t out_n, float *out_dev);

/* ---- fitting: the fit::Attend hooks (src/fit.rs:45-74) ---------------------------------------------------------
 *
 * tah_pack: one stored chunk from its f32 keys and values c ([2d][rc]: the d key rows then the d value rows) to the
 * record of format kv_format, quantised on the card exactly as the reference's pack (src/fit.rs:549-576). */
int tah_pack(tah_dev *dev, const float *c, int32_t d, int32_t rc, int32_t kv_format, uint8_t *out);

/* Attend::attend (src/fit.rs:46, Gpu src/gpu.rs:1471-1510): every training row's attention over all training rows
 * of one layer. q [rows][d] (already scaled), kv the layer's exact f32 keys and values in chunk layout
 * (2 * rows * d floats), out [rows][d] before the output projection. */
int tah_attend(tah_dev *dev, const float *q, const float *kv, int32_t rows, int32_t chunk, int32_t d, int32_t heads,
               float *out);

/* The column and row stages of a fit (Attend::columns and Attend::rows, src/fit.rs:54-65, the CPU loops at
 * src/fit.rs:326-423 and 486-540), with the cells kept on the card between them. x [rows][features] (numeric,
 * normalised), y [rows] (class index as a float, or the standardised target of a regression model), bases [digits]
 * the label digits' bases (one digit: {classes}), ind_scales [col_blocks][e] each block's
 * Block::query_scale(rows) for the inducing points' queries. Writes col_kv_out
 * [features][digits][col_blocks][2][e][inds] and reps_out [rows][d]. Feature groups and rows go in batches that
 * fit the working-memory budget. */
int tah_fit_represent(tah_dev *dev, const tah_weights *w, const float *x, const float *y, int32_t rows,
                      int32_t features, const int32_t *bases, int32_t digits, const float *ind_scales,
                      float *col_kv_out, float *reps_out);

/* The fit hooks one at a time, with the trait's own layouts, for an unmodified fit_raw_async (src/fit.rs:425-545).
 *
 * Attend::column_batch (src/fit.rs:54, Gpu src/gpu.rs:1502-1510): how many feature groups of `rows` training cells
 * tah_columns takes per call within the working-memory budget left now; 0 when the column stage is not offered
 * (weights uploaded without the fitting blocks, or not even one group fits). */
size_t tah_column_batch(const tah_dev *dev, const tah_weights *w, int32_t rows);
/* Attend::columns (src/fit.rs:57, Gpu src/gpu.rs:1512-1614): the column stage for `groups` feature groups at once
 * (one label digit). cells [rows][groups][e] holds their training cells through the input layer with the target's
 * embedding added, and is replaced by the cells after the stage; ind_q [col_blocks][inds][e] is each block's
 * inducing-point queries (scaled); rec receives what col_kv stores for these groups,
 * [groups][col_blocks][2][e][inds]. More groups than tah_column_batch allows fail with TAH_E_BUDGET. */
int tah_columns(tah_dev *dev, const tah_weights *w, float *cells, int32_t rows, int32_t groups, const float *ind_q,
                float *rec);
/* Attend::row_batch (src/fit.rs:60, Gpu src/gpu.rs:1616-1622): how many rows of `features` cells tah_rows takes per
 * call; 0 when the row stage is not offered. */
size_t tah_row_batch(const tah_dev *dev, const tah_weights *w, int32_t features);
/* Attend::rows (src/fit.rs:63, Gpu src/gpu.rs:1624-1648): the row stage for n rows, cells [n][features][e] (after
 * the column stage) to reps [n][d]. */
int tah_rows(tah_dev *dev, const tah_weights *w, const float *cells, int32_t n, int32_t features, float *reps);
/* Attend::attend_fits (src/fit.rs:50, Gpu src/gpu.rs:1498-1500): 1 if tah_attend can take a layer of `rows` rows of
 * width d within the working-memory budget, else 0 (the CPU then does that attention). */
int tah_attend_fits(const tah_dev *dev, int32_t rows, int32_t d);
/* Gpu::attend_rows (src/gpu.rs:1306-1322): attention outputs [nq][d] of queries q [nq][d] (already scaled) over keys
 * k and values v, each row-major [n][d], in full precision. */
int tah_attend_rows(tah_dev *dev, const float *q, const float *k, const float *v, int32_t nq, int32_t n, int32_t d,
                    int32_t heads, float *out);
/* Gpu::calibrate (src/gpu.rs:1355-1383): how fast this card does the in-context attention, in multiply-adds per
 * second: the best of repeated runs (at least three, then for about `ms` milliseconds) of 256 queries over 2,048 keys
 * (d = 512, 8 heads), timed from host buffers to host buffers. */
int tah_calibrate(tah_dev *dev, double ms, double *rate);
/* Gpu::stages (src/gpu.rs:744-746): fitting stages this device has done (each fit hook call it took; a
 * tah_fit_represent call counts as two, the column and the row stage). */
uint64_t tah_stages(const tah_dev *dev);
/* No counterpart in the reference: a measurement hook for benchmarks. Arms HIP events around each launch of the
 * many-query attention kernel (the in-context attention over a layer's tiles from 17 queries) on this device's
 * stream, for up to `launches` launches (0 disarms); one probe per process, arming again resets it. */
int tah_probe_attention(tah_dev *dev, int32_t launches);
/* Synchronises the device's stream; *launches = the launches recorded since arming or the last read, *ms = their
 * summed duration in milliseconds. TAH_E_ARG if the probe is not armed for this device. */
int tah_probe_read(tah_dev *dev, double *ms, int32_t *launches);

/* Receives layer `layer`'s stored records (tah_kv_record summed over its chunks, in host memory valid for the
 * duration of the call) while the in-context stage is fitted; non-zero stops the fit with TAH_E_SINK. */
typedef int (*tah_layer_sink)(void *ctx, int32_t layer, const uint8_t *records, size_t bytes);

/* Attend::in_context (src/fit.rs:67-73, Gpu src/gpu.rs:1650-1714): the whole in-context stage of one problem at
 * fit time. h [rows][d] is the row representations with the target's embedding added, scales [layers][d] what each
 * layer multiplies its queries by (Block::query_scale(rows)). Per layer, in order: keys and values of every row
 * (layer norm, projection), stored as chunk records of `chunk` rows in kv_format and handed to sink; then (except
 * after the last layer, whose outputs are never used, src/fit.rs:664-666) every row attends to all rows over the
 * exact f32 keys and values, and the output projection and feed-forward update h. */
int tah_in_context(tah_dev *dev, const tah_weights *w, const float *h, int32_t rows, const float *scales,
                   int32_t kv_format, int32_t chunk, tah_layer_sink sink, void *ctx);

/* ---- the regression head: QuantileDist (src/table.rs:292-346) ---------------------------------------------------
 *
 * A regression member's output rows read as distributions, as the reference reads each row on the host
 * (QuantileDist::new, mean, variance and icdf, applied per row at src/table.rs:479-486): q [rows][n] predicted
 * quantiles (n from 2 to 1024: the model's 999), alphas [n_alphas] (at most 64) the requested levels; writes
 * stats [rows][3 + n_alphas]: mean, sample variance, median (icdf at 0.5), then the icdf at each alpha, in f32,
 * summed in the reference's order (the tails beyond the first and last level through the device's logf). The
 * member average in f64 and the mapping back to the target's units stay with the caller (src/table.rs:481-494). */
int tah_quantile_stats(tah_dev *dev, const float *q, int32_t rows, int32_t n, const float *alphas,
                       int32_t n_alphas, float *stats);
/* The same with q and stats in device memory (alphas on the host); ordered on the library's stream. */
int tah_quantile_stats_dev(tah_dev *dev, const float *q_dev, int32_t rows, int32_t n, const float *alphas,
                           int32_t n_alphas, float *stats_dev);

#ifdef __cplusplus
}
#endif

#endif /* TAH_H */
