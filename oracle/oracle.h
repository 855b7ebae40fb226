/*
 * oracle.h - test infrastructure only: a plain C restatement of tabicl-anywhere's CPU path (the reference's
 * src/kern.rs, src/nn.rs, src/fit.rs, src/predict.rs), used as the checker for the HIP library and as the timed
 * CPU baseline. Nothing in the product links it.
 *
 * Layouts are the reference's: keys and values dimension-major ([d][r]), weights [out][in], fitted in-context
 * layers in stored chunk records (include/tah.h). Each function names the reference lines it follows.
 */
#ifndef TAH_ORACLE_H
#define TAH_ORACLE_H

#include "../include/tah.h"

#ifdef __cplusplus
extern "C" {
#endif

/* src/kern.rs:189-206, 227-253, 255-261, 263-268 */
float orc_exp1(float x);
float orc_erf1(float x);
float orc_tanh1(float x);
void orc_gelu(float *x, int n);
/* src/kern.rs:326-347 */
void orc_layer_norm(const float *x, int n, const float *w, const float *b, float *y);
/* y = w x + b, w [out][in] (src/kern.rs:64-130) */
void orc_linear(const float *w, const float *b, const float *x, int in, int out, float *y);

/* src/nn.rs:97-107 */
void orc_query_scale(const tah_block *b, int n, float *out);
/* src/nn.rs:130-152 */
void orc_query(const tah_block *b, const float *scale, const float *x, float *q);
/* src/nn.rs:156-164 */
void orc_feed_forward(const tah_block *b, float *x);

/* Kv::record, src/fit.rs:123-126: bytes of one stored chunk of rc rows. */
size_t orc_kv_record(int kv_format, int d, int rc);

/* src/fit.rs:549-576: one chunk c ([2d][rc] floats: K rows then V rows) to its stored record. */
void orc_pack(const float *c, int d, int rc, int kv_format, uint8_t *out);

/* One in-context layer's attention for nq queries (already scaled, [nq][d]) over stored chunk records
 * (the CPU loop of src/predict.rs:427-533 with Soft::update / update_int, src/nn.rs:194-258, and Soft::finish
 * src/nn.rs:280-286). key_parts > 1 splits the chunks into that many ranges merged with Soft::merge
 * (src/nn.rs:261-276, src/predict.rs:521-532). out is [nq][d]. */
void orc_attend_records(const float *q, int nq, const uint8_t *records, int kv_format, int rows, int chunk, int d,
                        int heads, int key_parts, float *out);

/* The whole in-context stage at prediction for one problem (src/predict.rs:381-586): h [n][d] is consumed,
 * out [n][out_n] gets the first out_n decoder outputs. records[l] is layer l, scales [layers][d]. */
void orc_in_context(const tah_model_desc *m, const float *scales, const uint8_t *const *records, int kv_format,
                    int rows, int chunk, float *h, int n, int out_n, float *out);

/* Column stage at fit for every feature group (src/fit.rs:300-423): x [rows][features], y [rows] (class index as
 * float, or regression target), bases [digits] label digits. Writes col_kv [features][digits][blocks][2][e][inds]
 * and the cells after the stage, emb [features][rows][e]. */
void orc_fit_columns(const tah_model_desc *m, const float *x, const float *y, int rows, int features,
                     const int *bases, int digits, int chunk, float *col_kv, float *emb);
/* Row stage at fit (src/fit.rs:486-540 with row_forward src/nn.rs:357-419): emb [features][rows][e] to
 * representations reps [rows][d]. */
void orc_fit_columns_of(const tah_model_desc *m, const float *x, const float *y, int rows, int features,
                        const int *groups, int ngroups, const int *bases, int digits, int chunk, float *col_kv,
                        float *emb);
void orc_fit_cells_rows(const tah_model_desc *m, const float *col_kv, const int *bases, int digits, const float *x,
                        const float *y, int n, int features, float *emb);
void orc_fit_rows(const tah_model_desc *m, const float *emb, int rows, int features, float *reps);
/* In-context stage at fit for one problem (src/fit.rs:577-747, CPU path): h [rows][d] already has the target's
 * embedding added and is consumed. Writes scales [layers][d] and each layer's stored records into
 * records[l] (orc_kv_record summed over chunks). If kv_f32 is not NULL, it receives each layer's exact f32
 * chunk records as well (layers x 2*rows*d floats, in chunk layout). */
void orc_fit_icl(const tah_model_desc *m, float *h, int rows, int chunk, int kv_format, float *scales,
                 uint8_t *const *records, float *kv_f32);
/* Fit-time all-rows attention of one layer (src/fit.rs:700-744): queries q [rows][d] (scaled) over the exact f32
 * keys and values of the same rows in chunk layout (kv, 2*rows*d floats), out [rows][d] (before out-proj). */
/* One in-context layer's keys and values [n][2d] for given rows; one in-context layer step of given rows over stored
 * records (in place). */
void orc_kv_rows(const tah_model_desc *m, int layer, const float *h, int n, float *kv);
void orc_icl_step(const tah_model_desc *m, int layer, const float *scale, const uint8_t *records, int kv_format,
                  int rows, int chunk, float *h, int n);
void orc_fit_attend(const float *q, const float *kv, int rows, int chunk, int d, int heads, float *out);

/* Column stage at prediction (src/predict.rs:282-353): x [n][features], col_kv as fitted; tok receives
 * [n][cls + features][e], class tokens first. */
void orc_embed(const tah_model_desc *m, const float *col_kv, int digits, const float *x, int n, int features,
               float *tok);
/* Row stage at prediction (src/predict.rs:356-372): tok [n][tokens][e] (consumed) to rep [n][d]. */
void orc_represent(const tah_model_desc *m, float *tok, int n, int tokens, float *rep);

/* Threads the oracle's parallel loops use (OpenMP; the reference spreads the same loops over rayon). */
void orc_set_threads(int n);
int orc_threads(void);

#ifdef __cplusplus
}
#endif

#endif
