// Internal declarations shared by the HIP sources of libtah_hip.so: the device handle, the weights and fitted
// model as they sit on the card, working memory, and the kernel launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/tah.h"

namespace tah {

// A HIP failure inside a call: carries the message reported through tah_last_error ("graphics card: ...").
struct DeviceError {
    std::string msg;
};
struct ArgError {
    std::string msg;
};
struct BudgetError {
    std::string msg;
};

#define TAH_HIP(expr)                                                                                     \
    do {                                                                                                  \
        hipError_t e_ = (expr);                                                                           \
        if (e_ != hipSuccess)                                                                             \
            throw ::tah::DeviceError{std::string("graphics card: ") + #expr + ": " + hipGetErrorString(e_)}; \
    } while (0)

// Kernel launches: the launch itself and any error it left.
#define TAH_LAUNCHED() TAH_HIP(hipGetLastError())

// ---- working memory ----------------------------------------------------------------------------------------
// Buffers a call borrows: kept between calls (allocating and freeing a few hundred MB per call costs more than
// a small prediction), never more in existence than the device's work budget.
struct Pool {
    struct Buf {
        void *p;
        size_t bytes;
        bool busy;
    };
    std::vector<Buf> bufs;
    size_t budget = size_t(16) << 30;  // MI355X holds 288 GB of HBM; the reference's 1.5 GB suits 24 GB cards
    size_t bytes = 0, peak = 0, overdrawn = 0;

    void *take(size_t bytes, int device);
    void give(void *p);
    void release_idle();
};

}  // namespace tah

// One GPU.
struct tah_dev {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    // pinned host staging for records on their way to a layer sink: two buffers (one being filled by the card while
    // the sink reads the other), kept between calls and grown as needed; two events marking their copies done
    void *pinned[2] = {nullptr, nullptr};
    size_t pinned_bytes = 0;
    hipEvent_t copied[2] = {nullptr, nullptr};
    std::mutex lock;
    std::string last_error;
    std::string name;
    tah::Pool pool;
    // fitting stages the card has done (each call of a fit hook it took rather than declined)
    std::atomic<uint64_t> stages{0};
    // this device's copy of the library's static scratch array (tah_stage_dev_noalloc), resolved at tah_open with
    // the device current: a device address, unlike the array's name in host code
    uint8_t *noalloc = nullptr;
    // a second stream (default priority) for work that runs beside the main stream's, and the events that fork to it
    // and join back
    hipStream_t side = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
};

// A block's tensors on the card (device pointers; nullptr where absent).
// A weight matrix W [N][K] uploaded as a split-fp16 image for gemm_split: 32-row tiles (rows in sigma32 order within
// a tile), then 16-column steps, each [hi, lo][k half][32 rows][8 halves] (2 KB); W scaled by 2^shift first. row0
// selects rows row0.. of it (a multiple of 32).
struct SplitW {
    const uint8_t *img = nullptr;
    int shift = 0, N = 0, K = 0, row0 = 0;
    SplitW rows(int r0) const {
        SplitW o = *this;
        o.row0 = r0;
        return o;
    }
};

struct DevBlock {
    int d, heads, ff, ss_hidden;
    const float *n1w, *n1b, *n2w, *n2b, *in_w, *in_b, *out_w, *out_b, *l1w, *l1b, *l2w, *l2b;
    const float *b0w, *b0b, *b2w, *b2b, *q0w, *q0b, *q2w, *q2b;
    // feed-forward weights as split-fp16 images for the fused feed-forward kernel (width 128, hidden 256), else null;
    // l1s / l2s: the powers of two they were scaled by
    const uint8_t *l1img, *l2img;
    int l1s, l2s;
    // width 128: in_w [384][128] and out_w [128][128] as the same images, for k_rows128 (rows128)
    const uint8_t *inimg, *outimg;
    int ins, outs;
    // the dense layers as gemm_split images (empty where the shape does not fit): in_w [3d][d], out_w, l1w, l2w and
    // the query MLP's q0w, q2w
    SplitW in_s, out_s, l1_s, l2_s, q0_s, q2_s;
};

struct tah_weights {
    tah_dev *dev;
    int ordinal;
    void *arena = nullptr;
    size_t bytes = 0;
    int e, d, group, inds, cls, max_classes, col_heads, row_heads, icl_heads;
    int col_blocks, row_blocks, icl_layers, dec_hidden, outputs, rope_half;
    std::vector<DevBlock> col_a1, col_a2, row, icl;
    const float *in_w, *in_b, *col_ind, *col_y, *cls_tokens, *rope_freqs, *out_lnw, *out_lnb;
    const float *icl_y, *lnw, *lnb, *dec0w, *dec0b, *dec2w, *dec2b;
    SplitW dec0_s;  // the decoder's first layer as a gemm_split image
    const float *col_scale;  // [e]: 1 / sqrt(column head width), what the column blocks' queries are multiplied by
    // the row stage's rotary tables, made at upload for positions 0 .. ROPE_POSITIONS - 1 (any token count up to
    // that reads a prefix): cos then sin of position * frequency, [2][ROPE_POSITIONS][rope_half], or null
    const float *rope_tab = nullptr;
    // the class tokens' keys and values in the first row block, [cls][2 e] (then cls e floats of room), made at upload
    // (they depend on the weights alone), or null without a row stage
    float *cls_kv = nullptr;
};

// Token positions the rotary tables cover: a row of at most this many tokens (class tokens and features).
constexpr int ROPE_POSITIONS = 16384;

struct tah_model {
    tah_dev *dev;
    int ordinal;
    int kv_format, rows, chunk, d, layers, heads;
    size_t layer_bytes;
    uint8_t *records = nullptr;  // layers x layer_bytes: the stored chunk records as they are, then their images
    bool images = false;         // head width 64: tile images follow each layer's records
    float *scales = nullptr;     // [layers][d]
    size_t bytes = 0;
    float *col_kv = nullptr;     // [features][digits][blocks][2][e][inds] (tah_model_set_columns)
    uint8_t *col_img = nullptr;  // the column blocks' key/value images of col_kv (column_images), where they apply
    int features = 0, digits = 0;
};

namespace tah {

enum Epi { EPI_NONE = 0, EPI_GELU = 1, EPI_RESID = 2, EPI_QMOD = 3, EPI_SCALE = 4 };

// Y[M][N] (leading dim ldy) = epi(X[M][K] (ldx) * W[N][K]^T + b[N]); EPI_RESID adds R (ldr, may alias Y).
// With lnw/lnb, X's rows are layer-normalised first inside the kernel (only where gemm_ln_fits).
void gemm(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const float *b, float *Y,
          int ldy, Epi epi, const float *R, int ldr, const float *lnw = nullptr, const float *lnb = nullptr,
          const float *scale = nullptr);
bool gemm_ln_fits(int M, int K, const float *X, int ldx, const float *W);

// q [M][N] (in place) = q * scale[(m % heads) * N + n] * (1 + tanh(X W^T + b)): the query MLP's modulation.
void gemm_qmod(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const float *b, float *q,
               const float *scale, int heads);

// The same on split-fp16 MFMA from a weight image (gemm_split.hip); EPI_SCALE multiplies by scale [N], EPI_QMOD as
// gemm_qmod with scale [heads][N].
bool gemm_split_fits(int N, int K);
void gemm_split(hipStream_t s, int M, int N, int K, const float *X, int ldx, const SplitW &w, const float *b, float *Y,
                int ldy, Epi epi, const float *R, int ldr, const float *scale, int heads);
// The split-fp16 kernels where the image fits and there are 512 rows or more, else gemm on the f32 weights. With
// lnw/lnb the rows of X are layer-normalised first: inside the kernel for K = 512, else through t [M][K].
void dense(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const SplitW &w, const float *b,
           float *Y, int ldy, Epi epi, const float *R, int ldr, const float *lnw = nullptr, const float *lnb = nullptr,
           float *t = nullptr);

// y[r] = layer_norm(x[r]) * w + b over rows of n numbers (eps 1e-5, biased variance).
void layer_norm(hipStream_t s, int rows, int n, const float *x, int ldx, const float *w, const float *b, float *y,
                int ldy);

// In place on q [rows][d] (after the query projection): q *= scale (no scalable softmax), or per head
// q_h *= scale_h * (1 + tanh(q2 gelu(q0 q_h + q0b) + q2b)). scratch holds rows * heads * ss_hidden floats.
void query_modulate(hipStream_t s, int rows, const DevBlock &b, const float *scale, float *q, float *scratch);
size_t query_scratch_floats(int rows, const DevBlock &b);
// The whole query MLP in one kernel (gemm_split.hip), for head width 64 and hidden width 64 with images.
bool qmlp_fused(const DevBlock &b);
// q = modulate(Wq norm1(X) + bq) for many rows in one launch: the split-K projection with the query MLP in its
// epilogue (d = 512, head width and query-MLP width 64; measured faster than the f32 projection and a separate
// query MLP from 64 rows up, and the few-row kernel takes up to eight)
bool query_split_fits(const DevBlock &b, int M, const float *X, int ldx, const float *Y);
void query_split(hipStream_t s, int M, const float *X, int ldx, const DevBlock &b, const float *scale, float *q);
void qmlp(hipStream_t s, int rows, const DevBlock &b, const float *scale, float *q);
// the same for one to three rows (d = 512): a workgroup per head, projection and query MLP in one launch
bool query_rows_fits(const DevBlock &b, int M, const float *X, int ldx, const float *Y);
void query_rows(hipStream_t s, int M, const float *X, int ldx, const DevBlock &b, const float *scale, float *q);

// Fused feed-forward sub-block (blocks.hip): x [M][128] += l2(gelu(l1(layer_norm2(x)))) in one kernel, the hidden
// layer kept in registers; for blocks of width 128 and hidden width 256 (ff_fused_shape), else the caller runs
// layer_norm and two GEMMs.
inline bool ff_fused_shape(int d, int ff) { return d == 128 && ff == 256; }
void ff_block(hipStream_t s, int M, float *x, const DevBlock &b);
// The attention half of a column block (norm1, query, attention to the cached inducing keys, output projection and
// residual) in one kernel, in place on cells (n rows x groups; cell (r, g) at row r * sr + g * sg); e = 128, 8 heads
// of 16, 128 inducing points (cell_block_fits).
// work: cell_block_work_bytes(groups) bytes, 16-byte aligned (the groups' key/value images).
bool cell_block_fits(const DevBlock &b);
// The attention half of a row block for every token of n rows of T tokens (tok [n][T][e] in place), from the keys
// and values kv [n][T][2 e] the projection made (unrotated); e = 128, 8 heads of 16, T <= 128 (row_block_fits).
// With ff (block_ff_fits) either kernel runs the block's feed-forward half as well, in the same launch; the row
// block with next as well (ff, row_kv_fits) forms that block's keys and values [n][T][2 e] from the result into
// kv_next (which may be kv), and then stores only the first keep tokens of each row's new values (the rest are
// then left as the attention half wrote them: for a next block that updates only those tokens).
bool row_block_fits(const DevBlock &b, int T);
bool block_ff_fits(const DevBlock &b);
bool row_kv_fits(const DevBlock &next);
void row_block(hipStream_t s, int n, int T, float *tok, const float *kv, const float *cosv, const float *sinv,
               const DevBlock &b, bool ff, const DevBlock *next = nullptr, float *kv_next = nullptr, int keep = -1);
size_t cell_block_work_bytes(int groups);
// The column stage's input layer as the first column block's input: cell (r, g) = in_w vals + in_b over the row's
// group values vals[k] = x[r][(g + 2^k) mod features] (k < group), or all -100 where every one of them is -100.
struct InCells {
    const float *x;            // the table rows [n][features]
    const float *in_w, *in_b;  // [e][group], [e]
    int features, group;
};
// With next as well (ff, row_kv_fits) the column block's result goes on to that row block's keys and values: cell
// (r, g)'s [2 e] at kv_next + (r sr + g sg) 2 e.
// images_ready: work holds the groups' images already (cell_images of the same kvbase), else they are made first.
// in (with ff and without next, groups of in_cells_group() values): the cells' values are formed from the table
// rows (InCells) instead of read; the block writes them whole (groups = features).
int in_cells_group();
void cell_block(hipStream_t s, int n, int groups, size_t sr, size_t sg, float *cells, const DevBlock &b,
                const float *qscale, const float *kvbase, size_t gstride, void *work, bool ff,
                const DevBlock *next = nullptr, float *kv_next = nullptr, bool images_ready = false,
                const InCells *in = nullptr);
// The groups' key/value images for cell_block (group g's keys and values at kvbase + g gstride) into work
// (cell_block_work_bytes(groups), 16-byte aligned).
void cell_images(hipStream_t s, int groups, const float *kvbase, size_t gstride, void *work);
// Y [M][N] = epi(X' W^T + b) for K = 128 and N a multiple of 128, W as such an image (scaled by 2^shift), X' = X or
// layer_norm(X) with lnw/lnb; EPI_NONE, EPI_SCALE (by scale [N]) or EPI_RESID (adds R, may alias Y).
void rows128(hipStream_t s, int M, int N, const float *X, int ldx, const uint8_t *wimg, int wshift, const float *b,
             float *Y, int ldy, Epi epi, const float *R, int ldr, const float *scale, const float *lnw,
             const float *lnb);

// Widest per-row scratch of an in-context block: its feed-forward hidden layer or its query MLP's hidden layers.
inline int icl_mid(const tah_weights *w) {
    int m = 0;
    for (auto &b : w->icl) m = std::max(m, std::max(b.ff, b.heads * b.ss_hidden));
    return m;
}

// The attention of nq queries q [nq][d] (scaled) over one stored in-context layer (chunk records on the card):
// out [nq][d], normalised. work must hold attention_work_bytes(...).
struct AttnShape {
    int nq, rows, chunk, d, heads, kv_format;
};
size_t attention_work_bytes(const AttnShape &a);
// Row-major keys and values kv [rows][2d] to f32 chunk records (2 * rows * d floats).
void to_records(hipStream_t s, int rows, int d, int chunk, const float *kv, float *rec32);
// f32 chunk records to i16/i8 records (the reference's quantiser, bit for bit).
void pack(hipStream_t s, int rows, int d, int chunk, int fmt, const float *rec32, uint8_t *recq);
// Keys and values of one stored layer as tiles per (key block of 64, head), the form a fitted layer of head width 64
// is held in on the card (its records are not kept) and the attention kernels read: f32 as fp16 hi/lo split images,
// i16 as code tiles with dequantisation factors, i8 as fp16 code images with the chunks' scales (attention.hip).
struct KvImages {
    uint8_t *images = nullptr;
    uint32_t *kvmax = nullptr;  // f32 and i16: the heads' largest |K|, |V| (dequantised)
    float *scales = nullptr;    // i8: per (chunk, head) the key scales, value scales and ratios
    int fmt = TAH_KV_F32;       // the stored format the tiles were made from
};
bool kv_images_apply(int kv_format, int d, int heads);
size_t kv_images_bytes(int rows, int chunk, int heads, int kv_format);
KvImages kv_images_at(uint8_t *base, int rows, int chunk, int heads, int kv_format);
void kv_images(hipStream_t s, int rows, int chunk, int d, int heads, int kv_format, const uint8_t *records,
               KvImages img);
// Queries from which the attention runs on the matrix cores over tile images (made for transient f32 layers of the
// fit from then on; a fitted model's layers of head width 64 are held as tiles at any query count)
constexpr int TAH_SPLIT16_MIN_Q = 4;

// Launch probe of the many-query attention kernel (attention.hip): arm for a stream with room for `launches`
// launches (0 disarms); read synchronises the stream, returns the launches recorded since the last read and their
// summed duration in ms.
void probe_arm(hipStream_t s, int launches);
int probe_read(hipStream_t s, double *ms);
// Over the layer's tiles when img holds them (any query count), else over its chunk records (head width 64: fewer
// than TAH_SPLIT16_MIN_Q queries only).
void attention(hipStream_t s, const AttnShape &a, const float *q, const uint8_t *records, float *out, void *work,
               const KvImages *img = nullptr);

// The regression head (quantiles.hip): per row of q [rows][n], mean, variance, median and icdf at alphas [na]
// (device) into stats [rows][3 + na].
void quantile_stats(hipStream_t s, int rows, int n, const float *q, int na, const float *alphas, float *stats);

// Column and row stages (stages.hip).
// The input layer for n rows x [n][features]: cells [n][cls + features][e], the weights' class tokens first where
// cls > 0 (cls 0: [n][features][e]); with kv (cls > 0) the class tokens' first-row-block keys and values cls_kv
// [cls][2 e] into kv [n][cls + features][2 e] as well.
void input_cells(hipStream_t s, const tah_weights *w, const float *x, int n, int features, float *cells, int cls = 0,
                 float *kv = nullptr, const float *cls_kv = nullptr);
size_t column_stage_floats(const tah_weights *w, int n, int features, int digits);
// col_images: the model's column images (column_images_bytes, made by column_images), or nullptr (made per call).
void column_stage(hipStream_t s, const tah_weights *w, const float *col_kv, int digits, const float *x, int n,
                  int features, float *cells, float *scratch, const uint8_t *col_images = nullptr);
// The column blocks' key/value images of a fitted column cache, made once per model (where the blocks run as the
// fused kernel, else 0 bytes): [digits][blocks] of cell_block_work_bytes(features) each.
size_t column_images_bytes(const tah_weights *w, int features, int digits);
void column_images(hipStream_t s, const tah_weights *w, const float *col_kv, int features, int digits, uint8_t *out);
void assemble_tokens(hipStream_t s, const tah_weights *w, const float *cells, int n, int features, float *tok);
// The column stage written straight into the row stage's tokens tok [n][cls + features][e] (no copy), where every
// column block runs as one fused kernel (column_tokens_fits: one label digit, the fused shapes); with kv as well
// the last column block forms the first row block's keys and values there ([n][T][2 e]: row_stage_kv of the row
// stage's scratch, for row_stage with kv_ready; where row_stage_takes_kv), the class tokens' from cls_kv
// (class_token_kv). scratch holds column_stage_floats floats.
bool column_tokens_fits(const tah_weights *w, int n, int features, int digits);
void column_stage_tokens(hipStream_t s, const tah_weights *w, const float *col_kv, const float *x, int n,
                         int features, float *tok, float *kv, const float *cls_kv, float *scratch,
                         const uint8_t *col_images = nullptr);
// The first row block's keys and values of the class tokens, [cls][2 e] into out (tmp: cls e floats).
void class_token_kv(hipStream_t s, const tah_weights *w, float *out, float *tmp);
size_t row_stage_floats(const tah_weights *w, int n, int T);
bool row_stage_takes_kv(const tah_weights *w, int n, int T);
float *row_stage_kv(const tah_weights *w, int n, int T, float *scratch);
// kv_ready: the first row block's keys and values are in row_stage_kv(scratch) already (row_stage_takes_kv).
void row_stage(hipStream_t s, const tah_weights *w, float *tok, int n, int T, const float *cosv, const float *sinv,
               float *rep, float *scratch, bool kv_ready = false);
// att: att_bytes of scratch (the fused kernel needs cell_block_work_bytes(groups) of it, else M e floats)
// ready: the groups' images for the fused kernel (cell_images of kvbase), or nullptr.
void column_block(hipStream_t s, const tah_weights *w, const DevBlock &b, float *cells, int n, int groups, size_t sr,
                  size_t sg, const float *kvbase, size_t gstride, float *t, float *q, float *att, size_t att_bytes,
                  float *mid, const uint8_t *ready = nullptr);

// The column stage of a fit (fit_stages.hip).
void fit_cells(hipStream_t s, const tah_weights *w, const float *x, int rows, int features, int g0, int gb, float *cells);
void add_y_cells(hipStream_t s, const tah_weights *w, const float *y, int rows, int gb, int digits, int divisor, int base,
                 float *cells);
void scale_by(hipStream_t s, size_t count, const float *src, float f, float *dst);
void add_to(hipStream_t s, size_t count, const float *x, float *sum);
void add_ind(hipStream_t s, size_t count, int inds, int e, const float *ind, float *hid);
void col_records(hipStream_t s, int gb, int inds, int e, const float *kv2, float *col_kv, size_t gstride, size_t off, int g0);
// cells between the trait's row-major [rows][g][e] and the fit's group-major [g][rows][e] (to_group_major says which
// way).
void regroup(hipStream_t s, int rows, int g, int e, const float *src, float *dst, bool to_group_major);
void tokens_gmajor(hipStream_t s, const tah_weights *w, int rb, int r0, int rows, int features, const float *emb, float *tok);
size_t ind_attention_work_bytes(const tah_weights *w, int rows, int gb);
void ind_attention(hipStream_t s, const tah_weights *w, int rows, int gb, const float *indq, const float *kv, float *out,
                   void *work);

}  // namespace tah
