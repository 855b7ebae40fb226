// The column and row stages of a fit on the card (the reference's Attend::columns and Attend::rows,
// src/fit.rs:54-65, with the CPU loops they replace at src/fit.rs:326-423 and src/fit.rs:486-540), keeping the
// cells resident between the two stages.
//
// Per batch of feature groups (cells [groups][rows][e], group-major so each group's cells are contiguous):
// input layer and target embedding (per label digit), then per column block: the inducing points' queries attend
// to the group's cells (k_ind_attn16: online softmax over key blocks of 64 cells, fp32 MFMA, split over key ranges
// and merged as in the in-context attention), the inducing points' output projection and feed-forward, their keys
// and values for the second attention written straight into the column cache layout, and the cells' own block
// against them (column_block, shared with prediction).
#include <algorithm>

#include "common.hpp"
#include "device_math.hpp"

namespace tah {

static dim3 blocks_of(size_t count) { return dim3((unsigned)((count + 255) / 256)); }

// cells [gb][rows][e] of feature groups g0.. through the input layer.
__global__ __launch_bounds__(256) void k_fit_cells(int rows, int features, int g0, int gb, int group, int e,
                                                    const float *__restrict__ x, const float *__restrict__ in_w,
                                                    const float *__restrict__ in_b, float *__restrict__ cells) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)gb * rows * e) return;
    const int o = (int)(i % e);
    const size_t r = (i / e) % rows;
    const int g = g0 + (int)(i / ((size_t)e * rows));
    const float *xr = x + r * features;
    float vals[8];
    bool missing = true;
    for (int k = 0; k < group; k++) {
        vals[k] = xr[(g + (1 << k)) % features];
        missing = missing && vals[k] == -100.0f;
    }
    if (missing) {
        cells[i] = -100.0f;
        return;
    }
    float s = 0.0f;
    for (int k = 0; k < group; k++) s += in_w[o * group + k] * vals[k];
    cells[i] = s + in_b[o];
}

// cells [gb][rows][e] += the target's embedding (Model::add_y, src/model.rs:188-200) of digit `(y / divisor) % base`
// (or y itself with one digit, or the number y for a regression model).
__global__ __launch_bounds__(256) void k_add_y(int rows, int gb, int e, int max_classes, int digits, int divisor, int base,
                                                const float *__restrict__ y, const float *__restrict__ table,
                                                float *__restrict__ cells) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)gb * rows * e) return;
    const int o = (int)(i % e);
    const size_t r = (i / e) % rows;
    if (max_classes > 0) {
        const int cls = digits > 1 ? ((int)y[r] / divisor) % base : (int)y[r];
        cells[i] += table[(size_t)cls * e + o];
    } else {
        cells[i] += table[o] * y[r] + table[e + o];
    }
}

__global__ __launch_bounds__(256) void k_scale_by(size_t count, const float *__restrict__ src, float f, float *__restrict__ dst) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) dst[i] = src[i] * f;
}

__global__ __launch_bounds__(256) void k_add_to(size_t count, const float *__restrict__ x, float *__restrict__ sum) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) sum[i] += x[i];
}

// hid [gb * inds][e] += ind [inds][e] (the inducing points' residual, src/fit.rs:388-390)
__global__ __launch_bounds__(256) void k_add_ind(size_t count, int inds, int e, const float *__restrict__ ind,
                                                  float *__restrict__ hid) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) hid[i] += ind[(i / e) % inds * e + i % e];
}

// kv2 [gb * inds][2e] to the column cache: for group g0 + gl, rec = col_kv + (g0 + gl) * gstride + off holds
// K [e][inds] then V [e][inds] (src/fit.rs:394-403).
__global__ __launch_bounds__(256) void k_col_records(int gb, int inds, int e, const float *__restrict__ kv2,
                                                      float *__restrict__ col_kv, size_t gstride, size_t off, int g0) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)gb * 2 * e * inds) return;
    const int k = (int)(i % inds);
    const int j = (int)((i / inds) % (2 * e));
    const int gl = (int)(i / ((size_t)inds * 2 * e));
    col_kv[(size_t)(g0 + gl) * gstride + off + (size_t)j * inds + k] = kv2[((size_t)gl * inds + k) * 2 * e + j];
}

// The inducing points' queries indq [inds][e] over one group's cells, keys and values from kv [gb][rows][2e].
// grid (gb, heads, query tiles of 64 x splits); 256 threads; head width 16.
__global__ __launch_bounds__(256) void k_ind_attn16(int rows, int inds, int e, int heads, const float *__restrict__ indq,
                                                     const float *__restrict__ kv, int kb_per_split,
                                                     float *__restrict__ part_o, float *__restrict__ part_ml,
                                                     float *__restrict__ out) {
    __shared__ float Ks[16][68];
    __shared__ float Vs[16][68];
    const int gl = blockIdx.x, h = blockIdx.y;
    const int ntq = inds / 64, qt = blockIdx.z % ntq, split = blockIdx.z / ntq, splits = gridDim.z / ntq;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const int qi = qt * 64 + wave * 16 + r16;
    const float4 qv = *reinterpret_cast<const float4 *>(indq + (size_t)qi * e + h * 16 + 4 * g4);
    const float qa[4] = {qv.x, qv.y, qv.z, qv.w};
    const int n_kb = (rows + 63) / 64;
    const int kb0 = split * kb_per_split, kb1 = min(n_kb, kb0 + kb_per_split);
    const float *base = kv + (size_t)gl * rows * 2 * e;
    float m = -INFINITY, l = 0.0f;
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const int lk = tid >> 2, c4 = (tid & 3) * 4;
    for (int kb = kb0; kb < kb1; kb++) {
        const int key0 = kb * 64;
        float4 kk = make_float4(0.0f, 0.0f, 0.0f, 0.0f), vv = kk;
        if (key0 + lk < rows) {
            const float *row = base + (size_t)(key0 + lk) * 2 * e + h * 16 + c4;
            kk = *reinterpret_cast<const float4 *>(row);
            vv = *reinterpret_cast<const float4 *>(row + e);
        }
        __syncthreads();
        Ks[c4][lk] = kk.x;
        Ks[c4 + 1][lk] = kk.y;
        Ks[c4 + 2][lk] = kk.z;
        Ks[c4 + 3][lk] = kk.w;
        Vs[c4][lk] = vv.x;
        Vs[c4 + 1][lk] = vv.y;
        Vs[c4 + 2][lk] = vv.z;
        Vs[c4 + 3][lk] = vv.w;
        __syncthreads();
        floatx4 sacc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            sacc[kt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < 4; t++) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(Ks[4 * g4 + t][16 * kt + r16], qa[t], sacc[kt], 0, 0, 0);
        }
        float mb = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                if (key0 + 16 * kt + 4 * g4 + v >= rows) sacc[kt][v] = -INFINITY;
                mb = fmaxf(mb, sacc[kt][v]);
            }
        mb = fmaxf(mb, __shfl_xor(mb, 16, 64));
        mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
        const float mnew = fmaxf(m, mb);
        const float alpha = fast_exp(m - mnew);
        float lb = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                sacc[kt][v] = fast_exp(sacc[kt][v] - mnew);
                lb += sacc[kt][v];
            }
        lb += __shfl_xor(lb, 16, 64);
        lb += __shfl_xor(lb, 32, 64);
        l = l * alpha + lb;
        m = mnew;
        acc *= alpha;
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            const float4 v4 = *reinterpret_cast<const float4 *>(&Vs[r16][16 * kt + 4 * g4]);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.x, sacc[kt][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.y, sacc[kt][1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.z, sacc[kt][2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(v4.w, sacc[kt][3], acc, 0, 0, 0);
        }
    }
    const size_t qr = (size_t)gl * inds + qi;  // the (group, inducing point) item
    if (splits == 1) {
        const float inv = 1.0f / l;
        *reinterpret_cast<float4 *>(out + qr * e + h * 16 + 4 * g4) = make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
    } else {
        const size_t nq = (size_t)gridDim.x * inds;
        const size_t at = ((size_t)split * nq + qr) * heads + h;
        *reinterpret_cast<float4 *>(part_o + at * 16 + 4 * g4) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        if (g4 == 0) {
            part_ml[at * 2] = m;
            part_ml[at * 2 + 1] = l;
        }
    }
}

// Any head width (the tiny test models): one thread per (group, inducing point, head), streaming over the rows.
__global__ __launch_bounds__(256) void k_ind_attn_plain(int gb, int rows, int inds, int e, int heads,
                                                         const float *__restrict__ indq, const float *__restrict__ kv,
                                                         float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)gb * inds * heads) return;
    const int h = (int)(i % heads), qi = (int)((i / heads) % inds), gl = (int)(i / ((size_t)heads * inds));
    const int hd = e / heads;
    const float *qr = indq + (size_t)qi * e + h * hd;
    const float *base = kv + (size_t)gl * rows * 2 * e;
    float *o = out + ((size_t)gl * inds + qi) * e + h * hd;
    float m = -INFINITY, l = 0.0f;
    for (int c = 0; c < hd; c++) o[c] = 0.0f;
    for (int r = 0; r < rows; r++) {
        const float *row = base + (size_t)r * 2 * e;
        float s = 0.0f;
        for (int c = 0; c < hd; c++) s += qr[c] * row[h * hd + c];
        const float mnew = fmaxf(m, s);
        const float alpha = fast_exp(m - mnew), p = fast_exp(s - mnew);
        l = l * alpha + p;
        for (int c = 0; c < hd; c++) o[c] = o[c] * alpha + p * row[e + h * hd + c];
        m = mnew;
    }
    for (int c = 0; c < hd; c++) o[c] /= l;
}

// tok [rb][T][e]: class tokens then cells of rows r0.. from emb [features][rows][e]. A workgroup per row, 16 bytes a
// thread (e a multiple of 4).
__global__ __launch_bounds__(256) void k_tokens_gmajor(int rb, int r0, int rows, int cls, int features, int e,
                                                        const float *__restrict__ cls_tokens,
                                                        const float *__restrict__ emb, float *__restrict__ tok) {
    const int r = blockIdx.x;
    if (r >= rb) return;
    const int e4 = e / 4, T = cls + features;
    float4 *dst = reinterpret_cast<float4 *>(tok + (size_t)r * T * e);
    for (int i = threadIdx.x; i < T * e4; i += 256) {
        const int t = i / e4, o = i - t * e4;
        const float4 *src = t < cls ? reinterpret_cast<const float4 *>(cls_tokens + (size_t)t * e)
                                    : reinterpret_cast<const float4 *>(emb + ((size_t)(t - cls) * rows + r0 + r) * e);
        dst[i] = src[o];
    }
}

// Cells of e floats between [rows][g][e] and [g][rows][e]: e / 4 threads a cell, 16 bytes each (e a multiple of 4).
__global__ __launch_bounds__(256) void k_regroup(int rows, int g, int e, const float *__restrict__ src,
                                                  float *__restrict__ dst, bool to_gmajor) {
    const int e4 = e / 4, per = 256 / e4;
    const int slot = threadIdx.x / e4, o = threadIdx.x - slot * e4;
    const long cell = (long)blockIdx.x * per + slot;  // in the destination's order
    if (slot >= per || cell >= (long)rows * g) return;
    long from;
    if (to_gmajor) {
        const long gi = cell / rows, r = cell - gi * rows;
        from = r * g + gi;
    } else {
        const long r = cell / g, gi = cell - r * g;
        from = gi * rows + r;
    }
    reinterpret_cast<float4 *>(dst)[cell * e4 + o] = reinterpret_cast<const float4 *>(src)[from * e4 + o];
}

void merge_splits(hipStream_t s, int nq, int d, int heads, int splits, const float *part_o, const float *part_ml,
                  float *out);

// ---- launchers ---------------------------------------------------------------------------------------------
void fit_cells(hipStream_t s, const tah_weights *w, const float *x, int rows, int features, int g0, int gb, float *cells) {
    if (w->group > 8 || w->group < 1) throw ArgError{"column stage: feature group size must be 1..8"};
    const size_t count = (size_t)gb * rows * w->e;
    hipLaunchKernelGGL(k_fit_cells, blocks_of(count), dim3(256), 0, s, rows, features, g0, gb, w->group, w->e, x, w->in_w,
                       w->in_b, cells);
    TAH_LAUNCHED();
}

void add_y_cells(hipStream_t s, const tah_weights *w, const float *y, int rows, int gb, int digits, int divisor, int base,
                 float *cells) {
    const size_t count = (size_t)gb * rows * w->e;
    hipLaunchKernelGGL(k_add_y, blocks_of(count), dim3(256), 0, s, rows, gb, w->e, w->max_classes, digits, divisor, base, y,
                       w->col_y, cells);
    TAH_LAUNCHED();
}

void scale_by(hipStream_t s, size_t count, const float *src, float f, float *dst) {
    hipLaunchKernelGGL(k_scale_by, blocks_of(count), dim3(256), 0, s, count, src, f, dst);
    TAH_LAUNCHED();
}

void add_to(hipStream_t s, size_t count, const float *x, float *sum) {
    hipLaunchKernelGGL(k_add_to, blocks_of(count), dim3(256), 0, s, count, x, sum);
    TAH_LAUNCHED();
}

void add_ind(hipStream_t s, size_t count, int inds, int e, const float *ind, float *hid) {
    hipLaunchKernelGGL(k_add_ind, blocks_of(count), dim3(256), 0, s, count, inds, e, ind, hid);
    TAH_LAUNCHED();
}

void col_records(hipStream_t s, int gb, int inds, int e, const float *kv2, float *col_kv, size_t gstride, size_t off, int g0) {
    const size_t count = (size_t)gb * 2 * e * inds;
    hipLaunchKernelGGL(k_col_records, blocks_of(count), dim3(256), 0, s, gb, inds, e, kv2, col_kv, gstride, off, g0);
    TAH_LAUNCHED();
}

void regroup(hipStream_t s, int rows, int g, int e, const float *src, float *dst, bool to_group_major) {
    if (e % 4 || e > 1024) throw ArgError{"regroup: cell width must be a multiple of 4, at most 1024"};
    const size_t per = 256 / (e / 4);
    hipLaunchKernelGGL(k_regroup, dim3((unsigned)(((size_t)rows * g + per - 1) / per)), dim3(256), 0, s, rows, g, e, src,
                       dst, to_group_major);
    TAH_LAUNCHED();
}

void tokens_gmajor(hipStream_t s, const tah_weights *w, int rb, int r0, int rows, int features, const float *emb, float *tok) {
    if (w->e % 4) throw ArgError{"row stage: embedding width must be a multiple of 4"};
    hipLaunchKernelGGL(k_tokens_gmajor, dim3(rb), dim3(256), 0, s, rb, r0, rows, w->cls, features, w->e, w->cls_tokens,
                       emb, tok);
    TAH_LAUNCHED();
}

static int ind_splits(const tah_weights *w, int rows, int gb) {
    const int n_kb = (rows + 63) / 64;
    const int tiles = gb * w->col_heads * std::max(1, w->inds / 64);
    int want = std::max(1, 1024 / std::max(1, tiles));
    want = std::min(want, std::max(1, n_kb / 2));
    const int per = (n_kb + want - 1) / want;
    return (n_kb + per - 1) / per;
}

static bool ind_mfma(const tah_weights *w) { return w->e / w->col_heads == 16 && w->inds % 64 == 0; }

size_t ind_attention_work_bytes(const tah_weights *w, int rows, int gb) {
    if (!ind_mfma(w)) return 0;
    const int splits = ind_splits(w, rows, gb);
    if (splits == 1) return 0;
    return sizeof(float) * (size_t)splits * gb * w->inds * w->col_heads * (w->e / w->col_heads + 2) + 256;
}

// The inducing points' queries indq [inds][e] over each of gb groups' cells (kv [gb][rows][2e]) to out
// [gb * inds][e], normalised.
void ind_attention(hipStream_t s, const tah_weights *w, int rows, int gb, const float *indq, const float *kv, float *out,
                   void *work) {
    const int e = w->e, heads = w->col_heads, inds = w->inds;
    if (!ind_mfma(w)) {
        hipLaunchKernelGGL(k_ind_attn_plain, blocks_of((size_t)gb * inds * heads), dim3(256), 0, s, gb, rows, inds, e, heads,
                           indq, kv, out);
        TAH_LAUNCHED();
        return;
    }
    const int splits = ind_splits(w, rows, gb);
    const int n_kb = (rows + 63) / 64;
    const int per = (n_kb + splits - 1) / splits;
    float *part_o = splits > 1 ? static_cast<float *>(work) : nullptr;
    float *part_ml = splits > 1 ? part_o + (size_t)splits * gb * inds * heads * (e / heads) : nullptr;
    hipLaunchKernelGGL(k_ind_attn16, dim3(gb, heads, (inds / 64) * splits), dim3(256), 0, s, rows, inds, e, heads, indq, kv,
                       per, part_o, part_ml, out);
    TAH_LAUNCHED();
    if (splits > 1) merge_splits(s, gb * inds, e, heads, splits, part_o, part_ml, out);
}

}  // namespace tah
