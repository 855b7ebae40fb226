// The column and row stages on the card: a test (or training) table's feature rows to row representations.
//
// Column stage (src/predict.rs:282-353, src/fit.rs:326-423): every cell is the input layer applied to three of its
// row's features (src/nn.rs:424-429; all -100 stays -100), then per column block a whole attention block against
// that feature group's 128 cached inducing-point keys and values (cached_block, src/nn.rs:291-301). All cells of
// all rows go through each dense layer as one GEMM; the attention is grouped by feature group: a workgroup holds
// one group's K and V for one head in LDS and attends 64 cells to its 128 keys with fp32 MFMA (head width 16),
// scores transposed so that each lane owns one cell, as in the in-context kernel.
//
// Row stage (row_forward, src/nn.rs:357-419): per row, the class tokens and the row's cells attend to each other
// with non-interleaved rotary positions (queries also scaled by 1/sqrt(head width)); the last block updates only
// the class tokens, which are then normalised and laid end to end as the row's representation.
#include <algorithm>

#include "common.hpp"
#include "device_math.hpp"

namespace tah {

// ---- input layer -------------------------------------------------------------------------------------------
// A workgroup per table row, four outputs a thread (e a multiple of 4); 32-bit index arithmetic throughout. From
// INPUT_ROWS_MIN rows (2,048 rows: 48.7 -> about 33 us); below, where one row's workgroup would serialise its cells,
// k_input_cells_few (one row: 0.642 against 0.652 ms a prediction; 256 rows 1.284 against 1.290 ms).
constexpr int INPUT_ROWS_MIN = 1024;
// The output rows hold cls class tokens (cls_tokens [cls][e]) before the cells: [n][cls + features][e] (cls 0: the
// cells alone); with kv as well the first row block's keys and values [n][cls + features][2 e] get the class tokens'
// (cls_kv [cls][2 e]).
__global__ __launch_bounds__(256) void k_input_cells(int n, int features, int group, int e, const float *__restrict__ x,
                                                      const float *__restrict__ in_w, const float *__restrict__ in_b,
                                                      float *__restrict__ cells, int cls,
                                                      const float *__restrict__ cls_tokens, float *__restrict__ kv,
                                                      const float *__restrict__ cls_kv) {
    // a workgroup per table row: the row's values in LDS; thread t keeps the weights of outputs 4 (t % 32) + 0..3
    // (of each 128 the cell has) and writes them for cells t / 32, t / 32 + 8, ...
    __shared__ float xs[1024];
    const int r = blockIdx.x;
    if (r >= n) return;
    for (int j = threadIdx.x; j < features; j += 256) xs[j] = x[(size_t)r * features + j];
    const size_t T = (size_t)cls + features;
    if (cls > 0) {
        float4 *t4 = reinterpret_cast<float4 *>(cells + (size_t)r * T * e);
        const float4 *c4 = reinterpret_cast<const float4 *>(cls_tokens);
        for (int i = threadIdx.x; i < cls * e / 4; i += 256) t4[i] = c4[i];
        if (kv) {
            float4 *k4 = reinterpret_cast<float4 *>(kv + (size_t)r * T * 2 * e);
            const float4 *ck4 = reinterpret_cast<const float4 *>(cls_kv);
            for (int i = threadIdx.x; i < cls * e / 2; i += 256) k4[i] = ck4[i];
        }
    }
    __syncthreads();
    const int q = threadIdx.x & 31;
    float *row = cells + ((size_t)r * T + cls) * e;
    for (int o = 4 * q; o < e; o += 128) {
        // in_w rows o .. o + 3 are 4 * group consecutive floats (16-byte aligned: o is a multiple of 4)
        float wv[32];
        const float4 *wp = reinterpret_cast<const float4 *>(in_w + (size_t)o * group);
        for (int i = 0; i < group; i++) {
            const float4 t = wp[i];
            wv[4 * i] = t.x; wv[4 * i + 1] = t.y; wv[4 * i + 2] = t.z; wv[4 * i + 3] = t.w;
        }
        const float4 bb = *reinterpret_cast<const float4 *>(in_b + o);
        for (int g = threadIdx.x >> 5; g < features; g += 8) {
            float vals[8];
            bool missing = true;
            for (int k = 0; k < group; k++) {
                int j = g + (1 << k);
                while (j >= features) j -= features;
                vals[k] = xs[j];
                missing = missing && vals[k] == -100.0f;
            }
            float4 v = make_float4(-100.0f, -100.0f, -100.0f, -100.0f);
            if (!missing) {
                float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                for (int k = 0; k < group; k++) {
#pragma unroll
                    for (int u = 0; u < 4; u++) acc[u] += wv[u * group + k] * vals[k];
                }
                v = make_float4(acc[0] + bb.x, acc[1] + bb.y, acc[2] + bb.z, acc[3] + bb.w);
            }
            *reinterpret_cast<float4 *>(row + (size_t)g * e + o) = v;
        }
    }
}

// Few table rows (below INPUT_ROWS_MIN): 32 threads a cell, so that the cells of one row spread over workgroups;
// row r's cells at cells + r ldr (the class tokens, if any, by k_class_tokens).
__global__ __launch_bounds__(256) void k_input_cells_few(int n, int features, int group, int e, const float *__restrict__ x,
                                                          const float *__restrict__ in_w, const float *__restrict__ in_b,
                                                          float *__restrict__ cells, size_t ldr) {
    const int cell = blockIdx.x * 8 + (threadIdx.x >> 5), q = threadIdx.x & 31;
    if (cell >= n * features) return;
    const int r = cell / features, g = cell - r * features;
    const float *xr = x + (size_t)r * features;
    float vals[8];
    bool missing = true;
    for (int k = 0; k < group; k++) {
        int j = g + (1 << k);
        while (j >= features) j -= features;
        vals[k] = xr[j];
        missing = missing && vals[k] == -100.0f;
    }
    float *dst = cells + (size_t)r * ldr + (size_t)g * e;
    for (int o = 4 * q; o < e; o += 128) {
        float4 v = make_float4(-100.0f, -100.0f, -100.0f, -100.0f);
        if (!missing) {
            float wv[32];
            const float4 *wp = reinterpret_cast<const float4 *>(in_w + (size_t)o * group);
            for (int i = 0; i < group; i++) {
                const float4 t = wp[i];
                wv[4 * i] = t.x; wv[4 * i + 1] = t.y; wv[4 * i + 2] = t.z; wv[4 * i + 3] = t.w;
            }
            const float4 bb = *reinterpret_cast<const float4 *>(in_b + o);
            float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            for (int k = 0; k < group; k++) {
#pragma unroll
                for (int u = 0; u < 4; u++) acc[u] += wv[u * group + k] * vals[k];
            }
            v = make_float4(acc[0] + bb.x, acc[1] + bb.y, acc[2] + bb.z, acc[3] + bb.w);
        }
        *reinterpret_cast<float4 *>(dst + o) = v;
    }
}

// ---- cells against a group's inducing points: head width 16, 16 * NT keys ----------------------------------------
// grid (tiles of 64 rows, heads, groups); 256 threads. q and out hold cell (r, g) at row r * sr + g * sg of e
// numbers ([n][features][e] at prediction, [groups][rows][e] at fit); group g's keys and values are
// K = kvbase + g * gstride ([e][inds]) and V = K + e * inds.
template <int NT>
__global__ __launch_bounds__(256) void k_cell_attn16(int n, size_t sr, size_t sg, int e, const float *__restrict__ q,
                                                      const float *__restrict__ kvbase, size_t gstride,
                                                      float *__restrict__ out) {
    constexpr int INDS = 16 * NT;
    __shared__ float Ks[16][INDS + 4];
    __shared__ float Vs[16][INDS + 4];
    const int h = blockIdx.y, g = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const float *K = kvbase + (size_t)g * gstride, *V = K + (size_t)e * INDS;
    for (int i = tid; i < 16 * INDS; i += 256) {
        const int c = i / INDS, k = i % INDS;
        Ks[c][k] = K[(size_t)(h * 16 + c) * INDS + k];
        Vs[c][k] = V[(size_t)(h * 16 + c) * INDS + k];
    }
    __syncthreads();
    const int r = blockIdx.x * 64 + wave * 16 + r16;
    const bool live = r < n;
    const size_t m = (size_t)r * sr + (size_t)g * sg;
    float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (live) qv = *reinterpret_cast<const float4 *>(q + m * e + h * 16 + 4 * g4);
    const float qa[4] = {qv.x, qv.y, qv.z, qv.w};
    floatx4 sacc[NT];
#pragma unroll
    for (int kt = 0; kt < NT; kt++) {
        sacc[kt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; t++) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(Ks[4 * g4 + t][16 * kt + r16], qa[t], sacc[kt], 0, 0, 0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < NT; kt++)
#pragma unroll
        for (int v = 0; v < 4; v++) mx = fmaxf(mx, sacc[kt][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float l = 0.0f;
#pragma unroll
    for (int kt = 0; kt < NT; kt++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            sacc[kt][v] = fast_exp(sacc[kt][v] - mx);
            l += sacc[kt][v];
        }
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kt = 0; kt < NT; kt++) {
        const float4 vv = *reinterpret_cast<const float4 *>(&Vs[r16][16 * kt + 4 * g4]);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, sacc[kt][0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, sacc[kt][1], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, sacc[kt][2], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, sacc[kt][3], acc, 0, 0, 0);
    }
    if (live) {
        const float inv = 1.0f / l;
        *reinterpret_cast<float4 *>(out + m * e + h * 16 + 4 * g4) = make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
    }
}

// ---- cells against their group's inducing keys on split-fp16 MFMA: head width 16, 128 keys ----------------------
// grid (ceil(n / 128), heads, groups); 256 threads. The group's keys and values of head h (the column cache,
// [coordinate][key] f32) are split into fp16 hi/lo in LDS by the workgroup (one key a thread, the head's largest
// magnitude scaled below 2^14), laid out as in k_row_attn_x3; wavefront w takes cells of rows 128 x + 32 w + 0..31.
// S^T = K Q^T over four 32-key tiles, a plain softmax over the 128 keys, O^T = V^T P^T.
__global__ __launch_bounds__(256) void k_cell_attn_x3(int n, size_t sr, size_t sg, int e, const float *__restrict__ q,
                                                       const float *__restrict__ kvbase, size_t gstride,
                                                       float *__restrict__ out) {
    constexpr int INDS = 128;
    __shared__ __align__(16) _Float16 Kh[2][128][8], Kl[2][128][8];
    __shared__ __align__(16) _Float16 Vh[8][2][16][8], Vl[8][2][16][8];
    __shared__ float red[2][4];
    const int h = blockIdx.y, grp = blockIdx.z;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *K = kvbase + (size_t)grp * gstride, *V = K + (size_t)e * INDS;
    float kv[16], vv[16];
    if (tid < INDS) {
#pragma unroll
        for (int c = 0; c < 16; c++) {
            kv[c] = K[(size_t)(h * 16 + c) * INDS + tid];
            vv[c] = V[(size_t)(h * 16 + c) * INDS + tid];
        }
    } else {
#pragma unroll
        for (int c = 0; c < 16; c++) kv[c] = vv[c] = 0.0f;
    }
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        mk = fmaxf(mk, fabsf(kv[i]));
        mv = fmaxf(mv, fabsf(vv[i]));
    }
    mk = wave_max(mk);
    mv = wave_max(mv);
    if (lane == 0) {
        red[0][wave] = mk;
        red[1][wave] = mv;
    }
    __syncthreads();
    const int sk = shift_for_max(fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3])));
    const int sv = shift_for_max(fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3])));
    if (tid < INDS) {
        halfx8 h0, l0, h1, l1;
        split8(kv, ldexpf(1.0f, sk), h0, l0);
        split8(kv + 8, ldexpf(1.0f, sk), h1, l1);
        *reinterpret_cast<halfx8 *>(&Kh[0][tid][0]) = h0;
        *reinterpret_cast<halfx8 *>(&Kl[0][tid][0]) = l0;
        *reinterpret_cast<halfx8 *>(&Kh[1][tid][0]) = h1;
        *reinterpret_cast<halfx8 *>(&Kl[1][tid][0]) = l1;
        const int st = tid >> 4, kg = (tid >> 3) & 1, t8 = tid & 7;
        const int sw = (2 * st + kg) & 15;
        const float fv = ldexpf(1.0f, sv);
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const float x = vv[c] * fv;
            const _Float16 hi = (_Float16)x;
            Vh[st][kg][c ^ sw][t8] = hi;
            Vl[st][kg][c ^ sw][t8] = (_Float16)(x - (float)hi);
        }
    }
    __syncthreads();
    const int r32 = lane & 31, g = lane >> 5;
    const int r = blockIdx.x * 128 + wave * 32 + r32;
    if (blockIdx.x * 128 + wave * 32 >= n) return;
    const bool live = r < n;
    const size_t m = (size_t)(live ? r : 0) * sr + (size_t)grp * sg;
    float qv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (live) load8(q + m * e + h * 16 + 8 * g, qv);
    float qmax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) qmax = fmaxf(qmax, fabsf(qv[k]));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
    const int sq = shift_for_max(qmax);
    halfx8 qh, ql;
    split8(qv, ldexpf(1.0f, sq), qh, ql);
    const float to_log2 = ldexpf(LOG2E, -(sk + sq));
    const int krow = sigma32(r32);
    floatx16 sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
#pragma unroll
        for (int v = 0; v < 16; v++) sc[kt][v] = 0.0f;
        const int key = 32 * kt + krow;
        const halfx8 ah = *reinterpret_cast<const halfx8 *>(&Kh[g][key][0]);
        const halfx8 al = *reinterpret_cast<const halfx8 *>(&Kl[g][key][0]);
        sc[kt] = mfma16x3(ah, al, qh, ql, sc[kt]);
#pragma unroll
        for (int v = 0; v < 16; v++) mx = fmaxf(mx, sc[kt][v]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float off = 12.0f - mx * to_log2;
    float l = 0.0f;
    halfx8 ph[8], pl[8];
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float p[8];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                p[t] = exp2_hw(fmaf(sc[kt][8 * hh + t], to_log2, off));
                l += p[t];
            }
            split8(p, 1.0f, ph[2 * kt + hh], pl[2 * kt + hh]);
        }
    l += __shfl_xor(l, 32, 64);
    floatx16 o;
#pragma unroll
    for (int v = 0; v < 16; v++) o[v] = 0.0f;
    halfx8 zero8;
#pragma unroll
    for (int t = 0; t < 8; t++) zero8[t] = (_Float16)0.0f;
#pragma unroll
    for (int st = 0; st < 8; st++) {
        halfx8 ah = zero8, al = zero8;
        if (r32 < 16) {
            const int row = r32 ^ ((2 * st + g) & 15);
            ah = *reinterpret_cast<const halfx8 *>(&Vh[st][g][row][0]);
            al = *reinterpret_cast<const halfx8 *>(&Vl[st][g][row][0]);
        }
        o = mfma16x3(ah, al, ph[st], pl[st], o);
    }
    if (!live) return;
    const float f = ldexpf(1.0f, -sv) / l;
    float *dst = out + m * e + h * 16;
    *reinterpret_cast<float4 *>(dst + 4 * g) = make_float4(o[0] * f, o[1] * f, o[2] * f, o[3] * f);
    *reinterpret_cast<float4 *>(dst + 8 + 4 * g) = make_float4(o[4] * f, o[5] * f, o[6] * f, o[7] * f);
}

// The same for a few rows (at most CELL_FEW_ROWS): a wavefront per (group, head), four a workgroup, lane = keys
// lane and lane + 64, in plain f32: the head's 16 key and value coordinates of the lane's two keys read once
// (each a coalesced 256-byte row of the column cache), then per row the scores, a softmax by wavefront reductions
// and the 16 weighted sums (one row: 10.5 us where k_cell_attn_x3 staged split images for 128-row tiles).
constexpr int CELL_FEW_ROWS = 3;
__global__ __launch_bounds__(256) void k_cell_attn_few(int n, int groups, int heads, size_t sr, size_t sg, int e,
                                                        const float *__restrict__ q, const float *__restrict__ kvbase,
                                                        size_t gstride, float *__restrict__ out) {
    constexpr int INDS = 128;
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= groups * heads) return;
    const int grp = item / heads, h = item % heads;
    const float *K = kvbase + (size_t)grp * gstride, *V = K + (size_t)e * INDS;
    float k0[16], k1[16], v0[16], v1[16];
#pragma unroll
    for (int c = 0; c < 16; c++) {
        const size_t row = (size_t)(h * 16 + c) * INDS;
        k0[c] = K[row + lane];
        k1[c] = K[row + lane + 64];
        v0[c] = V[row + lane];
        v1[c] = V[row + lane + 64];
    }
    for (int r = 0; r < n; r++) {
        const size_t m = (size_t)r * sr + (size_t)grp * sg;
        const float *qr = q + m * e + h * 16;
        float qv[16];
#pragma unroll
        for (int c = 0; c < 16; c += 4) {
            const float4 x = *reinterpret_cast<const float4 *>(qr + c);
            qv[c] = x.x;
            qv[c + 1] = x.y;
            qv[c + 2] = x.z;
            qv[c + 3] = x.w;
        }
        float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
        for (int c = 0; c < 16; c++) {
            s0 += qv[c] * k0[c];
            s1 += qv[c] * k1[c];
        }
        const float mx = wave_max(fmaxf(s0, s1));
        const float p0 = fast_exp(s0 - mx), p1 = fast_exp(s1 - mx);
        const float l = wave_sum(p0 + p1);
        float o[16];
#pragma unroll
        for (int c = 0; c < 16; c++) o[c] = wave_sum(p0 * v0[c] + p1 * v1[c]);
        if (lane < 16) {
            float oc = o[0];
#pragma unroll
            for (int c = 1; c < 16; c++)
                if (lane == c) oc = o[c];
            out[m * e + h * 16 + lane] = oc / l;
        }
    }
}

// Any head width and key count (the tiny test models): one thread per (cell, head).
__global__ __launch_bounds__(256) void k_cell_attn_plain(int n, int groups, size_t sr, size_t sg, int e, int heads,
                                                          int inds, const float *__restrict__ q,
                                                          const float *__restrict__ kvbase, size_t gstride,
                                                          float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * groups * heads) return;
    const int h = (int)(i % heads);
    const size_t cell = i / heads;
    const int g = (int)(cell % groups), hd = e / heads;
    const size_t m = (cell / groups) * sr + (size_t)g * sg;
    const float *K = kvbase + (size_t)g * gstride, *V = K + (size_t)e * inds;
    const float *qr = q + m * e + h * hd;
    float mx = -INFINITY;
    for (int k = 0; k < inds; k++) {
        float s = 0.0f;
        for (int c = 0; c < hd; c++) s += qr[c] * K[(size_t)(h * hd + c) * inds + k];
        mx = fmaxf(mx, s);
    }
    float l = 0.0f;
    float *o = out + m * e + h * hd;
    for (int c = 0; c < hd; c++) o[c] = 0.0f;
    for (int k = 0; k < inds; k++) {
        float s = 0.0f;
        for (int c = 0; c < hd; c++) s += qr[c] * K[(size_t)(h * hd + c) * inds + k];
        const float p = fast_exp(s - mx);
        l += p;
        for (int c = 0; c < hd; c++) o[c] += p * V[(size_t)(h * hd + c) * inds + k];
    }
    for (int c = 0; c < hd; c++) o[c] /= l;
}

// ---- rotary positions --------------------------------------------------------------------------------------
// qkv [rows][3e] with rows = n * T token rows (position = row % T). Queries also take 1/sqrt(hd).
__global__ __launch_bounds__(256) void k_rope(size_t rows, int T, int e, int heads, int half,
                                               const float *__restrict__ cosv, const float *__restrict__ sinv,
                                               float *__restrict__ qkv, float inv) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * heads * half) return;
    const int k = (int)(i % half);
    const int h = (int)((i / half) % heads);
    const size_t row = i / ((size_t)half * heads);
    const int t = (int)(row % T), hd = 2 * half;
    const float c = cosv[t * half + k], s = sinv[t * half + k];
    float *qh = qkv + row * 3 * e + h * hd;
    const float a = qh[k], b = qh[k + half];
    qh[k] = (a * c - b * s) * inv;
    qh[k + half] = (b * c + a * s) * inv;
    float *kh = qh + e;
    const float ka = kh[k], kb = kh[k + half];
    kh[k] = ka * c - kb * s;
    kh[k + half] = kb * c + ka * s;
}

// ---- attention within each row: head width 16, up to 16 * NT tokens -------------------------------------------
// grid (rows, heads); 256 threads. Queries are the first nq_tok tokens of each row; out is [n][nq_tok][e].
template <int NT>
__global__ __launch_bounds__(256) void k_row_attn16(int n, int T, int nq_tok, int e, const float *__restrict__ qkv,
                                                     float *__restrict__ out) {
    constexpr int KT = 16 * NT;
    __shared__ float Ks[16][KT + 4];
    __shared__ float Vs[16][KT + 4];
    const int r = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, r16 = lane & 15, g4 = lane >> 4;
    const float *base = qkv + (size_t)r * T * 3 * e;
    for (int i = tid; i < 16 * KT; i += 256) {
        const int k = i >> 4, c = i & 15;
        const bool ok = k < T;
        Ks[c][k] = ok ? base[(size_t)k * 3 * e + e + h * 16 + c] : 0.0f;
        Vs[c][k] = ok ? base[(size_t)k * 3 * e + 2 * e + h * 16 + c] : 0.0f;
    }
    __syncthreads();
    for (int qt = wave; qt * 16 < nq_tok; qt += 4) {
        const int t = qt * 16 + r16;
        const bool live = t < nq_tok;
        float4 qv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (live) qv = *reinterpret_cast<const float4 *>(base + (size_t)t * 3 * e + h * 16 + 4 * g4);
        const float qa[4] = {qv.x, qv.y, qv.z, qv.w};
        floatx4 sacc[NT];
#pragma unroll
        for (int kt = 0; kt < NT; kt++) {
            sacc[kt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int s = 0; s < 4; s++) sacc[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(Ks[4 * g4 + s][16 * kt + r16], qa[s], sacc[kt], 0, 0, 0);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < NT; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                if (16 * kt + 4 * g4 + v >= T) sacc[kt][v] = -INFINITY;
                mx = fmaxf(mx, sacc[kt][v]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        float l = 0.0f;
#pragma unroll
        for (int kt = 0; kt < NT; kt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                sacc[kt][v] = fast_exp(sacc[kt][v] - mx);
                l += sacc[kt][v];
            }
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        floatx4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kt = 0; kt < NT; kt++) {
            const float4 vv = *reinterpret_cast<const float4 *>(&Vs[r16][16 * kt + 4 * g4]);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.x, sacc[kt][0], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.y, sacc[kt][1], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.z, sacc[kt][2], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(vv.w, sacc[kt][3], acc, 0, 0, 0);
        }
        if (live) {
            const float inv = 1.0f / l;
            *reinterpret_cast<float4 *>(out + ((size_t)r * nq_tok + t) * e + h * 16 + 4 * g4) =
                make_float4(acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
        }
    }
}

// ---- the class tokens' attention within each row: head width 16, at most 4 queries, T <= 128 ----------------------
// grid n rows; 64 x heads threads (at most 8 heads), wavefront h head h. Few queries against at most 128 keys: plain f32 arithmetic,
// each row's keys and values read once by its workgroup (the heads' slices of a token side by side). Lane l takes
// tokens l and l + 64: their keys (rotated, the k_rope formula) and values, the scores of the (rotated, 1 / sqrt(16))
// queries, the softmax over the row's tokens by wavefront reductions; the weights and values then go through LDS,
// and lane c = 16 i + j forms coordinate j of query i's output. Keys of token t of row r at kv + r * kv_row +
// t * kv_tok (values e floats further), query i at q + r * q_row + i * q_tok.
constexpr int CLS_MAXQ = 4;
__global__ __launch_bounds__(512) void k_cls_attn(int n, int T, int nq, int e, const float *__restrict__ kv,
                                                   size_t kv_row, int kv_tok, const float *__restrict__ q, size_t q_row,
                                                   int q_tok, const float *__restrict__ cosv,
                                                   const float *__restrict__ sinv, float *__restrict__ out) {
    __shared__ float ps[8][CLS_MAXQ][128];            // [head][query][token] weights
    __shared__ __align__(16) float vs[8][128][16];    // [head][token][coordinate] values
    const int r = blockIdx.x, h = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const float *kr = kv + (size_t)r * kv_row + h * 16;
    float k2[2][16];
    bool tl[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int t = lane + 64 * j;
        tl[j] = t < T;
        const float *kp = kr + (size_t)(tl[j] ? t : 0) * kv_tok;
        float v16[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 a = *reinterpret_cast<const float4 *>(kp + 4 * i);
            const float4 b = *reinterpret_cast<const float4 *>(kp + e + 4 * i);
            k2[j][4 * i] = a.x; k2[j][4 * i + 1] = a.y; k2[j][4 * i + 2] = a.z; k2[j][4 * i + 3] = a.w;
            v16[4 * i] = b.x; v16[4 * i + 1] = b.y; v16[4 * i + 2] = b.z; v16[4 * i + 3] = b.w;
        }
        float cs[8], sn[8];
        load8(cosv + (tl[j] ? t : 0) * 8, cs);
        load8(sinv + (tl[j] ? t : 0) * 8, sn);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float a = k2[j][k], b = k2[j][k + 8];
            k2[j][k] = a * cs[k] - b * sn[k];
            k2[j][k + 8] = b * cs[k] + a * sn[k];
        }
        if (tl[j]) {
#pragma unroll
            for (int c = 0; c < 16; c += 4)
                *reinterpret_cast<float4 *>(&vs[h][t][c]) = make_float4(v16[c], v16[c + 1], v16[c + 2], v16[c + 3]);
        }
    }
    float lsum[CLS_MAXQ];
#pragma unroll
    for (int i = 0; i < CLS_MAXQ; i++) {
        if (i >= nq) break;
        // query i of head h, rotated at position i and scaled by 1 / sqrt(16) (every lane reads the same 64 bytes)
        float qv[16];
        load8(q + (size_t)r * q_row + (size_t)i * q_tok + h * 16, qv);
        load8(q + (size_t)r * q_row + (size_t)i * q_tok + h * 16 + 8, qv + 8);
        float cs[8], sn[8];
        load8(cosv + i * 8, cs);
        load8(sinv + i * 8, sn);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float a = qv[k], b = qv[k + 8];
            qv[k] = (a * cs[k] - b * sn[k]) * 0.25f;
            qv[k + 8] = (b * cs[k] + a * sn[k]) * 0.25f;
        }
        float sc[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            float a = 0.0f;
#pragma unroll
            for (int c = 0; c < 16; c++) a += qv[c] * k2[j][c];
            sc[j] = tl[j] ? a : -INFINITY;
        }
        const float mx = wave_max(fmaxf(sc[0], sc[1]));
        float l = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const float pj = tl[j] ? exp2_hw((sc[j] - mx) * LOG2E) : 0.0f;
            ps[h][i][lane + 64 * j] = pj;
            l += pj;
        }
        lsum[i] = wave_sum(l);
    }
    __syncthreads();
    // lane 16 i + j: coordinate j of query i's output, the weighted values summed over the tokens in order
    const int qi = lane >> 4, c = lane & 15;
    if (qi >= nq) return;
    float o = 0.0f;
    for (int t = 0; t < T; t++) o += ps[h][qi][t] * vs[h][t][c];
    float l = lsum[0];
#pragma unroll
    for (int i = 1; i < CLS_MAXQ; i++)
        if (qi == i) l = lsum[i];
    out[((size_t)r * nq + qi) * e + h * 16 + c] = o / l;
}

// ---- attention within each row on split-fp16 MFMA, rotary positions folded in: head width 16, T <= 128 ---------
// grid (rows, heads); 256 threads. The row's keys and values of head h are loaded once per workgroup (one thread per
// token), the keys rotated (RoPE, the k_rope formula), both scaled by the power of two that brings the head's
// largest magnitude below 2^14 and split into fp16 hi/lo in LDS: K as [k half][key][8], V^T as
// [16-key step][k half][coordinate][8] (every 16-lane read contiguous; coordinates XOR-swizzled by block so the
// scattered writes spread over the banks). Wavefront w then takes query tokens
// 32 w .. 32 w + 31 (lane = query, its two halves of the head's 16 coordinates on lanes l and l + 32, rotated
// with one cross-lane exchange and multiplied by 1 / sqrt(16)): S^T = K Q^T for four 32-key tiles (K in sigma32
// order), a plain softmax over the row's tokens (weights at most 2^12), and O^T = V^T P^T with the weights straight
// from the accumulators as the B operand; V^T fills 16 of the 32 A-operand rows (the rest are zeros).
// One dimension of n x heads workgroups: consecutive workgroups go to the eight XCDs in turn, and workgroup i takes
// (row, head) number (i % 8) G / 8 + i / 8, heads fastest: an XCD runs a row's heads together, so its L2 reads the
// row's keys and values once. Query token t of row r at q + r * q_row + t * q_tok (the projection's [T][3 e]
// layout, or the class tokens' own [cls][e]).
__global__ __launch_bounds__(256) void k_row_attn_x3(int n, int T, int nq_tok, int e, int heads,
                                                      const float *__restrict__ qkv,
                                                      const float *__restrict__ q, size_t q_row, int q_tok,
                                                      const float *__restrict__ cosv, const float *__restrict__ sinv,
                                                      float *__restrict__ out) {
    __shared__ __align__(16) _Float16 Kh[2][128][8], Kl[2][128][8];
    __shared__ __align__(16) _Float16 Vh[8][2][16][8], Vl[8][2][16][8];
    __shared__ float red[2][4];
    const int G = gridDim.x;
    const int item = G % 8 == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int r = item / heads, h = item - r * heads;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *base = qkv + (size_t)r * T * 3 * e;
    // keys and values, one token a thread
    float kv[16], vv[16];
    const bool tok_live = tid < T;
    if (tok_live) {
        const float *kp = base + (size_t)tid * 3 * e + e + h * 16;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 a = *reinterpret_cast<const float4 *>(kp + 4 * i);
            const float4 b = *reinterpret_cast<const float4 *>(kp + e + 4 * i);
            kv[4 * i] = a.x; kv[4 * i + 1] = a.y; kv[4 * i + 2] = a.z; kv[4 * i + 3] = a.w;
            vv[4 * i] = b.x; vv[4 * i + 1] = b.y; vv[4 * i + 2] = b.z; vv[4 * i + 3] = b.w;
        }
        float cs[8], sn[8];
        load8(cosv + tid * 8, cs);
        load8(sinv + tid * 8, sn);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float a = kv[k], b = kv[k + 8];
            kv[k] = a * cs[k] - b * sn[k];
            kv[k + 8] = b * cs[k] + a * sn[k];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) kv[i] = vv[i] = 0.0f;
    }
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        mk = fmaxf(mk, fabsf(kv[i]));
        mv = fmaxf(mv, fabsf(vv[i]));
    }
    mk = wave_max(mk);
    mv = wave_max(mv);
    if (lane == 0) {
        red[0][wave] = mk;
        red[1][wave] = mv;
    }
    __syncthreads();
    const int sk = shift_for_max(fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3])));
    const int sv = shift_for_max(fmaxf(fmaxf(red[1][0], red[1][1]), fmaxf(red[1][2], red[1][3])));
    if (tid < 128) {
        halfx8 h0, l0, h1, l1;
        split8(kv, ldexpf(1.0f, sk), h0, l0);
        split8(kv + 8, ldexpf(1.0f, sk), h1, l1);
        *reinterpret_cast<halfx8 *>(&Kh[0][tid][0]) = h0;
        *reinterpret_cast<halfx8 *>(&Kl[0][tid][0]) = l0;
        *reinterpret_cast<halfx8 *>(&Kh[1][tid][0]) = h1;
        *reinterpret_cast<halfx8 *>(&Kl[1][tid][0]) = l1;
        const int st = tid >> 4, kg = (tid >> 3) & 1, t8 = tid & 7;
        const int sw = (2 * st + kg) & 15;  // coordinate c of block (st, kg) sits at row c ^ sw: one write's 8
                                            // blocks then hit different banks
        const float fv = ldexpf(1.0f, sv);
#pragma unroll
        for (int c = 0; c < 16; c++) {
            const float x = vv[c] * fv;
            const _Float16 hi = (_Float16)x;
            Vh[st][kg][c ^ sw][t8] = hi;
            Vl[st][kg][c ^ sw][t8] = (_Float16)(x - (float)hi);
        }
    }
    __syncthreads();
    const int r32 = lane & 31, g = lane >> 5;
    const int qt = wave * 32 + r32;  // query token
    if (wave * 32 >= nq_tok) return;
    const bool live = qt < nq_tok;
    // this lane's half of the query's coordinates (8 g .. 8 g + 7), rotated with the other half from lane l ^ 32
    float qv[8];
    {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
        if (live) {
            const float *qp = q + (size_t)r * q_row + (size_t)qt * q_tok + h * 16 + 8 * g;
            a = *reinterpret_cast<const float4 *>(qp);
            b = *reinterpret_cast<const float4 *>(qp + 4);
        }
        qv[0] = a.x; qv[1] = a.y; qv[2] = a.z; qv[3] = a.w; qv[4] = b.x; qv[5] = b.y; qv[6] = b.z; qv[7] = b.w;
        const float sgn = g == 0 ? -1.0f : 1.0f;
        float cs[8] = {1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f, 1.0f}, sn[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
        if (live) {
            load8(cosv + qt * 8, cs);
            load8(sinv + qt * 8, sn);
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float other = __shfl_xor(qv[k], 32, 64);
            qv[k] = (qv[k] * cs[k] + sgn * other * sn[k]) * 0.25f;  // (a c - b s) or (b c + a s), times 1 / sqrt(16)
        }
    }
    float qmax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) qmax = fmaxf(qmax, fabsf(qv[k]));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
    const int sq = shift_for_max(qmax);
    halfx8 qh, ql;
    split8(qv, ldexpf(1.0f, sq), qh, ql);
    const float to_log2 = ldexpf(LOG2E, -(sk + sq));  // raw score -> score * log2 e (positive)
    // S^T: key tiles of 32, rows in sigma32 order; accumulator v of tile kt holds key 32 kt + 16 (v / 8) + 8 g + v % 8
    const int krow = sigma32(r32);
    floatx16 sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
#pragma unroll
        for (int v = 0; v < 16; v++) sc[kt][v] = 0.0f;
        const int key = 32 * kt + krow;  // keys past T are zero rows, masked below
        const halfx8 ah = *reinterpret_cast<const halfx8 *>(&Kh[g][key][0]);
        const halfx8 al = *reinterpret_cast<const halfx8 *>(&Kl[g][key][0]);
        sc[kt] = mfma16x3(ah, al, qh, ql, sc[kt]);
        if (32 * kt + 32 > T) {
#pragma unroll
            for (int v = 0; v < 16; v++)
                if (32 * kt + 16 * (v >> 3) + 8 * g + (v & 7) >= T) sc[kt][v] = -INFINITY;
        }
#pragma unroll
        for (int v = 0; v < 16; v++) mx = fmaxf(mx, sc[kt][v]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float off = 12.0f - mx * to_log2;
    float l = 0.0f;
    halfx8 ph[8], pl[8];  // 16-key step s = 2 kt + hh
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float p[8];
#pragma unroll
            for (int t = 0; t < 8; t++) {
                p[t] = exp2_hw(fmaf(sc[kt][8 * hh + t], to_log2, off));
                l += p[t];
            }
            split8(p, 1.0f, ph[2 * kt + hh], pl[2 * kt + hh]);
        }
    l += __shfl_xor(l, 32, 64);
    // O^T = V^T P^T: A rows 0..15 the coordinates, 16..31 zero
    floatx16 o;
#pragma unroll
    for (int v = 0; v < 16; v++) o[v] = 0.0f;
    halfx8 zero8;
#pragma unroll
    for (int t = 0; t < 8; t++) zero8[t] = (_Float16)0.0f;
#pragma unroll
    for (int st = 0; st < 8; st++) {
        if (16 * st >= T) break;
        halfx8 ah = zero8, al = zero8;
        if (r32 < 16) {
            const int row = r32 ^ ((2 * st + g) & 15);
            ah = *reinterpret_cast<const halfx8 *>(&Vh[st][g][row][0]);
            al = *reinterpret_cast<const halfx8 *>(&Vl[st][g][row][0]);
        }
        o = mfma16x3(ah, al, ph[st], pl[st], o);
    }
    if (!live) return;
    // accumulator v < 8 holds coordinate 8 (v / 4) + 4 g + v % 4 of this lane's query
    const float f = ldexpf(1.0f, -sv) / l;
    float *dst = out + ((size_t)r * nq_tok + qt) * e + h * 16;
    *reinterpret_cast<float4 *>(dst + 4 * g) = make_float4(o[0] * f, o[1] * f, o[2] * f, o[3] * f);
    *reinterpret_cast<float4 *>(dst + 8 + 4 * g) = make_float4(o[4] * f, o[5] * f, o[6] * f, o[7] * f);
}

// Any head width and token count: one thread per (row, query token, head).
__global__ __launch_bounds__(256) void k_row_attn_plain(int n, int T, int nq_tok, int e, int heads,
                                                         const float *__restrict__ qkv, float *__restrict__ out) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)n * nq_tok * heads) return;
    const int h = (int)(i % heads);
    const int t = (int)((i / heads) % nq_tok);
    const size_t r = i / ((size_t)heads * nq_tok);
    const int hd = e / heads;
    const float *base = qkv + r * T * 3 * e;
    const float *qr = base + (size_t)t * 3 * e + h * hd;
    float mx = -INFINITY;
    for (int k = 0; k < T; k++) {
        float s = 0.0f;
        for (int c = 0; c < hd; c++) s += qr[c] * base[(size_t)k * 3 * e + e + h * hd + c];
        mx = fmaxf(mx, s);
    }
    float l = 0.0f;
    float *o = out + (r * nq_tok + t) * e + h * hd;
    for (int c = 0; c < hd; c++) o[c] = 0.0f;
    for (int k = 0; k < T; k++) {
        float s = 0.0f;
        for (int c = 0; c < hd; c++) s += qr[c] * base[(size_t)k * 3 * e + e + h * hd + c];
        const float p = fast_exp(s - mx);
        l += p;
        for (int c = 0; c < hd; c++) o[c] += p * base[(size_t)k * 3 * e + 2 * e + h * hd + c];
    }
    for (int c = 0; c < hd; c++) o[c] /= l;
}

// ---- small copies ------------------------------------------------------------------------------------------
// tok [n][T][e]: class tokens, then the row's cells (cells [n][features][e]). A workgroup per row (grid.x rows in
// slabs of grid.y), 16 bytes a thread: a row of tok is the class tokens then the row's cells, both contiguous.
__global__ __launch_bounds__(256) void k_tokens(int n, int cls, int features, int e, const float *__restrict__ cls_tokens,
                                                 const float *__restrict__ cells, float *__restrict__ tok) {
    const int r = blockIdx.x;
    if (r >= n) return;
    const int head4 = cls * e / 4, body4 = features * e / 4;
    float4 *dst = reinterpret_cast<float4 *>(tok + (size_t)r * (cls + features) * e);
    const float4 *ct = reinterpret_cast<const float4 *>(cls_tokens);
    const float4 *src = reinterpret_cast<const float4 *>(cells + (size_t)r * features * e);
    for (int i = threadIdx.x; i < head4; i += 256) dst[i] = ct[i];
    for (int i = threadIdx.x; i < body4; i += 256) dst[head4 + i] = src[i];
}

// The class tokens of tok [n][T][e] (cls_tokens [cls][e] at tokens 0 .. cls - 1 of every row) and, with kv, their
// keys and values in kv [n][T][2 e] (cls_kv [cls][2 e]): a workgroup per row, 16 bytes a thread.
__global__ __launch_bounds__(256) void k_class_tokens(int n, int T, int cls, int e, const float *__restrict__ cls_tokens,
                                                       float *__restrict__ tok, const float *__restrict__ cls_kv,
                                                       float *__restrict__ kv) {
    const int r = blockIdx.x;
    if (r >= n) return;
    float4 *t4 = reinterpret_cast<float4 *>(tok + (size_t)r * T * e);
    const float4 *c4 = reinterpret_cast<const float4 *>(cls_tokens);
    for (int i = threadIdx.x; i < cls * e / 4; i += 256) t4[i] = c4[i];
    if (kv) {
        float4 *k4 = reinterpret_cast<float4 *>(kv + (size_t)r * T * 2 * e);
        const float4 *ck4 = reinterpret_cast<const float4 *>(cls_kv);
        for (int i = threadIdx.x; i < cls * e / 2; i += 256) k4[i] = ck4[i];
    }
}

// dst [n][k][e] = the first k tokens of each row of src [n][T][e]: a workgroup per row, 16 bytes a thread.
__global__ __launch_bounds__(256) void k_first_tokens(int n, int T, int k, int e, const float *__restrict__ src,
                                                       float *__restrict__ dst) {
    const int r = blockIdx.x;
    if (r >= n) return;
    const int c4 = k * e / 4;
    const float4 *s4 = reinterpret_cast<const float4 *>(src + (size_t)r * T * e);
    float4 *d4 = reinterpret_cast<float4 *>(dst + (size_t)r * k * e);
    for (int i = threadIdx.x; i < c4; i += 256) d4[i] = s4[i];
}

__global__ __launch_bounds__(256) void k_accumulate(size_t count, const float *__restrict__ x, float *__restrict__ sum) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) sum[i] += x[i];
}

// x = sum / digits (the prediction-side average over label digits, src/predict.rs:343-345)
__global__ __launch_bounds__(256) void k_divide(size_t count, const float *__restrict__ sum, float digits,
                                                 float *__restrict__ x) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) x[i] = sum[i] / digits;
}

static dim3 blocks_for(size_t count) { return dim3((unsigned)((count + 255) / 256)); }

// ---- host side ---------------------------------------------------------------------------------------------
void input_cells(hipStream_t s, const tah_weights *w, const float *x, int n, int features, float *cells, int cls,
                 float *kv, const float *cls_kv) {
    if (w->group > 8 || w->group < 1) throw ArgError{"column stage: feature group size must be 1..8"};
    if (w->e % 4) throw ArgError{"column stage: embedding width must be a multiple of 4"};
    if ((size_t)n * features > (size_t)INT32_MAX) throw ArgError{"column stage: too many cells"};
    if (cls < 0 || (cls > 0 && cls != w->cls) || (kv && (!cls || !cls_kv)))
        throw ArgError{"column stage: class tokens are the weights' own, and their keys and values need them"};
    const int T = cls + features;
    if (n >= INPUT_ROWS_MIN && features <= 1024) {
        hipLaunchKernelGGL(k_input_cells, dim3(n), dim3(256), 0, s, n, features, w->group, w->e, x, w->in_w, w->in_b,
                           cells, cls, w->cls_tokens, kv, cls_kv);
        TAH_LAUNCHED();
        return;
    }
    if (cls > 0) {
        hipLaunchKernelGGL(k_class_tokens, dim3(n), dim3(256), 0, s, n, T, cls, w->e, w->cls_tokens, cells, cls_kv, kv);
        TAH_LAUNCHED();
    }
    hipLaunchKernelGGL(k_input_cells_few, dim3((unsigned)(((size_t)n * features + 7) / 8)), dim3(256), 0, s, n,
                       features, w->group, w->e, x, w->in_w, w->in_b, cells + (size_t)cls * w->e, (size_t)T * w->e);
    TAH_LAUNCHED();
}

// At most this many rows (the cells or tokens of up to 16 table rows, or 512 rows' class tokens), the width-128
// projections and feed-forward run on the f32 kernels (16 x 16 tiles, SKINNY_ROWS), whose grids spread the weights
// over many compute units, rather than on the tile kernels, which stream every weight through each tile's workgroup
// (two rows 0.763 -> 0.661 ms, three 0.817 -> 0.707, eight 0.826 -> 0.753, 64 rows 0.918 -> 0.902).
constexpr int SMALL_ROWS = 2048;
// The row block's fused kernel (k_row_block, a workgroup per table row) from this many table rows up; below, the
// projections, the attention (a workgroup per row and head) and the output projection separately (measured: one
// row 0.84 -> 0.76 ms a prediction, 64 rows 1.43 -> 1.40 ms).
constexpr int ROW_BLOCK_MIN = 128;
constexpr int CLS_QUERIES_MIN = 512;

// x [M][e] += l2(gelu(l1(norm2 x))): the fused kernel where the block's shape has one (above SMALL_ROWS rows), else
// two GEMMs with the norm folded into the first where it fits, else layer_norm and two GEMMs (t [M][e] and mid [M][ff]
// scratch).
static void feed_forward(hipStream_t s, int M, float *x, const DevBlock &b, float *t, float *mid) {
    if (b.l1img && M > SMALL_ROWS) {
        ff_block(s, M, x, b);
        return;
    }
    const int e = b.d;
    if (gemm_ln_fits(M, e, x, e, b.l1w)) {
        gemm(s, M, b.ff, e, x, e, b.l1w, b.l1b, mid, b.ff, EPI_GELU, nullptr, 0, b.n2w, b.n2b);
        gemm(s, M, e, b.ff, mid, b.ff, b.l2w, b.l2b, x, e, EPI_RESID, x, e);
        return;
    }
    layer_norm(s, M, e, x, e, b.n2w, b.n2b, t, e);
    gemm(s, M, b.ff, e, t, e, b.l1w, b.l1b, mid, b.ff, EPI_GELU, nullptr, 0);
    gemm(s, M, e, b.ff, mid, b.ff, b.l2w, b.l2b, x, e, EPI_RESID, x, e);
}

// x [M][e] += out(att): the block's output projection and residual add
static void out_projection(hipStream_t s, int M, const float *att, const DevBlock &b, float *x) {
    const int e = b.d;
    if (b.outimg && M > SMALL_ROWS)
        rows128(s, M, e, att, e, b.outimg, b.outs, b.out_b, x, e, EPI_RESID, x, e, nullptr, nullptr, nullptr);
    else
        dense(s, M, e, e, att, e, b.out_w, b.out_s, b.out_b, x, e, EPI_RESID, x, e);
}

// The column blocks run as the fused kernel (k_cell_block, a workgroup per 128 rows of a feature) from this many
// rows: below, its workgroups run mostly empty and each streams the block's weights for a few cells (one row 0.645
// -> 0.706 ms a prediction; from 32 rows it pays: 64 rows 0.903 -> 0.895 ms, 256 rows 1.287 -> 1.268).
constexpr int CELL_BLOCK_MIN = 32;

// One column block (cached_block with a2) for all cells in place: n rows x groups, cell (r, g) at row r * sr + g * sg
// of cells; K/V of group g at kvbase + g * gstride.
void column_block(hipStream_t s, const tah_weights *w, const DevBlock &b, float *cells, int n, int groups, size_t sr,
                  size_t sg, const float *kvbase, size_t gstride, float *t, float *q, float *att, size_t att_bytes,
                  float *mid, const uint8_t *ready) {
    const int e = w->e;
    const int M = n * groups;
    if (cell_block_fits(b) && w->inds == 128 && n >= CELL_BLOCK_MIN && cell_block_work_bytes(groups) <= att_bytes) {
        // the attention half in one kernel, and the feed-forward half in it too where the fused kernel takes the
        // shape; the query and attention buffers are not needed, att holds the images
        const bool ff = block_ff_fits(b) && M > SMALL_ROWS;
        cell_block(s, n, groups, sr, sg, cells, b, w->col_scale, kvbase, gstride,
                   ready ? const_cast<uint8_t *>(ready) : static_cast<void *>(att), ff, nullptr, nullptr, ready);
        if (!ff) feed_forward(s, M, cells, b, t, mid);
        return;
    }
    if (b.inimg && b.ss_hidden == 0 && M > SMALL_ROWS) {
        // norm1, the query projection and its scale in one pass
        rows128(s, M, e, cells, e, b.inimg, b.ins, b.in_b, q, e, EPI_SCALE, nullptr, 0, w->col_scale, b.n1w, b.n1b);
    } else if (b.ss_hidden == 0 && gemm_ln_fits(M, e, cells, e, b.in_w)) {
        gemm(s, M, e, e, cells, e, b.in_w, b.in_b, q, e, EPI_SCALE, nullptr, 0, b.n1w, b.n1b, w->col_scale);
    } else {
        layer_norm(s, M, e, cells, e, b.n1w, b.n1b, t, e);
        gemm(s, M, e, e, t, e, b.in_w, b.in_b, q, e, EPI_NONE, nullptr, 0);
        if ((size_t)b.heads * b.ss_hidden > (size_t)b.ff)
            throw ArgError{"column stage: query MLP wider than the feed-forward"};
        query_modulate(s, M, b, w->col_scale, q, mid);
    }
    const int hd = e / b.heads;
    const dim3 grid((n + 63) / 64, b.heads, groups);
    if (hd == 16 && w->inds == 128 && n <= CELL_FEW_ROWS && (e % 4) == 0)
        hipLaunchKernelGGL(k_cell_attn_few, dim3((groups * b.heads + 3) / 4), dim3(256), 0, s, n, groups, b.heads, sr, sg,
                           e, q, kvbase, gstride, att);
    else if (hd == 16 && w->inds == 128)
        hipLaunchKernelGGL(k_cell_attn_x3, dim3((n + 127) / 128, b.heads, groups), dim3(256), 0, s, n, sr, sg, e, q,
                           kvbase, gstride, att);
    else if (hd == 16 && w->inds == 256)
        hipLaunchKernelGGL(k_cell_attn16<16>, grid, dim3(256), 0, s, n, sr, sg, e, q, kvbase, gstride, att);
    else
        hipLaunchKernelGGL(k_cell_attn_plain, blocks_for((size_t)M * b.heads), dim3(256), 0, s, n, groups, sr, sg, e,
                           b.heads, w->inds, q, kvbase, gstride, att);
    TAH_LAUNCHED();
    out_projection(s, M, att, b, cells);
    feed_forward(s, M, cells, b, t, mid);
}

static bool column_fused(const tah_weights *w, int n) {
    bool fused = w->inds == 128 && !w->col_a2.empty() && n >= CELL_BLOCK_MIN;
    for (auto &b : w->col_a2) fused = fused && cell_block_fits(b);
    return fused;
}

// The column stage's attention buffer: M e floats, or, where the blocks run as the fused kernel, its images of the
// groups' inducing keys and values (cell_block_work_bytes) where those are larger (below 257 rows at 100 features).
static size_t column_att_floats(const tah_weights *w, int n, int features) {
    const size_t M = (size_t)n * features;
    if (!column_fused(w, n)) return M * w->e;
    return std::max(M * w->e, (cell_block_work_bytes(features) + sizeof(float) - 1) / sizeof(float));
}

size_t column_stage_floats(const tah_weights *w, int n, int features, int digits) {
    int ff = 0;
    for (auto &b : w->col_a2) ff = std::max(ff, b.ff);
    const size_t M = (size_t)n * features;
    return M * (3 * (size_t)w->e + ff) + column_att_floats(w, n, features) + (digits > 1 ? 2 * M * w->e : 0);
}

// The column stage at prediction for n rows x [n][features] (device): cells [n * features][e] after the stage.
// col_kv [features][digits][blocks][2][e][inds] on the card. scratch holds column_stage_floats floats.
size_t column_images_bytes(const tah_weights *w, int features, int digits) {
    bool fits = w->inds == 128 && !w->col_a2.empty();
    for (auto &b : w->col_a2) fits = fits && cell_block_fits(b);
    return fits ? (size_t)digits * w->col_blocks * cell_block_work_bytes(features) : 0;
}

void column_images(hipStream_t s, const tah_weights *w, const float *col_kv, int features, int digits, uint8_t *out) {
    const int nb = w->col_blocks;
    const size_t per = 2 * (size_t)w->e * w->inds, gstride = (size_t)digits * nb * per;
    const size_t each = cell_block_work_bytes(features);
    for (int dg = 0; dg < digits; dg++)
        for (int bi = 0; bi < nb; bi++)
            cell_images(s, features, col_kv + ((size_t)dg * nb + bi) * per, gstride, out + ((size_t)dg * nb + bi) * each);
}

void column_stage(hipStream_t s, const tah_weights *w, const float *col_kv, int digits, const float *x, int n,
                  int features, float *cells, float *scratch, const uint8_t *col_images) {
    const int e = w->e, nb = w->col_blocks;
    int ff = 0;
    for (auto &b : w->col_a2) ff = std::max(ff, b.ff);
    const size_t M = (size_t)n * features;
    const size_t natt = column_att_floats(w, n, features);
    float *t = scratch, *q = t + M * e, *att = q + M * e, *mid = att + natt;
    float *plain = mid + M * ff, *sum = plain + M * e;
    const size_t per = 2 * (size_t)e * w->inds, gstride = (size_t)digits * nb * per;
    const size_t each = cell_block_work_bytes(features);
    auto ready = [&](int dg, int bi) {
        return col_images ? col_images + ((size_t)dg * nb + bi) * each : nullptr;
    };
    input_cells(s, w, x, n, features, cells);
    if (digits == 1) {
        for (int bi = 0; bi < nb; bi++)
            column_block(s, w, w->col_a2[bi], cells, n, features, features, 1, col_kv + bi * per, gstride, t, q, att,
                         natt * sizeof(float), mid, ready(0, bi));
        return;
    }
    const size_t count = M * e;
    TAH_HIP(hipMemcpyAsync(plain, cells, count * sizeof(float), hipMemcpyDeviceToDevice, s));
    TAH_HIP(hipMemsetAsync(sum, 0, count * sizeof(float), s));
    for (int dg = 0; dg < digits; dg++) {
        if (dg > 0) TAH_HIP(hipMemcpyAsync(cells, plain, count * sizeof(float), hipMemcpyDeviceToDevice, s));
        for (int bi = 0; bi < nb; bi++)
            column_block(s, w, w->col_a2[bi], cells, n, features, features, 1, col_kv + ((size_t)dg * nb + bi) * per, gstride,
                         t, q, att, natt * sizeof(float), mid, ready(dg, bi));
        hipLaunchKernelGGL(k_accumulate, blocks_for(count), dim3(256), 0, s, count, cells, sum);
        TAH_LAUNCHED();
    }
    hipLaunchKernelGGL(k_divide, blocks_for(count), dim3(256), 0, s, count, sum, (float)digits, cells);
    TAH_LAUNCHED();
}

bool column_tokens_fits(const tah_weights *w, int n, int features, int digits) {
    if (digits != 1 || !column_fused(w, n) || (size_t)n * features <= (size_t)SMALL_ROWS) return false;
    for (auto &b : w->col_a2)
        if (!block_ff_fits(b)) return false;
    return true;
}

void column_stage_tokens(hipStream_t s, const tah_weights *w, const float *col_kv, const float *x, int n,
                         int features, float *tok, float *kv, const float *cls_kv, float *scratch,
                         const uint8_t *col_images) {
    if (!column_tokens_fits(w, n, features, 1)) throw ArgError{"column stage: no fused path for this shape"};
    if (kv && !row_kv_fits(w->row.at(0))) throw ArgError{"column stage: the first row block takes no fused keys"};
    const int e = w->e, nb = w->col_blocks, cls = w->cls, T = cls + features;
    const size_t M = (size_t)n * features;
    if (!col_images && !scratch) throw ArgError{"column stage: no images and no scratch for them"};
    // column_stage's layout: its attention buffer holds the kernel's images (none needed over the model's own)
    float *att = col_images ? nullptr : scratch + 2 * M * e;
    const size_t per = 2 * (size_t)e * w->inds, gstride = (size_t)nb * per;
    // the input layer inside the first column block (the cells formed from the table rows there, not written and
    // read back), unless that block is also the last, which forms the row block's keys and values
    const bool fused_input = (nb > 1 || !kv) && w->group == in_cells_group();
    const InCells in{x, w->in_w, w->in_b, features, w->group};
    if (fused_input) {
        if (cls < 0 || (kv && (!cls || !cls_kv)))
            throw ArgError{"column stage: class tokens are the weights' own, and their keys and values need them"};
        if (cls > 0) {
            hipLaunchKernelGGL(k_class_tokens, dim3(n), dim3(256), 0, s, n, T, cls, e, w->cls_tokens, tok, cls_kv,
                               kv);
            TAH_LAUNCHED();
        }
    } else {
        input_cells(s, w, x, n, features, tok, cls, kv, cls_kv);
    }
    float *cells = tok + (size_t)cls * e;
    for (int bi = 0; bi < nb; bi++) {
        const bool last = bi == nb - 1 && kv;
        const uint8_t *ready = col_images ? col_images + (size_t)bi * cell_block_work_bytes(features) : nullptr;
        cell_block(s, n, features, T, 1, cells, w->col_a2[bi], w->col_scale, col_kv + bi * per, gstride,
                   ready ? const_cast<uint8_t *>(ready) : static_cast<void *>(att), true, last ? &w->row[0] : nullptr,
                   last ? kv + (size_t)cls * 2 * e : nullptr, ready != nullptr, bi == 0 && fused_input ? &in : nullptr);
    }
}

void class_token_kv(hipStream_t s, const tah_weights *w, float *out, float *tmp) {
    const DevBlock &b = w->row.at(0);
    const int e = w->e, cls = w->cls;
    const float *W = b.in_w + (size_t)e * e;  // the projection's key then value rows ([3 e][e])
    if (gemm_ln_fits(cls, e, w->cls_tokens, e, W)) {
        gemm(s, cls, 2 * e, e, w->cls_tokens, e, W, b.in_b + e, out, 2 * e, EPI_NONE, nullptr, 0, b.n1w, b.n1b);
    } else {
        layer_norm(s, cls, e, w->cls_tokens, e, b.n1w, b.n1b, tmp, e);
        gemm(s, cls, 2 * e, e, tmp, e, W, b.in_b + e, out, 2 * e, EPI_NONE, nullptr, 0);
    }
}


// The row stage's fused kernels: head width 16 with the rotary tables' 8 frequencies, at most 128 tokens (the
// rotary positions applied inside the attention kernels).
static bool row_fused(const tah_weights *w, int T) {
    return w->row_heads > 0 && w->e / w->row_heads == 16 && w->e % w->row_heads == 0 && w->rope_half == 8 && T <= 128;
}

// Whether row block bi runs as k_row_block (one kernel, a workgroup per row) for n rows of T tokens.
static bool row_block_path(const tah_weights *w, int bi, int n, int T) {
    return bi < w->row_blocks - 1 && row_fused(w, T) && row_block_fits(w->row[bi], T) && n >= ROW_BLOCK_MIN;
}

bool row_stage_takes_kv(const tah_weights *w, int n, int T) {
    return w->row_blocks >= 2 && row_block_path(w, 0, n, T) && row_kv_fits(w->row[0]);
}

// Whether row_stage runs n rows of T tokens on the fused kernels alone: every block before the last as k_row_block
// with its feed-forward half inside, the last through the class-token path and k_cls_attn. Its scratch is then
// compact: the keys and values [n T][2 e] and the class tokens' buffers ([n cls] rows), not the per-token buffers of
// the unfused kernels.
static bool row_stage_compact(const tah_weights *w, int n, int T) {
    const int last = w->row_blocks - 1;
    if (last < 1 || !row_fused(w, T)) return false;
    const size_t R = (size_t)n * T;
    for (int bi = 0; bi < last; bi++)
        if (!row_block_path(w, bi, n, T) || !block_ff_fits(w->row[bi]) || R <= SMALL_ROWS) return false;
    return w->row[last].inimg && n >= CLS_QUERIES_MIN && w->cls <= CLS_MAXQ && w->row_heads <= 8;
}

// The row stage's scratch, in floats; row_stage lays it out as:
//   compact:  t [M][e], qkv [R][2 e], att [M][e], mid [M][ff], xc [M][e], ac [M][e]      (M = n cls, R = n T)
//   else:     t [R][e], qkv [R][3 e], att [R][e], mid [R][ff], xc [M][e], ac [M][e]
size_t row_stage_floats(const tah_weights *w, int n, int T) {
    int ff = 0;
    for (auto &b : w->row) ff = std::max(ff, b.ff);
    const size_t R = (size_t)n * T, M = (size_t)n * w->cls, e = w->e;
    if (row_stage_compact(w, n, T)) return R * 2 * e + M * (4 * e + ff);
    return R * (5 * e + ff) + M * 2 * e;
}

float *row_stage_kv(const tah_weights *w, int n, int T, float *scratch) {
    return scratch + (row_stage_compact(w, n, T) ? (size_t)n * w->cls : (size_t)n * T) * w->e;
}

// The row stage for n rows: tok [n][T][e] (consumed) to rep [n][cls * e]. cosv/sinv [T][half] on the card.
void row_stage(hipStream_t s, const tah_weights *w, float *tok, int n, int T, const float *cosv, const float *sinv,
               float *rep, float *scratch, bool kv_ready) {
    if (kv_ready && !row_stage_takes_kv(w, n, T))
        throw ArgError{"row stage: the first block's keys and values were formed for a path it does not take"};
    const int e = w->e, heads = w->row_heads, cls = w->cls;
    int ff = 0;
    for (auto &b : w->row) ff = std::max(ff, b.ff);
    const size_t R = (size_t)n * T, M = (size_t)n * cls;
    const bool compact = row_stage_compact(w, n, T);  // the layouts of row_stage_floats
    const size_t rt = compact ? M : R;                // rows of t, att and mid
    float *t = scratch, *qkv = t + rt * e, *att = qkv + R * (compact ? 2 : 3) * e, *mid = att + rt * e;
    float *xc = mid + rt * ff, *ac = xc + M * e;
    const int hd = e / heads, half = w->rope_half;
    if (2 * half != hd) throw ArgError{"row stage: rotary frequencies must cover half the head width"};
    const float inv = 1.0f / sqrtf((float)hd);
    const int last = w->row_blocks - 1;
    const bool mfma = hd == 16 && T <= 256;
    const bool fused = row_fused(w, T);  // rotary positions applied inside k_row_attn_x3
    // the queries k_row_attn_x3 reads: the projection's [T][3 e] rows, or (the last block) the class tokens' [cls][e]
    const float *q_of = qkv;
    size_t q_row = (size_t)T * 3 * e;
    int q_tok = 3 * e;
    auto attend = [&](int nq_tok, float *dst) {
        if (fused)
            hipLaunchKernelGGL(k_row_attn_x3, dim3(n * heads), dim3(256), 0, s, n, T, nq_tok, e, heads, qkv, q_of,
                               q_row, q_tok, cosv, sinv, dst);
        else if (mfma && T <= 128)
            hipLaunchKernelGGL(k_row_attn16<8>, dim3(n, heads), dim3(256), 0, s, n, T, nq_tok, e, qkv, dst);
        else if (mfma)
            hipLaunchKernelGGL(k_row_attn16<16>, dim3(n, heads), dim3(256), 0, s, n, T, nq_tok, e, qkv, dst);
        else
            hipLaunchKernelGGL(k_row_attn_plain, blocks_for((size_t)n * nq_tok * heads), dim3(256), 0, s, n, T, nq_tok, e,
                               heads, qkv, dst);
        TAH_LAUNCHED();
    };
    // the last block's path: only the class tokens queried (from CLS_QUERIES_MIN rows), by k_cls_attn where it
    // takes the shape
    const bool cls_path = fused && w->row[last].inimg && n >= CLS_QUERIES_MIN;
    const bool cls_kernel = cls_path && cls <= CLS_MAXQ && heads <= 8;
    // kv_ready: this block's keys and values are in qkv [R][2 e] already (formed by the block before it)
    for (int bi = 0; bi <= last; bi++) {
        const DevBlock &b = w->row[bi];
        if (row_block_path(w, bi, n, T)) {
            // keys and values by the projection (its second and third 128-row blocks, qkv [R][2 e]) unless the
            // previous block formed them, then the attention half of the block in one kernel (and the feed-forward
            // half in it too where the fused kernel takes the shape, and then the next block's keys and values as
            // well where that block reads them as qkv [R][2 e]: a row block's or the class-token kernel)
            if (!kv_ready)
                rows128(s, (int)R, 2 * e, tok, e, b.inimg + (size_t)128 * e * 4, b.ins, b.in_b + e, qkv, 2 * e,
                        EPI_NONE, nullptr, 0, nullptr, b.n1w, b.n1b);
            const bool ff = block_ff_fits(b) && R > SMALL_ROWS;
            const DevBlock &nb = w->row[bi + 1];
            const bool chain = ff && row_kv_fits(nb) && (bi + 1 < last ? row_block_path(w, bi + 1, n, T) : cls_kernel);
            // before the class-token path only the class tokens' new values are read again (by k_first_tokens): the
            // others' are not stored (105 MB less written at 2,048 rows of 104 tokens)
            row_block(s, n, T, tok, qkv, cosv, sinv, b, ff, chain ? &nb : nullptr, qkv, chain && bi + 1 == last ? cls : T);
            kv_ready = chain;
            if (!ff) feed_forward(s, (int)R, tok, b, t, mid);
            continue;
        }
        if (bi == last && cls_path) {
            // the last block queries only the class tokens: keys and values for every token (the projection's second
            // and third 128-row blocks: qkv [R][2 e] for k_cls_attn, unless the previous block formed them, else into
            // qkv's [T][3 e] rows), queries for the class tokens alone, from their gathered copy (which the block
            // then updates); below CLS_QUERIES_MIN rows the extra launch costs more than the other tokens' queries
            // (2,048 rows 4.30 -> 4.25 ms, 64 and 256 rows 5 us slower)
            if (!kv_ready)
                rows128(s, (int)R, 2 * e, tok, e, b.inimg + (size_t)128 * e * 4, b.ins, b.in_b + e,
                        cls_kernel ? qkv : qkv + e, cls_kernel ? 2 * e : 3 * e, EPI_NONE, nullptr, 0, nullptr, b.n1w,
                        b.n1b);
            const int M = n * cls;
            hipLaunchKernelGGL(k_first_tokens, dim3(n), dim3(256), 0, s, n, T, cls, e, tok, xc);
            TAH_LAUNCHED();
            rows128(s, M, e, xc, e, b.inimg, b.ins, b.in_b, ac, e, EPI_NONE, nullptr, 0, nullptr, b.n1w, b.n1b);
            if (cls_kernel) {
                hipLaunchKernelGGL(k_cls_attn, dim3(n), dim3(64 * heads), 0, s, n, T, cls, e, qkv, (size_t)T * 2 * e,
                                   2 * e, ac, (size_t)cls * e, e, cosv, sinv, att);
                TAH_LAUNCHED();
            } else {
                q_of = ac;
                q_row = (size_t)cls * e;
                q_tok = e;
                attend(cls, att);
            }
            out_projection(s, M, att, b, xc);
            feed_forward(s, M, xc, b, t, mid);
            layer_norm(s, M, e, xc, e, w->out_lnw, w->out_lnb, rep, e);
            continue;
        }
        if (b.inimg && R > SMALL_ROWS) {
            rows128(s, (int)R, 3 * e, tok, e, b.inimg, b.ins, b.in_b, qkv, 3 * e, EPI_NONE, nullptr, 0, nullptr, b.n1w,
                    b.n1b);
        } else if (gemm_ln_fits((int)R, e, tok, e, b.in_w)) {
            gemm(s, (int)R, 3 * e, e, tok, e, b.in_w, b.in_b, qkv, 3 * e, EPI_NONE, nullptr, 0, b.n1w, b.n1b);
        } else {
            layer_norm(s, (int)R, e, tok, e, b.n1w, b.n1b, t, e);
            gemm(s, (int)R, 3 * e, e, t, e, b.in_w, b.in_b, qkv, 3 * e, EPI_NONE, nullptr, 0);
        }
        if (!fused) {
            hipLaunchKernelGGL(k_rope, blocks_for(R * heads * half), dim3(256), 0, s, R, T, e, heads, half, cosv, sinv,
                               qkv, inv);
            TAH_LAUNCHED();
        }
        if (bi < last) {
            attend(T, att);
            out_projection(s, (int)R, att, b, tok);
            feed_forward(s, (int)R, tok, b, t, mid);
        } else {
            // the last block: only the class tokens are queried and updated
            const int M = n * cls;
            attend(cls, ac);
            hipLaunchKernelGGL(k_first_tokens, dim3(n), dim3(256), 0, s, n, T, cls, e, tok, xc);
            TAH_LAUNCHED();
            out_projection(s, M, ac, b, xc);
            feed_forward(s, M, xc, b, t, mid);
            layer_norm(s, M, e, xc, e, w->out_lnw, w->out_lnb, rep, e);
        }
    }
}

void assemble_tokens(hipStream_t s, const tah_weights *w, const float *cells, int n, int features, float *tok) {
    if (w->e % 4) throw ArgError{"row stage: embedding width must be a multiple of 4"};
    hipLaunchKernelGGL(k_tokens, dim3(n), dim3(256), 0, s, n, w->cls, features, w->e, w->cls_tokens, cells, tok);
    TAH_LAUNCHED();
}

}  // namespace tah
