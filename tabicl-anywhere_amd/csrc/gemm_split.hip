// Dense layers on the fp16 matrix cores with split f32 operands: Y = epi(X W^T + b) for weights uploaded as split
// images (SplitW), the products formed as in device_math.hpp (three v_mfma_f32_32x32x16_f16 per f32 product).
//
// The product is formed transposed, Y^T = W X^T: each wavefront owns 32 rows of X, one per lane pair (lane l holds
// row l % 32 and, of every 16 columns, the eight 8 (l / 32) + 0..7) -- the B operand -- and 32 TN output columns.
// The weights are the A operand, read straight from their image (32-row tiles with the rows in sigma32 order, then
// 16-column steps: one coalesced 512-byte read per lane half), which puts eight consecutive output columns in each
// lane's accumulators v = 8 hh .. 8 hh + 7, stored as two 128-bit writes. No LDS: the four wavefronts of a
// workgroup take four row groups of one column tile, so the weight tile they all read is shared through the caches.
//
// X is scaled per row and per chunk of 128 columns by a power of two (the chunk's largest magnitude below 2^14)
// before splitting; the accumulators are rescaled (exactly) from one chunk's power to the next and unscaled in the
// epilogue. (Products with K = 128 over many rows, the column and row stages', use k_rows128 in blocks.hip, which
// keeps the weights in LDS and can fold a layer normalisation in front.)
#include "common.hpp"
#include "device_math.hpp"

namespace tah {

struct SplitEpi {
    const float *R;      // EPI_RESID: added; EPI_QMOD: the query being modulated (may alias Y)
    int ldr;
    const float *scale;  // EPI_SCALE: [N]; EPI_QMOD: [heads][N]; the fused query MLP: [N] (head h at 64 h)
    int heads;
    // the fused query MLP (k_gemm_splitk4 with QM): W0 and W2 as gemm_split images, their shifts and biases
    const uint8_t *w0 = nullptr, *w2 = nullptr;
    int s0 = 0, s2 = 0;
    const float *b0 = nullptr, *b2 = nullptr;
};

template <int EPI, int TN>
__global__ __launch_bounds__(256, 3) void k_gemm_split(int M, int N, int K, const float *__restrict__ X, int ldx,
                                                        const uint8_t *__restrict__ wimg, int wshift,
                                                        const float *__restrict__ b, float *Y, int ldy, SplitEpi ea) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int m = (blockIdx.y * 4 + wave) * 32 + r32;
    const bool live = m < M;
    const int tile0 = blockIdx.x * TN;  // first 32-column tile of this wavefront
    const int KS = K / 16;
    const float *xrow = X + (size_t)(live ? m : 0) * ldx;

    floatx16 acc[TN];
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;
    int eprev = 0;
    for (int k0 = 0; k0 < K; k0 += 128) {
        const int nks = min(8, (K - k0) / 16);
        float xv[8][8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
            if (live && ks < nks) {
                const float *src = xrow + k0 + 16 * ks + 8 * g;
                a = *reinterpret_cast<const float4 *>(src);
                c = *reinterpret_cast<const float4 *>(src + 4);
            }
            xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
            xv[ks][4] = c.x; xv[ks][5] = c.y; xv[ks][6] = c.z; xv[ks][7] = c.w;
        }
        float xmax = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
        xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
        const int e = shift_for_max(xmax);
        if (k0 > 0) {
            const float r = ldexpf(1.0f, e - eprev);
#pragma unroll
            for (int j = 0; j < TN; j++) acc[j] *= r;
        }
        eprev = e;
        const float f = ldexpf(1.0f, e);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            if (ks >= nks) break;
            halfx8 xh, xl;
            split8(xv[ks], f, xh, xl);
            const int kk = k0 / 16 + ks;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint8_t *w = wimg + ((size_t)(tile0 + j) * KS + kk) * 2048 + (g * 32 + r32) * 16;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(w);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(w + 1024);
                acc[j] = mfma16x3(ah, al, xh, xl, acc[j]);
            }
        }
    }
    if (!live) return;
    // column of accumulator v of tile j: 32 (tile0 + j) + 16 (v / 8) + 8 g + v % 8
    const float u = ldexpf(1.0f, -(wshift + eprev));
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int n0 = 32 * (tile0 + j) + 16 * hh + 8 * g;
            float yv[8];
#pragma unroll
            for (int t = 0; t < 8; t++) yv[t] = acc[j][8 * hh + t] * u;
            if (b) {
                const float4 ba = *reinterpret_cast<const float4 *>(b + n0);
                const float4 bb = *reinterpret_cast<const float4 *>(b + n0 + 4);
                yv[0] += ba.x; yv[1] += ba.y; yv[2] += ba.z; yv[3] += ba.w;
                yv[4] += bb.x; yv[5] += bb.y; yv[6] += bb.z; yv[7] += bb.w;
            }
            if (EPI == EPI_GELU) {
#pragma unroll
                for (int t = 0; t < 8; t++) yv[t] = gelu(yv[t]);
            }
            if (EPI == EPI_SCALE) {
                const float4 sa = *reinterpret_cast<const float4 *>(ea.scale + n0);
                const float4 sb = *reinterpret_cast<const float4 *>(ea.scale + n0 + 4);
                yv[0] *= sa.x; yv[1] *= sa.y; yv[2] *= sa.z; yv[3] *= sa.w;
                yv[4] *= sb.x; yv[5] *= sb.y; yv[6] *= sb.z; yv[7] *= sb.w;
            }
            if (EPI == EPI_RESID || EPI == EPI_QMOD) {
                const float *rp = ea.R + (size_t)m * ea.ldr + n0;
                const float4 ra = *reinterpret_cast<const float4 *>(rp);
                const float4 rb = *reinterpret_cast<const float4 *>(rp + 4);
                const float rv[8] = {ra.x, ra.y, ra.z, ra.w, rb.x, rb.y, rb.z, rb.w};
                if (EPI == EPI_RESID) {
#pragma unroll
                    for (int t = 0; t < 8; t++) yv[t] += rv[t];
                } else {
                    const float *sp = ea.scale + (size_t)(m % ea.heads) * N + n0;
#pragma unroll
                    for (int t = 0; t < 8; t++) yv[t] = rv[t] * (sp[t] * (1.0f + tanh1(yv[t])));
                }
            }
            float *dst = Y + (size_t)m * ldy + n0;
            *reinterpret_cast<float4 *>(dst) = make_float4(yv[0], yv[1], yv[2], yv[3]);
            *reinterpret_cast<float4 *>(dst + 4) = make_float4(yv[4], yv[5], yv[6], yv[7]);
        }
}

// ---- the query MLP of the scalable softmax, whole, for head width 64 and hidden width 64 ------------------------
// q *= scale[h] * (1 + tanh1(W2 gelu(W0 q + b0) + b2)) (src/nn.rs:130-152) for the 32 query-heads of a wavefront:
// lane l holds query-head l % 32, its 64 coordinates 16 ks + 8 (l / 32) + t in xv[ks][t] (split once here); H^T =
// W0 X^T with W0's rows in sigma32 order leaves the hidden layer in registers as the B operand of Y^T = W2 H^T, and
// the lane's output columns are exactly the input columns it holds, so the modulation needs no second read of q.
// W0 and W2 are read from their gemm_split images; sc = the head's 64 scales; the result goes to dst (the
// query-head's 64 values), nowhere where dst is null.
__device__ __forceinline__ void qmlp64_lane(const float (&xv)[4][8], int r32, int g, const uint8_t *__restrict__ w0,
                                            int s0, const float *__restrict__ b0, const uint8_t *__restrict__ w2,
                                            int s2, const float *__restrict__ b2, const float *__restrict__ sc,
                                            float *dst) {
    float xmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
#pragma unroll
        for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
    xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
    const int sx = shift_for_max(xmax);
    halfx8 xh[4], xl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) split8(xv[ks], ldexpf(1.0f, sx), xh[ks], xl[ks]);
    // hidden = gelu(W0 x + b0): 2 tiles of 32, 4 steps of 16 (image: (tile * 4 + step) * 2 KB)
    floatx16 hacc[2];
#pragma unroll
    for (int T = 0; T < 2; T++) {
#pragma unroll
        for (int v = 0; v < 16; v++) hacc[T][v] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const uint8_t *w = w0 + ((size_t)T * 4 + ks) * 2048 + (g * 32 + r32) * 16;
            hacc[T] = mfma16x3(*reinterpret_cast<const halfx8 *>(w), *reinterpret_cast<const halfx8 *>(w + 1024),
                               xh[ks], xl[ks], hacc[T]);
        }
    }
    const float u0 = ldexpf(1.0f, -(sx + s0));
    float hmax = 0.0f;
#pragma unroll
    for (int T = 0; T < 2; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float *bp = b0 + 32 * T + 16 * hh + 8 * g;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float hv = gelu(hacc[T][8 * hh + t] * u0 + bp[t]);
                hacc[T][8 * hh + t] = hv;
                hmax = fmaxf(hmax, fabsf(hv));
            }
        }
    hmax = fmaxf(hmax, __shfl_xor(hmax, 32, 64));
    const int sh = shift_for_max(hmax);
    halfx8 hh8[4], hl8[4];
#pragma unroll
    for (int T = 0; T < 2; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float hv[8];
#pragma unroll
            for (int t = 0; t < 8; t++) hv[t] = hacc[T][8 * hh + t];
            split8(hv, ldexpf(1.0f, sh), hh8[2 * T + hh], hl8[2 * T + hh]);
        }
    // y = W2 hidden + b2; q *= scale (1 + tanh1(y)); output column 32 T + 16 hh + 8 g + t is input step 2 T + hh
    floatx16 yacc[2];
#pragma unroll
    for (int T = 0; T < 2; T++) {
#pragma unroll
        for (int v = 0; v < 16; v++) yacc[T][v] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const uint8_t *w = w2 + ((size_t)T * 4 + ks) * 2048 + (g * 32 + r32) * 16;
            yacc[T] = mfma16x3(*reinterpret_cast<const halfx8 *>(w), *reinterpret_cast<const halfx8 *>(w + 1024),
                               hh8[ks], hl8[ks], yacc[T]);
        }
    }
    if (!dst) return;
    const float u2 = ldexpf(1.0f, -(sh + s2));
#pragma unroll
    for (int T = 0; T < 2; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int n0 = 32 * T + 16 * hh + 8 * g;
            float out[8];
#pragma unroll
            for (int t = 0; t < 8; t++)
                out[t] = xv[2 * T + hh][t] * (sc[n0 + t] * (1.0f + tanh1(yacc[T][8 * hh + t] * u2 + b2[n0 + t])));
            *reinterpret_cast<float4 *>(dst + n0) = make_float4(out[0], out[1], out[2], out[3]);
            *reinterpret_cast<float4 *>(dst + n0 + 4) = make_float4(out[4], out[5], out[6], out[7]);
        }
}

// The same query MLP for a workgroup's finished 32-row tile of NH heads, shared out: wavefront 2 h + T forms hidden
// tile T (32 units) and then output tile T of head h on the matrix cores, and all NT threads take the element-wise
// work between (GELU, then the modulation and the store), which on one wavefront a head was most of the tail.
// qt: the tile's query values, [32 rows][ldq] with head h at column 64 h; hs, ys: [NH][32][QMP] of LDS each (the
// hidden layer, the MLP's output). Same operations per value as qmlp64_lane: the products sum in the same order and
// each row's powers of two are taken over the same 64 values, so the results are the same bits. The weights, biases
// and the heads' 64 NH scales come read (qmlp64_read); Y: row 0 of the tile at head 0's first column; rows: the
// tile's live rows (the others are not stored). Wavefronts 2 NH.. only join the element-wise phases; the caller has
// made qt visible to the whole workgroup.
constexpr int QMP = 68;  // row pitch of the hidden layer and output tiles in LDS

// The operands of qmlp64_tile a thread reads, issued by qmlp64_read where their latency can overlap other work.
template <int CH>
struct QmlpOps {
    halfx8 a0h[4], a0l[4], a2h[4], a2l[4];  // the wavefront's tile of W0 and of W2, four 16-column steps
    float bz[2][8], by[2][8];               // b0 and b2 at the lane's 16 hidden / output columns
    float4 scv[CH];                         // the scales of the thread's chunks in the modulation
};

template <int NH, int NT>
__device__ __forceinline__ QmlpOps<NH * 512 / NT> qmlp64_read(int tid, const uint8_t *w0, const float *b0,
                                                              const uint8_t *w2, const float *b2, const float *sc) {
    static_assert(NT >= 128 * NH && (NH * 512) % NT == 0, "two wavefronts a head, whole float4 chunks a thread");
    constexpr int CH = NH * 512 / NT;  // float4 chunks of the heads' 32 x 64 values a thread
    const int lane = tid & 63, wave = tid >> 6, r32 = lane & 31, g = lane >> 5, T = wave & 1;
    QmlpOps<CH> o;
    if (wave < 2 * NH) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const size_t off = ((size_t)T * 4 + ks) * 2048 + (g * 32 + r32) * 16;
            o.a0h[ks] = *reinterpret_cast<const halfx8 *>(w0 + off);
            o.a0l[ks] = *reinterpret_cast<const halfx8 *>(w0 + off + 1024);
            o.a2h[ks] = *reinterpret_cast<const halfx8 *>(w2 + off);
            o.a2l[ks] = *reinterpret_cast<const halfx8 *>(w2 + off + 1024);
        }
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            load8(b0 + 32 * T + 16 * hh + 8 * g, o.bz[hh]);
            load8(b2 + 32 * T + 16 * hh + 8 * g, o.by[hh]);
        }
    }
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int c = tid + NT * i;
        o.scv[i] = *reinterpret_cast<const float4 *>(sc + 64 * (c >> 9) + 4 * (c & 15));
    }
    return o;
}

template <int NH, int NT>
__device__ __forceinline__ void qmlp64_tile(const float *qt, int ldq, float *hs, float *ys, int tid,
                                            const QmlpOps<NH * 512 / NT> &o, int s0, int s2, float *Y, int ldy,
                                            int rows) {
    constexpr int CH = NH * 512 / NT;
    const int lane = tid & 63, wave = tid >> 6, r32 = lane & 31, g = lane >> 5;
    const bool mm = wave < 2 * NH;
    const int h = mm ? wave >> 1 : 0, T = wave & 1;
    float *hrow = hs + (h * 32 + r32) * QMP;
    if (mm) {
        float xv[4][8];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) load8(&qt[r32 * ldq + 64 * h + 16 * ks + 8 * g], xv[ks]);
        float xmax = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
        xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
        const int sx = shift_for_max(xmax);
        floatx16 acc;
#pragma unroll
        for (int v = 0; v < 16; v++) acc[v] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            halfx8 xh, xl;
            split8(xv[ks], ldexpf(1.0f, sx), xh, xl);
            acc = mfma16x3(o.a0h[ks], o.a0l[ks], xh, xl, acc);
        }
        const float u0 = ldexpf(1.0f, -(sx + s0));
        // hidden unit 32 T + 16 hh + 8 g + t of the lane's row: its pre-activation
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float z[8];
#pragma unroll
            for (int t = 0; t < 8; t++) z[t] = acc[8 * hh + t] * u0 + o.bz[hh][t];
            *reinterpret_cast<float4 *>(hrow + 32 * T + 16 * hh + 8 * g) = make_float4(z[0], z[1], z[2], z[3]);
            *reinterpret_cast<float4 *>(hrow + 32 * T + 16 * hh + 8 * g + 4) = make_float4(z[4], z[5], z[6], z[7]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int c = tid + NT * i;
        float4 *p = reinterpret_cast<float4 *>(hs + (c >> 4) * QMP + 4 * (c & 15));
        const float4 z = *p;
        *p = make_float4(gelu(z.x), gelu(z.y), gelu(z.z), gelu(z.w));
    }
    __syncthreads();
    if (mm) {
        float hv[4][8];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) load8(hrow + 16 * ks + 8 * g, hv[ks]);
        float hmax = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) hmax = fmaxf(hmax, fabsf(hv[ks][t]));
        hmax = fmaxf(hmax, __shfl_xor(hmax, 32, 64));
        const int sh = shift_for_max(hmax);
        floatx16 acc;
#pragma unroll
        for (int v = 0; v < 16; v++) acc[v] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            halfx8 hh8, hl8;
            split8(hv[ks], ldexpf(1.0f, sh), hh8, hl8);
            acc = mfma16x3(o.a2h[ks], o.a2l[ks], hh8, hl8, acc);
        }
        const float u2 = ldexpf(1.0f, -(sh + s2));
        float *yrow = ys + (h * 32 + r32) * QMP + 32 * T + 8 * g;
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float y[8];
#pragma unroll
            for (int t = 0; t < 8; t++) y[t] = acc[8 * hh + t] * u2 + o.by[hh][t];
            *reinterpret_cast<float4 *>(yrow + 16 * hh) = make_float4(y[0], y[1], y[2], y[3]);
            *reinterpret_cast<float4 *>(yrow + 16 * hh + 4) = make_float4(y[4], y[5], y[6], y[7]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int c = tid + NT * i, hr = c >> 4, hd = hr >> 5, r = hr & 31, c4 = 4 * (c & 15);
        if (r >= rows) continue;
        const float4 y = *reinterpret_cast<const float4 *>(ys + hr * QMP + c4);
        const float4 q = *reinterpret_cast<const float4 *>(qt + r * ldq + 64 * hd + c4);
        const float4 s = o.scv[i];
        *reinterpret_cast<float4 *>(Y + (size_t)r * ldy + 64 * hd + c4) =
            make_float4(q.x * (s.x * (1.0f + tanh1(y.x))), q.y * (s.y * (1.0f + tanh1(y.y))),
                        q.z * (s.z * (1.0f + tanh1(y.z))), q.w * (s.w * (1.0f + tanh1(y.w))));
    }
}

// Few rows and long rows (the in-context stage: 2,048 queries, K = 512 or 1024): one workgroup per 32 rows x 128
// columns, its W wavefronts splitting K W ways (four or eight, each in chunks of CW columns with their own per-row
// powers of two), then summing their partial products -- unscaled to f32 -- through LDS; wavefront w finishes
// tile w (W = 4) or half of tile w / 2 (W = 8). W times the wavefronts of k_gemm_split on the same grid of outputs,
// each with 1 / W of the dependent chain. With QM (the query projection, 64 or 128 columns = one or two heads of 64), the finished tile
// goes through LDS and the workgroup runs the heads' query MLP on it (qmlp64_tile): no separate launch.
constexpr int SPLITK_MAX_KQ = 512;  // each wavefront's share of K at most (K at most 2048)

// 16 bytes a lane from src to dst + 16 lane by DMA (dst wavefront-uniform)
__device__ __forceinline__ void copy16_to_lds(const float *src, uint8_t *dst) {
    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(src), dst, 16, 0, 0);
}


// W = 8 (four tiles a workgroup only, no QM): eight wavefronts split K eight ways, two a SIMD, each with half the
// dependent chain of four; a wavefront's chunk is then CW = 64 columns when K = 512.
template <int EPI, bool LN, int TN, bool QM = false, int W = 4, int CW = 128>
__global__ __launch_bounds__(64 * W, 2) void k_gemm_splitk4(int M, int N, int K, const float *__restrict__ X, int ldx,
                                                             const uint8_t *__restrict__ wimg, int wshift,
                                                             const float *__restrict__ b, float *Y, int ldy, SplitEpi ea,
                                                             const float *__restrict__ lnw, const float *__restrict__ lnb) {
    static_assert(W == 4 || (W == 8 && TN == 4), "eight wavefronts: four tiles a workgroup");
    static_assert(CW == 128 || CW == 64, "chunks of 64 or 128 columns");
    constexpr int C4 = CW / 4;  // float4 columns of a chunk row
    constexpr bool HALVES = TN == 2 || W == 8;  // a wavefront finishes half a tile
    // per wavefront 16 KB: its rows' chunk (32 rows x C4 float4, swizzled) while the products run, then its partial
    // sums [tile][accumulator][lane]
    __shared__ __align__(16) float stage[W][16 * 64 * 4];
    auto red = [&](int w, int T, int v) { return &stage[w][(T * 16 + v) * 64]; };
    __shared__ float rsum[W][32];  // LN: per-wavefront partial row sums
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    // one dimension of (N / 32 TN) x ceil(M / 32) workgroups; consecutive workgroups go to the eight XCDs in turn, so
    // workgroup i takes tile (i % 8) G / 8 + i / 8, column tiles fastest: the tiles an XCD runs share row panels
    // (its L2 reads their rows of X once; 2,048 rows: 9.5 -> 9.2 us out-projection, 14.5 -> 12.7 us second
    // feed-forward layer)
    const int gx = N / (32 * TN), G = gridDim.x;
    const int tile = G % 8 == 0 ? (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3) : blockIdx.x;
    const int bxt = tile % gx;
    const int m = tile / gx * 32 + r32;
    const bool live = m < M;
    const int nt0 = bxt * TN;
    const int KS = K / 16, kq = K / W, kend = (wave + 1) * kq;
    floatx16 acc[TN];
#pragma unroll
    for (int T = 0; T < TN; T++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[T][v] = 0.0f;
    int eprev = 0;
    // weight operands of this wavefront's 16-column steps j, two steps ahead of the products; the first two are
    // issued before the rows are read, so that their latency overlaps the rows' and the layer norm's
    const uint8_t *wl = wimg + ((size_t)nt0 * KS + wave * kq / 16) * 2048 + (g * 32 + r32) * 16;
    const int nsteps = kq / 16;
    auto wload = [&](int j, halfx8 (&w)[TN][2]) {
#pragma unroll
        for (int T = 0; T < TN; T++) {
            const uint8_t *src = wl + ((size_t)T * KS + j) * 2048;
            w[T][0] = *reinterpret_cast<const halfx8 *>(src);
            w[T][1] = *reinterpret_cast<const halfx8 *>(src + 1024);
        }
    };
    halfx8 wb[3][TN][2];
    wload(0, wb[0]);
    if (nsteps > 1) wload(1, wb[1]);
#pragma unroll
    for (int it = 0; it < (LN ? 1 : SPLITK_MAX_KQ / CW); it++) {  // with the layer norm, K = W CW = 512
        const int k0 = wave * kq + CW * it;
        if (k0 >= kend) break;
        float xv[CW / 16][8];
        {
            // a whole chunk (K is a multiple of W CW): the wavefront's 32 rows x CW columns copied into its staging by
            // DMA, copy i lane l filling float4 slot 64 i + l = row (64 i + l) / C4, float4 column ((64 i + l) % C4) ^
            // (row % 16), so that each load instruction reads whole runs of rows (a lane a row, as below, touched 32
            // rows an instruction) and the reads back, a row a lane, fall on distinct bank groups; rows past M read
            // row M - 1
            const int m0 = tile / gx * 32;
            uint8_t *st = reinterpret_cast<uint8_t *>(stage[wave]);
#pragma unroll
            for (int i = 0; i < CW / 8; i++) {
                const int slot = 64 * i + lane, row = slot / C4, c = (slot % C4) ^ (row & 15);
                copy16_to_lds(X + (size_t)min(m0 + row, M - 1) * ldx + k0 + 4 * c, st + 1024 * i);
            }
            __builtin_amdgcn_s_waitcnt(0);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int ks = 0; ks < CW / 16; ks++) {
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const int c = 4 * ks + 2 * g + hf;
                    const float4 a = *reinterpret_cast<const float4 *>(st + 16 * (r32 * C4 + (c ^ (r32 & 15))));
                    xv[ks][4 * hf] = a.x; xv[ks][4 * hf + 1] = a.y; xv[ks][4 * hf + 2] = a.z; xv[ks][4 * hf + 3] = a.w;
                }
            }
        }
        if (LN) {
            // K = 512: this wavefront holds columns CW w .. CW w + CW - 1 of its 32 rows; the row's sums go
            // through LDS (two passes: mean, then biased variance; eps 1e-5)
            auto row_total = [&]() {
                float t = rsum[0][r32];
#pragma unroll
                for (int w = 1; w < W; w++) t += rsum[w][r32];
                return t;
            };
            float sum = 0.0f;
#pragma unroll
            for (int ks = 0; ks < CW / 16; ks++)
#pragma unroll
                for (int t = 0; t < 8; t++) sum += xv[ks][t];
            sum += __shfl_xor(sum, 32, 64);
            if (g == 0) rsum[wave][r32] = sum;
            __syncthreads();
            const float mean = row_total() / (float)K;
            float sq = 0.0f;
#pragma unroll
            for (int ks = 0; ks < CW / 16; ks++)
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const float dv = xv[ks][t] - mean;
                    sq += dv * dv;
                }
            sq += __shfl_xor(sq, 32, 64);
            __syncthreads();
            if (g == 0) rsum[wave][r32] = sq;
            __syncthreads();
            const float inv = 1.0f / sqrtf(row_total() / (float)K + 1e-5f);
#pragma unroll
            for (int ks = 0; ks < CW / 16; ks++) {
                float wv[8], bv[8];
                const int c0 = k0 + 16 * ks + 8 * g;
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    wv[t] = lnw[c0 + t];
                    bv[t] = lnb[c0 + t];
                }
#pragma unroll
                for (int t = 0; t < 8; t++) xv[ks][t] = (xv[ks][t] - mean) * inv * wv[t] + bv[t];
            }
        }
        float xmax = 0.0f;
#pragma unroll
        for (int ks = 0; ks < CW / 16; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
        xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
        const int e = shift_for_max(xmax);
        if (k0 > wave * kq) {
            const float r = ldexpf(1.0f, e - eprev);
#pragma unroll
            for (int T = 0; T < TN; T++) acc[T] *= r;
        }
        eprev = e;
        const float f = ldexpf(1.0f, e);
#pragma unroll
        for (int ks = 0; ks < CW / 16; ks++) {
            const int j = (CW / 16) * it + ks;
            if (j + 2 < nsteps) wload(j + 2, wb[(j + 2) % 3]);
            halfx8 xh, xl;
            split8(xv[ks], f, xh, xl);
#pragma unroll
            for (int T = 0; T < TN; T++) acc[T] = mfma16x3(wb[j % 3][T][0], wb[j % 3][T][1], xh, xl, acc[T]);
        }
    }
    // with QM, the query MLP's operands are read now, their latency behind the partial sums' reduction
    QmlpOps<(TN / 2) * 512 / (64 * W)> qo;
    if constexpr (QM)
        qo = qmlp64_read<TN / 2, 64 * W>(tid, ea.w0, ea.b0, ea.w2, ea.b2, ea.scale + 64 * (TN / 2) * bxt);
    const float u = ldexpf(1.0f, -(wshift + eprev));
#pragma unroll
    for (int T = 0; T < TN; T++)
#pragma unroll
        for (int v = 0; v < 16; v++) red(wave, T, v)[lane] = acc[T][v] * u;
    __syncthreads();
    if constexpr (QM) {
        static_assert(TN == 4 || TN == 2, "the fused query MLP takes whole heads (64 columns) per workgroup");
        constexpr int LD = 32 * TN + 4;  // the tile's row pitch in LDS
        // wavefront w: tile w of four (rows r32, columns 32 w + 16 hh + 8 g + t of the workgroup's), or half w % 2 of
        // tile w / 2 (of two; of four with W = 8); bias added
        const int T = HALVES ? wave >> 1 : wave;
        float yq[2][8];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            if (HALVES && hh != (wave & 1)) continue;
            const int n0 = 32 * (nt0 + T) + 16 * hh + 8 * g;
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int v = 8 * hh + t;
                float y = red(0, T, v)[lane];
#pragma unroll
                for (int w = 1; w < W; w++) y += red(w, T, v)[lane];
                yq[hh][t] = y + b[n0 + t];
            }
        }
        __syncthreads();  // the partial sums are all read: their LDS holds the tile next, [32 rows][LD]
        float *qt = &stage[0][0];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            if (HALVES && hh != (wave & 1)) continue;
#pragma unroll
            for (int t = 0; t < 8; t++) qt[r32 * LD + 32 * T + 16 * hh + 8 * g + t] = yq[hh][t];
        }
        __syncthreads();
        // the hidden layer and the MLP's output after the tile, in the partial sums' LDS
        static_assert(32 * LD + 2 * (TN / 2) * 32 * QMP <= W * 16 * 64 * 4, "the query MLP's tiles fit in LDS");
        float *hs = qt + 32 * LD;
        const int m0 = tile / gx * 32;
        qmlp64_tile<TN / 2, 64 * W>(qt, LD, hs, hs + (TN / 2) * 32 * QMP, tid, qo, ea.s0, ea.s2,
                                    Y + (size_t)m0 * ldy + 64 * (TN / 2) * bxt, ldy, min(32, M - m0));
        return;
    }
    if (!live) return;
    // wavefront w sums tile w (both halves) of four, or half w % 2 of tile w / 2 (of two; of four with W = 8), the
    // partials in wavefront order
    const int T = HALVES ? wave >> 1 : wave;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
        if (HALVES && hh != (wave & 1)) continue;
        const int n0 = 32 * (nt0 + T) + 16 * hh + 8 * g;
        float yv[8];
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const int v = 8 * hh + t;
            float y = red(0, T, v)[lane];
#pragma unroll
            for (int w = 1; w < W; w++) y += red(w, T, v)[lane];
            yv[t] = y;
        }
        if (b) {
            const float4 ba = *reinterpret_cast<const float4 *>(b + n0);
            const float4 bb = *reinterpret_cast<const float4 *>(b + n0 + 4);
            yv[0] += ba.x; yv[1] += ba.y; yv[2] += ba.z; yv[3] += ba.w;
            yv[4] += bb.x; yv[5] += bb.y; yv[6] += bb.z; yv[7] += bb.w;
        }
        if (EPI == EPI_GELU) {
#pragma unroll
            for (int t = 0; t < 8; t++) yv[t] = gelu(yv[t]);
        }
        if (EPI == EPI_RESID) {
            const float *rp = ea.R + (size_t)m * ea.ldr + n0;
            const float4 ra = *reinterpret_cast<const float4 *>(rp);
            const float4 rb = *reinterpret_cast<const float4 *>(rp + 4);
            yv[0] += ra.x; yv[1] += ra.y; yv[2] += ra.z; yv[3] += ra.w;
            yv[4] += rb.x; yv[5] += rb.y; yv[6] += rb.z; yv[7] += rb.w;
        }
        float *dst = Y + (size_t)m * ldy + n0;
        *reinterpret_cast<float4 *>(dst) = make_float4(yv[0], yv[1], yv[2], yv[3]);
        *reinterpret_cast<float4 *>(dst + 4) = make_float4(yv[4], yv[5], yv[6], yv[7]);
    }
}

// Few rows (4 to FEW_ROWS: the in-context stage of a small batch): one workgroup per 32 rows x 32 TN columns, its
// eight wavefronts splitting K = 128 NST eight ways (NST 16-column steps each, one power of two per row and
// wavefront). With so few steps a pipelined loop waits for memory once per step or two; here every global read of
// the workgroup is issued at its start -- the wavefront's weight steps, its rows' slice of X, the epilogue's bias and
// residual (a bias is required), with LN the norm's weights and with QM the query MLP's weight images, biases and
// scales (both staged in LDS) -- so that one memory latency precedes the products. The partial products, unscaled to f32, are summed
// through LDS in wavefront order; wavefront w finishes accumulators 2 w and 2 w + 1 of every tile (two adjacent
// columns of the lane's row). With QM (one head of 64 columns a workgroup, TN = 2) the finished tile goes through
// LDS and the workgroup runs the head's query MLP on it (qmlp64_tile) from the staged weights.
constexpr int FEW_WAVES = 8;
// up to this many rows (the split-K kernel beyond: 384 rows 1.509 -> 1.330 ms a prediction, 512 rows 1.683 ->
// 1.525, 1,024 rows 2.496 -> 2.403 ms; at 2,048 rows the split-K kernel's four tiles a workgroup win)
constexpr int FEW_ROWS = 1024;
// up to this many rows the f32 kernels (k_gemv, k_qmlp_rows) take the dense layers: their work grows with the rows,
// and from 4 rows k_dense_few is faster
constexpr int GEMV_SPLIT_ROWS = 3;
constexpr int QPITCH = 68;  // row pitch of the query tile in LDS

template <int EPI, bool LN, int TN, int NST, bool QM>
__global__ __launch_bounds__(512) void k_dense_few(int M, const float *__restrict__ X, int ldx,
                                                    const uint8_t *__restrict__ wimg, int wshift,
                                                    const float *__restrict__ b, float *Y, int ldy, SplitEpi ea,
                                                    const float *__restrict__ lnw, const float *__restrict__ lnb) {
    static_assert(!QM || (TN == 2 && LN && EPI == EPI_NONE), "the query MLP follows the normed query projection");
    static_assert(!LN || NST == 4, "the fused layer norm takes K = 512, one column a thread");
    constexpr int K = 16 * NST * FEW_WAVES, KS = K / 16;
    // per wavefront: its rows' K slice (32 rows x 4 NST float4, xrow_at's order), then over it the wavefront's partial
    // sums [tile][accumulator pair][lane] (float2)
    constexpr int STG = 32 * 64 * NST;  // bytes
    static_assert(TN * 8 * 64 * 8 <= STG, "a wavefront's partial sums fit its staging");
    __shared__ __align__(16) uint8_t stage[FEW_WAVES * STG];
    auto red = [&](int w, int T, int pr) { return reinterpret_cast<float2 *>(stage + w * STG) + (T * 8 + pr) * 64; };
    __shared__ float rsum[FEW_WAVES][32];
    __shared__ float lns[LN ? 2 * K : 1];
    __shared__ __align__(16) uint8_t qimg[QM ? 2 * 8 * 2048 : 16];
    __shared__ float qvec[QM ? 3 * 64 : 1];
    __shared__ __align__(16) float qt[QM ? 32 * QPITCH : 4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int m = blockIdx.y * 32 + r32;
    const bool live = m < M;
    const int mr = live ? m : 0;  // rows past M read row 0 and are never stored
    const int nt0 = blockIdx.x * TN;
    const int k0 = wave * 16 * NST;

    halfx8 wh[NST][TN], wl[NST][TN];
    const uint8_t *wp = wimg + ((size_t)nt0 * KS + wave * NST) * 2048 + (g * 32 + r32) * 16;
#pragma unroll
    for (int j = 0; j < NST; j++)
#pragma unroll
        for (int T = 0; T < TN; T++) {
            const uint8_t *src = wp + ((size_t)T * KS + j) * 2048;
            wh[j][T] = *reinterpret_cast<const halfx8 *>(src);
            wl[j][T] = *reinterpret_cast<const halfx8 *>(src + 1024);
        }
    // this wavefront's rows, columns k0 .. k0 + 16 NST - 1, copied into its staging by DMA: copy i, lane l fills
    // float4 slot 64 i + l, which holds row (64 i + l) / (4 NST), float4 column c ^ (row % 16) of it with c the slot
    // within the row -- each copy reads whole runs of rows (a lane a row, as the B operand wants them, touched 32 rows
    // a load: 64 rows 5.9 -> 4.6 us for the output projection), and the B operand's reads, a row a lane, fall on
    // distinct bank groups
    {
        constexpr int F4 = 4 * NST;  // float4 per row
        const int m0 = blockIdx.y * 32;
        static_assert(NST == 4 || NST == 8, "16 or 32 float4 a row: the swizzle stays inside the row");
#pragma unroll
        for (int i = 0; i < 2 * NST; i++) {
            const int slot = 64 * i + lane, row = slot / F4, c = (slot % F4) ^ (row & 15);
            const float *src = X + (size_t)min(m0 + row, M - 1) * ldx + k0 + 4 * c;
            copy16_to_lds(src, stage + wave * STG + 1024 * i);
        }
    }
    auto xrow_at = [&](int j, int hf) {  // row r32, float4 column 4 j + 2 g + hf
        const int c = 4 * j + 2 * g + hf;
        return *reinterpret_cast<const float4 *>(stage + wave * STG + 16 * (r32 * 4 * NST + (c ^ (r32 & 15))));
    };
    // this thread's outputs: accumulators 2 wave, 2 wave + 1 of each tile, i.e. columns nc, nc + 1 of the tile
    const int nc = 16 * (wave >> 2) + 8 * g + 2 * (wave & 3);
    float2 bias[TN], res[TN];
#pragma unroll
    for (int T = 0; T < TN; T++) {
        const int n = 32 * (nt0 + T) + nc;
        bias[T] = *reinterpret_cast<const float2 *>(b + n);
        res[T] = EPI == EPI_RESID ? *reinterpret_cast<const float2 *>(ea.R + (size_t)mr * ea.ldr + n)
                                  : make_float2(0.0f, 0.0f);
    }
    float lw = 0.0f, lb = 0.0f;
    if (LN) {
        lw = lnw[tid];
        lb = lnb[tid];
    }
    u32x4 qs[4];
    float qv = 0.0f;
    if (QM) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            qs[i] = *reinterpret_cast<const u32x4 *>((i < 2 ? ea.w0 : ea.w2) + 16 * (tid + 512 * (i & 1)));
        // threads 0..191: b0, b2, the head's scales (the rest reread the last scale, unused)
        qv = *(tid < 64 ? ea.b0 + tid : tid < 128 ? ea.b2 + (tid - 64) : ea.scale + 64 * blockIdx.x + min(tid - 128, 63));
    }

    float xv[NST][8];
    __builtin_amdgcn_s_waitcnt(0);  // every read of this thread, its rows' copies included, has landed
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // and every lane's: the wavefront's staging is whole
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int j = 0; j < NST; j++) {
        const float4 a = xrow_at(j, 0), c = xrow_at(j, 1);
        xv[j][0] = a.x; xv[j][1] = a.y; xv[j][2] = a.z; xv[j][3] = a.w;
        xv[j][4] = c.x; xv[j][5] = c.y; xv[j][6] = c.z; xv[j][7] = c.w;
    }
    if (LN) {
        // this wavefront holds columns k0 .. k0 + 63 of its 32 rows; the rows' sums go through LDS (two passes:
        // mean, then biased variance; eps 1e-5)
        lns[tid] = lw;
        lns[K + tid] = lb;
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < NST; j++)
#pragma unroll
            for (int t = 0; t < 8; t++) sum += xv[j][t];
        sum += __shfl_xor(sum, 32, 64);
        if (g == 0) rsum[wave][r32] = sum;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int i = 0; i < FEW_WAVES; i++) tot += rsum[i][r32];
        const float mean = tot / (float)K;
        float sq = 0.0f;
#pragma unroll
        for (int j = 0; j < NST; j++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float dv = xv[j][t] - mean;
                sq += dv * dv;
            }
        sq += __shfl_xor(sq, 32, 64);
        __syncthreads();
        if (g == 0) rsum[wave][r32] = sq;
        __syncthreads();
        tot = 0.0f;
#pragma unroll
        for (int i = 0; i < FEW_WAVES; i++) tot += rsum[i][r32];
        const float inv = 1.0f / sqrtf(tot / (float)K + 1e-5f);
#pragma unroll
        for (int j = 0; j < NST; j++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const int c = k0 + 16 * j + 8 * g + t;
                xv[j][t] = (xv[j][t] - mean) * inv * lns[c] + lns[K + c];
            }
    }
    float xmax = 0.0f;
#pragma unroll
    for (int j = 0; j < NST; j++)
#pragma unroll
        for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[j][t]));
    xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
    const int e = shift_for_max(xmax);
    const float f = ldexpf(1.0f, e);
    floatx16 acc[TN];
#pragma unroll
    for (int T = 0; T < TN; T++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[T][v] = 0.0f;
#pragma unroll
    for (int j = 0; j < NST; j++) {
        halfx8 xh, xl;
        split8(xv[j], f, xh, xl);
#pragma unroll
        for (int T = 0; T < TN; T++) acc[T] = mfma16x3(wh[j][T], wl[j][T], xh, xl, acc[T]);
    }
    const float u = ldexpf(1.0f, -(wshift + e));
    // (the staging's rows were all read into xv before the products: the partial sums may overwrite them)
#pragma unroll
    for (int T = 0; T < TN; T++)
#pragma unroll
        for (int p = 0; p < 8; p++) red(wave, T, p)[lane] = make_float2(acc[T][2 * p] * u, acc[T][2 * p + 1] * u);
    if (QM) {
#pragma unroll
        for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4 *>(qimg + 16 * (tid + 512 * i)) = qs[i];
        if (tid < 192) qvec[tid] = qv;
    }
    __syncthreads();
#pragma unroll
    for (int T = 0; T < TN; T++) {
        float2 s = red(0, T, wave)[lane];
#pragma unroll
        for (int i = 1; i < FEW_WAVES; i++) {
            const float2 o = red(i, T, wave)[lane];
            s.x += o.x;
            s.y += o.y;
        }
        float y0 = s.x + bias[T].x, y1 = s.y + bias[T].y;
        if (EPI == EPI_GELU) {
            y0 = gelu(y0);
            y1 = gelu(y1);
        }
        if (EPI == EPI_RESID) {
            y0 += res[T].x;
            y1 += res[T].y;
        }
        if (QM) {
            qt[r32 * QPITCH + 32 * T + nc] = y0;
            qt[r32 * QPITCH + 32 * T + nc + 1] = y1;
        } else if (live) {
            *reinterpret_cast<float2 *>(Y + (size_t)m * ldy + 32 * (nt0 + T) + nc) = make_float2(y0, y1);
        }
    }
    if (QM) {
        __syncthreads();  // the tile is whole and the partial sums are all read: their LDS takes the MLP's tiles
        static_assert(2 * 32 * QMP * 4 <= sizeof(stage), "the query MLP's tiles fit in LDS");
        float *hs = reinterpret_cast<float *>(stage);
        const int m0 = blockIdx.y * 32;
        const QmlpOps<1> qo = qmlp64_read<1, 512>(tid, qimg, qvec, qimg + 8 * 2048, qvec + 64, qvec + 128);
        qmlp64_tile<1, 512>(qt, QPITCH, hs, hs + 32 * QMP, tid, qo, ea.s0, ea.s2, Y + (size_t)m0 * ldy + 64 * blockIdx.x,
                            ldy, min(32, M - m0));
    }
}

template <int NST>
static void launch_few(hipStream_t s, int M, int N, const float *X, int ldx, const uint8_t *img, int shift,
                       const float *b, float *Y, int ldy, Epi epi, const SplitEpi &ea, const float *lnw,
                       const float *lnb) {
    const dim3 grid(N / 32, (M + 31) / 32);
    const bool ln = lnw != nullptr;
    if (NST == 4 && ln) {
        if (epi == EPI_NONE)
            hipLaunchKernelGGL((k_dense_few<EPI_NONE, NST == 4, 1, NST, false>), grid, dim3(512), 0, s, M, X, ldx, img,
                               shift, b, Y, ldy, ea, lnw, lnb);
        else if (epi == EPI_GELU)
            hipLaunchKernelGGL((k_dense_few<EPI_GELU, NST == 4, 1, NST, false>), grid, dim3(512), 0, s, M, X, ldx, img,
                               shift, b, Y, ldy, ea, lnw, lnb);
        else
            hipLaunchKernelGGL((k_dense_few<EPI_RESID, NST == 4, 1, NST, false>), grid, dim3(512), 0, s, M, X, ldx,
                               img, shift, b, Y, ldy, ea, lnw, lnb);
    } else if (epi == EPI_NONE) {
        hipLaunchKernelGGL((k_dense_few<EPI_NONE, false, 1, NST, false>), grid, dim3(512), 0, s, M, X, ldx, img, shift,
                           b, Y, ldy, ea, nullptr, nullptr);
    } else if (epi == EPI_GELU) {
        hipLaunchKernelGGL((k_dense_few<EPI_GELU, false, 1, NST, false>), grid, dim3(512), 0, s, M, X, ldx, img, shift,
                           b, Y, ldy, ea, nullptr, nullptr);
    } else {
        hipLaunchKernelGGL((k_dense_few<EPI_RESID, false, 1, NST, false>), grid, dim3(512), 0, s, M, X, ldx, img,
                           shift, b, Y, ldy, ea, nullptr, nullptr);
    }
    TAH_LAUNCHED();
}

// grid ceil(M / 128); 256 threads: q [rows * heads][64] in place, wavefront w the query-heads of rows 32 (4 x + w) +
// 0..31 of that view.
__global__ __launch_bounds__(256) void k_qmlp64(int M, int heads, float *__restrict__ q, const uint8_t *__restrict__ w0,
                                                int s0, const float *__restrict__ b0, const uint8_t *__restrict__ w2,
                                                int s2, const float *__restrict__ b2, const float *__restrict__ scale) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int m = (blockIdx.x * 4 + wave) * 32 + r32;
    const bool live = m < M;
    float *qr = q + (size_t)(live ? m : 0) * 64;
    float xv[4][8];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
        if (live) {
            a = *reinterpret_cast<const float4 *>(qr + 16 * ks + 8 * g);
            c = *reinterpret_cast<const float4 *>(qr + 16 * ks + 8 * g + 4);
        }
        xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
        xv[ks][4] = c.x; xv[ks][5] = c.y; xv[ks][6] = c.z; xv[ks][7] = c.w;
    }
    qmlp64_lane(xv, r32, g, w0, s0, b0, w2, s2, b2, scale + (size_t)(m % heads) * 64, live ? qr : nullptr);
}

// The same for a few rows (at most QR_ROWS): one workgroup per row, wavefront h its query-head h, in plain f32. The
// MLP's two 64 x 64 weight matrices (shared by the heads) are staged in LDS once per workgroup, rows padded so that
// lane j's reads of row j hit distinct banks; lane j forms hidden unit j, then output j, each a 64-term dot product
// summed in order and the bias added after, as the reference's linear does (src/kern.rs:125-130).
constexpr int QR_ROWS = 8;
__global__ __launch_bounds__(512) void k_qmlp_rows(int heads, float *__restrict__ q, const float *__restrict__ w0,
                                                   const float *__restrict__ b0, const float *__restrict__ w2,
                                                   const float *__restrict__ b2, const float *__restrict__ scale) {
    __shared__ float W0[64][65], W2[64][65], xs[8][64], hs[8][64];
    const int tid = threadIdx.x, lane = tid & 63, h = tid >> 6;
    for (int i = tid; i < 64 * 64; i += 512) {
        W0[i >> 6][i & 63] = w0[i];
        W2[i >> 6][i & 63] = w2[i];
    }
    float *qr = q + ((size_t)blockIdx.x * heads + h) * 64;
    const bool live = h < heads;
    const float x = live ? qr[lane] : 0.0f;
    xs[h][lane] = x;
    __syncthreads();
    float a = 0.0f;
#pragma unroll 16
    for (int k = 0; k < 64; k++) a += W0[lane][k] * xs[h][k];
    hs[h][lane] = gelu(a + b0[lane]);
    __syncthreads();
    float o = 0.0f;
#pragma unroll 16
    for (int k = 0; k < 64; k++) o += W2[lane][k] * hs[h][k];
    o += b2[lane];
    if (live) qr[lane] = x * (scale[h * 64 + lane] * (1.0f + tanh1(o)));
}

// The query of one to QROWS rows in one launch (src/nn.rs:130-152: layer_norm1, the query projection, the query MLP
// and the modulation), a workgroup per head of 64 columns, d = 512, in plain f32. Thread t forms column t / 16's
// partial dot product over the K columns 4 (t % 16 + 16 i) .. + 3, i < 8; every global read of the workgroup -- its 64 weight
// rows (128 KB), the MLP's two matrices, the biases and scales -- is issued at its start, so that one memory latency
// precedes the sums, where the projection and the MLP as two launches took two (the MLP's on one workgroup). The
// rows are normalised once in LDS; the 16 partials of a column, or of a hidden or output unit of the MLP, are summed
// across their 16 lanes.
constexpr int QROWS = 3;
__global__ __launch_bounds__(1024) void k_query_rows(int M, const float *__restrict__ X, int ldx,
                                                     const float *__restrict__ W, const float *__restrict__ bq,
                                                     const float *__restrict__ n1w, const float *__restrict__ n1b,
                                                     const float *__restrict__ w0, const float *__restrict__ b0,
                                                     const float *__restrict__ w2, const float *__restrict__ b2,
                                                     const float *__restrict__ scale, float *__restrict__ Y, int ldy) {
    constexpr int D = 512;
    __shared__ __align__(16) float xs[QROWS][D];
    __shared__ float stat[QROWS][2];
    __shared__ __align__(16) float qs[QROWS][64], hs[QROWS][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.x, c = tid >> 4, sl = tid & 15;
    // columns 4 (sl + 16 i) .. + 3 of the weight row, i < 8: each load instruction reads 256 contiguous bytes of a
    // row per 16 lanes (a thread's 128 contiguous bytes took 15.6 us a launch, 64 rows touched per instruction)
    float4 wv[8];
    const float4 *wp = reinterpret_cast<const float4 *>(W + (size_t)(64 * h + c) * D) + sl;
#pragma unroll
    for (int i = 0; i < 8; i++) wv[i] = wp[16 * i];
    // the MLP: thread t's unit j = t / 16 and K slice 4 (t % 16) of both matrices
    const float4 m0 = *reinterpret_cast<const float4 *>(w0 + c * 64 + 4 * sl);
    const float4 m2 = *reinterpret_cast<const float4 *>(w2 + c * 64 + 4 * sl);
    const float bqc = bq[64 * h + c], b0c = b0[c], b2c = b2[c], scc = scale[64 * h + c];
    // the rows, four values a thread, with their norm weights
    const bool xt = tid < M * (D / 4);
    const int xr = tid / (D / 4), xk = 4 * (tid % (D / 4));
    float4 g4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c4 = g4;
    if (xt) {
        *reinterpret_cast<float4 *>(&xs[xr][xk]) = *reinterpret_cast<const float4 *>(X + (size_t)xr * ldx + xk);
        g4 = *reinterpret_cast<const float4 *>(n1w + xk);
        c4 = *reinterpret_cast<const float4 *>(n1b + xk);
    }
    __syncthreads();
    if (wave < M) {
        // row `wave`: two passes (mean, then biased variance; eps 1e-5)
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < D / 64; i++) sum += xs[wave][lane + 64 * i];
        const float mean = wave_sum(sum) / (float)D;
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < D / 64; i++) {
            const float dv = xs[wave][lane + 64 * i] - mean;
            sq += dv * dv;
        }
        const float inv = 1.0f / sqrtf(wave_sum(sq) / (float)D + 1e-5f);
        if (lane == 0) {
            stat[wave][0] = mean;
            stat[wave][1] = inv;
        }
    }
    __syncthreads();
    if (xt) {
        const float mean = stat[xr][0], inv = stat[xr][1];
        float4 x = *reinterpret_cast<const float4 *>(&xs[xr][xk]);
        x.x = (x.x - mean) * inv * g4.x + c4.x;
        x.y = (x.y - mean) * inv * g4.y + c4.y;
        x.z = (x.z - mean) * inv * g4.z + c4.z;
        x.w = (x.w - mean) * inv * g4.w + c4.w;
        *reinterpret_cast<float4 *>(&xs[xr][xk]) = x;
    }
    __syncthreads();
    // the projection: column c, K slice sl; the slice sums over the 16 lanes of the column
    auto sum16 = [](float v) {
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
        return v;
    };
#pragma unroll
    for (int r = 0; r < QROWS; r++) {
        if (r >= M) break;
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 x = *reinterpret_cast<const float4 *>(&xs[r][4 * sl + 64 * i]);
            a += (wv[i].x * x.x + wv[i].y * x.y) + (wv[i].z * x.z + wv[i].w * x.w);
        }
        a = sum16(a);
        if (sl == 0) qs[r][c] = a + bqc;
    }
    __syncthreads();
    // hidden unit c of the MLP
#pragma unroll
    for (int r = 0; r < QROWS; r++) {
        if (r >= M) break;
        const float4 x = *reinterpret_cast<const float4 *>(&qs[r][4 * sl]);
        const float a = sum16((m0.x * x.x + m0.y * x.y) + (m0.z * x.z + m0.w * x.w));
        if (sl == 0) hs[r][c] = gelu(a + b0c);
    }
    __syncthreads();
    // output c of the MLP, then the modulation of query coordinate c
#pragma unroll
    for (int r = 0; r < QROWS; r++) {
        if (r >= M) break;
        const float4 x = *reinterpret_cast<const float4 *>(&hs[r][4 * sl]);
        const float o = sum16((m2.x * x.x + m2.y * x.y) + (m2.z * x.z + m2.w * x.w)) + b2c;
        if (sl == 0) Y[(size_t)r * ldy + 64 * h + c] = qs[r][c] * (scc * (1.0f + tanh1(o)));
    }
}

bool query_rows_fits(const DevBlock &b, int M, const float *X, int ldx, const float *Y) {
    return M >= 1 && M <= QROWS && b.d == 512 && b.heads == 8 && qmlp_fused(b) && b.in_w && b.in_b && b.n1w && b.n1b &&
           b.q0w && b.q0b && b.q2w && b.q2b && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(b.in_w) & 15) == 0 && (reinterpret_cast<uintptr_t>(b.q0w) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(b.q2w) & 15) == 0 && (reinterpret_cast<uintptr_t>(b.n1w) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(b.n1b) & 15) == 0 && Y != nullptr;
}

void query_rows(hipStream_t s, int M, const float *X, int ldx, const DevBlock &b, const float *scale, float *q) {
    if (!query_rows_fits(b, M, X, ldx, q)) throw ArgError{"query_rows: shape not supported"};
    hipLaunchKernelGGL(k_query_rows, dim3(b.heads), dim3(1024), 0, s, M, X, ldx, b.in_w, b.in_b, b.n1w, b.n1b, b.q0w,
                       b.q0b, b.q2w, b.q2b, scale, q, b.d);
    TAH_LAUNCHED();
}

bool qmlp_fused(const DevBlock &b) {
    return b.heads > 0 && b.d == 64 * b.heads && b.ss_hidden == 64 && b.q0_s.img && b.q2_s.img && b.q0_s.K == 64 &&
           b.q2_s.K == 64 && b.q0_s.N == 64 && b.q2_s.N == 64;
}

void qmlp(hipStream_t s, int rows, const DevBlock &b, const float *scale, float *q) {
    const int M = rows * b.heads;
    if (M <= 0) return;
    if (rows <= QR_ROWS && b.heads <= 8 && b.q0w && b.q2w) {
        hipLaunchKernelGGL(k_qmlp_rows, dim3(rows), dim3(512), 0, s, b.heads, q, b.q0w, b.q0b, b.q2w, b.q2b, scale);
        TAH_LAUNCHED();
        return;
    }
    hipLaunchKernelGGL(k_qmlp64, dim3((M + 127) / 128), dim3(256), 0, s, M, b.heads, q, b.q0_s.img, b.q0_s.shift, b.q0b,
                       b.q2_s.img, b.q2_s.shift, b.q2b, scale);
    TAH_LAUNCHED();
}

bool gemm_split_fits(int N, int K) { return N > 0 && N % 32 == 0 && K > 0 && K % 16 == 0; }

template <int EPI>
static void launch_split(hipStream_t s, int M, int N, int K, const float *X, int ldx, const SplitW &w, const float *b,
                         float *Y, int ldy, const SplitEpi &ea) {
    const int row_groups = (M + 127) / 128;
    // two column tiles a wavefront halves the reads of X, when there are waves enough to fill the chip without
    const bool wide = N % 64 == 0 && (long)row_groups * 4 * (N / 64) >= 2048;
    if (wide)
        hipLaunchKernelGGL((k_gemm_split<EPI, 2>), dim3(N / 64, row_groups), dim3(256), 0, s, M, N, K, X, ldx, w.img,
                           w.shift, b, Y, ldy, ea);
    else
        hipLaunchKernelGGL((k_gemm_split<EPI, 1>), dim3(N / 32, row_groups), dim3(256), 0, s, M, N, K, X, ldx, w.img,
                           w.shift, b, Y, ldy, ea);
    TAH_LAUNCHED();
}

void gemm_split(hipStream_t s, int M, int N, int K, const float *X, int ldx, const SplitW &w, const float *b, float *Y,
                int ldy, Epi epi, const float *R, int ldr, const float *scale, int heads) {
    if (M <= 0) return;
    if (!w.img || !gemm_split_fits(N, K) || K != w.K || w.row0 % 32 || N + w.row0 > w.N)
        throw ArgError{"gemm_split: the weight image does not fit the product"};
    if ((size_t)(M + 127) / 128 > 65535) throw ArgError{"gemm_split: too many rows for one launch"};
    if ((ldx % 4) || (ldy % 4) || (reinterpret_cast<uintptr_t>(X) & 15) || (reinterpret_cast<uintptr_t>(Y) & 15))
        throw ArgError{"gemm_split: rows must be 16-byte aligned"};
    const SplitEpi ea{R, ldr, scale, heads > 0 ? heads : 1};
    SplitW sub = w;
    sub.img = w.img + (size_t)(w.row0 / 32) * (w.K / 16) * 2048;
    switch (epi) {
        case EPI_NONE: launch_split<EPI_NONE>(s, M, N, K, X, ldx, sub, b, Y, ldy, ea); break;
        case EPI_GELU: launch_split<EPI_GELU>(s, M, N, K, X, ldx, sub, b, Y, ldy, ea); break;
        case EPI_RESID: launch_split<EPI_RESID>(s, M, N, K, X, ldx, sub, b, Y, ldy, ea); break;
        case EPI_QMOD: launch_split<EPI_QMOD>(s, M, N, K, X, ldx, sub, b, Y, ldy, ea); break;
        case EPI_SCALE: launch_split<EPI_SCALE>(s, M, N, K, X, ldx, sub, b, Y, ldy, ea); break;
        default: throw ArgError{"gemm_split: unknown epilogue"};
    }
}

template <bool LN, int TN, int W = 4, int CW = 128>
static void launch_splitk4_tiles(hipStream_t s, int M, int N, int K, const float *X, int ldx, const uint8_t *img,
                                 int shift, const float *b, float *Y, int ldy, Epi epi, const SplitEpi &ea,
                                 const float *lnw, const float *lnb) {
    const dim3 grid((N / (32 * TN)) * ((M + 31) / 32));
    switch (epi) {
        case EPI_NONE:
            hipLaunchKernelGGL((k_gemm_splitk4<EPI_NONE, LN, TN, false, W, CW>), grid, dim3(64 * W), 0, s, M, N, K, X,
                               ldx, img, shift, b, Y, ldy, ea, lnw, lnb);
            break;
        case EPI_GELU:
            hipLaunchKernelGGL((k_gemm_splitk4<EPI_GELU, LN, TN, false, W, CW>), grid, dim3(64 * W), 0, s, M, N, K, X,
                               ldx, img, shift, b, Y, ldy, ea, lnw, lnb);
            break;
        default:
            hipLaunchKernelGGL((k_gemm_splitk4<EPI_RESID, LN, TN, false, W, CW>), grid, dim3(64 * W), 0, s, M, N, K, X,
                               ldx, img, shift, b, Y, ldy, ea, lnw, lnb);
            break;
    }
    TAH_LAUNCHED();
}

// Four tiles a workgroup from 2,048 rows (two, with twice the workgroups, measured slower there); two below 512 rows,
// where the few workgroups each stream half the weights
constexpr int SPLITK_TWO_TILES_ROWS = 512;
// workgroups of eight wavefronts the card runs at once (one a compute unit)
constexpr long SPLITK_ONE_ROUND = 256;

template <bool LN>
static void launch_splitk4(hipStream_t s, int M, int N, int K, const float *X, int ldx, const uint8_t *img, int shift,
                           const float *b, float *Y, int ldy, Epi epi, const SplitEpi &ea, const float *lnw,
                           const float *lnb) {
    if (M <= SPLITK_TWO_TILES_ROWS && N % 64 == 0) {
        launch_splitk4_tiles<LN, 2>(s, M, N, K, X, ldx, img, shift, b, Y, ldy, epi, ea, lnw, lnb);
        return;
    }
    // eight wavefronts where the four-tile grid is at most one workgroup a compute unit and no layer norm spans them
    // (2,048 rows: out-projection 10.2 -> 10.0 us, second feed-forward layer 15.3 -> 14.4 us; the first feed-forward
    // layer's 512 workgroups would run in two rounds, 16.6 -> 19.5 us, and so would 10,000 rows' grids: 46 -> 67 us)
    if constexpr (!LN) {
        if ((K == 512 || K == 1024) && (long)(N / 128) * ((M + 31) / 32) <= SPLITK_ONE_ROUND) {
            if (K == 512)
                launch_splitk4_tiles<LN, 4, 8, 64>(s, M, N, K, X, ldx, img, shift, b, Y, ldy, epi, ea, lnw, lnb);
            else
                launch_splitk4_tiles<LN, 4, 8, 128>(s, M, N, K, X, ldx, img, shift, b, Y, ldy, epi, ea, lnw, lnb);
            return;
        }
    }
    launch_splitk4_tiles<LN, 4>(s, M, N, K, X, ldx, img, shift, b, Y, ldy, epi, ea, lnw, lnb);
}

// the query projection's one-head-a-workgroup grid up to this many workgroups: the card's compute units
constexpr long QUERY_ONE_HEAD_TILES = 256;

bool query_split_fits(const DevBlock &b, int M, const float *X, int ldx, const float *Y) {
    const SplitW &w = b.in_s;
    return M > GEMV_SPLIT_ROWS && w.img && b.in_b && w.row0 == 0 && w.K == b.d && b.d == 512 && b.d % 128 == 0 && b.heads > 0 &&
           b.d == 64 * b.heads && qmlp_fused(b) && b.n1w && b.n1b && ldx % 4 == 0 &&
           (reinterpret_cast<uintptr_t>(X) & 15) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0 &&
           (size_t)(M + 31) / 32 <= 65535;
}

void query_split(hipStream_t s, int M, const float *X, int ldx, const DevBlock &b, const float *scale, float *q) {
    if (!query_split_fits(b, M, X, ldx, q)) throw ArgError{"query_split: shape not supported"};
    SplitEpi ea{nullptr, 0, scale, b.heads};
    ea.w0 = b.q0_s.img;
    ea.s0 = b.q0_s.shift;
    ea.b0 = b.q0b;
    ea.w2 = b.q2_s.img;
    ea.s2 = b.q2_s.shift;
    ea.b2 = b.q2b;
    const int d = b.d;
    if (M <= FEW_ROWS) {
        hipLaunchKernelGGL((k_dense_few<EPI_NONE, true, 2, 4, true>), dim3(d / 64, (M + 31) / 32), dim3(512), 0, s, M,
                           X, ldx, b.in_s.img, b.in_s.shift, b.in_b, q, d, ea, b.n1w, b.n1b);
        TAH_LAUNCHED();
        return;
    }
    // a workgroup per head while that grid fits one workgroup a compute unit (twice the workgroups, each streaming
    // half the weights: 1,024 rows 10.3 against 12.9 us), two heads a workgroup beyond (1,536 rows 13.1 against 14.6
    // us, 2,048 rows 13.6 against 15.2, 10,000 rows 48.2 against 57.7), on eight wavefronts while those are one round
    // of workgroups (2,048 rows 15.7 -> 13.6 us)
    const long tiles = (long)(d / 64) * ((M + 31) / 32);
    if (tiles <= QUERY_ONE_HEAD_TILES)
        hipLaunchKernelGGL((k_gemm_splitk4<EPI_NONE, true, 2, true>), dim3(tiles), dim3(256), 0, s, M, d, d, X, ldx,
                           b.in_s.img, b.in_s.shift, b.in_b, q, d, ea, b.n1w, b.n1b);
    else if (tiles / 2 <= SPLITK_ONE_ROUND)
        hipLaunchKernelGGL((k_gemm_splitk4<EPI_NONE, true, 4, true, 8, 64>), dim3(tiles / 2), dim3(512), 0, s, M, d,
                           d, X, ldx, b.in_s.img, b.in_s.shift, b.in_b, q, d, ea, b.n1w, b.n1b);
    else
        hipLaunchKernelGGL((k_gemm_splitk4<EPI_NONE, true, 4, true>), dim3(tiles / 2), dim3(256), 0, s, M, d, d, X,
                           ldx, b.in_s.img, b.in_s.shift, b.in_b, q, d, ea, b.n1w, b.n1b);
    TAH_LAUNCHED();
}

void dense(hipStream_t s, int M, int N, int K, const float *X, int ldx, const float *W, const SplitW &w, const float *b,
           float *Y, int ldy, Epi epi, const float *R, int ldr, const float *lnw, const float *lnb, float *t) {
    const bool img = w.img && gemm_split_fits(N, K) && K == w.K && w.row0 % 32 == 0 && N + w.row0 <= w.N &&
                     ldx % 4 == 0 && ldy % 4 == 0 && (reinterpret_cast<uintptr_t>(X) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
    const bool epis = epi == EPI_NONE || epi == EPI_GELU || epi == EPI_RESID;
    if (img && epis && b && M > GEMV_SPLIT_ROWS && M <= FEW_ROWS && N % 32 == 0 && (K == 512 || (K == 1024 && !lnw))) {
        if ((ldx % 4) || (reinterpret_cast<uintptr_t>(X) & 15) || (R && ldr % 2))
            throw ArgError{"dense: rows must be 16-byte aligned"};
        const SplitEpi ea{R, ldr, nullptr, 1};
        const uint8_t *sub = w.img + (size_t)(w.row0 / 32) * (w.K / 16) * 2048;
        if (K == 512)
            launch_few<4>(s, M, N, X, ldx, sub, w.shift, b, Y, ldy, epi, ea, lnw, lnb);
        else
            launch_few<8>(s, M, N, X, ldx, sub, w.shift, b, Y, ldy, epi, ea, nullptr, nullptr);
        return;
    }
    // from 64 rows the split kernels win (two tiles a workgroup below 512 rows: a 64-row prediction 1.285 against
    // 1.316 ms on the f32 kernels, 256 rows 1.52 against 1.61 ms with four tiles)
    const bool split = img && M >= 64 && epis;
    const bool k4 = split && N % 128 == 0 && K % 512 == 0 && K <= 4 * SPLITK_MAX_KQ;  // whole 128-column chunks
    if (lnw && !split && W && gemm_ln_fits(M, K, X, ldx, W)) {
        // few rows: the layer norm inside the product's kernel
        gemm(s, M, N, K, X, ldx, W, b, Y, ldy, epi, R, ldr, lnw, lnb);
        return;
    }
    if (lnw && !(k4 && K == 512)) {
        // layer normalisation first, into t
        if (!t) throw ArgError{"dense: layer normalisation needs a scratch buffer"};
        layer_norm(s, M, K, X, ldx, lnw, lnb, t, K);
        X = t;
        ldx = K;
        lnw = lnb = nullptr;
    }
    if (!split) {
        gemm(s, M, N, K, X, ldx, W, b, Y, ldy, epi, R, ldr);
        return;
    }
    if (k4) {
        if ((size_t)(M + 31) / 32 > 65535) throw ArgError{"dense: too many rows for one launch"};
        const SplitEpi ea{R, ldr, nullptr, 1};
        const uint8_t *sub = w.img + (size_t)(w.row0 / 32) * (w.K / 16) * 2048;
        if (lnw)
            launch_splitk4<true>(s, M, N, K, X, ldx, sub, w.shift, b, Y, ldy, epi, ea, lnw, lnb);
        else
            launch_splitk4<false>(s, M, N, K, X, ldx, sub, w.shift, b, Y, ldy, epi, ea, nullptr, nullptr);
        return;
    }
    gemm_split(s, M, N, K, X, ldx, w, b, Y, ldy, epi, R, ldr, nullptr, 1);
}

}  // namespace tah
