// Fused transformer sub-blocks for the column and row stages, on the fp16 matrix cores with split f32 operands.
//
// The feed-forward sub-block x += l2(gelu(l1(layer_norm2(x)))) (src/nn.rs:154-170 after the attention; the
// reference runs it as kern::layer_norm, two kern::linear and kern::gelu passes, src/predict.rs:233-246) runs as one
// kernel for width 128 and hidden width 256, the shape of the full-size column and row blocks:
//
//  * each wavefront owns 32 rows and keeps them in registers from start to end; the products are formed transposed,
//    H^T = W1 X^T and Y^T = W2 H^T, with the rows as the B operand (lane l holds row l % 32, eight consecutive
//    columns 8 (l / 32) + 0..7 of each 16-column step);
//  * the A operands, the weights, are read with their rows in sigma32 order, which leaves each lane's accumulators
//    holding eight consecutive hidden units: exactly the B operand of the second product, so the hidden layer
//    never leaves the registers;
//  * the weights stream through two 32 KB LDS buffers, one slice per step, copied global -> LDS by DMA
//    (global_load_lds_dwordx4) and shared by the workgroup's four wavefronts. They are stored pre-split at upload
//    in exactly the order of those slices (weight_image in the C ABI: blocks of 128 rows, then 16-column steps);
//  * the first product runs in two halves of 128 hidden units, and each product's matrix work overlaps the vector
//    work of the half before it: half 1's products under half 0's bias, GELU and split, then the second product's
//    sums over half 0 under half 1's (the vector work is as long as the matrix work here; run one after the other,
//    the matrix cores idle through it);
//  * the first layer's bias is staged in LDS, so that the reads next to the GELU wait for LDS, not for the caches;
//  * layer normalisation needs each row's sums: a row's 128 values sit on lanes l and l + 32, so one cross-lane step;
//  * each row is scaled by its own power of two before splitting (its largest magnitude below 2^14; each half of
//    the hidden layer by its own), the weights by one per matrix; the products are unscaled in the epilogues.
#include "common.hpp"
#include "device_math.hpp"

namespace tah {

constexpr int CPS = 4;              // 16-column steps (8 KB of a 128-row weight block) per weight slice
constexpr int SLAB = CPS * 8192;    // one weight slice in LDS
constexpr int NSL = 8 * 8192 / SLAB;  // slices per 128 x 128 weight block

// bytes (a multiple of 16 * THREADS) from global to LDS by THREADS threads, 16 bytes a lane; in copy i wavefront w's
// 64 lanes fill the 1 KB at 16 THREADS i + 1024 w (a wavefront-uniform LDS base, the lanes' offsets implicit)
template <int THREADS = 256>
__device__ __forceinline__ void dma_to_lds(const uint8_t *src, uint8_t *dst, int bytes, int tid) {
    for (int o = 0; o < bytes; o += 16 * THREADS)
        __builtin_amdgcn_global_load_lds(src + o + 16 * tid, dst + o + 1024 * (tid >> 6), 16, 0, 0);
}

constexpr int FFW = 4;  // wavefronts (of 32 rows each) per k_ff128 workgroup (eight, one workgroup a CU, measured slower)

// The feed-forward body's start, by all 256 threads of a workgroup: the first weight slice's copy into slab (two
// slices, 64 KB of LDS) and the first layer's bias into bias1 (256 floats of LDS).
__device__ __forceinline__ void ff128_start(uint8_t *slab, float *bias1, const uint8_t *__restrict__ w1img,
                                            const float *__restrict__ b1, int tid) {
    dma_to_lds<64 * FFW>(w1img, slab, SLAB, tid);
    if (tid < 64) reinterpret_cast<float4 *>(bias1)[tid] = reinterpret_cast<const float4 *>(b1)[tid];
}

// Layer normalisation of this lane's half row xv (columns 16 ks + 8 g + t; the other half on lane l ^ 32) with
// lnw / lnb in place (two passes, biased variance, eps 1e-5), then its split as the B operand of a 128-column product,
// scaled by the row's power of two 2^sx (its largest magnitude below 2^14); returns sx.
__device__ __forceinline__ int norm_split(float (&xv)[8][8], const float *__restrict__ lnw,
                                          const float *__restrict__ lnb, int g, halfx8 (&xh)[8], halfx8 (&xl)[8]) {
    constexpr int E = 128;
    float sum = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int t = 0; t < 8; t++) sum += xv[ks][t];
    sum += __shfl_xor(sum, 32, 64);
    const float mean = sum / (float)E;
    float sq = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float dv = xv[ks][t] - mean;
            sq += dv * dv;
        }
    sq += __shfl_xor(sq, 32, 64);
    const float inv = 1.0f / sqrtf(sq / (float)E + 1e-5f);
    float xmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        const float4 wa = *reinterpret_cast<const float4 *>(lnw + 16 * ks + 8 * g);
        const float4 wb = *reinterpret_cast<const float4 *>(lnw + 16 * ks + 8 * g + 4);
        const float4 ba = *reinterpret_cast<const float4 *>(lnb + 16 * ks + 8 * g);
        const float4 bb = *reinterpret_cast<const float4 *>(lnb + 16 * ks + 8 * g + 4);
        const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
        const float bv[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
#pragma unroll
        for (int t = 0; t < 8; t++) {
            xv[ks][t] = (xv[ks][t] - mean) * inv * wv[t] + bv[t];
            xmax = fmaxf(xmax, fabsf(xv[ks][t]));
        }
    }
    xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
    const int sx = shift_for_max(xmax);
#pragma unroll
    for (int ks = 0; ks < 8; ks++) split8(xv[ks], ldexpf(1.0f, sx), xh[ks], xl[ks]);
    return sx;
}

// The next block's key and value projection, formed from a feed-forward's result in the same kernel (ff128_rows with
// KV): img the [2 e][e] weight image (the keys' 128 rows, then the values'), shift its power of two, lnw / lnb the
// next block's first normalisation, b its 2 e biases, out the lane's token's [2 e] row (keys, then values).
struct KvNext {
    const uint8_t *img;
    int shift;
    const float *lnw, *lnb, *b;
    float *out;
};

// x += l2(gelu(l1(norm2 x))) + b2 for 32 rows a wavefront (after ff128_start, all 256 threads): xv holds this lane's
// half of its row (columns 16 ks + 8 g + t); xrow is the row's storage, which holds x (read back for the residual
// add) and takes the result (not where !live or !keep). With KV the result goes on, still in registers, through kn's
// normalisation and projection (its four weight slices streamed after W2's) to kn.out (not where !live).
template <bool KV = false>
__device__ __forceinline__ void ff128_rows(float (&xv)[8][8], bool live, float *xrow, uint8_t *slab, const float *bias1,
                                           const float *__restrict__ lnw, const float *__restrict__ lnb,
                                           const uint8_t *__restrict__ w1img, int s1,
                                           const uint8_t *__restrict__ w2img, const float *__restrict__ b2, int s2,
                                           int tid, const KvNext &kn = KvNext{}, bool keep = true) {
    constexpr int E = 128;
    const int lane = tid & 63;
    const int r32 = lane & 31, g = lane >> 5;
    halfx8 xh[8], xl[8];
    const int sx = norm_split(xv, lnw, lnb, g, xh, xl);

    // H^T = W1 X^T in two halves of 128 hidden units (4 tiles of 32 each); the weights stream as slices of CPS
    // 16-column steps, W1's (half-major) then W2's, slice j into buffer j % 2
    const int arow = sigma32(r32);
    // slices 0 .. 2 NSL - 1: W1 (two 128-row blocks), then 2 NSL .. 4 NSL - 1: W2 (128 rows, 256 columns), then
    // with KV 4 NSL .. 6 NSL - 1: the next block's key and value weights (two 128-row blocks)
    constexpr int NSLICES = (KV ? 6 : 4) * NSL;
    auto slice = [&](int j) {
        return j < 2 * NSL   ? w1img + (size_t)j * SLAB
               : j < 4 * NSL ? w2img + (size_t)(j - 2 * NSL) * SLAB
                             : kn.img + (size_t)(j - 4 * NSL) * SLAB;
    };
    halfx8 hh8[16], hl8[16];  // the hidden layer, split: 16-unit step k = 2 T + hh of half 0, then of half 1
    static_assert(NSL == 2, "two slices a 128-row weight block: two tiles of the other half activated a slice");

    // wait for slice j (and free slice j - 1's buffer), start slice j + 1's copy; slice j in LDS
    auto next = [&](int j) {
        __builtin_amdgcn_s_waitcnt(0);  // this wavefront's copies of slice j have landed
        __syncthreads();                // everyone's have; slice j - 1's buffer is free
        if (j + 1 < NSLICES) dma_to_lds<64 * FFW>(slice(j + 1), slab + ((j + 1) & 1) * SLAB, SLAB, tid);
        return static_cast<const uint8_t *>(slab + (j & 1) * SLAB);
    };
    // acc[T] += (rows 32 T .. 32 T + 31 of the slice's weights) B over the slice's CPS 16-column steps
    auto mma = [&](floatx16 (&acc)[4], const uint8_t *sl, const halfx8 *bh, const halfx8 *bl, int rows) {
#pragma unroll
        for (int c = 0; c < CPS; c++)
#pragma unroll
            for (int T = 0; T < 4; T++) {
                const int n = 32 * T + arow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(sl + c * 8192 + (g * rows + n) * 16);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(sl + c * 8192 + ((2 + g) * rows + n) * 16);
                acc[T] = mfma16x3(ah, al, bh[c], bl[c], acc[T]);
            }
    };
    // hidden unit of accumulator v of tile T of half h: 128 h + 32 T + 16 (v / 8) + 8 g + v % 8; bias and GELU in
    // place, the running largest magnitude in mx
    const float u1 = ldexpf(1.0f, -(sx + s1));
    auto act = [&](floatx16 &a, int half, int T, float &mx) {
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const float *bp = bias1 + 128 * half + 32 * T + 16 * hh + 8 * g;
            const float4 ba = *reinterpret_cast<const float4 *>(bp), bb = *reinterpret_cast<const float4 *>(bp + 4);
            const float bv[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float hv = gelu(a[8 * hh + t] * u1 + bv[t]);
                a[8 * hh + t] = hv;
                mx = fmaxf(mx, fabsf(hv));
            }
        }
    };
    // a half of the hidden layer, activated, scaled by its own power of two and split into hh8 / hl8
    auto split_half = [&](floatx16 (&a)[4], float mx, int half) {
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const int sh = shift_for_max(mx);
#pragma unroll
        for (int T = 0; T < 4; T++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                float hv[8];
#pragma unroll
                for (int t = 0; t < 8; t++) hv[t] = a[T][8 * hh + t];
                split8(hv, ldexpf(1.0f, sh), hh8[8 * half + 2 * T + hh], hl8[8 * half + 2 * T + hh]);
            }
        return sh;
    };

    // The four products run in slice order (W1's two halves, then W2's two halves of hidden units); each one's
    // matrix work overlaps the vector work of the half before it: H^T half 1 = W1 X^T under GELU of half 0, and
    // Y^T = W2 H^T over half 0 under GELU of half 1. Y's sums over the two halves carry the halves' own scales: between
    // them they are rescaled (exactly) to the second's.
    floatx16 acc0[4], acc1[4], y[4];
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            acc0[T][v] = 0.0f;
            acc1[T][v] = 0.0f;
            y[T][v] = 0.0f;
        }
#pragma unroll
    for (int st = 0; st < NSL; st++) mma(acc0, next(st), xh + CPS * st, xl + CPS * st, 128);
    float m0 = 0.0f;
#pragma unroll
    for (int st = 0; st < NSL; st++) {
        mma(acc1, next(NSL + st), xh + CPS * st, xl + CPS * st, 128);
        act(acc0[2 * st], 0, 2 * st, m0);
        act(acc0[2 * st + 1], 0, 2 * st + 1, m0);
    }
    const int sh0 = split_half(acc0, m0, 0);
    float m1 = 0.0f;
#pragma unroll
    for (int st = 0; st < NSL; st++) {
        mma(y, next(2 * NSL + st), hh8 + CPS * st, hl8 + CPS * st, E);
        act(acc1[2 * st], 1, 2 * st, m1);
        act(acc1[2 * st + 1], 1, 2 * st + 1, m1);
    }
    const int sh1 = split_half(acc1, m1, 1);
    {
        const float r = ldexpf(1.0f, sh1 - sh0);
#pragma unroll
        for (int T = 0; T < 4; T++) y[T] *= r;
    }
#pragma unroll
    for (int st = 0; st < NSL; st++) mma(y, next(3 * NSL + st), hh8 + 8 + CPS * st, hl8 + 8 + CPS * st, E);
    if (!KV && !live) return;
    // output column of accumulator v of tile T: 32 T + 16 (v / 8) + 8 g + v % 8; x += y + b2 (a lane that is not live
    // reads its row's first token, which is there, and stores nothing)
    const float u2 = ldexpf(1.0f, -(sh1 + s2));
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int c0 = 32 * T + 16 * hh + 8 * g;
            float *dst = xrow + c0;
            float rv[8], bv[8], xo[8];
            load8(dst, rv);
            load8(b2 + c0, bv);
#pragma unroll
            for (int t = 0; t < 8; t++) xo[t] = y[T][8 * hh + t] * u2 + bv[t] + rv[t];
            if (live && keep) {
                *reinterpret_cast<float4 *>(dst) = make_float4(xo[0], xo[1], xo[2], xo[3]);
                *reinterpret_cast<float4 *>(dst + 4) = make_float4(xo[4], xo[5], xo[6], xo[7]);
            }
            if constexpr (KV) {
#pragma unroll
                for (int t = 0; t < 8; t++) xv[2 * T + hh][t] = xo[t];
            }
        }
    if constexpr (KV) {
        // the next block's keys (slices 4 NSL ..) then values (6 NSL - NSL ..): 128 outputs each, as four 32-row tiles
        const int sk = norm_split(xv, kn.lnw, kn.lnb, g, xh, xl);
        const float uk = ldexpf(1.0f, -(sk + kn.shift));
#pragma unroll
        for (int part = 0; part < 2; part++) {
            floatx16 a[4];
#pragma unroll
            for (int T = 0; T < 4; T++)
#pragma unroll
                for (int v = 0; v < 16; v++) a[T][v] = 0.0f;
#pragma unroll
            for (int st = 0; st < NSL; st++) mma(a, next(4 * NSL + NSL * part + st), xh + CPS * st, xl + CPS * st, 128);
#pragma unroll
            for (int T = 0; T < 4; T++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const int c0 = 128 * part + 32 * T + 16 * hh + 8 * g;
                    float bv[8], o[8];
                    load8(kn.b + c0, bv);
#pragma unroll
                    for (int t = 0; t < 8; t++) o[t] = a[T][8 * hh + t] * uk + bv[t];
                    if (live) {
                        *reinterpret_cast<float4 *>(kn.out + c0) = make_float4(o[0], o[1], o[2], o[3]);
                        *reinterpret_cast<float4 *>(kn.out + c0 + 4) = make_float4(o[4], o[5], o[6], o[7]);
                    }
                }
        }
    }
}

// grid ceil(M / (32 FFW)); 64 FFW threads. x [M][128] in place.
__global__ __launch_bounds__(64 * FFW, 2) void k_ff128(int M, float *__restrict__ x, const float *__restrict__ lnw,
                                                   const float *__restrict__ lnb, const uint8_t *__restrict__ w1img,
                                                   const float *__restrict__ b1, int s1,
                                                   const uint8_t *__restrict__ w2img, const float *__restrict__ b2,
                                                   int s2) {
    constexpr int E = 128;
    __shared__ __align__(16) uint8_t slab[2 * SLAB];
    __shared__ __align__(16) float bias1[256];  // b1, read next to the GELU it feeds (an LDS read's short wait)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int m = blockIdx.x * 32 * FFW + wave * 32 + r32;
    const bool live = m < M;
    ff128_start(slab, bias1, w1img, b1, tid);

    // this lane's half of row m: columns 16 ks + 8 g + t
    float xv[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
        if (live) {
            const float *src = x + (size_t)m * E + 16 * ks + 8 * g;
            a = *reinterpret_cast<const float4 *>(src);
            b = *reinterpret_cast<const float4 *>(src + 4);
        }
        xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
        xv[ks][4] = b.x; xv[ks][5] = b.y; xv[ks][6] = b.z; xv[ks][7] = b.w;
    }
    ff128_rows(xv, live, x + (size_t)(live ? m : 0) * E, slab, bias1, lnw, lnb, w1img, s1, w2img, b2, s2, tid);
}

// The same sub-block for few rows (grids of at most one workgroup a compute unit): 64 rows a workgroup, each row
// group of 32 on two wavefronts that take one half of the 256 hidden units each -- wavefront w rows 32 (2 x + w / 2)
// .. + 31, hidden units 128 (w % 2) .. + 127 -- so that each wavefront's chain of products and GELU is half as long
// and twice the compute units share the rows (6,400 rows: 19 us a launch on 100 workgroups, where 50 workgroups of
// 128 rows with one wavefront a row group took 23 us).
// Both halves' weight slices stream together, two 32 KB slices a step through a two-step ring (128 KB of LDS): step
// 0 / 1 W1's column halves (K) of both hidden halves, step 2 / 3 W2's columns over each hidden half. The odd
// wavefront's sums over its half go through LDS to the even one, which adds its own, the bias and the residual.
__global__ __launch_bounds__(256, 1) void k_ff128h(int M, float *__restrict__ x, const float *__restrict__ lnw,
                                                   const float *__restrict__ lnb, const uint8_t *__restrict__ w1img,
                                                   const float *__restrict__ b1, int s1,
                                                   const uint8_t *__restrict__ w2img, const float *__restrict__ b2,
                                                   int s2) {
    constexpr int E = 128, STEP = 2 * SLAB;
    constexpr int HP = E + 4;  // the half sums' row pitch in floats: rows 16 bytes apart in the banks
    static_assert(NSL == 2 && 2 * 32 * HP * 4 <= STEP, "two slices a step; the half sums fit a step buffer");
    __shared__ __align__(16) uint8_t ring[2 * STEP];
    __shared__ __align__(16) float bias1[256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int rg = wave >> 1, hf = wave & 1;
    const int m = blockIdx.x * 64 + rg * 32 + r32;
    const bool live = m < M;
    // step t's two slices: W1 (t < 2) block h, K half t: slice 2 h + t; W2 (t >= 2) K steps of hidden half h,
    // K half t - 2: slice 2 NSL + 2 h + (t - 2); half h's slice lands at h * SLAB of the step's buffer
    auto step_copy = [&](int t) {
        uint8_t *dst = ring + (t & 1) * STEP;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const uint8_t *src = t < 2 ? w1img + (size_t)(2 * h + t) * SLAB : w2img + (size_t)(2 * h + t - 2) * SLAB;
            dma_to_lds<256>(src, dst + h * SLAB, SLAB, tid);
        }
    };
    step_copy(0);
    if (tid < 64) reinterpret_cast<float4 *>(bias1)[tid] = reinterpret_cast<const float4 *>(b1)[tid];
    float xv[8][8];
    float *xrow = x + (size_t)(live ? m : 0) * E;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
        if (live) {
            a = *reinterpret_cast<const float4 *>(xrow + 16 * ks + 8 * g);
            c = *reinterpret_cast<const float4 *>(xrow + 16 * ks + 8 * g + 4);
        }
        xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
        xv[ks][4] = c.x; xv[ks][5] = c.y; xv[ks][6] = c.z; xv[ks][7] = c.w;
    }
    halfx8 xh[8], xl[8];
    const int sx = norm_split(xv, lnw, lnb, g, xh, xl);
    const int arow = sigma32(r32);
    // wait for step t (and free step t - 1's buffer), start step t + 1's copies; this wavefront's slice of step t
    auto next = [&](int t) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (t + 1 < 4) step_copy(t + 1);
        return static_cast<const uint8_t *>(ring + (t & 1) * STEP + hf * SLAB);
    };
    auto mma = [&](floatx16 (&acc)[4], const uint8_t *sl, const halfx8 *bh, const halfx8 *bl, int rows) {
#pragma unroll
        for (int c = 0; c < CPS; c++)
#pragma unroll
            for (int T = 0; T < 4; T++) {
                const int n = 32 * T + arow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(sl + c * 8192 + (g * rows + n) * 16);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(sl + c * 8192 + ((2 + g) * rows + n) * 16);
                acc[T] = mfma16x3(ah, al, bh[c], bl[c], acc[T]);
            }
    };
    floatx16 acc[4], y[4];
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            acc[T][v] = 0.0f;
            y[T][v] = 0.0f;
        }
    // H^T over this wavefront's hidden half: W1's two column halves
#pragma unroll
    for (int t = 0; t < 2; t++) mma(acc, next(t), xh + CPS * t, xl + CPS * t, 128);
    // bias and GELU (hidden unit of accumulator v of tile T: 128 hf + 32 T + 16 (v / 8) + 8 g + v % 8), then the
    // half's split at its own power of two
    const float u1 = ldexpf(1.0f, -(sx + s1));
    float mx = 0.0f;
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float bv[8];
            load8(bias1 + 128 * hf + 32 * T + 16 * hh + 8 * g, bv);
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float hv = gelu(acc[T][8 * hh + t] * u1 + bv[t]);
                acc[T][8 * hh + t] = hv;
                mx = fmaxf(mx, fabsf(hv));
            }
        }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const int sh = shift_for_max(mx);
    halfx8 hh8[8], hl8[8];
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            float hv[8];
#pragma unroll
            for (int t = 0; t < 8; t++) hv[t] = acc[T][8 * hh + t];
            split8(hv, ldexpf(1.0f, sh), hh8[2 * T + hh], hl8[2 * T + hh]);
        }
    // Y^T over this half's hidden units: W2's two K halves of it
#pragma unroll
    for (int t = 2; t < 4; t++) mma(y, next(t), hh8 + CPS * (t - 2), hl8 + CPS * (t - 2), E);
    // the odd wavefront's sums (unscaled) into step 0's buffer (free: every wavefront is past step 2), then the even
    // one finishes: x += y_even + y_odd + b2 (output column of accumulator v of tile T: 32 T + 16 (v / 8) + 8 g + v % 8)
    const float u2 = ldexpf(1.0f, -(sh + s2));
    float *half_sums = reinterpret_cast<float *>(ring) + rg * 32 * HP;  // [32 rows][HP]: this row group's
    if (hf) {
#pragma unroll
        for (int T = 0; T < 4; T++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                float o[8];
#pragma unroll
                for (int t = 0; t < 8; t++) o[t] = y[T][8 * hh + t] * u2;
                float *dst = half_sums + r32 * HP + 32 * T + 16 * hh + 8 * g;
                *reinterpret_cast<float4 *>(dst) = make_float4(o[0], o[1], o[2], o[3]);
                *reinterpret_cast<float4 *>(dst + 4) = make_float4(o[4], o[5], o[6], o[7]);
            }
    }
    __syncthreads();
    if (hf || !live) return;
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int c0 = 32 * T + 16 * hh + 8 * g;
            float rv[8], bv[8], ov[8], xo[8];
            load8(xrow + c0, rv);
            load8(b2 + c0, bv);
            load8(half_sums + r32 * HP + c0, ov);
#pragma unroll
            for (int t = 0; t < 8; t++) xo[t] = ((y[T][8 * hh + t] * u2 + ov[t]) + bv[t]) + rv[t];
            *reinterpret_cast<float4 *>(xrow + c0) = make_float4(xo[0], xo[1], xo[2], xo[3]);
            *reinterpret_cast<float4 *>(xrow + c0 + 4) = make_float4(xo[4], xo[5], xo[6], xo[7]);
        }
}

void ff_block(hipStream_t s, int M, float *x, const DevBlock &b) {
    if (M <= 0) return;
    if (!ff_fused_shape(b.d, b.ff) || !b.l1img || !b.l2img) throw ArgError{"ff_block: no fused weights for this shape"};
    // few rows: the hidden-split kernel while its grid fits the compute units once
    if ((M + 63) / 64 <= 256)
        hipLaunchKernelGGL(k_ff128h, dim3((M + 63) / 64), dim3(256), 0, s, M, x, b.n2w, b.n2b, b.l1img, b.l1b, b.l1s,
                           b.l2img, b.l2b, b.l2s);
    else
        hipLaunchKernelGGL(k_ff128, dim3((M + 32 * FFW - 1) / (32 * FFW)), dim3(64 * FFW), 0, s, M, x, b.n2w, b.n2b,
                           b.l1img, b.l1b, b.l1s, b.l2img, b.l2b, b.l2s);
    TAH_LAUNCHED();
}

// ---- projections of width 128 over many rows ----------------------------------------------------------------------
// Y [M][N] = epi(X' W^T + b), K = 128: the column stage's query projection (with norm1 and the query scale folded
// in), the row stage's query/key/value projection (with norm1) and both stages' output projections (with the
// residual add). Each wavefront owns 32 rows of X, split once (per-row power of two) and kept in registers as the B
// operand; the weights, one block of 128 output columns at a time (64 KB: the same image as the feed-forward's,
// 128-row blocks of 16-column steps), are copied global -> LDS by DMA and shared by the four wavefronts, and each
// block's four 32-column tiles are formed with sigma32-ordered rows so that the epilogue writes eight consecutive
// columns per lane. Two workgroups share a compute unit (2 x 64 KB of LDS). grid (row tiles of 128, column groups):
// with few row tiles the column blocks are dealt out over blockIdx.y (each workgroup then splits its rows for its
// blocks only), so that their weight copies run on different compute units at once rather than one after another.
template <int EPI, bool LN>
__global__ __launch_bounds__(256, 2) void k_rows128(int M, int N, const float *__restrict__ X, int ldx,
                                                     const uint8_t *__restrict__ wimg, int wshift,
                                                     const float *__restrict__ b, float *Y, int ldy,
                                                     const float *R, int ldr, const float *__restrict__ scale,
                                                     const float *__restrict__ lnw, const float *__restrict__ lnb) {
    constexpr int BLK = 65536;  // one block of 128 output columns: 8 steps of 8 KB
    __shared__ __align__(16) uint8_t wl[BLK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int m = blockIdx.x * 128 + wave * 32 + r32;
    const bool live = m < M;
    const int cb0 = blockIdx.y, cbs = gridDim.y;  // this workgroup's column blocks: cb0, cb0 + cbs, ...
    dma_to_lds(wimg + (size_t)cb0 * BLK, wl, BLK, tid);

    float xv[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
        if (live) {
            const float *src = X + (size_t)m * ldx + 16 * ks + 8 * g;
            a = *reinterpret_cast<const float4 *>(src);
            c = *reinterpret_cast<const float4 *>(src + 4);
        }
        xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
        xv[ks][4] = c.x; xv[ks][5] = c.y; xv[ks][6] = c.z; xv[ks][7] = c.w;
    }
    if (LN) {
        float sum = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) sum += xv[ks][t];
        sum += __shfl_xor(sum, 32, 64);
        const float mean = sum / 128.0f;
        float sq = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float dv = xv[ks][t] - mean;
                sq += dv * dv;
            }
        sq += __shfl_xor(sq, 32, 64);
        const float inv = 1.0f / sqrtf(sq / 128.0f + 1e-5f);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const float4 wa = *reinterpret_cast<const float4 *>(lnw + 16 * ks + 8 * g);
            const float4 wb = *reinterpret_cast<const float4 *>(lnw + 16 * ks + 8 * g + 4);
            const float4 ba = *reinterpret_cast<const float4 *>(lnb + 16 * ks + 8 * g);
            const float4 bb = *reinterpret_cast<const float4 *>(lnb + 16 * ks + 8 * g + 4);
            const float wv[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
            const float bv[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
#pragma unroll
            for (int t = 0; t < 8; t++) xv[ks][t] = (xv[ks][t] - mean) * inv * wv[t] + bv[t];
        }
    }
    float xmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
    xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
    const int sx = shift_for_max(xmax);
    halfx8 xh[8], xl[8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) split8(xv[ks], ldexpf(1.0f, sx), xh[ks], xl[ks]);
    const float u = ldexpf(1.0f, -(sx + wshift));
    const int arow = sigma32(r32);

    for (int cb = cb0; cb < N / 128; cb += cbs) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // block cb of the weights is in LDS
        floatx16 acc[4];
#pragma unroll
        for (int T = 0; T < 4; T++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[T][v] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int T = 0; T < 4; T++) {
                const int n = 32 * T + arow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(wl + ks * 8192 + (g * 128 + n) * 16);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(wl + ks * 8192 + ((2 + g) * 128 + n) * 16);
                acc[T] = mfma16x3(ah, al, xh[ks], xl[ks], acc[T]);
            }
        __syncthreads();  // everyone is done with block cb
        if (cb + cbs < N / 128) dma_to_lds(wimg + (size_t)(cb + cbs) * BLK, wl, BLK, tid);
        if (!live) continue;
        // column of accumulator v of tile T: 128 cb + 32 T + 16 (v / 8) + 8 g + v % 8
#pragma unroll
        for (int T = 0; T < 4; T++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int n0 = 128 * cb + 32 * T + 16 * hh + 8 * g;
                const float4 ba = *reinterpret_cast<const float4 *>(b + n0);
                const float4 bb = *reinterpret_cast<const float4 *>(b + n0 + 4);
                const float bv[8] = {ba.x, ba.y, ba.z, ba.w, bb.x, bb.y, bb.z, bb.w};
                float yv[8];
#pragma unroll
                for (int t = 0; t < 8; t++) yv[t] = acc[T][8 * hh + t] * u + bv[t];
                if (EPI == EPI_SCALE) {
                    const float4 sa = *reinterpret_cast<const float4 *>(scale + n0);
                    const float4 sb = *reinterpret_cast<const float4 *>(scale + n0 + 4);
                    yv[0] *= sa.x; yv[1] *= sa.y; yv[2] *= sa.z; yv[3] *= sa.w;
                    yv[4] *= sb.x; yv[5] *= sb.y; yv[6] *= sb.z; yv[7] *= sb.w;
                }
                if (EPI == EPI_RESID) {
                    const float *rp = R + (size_t)m * ldr + n0;
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
}

// ---- fused column block, attention half ---------------------------------------------------------------------------
// x += out(attend(scale * (Wq layer_norm1(x) + bq), K_g, V_g)) + bo for the cells of one group against the group's
// cached inducing keys and values (src/nn.rs:291-301 with src/nn.rs:130-152), for e = 128, 8 heads of 16 and 128
// inducing points, in one pass: the queries and the attention's output never leave the registers.
//
// The group's keys and values are first made into one 16 KB image per (group, head), in the LDS layout the attention
// reads (k_cell_images): keys [dims half][key][8] and V^T [16-key step][8-key half][row][8], hi halves then lo
// halves, scaled by the head's power of two (its largest magnitude below 2^14; the two shifts beside the images).
// V^T's rows are the coordinates with bits 2 and 3 swapped, xor the step's swizzle: O^T's accumulators 0..7 then
// hold coordinates 8 (l / 32) + 0..7 of lane l's cell, the B operand of the output projection's step for the head.
constexpr int CIMG = 16384;  // bytes of one (group, head) image

// grid (groups, 8); 256 threads: thread t takes key t % 128, coordinates 8 (t / 128) + 0..7 of head blockIdx.y.
__global__ __launch_bounds__(256) void k_cell_images(const float *__restrict__ kvbase, size_t gstride,
                                                      uint8_t *__restrict__ images, int *__restrict__ shifts) {
    constexpr int E = 128, INDS = 128;
    __shared__ float red[2][4];
    const int grp = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int key = tid & 127, half = tid >> 7;
    const float *K = kvbase + (size_t)grp * gstride, *V = K + (size_t)E * INDS;
    float kv[8], vv[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
        kv[c] = K[(size_t)(16 * h + 8 * half + c) * INDS + key];
        vv[c] = V[(size_t)(16 * h + 8 * half + c) * INDS + key];
    }
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        mk = fmaxf(mk, fabsf(kv[c]));
        mv = fmaxf(mv, fabsf(vv[c]));
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
    uint8_t *img = images + ((size_t)grp * 8 + h) * CIMG;
    _Float16 *Kh = reinterpret_cast<_Float16 *>(img), *Kl = Kh + 2 * 128 * 8;
    _Float16 *Vh = Kl + 2 * 128 * 8, *Vl = Vh + 8 * 2 * 16 * 8;
    halfx8 h0, l0;
    split8(kv, ldexpf(1.0f, sk), h0, l0);
    *reinterpret_cast<halfx8 *>(Kh + (half * 128 + key) * 8) = h0;
    *reinterpret_cast<halfx8 *>(Kl + (half * 128 + key) * 8) = l0;
    const int st = key >> 4, kg = (key >> 3) & 1, t8 = key & 7;
    const int sw = (2 * st + kg) & 15;
    const float fv = ldexpf(1.0f, sv);
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const int cd = 8 * half + c;
        const int row = ((cd & 3) | ((cd & 4) << 1) | ((cd & 8) >> 1)) ^ sw;
        const float x = vv[c] * fv;
        const _Float16 hi = (_Float16)x;
        Vh[((st * 2 + kg) * 16 + row) * 8 + t8] = hi;
        Vl[((st * 2 + kg) * 16 + row) * 8 + t8] = (_Float16)(x - (float)hi);
    }
    if (tid == 0) {
        shifts[(grp * 8 + h) * 2] = sk;
        shifts[(grp * 8 + h) * 2 + 1] = sv;
    }
}

// The input layer's value of one cell at coordinates c0 .. c0 + 7 (InCells with IN_GROUP values a group; the
// products summed over the group in order, then the bias, as k_input_cells forms them): vals are the cell's group
// values, missing whether all are -100.
constexpr int IN_GROUP = 3;
__device__ __forceinline__ void in_cell_vals(const InCells &ic, int r, int f, float (&vals)[IN_GROUP], bool &missing) {
    missing = true;
    const float *xr = ic.x + (size_t)r * ic.features;
#pragma unroll
    for (int k = 0; k < IN_GROUP; k++) {
        vals[k] = xr[(f + (1 << k)) % ic.features];
        missing = missing && vals[k] == -100.0f;
    }
}
__device__ __forceinline__ void in_cell8(const InCells &ic, const float (&vals)[IN_GROUP], bool missing, int c0,
                                         float (&out)[8]) {
    float wv[8 * IN_GROUP], bv[8];
#pragma unroll
    for (int i = 0; i < 2 * IN_GROUP; i++) {
        const float4 t = *reinterpret_cast<const float4 *>(ic.in_w + (size_t)c0 * IN_GROUP + 4 * i);
        wv[4 * i] = t.x; wv[4 * i + 1] = t.y; wv[4 * i + 2] = t.z; wv[4 * i + 3] = t.w;
    }
    load8(ic.in_b + c0, bv);
#pragma unroll
    for (int t = 0; t < 8; t++) {
        float a = 0.0f;
#pragma unroll
        for (int k = 0; k < IN_GROUP; k++) a += wv[t * IN_GROUP + k] * vals[k];
        out[t] = missing ? -100.0f : a + bv[t];
    }
}

// grid (ceil(n / 128), groups); 256 threads; wavefront w owns cells of rows 128 x + 32 w + 0..31 of group blockIdx.y
// (cell (r, g) at row r sr + g sg of cells), lane l cell l % 32, as the B operand of every product:
//  * query projection H^T = Wq X^T as in k_rows128 (its accumulators hold, for each head, eight consecutive query
//    coordinates 8 (l / 32) + 0..7: the B operand of the head's S^T = K Q^T);
//  * per head, S^T = K Q^T, a softmax over the 128 keys in two halves and O^T = V^T P^T (V^T fills 16 of the 32 A
//    rows; the other lanes read a zero block), then the head's step of the output projection;
//  * LDS (64 KB, two workgroups a compute unit): the query weights (64 KB) first; then the output projection's
//    16-column steps (8 KB each) in four slots, refilled three heads ahead, and two head images, the next one copied
//    in (global_load_lds) while the current one is used: one barrier per head.
// The output projection's input is scaled by one power of two for all heads, lowered (and the sums rescaled) when a
// head's values are larger than all before: every head's output is at most its values' largest magnitude.
// With FF the block's feed-forward half follows in the same kernel (ff128_rows, its weight slices in the same 64 KB
// of LDS): the cells' new values stay in registers as its input; they are written out as well, for its residual add.
// With KV as well the result goes on to the first row block's keys and values (ff128_rows with KV): cell (r, g)'s at
// kn.out + (r sr + g sg) 2 e. With IN the cells' values are the input layer's (in_cell8, from the table rows ic),
// formed again for the residual add, and the cells are only written.
template <bool FF, bool KV, bool IN = false>
__global__ __launch_bounds__(256, 2) void k_cell_block(int n, size_t sr, size_t sg, float *cells,
                                                        const float *__restrict__ n1w, const float *__restrict__ n1b,
                                                        const uint8_t *__restrict__ qimg, int qshift,
                                                        const float *__restrict__ qb, const float *__restrict__ qscale,
                                                        const uint8_t *__restrict__ images, const int *__restrict__ shifts,
                                                        const uint8_t *__restrict__ oimg, int oshift,
                                                        const float *__restrict__ ob, const float *__restrict__ n2w, const float *__restrict__ n2b,
                                                        const uint8_t *__restrict__ w1img, const float *__restrict__ b1,
                                                        int s1, const uint8_t *__restrict__ w2img,
                                                        const float *__restrict__ b2, int s2, KvNext kn,
                                                        InCells ic) {
    static_assert(FF || !KV, "the next block's keys and values come from the feed-forward's registers");
    constexpr int E = 128;
    __shared__ __align__(16) uint8_t lds[65536];
    __shared__ __align__(16) float ffb[FF ? 256 : 4];  // FF: the first feed-forward layer's bias
    __shared__ __align__(16) uint8_t zero[16], ones[16];  // eight fp16 zeros, eight fp16 ones
    __shared__ __align__(16) float qbs[2][128];  // the query bias and scale
    uint8_t *const wo = lds;           // output projection steps, four slots of 8 KB
    uint8_t *const kvl = lds + 32768;  // two head images
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int grp = blockIdx.y;
    const int r = blockIdx.x * 128 + wave * 32 + r32;
    const bool live = r < n;
    const size_t m = (size_t)(live ? r : 0) * sr + (size_t)grp * sg;
    const uint8_t *gimg = images + (size_t)grp * 8 * CIMG;
    const int *gsh = shifts + grp * 16;
    dma_to_lds(qimg, lds, 65536, tid);
    if (tid < 4) reinterpret_cast<uint32_t *>(zero)[tid] = 0u;
    else if (tid < 8) reinterpret_cast<uint32_t *>(ones)[tid - 4] = 0x3c003c00u;
    if (tid < 64)
        reinterpret_cast<float4 *>(&qbs[0][0])[tid] =
            *reinterpret_cast<const float4 *>(tid < 32 ? qb + 4 * tid : qscale + 4 * (tid - 32));

    // this wavefront's cells: layer norm, then split as the B operand (coordinates 16 ks + 8 g + t)
    float xv[8][8];
    if constexpr (IN) {
        float vals[IN_GROUP];
        bool missing;
        in_cell_vals(ic, live ? r : 0, grp, vals, missing);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) in_cell8(ic, vals, missing, 16 * ks + 8 * g, xv[ks]);
    } else {
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
            if (live) {
                const float *src = cells + m * E + 16 * ks + 8 * g;
                a = *reinterpret_cast<const float4 *>(src);
                c = *reinterpret_cast<const float4 *>(src + 4);
            }
            xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
            xv[ks][4] = c.x; xv[ks][5] = c.y; xv[ks][6] = c.z; xv[ks][7] = c.w;
        }
    }
    {
        float sum = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) sum += xv[ks][t];
        sum += __shfl_xor(sum, 32, 64);
        const float mean = sum / 128.0f;
        float sq = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float dv = xv[ks][t] - mean;
                sq += dv * dv;
            }
        sq += __shfl_xor(sq, 32, 64);
        const float inv = 1.0f / sqrtf(sq / 128.0f + 1e-5f);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            float wv[8], bv[8];
            load8(n1w + 16 * ks + 8 * g, wv);
            load8(n1b + 16 * ks + 8 * g, bv);
#pragma unroll
            for (int t = 0; t < 8; t++) xv[ks][t] = (xv[ks][t] - mean) * inv * wv[t] + bv[t];
        }
    }
    float xmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
    xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
    const int sx = shift_for_max(xmax);
    const int arow = sigma32(r32);

    // query projection: accumulator v of tile T holds column 32 T + 16 (v / 8) + 8 g + v % 8, i.e. head 2 T + v / 8,
    // coordinate 8 g + v % 8
    floatx16 qa[4];
    {
        halfx8 xh[8], xl[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++) split8(xv[ks], ldexpf(1.0f, sx), xh[ks], xl[ks]);
#pragma unroll
        for (int T = 0; T < 4; T++)
#pragma unroll
            for (int v = 0; v < 16; v++) qa[T][v] = 0.0f;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // the query weights are in LDS
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int T = 0; T < 4; T++) {
                const int nn = 32 * T + arow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(lds + ks * 8192 + (g * 128 + nn) * 16);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(lds + ks * 8192 + ((2 + g) * 128 + nn) * 16);
                qa[T] = mfma16x3(ah, al, xh[ks], xl[ks], qa[T]);
            }
        __builtin_amdgcn_sched_barrier(0);  // the epilogue's loads stay after the products (registers)
        const float u = ldexpf(1.0f, -(sx + qshift));
#pragma unroll
        for (int T = 0; T < 4; T++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int n0 = 32 * T + 16 * hh + 8 * g;
                float bv[8], cv[8];
                load8(&qbs[0][n0], bv);
                load8(&qbs[1][n0], cv);
#pragma unroll
                for (int t = 0; t < 8; t++) qa[T][8 * hh + t] = (qa[T][8 * hh + t] * u + bv[t]) * cv[t];
            }
#pragma unroll
        for (int T = 0; T < 4; T++) asm volatile("" : "+v"(qa[T]));  // finished here, not at each head's first use
    }
    __syncthreads();  // everyone is done with the query weights
    dma_to_lds(oimg, wo, 32768, tid);  // output projection steps 0..3 (heads 0..3)
    dma_to_lds(gimg, kvl, CIMG, tid);  // head 0

    floatx16 acc[4];
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[T][v] = 0.0f;
    int so = 1 << 30;  // the output projection's input scale (log2), lowered as heads need
#pragma unroll
    for (int h = 0; h < 8; h++) {
        const int par = h & 1;
        // lane-dependent offsets recomputed per head (an opaque copy of the lane index): kept live across all eight
        // heads they would take the registers the products need
        int hl = lane;
        asm volatile("" : "+v"(hl));
        const int r32 = hl & 31, g = hl >> 5, krow = sigma32(r32), arow = krow;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // head h's image and step h of the output weights have landed; head h - 1 is done
        if (h + 1 < 8) dma_to_lds(gimg + (size_t)(h + 1) * CIMG, kvl + (par ^ 1) * CIMG, CIMG, tid);
        if (h >= 1 && h + 3 < 8) dma_to_lds(oimg + (size_t)(h + 3) * 8192, wo + ((h + 3) & 3) * 8192, 8192, tid);
        const int sk = gsh[2 * h], sv = gsh[2 * h + 1];
        const _Float16 *Kh = reinterpret_cast<const _Float16 *>(kvl + par * CIMG), *Kl = Kh + 2 * 128 * 8;
        const _Float16 *Vh = Kl + 2 * 128 * 8, *Vl = Vh + 8 * 2 * 16 * 8;
        // this head's query coordinates 8 g + t
        float qv[8];
#pragma unroll
        for (int t = 0; t < 8; t++) qv[t] = qa[h >> 1][8 * (h & 1) + t];
        float qmax = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) qmax = fmaxf(qmax, fabsf(qv[t]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
        const int sq = shift_for_max(qmax);
        halfx8 qh, ql;
        split8(qv, ldexpf(1.0f, sq), qh, ql);
        const float to_log2 = ldexpf(LOG2E, -(sk + sq));
        // two halves of 64 keys, the softmax against a reference maximum raised only when a half passes it by more
        // than 3 (weights exp2(t - ref + 12) below 2^15)
        float ref = -INFINITY;
        floatx16 o;
#pragma unroll
        for (int v = 0; v < 16; v++) o[v] = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
            floatx16 sc[2];
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 2; j++) {
#pragma unroll
                for (int v = 0; v < 16; v++) sc[j][v] = 0.0f;
                const int key = 64 * k2 + 32 * j + krow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(Kh + (g * 128 + key) * 8);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(Kl + (g * 128 + key) * 8);
                sc[j] = mfma16x3(ah, al, qh, ql, sc[j]);
#pragma unroll
                for (int v = 0; v < 16; v++) mx = fmaxf(mx, sc[j][v]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * to_log2;
            const bool grow = mx > ref + 3.0f;
            if (__any(grow)) {
                const float nref = grow ? mx : ref;
                const float alpha = exp2_hw(ref - nref);
                o *= alpha;
                ref = nref;
            }
            const float off = 12.0f - ref;
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    float p[8];
#pragma unroll
                    for (int t = 0; t < 8; t++) p[t] = exp2_hw(fmaf(sc[j][8 * hh + t], to_log2, off));
                    halfx8 ph, pl;
                    split8(p, 1.0f, ph, pl);
                    // 16-key step st (keys 16 st + 8 g + 0..7 of this lane's weights). A rows 16 and 20 are ones (hi)
                    // and zeros (lo), the other rows past 15 zeros: accumulator 8 of every lane sums the weights
                    const int st = 4 * k2 + 2 * j + hh;
                    const int row = r32 ^ ((2 * st + g) & 15);
                    const uint8_t *pad = (r32 & 11) == 0 ? ones : zero;
                    const _Float16 *vh = r32 < 16 ? Vh + ((st * 2 + g) * 16 + row) * 8
                                                   : reinterpret_cast<const _Float16 *>(pad);
                    const _Float16 *vl = r32 < 16 ? Vl + ((st * 2 + g) * 16 + row) * 8
                                                   : reinterpret_cast<const _Float16 *>(zero);
                    o = mfma16x3(*reinterpret_cast<const halfx8 *>(vh), *reinterpret_cast<const halfx8 *>(vl), ph, pl,
                                 o);
                }
        }
        const float l = o[8];  // the weights' sum (row 16 + 4 g of O^T)
        // accumulators 0..7: this cell's coordinates 8 g + 0..7 of the head, in units of 2^sv; |o / l| < 2^(14 - sv)
        if (sv < so) {
            if (so != (1 << 30)) {
                const float rs = ldexpf(1.0f, sv - so);
#pragma unroll
                for (int T = 0; T < 4; T++) acc[T] *= rs;
            }
            so = sv;
        }
        float ov[8];
        const float f = ldexpf(1.0f, so - sv) / l;
#pragma unroll
        for (int t = 0; t < 8; t++) ov[t] = o[t] * f;
        halfx8 oh, ol;
        split8(ov, 1.0f, oh, ol);
        const uint8_t *ws = wo + (h & 3) * 8192;
#pragma unroll
        for (int T = 0; T < 4; T++) {
            const int nn = 32 * T + arow;
            const halfx8 ah = *reinterpret_cast<const halfx8 *>(ws + (g * 128 + nn) * 16);
            const halfx8 al = *reinterpret_cast<const halfx8 *>(ws + ((2 + g) * 128 + nn) * 16);
            acc[T] = mfma16x3(ah, al, oh, ol, acc[T]);
        }
    }
    if (!FF && !live) return;
    // column of accumulator v of tile T: 32 T + 16 (v / 8) + 8 g + v % 8
    const float u = ldexpf(1.0f, -(so + oshift));
    float *xrow = cells + m * E;
    float xn[8][8];  // the new values as the feed-forward's input: columns 16 ks + 8 g + t
    float ivals[IN_GROUP];  // IN: the cell's group values again
    bool imiss = false;
    if constexpr (IN) in_cell_vals(ic, live ? r : 0, grp, ivals, imiss);
#pragma unroll
    for (int T = 0; T < 4; T++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int n0 = 32 * T + 16 * hh + 8 * g;
            float bv[8], xr[8];
            load8(ob + n0, bv);
            if constexpr (IN)
                in_cell8(ic, ivals, imiss, n0, xr);
            else
                load8(xrow + n0, xr);
#pragma unroll
            for (int t = 0; t < 8; t++) xn[2 * T + hh][t] = xr[t] + acc[T][8 * hh + t] * u + bv[t];
            if (live) {
                *reinterpret_cast<float4 *>(xrow + n0) = make_float4(xn[2 * T + hh][0], xn[2 * T + hh][1],
                                                                     xn[2 * T + hh][2], xn[2 * T + hh][3]);
                *reinterpret_cast<float4 *>(xrow + n0 + 4) = make_float4(xn[2 * T + hh][4], xn[2 * T + hh][5],
                                                                         xn[2 * T + hh][6], xn[2 * T + hh][7]);
            }
        }
    if constexpr (FF) {
        __syncthreads();  // every wavefront is done with the attention's LDS (no copy is in flight after head 7)
        ff128_start(lds, ffb, w1img, b1, tid);
        if constexpr (KV) {
            kn.out += m * 2 * E;
            ff128_rows<true>(xn, live, xrow, lds, ffb, n2w, n2b, w1img, s1, w2img, b2, s2, tid, kn);
        } else {
            ff128_rows(xn, live, xrow, lds, ffb, n2w, n2b, w1img, s1, w2img, b2, s2, tid);
        }
    }
}

// ---- fused row block, attention half ------------------------------------------------------------------------------
// x += out(attend(rope(Wq layer_norm1(x) + bq) / 4, rope(K), V)) + bo for every token of one row over all the row's
// tokens (src/nn.rs:357-419, Rope src/nn.rs:304-321), for e = 128, 8 heads of 16 and T <= 128 tokens; the keys and
// values [T][2 e] (k then v per token, without rotation) come from a projection before it.
// grid n rows; 256 threads; wavefront w owns tokens 32 w + 0..31 of row blockIdx.x, lane l token l % 32, as the B
// operand of every product (as in k_cell_block):
//  * the query projection as in k_cell_block, its accumulators rotated in registers (a coordinate's partner for the
//    rotation sits on lane l ^ 32) and scaled by 1 / sqrt(16);
//  * per head the workgroup stages the row's keys (rotated) and values into LDS split into fp16 halves, scaled by the
//    head's power of two (one wavefront-pair's maximum each, across wavefronts through LDS): threads 0..127 a key
//    each, threads 128..255 a value each, for the next head while the current one is attended (two barriers a head);
//  * keys past T are masked; the attention and the output projection then run as in k_cell_block.
// With FF the block's feed-forward half follows in the same kernel, as in k_cell_block; with KV as well the next
// row block's keys and values (kn.out [n][T][2 e], which may be kv itself: a workgroup reads only its own row's keys
// and values, all of them before its feed-forward half starts).
template <bool FF, bool KV>
__global__ __launch_bounds__(256, 2) void k_row_block(int T, int keep, float *tok, const float *kv,
                                                       const float *__restrict__ cosv, const float *__restrict__ sinv,
                                                       const float *__restrict__ n1w, const float *__restrict__ n1b,
                                                       const uint8_t *__restrict__ qimg, int qshift,
                                                       const float *__restrict__ qb, const uint8_t *__restrict__ oimg,
                                                       int oshift, const float *__restrict__ ob, const float *__restrict__ n2w, const float *__restrict__ n2b,
                                                       const uint8_t *__restrict__ w1img, const float *__restrict__ b1,
                                                       int s1, const uint8_t *__restrict__ w2img,
                                                       const float *__restrict__ b2, int s2, KvNext kn) {
    static_assert(FF || !KV, "the next block's keys and values come from the feed-forward's registers");
    constexpr int E = 128;
    __shared__ __align__(16) uint8_t lds[65536];
    __shared__ __align__(16) float ffb[FF ? 256 : 4];  // FF: the first feed-forward layer's bias
    __shared__ __align__(16) uint8_t zero[16], ones[16];
    __shared__ __align__(16) float qbs[128];
    __shared__ __align__(16) float cst[2][128][8];  // cos, sin of token t, pair k
    __shared__ float red[2][2][2];                  // [head parity][keys, values][wavefront of the pair]
    __shared__ int shs[2][2];                       // [buffer][keys, values]: the staged head's scales
    uint8_t *const wo = lds;
    uint8_t *const kvl = lds + 32768;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, g = lane >> 5;
    const int row = blockIdx.x;
    const int tk = wave * 32 + r32;  // this lane's token
    const bool live = tk < T;
    float *xrow = tok + ((size_t)row * T + (live ? tk : 0)) * E;
    const float *kvrow = kv + (size_t)row * T * 2 * E;
    dma_to_lds(qimg, lds, 65536, tid);
    if (tid < 4) reinterpret_cast<uint32_t *>(zero)[tid] = 0u;
    else if (tid < 8) reinterpret_cast<uint32_t *>(ones)[tid - 4] = 0x3c003c00u;
    if (tid < 32) reinterpret_cast<float4 *>(qbs)[tid] = *reinterpret_cast<const float4 *>(qb + 4 * tid);
    if (tid < T) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            cst[0][tid][k] = cosv[tid * 8 + k];
            cst[1][tid][k] = sinv[tid * 8 + k];
        }
    }

    // staging of head h: thread t < 128 takes key t (16 coordinates, rotated), thread 128 + t value t
    const int st_tok = tid & 127;
    const bool st_key = tid < 128, st_live = st_tok < T;
    float stv[16];
    auto stage_load = [&](int h, int par) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (st_live) a = *reinterpret_cast<const float4 *>(kvrow + (size_t)st_tok * 2 * E + (st_key ? 0 : E) + 16 * h + 4 * i);
            stv[4 * i] = a.x; stv[4 * i + 1] = a.y; stv[4 * i + 2] = a.z; stv[4 * i + 3] = a.w;
        }
        float mx = 0.0f;
#pragma unroll
        for (int c = 0; c < 16; c++) mx = fmaxf(mx, fabsf(stv[c]));
        mx = wave_max(mx);
        if (lane == 0) red[par][wave >> 1][wave & 1] = mx;
    };
    auto stage_store = [&](int par) {
        // the keys' maximum is over the unrotated values: rotation keeps each pair's norm, so the rotated values stay
        // within sqrt(2) of it, and the split's scale (a maximum below 2^14) leaves that room
        const int s = shift_for_max(fmaxf(red[par][st_key ? 0 : 1][0], red[par][st_key ? 0 : 1][1]) * 1.5f);
        const float f = ldexpf(1.0f, s);
        if (st_tok == 0) shs[par][st_key ? 0 : 1] = s;
        _Float16 *Kh = reinterpret_cast<_Float16 *>(kvl + par * 16384), *Kl = Kh + 2 * 128 * 8;
        _Float16 *Vh = Kl + 2 * 128 * 8, *Vl = Vh + 8 * 2 * 16 * 8;
        if (st_key) {
            float rk[16];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float c = cst[0][st_tok][k], sn = cst[1][st_tok][k];
                rk[k] = stv[k] * c - stv[k + 8] * sn;
                rk[k + 8] = stv[k + 8] * c + stv[k] * sn;
            }
            halfx8 h0, l0, h1, l1;
            split8(rk, f, h0, l0);
            split8(rk + 8, f, h1, l1);
            *reinterpret_cast<halfx8 *>(Kh + st_tok * 8) = h0;
            *reinterpret_cast<halfx8 *>(Kl + st_tok * 8) = l0;
            *reinterpret_cast<halfx8 *>(Kh + (128 + st_tok) * 8) = h1;
            *reinterpret_cast<halfx8 *>(Kl + (128 + st_tok) * 8) = l1;
        } else {
            const int st = st_tok >> 4, kg = (st_tok >> 3) & 1, t8 = st_tok & 7;
            const int sw = (2 * st + kg) & 15;
#pragma unroll
            for (int cd = 0; cd < 16; cd++) {
                const int rw = ((cd & 3) | ((cd & 4) << 1) | ((cd & 8) >> 1)) ^ sw;
                const float x = stv[cd] * f;
                const _Float16 hi = (_Float16)x;
                Vh[((st * 2 + kg) * 16 + rw) * 8 + t8] = hi;
                Vl[((st * 2 + kg) * 16 + rw) * 8 + t8] = (_Float16)(x - (float)hi);
            }
        }
        return s;
    };
    stage_load(0, 0);

    // this wavefront's tokens: layer norm, then split as the B operand (coordinates 16 ks + 8 g + t)
    float xv[8][8];
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), c = a;
        if (live) {
            a = *reinterpret_cast<const float4 *>(xrow + 16 * ks + 8 * g);
            c = *reinterpret_cast<const float4 *>(xrow + 16 * ks + 8 * g + 4);
        }
        xv[ks][0] = a.x; xv[ks][1] = a.y; xv[ks][2] = a.z; xv[ks][3] = a.w;
        xv[ks][4] = c.x; xv[ks][5] = c.y; xv[ks][6] = c.z; xv[ks][7] = c.w;
    }
    {
        float sum = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) sum += xv[ks][t];
        sum += __shfl_xor(sum, 32, 64);
        const float mean = sum / 128.0f;
        float sq = 0.0f;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int t = 0; t < 8; t++) {
                const float dv = xv[ks][t] - mean;
                sq += dv * dv;
            }
        sq += __shfl_xor(sq, 32, 64);
        const float inv = 1.0f / sqrtf(sq / 128.0f + 1e-5f);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            float wv[8], bv[8];
            load8(n1w + 16 * ks + 8 * g, wv);
            load8(n1b + 16 * ks + 8 * g, bv);
#pragma unroll
            for (int t = 0; t < 8; t++) xv[ks][t] = (xv[ks][t] - mean) * inv * wv[t] + bv[t];
        }
    }
    float xmax = 0.0f;
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int t = 0; t < 8; t++) xmax = fmaxf(xmax, fabsf(xv[ks][t]));
    xmax = fmaxf(xmax, __shfl_xor(xmax, 32, 64));
    const int sx = shift_for_max(xmax);

    // query projection (accumulator v of tile T: head 2 T + v / 8, coordinate 8 g + v % 8), bias, rotation, 1 / 4
    floatx16 qa[4];
    {
        const int arow = sigma32(r32);
        halfx8 xh[8], xl[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++) split8(xv[ks], ldexpf(1.0f, sx), xh[ks], xl[ks]);
#pragma unroll
        for (int T4 = 0; T4 < 4; T4++)
#pragma unroll
            for (int v = 0; v < 16; v++) qa[T4][v] = 0.0f;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // the query weights, bias and rotation tables are in LDS; the first head's maxima in red
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
#pragma unroll
            for (int T4 = 0; T4 < 4; T4++) {
                const int nn = 32 * T4 + arow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(lds + ks * 8192 + (g * 128 + nn) * 16);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(lds + ks * 8192 + ((2 + g) * 128 + nn) * 16);
                qa[T4] = mfma16x3(ah, al, xh[ks], xl[ks], qa[T4]);
            }
        __builtin_amdgcn_sched_barrier(0);
        const float u = ldexpf(1.0f, -(sx + qshift));
        const int ct = live ? tk : 0;
        float cs[8], sn[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            cs[k] = cst[0][ct][k];
            sn[k] = cst[1][ct][k];
        }
        const float sgn = g == 0 ? -1.0f : 1.0f;
#pragma unroll
        for (int T4 = 0; T4 < 4; T4++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                float bv[8];
                load8(qbs + 32 * T4 + 16 * hh + 8 * g, bv);
#pragma unroll
                for (int t = 0; t < 8; t++) {
                    const float qv = qa[T4][8 * hh + t] * u + bv[t];
                    const auto sw2 = __builtin_amdgcn_permlane32_swap(__float_as_uint(qv), __float_as_uint(qv), false, false);
                    const float other = __uint_as_float(g ? sw2[0] : sw2[1]);  // the coordinate 8 away, lane l ^ 32
                    qa[T4][8 * hh + t] = (qv * cs[t] + sgn * other * sn[t]) * 0.25f;
                }
            }
#pragma unroll
        for (int T4 = 0; T4 < 4; T4++) asm volatile("" : "+v"(qa[T4]));
    }
    __syncthreads();  // everyone is done with the query weights
    dma_to_lds(oimg, wo, 32768, tid);
    stage_store(0);
    stage_load(1, 1);

    floatx16 acc[4];
#pragma unroll
    for (int T4 = 0; T4 < 4; T4++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[T4][v] = 0.0f;
    int so = 1 << 30;
#pragma unroll
    for (int h = 0; h < 8; h++) {
        const int par = h & 1;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // head h's keys and values are staged, head h + 1's maxima are in red; step h of the output
                          // weights has landed; everyone is done with head h - 1 and its buffer
        if (h >= 1 && h + 3 < 8) dma_to_lds(oimg + (size_t)(h + 3) * 8192, wo + ((h + 3) & 3) * 8192, 8192, tid);
        // one head ahead: head h + 1 into the buffer head h - 1 used, then head h + 2's values into registers
        if (h + 1 < 8) stage_store(par ^ 1);
        if (h + 2 < 8) stage_load(h + 2, par);
        const int skh = shs[par][0], svh = shs[par][1];
        int hl = lane;
        asm volatile("" : "+v"(hl));
        const int r32h = hl & 31, gh = hl >> 5, krow = sigma32(r32h), arow = krow;
        const _Float16 *Kh = reinterpret_cast<const _Float16 *>(kvl + par * 16384), *Kl = Kh + 2 * 128 * 8;
        const _Float16 *Vh = Kl + 2 * 128 * 8, *Vl = Vh + 8 * 2 * 16 * 8;
        // this head's query coordinates: tile 0 holds heads h and h + 1 of an even h (the tiles shift down by one
        // after every second head, so that no register is indexed by the head)
        float qv[8];
#pragma unroll
        for (int t = 0; t < 8; t++) qv[t] = par ? qa[0][8 + t] : qa[0][t];
        float qmax = 0.0f;
#pragma unroll
        for (int t = 0; t < 8; t++) qmax = fmaxf(qmax, fabsf(qv[t]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
        const int sq = shift_for_max(qmax);
        halfx8 qh, ql;
        split8(qv, ldexpf(1.0f, sq), qh, ql);
        const float to_log2 = ldexpf(LOG2E, -(skh + sq));
        float ref = -INFINITY;
        floatx16 o;
#pragma unroll
        for (int v = 0; v < 16; v++) o[v] = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < 2; k2++) {
            floatx16 sc[2];
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < 2; j++) {
#pragma unroll
                for (int v = 0; v < 16; v++) sc[j][v] = 0.0f;
                const int key = 64 * k2 + 32 * j + krow;
                const halfx8 ah = *reinterpret_cast<const halfx8 *>(Kh + (gh * 128 + key) * 8);
                const halfx8 al = *reinterpret_cast<const halfx8 *>(Kl + (gh * 128 + key) * 8);
                sc[j] = mfma16x3(ah, al, qh, ql, sc[j]);
                // accumulator v holds key 64 k2 + 32 j + 16 (v / 8) + 8 g + v % 8
                const int lim = T - (64 * k2 + 32 * j) - 8 * gh;
                if (lim < 32) {
#pragma unroll
                    for (int v = 0; v < 16; v++)
                        if (16 * (v >> 3) + (v & 7) >= lim) sc[j][v] = -INFINITY;
                }
#pragma unroll
                for (int v = 0; v < 16; v++) mx = fmaxf(mx, sc[j][v]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64)) * to_log2;
            const bool grow = mx > ref + 3.0f;
            if (__any(grow)) {
                const float nref = grow ? mx : ref;
                const float alpha = exp2_hw(ref - nref);
                o *= alpha;
                ref = nref;
            }
            const float off = 12.0f - ref;
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const int st = 4 * k2 + 2 * j + hh;
                    if (16 * st >= T) continue;  // keys 16 st .. 16 st + 15 all past the row's tokens: weights 0
                    float p[8];
#pragma unroll
                    for (int t = 0; t < 8; t++) p[t] = exp2_hw(fmaf(sc[j][8 * hh + t], to_log2, off));
                    halfx8 ph, pl;
                    split8(p, 1.0f, ph, pl);
                    const int rw = r32h ^ ((2 * st + gh) & 15);
                    const uint8_t *pad = (r32h & 11) == 0 ? ones : zero;
                    const _Float16 *vh = r32h < 16 ? Vh + ((st * 2 + gh) * 16 + rw) * 8
                                                    : reinterpret_cast<const _Float16 *>(pad);
                    const _Float16 *vl = r32h < 16 ? Vl + ((st * 2 + gh) * 16 + rw) * 8
                                                    : reinterpret_cast<const _Float16 *>(zero);
                    o = mfma16x3(*reinterpret_cast<const halfx8 *>(vh), *reinterpret_cast<const halfx8 *>(vl), ph, pl,
                                 o);
                }
        }
        const float l = o[8];
        if (svh < so) {
            if (so != (1 << 30)) {
                const float rs = ldexpf(1.0f, svh - so);
#pragma unroll
                for (int T4 = 0; T4 < 4; T4++) acc[T4] *= rs;
            }
            so = svh;
        }
        float ov[8];
        const float f = ldexpf(1.0f, so - svh) / l;
#pragma unroll
        for (int t = 0; t < 8; t++) ov[t] = o[t] * f;
        halfx8 oh, ol;
        split8(ov, 1.0f, oh, ol);
        const uint8_t *ws = wo + (h & 3) * 8192;
#pragma unroll
        for (int T4 = 0; T4 < 4; T4++) {
            const int nn = 32 * T4 + arow;
            const halfx8 ah = *reinterpret_cast<const halfx8 *>(ws + (gh * 128 + nn) * 16);
            const halfx8 al = *reinterpret_cast<const halfx8 *>(ws + ((2 + gh) * 128 + nn) * 16);
            acc[T4] = mfma16x3(ah, al, oh, ol, acc[T4]);
        }
        if (par) {
            qa[0] = qa[1];
            qa[1] = qa[2];
            qa[2] = qa[3];
        }
    }
    if (!FF && !live) return;
    const float u = ldexpf(1.0f, -(so + oshift));
    float xn[8][8];  // the new values as the feed-forward's input: columns 16 ks + 8 g + t
#pragma unroll
    for (int T4 = 0; T4 < 4; T4++)
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int n0 = 32 * T4 + 16 * hh + 8 * g;
            float bv[8], xr[8];
            load8(ob + n0, bv);
            load8(xrow + n0, xr);
#pragma unroll
            for (int t = 0; t < 8; t++) xn[2 * T4 + hh][t] = xr[t] + acc[T4][8 * hh + t] * u + bv[t];
            if (live) {
                *reinterpret_cast<float4 *>(xrow + n0) = make_float4(xn[2 * T4 + hh][0], xn[2 * T4 + hh][1],
                                                                     xn[2 * T4 + hh][2], xn[2 * T4 + hh][3]);
                *reinterpret_cast<float4 *>(xrow + n0 + 4) = make_float4(xn[2 * T4 + hh][4], xn[2 * T4 + hh][5],
                                                                         xn[2 * T4 + hh][6], xn[2 * T4 + hh][7]);
            }
        }
    if constexpr (FF) {
        __syncthreads();  // every wavefront is done with the attention's LDS (no copy is in flight after head 7)
        ff128_start(lds, ffb, w1img, b1, tid);
        if constexpr (KV) {
            kn.out += ((size_t)row * T + (live ? tk : 0)) * 2 * E;
            ff128_rows<true>(xn, live, xrow, lds, ffb, n2w, n2b, w1img, s1, w2img, b2, s2, tid, kn, tk < keep);
        } else {
            ff128_rows(xn, live, xrow, lds, ffb, n2w, n2b, w1img, s1, w2img, b2, s2, tid);
        }
    }
}

bool row_block_fits(const DevBlock &b, int T) {
    return b.d == 128 && b.heads == 8 && b.inimg && b.outimg && T >= 1 && T <= 128;
}

bool block_ff_fits(const DevBlock &b) { return ff_fused_shape(b.d, b.ff) && b.l1img && b.l2img; }

bool row_kv_fits(const DevBlock &next) { return next.d == 128 && next.inimg && next.in_b && next.n1w && next.n1b; }

void row_block(hipStream_t s, int n, int T, float *tok, const float *kv, const float *cosv, const float *sinv,
               const DevBlock &b, bool ff, const DevBlock *next, float *kv_next, int keep) {
    if (n <= 0) return;
    if (!row_block_fits(b, T) || (reinterpret_cast<uintptr_t>(tok) & 15) || (reinterpret_cast<uintptr_t>(kv) & 15))
        throw ArgError{"row_block: needs e = 128, 8 heads, weight images, at most 128 tokens and aligned rows"};
    if (ff && !block_ff_fits(b)) throw ArgError{"row_block: no fused feed-forward weights for this shape"};
    if (next && (!ff || !row_kv_fits(*next) || !kv_next || (reinterpret_cast<uintptr_t>(kv_next) & 15)))
        throw ArgError{"row_block: the next block's keys and values need the fused feed-forward, e = 128, its "
                       "projection image and an aligned destination"};
    if (keep < 0) keep = T;
    if (keep > T || (keep < T && !next))
        throw ArgError{"row_block: only a block that forms the next one's keys and values may leave tokens unwritten"};
    if (next) {
        const KvNext kn{next->inimg + (size_t)128 * 128 * 4, next->ins, next->n1w, next->n1b, next->in_b + 128,
                        kv_next};
        hipLaunchKernelGGL((k_row_block<true, true>), dim3(n), dim3(256), 0, s, T, keep, tok, kv, cosv, sinv, b.n1w, b.n1b,
                           b.inimg, b.ins, b.in_b, b.outimg, b.outs, b.out_b, b.n2w, b.n2b, b.l1img, b.l1b, b.l1s,
                           b.l2img, b.l2b, b.l2s, kn);
    } else if (ff) {
        hipLaunchKernelGGL((k_row_block<true, false>), dim3(n), dim3(256), 0, s, T, T, tok, kv, cosv, sinv, b.n1w, b.n1b,
                           b.inimg, b.ins, b.in_b, b.outimg, b.outs, b.out_b, b.n2w, b.n2b, b.l1img, b.l1b, b.l1s,
                           b.l2img, b.l2b, b.l2s, KvNext{});
    } else {
        hipLaunchKernelGGL((k_row_block<false, false>), dim3(n), dim3(256), 0, s, T, T, tok, kv, cosv, sinv, b.n1w,
                           b.n1b, b.inimg, b.ins, b.in_b, b.outimg, b.outs, b.out_b, nullptr, nullptr, nullptr,
                           nullptr, 0, nullptr, nullptr, 0, KvNext{});
    }
    TAH_LAUNCHED();
}

bool cell_block_fits(const DevBlock &b) {
    return b.d == 128 && b.heads == 8 && b.ss_hidden == 0 && b.inimg && b.outimg;
}

int in_cells_group() { return IN_GROUP; }

size_t cell_block_work_bytes(int groups) { return (size_t)groups * 8 * (CIMG + 2 * sizeof(int)); }

void cell_images(hipStream_t s, int groups, const float *kvbase, size_t gstride, void *work) {
    if (groups <= 0) return;
    if (reinterpret_cast<uintptr_t>(work) & 15) throw ArgError{"cell_images: the work buffer must be 16-byte aligned"};
    uint8_t *images = static_cast<uint8_t *>(work);
    int *shifts = reinterpret_cast<int *>(images + (size_t)groups * 8 * CIMG);
    hipLaunchKernelGGL(k_cell_images, dim3(groups, 8), dim3(256), 0, s, kvbase, gstride, images, shifts);
    TAH_LAUNCHED();
}

void cell_block(hipStream_t s, int n, int groups, size_t sr, size_t sg, float *cells, const DevBlock &b,
                const float *qscale, const float *kvbase, size_t gstride, void *work, bool ff, const DevBlock *next,
                float *kv_next, bool images_ready, const InCells *in) {
    if (n <= 0 || groups <= 0) return;
    if (in && (!ff || next || !in->x || !in->in_w || !in->in_b || in->features != groups ||
               in->group != IN_GROUP || b.d != 128 || (reinterpret_cast<uintptr_t>(in->in_w) & 15) ||
               (reinterpret_cast<uintptr_t>(in->in_b) & 15)))
        throw ArgError{"cell_block: the input layer goes into the first block only, with its feed-forward half, "
                       "three values a group, e = 128, one group a feature and aligned weights"};
    if (!cell_block_fits(b) || (reinterpret_cast<uintptr_t>(cells) & 15) || (reinterpret_cast<uintptr_t>(work) & 15))
        throw ArgError{"cell_block: needs e = 128, 8 heads, weight images and 16-byte aligned cells and work"};
    if (ff && !block_ff_fits(b)) throw ArgError{"cell_block: no fused feed-forward weights for this shape"};
    if (next && (!ff || !row_kv_fits(*next) || !kv_next || (reinterpret_cast<uintptr_t>(kv_next) & 15)))
        throw ArgError{"cell_block: the row block's keys and values need the fused feed-forward, e = 128, its "
                       "projection image and an aligned destination"};
    uint8_t *images = static_cast<uint8_t *>(work);
    int *shifts = reinterpret_cast<int *>(images + (size_t)groups * 8 * CIMG);
    if (!images_ready) cell_images(s, groups, kvbase, gstride, work);
    const dim3 grid((n + 127) / 128, groups);
    if (next) {
        const KvNext kn{next->inimg + (size_t)128 * 128 * 4, next->ins, next->n1w, next->n1b, next->in_b + 128,
                        kv_next};
        hipLaunchKernelGGL((k_cell_block<true, true>), grid, dim3(256), 0, s, n, sr, sg, cells, b.n1w, b.n1b, b.inimg,
                           b.ins, b.in_b, qscale, images, shifts, b.outimg, b.outs, b.out_b, b.n2w, b.n2b, b.l1img,
                           b.l1b, b.l1s, b.l2img, b.l2b, b.l2s, kn, InCells{});
    } else if (ff && in) {
        hipLaunchKernelGGL((k_cell_block<true, false, true>), grid, dim3(256), 0, s, n, sr, sg, cells, b.n1w, b.n1b,
                           b.inimg, b.ins, b.in_b, qscale, images, shifts, b.outimg, b.outs, b.out_b, b.n2w, b.n2b,
                           b.l1img, b.l1b, b.l1s, b.l2img, b.l2b, b.l2s, KvNext{}, *in);
    } else if (ff) {
        hipLaunchKernelGGL((k_cell_block<true, false>), grid, dim3(256), 0, s, n, sr, sg, cells, b.n1w, b.n1b, b.inimg,
                           b.ins, b.in_b, qscale, images, shifts, b.outimg, b.outs, b.out_b, b.n2w, b.n2b, b.l1img,
                           b.l1b, b.l1s, b.l2img, b.l2b, b.l2s, KvNext{}, InCells{});
    } else {
        hipLaunchKernelGGL((k_cell_block<false, false>), grid, dim3(256), 0, s, n, sr, sg, cells, b.n1w, b.n1b,
                           b.inimg, b.ins, b.in_b, qscale, images, shifts, b.outimg, b.outs, b.out_b, nullptr, nullptr,
                           nullptr, nullptr, 0, nullptr, nullptr, 0, KvNext{}, InCells{});
    }
    TAH_LAUNCHED();
}

void rows128(hipStream_t s, int M, int N, const float *X, int ldx, const uint8_t *wimg, int wshift, const float *b,
             float *Y, int ldy, Epi epi, const float *R, int ldr, const float *scale, const float *lnw,
             const float *lnb) {
    if (M <= 0) return;
    if (!wimg || N <= 0 || N % 128 || ldx % 4 || ldy % 4 || (reinterpret_cast<uintptr_t>(X) & 15) ||
        (reinterpret_cast<uintptr_t>(Y) & 15))
        throw ArgError{"rows128: needs a weight image, output width a multiple of 128 and 16-byte aligned rows"};
    // column blocks over workgroups while that fills the compute units at most twice over (two workgroups a unit),
    // and only where the output does not overlap the input (a workgroup's rows are read once, before any block)
    const int tiles = (M + 127) / 128, blocks = N / 128;
    const char *xb = reinterpret_cast<const char *>(X), *yb = reinterpret_cast<const char *>(Y);
    const bool apart = yb >= xb + ((size_t)(M - 1) * ldx + 128) * sizeof(float) ||
                       xb >= yb + ((size_t)(M - 1) * ldy + N) * sizeof(float);
    const dim3 grid(tiles, apart && (long)tiles * blocks <= 512 ? blocks : 1);
    const bool ln = lnw != nullptr;
    if (epi == EPI_NONE && ln)
        hipLaunchKernelGGL((k_rows128<EPI_NONE, true>), grid, dim3(256), 0, s, M, N, X, ldx, wimg, wshift, b, Y, ldy, R,
                           ldr, scale, lnw, lnb);
    else if (epi == EPI_NONE)
        hipLaunchKernelGGL((k_rows128<EPI_NONE, false>), grid, dim3(256), 0, s, M, N, X, ldx, wimg, wshift, b, Y, ldy, R,
                           ldr, scale, lnw, lnb);
    else if (epi == EPI_SCALE && ln)
        hipLaunchKernelGGL((k_rows128<EPI_SCALE, true>), grid, dim3(256), 0, s, M, N, X, ldx, wimg, wshift, b, Y, ldy, R,
                           ldr, scale, lnw, lnb);
    else if (epi == EPI_RESID && !ln)
        hipLaunchKernelGGL((k_rows128<EPI_RESID, false>), grid, dim3(256), 0, s, M, N, X, ldx, wimg, wshift, b, Y, ldy,
                           R, ldr, scale, lnw, lnb);
    else
        throw ArgError{"rows128: unsupported epilogue"};
    TAH_LAUNCHED();
}

}  // namespace tah
