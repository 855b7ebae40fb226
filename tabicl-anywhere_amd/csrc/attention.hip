// In-context attention of query rows over one stored layer of training-row keys and values: the bundle's chunk
// records (f32, or i16/i8 codes with per-chunk, per-coordinate scales, dequantised on the card), or the tile images
// made of them. This replaces the reference's streaming loop (src/predict.rs:427-533 with Soft::update/update_int,
// src/nn.rs:194-258) and its WGSL attend/merge shaders (src/gpu.rs:492-627).
//
// Keys are visited in blocks of 64 that never straddle a stored chunk. Each workgroup keeps, per query and head,
// the running maximum m, weight sum l and weighted value sum o over its range of key blocks (the online softmax
// of Soft); when the keys are split over several workgroups, their (m, l, o) are combined by a log-sum-exp merge
// (Soft::merge, src/nn.rs:261-276) and divided through (Soft::finish).
//
// The kernels:
//  * k_attn_split64: head width 64 over tile images (below; any cache format) from 17 queries, 32 queries a
//    wavefront. Every f32
//    product runs on the fp16 matrix cores as three products of fp16 halves (device_math.hpp): the error is that
//    of an f32 dot product, at v_mfma_f32_32x32x16_f16's rate (2 PFLOP/s sustained, 16x that of the f32 matrix
//    instructions). Operands are scaled by powers of two first (exact): each query to a maximum near 2^14, each
//    head's keys and values by the layer's maximum, and the softmax weights to at most 2^15, so that no half
//    overflows and the low halves stay normal for all but negligible elements.
//  * k_attn_few: head width 64, 1 to 16 queries over f32 images and i8 code images (2 to 16 over i16 code tiles):
//    the four wavefronts of a workgroup split each key block, with the queries as the 16 columns of 16 x 16
//    products, and merge their softmax states at the end.
//  * k_attn_decode_w: head width 64 and few queries (or no images), from the records: 256 threads per (six key
//    blocks, head, 8 queries), each wavefront streaming a key block at a time with no barrier (lane = key for the
//    scores, lane = coordinate for the weighted sum), integer codes scaled through the query and the sums.
//  * k_attn_decode: any other head width up to 64 (the tiny test models): the same with one wavefront.
// All of them leave the running maximum in log2 units (score * log2 e) for the split merge (head width 64:
// k_attn_merge64 for few key ranges, k_attn_merge_w for many; k_attn_merge otherwise).
#include <algorithm>

#include <atomic>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "device_math.hpp"

namespace tah {

constexpr int KB = 64;   // keys per block
constexpr int QG = 8;    // queries per decode workgroup
// Queries from which a layer's tiles are read by the matrix kernel rather than the decode kernel. Over f32 images and
// i8 code images from one query: the matrix kernel reads a tile with whole-row DMA copies, where the decode kernel's
// lanes each read a row of their own (one row: 0.694 -> 0.575 ms a prediction, 0.595 ms from the records before the
// layers were held as tiles). Over i16 code tiles from 4 (its kernel has 8 wavefronts and a staging ring, one
// workgroup a compute unit: one row after a MALL flush 0.813 -> 0.930 ms with it).
inline int split16_min_q(int kv_format) { return kv_format == TAH_KV_I16 ? TAH_SPLIT16_MIN_Q : 1; }

struct KeyBlocks {
    int bpc;       // key blocks per full chunk
    int n_chunks;  // stored chunks
    int last_rc;   // rows of the last chunk
    int n_kb;      // key blocks in all
};

__host__ __device__ inline KeyBlocks key_blocks(int rows, int chunk) {
    KeyBlocks k;
    k.bpc = (chunk + KB - 1) / KB;
    k.n_chunks = (rows + chunk - 1) / chunk;
    k.last_rc = rows - (k.n_chunks - 1) * chunk;
    k.n_kb = (k.n_chunks - 1) * k.bpc + (k.last_rc + KB - 1) / KB;
    return k;
}

__host__ __device__ inline size_t record_bytes(int fmt, int d, int rc) {
    const size_t w = fmt == TAH_KV_F32 ? 4 : (fmt == TAH_KV_I16 ? 2 : 1);
    return 2 * (size_t)d * rc * w + (fmt == TAH_KV_F32 ? 0 : 8 * (size_t)d);
}

// Where key block kb lives: its chunk's record, the chunk's row count and the block's first row in it.
struct Where {
    const uint8_t *rec;
    int rc, o, nk;
};

__device__ inline Where locate(const KeyBlocks &k, int kb, const uint8_t *records, int fmt, int d, int chunk) {
    Where w;
    const int ci = kb / k.bpc, j = kb % k.bpc;
    w.rec = records + (size_t)ci * record_bytes(fmt, d, chunk);
    w.rc = ci == k.n_chunks - 1 ? k.last_rc : chunk;
    w.o = j * KB;
    w.nk = min(KB, w.rc - w.o);
    return w;
}

// Element (coordinate c of the 2d stacked K;V rows, key r) of a record, widened and scaled to f32.
template <int FMT>
__device__ __forceinline__ float rec_value(const uint8_t *rec, int d, int rc, int c, int r) {
    if (FMT == TAH_KV_F32) return reinterpret_cast<const float *>(rec)[(size_t)c * rc + r];
    const float sc = reinterpret_cast<const float *>(rec)[c];
    const uint8_t *body = rec + 8 * (size_t)d;
    if (FMT == TAH_KV_I16) return (float)reinterpret_cast<const int16_t *>(body)[(size_t)c * rc + r] * sc;
    return (float)reinterpret_cast<const int8_t *>(body)[(size_t)c * rc + r] * sc;
}

// Sixteen consecutive keys (from key o16) of stacked coordinate c, widened, into dst[0..16). Fast path when the
// row segment is whole and 16-byte aligned.
template <int FMT>
__device__ __forceinline__ void load16(const uint8_t *rec, int d, int rc, int c, int o16, int nk_left, bool fast,
                                       float *dst) {
    if (fast) {
        if (FMT == TAH_KV_F32) {
            const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(rec) + (size_t)c * rc + o16);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 v = p[i];
                dst[4 * i] = v.x;
                dst[4 * i + 1] = v.y;
                dst[4 * i + 2] = v.z;
                dst[4 * i + 3] = v.w;
            }
        } else {
            const float sc = reinterpret_cast<const float *>(rec)[c];
            const uint8_t *body = rec + 8 * (size_t)d;
            if (FMT == TAH_KV_I16) {
                const int16_t *p = reinterpret_cast<const int16_t *>(body) + (size_t)c * rc + o16;
                const uint4 a = reinterpret_cast<const uint4 *>(p)[0], b = reinterpret_cast<const uint4 *>(p)[1];
                const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    dst[2 * i] = (float)(int16_t)(w[i] & 0xffffu) * sc;
                    dst[2 * i + 1] = (float)(int16_t)(w[i] >> 16) * sc;
                }
            } else {
                const int8_t *p = reinterpret_cast<const int8_t *>(body) + (size_t)c * rc + o16;
                const uint4 a = reinterpret_cast<const uint4 *>(p)[0];
                const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int j = 0; j < 4; j++) dst[4 * i + j] = (float)(int8_t)((w[i] >> (8 * j)) & 0xffu) * sc;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; i++) dst[i] = i < nk_left ? rec_value<FMT>(rec, d, rc, c, o16 + i) : 0.0f;
    }
}

// ---- tiles: the form in which a layer of head width 64 is held on the card (its records are not kept) --------------
// f32 caches: split images, the keys and values split into fp16 halves and laid out as the split kernel's LDS image.
// One image per (key block, head), 32 KB: K hi, K lo as [64 keys][64 coordinates] and V hi, V lo as
// [64 coordinates][64 keys], fp16, each 128-byte row split in eight 16-byte chunks stored XOR-swizzled by row: the
// 64-bank LDS serves a 128-bit read 16 lanes at a time, and the 16 rows one such group reads (at one logical chunk)
// then fall on 16 different 16-byte bank groups. Keys past the end of a short block are zeros. Each head's
// keys are scaled by 2^sk and values by 2^sv, the powers of two that bring the layer's largest magnitude of that
// head below 2^14; kvmax holds those maxima (f32 bits) per head, [heads][2].
constexpr int IMG = 32768;
// i8 caches: code images. The codes are integers of at most 127 in magnitude, exact in fp16, so an image holds them
// as they are, one plane each (K codes [key][coordinate], then V codes [coordinate][key], in the layout of the
// planes above), and the scales stay beside them: per (chunk, head) the head's 64 key scales, its 64 value scales
// (a zero scale, whose coordinate's codes are all zero, stored as 1) and the 64 ratios of the previous chunk's value
// scales to these (1 for the first chunk): scale table [chunks][heads][3][64]. Scores are then (q * key scales) .
// codes, two products of the split query with the codes; the weighted sums codes . weights, two products of the split
// weights, kept in units of the current chunk's value scales (multiplied by the ratios when a chunk begins, by the
// value scales at the end).
constexpr int IMG8 = 16384;
constexpr int SCL = 768;  // bytes of one (chunk, head)'s scales
// i16 caches: code tiles, 16.5 KB per (key block, head): the K codes as [64 keys][64 coordinates], then the block's
// chunk's 64 key factors, then the V codes as [64 coordinates][64 keys], then its 64 value factors; int16 codes in
// 128-byte rows in order (not swizzled: the attention kernel swizzles as it writes its LDS images, and the decode
// kernel reads whole rows), zeros past a short block's end. The codes are not exact in fp16 (up to 32767), so the
// attention kernel dequantises them itself: each factor is the chunk's scale of that coordinate times 2^sk (2^sv),
// the power of two that brings the head's largest dequantised |K| (|V|) below 2^14, as for f32 images (kvmax, the
// maxima, [heads][2]). Every block carries its chunk's factors, so that one copy brings a half tile and its factors.
constexpr int HALF16 = 8192 + 256;  // a half tile: 64 rows of codes, then 64 factors
constexpr int IMG16 = 2 * HALF16;

__host__ __device__ constexpr int img_bytes(int fmt) { return fmt == TAH_KV_F32 ? IMG : (fmt == TAH_KV_I16 ? IMG16 : IMG8); }

__host__ __device__ inline size_t image_bytes_of(int rows, int chunk, int heads, int fmt) {
    return (size_t)key_blocks(rows, chunk).n_kb * heads * img_bytes(fmt);
}

// rows r and r + 1 already sit in different bank halves (128-byte rows); rows of one parity among 16 consecutive ones
// get eight different chunks
__device__ __forceinline__ int swz(int r, int c) { return c ^ ((r >> 1) & 7); }

// ---- decode kernel: any head width <= 64, few queries --------------------------------------------------------
// grid (splits, heads, query groups of QG); 64 threads.
template <int FMT>
__global__ __launch_bounds__(64) void k_attn_decode(int nq, int rows, int chunk, int d, int heads,
                                                     const float *__restrict__ q, const uint8_t *__restrict__ records,
                                                     int kb_per_split, float *__restrict__ part_o,
                                                     float *__restrict__ part_ml, float *__restrict__ out) {
    __shared__ float Qs[QG][64];
    __shared__ float Ks[64][KB + 1];
    __shared__ float Vs[64][KB + 1];
    __shared__ float Ps[QG][KB];
    const int lane = threadIdx.x;
    const int split = blockIdx.x, h = blockIdx.y, q0 = blockIdx.z * QG;
    const int splits = gridDim.x;
    const int hd = d / heads;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const int kb0 = split * kb_per_split, kb1 = min(kbs.n_kb, kb0 + kb_per_split);
    for (int qi = 0; qi < QG; qi++) Qs[qi][lane] = (lane < hd && q0 + qi < nq) ? q[(size_t)(q0 + qi) * d + h * hd + lane] : 0.0f;
    float m[QG], l[QG], o[QG];
#pragma unroll
    for (int qi = 0; qi < QG; qi++) {
        m[qi] = -INFINITY;
        l[qi] = 0.0f;
        o[qi] = 0.0f;
    }
    for (int kb = kb0; kb < kb1; kb++) {
        const Where w = locate(kbs, kb, records, FMT, d, chunk);
        __syncthreads();
        for (int c = 0; c < hd; c++) {
            Ks[c][lane] = lane < w.nk ? rec_value<FMT>(w.rec, d, w.rc, h * hd + c, w.o + lane) : 0.0f;
            Vs[c][lane] = lane < w.nk ? rec_value<FMT>(w.rec, d, w.rc, d + h * hd + c, w.o + lane) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int qi = 0; qi < QG; qi++) {
            float s = 0.0f;
            for (int c = 0; c < hd; c++) s += Qs[qi][c] * Ks[c][lane];
            if (lane >= w.nk) s = -INFINITY;
            const float mnew = fmaxf(m[qi], wave_max(s));
            const float alpha = fast_exp(m[qi] - mnew);
            const float p = lane < w.nk ? fast_exp(s - mnew) : 0.0f;
            l[qi] = l[qi] * alpha + wave_sum(p);
            m[qi] = mnew;
            o[qi] *= alpha;
            Ps[qi][lane] = p;
        }
        __syncthreads();
        if (lane < hd) {
#pragma unroll
            for (int qi = 0; qi < QG; qi++) {
                float a = 0.0f;
                for (int k = 0; k < KB; k++) a += Ps[qi][k] * Vs[lane][k];
                o[qi] += a;
            }
        }
    }
    if (lane >= hd) return;
#pragma unroll
    for (int qi = 0; qi < QG; qi++) {
        const int qr = q0 + qi;
        if (qr >= nq) break;
        if (splits == 1) {
            out[(size_t)qr * d + h * hd + lane] = o[qi] / l[qi];
        } else {
            const size_t at = ((size_t)split * nq + qr) * heads + h;
            part_o[at * hd + lane] = o[qi];
            if (lane == 0) {
                part_ml[at * 2] = m[qi] * LOG2E;
                part_ml[at * 2 + 1] = l[qi];
            }
        }
    }
}

// ---- decode kernel for head width 64: few queries, bandwidth-bound ------------------------------------------
// ---- decode kernel with independent wavefronts: head width 64, at most QG queries ------------------------------
// grid (splits, heads, query groups of QG); 256 threads. Each wavefront streams its own key blocks of the
// workgroup's range (kb0 + w, kb0 + w + 4, ...) straight from the stored records, with no barrier between blocks, so
// every wavefront keeps a whole block's loads in flight: the scores with lane = key (a coordinate's 64 keys are one
// coalesced row of the record), the weighted values with lane = coordinate (its 64 keys are 64 contiguous values).
// Integer codes are used as stored: the chunk's key scales multiply the query and its value scales the block's
// weighted sum (Soft::update_int, src/nn.rs:233-258). The wavefronts' (m, l, o) are merged through LDS at the end.
template <int FMT>
__device__ __forceinline__ float raw_at(const uint8_t *body, size_t i) {
    if (FMT == TAH_KV_F32) return reinterpret_cast<const float *>(body)[i];
    if (FMT == TAH_KV_I16) return (float)reinterpret_cast<const int16_t *>(body)[i];
    return (float)reinterpret_cast<const int8_t *>(body)[i];
}

// The 64 values of stacked coordinate c for keys o.. o + 63 of a record (raw: codes unscaled), zero past nk.
template <int FMT>
__device__ __forceinline__ void row64(const uint8_t *body, int rc, int c, int o, int nk, bool fast, float (&v)[64]) {
    if (fast) {
        if (FMT == TAH_KV_F32) {
            const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(body) + (size_t)c * rc + o);
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float4 x = p[i];
                v[4 * i] = x.x;
                v[4 * i + 1] = x.y;
                v[4 * i + 2] = x.z;
                v[4 * i + 3] = x.w;
            }
        } else if (FMT == TAH_KV_I16) {
            const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const int16_t *>(body) + (size_t)c * rc + o);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint4 x = p[i];
                const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    v[8 * i + 2 * j] = (float)(int16_t)(w[j] & 0xffffu);
                    v[8 * i + 2 * j + 1] = (float)(int16_t)(w[j] >> 16);
                }
            }
        } else {
            const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const int8_t *>(body) + (size_t)c * rc + o);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint4 x = p[i];
                const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                for (int j = 0; j < 4; j++)
#pragma unroll
                    for (int b = 0; b < 4; b++) v[16 * i + 4 * j + b] = (float)(int8_t)((w[j] >> (8 * b)) & 0xffu);
            }
        }
    } else {
        // every load in bounds (the key clamped to the block's last), the keys past it zeroed after: no branches
#pragma unroll
        for (int k = 0; k < 64; k++) {
            const float x = raw_at<FMT>(body, (size_t)c * rc + o + min(k, nk - 1));
            v[k] = k < nk ? x : 0.0f;
        }
    }
}

// A tile row (64 values, widened to f32, unscaled) of key block kb's tile (the layouts of the split images, code tiles
// and code images below): VALS false the K row of key r, true the V row of coordinate r.
template <int FMT, bool VALS>
__device__ __forceinline__ void tile_row(const uint8_t *tile, int r, float (&v)[64]) {
#pragma unroll
    for (int c = 0; c < 8; c++) {
        if constexpr (FMT == TAH_KV_I16) {
            const uint4 x = *reinterpret_cast<const uint4 *>(tile + (VALS ? HALF16 : 0) + r * 128 + c * 16);
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                v[8 * c + 2 * t] = (float)(int16_t)(w[t] & 0xffffu);
                v[8 * c + 2 * t + 1] = (float)(int16_t)(w[t] >> 16);
            }
        } else {
            const int off = (FMT == TAH_KV_F32 ? (VALS ? 16384 : 0) : (VALS ? 8192 : 0)) + r * 128 + swz(r, c) * 16;
            const halfx8 hi = *reinterpret_cast<const halfx8 *>(tile + off);
            if constexpr (FMT == TAH_KV_F32) {
                const halfx8 lo = *reinterpret_cast<const halfx8 *>(tile + off + 8192);
                const u32x4 hw = __builtin_bit_cast(u32x4, hi), lw = __builtin_bit_cast(u32x4, lo);
#pragma unroll
                for (int t = 0; t < 4; t++) join2(hw[t], lw[t], v[8 * c + 2 * t], v[8 * c + 2 * t + 1]);
            } else {
#pragma unroll
                for (int t = 0; t < 8; t++) v[8 * c + t] = (float)hi[t];
            }
        }
    }
}

// TILES: over a layer's tiles (records is then the tiles' base; kvmax the f32 and i16 maxima, scl the i16 factors or
// the i8 scales) instead of its records: lane = key reads its key's 64 coordinates as one row of the tile, lane =
// coordinate its 64 keys; every format is scaled through the query (keys) and the sums (values) as integer codes are.
template <int FMT, bool TILES>
__global__ __launch_bounds__(256) void k_attn_decode_w(int nq, int rows, int chunk, int d, int heads,
                                                       const float *__restrict__ q, const uint8_t *__restrict__ records,
                                                       const uint32_t *__restrict__ kvmax,
                                                       const float *__restrict__ scl, int kb_per_split,
                                                       float *__restrict__ part_o, float *__restrict__ part_ml,
                                                       float *__restrict__ out) {
    __shared__ float Qs[QG][64];
    __shared__ float Qk[4][QG][64];  // INT: each wavefront's queries times its block's key scales
    __shared__ float Ps[4][QG][KB];
    __shared__ float Wml[4][QG][2];
    __shared__ float Wo[4][QG][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x, h = blockIdx.y, q0 = blockIdx.z * QG;
    const int splits = gridDim.x;
    const int nqg = min(QG, nq - q0);
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const int kb0 = split * kb_per_split, kb1 = min(kbs.n_kb, kb0 + kb_per_split);
    constexpr bool INT = FMT != TAH_KV_F32 || TILES;  // keys scaled through the query, values through the sums
    const int width = FMT == TAH_KV_F32 ? 4 : (FMT == TAH_KV_I16 ? 2 : 1);
    // TILES, f32 and i16: the head's powers of two (the tiles hold K 2^sk, V 2^sv)
    float uk = 1.0f, uv = 1.0f;
    if constexpr (TILES && FMT != TAH_KV_I8) {
        uk = ldexpf(1.0f, -shift_for(kvmax[h * 2]));
        uv = ldexpf(1.0f, -shift_for(kvmax[h * 2 + 1]));
    }
    for (int i = tid; i < QG * 64; i += 256) {
        const int qi = i >> 6, c = i & 63;
        Qs[qi][c] = qi < nqg ? q[(size_t)(q0 + qi) * d + h * 64 + c] : 0.0f;
    }
    __syncthreads();
    float m[QG], l[QG], o[QG];
#pragma unroll
    for (int qi = 0; qi < QG; qi++) {
        m[qi] = -INFINITY;
        l[qi] = 0.0f;
        o[qi] = 0.0f;
    }
    for (int kb = kb0 + wave; kb < kb1; kb += 4) {
        const Where w = locate(kbs, kb, records, FMT, d, chunk);
        const uint8_t *body = INT ? w.rec + 8 * (size_t)d : w.rec;
        const bool kin = lane < w.nk;
        const bool fast = w.nk == KB && ((size_t)w.rc * width) % 16 == 0;
        // keys: lane = key, coordinates 0..63 of this head (lanes past the block's keys read its last key and are
        // masked below); values: lane = coordinate, keys 0..63 of the block
        float kc[64], vr[64];
        const int kl = min(lane, w.nk - 1);
        float ks = 1.0f, vs = 1.0f;
        if constexpr (TILES) {
            const uint8_t *tile = records + ((size_t)kb * heads + h) * img_bytes(FMT);
            tile_row<FMT, false>(tile, kl, kc);
            tile_row<FMT, true>(tile, lane, vr);
            const int ci = kb / kbs.bpc;
            if constexpr (FMT == TAH_KV_F32) {
                ks = uk;
                vs = uv;
            } else if constexpr (FMT == TAH_KV_I16) {
                ks = reinterpret_cast<const float *>(tile + 8192)[lane] * uk;
                vs = reinterpret_cast<const float *>(tile + HALF16 + 8192)[lane] * uv;
            } else {
                const float *sc8 = scl + ((size_t)ci * heads + h) * 192;
                ks = sc8[lane];
                vs = sc8[64 + lane];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 64; c++) kc[c] = raw_at<FMT>(body, (size_t)(h * 64 + c) * w.rc + w.o + kl);
            row64<FMT>(body, w.rc, d + h * 64 + lane, w.o, w.nk, fast, vr);
            if constexpr (INT) {
                // the chunk's scales of this head: keys' multiply the queries (lane = coordinate), values' the sums
                const float *sc = reinterpret_cast<const float *>(w.rec);
                ks = sc[h * 64 + lane];
                vs = sc[d + h * 64 + lane];
            }
        }
        if (INT) {
#pragma unroll
            for (int qi = 0; qi < QG; qi++)
                if (qi < nqg) Qk[wave][qi][lane] = Qs[qi][lane] * ks;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
#pragma unroll
        for (int qi = 0; qi < QG; qi++) {
            if (qi >= nqg) break;  // (uniform) no query in this slot
            float sc = 0.0f;
#pragma unroll
            for (int c = 0; c < 64; c++) sc += (INT ? Qk[wave][qi][c] : Qs[qi][c]) * kc[c];
            if (!kin) sc = -INFINITY;
            const float mnew = fmaxf(m[qi], wave_max(sc));
            const float alpha = fast_exp(m[qi] - mnew);
            const float p = kin ? fast_exp(sc - mnew) : 0.0f;
            l[qi] = l[qi] * alpha + wave_sum(p);
            m[qi] = mnew;
            o[qi] *= alpha;
            Ps[wave][qi][lane] = p;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int qi = 0; qi < QG; qi++) {
            if (qi >= nqg) break;
            float a = 0.0f;
#pragma unroll
            for (int k = 0; k < KB; k++) a += Ps[wave][qi][k] * vr[k];
            o[qi] += INT ? a * vs : a;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();  // the weights are read before the next block's are written
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
#pragma unroll
    for (int qi = 0; qi < QG; qi++) {
        if (qi >= nqg) break;
        Wo[wave][qi][lane] = o[qi];
        if (lane == 0) {
            Wml[wave][qi][0] = m[qi];
            Wml[wave][qi][1] = l[qi];
        }
    }
    __syncthreads();
    // wavefront w finishes queries w and w + 4
    for (int qi = wave; qi < nqg; qi += 4) {
        float M = -INFINITY;
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (Wml[u][qi][1] > 0.0f) M = fmaxf(M, Wml[u][qi][0]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float f = Wml[u][qi][1] > 0.0f ? fast_exp(Wml[u][qi][0] - M) : 0.0f;
            L += Wml[u][qi][1] * f;
            O += Wo[u][qi][lane] * f;
        }
        const int qr = q0 + qi;
        if (splits == 1) {
            out[(size_t)qr * d + h * 64 + lane] = O / L;
        } else {
            const size_t at = ((size_t)split * nq + qr) * heads + h;
            part_o[at * 64 + lane] = O;
            if (lane == 0) {
                part_ml[at * 2] = M * LOG2E;
                part_ml[at * 2 + 1] = L;
            }
        }
    }
}


__global__ __launch_bounds__(64) void k_zero_u32(int n, uint32_t *__restrict__ p) {
    const int i = blockIdx.x * 64 + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// grid (key blocks, heads); 256 threads: the largest |K| and |V| of each head, by integer max on the f32 bits
// (non-negative floats order as their bit patterns).
template <int FMT>
__global__ __launch_bounds__(256) void k_kv_absmax(int rows, int chunk, int d, int heads, const uint8_t *__restrict__ records,
                                                    uint32_t *__restrict__ kvmax) {
    __shared__ float red[2][4];
    const int kb = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const Where w = locate(kbs, kb, records, FMT, d, chunk);
    const int lc = tid >> 2, seg = (tid & 3) * 16;
    const int width = FMT == TAH_KV_F32 ? 4 : (FMT == TAH_KV_I16 ? 2 : 1);
    const bool fast = w.nk == KB && ((size_t)w.rc * width) % 16 == 0;
    float tk[16], tv[16];
    load16<FMT>(w.rec, d, w.rc, h * 64 + lc, w.o + seg, w.nk - seg, fast, tk);
    load16<FMT>(w.rec, d, w.rc, d + h * 64 + lc, w.o + seg, w.nk - seg, fast, tv);
    float mk = 0.0f, mv = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        mk = fmaxf(mk, fabsf(tk[i]));
        mv = fmaxf(mv, fabsf(tv[i]));
    }
    mk = wave_max(mk);
    mv = wave_max(mv);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = mk;
        red[1][tid >> 6] = mv;
    }
    __syncthreads();
    if (tid < 2) {
        const float m = fmaxf(fmaxf(red[tid][0], red[tid][1]), fmaxf(red[tid][2], red[tid][3]));
        atomicMax(kvmax + h * 2 + tid, __float_as_uint(m));
    }
}

// grid (key blocks, heads); 256 threads: one tile image.
template <int FMT>
__global__ __launch_bounds__(256) void k_kv_images(int rows, int chunk, int d, int heads,
                                                    const uint8_t *__restrict__ records,
                                                    const uint32_t *__restrict__ kvmax, uint8_t *__restrict__ images) {
    __shared__ float Ks[64][KB + 1];  // [coordinate][key]
    __shared__ float Vs[64][KB + 1];
    const int kb = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const Where w = locate(kbs, kb, records, FMT, d, chunk);
    const int lc = tid >> 2, seg = (tid & 3) * 16;
    const int width = FMT == TAH_KV_F32 ? 4 : (FMT == TAH_KV_I16 ? 2 : 1);
    const bool fast = w.nk == KB && ((size_t)w.rc * width) % 16 == 0;
    float tk[16], tv[16];
    load16<FMT>(w.rec, d, w.rc, h * 64 + lc, w.o + seg, w.nk - seg, fast, tk);
    load16<FMT>(w.rec, d, w.rc, d + h * 64 + lc, w.o + seg, w.nk - seg, fast, tv);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        Ks[lc][seg + i] = tk[i];
        Vs[lc][seg + i] = tv[i];
    }
    __syncthreads();
    const float fk = ldexpf(1.0f, shift_for(kvmax[h * 2])), fv = ldexpf(1.0f, shift_for(kvmax[h * 2 + 1]));
    uint8_t *img = images + ((size_t)kb * heads + h) * IMG;
    for (int u = tid; u < 512; u += 256) {
        const int r = u >> 3, c = u & 7;
        halfx8 kh, kl, vh, vl;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            const float x = Ks[8 * c + t][r] * fk;  // key r, coordinate 8c + t
            const _Float16 xh = (_Float16)x;
            kh[t] = xh;
            kl[t] = (_Float16)(x - (float)xh);
            const float y = Vs[r][8 * c + t] * fv;  // coordinate r, key 8c + t
            const _Float16 yh = (_Float16)y;
            vh[t] = yh;
            vl[t] = (_Float16)(y - (float)yh);
        }
        *reinterpret_cast<halfx8 *>(img + r * 128 + swz(r, c) * 16) = kh;
        *reinterpret_cast<halfx8 *>(img + 8192 + r * 128 + swz(r, c) * 16) = kl;
        *reinterpret_cast<halfx8 *>(img + 16384 + r * 128 + swz(r, c) * 16) = vh;
        *reinterpret_cast<halfx8 *>(img + 24576 + r * 128 + swz(r, c) * 16) = vl;
    }
}

// grid (key blocks, heads); 256 threads: one code image of an i8 layer, and (by a chunk's first block) the chunk's
// scales of the head. Thread t: coordinate t / 4, keys 16 (t % 4) .. + 15 of the block (zeros past its end).
__global__ __launch_bounds__(256) void k_kv_codes(int rows, int chunk, int d, int heads, const uint8_t *__restrict__ records,
                                                  uint8_t *__restrict__ images, float *__restrict__ scales) {
    __shared__ _Float16 Ks[64][KB + 8];  // [coordinate][key]
    __shared__ _Float16 Vs[64][KB + 8];
    const int kb = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const Where w = locate(kbs, kb, records, TAH_KV_I8, d, chunk);
    const int lc = tid >> 2, seg = (tid & 3) * 16;
    const int8_t *body = reinterpret_cast<const int8_t *>(w.rec + 8 * (size_t)d);
    const int8_t *kr = body + (size_t)(h * 64 + lc) * w.rc + w.o, *vr = body + (size_t)(d + h * 64 + lc) * w.rc + w.o;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const bool in = seg + i < w.nk;
        Ks[lc][seg + i] = (_Float16)(in ? (float)kr[seg + i] : 0.0f);
        Vs[lc][seg + i] = (_Float16)(in ? (float)vr[seg + i] : 0.0f);
    }
    if (kb % kbs.bpc == 0 && tid < 192) {
        // the record's scales: d key scales then d value scales (the previous chunk's record precedes it)
        const int ci = kb / kbs.bpc, c = tid & 63;
        const float *sc = reinterpret_cast<const float *>(w.rec);
        float v;
        if (tid < 64) {
            v = sc[h * 64 + c];
        } else {
            const float vs = sc[d + h * 64 + c], vsn = vs == 0.0f ? 1.0f : vs;
            if (tid < 128) {
                v = vsn;
            } else {
                const float *pc = reinterpret_cast<const float *>(w.rec - record_bytes(TAH_KV_I8, d, chunk));
                const float pv = ci == 0 ? 1.0f : pc[d + h * 64 + c];
                v = ci == 0 ? 1.0f : (pv == 0.0f ? 1.0f : pv) / vsn;
            }
        }
        scales[((size_t)ci * heads + h) * 192 + tid] = v;
    }
    __syncthreads();
    uint8_t *img = images + ((size_t)kb * heads + h) * IMG8;
    for (int u = tid; u < 512; u += 256) {
        const int r = u >> 3, c = u & 7;
        halfx8 kc, vc;
#pragma unroll
        for (int t = 0; t < 8; t++) {
            kc[t] = Ks[8 * c + t][r];  // key r, coordinate 8c + t
            vc[t] = Vs[r][8 * c + t];  // coordinate r, key 8c + t
        }
        *reinterpret_cast<halfx8 *>(img + r * 128 + swz(r, c) * 16) = kc;
        *reinterpret_cast<halfx8 *>(img + 8192 + r * 128 + swz(r, c) * 16) = vc;
    }
}

// grid (key blocks, heads); 256 threads: one code tile of an i16 layer with its chunk's dequantisation factors. Thread t: coordinate t / 4, keys 16 (t % 4) .. + 15 of the block (zeros past
// its end). kvmax (k_kv_absmax) holds the head's largest dequantised |K| and |V|.
__global__ __launch_bounds__(256) void k_kv_tiles16(int rows, int chunk, int d, int heads,
                                                    const uint8_t *__restrict__ records,
                                                    const uint32_t *__restrict__ kvmax, uint8_t *__restrict__ tiles) {
    __shared__ int16_t Ks[64][KB + 8];  // [coordinate][key]
    const int kb = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const Where w = locate(kbs, kb, records, TAH_KV_I16, d, chunk);
    const int lc = tid >> 2, seg = (tid & 3) * 16;
    const int16_t *body = reinterpret_cast<const int16_t *>(w.rec + 8 * (size_t)d);
    const int16_t *kr = body + (size_t)(h * 64 + lc) * w.rc + w.o, *vr = body + (size_t)(d + h * 64 + lc) * w.rc + w.o;
    uint8_t *tile = tiles + ((size_t)kb * heads + h) * IMG16;
    int16_t vv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const bool in = seg + i < w.nk;
        Ks[lc][seg + i] = in ? kr[seg + i] : (int16_t)0;
        vv[i] = in ? vr[seg + i] : (int16_t)0;
    }
    // V codes: row lc, keys seg .. seg + 15
    *reinterpret_cast<uint4 *>(tile + HALF16 + lc * 128 + seg * 2) = *reinterpret_cast<const uint4 *>(vv);
    *reinterpret_cast<uint4 *>(tile + HALF16 + lc * 128 + seg * 2 + 16) = *reinterpret_cast<const uint4 *>(vv + 8);
    if (tid < 128) {
        // the record's scales (d key scales then d value scales) times the head's powers of two, after each half
        const int c = tid & 63, which = tid >> 6;
        const float *sc = reinterpret_cast<const float *>(w.rec);
        const float f = ldexpf(1.0f, shift_for(kvmax[h * 2 + which]));
        reinterpret_cast<float *>(tile + which * HALF16 + 8192)[c] = sc[which * d + h * 64 + c] * f;
    }
    __syncthreads();
    // K codes: row = key, 8 coordinates a 16-byte chunk
    for (int u = tid; u < 512; u += 256) {
        const int r = u >> 3, c = u & 7;
        int16_t kc[8];
#pragma unroll
        for (int t = 0; t < 8; t++) kc[t] = Ks[8 * c + t][r];
        *reinterpret_cast<uint4 *>(tile + r * 128 + c * 16) = *reinterpret_cast<const uint4 *>(kc);
    }
}

// ---- split-fp16 MFMA kernel: head width 64 over tile images --------------------------------------------------
// A flat grid of qtiles x heads x splits workgroups of WAVES wavefronts x 32 queries (the flat index remapped so that
// the query tiles sharing a (head, key range) run on the same XCD: workgroup i is dispatched to XCD i % 8, and the
// tiles of one (head, range) then read the same images through one L2), two wavefronts a SIMD: 8 wavefronts (256 queries, one workgroup a compute unit) for many queries, 4 (two
// workgroups a compute unit) otherwise. Key blocks of 64 stream through LDS in two rings of two 16 KB buffers, one
// for the blocks' key halves (K hi, K lo) and one for their value halves (V hi, V lo), copied global -> LDS directly
// (global_load_lds_dwordx4); one barrier per block.
//
// Each wavefront forms S^T = K Q^T for two halves of 32 keys with v_mfma_f32_32x32x16_f16: lane l owns query l % 32
// and holds 16 of the half's keys. The A operand's row i takes key sigma(i) (bits 3 and 2 of i swapped), which puts
// eight consecutive keys (16 (v / 8) + 8 (l / 32) + v % 8) in each lane's accumulators v = 8 hh..8 hh + 7: exactly
// the B operand that O^T = V^T P^T needs for a reduction over 16 keys, so the weights never leave the lane.
//
// The loop is software-pipelined one block deep: while block kb's softmax weights are formed on the VALU, the
// matrix cores compute block kb + 1's scores, then block kb's weighted values; one scheduling region per block
// interleaves the three (sched_group_barrier), so that each wavefront keeps its own matrix work queued under its
// vector work. Block kb's keys are thus read one block ahead of its values: in step kb the buffers hold keys kb + 1
// and values kb, and the copies bring in keys kb + 2 and values kb + 1.
//
// The softmax runs in log2 units against a reference maximum that is raised only when a block's maximum passes it by
// more than 3 (then the sums are rescaled): weights exp2(t - ref + 12) stay below 2^15, inside fp16, and most blocks
// skip the rescaling.

// Half an image (its keys or its values: BYTES, 16 KB of split values or 8 KB of codes) into an LDS buffer, 16 bytes
// a lane: in copy i, wavefront w fills the 1 KB at chunk 64 (WAVES i + w) (a wavefront-uniform LDS base; the lanes'
// offsets are implicit).
template <int WAVES, int BYTES>
__device__ __forceinline__ void half_image_to_lds(const uint8_t *src, uint8_t *dst, int tid) {
    constexpr int T = 64 * WAVES, CHUNKS = BYTES / 16;
    static_assert(BYTES % 16 == 0, "whole 16-byte copies");
    const int w = tid >> 6;
#pragma unroll
    for (int i = 0; i < (CHUNKS + T - 1) / T; i++) {
        const int base = i * T + 64 * w;
        // lanes past the last copy stay idle (a copy a lane: each writes its own 16 bytes at dst + 16 (base + lane))
        if (CHUNKS % T == 0 || base + (tid & 63) < CHUNKS)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4 *>(src) + base + (tid & 63), dst + 16 * base, 16,
                                             0, 0);
    }
}

// i16 staging (k_attn_split64 with STAGED): half a code tile (8 KB of codes and its 256 bytes of factors, keys or
// values) into a staging slot's half by DMA: 528 copies of 16 bytes, the last 16 by wavefront 0.
template <int WAVES>
__device__ __forceinline__ void stage_half16(const uint8_t *src, uint8_t *dst, int tid) {
    half_image_to_lds<WAVES, HALF16>(src, dst, tid);
}

// A staging slot's key codes into the split image kdst (K hi, K lo) and its value codes into vdst (V hi, V lo), either
// null for none: the dequantised values (code times its coordinate's factor, in f32) split into fp16 halves, written
// swizzled as the images are; each thread takes 16 bytes (8 codes) of a 128-byte row at a time.
template <int WAVES>
__device__ __forceinline__ void convert16(const uint8_t *st, uint8_t *kdst, uint8_t *vdst, int tid) {
#pragma unroll
    for (int i = 0; i < 512 / (64 * WAVES); i++) {
        const int u = tid + 64 * WAVES * i, r = u >> 3, c = u & 7;
        const int off = r * 128 + swz(r, c) * 16;
        if (kdst) {
            // key r, coordinates 8 c .. 8 c + 7, each with its own factor
            float f[8];
            load8(reinterpret_cast<const float *>(st + 8192) + 8 * c, f);
            halfx8 hi, lo;
            dequant_split8(*reinterpret_cast<const uint4 *>(st + r * 128 + c * 16), f, hi, lo);
            *reinterpret_cast<halfx8 *>(kdst + off) = hi;
            *reinterpret_cast<halfx8 *>(kdst + 8192 + off) = lo;
        }
        if (vdst) {
            // coordinate r, keys 8 c .. 8 c + 7, one factor
            const float fv = reinterpret_cast<const float *>(st + HALF16 + 8192)[r];
            const float f[8] = {fv, fv, fv, fv, fv, fv, fv, fv};
            halfx8 hi, lo;
            dequant_split8(*reinterpret_cast<const uint4 *>(st + HALF16 + r * 128 + c * 16), f, hi, lo);
            *reinterpret_cast<halfx8 *>(vdst + off) = hi;
            *reinterpret_cast<halfx8 *>(vdst + 8192 + off) = lo;
        }
    }
}

template <bool B>
struct Flag {
    static constexpr bool value = B;
};

// With CODES (i8 caches) the images hold the codes and `scl` the scales (k_kv_codes): the scores are two products of
// the query, multiplied by the chunk's key scales and split again whenever a block starts a new chunk (the raw query
// waits in LDS), with the key codes; the weighted sums two products of the split weights with the value codes, kept
// in units of the current chunk's value scales (multiplied by the table's ratios when a block begins a chunk, by the
// last chunk's value scales at the end: no second set of sums). The scales of a chunk are copied into a four-deep LDS
// ring (DMA, two blocks ahead like the images), which a chunk's blocks use until the one after next begins.
//
// With an i16 cache (STAGED) the tiles hold codes (k_kv_tiles16), which are not exact in fp16: each half tile (8 KB of
// codes and its 256 bytes of factors) is copied into one of two LDS staging slots by DMA, one block earlier than an
// image would be, and at the next step every thread dequantises 8 codes of each half (code times its coordinate's factor,
// in f32) and writes them split into the same LDS images as an f32 layer's, which the rest of the kernel reads
// unchanged. In step kb the staging slot of its parity holds keys kb + 2 and values kb + 1 (converted then), and the
// copies bring keys kb + 3 and values kb + 2 into the other.
template <int WAVES, int FMT>
__global__ __launch_bounds__(64 * WAVES, 2) void k_attn_split64(int nq, int rows, int chunk, int d, int heads,
                                                               const float *__restrict__ q,
                                                               const uint8_t *__restrict__ images,
                                                               const uint32_t *__restrict__ kvmax,
                                                               const float *__restrict__ scl, int kb_per_split,
                                                               int qtiles, int splits, float *__restrict__ part_o,
                                                               float *__restrict__ part_ml, float *__restrict__ out) {
    constexpr bool CODES = FMT == TAH_KV_I8;    // fp16 code images, scales applied in the kernel
    constexpr bool STAGED = FMT == TAH_KV_I16;  // int16 code tiles dequantised into split images in the kernel
    constexpr int HB = CODES ? IMG8 / 2 : IMG / 2;  // bytes of an LDS image's keys (or values)
    constexpr int IS = img_bytes(FMT);              // bytes of a tile in memory
    constexpr int SG = IMG16;                       // STAGED: a staging slot, a whole code tile
    __shared__ __align__(16) uint8_t kt[2][HB], vt[2][HB];
    __shared__ __align__(16) float sb[CODES ? 4 : 1][192];  // CODES: scale ring, [chunk % 4][key, value, ratio]
    // CODES: each lane's 32 query coordinates, kept for the per-chunk splits: [wavefront][8 chunks of 4][lane][4];
    // STAGED: the two staging slots (one array for both: the compiler's host pass refuses the kernel with them apart)
    __shared__ __align__(16) uint8_t side[CODES ? WAVES * 8192 : (STAGED ? 2 * SG : 16)];
    float (*qraw)[8 * 64 * 4] = reinterpret_cast<float (*)[8 * 64 * 4]>(side);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int total = qtiles * heads * splits;
    int flat = blockIdx.x;
    if (total % 8 == 0) flat = (flat % 8) * (total / 8) + flat / 8;
    const int qt = flat % qtiles, pair = flat / qtiles;
    const int h = pair % heads, split = pair / heads;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const int kb0 = split * kb_per_split, kb1 = min(kbs.n_kb, kb0 + kb_per_split);
    const int r32 = lane & 31, g = lane >> 5;
    const int qrow = qt * 32 * WAVES + wave * 32 + r32;
    const bool qlive = qrow < nq;
    const uint8_t *head_images = images + (size_t)h * IS;
    const size_t kb_stride = (size_t)heads * IS;
    // CODES: chunk ci's scales of this head into ring slot ci % 4 (wavefront 0, 48 lanes x 16 bytes)
    auto scales_to_lds = [&](int ci) {
        if (wave == 0 && lane < 48)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint8_t *>(scl + ((size_t)ci * heads + h) * 192 + 4 * lane),
                                             reinterpret_cast<uint8_t *>(&sb[ci & 3][0]), 16, 0, 0);
    };
    // STAGED: block kb's key codes and key factors into staging slot sl; its value codes and value factors
    auto stage_keys = [&](int kb, int sl) { stage_half16<WAVES>(head_images + kb * kb_stride, side + sl * SG, tid); };
    auto stage_values = [&](int kb, int sl) {
        stage_half16<WAVES>(head_images + kb * kb_stride + HALF16, side + sl * SG + HALF16, tid);
    };
    auto convert = [&](int sl, int kdst, int vdst) {
        convert16<WAVES>(side + sl * SG, kdst >= 0 ? kt[kdst] : nullptr, vdst >= 0 ? vt[vdst] : nullptr, tid);
    };
    if (kb0 < kb1) {
        if constexpr (STAGED) {
            // the first two blocks' keys and the first block's values converted here; then the staging slot of
            // step kb0 filled (keys kb0 + 2, values kb0 + 1)
            stage_keys(kb0, 0);
            stage_values(kb0, 0);
            if (kb0 + 1 < kb1) stage_keys(kb0 + 1, 1);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            convert(0, 0, 0);
            if (kb0 + 1 < kb1) convert(1, 1, -1);
            __syncthreads();  // both slots are read before slot 0 is written again
            if (kb0 + 2 < kb1) stage_keys(kb0 + 2, 0);
            if (kb0 + 1 < kb1) stage_values(kb0 + 1, 0);
        } else {
            half_image_to_lds<WAVES, HB>(head_images + kb0 * kb_stride, kt[0], tid);
            half_image_to_lds<WAVES, HB>(head_images + kb0 * kb_stride + HB, vt[0], tid);
            if (kb0 + 1 < kb1) half_image_to_lds<WAVES, HB>(head_images + (kb0 + 1) * kb_stride, kt[1], tid);
        }
        if constexpr (CODES) {
            scales_to_lds(kb0 / kbs.bpc);
            if (kb0 + 1 < kb1 && (kb0 + 1) % kbs.bpc == 0) scales_to_lds((kb0 + 1) / kbs.bpc);
        }
    }

    // this lane's query coordinates 16 dc + 8 g + t, scaled to a maximum magnitude near 2^14 and split
    float qv[4][8];
#pragma unroll
    for (int dc = 0; dc < 4; dc++) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b = a;
        if (qlive) {
            const float *src = q + (size_t)qrow * d + h * 64 + 16 * dc + 8 * g;
            a = *reinterpret_cast<const float4 *>(src);
            b = *reinterpret_cast<const float4 *>(src + 4);
        }
        qv[dc][0] = a.x; qv[dc][1] = a.y; qv[dc][2] = a.z; qv[dc][3] = a.w;
        qv[dc][4] = b.x; qv[dc][5] = b.y; qv[dc][6] = b.z; qv[dc][7] = b.w;
    }
    // the query split into fp16 halves at a maximum near 2^14 (CODES: times chunk ci's key scales first); returns the
    // factor that takes a raw score to score * log2 e
    halfx8 qh[4], ql[4];
    if constexpr (CODES) {
#pragma unroll
        for (int dc = 0; dc < 4; dc++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++)
                *reinterpret_cast<float4 *>(&qraw[wave][((2 * dc + hf) * 64 + lane) * 4]) =
                    make_float4(qv[dc][4 * hf], qv[dc][4 * hf + 1], qv[dc][4 * hf + 2], qv[dc][4 * hf + 3]);
    }
    auto qsplit = [&](int ci) {
        float qs[4][8];
#pragma unroll
        for (int dc = 0; dc < 4; dc++) {
            if constexpr (CODES) {
                float ks[8];
                load8(&sb[ci & 3][16 * dc + 8 * g], ks);
#pragma unroll
                for (int hf = 0; hf < 2; hf++) {
                    const float4 r4 = *reinterpret_cast<const float4 *>(&qraw[wave][((2 * dc + hf) * 64 + lane) * 4]);
                    qs[dc][4 * hf] = r4.x * ks[4 * hf];
                    qs[dc][4 * hf + 1] = r4.y * ks[4 * hf + 1];
                    qs[dc][4 * hf + 2] = r4.z * ks[4 * hf + 2];
                    qs[dc][4 * hf + 3] = r4.w * ks[4 * hf + 3];
                }
            } else {
#pragma unroll
                for (int t = 0; t < 8; t++) qs[dc][t] = qv[dc][t];
            }
        }
        float qmax = 0.0f;
#pragma unroll
        for (int dc = 0; dc < 4; dc++)
#pragma unroll
            for (int t = 0; t < 8; t++) qmax = fmaxf(qmax, fabsf(qs[dc][t]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
        const int eq = shift_for(__float_as_uint(qmax));
#pragma unroll
        for (int dc = 0; dc < 4; dc++) {
            u32x4 hw, lw;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                uint32_t hi, lo;
                split2(ldexpf(qs[dc][2 * t], eq), ldexpf(qs[dc][2 * t + 1], eq), hi, lo);
                hw[t] = hi;
                lw[t] = lo;
            }
            qh[dc] = __builtin_bit_cast(halfx8, hw);
            ql[dc] = __builtin_bit_cast(halfx8, lw);
        }
        return ldexpf(LOG2E, -((CODES ? 0 : shift_for(kvmax[h * 2])) + eq));
    };
    const int sv = CODES ? 0 : shift_for(kvmax[h * 2 + 1]);
    float tl_q = CODES ? 0.0f : qsplit(0);  // CODES: split per chunk, below
    int qchunk = -1;

    // A-operand row of this lane in a 32-key half: key sigma(r32)
    const int krow = sigma32(r32);
    float ref = -INFINITY, l = 0.0f;
    floatx16 acc_o[2];  // CODES: in units of the current chunk's value scales
#pragma unroll
    for (int db = 0; db < 2; db++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc_o[db][v] = 0.0f;
    // CODES: acc_o *= row `which` (1 value scales, 2 ratios) of chunk ci's scales; accumulator v of dim block db holds
    // coordinate 32 db + 8 (v / 4) + 4 g + v % 4
    auto scale_sums = [&](int ci, int which) {
        const float *f = &sb[ci & 3][64 * which];
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int v4 = 0; v4 < 4; v4++) {
                const float4 f4 = *reinterpret_cast<const float4 *>(f + 32 * db + 8 * v4 + 4 * g);
                acc_o[db][4 * v4] *= f4.x;
                acc_o[db][4 * v4 + 1] *= f4.y;
                acc_o[db][4 * v4 + 2] *= f4.z;
                acc_o[db][4 * v4 + 3] *= f4.w;
            }
    };
    floatx16 zero;
#pragma unroll
    for (int v = 0; v < 16; v++) zero[v] = 0.0f;

    // block kb's raw scores: keys past the block's end set to -inf, then the maximum over the query's 64 keys (both
    // halves of the wavefront) in log2 units
    auto mask_and_max = [&](floatx16 (&sc)[2], int kb, float to_log2) {
        const int ci = kb / kbs.bpc;
        const int nk = min(KB, (ci == kbs.n_chunks - 1 ? kbs.last_rc : chunk) - (kb % kbs.bpc) * KB);
        if (nk < KB) {
            const int lim = nk - 8 * g;  // accumulator v of half kh is a key while 32 kh + 16 (v / 8) + v % 8 < lim
#pragma unroll
            for (int kh = 0; kh < 2; kh++)
#pragma unroll
                for (int v = 0; v < 16; v++)
                    if (32 * kh + 16 * (v >> 3) + (v & 7) >= lim) sc[kh][v] = -INFINITY;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int v = 0; v < 16; v++) mb = fmaxf(mb, sc[kh][v]);
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
        return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * to_log2;
    };
    // CODES: the query split for block kb's chunk, if that is not the current split already (outside the products'
    // scheduling regions, so that the split's temporaries are dead before them)
    auto query_for = [&](int kb) {
        if constexpr (CODES) {
            const int ci = kb / kbs.bpc;
            if (ci != qchunk) {
                tl_q = qsplit(ci);
                qchunk = ci;
            }
        }
    };
    // S^T of a block from its key half in LDS, products in the order the operands are read (coordinate step outer);
    // returns the block's raw-score factor
    auto scores = [&](const uint8_t *tile, floatx16 (&sc)[2]) {
        halfx8 khi[4][2], klo[4][2];
#pragma unroll
        for (int dc = 0; dc < 4; dc++)
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
                const int r = 32 * kh + krow;
                const int off = r * 128 + swz(r, 2 * dc + g) * 16;
                khi[dc][kh] = *reinterpret_cast<const halfx8 *>(tile + off);
                if constexpr (!CODES) klo[dc][kh] = *reinterpret_cast<const halfx8 *>(tile + 8192 + off);
            }
#pragma unroll
        for (int dc = 0; dc < 4; dc++)
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
                sc[kh] = mfma16(khi[dc][kh], qh[dc], dc == 0 ? zero : sc[kh]);
                sc[kh] = mfma16(khi[dc][kh], ql[dc], sc[kh]);
                if constexpr (!CODES) sc[kh] = mfma16(klo[dc][kh], qh[dc], sc[kh]);
            }
        return tl_q;
    };
    // step kb: cur holds block kb's scores; with NEXT, block kb + 1's go into nxt
    // step kb: cur holds block kb's scores (raw-score factor tl_cur); with NEXT, block kb + 1's go into nxt (tl_nxt)
    auto step = [&](auto next_flag, floatx16 (&cur)[2], floatx16 (&nxt)[2], float tl_cur, float &tl_nxt, int kb) {
        constexpr bool NEXT = decltype(next_flag)::value;
        const int sl = (kb - kb0) & 1;
        __builtin_amdgcn_s_waitcnt(0);  // this wavefront's copies of keys kb + 1 and values kb have landed
        __syncthreads();                // everyone's have, and step kb - 1's buffers are no longer read
        if constexpr (STAGED) {
            convert(sl, kb + 2 < kb1 ? sl : -1, kb + 1 < kb1 ? (sl ^ 1) : -1);
            if (kb + 3 < kb1) stage_keys(kb + 3, sl ^ 1);
            if (kb + 2 < kb1) stage_values(kb + 2, sl ^ 1);
            __builtin_amdgcn_sched_barrier(0);  // the conversion stays out of the products' scheduling region
        } else {
            if (kb + 2 < kb1) half_image_to_lds<WAVES, HB>(head_images + (kb + 2) * kb_stride, kt[sl], tid);
            if (kb + 1 < kb1) half_image_to_lds<WAVES, HB>(head_images + (kb + 1) * kb_stride + HB, vt[sl ^ 1], tid);
        }
        if constexpr (CODES) {
            if (kb + 2 < kb1 && (kb + 2) % kbs.bpc == 0) scales_to_lds((kb + 2) / kbs.bpc);
            if (kb > kb0 && kb % kbs.bpc == 0) scale_sums(kb / kbs.bpc, 2);  // block kb begins a chunk
        }
        if constexpr (NEXT) query_for(kb + 1);
        const float mb = mask_and_max(cur, kb, tl_cur);
        const bool grow = mb > ref + 3.0f;
        if (__any(grow)) {
            const float nref = grow ? mb : ref;
            const float alpha = exp2_hw(ref - nref);
            l *= alpha;
#pragma unroll
            for (int db = 0; db < 2; db++) acc_o[db] *= alpha;
            ref = nref;
        }
        const float off = 12.0f - ref;
        const float to_log2 = tl_cur;
        if constexpr (NEXT) tl_nxt = scores(kt[sl ^ 1], nxt);
        // block kb's weights, split into fp16 halves for the products
        halfx8 ph[2][2], pl[2][2];
        float ps = 0.0f;
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                u32x4 hw, lw;
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const float p0 = exp2_hw(fmaf(cur[kh][8 * hh + 2 * t], to_log2, off));
                    const float p1 = exp2_hw(fmaf(cur[kh][8 * hh + 2 * t + 1], to_log2, off));
                    ps += p0 + p1;
                    uint32_t hi, lo;
                    split2(p0, p1, hi, lo);
                    hw[t] = hi;
                    lw[t] = lo;
                }
                ph[kh][hh] = __builtin_bit_cast(halfx8, hw);
                pl[kh][hh] = __builtin_bit_cast(halfx8, lw);
            }
        // O^T += V^T P^T over four 16-key steps, in the order the weights are formed
        const uint8_t *vtile = vt[sl];
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int db = 0; db < 2; db++) {
                    const int r = 32 * db + r32;
                    const int voff = r * 128 + swz(r, 4 * kh + 2 * hh + g) * 16;
                    const halfx8 vhi = *reinterpret_cast<const halfx8 *>(vtile + voff);
                    if constexpr (CODES) {
                        acc_o[db] = mfma16(vhi, ph[kh][hh], acc_o[db]);
                        acc_o[db] = mfma16(vhi, pl[kh][hh], acc_o[db]);
                    } else {
                        const halfx8 vlo = *reinterpret_cast<const halfx8 *>(vtile + 8192 + voff);
                        acc_o[db] = mfma16(vhi, ph[kh][hh], acc_o[db]);
                        acc_o[db] = mfma16(vhi, pl[kh][hh], acc_o[db]);
                        acc_o[db] = mfma16(vlo, ph[kh][hh], acc_o[db]);
                    }
                }
        l += ps;
        if constexpr (NEXT && CODES) {
            // one region: 8 key and 8 value operand reads, 16 + 16 products and the weights' VALU work
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
                if (i < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                if (i < 8) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        } else if constexpr (NEXT) {
            // one region: 16 key and 16 value operand reads, 24 + 24 products and the weights' VALU work (their
            // exponents, splits and sum), two VALU operations placed after each product and the rest left to the
            // scheduler (four a product while the scores run, as the loop had with its register copies, measured
            // 2-3% slower a launch: 0.1161 -> 0.1127 ms)
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
            }
#pragma unroll
            for (int i = 0; i < 24; i++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
                if (i < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        }
    };
    if (kb0 < kb1) {
        floatx16 sa[2], sbk[2];
        float ta = 0.0f, tb = 0.0f;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        query_for(kb0);
        ta = scores(kt[0], sa);
        // two steps an iteration, so that the score registers swap roles without copies, and the last one or two
        // blocks after the loop: with an exit between the loop's two steps the compiler kept the weighted sums and
        // the scores in other registers on each side of it and copied them (about 40 moves a step, and spills)
        int kb = kb0;
        for (; kb + 2 < kb1; kb += 2) {
            step(Flag<true>{}, sa, sbk, ta, tb, kb);
            step(Flag<true>{}, sbk, sa, tb, ta, kb + 1);
        }
        if (kb + 1 < kb1) {
            step(Flag<true>{}, sa, sbk, ta, tb, kb);
            step(Flag<false>{}, sbk, sa, tb, ta, kb + 1);
        } else {
            step(Flag<false>{}, sa, sbk, ta, tb, kb);
        }
    }
    if constexpr (CODES)
        if (kb0 < kb1) scale_sums((kb1 - 1) / kbs.bpc, 1);  // into true units: the last chunk's value scales
    // the two halves of the wavefront hold the same queries' sums over different keys (lanes l and l ^ 32)
    {
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
        l = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    // the output's row and lane half again from the thread index, through an opaque copy: not held across the loop
    int tid_e = tid;
    asm volatile("" : "+v"(tid_e));
    const int lane_e = tid_e & 63, g_e = lane_e >> 5;
    const int qrow_e = qt * 32 * WAVES + (tid_e >> 6) * 32 + (lane_e & 31);
    if (qrow_e >= nq) return;
    // accumulator v of dim block db holds coordinate 32 db + 8 (v / 4) + 4 g + v % 4
    const float unscale = ldexpf(1.0f, -sv);
    if (splits == 1) {
        const float f = unscale / l;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int v4 = 0; v4 < 4; v4++)
                *reinterpret_cast<float4 *>(out + (size_t)qrow_e * d + h * 64 + 32 * db + 8 * v4 + 4 * g_e) =
                    make_float4(acc_o[db][4 * v4] * f, acc_o[db][4 * v4 + 1] * f, acc_o[db][4 * v4 + 2] * f,
                                acc_o[db][4 * v4 + 3] * f);
    } else {
        const size_t at = ((size_t)split * nq + qrow_e) * heads + h;
#pragma unroll
        for (int db = 0; db < 2; db++)
#pragma unroll
            for (int v4 = 0; v4 < 4; v4++)
                *reinterpret_cast<float4 *>(part_o + at * 64 + 32 * db + 8 * v4 + 4 * g_e) =
                    make_float4(acc_o[db][4 * v4] * unscale, acc_o[db][4 * v4 + 1] * unscale,
                                acc_o[db][4 * v4 + 2] * unscale, acc_o[db][4 * v4 + 3] * unscale);
        if (g_e == 0) {
            part_ml[at * 2] = ref;
            part_ml[at * 2 + 1] = l;
        }
    }
}

// ---- few-query kernel: head width 64, 1 to FEW_Q queries, over f32 split images or i16 / i8 codes --------------
// grid heads x splits (workgroup i: head i % heads, key range i / heads); 256 threads. With few queries the 32-query
// products of k_attn_split64 leave most of their columns (and whole wavefronts) idle while the kernel waits on
// memory; here the four wavefronts share each 64-key block and split it, wavefront w taking keys 16 w .. 16 w + 15,
// with the queries as the columns of 16 x 16 products, G groups of 16:
//  * S = K Q^T with v_mfma_f32_16x16x32_f16, three products of split halves per 32 coordinates: lane l then holds
//    query 16 g + l % 16 against keys 16 w + 4 (l / 16) + 0..3, which is exactly the B operand of
//  * O^T += V^T P^T with v_mfma_f32_16x16x16_f16 over the wavefront's 16 keys, for four blocks of 16 coordinates.
// The keys' and values' operands are read once a block for all G groups. Each wavefront runs its own online softmax
// over its keys (as k_attn_split64: log2 units, the reference maximum raised when a block passes it by more than 3);
// at the end the four are merged through LDS into the same partials, or output, as k_attn_split64 leaves. The
// blocks stream through a ring of LDS slots by DMA (f32: four 32 KB slots, three blocks in flight while one is used;
// i16 and i8: six 20 KB slots), one barrier a block. Launched for one group (up to 16 queries): with two or four groups (17 to 64 queries) it measured slower
// than k_attn_split64 (f32, 17 / 33 / 64 rows 0.836 / 0.852 / 0.884 -> 0.852 / 0.922 / 0.977 ms a prediction; i8 with
// two groups, 17 / 24 / 32 rows 0.841 / 0.848 / 0.870 -> 0.844 / 0.852 / 0.876 ms), whose 32-query products then have
// work for their columns.
constexpr int FEW_Q = 16;
// i16 code tiles from this many queries: the decode kernel measured faster at one query and slower from two (2 / 3 /
// 4 / 8 / 16 rows 0.625 / 0.692 / 0.763 / 0.798 / 0.877 -> 0.606 / 0.644 / 0.707 / 0.741 / 0.825 ms with this kernel)
constexpr int FEW16_FROM = 2;

typedef _Float16 halfx4 __attribute__((ext_vector_type(4)));

// s_waitcnt immediates that wait for at most n vector-memory operations in flight (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, export and LDS counts left at their maxima)
constexpr int vmcnt_at_most(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// the maximum (sum) of x over lanes l, l ^ 16 (rows of 16 swapped in pairs) and over lanes l, l ^ 32
__device__ __forceinline__ float max16(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float max32(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float sum16(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float sum32(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

template <int G, int FMT>
__global__ __launch_bounds__(256, 1) void k_attn_few(int nq, int rows, int chunk, int d, int heads,
                                                      const float *__restrict__ q, const uint8_t *__restrict__ images,
                                                      const uint32_t *__restrict__ kvmax, const float *__restrict__ scl,
                                                      int kb_per_split, int splits, float *__restrict__ part_o,
                                                      float *__restrict__ part_ml, float *__restrict__ out) {
    // CODES16: the layer's i16 code tiles (16.5 KB, a 20 KB slot), widened, scaled and split as each wavefront reads
    // its operands. CODES8: the layer's i8 code images (16 KB, exact in fp16), each block copied with its chunk's
    // scales after it (key scales, value scales, ratios: 768 bytes, in a 20 KB slot); the scores are two products of
    // the query times the chunk's key scales (split again when a block begins a chunk) with the key codes, the weighted
    // sums two products of the split weights with the value codes, kept in units of the current chunk's value scales
    // (times the ratios when a block begins a chunk, times the last chunk's value scales at the end). Both: six slots,
    // all of a typical range's blocks in flight at once.
    constexpr bool CODES16 = FMT == TAH_KV_I16, CODES8 = FMT == TAH_KV_I8;
    constexpr int TB = img_bytes(FMT), SLOTS = CODES16 || CODES8 ? 6 : 4;
    constexpr int EXTRA = CODES8 ? SCL / 16 : 1;  // copies past the tile: the chunk's scales, or its last 16 bytes again
    constexpr int PER_BLOCK = (TB + (CODES8 ? SCL : 0) + 4095) / 4096, SLOT = 4096 * PER_BLOCK;  // whole rounds
    constexpr int NQ = 16 * G;
    static_assert(4 * 64 * NQ * 4 + 2 * 4 * NQ * 4 <= SLOT * SLOTS, "the merge fits in the ring");
    static_assert((SLOTS - 2) * PER_BLOCK < 64, "the waits' counts fit the counter");
    __shared__ __align__(16) uint8_t ring[SLOTS][SLOT];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qi = lane & 15, lg = lane >> 4;
    const int h = blockIdx.x % heads, split = blockIdx.x / heads;
    const KeyBlocks kbs = key_blocks(rows, chunk);
    const int kb0 = split * kb_per_split, kb1 = min(kbs.n_kb, kb0 + kb_per_split);
    const uint8_t *head_images = images + (size_t)h * TB;
    const size_t kb_stride = (size_t)heads * TB;
    // tile kb into a ring slot: PER_BLOCK copies of 16 bytes a thread, none of them conditional, so that every
    // wavefront's count of copies a block is the same for the waits below; the lanes past the tile copy the block's
    // chunk's scales (CODES8) or the tile's last 16 bytes again, the ones past those the last 16 bytes of them again,
    // into the slot's padding. Over code tiles the compiler also waits for every copy in flight before the loop's
    // first LDS read (its own wait, not one of the waits below): all of a range's blocks (five, typically) are then
    // in flight from the start
    auto tile_to_lds = [&](int kb, uint8_t *slot) {
        const uint4 *src = reinterpret_cast<const uint4 *>(head_images + kb * kb_stride);
        const uint4 *extra = src + TB / 16 - 1;
        if constexpr (CODES8) extra = reinterpret_cast<const uint4 *>(scl + ((size_t)(kb / kbs.bpc) * heads + h) * 192);
#pragma unroll
        for (int i = 0; i < PER_BLOCK; i++) {
            const int base = 256 * i + 64 * wave, at = base + lane;
            const uint4 *p = at < TB / 16 ? src + at : extra + min(at - TB / 16, EXTRA - 1);
            __builtin_amdgcn_global_load_lds(p, slot + 16 * base, 16, 0, 0);
        }
    };

    // query 16 g + qi's coordinates 32 ks + 8 lg + t (the B operand of the scores), loaded without a branch (a lane
    // past the last query reads query 0 and zeroes it), then the first blocks' copies issued
    float4 raw[G][4];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float *src = q + (size_t)min(16 * g + qi, nq - 1) * d + h * 64 + 8 * lg;
#pragma unroll
        for (int j = 0; j < 4; j++) raw[g][j] = *reinterpret_cast<const float4 *>(src + 32 * (j >> 1) + 4 * (j & 1));
    }
#pragma unroll
    for (int i = 0; i < SLOTS - 1; i++)
        if (kb0 + i < kb1) tile_to_lds(kb0 + i, ring[i]);
    // each query (CODES8: times the chunk's key scales ksc, at coordinates 32 ks + 8 lg + t) scaled to a maximum near
    // 2^14 and split
    float qraw[G][2][8];
#pragma unroll
    for (int g = 0; g < G; g++) {
        const float live = 16 * g + qi < nq ? 1.0f : 0.0f;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            const float4 a = raw[g][2 * ks], b = raw[g][2 * ks + 1];
            qraw[g][ks][0] = a.x * live; qraw[g][ks][1] = a.y * live; qraw[g][ks][2] = a.z * live;
            qraw[g][ks][3] = a.w * live; qraw[g][ks][4] = b.x * live; qraw[g][ks][5] = b.y * live;
            qraw[g][ks][6] = b.z * live; qraw[g][ks][7] = b.w * live;
        }
    }
    halfx8 qh[G][2], ql[G][2];
    float to_log2[G];
    const int sk = CODES8 ? 0 : shift_for(kvmax[h * 2]), sv = CODES8 ? 0 : shift_for(kvmax[h * 2 + 1]);
    auto split_queries = [&](const float *ksc) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            float qv[2][8];
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                float f[8];
                if constexpr (CODES8) load8(ksc + 32 * ks + 8 * lg, f);
#pragma unroll
                for (int t = 0; t < 8; t++) qv[ks][t] = CODES8 ? qraw[g][ks][t] * f[t] : qraw[g][ks][t];
            }
            float qmax = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
#pragma unroll
                for (int t = 0; t < 8; t++) qmax = fmaxf(qmax, fabsf(qv[ks][t]));
            const int eq = shift_for_max(max32(max16(qmax)));
#pragma unroll
            for (int ks = 0; ks < 2; ks++) split8(qv[ks], ldexpf(1.0f, eq), qh[g][ks], ql[g][ks]);
            to_log2[g] = ldexpf(LOG2E, -(sk + eq));
        }
    };
    if constexpr (!CODES8) split_queries(nullptr);

    float ref[G], l[G];
    floatx4 acc[G][4];  // O^T: coordinate 16 m + 4 lg + i of query 16 g + qi, in units of 2^sv (CODES8: of the chunk's
                        // value scales)
#pragma unroll
    for (int g = 0; g < G; g++) {
        ref[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; m++) acc[g][m] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const int krow = 16 * wave + (lane & 15);                      // the scores' A row: key krow
    const int vchunk = 2 * wave + (lg >> 1), voff = 8 * (lg & 1);  // the values' A operand: keys 16 wave + 4 lg + ..
    for (int kb = kb0; kb < kb1; kb++) {
        // block kb's copies have landed (the ones after it may still be in flight), everyone's, and everyone is done
        // with block kb - 1, whose slot the copy of block kb + SLOTS - 1 then takes
        const int ahead = min(kb1 - 1, kb + SLOTS - 2) - kb;
        switch (ahead) {
            case 0: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(0)); break;
            case 1: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(PER_BLOCK)); break;
            case 2: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(2 * PER_BLOCK)); break;
            case 3: __builtin_amdgcn_s_waitcnt(vmcnt_at_most(3 * PER_BLOCK)); break;
            default: __builtin_amdgcn_s_waitcnt(vmcnt_at_most((SLOTS - 2) * PER_BLOCK)); break;
        }
        __syncthreads();
        if (kb + SLOTS - 1 < kb1)
            tile_to_lds(kb + SLOTS - 1, ring[(kb + SLOTS - 1 - kb0) % SLOTS]);
        const int ci = kb / kbs.bpc;
        const int nk = min(KB, (ci == kbs.n_chunks - 1 ? kbs.last_rc : chunk) - (kb % kbs.bpc) * KB);
        const uint8_t *img = ring[(kb - kb0) % SLOTS];
        if constexpr (CODES8) {
            // a block that begins the range or a chunk: the sums into this chunk's value units (after the first), the
            // queries split with its key scales (every wavefront, whether or not its keys are past the block's end)
            const float *sct = reinterpret_cast<const float *>(img + TB);
            if (kb == kb0 || kb % kbs.bpc == 0) {
                if (kb > kb0) {
#pragma unroll
                    for (int m = 0; m < 4; m++) {
                        const float4 r4 = *reinterpret_cast<const float4 *>(sct + 128 + 16 * m + 4 * lg);
#pragma unroll
                        for (int g = 0; g < G; g++) acc[g][m] *= floatx4{r4.x, r4.y, r4.z, r4.w};
                    }
                }
                split_queries(sct);
            }
        }
        if (16 * wave >= nk) continue;  // this wavefront's keys are all past the block's end
        halfx8 khi[2], klo[2];
        halfx4 vhi[4], vlo[4];
        if constexpr (CODES8) {
            // the codes as they are (exact in fp16): one plane each, laid out as the f32 images' high planes
#pragma unroll
            for (int ks = 0; ks < 2; ks++)
                khi[ks] = *reinterpret_cast<const halfx8 *>(img + krow * 128 + swz(krow, 4 * ks + lg) * 16);
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int r = 16 * m + (lane & 15);
                vhi[m] = *reinterpret_cast<const halfx4 *>(img + 8192 + r * 128 + swz(r, vchunk) * 16 + voff);
            }
        } else if constexpr (CODES16) {
            // key krow's codes at coordinates 32 ks + 8 lg + 0..7 times their factors; coordinate 16 m + lane % 16's
            // codes of keys 16 wave + 4 lg + 0..3 times its factor (the tile's rows are not swizzled)
            const float *kf = reinterpret_cast<const float *>(img + 8192);
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                float f[8];
                load8(kf + 32 * ks + 8 * lg, f);
                dequant_split8(*reinterpret_cast<const uint4 *>(img + krow * 128 + (4 * ks + lg) * 16), f, khi[ks], klo[ks]);
            }
            const uint8_t *vt = img + HALF16;
            const float *vf = reinterpret_cast<const float *>(vt + 8192);
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int r = 16 * m + (lane & 15);
                const uint2 c = *reinterpret_cast<const uint2 *>(vt + r * 128 + 32 * wave + 8 * lg);
                const float fv = vf[r];
                uint32_t h01, l01, h23, l23;
                split2((float)(int16_t)(c.x & 0xffffu) * fv, (float)(int16_t)(c.x >> 16) * fv, h01, l01);
                split2((float)(int16_t)(c.y & 0xffffu) * fv, (float)(int16_t)(c.y >> 16) * fv, h23, l23);
                vhi[m] = __builtin_bit_cast(halfx4, make_uint2(h01, h23));
                vlo[m] = __builtin_bit_cast(halfx4, make_uint2(l01, l23));
            }
        } else {
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                const int off = krow * 128 + swz(krow, 4 * ks + lg) * 16;
                khi[ks] = *reinterpret_cast<const halfx8 *>(img + off);
                klo[ks] = *reinterpret_cast<const halfx8 *>(img + 8192 + off);
            }
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int r = 16 * m + (lane & 15);
                const int vo = r * 128 + swz(r, vchunk) * 16 + voff;
                vhi[m] = *reinterpret_cast<const halfx4 *>(img + 16384 + vo);
                vlo[m] = *reinterpret_cast<const halfx4 *>(img + 24576 + vo);
            }
        }
        floatx4 sc[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            sc[g] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                sc[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi[ks], qh[g][ks], sc[g], 0, 0, 0);
                sc[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(khi[ks], ql[g][ks], sc[g], 0, 0, 0);
                if constexpr (!CODES8) sc[g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(klo[ks], qh[g][ks], sc[g], 0, 0, 0);
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++) {
            if (nk < KB) {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (16 * wave + 4 * lg + i >= nk) sc[g][i] = -INFINITY;
            }
            const float mb = max32(max16(fmaxf(fmaxf(sc[g][0], sc[g][1]), fmaxf(sc[g][2], sc[g][3])))) * to_log2[g];
            const bool grow = mb > ref[g] + 3.0f;
            if (__any(grow)) {
                const float nref = grow ? mb : ref[g];
                const float alpha = exp2_hw(ref[g] - nref);
                l[g] *= alpha;
#pragma unroll
                for (int m = 0; m < 4; m++) acc[g][m] *= alpha;
                ref[g] = nref;
            }
            const float off = 12.0f - ref[g];
            float p[4];
#pragma unroll
            for (int i = 0; i < 4; i++) p[i] = exp2_hw(fmaf(sc[g][i], to_log2[g], off));
            l[g] += (p[0] + p[1]) + (p[2] + p[3]);
            uint32_t h01, l01, h23, l23;
            split2(p[0], p[1], h01, l01);
            split2(p[2], p[3], h23, l23);
            const halfx4 ph = __builtin_bit_cast(halfx4, make_uint2(h01, h23));
            const halfx4 pl = __builtin_bit_cast(halfx4, make_uint2(l01, l23));
#pragma unroll
            for (int m = 0; m < 4; m++) {
                acc[g][m] = __builtin_amdgcn_mfma_f32_16x16x16f16(vhi[m], ph, acc[g][m], 0, 0, 0);
                acc[g][m] = __builtin_amdgcn_mfma_f32_16x16x16f16(vhi[m], pl, acc[g][m], 0, 0, 0);
                if constexpr (!CODES8) acc[g][m] = __builtin_amdgcn_mfma_f32_16x16x16f16(vlo[m], ph, acc[g][m], 0, 0, 0);
            }
        }
    }

    if constexpr (CODES8) {
        // the sums into true units: the last block's chunk's value scales (its slot is intact until the barrier below)
        const float *sct = reinterpret_cast<const float *>(ring[(kb1 - 1 - kb0) % SLOTS] + TB);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const float4 v4 = *reinterpret_cast<const float4 *>(sct + 64 + 16 * m + 4 * lg);
#pragma unroll
            for (int g = 0; g < G; g++) acc[g][m] *= floatx4{v4.x, v4.y, v4.z, v4.w};
        }
    }
    // the four wavefronts' (maximum, sum, weighted sums) through LDS (the ring is free: the last block's wait was for
    // every copy), merged as the split merge merges key ranges
    __syncthreads();
    float *mref = reinterpret_cast<float *>(&ring[0][0]);  // [wavefront][query]
    float *msum = mref + 4 * NQ;                           // [wavefront][query]
    float *macc = msum + 4 * NQ;                           // [wavefront][coordinate][query]
#pragma unroll
    for (int g = 0; g < G; g++) {
        // the query's weight sum over the wavefront's keys (lanes l, l ^ 16, l ^ 32, l ^ 48 hold query 16 g + l % 16)
        const float lw = sum32(sum16(l[g]));
        if (lg == 0) {
            mref[wave * NQ + 16 * g + qi] = ref[g];
            msum[wave * NQ + 16 * g + qi] = lw;
        }
#pragma unroll
        for (int m = 0; m < 4; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) macc[(wave * 64 + 16 * m + 4 * lg + i) * NQ + 16 * g + qi] = acc[g][m][i];
    }
    __syncthreads();
    // thread t: queries t / 16 + 16 g, coordinates 4 (t % 16) .. + 3
    const int oc = 4 * (tid & 15);
    const float unscale = ldexpf(1.0f, -sv);
#pragma unroll
    for (int g = 0; g < G; g++) {
        const int oq = (tid >> 4) + 16 * g;
        if (oq >= nq) break;
        float m = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; w++)
            if (msum[w * NQ + oq] > 0.0f) m = fmaxf(m, mref[w * NQ + oq]);
        float L = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const float ls = msum[w * NQ + oq];
            const float f = ls > 0.0f ? exp2_hw(mref[w * NQ + oq] - m) : 0.0f;
            L += ls * f;
#pragma unroll
            for (int j = 0; j < 4; j++) o[j] += macc[(w * 64 + oc + j) * NQ + oq] * f;
        }
        if (splits == 1) {
            const float fo = unscale / L;
            *reinterpret_cast<float4 *>(out + (size_t)oq * d + h * 64 + oc) =
                make_float4(o[0] * fo, o[1] * fo, o[2] * fo, o[3] * fo);
        } else {
            const size_t at = ((size_t)split * nq + oq) * heads + h;
            *reinterpret_cast<float4 *>(part_o + at * 64 + oc) =
                make_float4(o[0] * unscale, o[1] * unscale, o[2] * unscale, o[3] * unscale);
            if (oc == 0) {
                part_ml[at * 2] = m;
                part_ml[at * 2 + 1] = L;
            }
        }
    }
}

// ---- split merge: Soft::merge then Soft::finish ---------------------------------------------------------------
// grid nq * heads; 64 threads. The largest running maximum first (lanes over splits), then one pass over the
// splits accumulating each one's weight sum and weighted values rescaled to it; loads are independent across
// splits, so they stream. Maxima are in log2 units when log2_units is set, natural units otherwise.
__global__ __launch_bounds__(64) void k_attn_merge(int nq, int d, int heads, int splits, int log2_units,
                                                    const float *__restrict__ part_o,
                                                    const float *__restrict__ part_ml, float *__restrict__ out) {
    const int item = blockIdx.x, lane = threadIdx.x;
    const int qr = item / heads, h = item % heads, hd = d / heads;
    const size_t stride = (size_t)nq * heads;  // between splits, in (query, head) items
    const size_t base = (size_t)qr * heads + h;
    float M = -INFINITY;
    for (int s = lane; s < splits; s += 64) {
        const size_t at = s * stride + base;
        if (part_ml[at * 2 + 1] > 0.0f) M = fmaxf(M, part_ml[at * 2]);
    }
    M = wave_max(M);
    for (int c = lane; c < hd; c += 64) {
        float L = 0.0f, O = 0.0f;
#pragma unroll 8
        for (int s = 0; s < splits; s++) {
            const size_t at = s * stride + base;
            const float ls = part_ml[at * 2 + 1];
            const float dm = part_ml[at * 2] - M;
            const float f = ls > 0.0f ? (log2_units ? exp2_hw(dm) : fast_exp(dm)) : 0.0f;
            L += ls * f;
            O += part_o[at * hd + c] * f;
        }
        out[(size_t)qr * d + h * hd + c] = O / L;
    }
}

constexpr int MERGE64_MAX = 16;  // k_attn_merge64 takes at most this many key ranges

// Head width 64, maxima in log2 units: 16 threads per (query, head), four coordinates each, every split's (m, l) and
// partial sums loaded independently (one wave of loads in flight, not a chain).
__global__ __launch_bounds__(256) void k_attn_merge64(int items, int heads, int splits, const float *__restrict__ part_o,
                                                      const float *__restrict__ part_ml, float *__restrict__ out) {
    const int i = blockIdx.x * 16 + (threadIdx.x >> 4), c4 = (threadIdx.x & 15) * 4;
    if (i >= items) return;
    const size_t stride = (size_t)items;  // between splits, in (query, head) items
    // all loads issued before any value is used (a loop over the ranges had each range's loads wait for the last's)
    float2 ml[MERGE64_MAX];
    float4 po[MERGE64_MAX];
#pragma unroll
    for (int sp = 0; sp < MERGE64_MAX; sp++)
        if (sp < splits) {
            const size_t at = sp * stride + i;
            ml[sp] = *reinterpret_cast<const float2 *>(part_ml + at * 2);
            po[sp] = *reinterpret_cast<const float4 *>(part_o + at * 64 + c4);
        }
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < MERGE64_MAX; sp++)
        if (sp < splits && ml[sp].y > 0.0f) M = fmaxf(M, ml[sp].x);
    float L = 0.0f;
    float4 O = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int sp = 0; sp < MERGE64_MAX; sp++)
        if (sp < splits) {
            const float f = ml[sp].y > 0.0f ? exp2_hw(ml[sp].x - M) : 0.0f;
            L += ml[sp].y * f;
            O.x += po[sp].x * f;
            O.y += po[sp].y * f;
            O.z += po[sp].z * f;
            O.w += po[sp].w * f;
        }
    const int qr = i / heads, h = i - qr * heads;
    *reinterpret_cast<float4 *>(out + ((size_t)qr * heads + h) * 64 + c4) = make_float4(O.x / L, O.y / L, O.z / L, O.w / L);
}

// Split merge for head width 64 and many key ranges: a wavefront per (query, head), four a workgroup, lane =
// coordinate; its ranges in passes of MWW with every load of a pass issued before the sums, no LDS (64 queries x 8
// heads over 32 ranges: 3.9 us, where a 1,024-thread workgroup per (query, head) combining its wavefronts through
// LDS took 7.6 us).
constexpr int MWW = 16;
__global__ __launch_bounds__(256) void k_attn_merge_w(int items, int splits, const float *__restrict__ part_o,
                                                      const float *__restrict__ part_ml, float *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (i >= items) return;
    const size_t stride = (size_t)items;  // between splits, in (query, head) items
    float M = -INFINITY, L = 0.0f, O = 0.0f;
    for (int s0 = 0; s0 < splits; s0 += MWW) {
        float2 ml[MWW];
        float po[MWW];
#pragma unroll
        for (int u = 0; u < MWW; u++) {
            // past the last range: its own values reread (in bounds) and given no weight
            const size_t at = (size_t)min(s0 + u, splits - 1) * stride + i;
            ml[u] = *reinterpret_cast<const float2 *>(part_ml + at * 2);
            po[u] = part_o[at * 64 + lane];
            if (s0 + u >= splits) ml[u] = make_float2(-INFINITY, 0.0f);
        }
        float cm = M;
#pragma unroll
        for (int u = 0; u < MWW; u++)
            if (ml[u].y > 0.0f) cm = fmaxf(cm, ml[u].x);
        const float r = M == -INFINITY ? 0.0f : exp2_hw(M - cm);
        L *= r;
        O *= r;
        M = cm;
#pragma unroll
        for (int u = 0; u < MWW; u++) {
            const float f = ml[u].y > 0.0f ? exp2_hw(ml[u].x - M) : 0.0f;
            L += ml[u].y * f;
            O += po[u] * f;
        }
    }
    out[(size_t)i * 64 + lane] = O / L;
}

void merge_splits(hipStream_t s, int nq, int d, int heads, int splits, const float *part_o, const float *part_ml,
                  float *out) {
    hipLaunchKernelGGL(k_attn_merge, dim3(nq * heads), dim3(64), 0, s, nq, d, heads, splits, 0, part_o, part_ml, out);
    TAH_LAUNCHED();
}

// ---- planning and launch --------------------------------------------------------------------------------------
struct AttnPlan {
    bool split16, few;  // few: k_attn_few (any tiles, at most FEW_Q queries; i16 from FEW16_FROM)
    int splits, kb_per_split, groups, waves;
};

bool kv_images_apply(int kv_format, int d, int heads) {
    return kv_format >= TAH_KV_F32 && kv_format <= TAH_KV_I8 && heads > 0 && d == 64 * heads;
}

// The tiles, then (256-aligned) a 256-byte slot for f32 and i16's maxima, then the i8 scales.
size_t kv_images_bytes(int rows, int chunk, int heads, int kv_format) {
    const size_t chunks = key_blocks(rows, chunk).n_chunks;
    const size_t tail = kv_format == TAH_KV_I8 ? chunks * heads * SCL : 0;
    return ((image_bytes_of(rows, chunk, heads, kv_format) + 255) / 256) * 256 +
           ((sizeof(uint32_t) * 2 * (size_t)heads + 255) / 256) * 256 + tail;
}

template <int FMT>
static void launch_absmax(hipStream_t s, int rows, int chunk, int d, int heads, const uint8_t *records, KvImages img) {
    const KeyBlocks k = key_blocks(rows, chunk);
    hipLaunchKernelGGL(k_zero_u32, dim3((2 * heads + 63) / 64), dim3(64), 0, s, 2 * heads, img.kvmax);
    TAH_LAUNCHED();
    hipLaunchKernelGGL(k_kv_absmax<FMT>, dim3(k.n_kb, heads), dim3(256), 0, s, rows, chunk, d, heads, records, img.kvmax);
    TAH_LAUNCHED();
}

void kv_images(hipStream_t s, int rows, int chunk, int d, int heads, int kv_format, const uint8_t *records,
               KvImages img) {
    if (!kv_images_apply(kv_format, d, heads)) throw ArgError{"key/value tiles need head width 64"};
    if (kv_format != img.fmt) throw ArgError{"key/value tiles: laid out for another format"};
    const KeyBlocks k = key_blocks(rows, chunk);
    switch (kv_format) {
        case TAH_KV_F32:
            launch_absmax<TAH_KV_F32>(s, rows, chunk, d, heads, records, img);
            hipLaunchKernelGGL(k_kv_images<TAH_KV_F32>, dim3(k.n_kb, heads), dim3(256), 0, s, rows, chunk, d, heads,
                               records, img.kvmax, img.images);
            break;
        case TAH_KV_I16:
            launch_absmax<TAH_KV_I16>(s, rows, chunk, d, heads, records, img);
            hipLaunchKernelGGL(k_kv_tiles16, dim3(k.n_kb, heads), dim3(256), 0, s, rows, chunk, d, heads, records,
                               img.kvmax, img.images);
            break;
        default:
            hipLaunchKernelGGL(k_kv_codes, dim3(k.n_kb, heads), dim3(256), 0, s, rows, chunk, d, heads, records,
                               img.images, img.scales);
            break;
    }
    TAH_LAUNCHED();
}

KvImages kv_images_at(uint8_t *base, int rows, int chunk, int heads, int kv_format) {
    KvImages img;
    img.fmt = kv_format;
    img.images = base;
    uint8_t *tail = base + ((image_bytes_of(rows, chunk, heads, kv_format) + 255) / 256) * 256;
    img.kvmax = reinterpret_cast<uint32_t *>(tail);
    if (kv_format == TAH_KV_I8)
        img.scales = reinterpret_cast<float *>(tail + ((sizeof(uint32_t) * 2 * (size_t)heads + 255) / 256) * 256);
    return img;
}

static AttnPlan plan(const AttnShape &a, bool images) {
    AttnPlan p;
    const KeyBlocks k = key_blocks(a.rows, a.chunk);
    const int hd = a.d / a.heads;
    const bool tiles = hd == 64 && images && kv_images_apply(a.kv_format, a.d, a.heads);
    p.few = tiles && a.nq <= FEW_Q && (a.kv_format != TAH_KV_I16 || a.nq >= FEW16_FROM);
    p.split16 = tiles && (p.few || a.nq >= split16_min_q(a.kv_format));
    // k_attn_split64: 256 queries a workgroup (one a compute unit, one wave of them) from 768 queries on, else 128
    // (at 512 / 640 rows f32 1.376 / 1.740 -> 1.368 / 1.717 ms and i8 1.337 / 1.705 -> 1.330 / 1.676 ms with the
    // smaller tiles than from 512; from 1,024 or 1,536 queries f32 was slower at 768 to 1,280); an i16 layer's (whose
    // staging takes 33 KB of LDS more, one workgroup a compute unit) 256 from 129 queries on, and 128 for one tile of
    // up to 128 queries (its wavefronts without live queries then do not share the SIMDs: 4 / 16 / 64 rows 0.771 /
    // 0.882 / 0.931 -> 0.762 / 0.877 / 0.928 ms; at 256 and 384 rows four wavefronts were 4.5% slower)
    const int eight_from = a.kv_format == TAH_KV_I16 ? 129 : 768;
    p.waves = p.split16 && a.nq >= eight_from ? 8 : 4;
    const int per_group = p.split16 ? 32 * p.waves : QG;
    p.groups = (a.nq + per_group - 1) / per_group;
    // enough workgroups to fill the 256 compute units about once, each with at least 2 key blocks: more, shorter key
    // ranges measured slower at every batch (the merge and each workgroup's fixed costs grow with them; 64 queries:
    // 22 us at 256 workgroups against 36 at 632; f32 tiles at two workgroups a compute unit for two or more 128-query
    // tiles, up to 32 ranges: 256 / 384 rows 1.122 / 1.338 ms against 1.097 / 1.291 ms at one, whose 16 or fewer
    // ranges k_attn_merge64 takes). The i8 code images, half the products and bytes a block, keep two workgroups a
    // compute unit there (at one, 160-448 rows took 2-4% longer).
    if (!p.split16 && hd == 64) {
        // the decode kernel's wavefronts each take a key block of their own: six blocks a workgroup, two of its four
        // wavefronts taking a second (fewer ranges for the merge: an i16 row 0.583 -> 0.556 ms, two rows 0.640 ->
        // 0.621 ms against four blocks; three rows unchanged; 8 / 12 / 16 blocks slower)
        p.kb_per_split = std::min(6, k.n_kb);
        p.splits = (k.n_kb + p.kb_per_split - 1) / p.kb_per_split;
        return p;
    }
    const long target = p.waves == 4 && p.groups > 1 && a.kv_format == TAH_KV_I8 ? 512 : 256;
    // the key ranges: the count whose rounds of workgroups times (blocks per range + 2, a workgroup's fixed cost in
    // blocks: its queries' load and split, its partials, their share of the merge) is least, the fewest ranges of
    // equal cost (768 queries: 10 ranges, 240 workgroups in one round, where 11 made 264, a second round of 8; the
    // fit's 10,000 queries: 4 ranges, 5 rounds of 40 blocks, where one range made 320 workgroups, 2 rounds of 157;
    // without the fixed cost the count would grow to 32 ranges of 5 blocks at 768 queries, which measured slower)
    const long per = (long)p.groups * a.heads, most = std::max(1L, (long)(k.n_kb + 1) / 2);
    auto cost = [&](long s) { return ((per * s + target - 1) / target) * ((k.n_kb + s - 1) / s + 2); };
    long want = 1;
    for (long s = 2; s <= most; s++)
        if (cost(s) < cost(want)) want = s;
    p.kb_per_split = (int)((k.n_kb + want - 1) / want);
    p.splits = (k.n_kb + p.kb_per_split - 1) / p.kb_per_split;
    return p;
}

// Callers hand a layer of head width 64 over as tiles from TAH_SPLIT16_MIN_Q queries on (a fitted model's layers at
// any query count), and attention() refuses such a shape without them: the plan below is the one that runs.
static bool images_expected(const AttnShape &a) {
    return a.nq >= TAH_SPLIT16_MIN_Q && kv_images_apply(a.kv_format, a.d, a.heads);
}

// Room for the split partials of whichever plan runs: over tiles where they apply (a fitted layer of head width 64 is
// read as tiles at any query count), or below TAH_SPLIT16_MIN_Q queries also over records (a transient layer).
size_t attention_work_bytes(const AttnShape &a) {
    const bool tiles = kv_images_apply(a.kv_format, a.d, a.heads);
    int splits = plan(a, tiles).splits;
    if (!images_expected(a)) splits = std::max(splits, plan(a, false).splits);
    if (splits == 1) return 0;
    const int hd = a.d / a.heads;
    return sizeof(float) * (size_t)splits * a.nq * a.heads * (hd + 2) + 256;
}

template <int FMT>
static void launch(hipStream_t s, const AttnShape &a, const AttnPlan &p, const float *q, const uint8_t *records,
                   const KvImages *img, float *out, float *part_o, float *part_ml) {
    if (img) {
        hipLaunchKernelGGL((k_attn_decode_w<FMT, true>), dim3(p.splits, a.heads, p.groups), dim3(256), 0, s, a.nq,
                           a.rows, a.chunk, a.d, a.heads, q, img->images, img->kvmax, img->scales, p.kb_per_split,
                           part_o, part_ml, out);
    } else if (a.d / a.heads == 64) {
        hipLaunchKernelGGL((k_attn_decode_w<FMT, false>), dim3(p.splits, a.heads, p.groups), dim3(256), 0, s, a.nq,
                           a.rows, a.chunk, a.d, a.heads, q, records, nullptr, nullptr, p.kb_per_split, part_o,
                           part_ml, out);
    } else {
        hipLaunchKernelGGL(k_attn_decode<FMT>, dim3(p.splits, a.heads, p.groups), dim3(64), 0, s, a.nq, a.rows, a.chunk,
                           a.d, a.heads, q, records, p.kb_per_split, part_o, part_ml, out);
    }
    TAH_LAUNCHED();
}

template <int WAVES, int FMT>
static void launch_split(hipStream_t s, const AttnShape &a, const AttnPlan &p, const float *q, const KvImages &img,
                         float *out, float *part_o, float *part_ml) {
    hipLaunchKernelGGL((k_attn_split64<WAVES, FMT>), dim3(p.groups * a.heads * p.splits), dim3(64 * WAVES), 0, s, a.nq,
                       a.rows, a.chunk, a.d, a.heads, q, img.images, img.kvmax, img.scales, p.kb_per_split, p.groups,
                       p.splits, part_o, part_ml, out);
    TAH_LAUNCHED();
}

// ---- launch probe ---------------------------------------------------------------------------------------------------
// While armed for a stream, each launch of the many-query kernel (k_attn_split64) on it is bracketed by a pair of HIP
// events, up to the armed number of launches; probe_read sums their elapsed times. One probe per process.
namespace {
std::mutex probe_mu;
std::atomic<bool> probe_on{false};
hipStream_t probe_stream = nullptr;
std::vector<hipEvent_t> probe_ev;
int probe_used = 0;

void probe_free() {
    for (hipEvent_t e : probe_ev) (void)hipEventDestroy(e);
    probe_ev.clear();
    probe_used = 0;
    probe_stream = nullptr;
    probe_on = false;
}

// the next unused pair of events if the probe is armed for s, else null
hipEvent_t *probe_slot(hipStream_t s) {
    if (!probe_on.load(std::memory_order_relaxed)) return nullptr;
    std::lock_guard<std::mutex> lk(probe_mu);
    if (s != probe_stream || 2 * (probe_used + 1) > (int)probe_ev.size()) return nullptr;
    return &probe_ev[2 * probe_used++];
}
}  // namespace

void probe_arm(hipStream_t s, int launches) {
    std::lock_guard<std::mutex> lk(probe_mu);
    probe_free();
    if (launches <= 0) return;
    probe_ev.resize(2 * (size_t)launches);
    for (size_t i = 0; i < probe_ev.size(); i++) {
        if (hipEventCreate(&probe_ev[i]) != hipSuccess) {
            probe_ev.resize(i);
            probe_free();
            throw ArgError{"probe: cannot create its events"};
        }
    }
    probe_stream = s;
    probe_on = true;
}

int probe_read(hipStream_t s, double *ms) {
    std::lock_guard<std::mutex> lk(probe_mu);
    if (!probe_on || s != probe_stream) throw ArgError{"probe: not armed for this device"};
    TAH_HIP(hipStreamSynchronize(s));
    double total = 0.0;
    for (int i = 0; i < probe_used; i++) {
        float t = 0.0f;
        TAH_HIP(hipEventElapsedTime(&t, probe_ev[2 * i], probe_ev[2 * i + 1]));
        total += t;
    }
    *ms = total;
    const int n = probe_used;
    probe_used = 0;
    return n;
}

void attention(hipStream_t s, const AttnShape &a, const float *q, const uint8_t *records, float *out, void *work,
               const KvImages *img) {
    if (a.nq <= 0) return;
    const int hd = a.d / a.heads;
    if (a.d % a.heads != 0 || hd > 64 || a.rows <= 0 || a.chunk <= 0)
        throw ArgError{"attention: head width must divide d and be at most 64, rows and chunk positive"};
    if ((size_t)a.nq > (size_t)65535 * 8) throw ArgError{"attention: too many queries for one launch"};
    const bool have = img != nullptr && img->images != nullptr;
    if (images_expected(a) && !have) throw ArgError{"attention: head width 64 from 4 queries on needs the tiles"};
    if (have && (img->fmt != a.kv_format || !kv_images_apply(a.kv_format, a.d, a.heads)))
        throw ArgError{"attention: tiles of another cache format or shape"};
    if (!have && !records) throw ArgError{"attention: neither records nor tiles"};
    const AttnPlan p = plan(a, have);
    float *part_o = nullptr, *part_ml = nullptr;
    if (p.splits > 1) {
        part_o = static_cast<float *>(work);
        part_ml = part_o + (size_t)p.splits * a.nq * a.heads * hd;
    }
    if (p.few) {
        const dim3 grid(a.heads * p.splits);
        if (a.kv_format == TAH_KV_I16)
            hipLaunchKernelGGL((k_attn_few<FEW_Q / 16, TAH_KV_I16>), grid, dim3(256), 0, s, a.nq, a.rows, a.chunk, a.d,
                               a.heads, q, img->images, img->kvmax, img->scales, p.kb_per_split, p.splits, part_o,
                               part_ml, out);
        else if (a.kv_format == TAH_KV_I8)
            hipLaunchKernelGGL((k_attn_few<FEW_Q / 16, TAH_KV_I8>), grid, dim3(256), 0, s, a.nq, a.rows, a.chunk, a.d,
                               a.heads, q, img->images, img->kvmax, img->scales, p.kb_per_split, p.splits, part_o,
                               part_ml, out);
        else
            hipLaunchKernelGGL((k_attn_few<FEW_Q / 16, TAH_KV_F32>), grid, dim3(256), 0, s, a.nq, a.rows, a.chunk, a.d,
                               a.heads, q, img->images, img->kvmax, img->scales, p.kb_per_split, p.splits, part_o,
                               part_ml, out);
        TAH_LAUNCHED();
    } else if (p.split16) {
        hipEvent_t *pe = probe_slot(s);
        if (pe) TAH_HIP(hipEventRecord(pe[0], s));
        switch (a.kv_format) {
            case TAH_KV_F32:
                if (p.waves == 8) launch_split<8, TAH_KV_F32>(s, a, p, q, *img, out, part_o, part_ml);
                else launch_split<4, TAH_KV_F32>(s, a, p, q, *img, out, part_o, part_ml);
                break;
            case TAH_KV_I16:
                if (p.waves == 8) launch_split<8, TAH_KV_I16>(s, a, p, q, *img, out, part_o, part_ml);
                else launch_split<4, TAH_KV_I16>(s, a, p, q, *img, out, part_o, part_ml);
                break;
            default:
                if (p.waves == 8) launch_split<8, TAH_KV_I8>(s, a, p, q, *img, out, part_o, part_ml);
                else launch_split<4, TAH_KV_I8>(s, a, p, q, *img, out, part_o, part_ml);
                break;
        }
        if (pe) TAH_HIP(hipEventRecord(pe[1], s));
    } else switch (a.kv_format) {
        case TAH_KV_F32: launch<TAH_KV_F32>(s, a, p, q, records, have ? img : nullptr, out, part_o, part_ml); break;
        case TAH_KV_I16: launch<TAH_KV_I16>(s, a, p, q, records, have ? img : nullptr, out, part_o, part_ml); break;
        case TAH_KV_I8: launch<TAH_KV_I8>(s, a, p, q, records, have ? img : nullptr, out, part_o, part_ml); break;
        default: throw ArgError{"attention: unknown key/value format"};
    }
    if (p.splits > 1) {
        if (a.d == 64 * a.heads && p.splits <= MERGE64_MAX)  // many queries, few splits (else lanes over splits win)
            hipLaunchKernelGGL(k_attn_merge64, dim3((a.nq * a.heads + 15) / 16), dim3(256), 0, s, a.nq * a.heads,
                               a.heads, p.splits, part_o, part_ml, out);
        else if (a.d == 64 * a.heads)
            hipLaunchKernelGGL(k_attn_merge_w, dim3((a.nq * a.heads + 3) / 4), dim3(256), 0, s, a.nq * a.heads,
                               p.splits, part_o, part_ml, out);
        else
            hipLaunchKernelGGL(k_attn_merge, dim3(a.nq * a.heads), dim3(64), 0, s, a.nq, a.d, a.heads, p.splits, 1,
                               part_o, part_ml, out);
        TAH_LAUNCHED();
    }
}

}  // namespace tah
