// The C ABI (include/tah.h): device handles, working memory, weights and fitted models on the card, and the
// in-context passes built from the kernels. Host code only; every kernel lives in the other sources.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <memory>
#include <new>

#include "common.hpp"

using namespace tah;

// ---- working memory --------------------------------------------------------------------------------------------
namespace tah {

void *Pool::take(size_t want, int device) {
    want = (want + 255) & ~size_t(255);
    if (want == 0) want = 256;
    // the smallest idle buffer that is big enough and at most an eighth bigger (so a call's buffers never hold more
    // than 9/8 of what it asked for, which the batch sizes allow for)
    int best = -1;
    for (size_t i = 0; i < bufs.size(); i++)
        if (!bufs[i].busy && bufs[i].bytes >= want && bufs[i].bytes <= want + want / 8 &&
            (best < 0 || bufs[i].bytes < bufs[best].bytes))
            best = (int)i;
    if (best >= 0) {
        bufs[best].busy = true;
        return bufs[best].p;
    }
    if (bytes + want > budget) release_idle();
    if (bytes + want > budget) {
        overdrawn = std::max(overdrawn, bytes + want - budget);
        throw BudgetError{"graphics card: working memory budget exceeded (" + std::to_string(bytes + want) + " > " +
                          std::to_string(budget) + " bytes)"};
    }
    void *p = nullptr;
    TAH_HIP(hipMalloc(&p, want));
    bufs.push_back({p, want, true});
    bytes += want;
    peak = std::max(peak, bytes);
    (void)device;
    return p;
}

void Pool::give(void *p) {
    for (auto &b : bufs)
        if (b.p == p) b.busy = false;
}

void Pool::release_idle() {
    std::vector<Buf> keep;
    for (auto &b : bufs) {
        if (b.busy) {
            keep.push_back(b);
        } else {
            (void)hipFree(b.p);
            bytes -= b.bytes;
        }
    }
    bufs.swap(keep);
}

}  // namespace tah

// Borrowed working buffers of one call, given back when it ends.
struct Loans {
    tah_dev *dev;
    std::vector<void *> held;
    explicit Loans(tah_dev *d) : dev(d) {}
    template <class T>
    T *take(size_t count) {
        void *p = dev->pool.take(count * sizeof(T), dev->ordinal);
        held.push_back(p);
        return static_cast<T *>(p);
    }
    ~Loans() {
        for (void *p : held) dev->pool.give(p);
    }
};

static size_t busy_bytes(const Pool &p) {
    size_t b = 0;
    for (auto &x : p.bufs)
        if (x.busy) b += x.bytes;
    return b;
}

// The same for one buffer of `bytes` bytes.
static size_t loan_raw(size_t bytes) {
    const size_t want = (bytes + 255) & ~size_t(255);
    return want + want / 8 + 256;
}

// Rows a call takes at a time: all n when their working memory fits the room the budget leaves, else the largest
// halving of n that fits (rows are independent); an OutOfMemory error when not even one row fits.
template <class F>
static int batch_rows(const tah_dev *dev, int n, F bytes_of) {
    const size_t used = busy_bytes(dev->pool);
    const size_t room = dev->pool.budget > used ? dev->pool.budget - used : 0;
    int b = std::max(n, 1);
    while (b > 1 && bytes_of(b) > room) b = (b + 1) / 2;
    if (bytes_of(b) > room) throw BudgetError{"graphics card: one row does not fit the working-memory budget"};
    return b;
}

// Bytes Loans may hold for buffers of these many floats: each rounded to 256 bytes, and up to an eighth more when
// the pool hands out an idle buffer a little larger than asked.
static size_t loan_bytes(std::initializer_list<size_t> floats) {
    size_t b = 0;
    for (size_t f : floats) {
        const size_t want = (f * sizeof(float) + 255) & ~size_t(255);
        b += want + want / 8 + 256;
    }
    return b;
}

struct SinkError {
    int status;
};

template <class F>
static int guarded(tah_dev *dev, F &&f) {
    if (!dev) return TAH_E_ARG;
    std::lock_guard<std::mutex> g(dev->lock);
    try {
        hipError_t e = hipSetDevice(dev->ordinal);
        if (e != hipSuccess) throw DeviceError{std::string("graphics card: hipSetDevice: ") + hipGetErrorString(e)};
        return f();
    } catch (const DeviceError &e) {
        dev->last_error = e.msg;
        return TAH_E_DEVICE;
    } catch (const ArgError &e) {
        dev->last_error = e.msg;
        return TAH_E_ARG;
    } catch (const BudgetError &e) {
        dev->last_error = e.msg;
        return TAH_E_BUDGET;
    } catch (const SinkError &e) {
        dev->last_error = "layer sink returned " + std::to_string(e.status);
        return TAH_E_SINK;
    } catch (const std::bad_alloc &) {
        dev->last_error = "out of host memory";
        return TAH_E_BUDGET;
    } catch (const std::exception &e) {
        // nothing may unwind through extern "C": any other failure is the card's, and the caller answers on the CPU
        dev->last_error = std::string("graphics card: ") + e.what();
        return TAH_E_DEVICE;
    } catch (...) {
        dev->last_error = "graphics card: unexpected failure";
        return TAH_E_DEVICE;
    }
}

extern "C" size_t tah_kv_record(int32_t kv_format, int32_t d, int32_t rc) {
    const size_t w = kv_format == TAH_KV_F32 ? 4 : (kv_format == TAH_KV_I16 ? 2 : 1);
    return 2 * (size_t)d * rc * w + (kv_format == TAH_KV_F32 ? 0 : 8 * (size_t)d);
}

static size_t layer_bytes(int fmt, int rows, int chunk, int d) {
    return (size_t)(rows / chunk) * tah_kv_record(fmt, d, chunk) + (rows % chunk ? tah_kv_record(fmt, d, rows % chunk) : 0);
}

static size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// Device memory for tah_stage_dev_noalloc, one copy per GPU for the life of the process. Host code never uses this
// name as an address: tah_open looks up each device's copy with hipGetSymbolAddress and keeps it in tah_dev.
static __device__ __align__(256) uint8_t scratch[TAH_NOALLOC_SCRATCH_BYTES];

// ---- device handle ---------------------------------------------------------------------------------------------
extern "C" int tah_open(int32_t ordinal, tah_dev **out) {
    if (!out) return TAH_E_ARG;
    *out = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || ordinal < 0 || ordinal >= count) return TAH_E_DEVICE;
    tah_dev *dev = new (std::nothrow) tah_dev();
    if (!dev) return TAH_E_BUDGET;
    dev->ordinal = ordinal;
    int rc = guarded(dev, [&] {
        hipDeviceProp_t prop;
        TAH_HIP(hipGetDeviceProperties(&prop, ordinal));
        dev->name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
        TAH_HIP(hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking));
        TAH_HIP(hipStreamCreateWithFlags(&dev->side, hipStreamNonBlocking));
        TAH_HIP(hipEventCreateWithFlags(&dev->fork_ev, hipEventDisableTiming));
        TAH_HIP(hipEventCreateWithFlags(&dev->join_ev, hipEventDisableTiming));
        void *p = nullptr;
        TAH_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        dev->noalloc = static_cast<uint8_t *>(p);
        return TAH_OK;
    });
    if (rc != TAH_OK) {
        if (dev->fork_ev) (void)hipEventDestroy(dev->fork_ev);
        if (dev->join_ev) (void)hipEventDestroy(dev->join_ev);
        if (dev->side) (void)hipStreamDestroy(dev->side);
        if (dev->stream) (void)hipStreamDestroy(dev->stream);
        delete dev;
        return rc;
    }
    *out = dev;
    return TAH_OK;
}

extern "C" void tah_close(tah_dev *dev) {
    if (!dev) return;
    {
        std::lock_guard<std::mutex> g(dev->lock);
        (void)hipSetDevice(dev->ordinal);
        if (dev->stream) (void)hipStreamSynchronize(dev->stream);
        for (auto &b : dev->pool.bufs) (void)hipFree(b.p);
        dev->pool.bufs.clear();
        for (int i = 0; i < 2; i++) {
            if (dev->pinned[i]) (void)hipHostFree(dev->pinned[i]);
            if (dev->copied[i]) (void)hipEventDestroy(dev->copied[i]);
        }
        if (dev->side) (void)hipStreamSynchronize(dev->side);
        if (dev->fork_ev) (void)hipEventDestroy(dev->fork_ev);
        if (dev->join_ev) (void)hipEventDestroy(dev->join_ev);
        if (dev->side) (void)hipStreamDestroy(dev->side);
        if (dev->stream) (void)hipStreamDestroy(dev->stream);
    }
    delete dev;
}

extern "C" const char *tah_last_error(const tah_dev *dev) { return dev ? dev->last_error.c_str() : "no device"; }

extern "C" int tah_device_name(const tah_dev *dev, char *buf, size_t len) {
    if (!dev || !buf || len == 0) return TAH_E_ARG;
    std::snprintf(buf, len, "%s", dev->name.c_str());
    return TAH_OK;
}

extern "C" int tah_set_work_budget(tah_dev *dev, size_t bytes) {
    return guarded(dev, [&] {
        dev->pool.budget = bytes;
        if (dev->pool.bytes > bytes) dev->pool.release_idle();
        return TAH_OK;
    });
}

extern "C" size_t tah_work_budget(const tah_dev *dev) { return dev ? dev->pool.budget : 0; }

extern "C" int tah_working(const tah_dev *dev, size_t *now, size_t *peak) {
    if (!dev) return TAH_E_ARG;
    if (now) *now = dev->pool.bytes;
    if (peak) *peak = dev->pool.peak;
    return TAH_OK;
}

extern "C" size_t tah_overdrawn(const tah_dev *dev) { return dev ? dev->pool.overdrawn : 0; }

extern "C" int tah_release(tah_dev *dev) {
    return guarded(dev, [&] {
        TAH_HIP(hipStreamSynchronize(dev->stream));
        dev->pool.release_idle();
        dev->pool.peak = dev->pool.bytes;
        return TAH_OK;
    });
}

extern "C" int tah_sync(tah_dev *dev) {
    return guarded(dev, [&] {
        TAH_HIP(hipStreamSynchronize(dev->stream));
        return TAH_OK;
    });
}

extern "C" void *tah_stream(tah_dev *dev) { return dev ? (void *)dev->stream : nullptr; }

// ---- weights ---------------------------------------------------------------------------------------------------
namespace {

// Lays tensors out in one device allocation (each 256-byte aligned), then copies them in.
struct Packer {
    struct Item {
        const void *src;
        size_t bytes;
        const void **dst;
    };
    std::vector<Item> items;
    std::vector<std::unique_ptr<std::vector<uint8_t>>> owned;  // buffers made here (weight images)
    size_t bytes = 0;
    void add(const float *src, size_t n, const float **dst) {
        if (!src || n == 0) {
            *dst = nullptr;
            return;
        }
        items.push_back({src, n * sizeof(float), reinterpret_cast<const void **>(dst)});
        bytes += align256(n * sizeof(float));
    }
    void add_bytes(std::vector<uint8_t> &&buf, const uint8_t **dst) {
        owned.push_back(std::make_unique<std::vector<uint8_t>>(std::move(buf)));
        items.push_back({owned.back()->data(), owned.back()->size(), reinterpret_cast<const void **>(dst)});
        bytes += align256(owned.back()->size());
    }
};

// W [N][K] (N a multiple of 128, K of 16) scaled by 2^shift (its largest magnitude below 2^14) and split into fp16
// hi/lo, in the order the fused blocks stream it through LDS: per block of 128 rows rb, per 16 columns ks,
// [hi, lo][k half g][row n of the block][8 halves of W[128 rb + n][16 ks + 8 g + t]] (8 KB a step).
static int weight_shift(const float *W, size_t n) {
    float mx = 0.0f;
    for (size_t i = 0; i < n; i++) mx = std::max(mx, std::fabs(W[i]));
    int e = 0;
    (void)std::frexp(mx, &e);
    return 14 - e;
}

static inline void split_half(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// W [N][K] as a gemm_split image (SplitW): 32-row tiles, rows sigma32-ordered within a tile, 16-column steps of
// [hi, lo][k half g][32 rows][8 halves].
static void add_split(Packer &pk, const float *W, int N, int K, SplitW &o) {
    o = SplitW{};
    if (!W || N <= 0 || N % 32 || K <= 0 || K % 16) return;
    o.shift = weight_shift(W, (size_t)N * K);
    o.N = N;
    o.K = K;
    const float f = std::ldexp(1.0f, o.shift);
    std::vector<uint8_t> out((size_t)N * K * 4);
    _Float16 *img = reinterpret_cast<_Float16 *>(out.data());
    for (int tile = 0; tile < N / 32; tile++)
        for (int ks = 0; ks < K / 16; ks++) {
            _Float16 *step = img + ((size_t)tile * (K / 16) + ks) * 1024;  // 2 KB = 1024 halves
            for (int g = 0; g < 2; g++)
                for (int slot = 0; slot < 32; slot++) {
                    const int row = 32 * tile + ((slot & 16) | ((slot & 4) << 1) | ((slot & 8) >> 1) | (slot & 3));
                    for (int t = 0; t < 8; t++) {
                        _Float16 hi, lo;
                        split_half(W[(size_t)row * K + 16 * ks + 8 * g + t] * f, hi, lo);
                        step[(g * 32 + slot) * 8 + t] = hi;
                        step[((2 + g) * 32 + slot) * 8 + t] = lo;
                    }
                }
        }
    pk.add_bytes(std::move(out), &o.img);
}

static std::vector<uint8_t> weight_image(const float *W, int N, int K, int &shift) {
    shift = weight_shift(W, (size_t)N * K);
    const float f = std::ldexp(1.0f, shift);
    std::vector<uint8_t> out((size_t)N * K * 4);
    _Float16 *o = reinterpret_cast<_Float16 *>(out.data());
    for (int rb = 0; rb < N / 128; rb++)
        for (int ks = 0; ks < K / 16; ks++)
            for (int part = 0; part < 2; part++)
                for (int g = 0; g < 2; g++)
                    for (int n = 128 * rb; n < 128 * rb + 128; n++)
                        for (int t = 0; t < 8; t++) {
                            _Float16 hi, lo;
                            split_half(W[(size_t)n * K + 16 * ks + 8 * g + t] * f, hi, lo);
                            *o++ = part == 0 ? hi : lo;
                        }
    return out;
}

void add_block(Packer &pk, const tah_block &b, DevBlock &o) {
    o.d = b.d;
    o.heads = b.heads;
    o.ff = b.ff;
    o.ss_hidden = b.ss_hidden;
    const size_t d = b.d, ff = b.ff, hid = b.ss_hidden, hd = b.heads ? b.d / b.heads : 0;
    pk.add(b.n1w, d, &o.n1w);
    pk.add(b.n1b, d, &o.n1b);
    pk.add(b.n2w, d, &o.n2w);
    pk.add(b.n2b, d, &o.n2b);
    pk.add(b.in_w, 3 * d * d, &o.in_w);
    pk.add(b.in_b, 3 * d, &o.in_b);
    pk.add(b.out_w, d * d, &o.out_w);
    pk.add(b.out_b, d, &o.out_b);
    pk.add(b.l1w, ff * d, &o.l1w);
    pk.add(b.l1b, ff, &o.l1b);
    pk.add(b.l2w, d * ff, &o.l2w);
    pk.add(b.l2b, d, &o.l2b);
    if (hid) {
        pk.add(b.b0w, hid, &o.b0w);
        pk.add(b.b0b, hid, &o.b0b);
        pk.add(b.b2w, d * hid, &o.b2w);
        pk.add(b.b2b, d, &o.b2b);
        pk.add(b.q0w, hid * hd, &o.q0w);
        pk.add(b.q0b, hid, &o.q0b);
        pk.add(b.q2w, hd * hid, &o.q2w);
        pk.add(b.q2b, hd, &o.q2b);
    } else {
        o.b0w = o.b0b = o.b2w = o.b2b = o.q0w = o.q0b = o.q2w = o.q2b = nullptr;
    }
    o.l1img = o.l2img = o.inimg = o.outimg = nullptr;
    o.in_s = o.out_s = o.l1_s = o.l2_s = o.q0_s = o.q2_s = SplitW{};
    if (b.d == 128) {
        // the column and row stages' shape: the fused kernels of blocks.hip
        if (b.in_w) pk.add_bytes(weight_image(b.in_w, 3 * b.d, b.d, o.ins), &o.inimg);
        if (b.out_w) pk.add_bytes(weight_image(b.out_w, b.d, b.d, o.outs), &o.outimg);
    } else {
        add_split(pk, b.in_w, 3 * b.d, b.d, o.in_s);
        add_split(pk, b.out_w, b.d, b.d, o.out_s);
    }
    if (ff_fused_shape(b.d, b.ff) && b.l1w && b.l2w) {
        pk.add_bytes(weight_image(b.l1w, b.ff, b.d, o.l1s), &o.l1img);
        pk.add_bytes(weight_image(b.l2w, b.d, b.ff, o.l2s), &o.l2img);
    } else {
        add_split(pk, b.l1w, b.ff, b.d, o.l1_s);
        add_split(pk, b.l2w, b.d, b.ff, o.l2_s);
    }
    if (hid) {
        add_split(pk, b.q0w, b.ss_hidden, (int)hd, o.q0_s);
        add_split(pk, b.q2w, (int)hd, b.ss_hidden, o.q2_s);
    }
}

bool block_ok(const tah_block &b) {
    return b.d > 0 && b.heads > 0 && b.d % b.heads == 0 && b.ff > 0 && b.ss_hidden >= 0 && b.n1w && b.n1b && b.n2w &&
           b.n2b && b.in_w && b.in_b && b.out_w && b.out_b && b.l1w && b.l1b && b.l2w && b.l2b &&
           (b.ss_hidden == 0 || (b.b0w && b.b0b && b.b2w && b.b2b && b.q0w && b.q0b && b.q2w && b.q2b));
}

}  // namespace

extern "C" int tah_weights_upload(tah_dev *dev, const tah_model_desc *m, tah_weights **out) {
    if (!m || !out) return TAH_E_ARG;
    *out = nullptr;
    return guarded(dev, [&] {
        if (m->e <= 0 || m->d <= 0 || m->icl_layers <= 0 || m->icl_heads <= 0 || m->d % m->icl_heads || !m->icl ||
            m->dec_hidden <= 0 || m->outputs <= 0 || !m->lnw || !m->lnb || !m->dec0w || !m->dec0b || !m->dec2w || !m->dec2b)
            throw ArgError{"weights: incomplete model description"};
        for (int l = 0; l < m->icl_layers; l++)
            if (!block_ok(m->icl[l]) || m->icl[l].d != m->d) throw ArgError{"weights: bad in-context block"};
        auto *w = new tah_weights();
        w->dev = dev;
        w->ordinal = dev->ordinal;
        w->e = m->e;
        w->d = m->d;
        w->group = m->group;
        w->inds = m->inds;
        w->cls = m->cls;
        w->max_classes = m->max_classes;
        w->col_heads = m->col_heads;
        w->row_heads = m->row_heads;
        w->icl_heads = m->icl_heads;
        w->col_blocks = m->col_blocks;
        w->row_blocks = m->row_blocks;
        w->icl_layers = m->icl_layers;
        w->dec_hidden = m->dec_hidden;
        w->outputs = m->outputs;
        w->rope_half = m->rope_half;
        Packer pk;
        const size_t e = m->e, d = m->d, ytab = m->max_classes > 0 ? m->max_classes : 2;
        pk.add(m->in_w, e * m->group, &w->in_w);
        pk.add(m->in_b, e, &w->in_b);
        pk.add(m->col_ind, (size_t)m->col_blocks * m->inds * e, &w->col_ind);
        pk.add(m->col_y, ytab * e, &w->col_y);
        pk.add(m->cls_tokens, (size_t)m->cls * e, &w->cls_tokens);
        pk.add(m->rope_freqs, m->rope_half, &w->rope_freqs);
        // Rope::new (src/nn.rs:304-321) for every position a row can have
        std::vector<float> rope;
        if (m->rope_freqs && m->rope_half > 0) {
            const size_t half = m->rope_half;
            rope.resize(2 * (size_t)ROPE_POSITIONS * half);
            for (int p = 0; p < ROPE_POSITIONS; p++)
                for (size_t i = 0; i < half; i++) {
                    const float a = (float)p * m->rope_freqs[i];
                    rope[(size_t)p * half + i] = cosf(a);
                    rope[((size_t)ROPE_POSITIONS + p) * half + i] = sinf(a);
                }
            pk.add(rope.data(), rope.size(), &w->rope_tab);
        }
        pk.add(m->out_lnw, e, &w->out_lnw);
        pk.add(m->out_lnb, e, &w->out_lnb);
        pk.add(m->icl_y, ytab * d, &w->icl_y);
        pk.add(m->lnw, d, &w->lnw);
        pk.add(m->lnb, d, &w->lnb);
        pk.add(m->dec0w, (size_t)m->dec_hidden * d, &w->dec0w);
        pk.add(m->dec0b, m->dec_hidden, &w->dec0b);
        add_split(pk, m->dec0w, m->dec_hidden, (int)d, w->dec0_s);
        pk.add(m->dec2w, (size_t)m->outputs * m->dec_hidden, &w->dec2w);
        pk.add(m->dec2b, m->outputs, &w->dec2b);
        std::vector<float> col_scale;
        if (m->col_heads > 0 && m->e % m->col_heads == 0) {
            col_scale.assign(m->e, 1.0f / sqrtf((float)(m->e / m->col_heads)));
            pk.add(col_scale.data(), col_scale.size(), &w->col_scale);
        } else {
            w->col_scale = nullptr;
        }
        w->icl.resize(m->icl_layers);
        for (int l = 0; l < m->icl_layers; l++) add_block(pk, m->icl[l], w->icl[l]);
        if (m->col_a2 && m->col_blocks > 0) {
            w->col_a2.resize(m->col_blocks);
            for (int i = 0; i < m->col_blocks; i++) add_block(pk, m->col_a2[i], w->col_a2[i]);
        }
        if (m->col_a1 && m->col_blocks > 0) {
            w->col_a1.resize(m->col_blocks);
            for (int i = 0; i < m->col_blocks; i++) add_block(pk, m->col_a1[i], w->col_a1[i]);
        }
        if (m->row && m->row_blocks > 0) {
            w->row.resize(m->row_blocks);
            for (int i = 0; i < m->row_blocks; i++) add_block(pk, m->row[i], w->row[i]);
        }
        // room for the class tokens' first-row-block keys and values, filled on the card below
        std::vector<float> cls_room;
        const bool cls_kv = !w->row.empty() && m->cls > 0 && m->cls_tokens;
        const float *cls_at = nullptr;
        if (cls_kv) {
            cls_room.assign((size_t)m->cls * 3 * e, 0.0f);
            pk.add(cls_room.data(), cls_room.size(), &cls_at);
        }
        try {
            TAH_HIP(hipMalloc(&w->arena, std::max<size_t>(pk.bytes, 256)));
            w->bytes = pk.bytes;
            size_t at = 0;
            for (auto &it : pk.items) {
                void *dst = static_cast<char *>(w->arena) + at;
                TAH_HIP(hipMemcpy(dst, it.src, it.bytes, hipMemcpyHostToDevice));
                *it.dst = dst;
                at += align256(it.bytes);
            }
            if (cls_kv) {
                w->cls_kv = const_cast<float *>(cls_at);
                class_token_kv(dev->stream, w, w->cls_kv, w->cls_kv + (size_t)w->cls * 2 * w->e);
                TAH_HIP(hipStreamSynchronize(dev->stream));
            }
        } catch (...) {
            if (w->arena) (void)hipFree(w->arena);
            delete w;
            throw;
        }
        *out = w;
        return TAH_OK;
    });
}

extern "C" size_t tah_weights_bytes(const tah_weights *w) { return w ? w->bytes : 0; }

extern "C" void tah_weights_free(tah_weights *w) {
    // independent of the device handle, which may already be closed; hipFree waits for work that uses the memory
    if (!w) return;
    (void)hipSetDevice(w->ordinal);
    if (w->arena) (void)hipFree(w->arena);
    delete w;
}

// ---- fitted model ----------------------------------------------------------------------------------------------
static AttnShape shape_of(const tah_model *m, int heads, int nq) {
    return AttnShape{nq, m->rows, m->chunk, m->d, heads, m->kv_format};
}

// Layer l's stored records (a model whose layers are held as tiles keeps none), or its tiles.
static const uint8_t *layer_of(const tah_model *m, int l) {
    return m->images ? nullptr : m->records + (size_t)l * m->layer_bytes;
}

static KvImages images_of(const tah_model *m, int l) {
    if (!m->images) return KvImages{};
    return kv_images_at(m->records + (size_t)l * m->layer_bytes, m->rows, m->chunk, m->heads, m->kv_format);
}

// The images of f32 records rec32 in a loaned buffer when the split-fp16 kernel applies to a's queries, else none.
static const KvImages *loan_images(hipStream_t s, Loans &loans, const AttnShape &a, const uint8_t *rec32, KvImages &img) {
    if (a.nq < TAH_SPLIT16_MIN_Q || !kv_images_apply(a.kv_format, a.d, a.heads)) return nullptr;
    img = kv_images_at(loans.take<uint8_t>(kv_images_bytes(a.rows, a.chunk, a.heads, a.kv_format)), a.rows, a.chunk,
                       a.heads, a.kv_format);
    kv_images(s, a.rows, a.chunk, a.d, a.heads, a.kv_format, rec32, img);
    return &img;
}

// Per layer: (head width 64) the layer's tiles in place of its records (split-fp16 images of f32 records, the codes
// of i16 and i8 records with their factors or scales), each format held once; other head widths keep the records as
// they are.
static size_t model_layer_bytes(int kv_format, int rows, int chunk, int d, int heads) {
    if (kv_images_apply(kv_format, d, heads)) return align256(kv_images_bytes(rows, chunk, heads, kv_format));
    return align256(layer_bytes(kv_format, rows, chunk, d));
}

extern "C" size_t tah_model_bytes(const tah_weights *w, int32_t kv_format, int32_t rows, int32_t chunk) {
    if (!w || rows <= 0 || chunk <= 0 || kv_format < 0 || kv_format > 2) return 0;
    const int d = w->d, layers = w->icl_layers;
    return (size_t)layers * model_layer_bytes(kv_format, rows, chunk, d, w->icl_heads) +
           align256(sizeof(float) * layers * d);
}

extern "C" int tah_model_load(tah_dev *dev, const tah_weights *w, int32_t kv_format, int32_t rows, int32_t chunk,
                              const uint8_t *const *layer_records, const float *scales, tah_model **out) {
    if (!out || !w || !layer_records || !scales) return TAH_E_ARG;
    *out = nullptr;
    return guarded(dev, [&] {
        if (rows <= 0 || chunk <= 0 || kv_format < 0 || kv_format > 2) throw ArgError{"model: bad rows, chunk or format"};
        for (int l = 0; l < w->icl_layers; l++)
            if (!layer_records[l]) throw ArgError{"model: missing layer records"};
        auto *m = new tah_model();
        m->dev = dev;
        m->ordinal = dev->ordinal;
        m->kv_format = kv_format;
        m->rows = rows;
        m->chunk = chunk;
        m->d = w->d;
        m->layers = w->icl_layers;
        m->heads = w->icl_heads;
        m->layer_bytes = model_layer_bytes(kv_format, rows, chunk, w->d, w->icl_heads);
        m->images = kv_images_apply(kv_format, w->d, w->icl_heads);
        m->bytes = tah_model_bytes(w, kv_format, rows, chunk);
        const size_t lb = layer_bytes(kv_format, rows, chunk, w->d);
        uint8_t *staging = nullptr;  // one layer's records on their way into its tiles
        try {
            TAH_HIP(hipMalloc(&m->records, m->bytes));
            m->scales = reinterpret_cast<float *>(m->records + (size_t)m->layers * m->layer_bytes);
            if (m->images) TAH_HIP(hipMalloc(&staging, lb));
            for (int l = 0; l < m->layers; l++) {
                if (m->images) {
                    // the copy waits for the previous layer's tiles to be made from the staging buffer
                    TAH_HIP(hipMemcpyAsync(staging, layer_records[l], lb, hipMemcpyHostToDevice, dev->stream));
                    kv_images(dev->stream, rows, chunk, m->d, m->heads, kv_format, staging, images_of(m, l));
                    TAH_HIP(hipStreamSynchronize(dev->stream));
                } else {
                    TAH_HIP(hipMemcpy(m->records + (size_t)l * m->layer_bytes, layer_records[l], lb,
                                      hipMemcpyHostToDevice));
                }
            }
            TAH_HIP(hipMemcpy(m->scales, scales, sizeof(float) * m->layers * m->d, hipMemcpyHostToDevice));
            if (staging) TAH_HIP(hipFree(staging));
            staging = nullptr;
        } catch (...) {
            if (staging) (void)hipFree(staging);
            if (m->records) (void)hipFree(m->records);
            delete m;
            throw;
        }
        *out = m;
        return TAH_OK;
    });
}

extern "C" void tah_model_free(tah_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->ordinal);
    if (m->records) (void)hipFree(m->records);
    if (m->col_kv) (void)hipFree(m->col_kv);
    if (m->col_img) (void)hipFree(m->col_img);
    delete m;
}

// ---- prediction ------------------------------------------------------------------------------------------------

extern "C" int tah_attend_resident_dev(tah_dev *dev, const tah_model *model, int32_t layer, const float *q_dev,
                                       int32_t nq, float *out_dev) {
    if (!model || !q_dev || !out_dev) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (layer < 0 || layer >= model->layers || nq < 0) throw ArgError{"attend: bad layer or row count"};
        Loans loans(dev);
        const AttnShape a = shape_of(model, model->heads, nq);
        void *work = loans.take<uint8_t>(attention_work_bytes(a));
        const KvImages img = images_of(model, layer);
        attention(dev->stream, a, q_dev, layer_of(model, layer), out_dev, work, &img);
        return TAH_OK;
    });
}

extern "C" int tah_attend_resident(tah_dev *dev, const tah_model *model, int32_t layer, const float *q, int32_t nq,
                                   float *out) {
    if (!model || !q || !out) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (layer < 0 || layer >= model->layers || nq < 0) throw ArgError{"attend: bad layer or row count"};
        if (nq == 0) return TAH_OK;
        Loans loans(dev);
        const size_t n = (size_t)nq * model->d;
        float *qd = loans.take<float>(n), *od = loans.take<float>(n);
        const AttnShape a = shape_of(model, model->heads, nq);
        void *work = loans.take<uint8_t>(attention_work_bytes(a));
        TAH_HIP(hipMemcpyAsync(qd, q, n * sizeof(float), hipMemcpyHostToDevice, dev->stream));
        const KvImages img = images_of(model, layer);
        attention(dev->stream, a, qd, layer_of(model, layer), od, work, &img);
        TAH_HIP(hipMemcpyAsync(out, od, n * sizeof(float), hipMemcpyDeviceToHost, dev->stream));
        TAH_HIP(hipStreamSynchronize(dev->stream));
        return TAH_OK;
    });
}

// Working buffers of the in-context stage for nq rows: t, q, att [nq][d], mid [nq][wide], the attention's split
// partials.
struct StageBufs {
    float *t, *q, *att, *mid;
    void *work;
};

static size_t stage_floats_wide(const tah_weights *w) { return (size_t)std::max(icl_mid(w), w->dec_hidden); }

static StageBufs stage_bufs(const tah_weights *w, const tah_model *model, int nq, Loans &loans) {
    StageBufs b;
    b.t = loans.take<float>((size_t)nq * w->d);
    b.q = loans.take<float>((size_t)nq * w->d);
    b.att = loans.take<float>((size_t)nq * w->d);
    b.mid = loans.take<float>((size_t)nq * stage_floats_wide(w));
    b.work = loans.take<uint8_t>(attention_work_bytes(shape_of(model, w->icl_heads, nq)));
    return b;
}

// The in-context stage for nq rows already on the card (src/predict.rs:413-585): h is updated in place.
static void stage_rows_with(tah_dev *dev, const tah_weights *w, const tah_model *model, float *h, int nq, int out_n,
                            float *out, const StageBufs &bb) {
    const int d = w->d, heads = w->icl_heads;
    hipStream_t s = dev->stream;
    float *t = bb.t, *q = bb.q, *att = bb.att, *mid = bb.mid;
    const AttnShape a = shape_of(model, heads, nq);
    for (int l = 0; l < w->icl_layers; l++) {
        const DevBlock &b = w->icl[l];
        // query: q = modulate(Wq norm1(h) + bq)  (src/nn.rs:130-152)
        const float *scale = model->scales + (size_t)l * d;
        if (query_split_fits(b, nq, h, d, q)) {
            query_split(s, nq, h, d, b, scale, q);
        } else if (query_rows_fits(b, nq, h, d, q)) {
            query_rows(s, nq, h, d, b, scale, q);
        } else {
            dense(s, nq, d, d, h, d, b.in_w, b.in_s.rows(0), b.in_b, q, d, EPI_NONE, nullptr, 0, b.n1w, b.n1b, t);
            query_modulate(s, nq, b, scale, q, mid);
        }
        // attention over the stored layer, then h += out(att)  (src/predict.rs:421-551)
        const KvImages img = images_of(model, l);
        attention(s, a, q, layer_of(model, l), att, bb.work, &img);
        dense(s, nq, d, d, att, d, b.out_w, b.out_s, b.out_b, h, d, EPI_RESID, h, d);
        // h += l2(gelu(l1(norm2 h)))  (src/predict.rs:552-568)
        dense(s, nq, b.ff, d, h, d, b.l1w, b.l1_s, b.l1b, mid, b.ff, EPI_GELU, nullptr, 0, b.n2w, b.n2b, t);
        dense(s, nq, d, b.ff, mid, b.ff, b.l2w, b.l2_s, b.l2b, h, d, EPI_RESID, h, d);
    }
    // decoder, first out_n outputs  (src/predict.rs:570-585)
    dense(s, nq, w->dec_hidden, d, h, d, w->dec0w, w->dec0_s, w->dec0b, mid, w->dec_hidden, EPI_GELU, nullptr, 0, w->lnw,
          w->lnb, t);
    gemm(s, nq, out_n, w->dec_hidden, mid, w->dec_hidden, w->dec2w, w->dec2b, out, out_n, EPI_NONE, nullptr, 0);
}

static void stage_rows(tah_dev *dev, const tah_weights *w, const tah_model *model, float *h, int nq, int out_n,
                       float *out, Loans &loans) {
    stage_rows_with(dev, w, model, h, nq, out_n, out, stage_bufs(w, model, nq, loans));
}

static void check_stage(const tah_weights *w, const tah_model *model, int nq, int out_n) {
    if (!w || !model) throw ArgError{"stage: no weights or model"};
    if (model->d != w->d || model->layers != w->icl_layers) throw ArgError{"stage: model and weights disagree"};
    if (nq < 0 || out_n <= 0 || out_n > w->outputs) throw ArgError{"stage: bad row or output count"};
}

// Working bytes of the in-context stage for k rows (stage_bufs plus the rows' own copy and their outputs).
static size_t stage_batch_bytes(const tah_weights *w, const tah_model *model, int k, int out_n) {
    const size_t kk = (size_t)k;
    return loan_bytes({kk * w->d, kk * out_n, kk * w->d, kk * w->d, kk * w->d, kk * stage_floats_wide(w)}) +
           loan_raw(attention_work_bytes(shape_of(model, w->icl_heads, k)));
}

extern "C" int tah_stage_dev(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *h_dev, int32_t nq,
                             int32_t out_n, float *out_dev) {
    if (!h_dev || !out_dev) return TAH_E_ARG;
    return guarded(dev, [&] {
        check_stage(w, model, nq, out_n);
        if (nq == 0) return TAH_OK;
        const int batch = batch_rows(dev, nq, [&](int k) { return stage_batch_bytes(w, model, k, out_n); });
        for (int r0 = 0; r0 < nq; r0 += batch) {
            const int k = std::min(batch, nq - r0);
            Loans loans(dev);
            float *h = loans.take<float>((size_t)k * w->d);
            TAH_HIP(hipMemcpyAsync(h, h_dev + (size_t)r0 * w->d, sizeof(float) * k * w->d, hipMemcpyDeviceToDevice,
                                   dev->stream));
            stage_rows(dev, w, model, h, k, out_n, out_dev + (size_t)r0 * out_n, loans);
        }
        return TAH_OK;
    });
}

extern "C" int tah_stage(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *h, int32_t nq,
                         int32_t out_n, float *out) {
    if (!h || !out) return TAH_E_ARG;
    return guarded(dev, [&] {
        check_stage(w, model, nq, out_n);
        if (nq == 0) return TAH_OK;
        const int batch = batch_rows(dev, nq, [&](int k) { return stage_batch_bytes(w, model, k, out_n); });
        for (int r0 = 0; r0 < nq; r0 += batch) {
            const int k = std::min(batch, nq - r0);
            Loans loans(dev);
            float *hd = loans.take<float>((size_t)k * w->d);
            float *od = loans.take<float>((size_t)k * out_n);
            TAH_HIP(hipMemcpyAsync(hd, h + (size_t)r0 * w->d, sizeof(float) * k * w->d, hipMemcpyHostToDevice,
                                   dev->stream));
            stage_rows(dev, w, model, hd, k, out_n, od, loans);
            TAH_HIP(hipMemcpyAsync(out + (size_t)r0 * out_n, od, sizeof(float) * k * out_n, hipMemcpyDeviceToHost,
                                   dev->stream));
            TAH_HIP(hipStreamSynchronize(dev->stream));  // the loans go back to the pool with the batch
        }
        return TAH_OK;
    });
}

// The in-context stage without allocating: every working buffer is carved from this device's static scratch array.
// No hipMalloc, hipFree or pool call happens, so callers that cannot allocate (graph capture, serving loops) can use
// it. Calls on one GPU share the array: two calls that overlap on one GPU (from two device handles, whose streams
// are not ordered with each other) race.
extern "C" int tah_stage_dev_noalloc(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *h_dev,
                                     int32_t nq, int32_t out_n, float *out_dev) {
    if (!h_dev || !out_dev) return TAH_E_ARG;
    return guarded(dev, [&] {
        check_stage(w, model, nq, out_n);
        if (nq > TAH_NOALLOC_MAX_ROWS)
            throw ArgError{"stage_noalloc: at most " + std::to_string(TAH_NOALLOC_MAX_ROWS) + " rows a call"};
        if (nq == 0) return TAH_OK;
        if (!dev->noalloc) throw DeviceError{"graphics card: the scratch array was not resolved"};
        const size_t wide = stage_floats_wide(w), rows_d = (size_t)nq * w->d;
        const size_t sizes[] = {rows_d * 4, rows_d * 4, rows_d * 4, rows_d * 4, (size_t)nq * wide * 4,
                                attention_work_bytes(shape_of(model, w->icl_heads, nq))};
        size_t need = 0;
        for (size_t b : sizes) need += align256(b);
        if (need > TAH_NOALLOC_SCRATCH_BYTES)
            throw ArgError{"stage_noalloc: this model needs " + std::to_string(need) + " bytes of scratch for " +
                           std::to_string(nq) + " rows, more than the " + std::to_string(TAH_NOALLOC_SCRATCH_BYTES) +
                           " the library holds"};
        uint8_t *at = dev->noalloc;
        auto carve = [&](size_t bytes) {
            uint8_t *p = at;
            at += align256(bytes);
            return p;
        };
        float *h = reinterpret_cast<float *>(carve(sizes[0]));
        StageBufs bb;
        bb.t = reinterpret_cast<float *>(carve(sizes[1]));
        bb.q = reinterpret_cast<float *>(carve(sizes[2]));
        bb.att = reinterpret_cast<float *>(carve(sizes[3]));
        bb.mid = reinterpret_cast<float *>(carve(sizes[4]));
        bb.work = carve(sizes[5]);
        // every buffer is written before it is read (the partials by the attention's key ranges before their merge),
        // so nothing left by an earlier call needs clearing
        TAH_HIP(hipMemcpyAsync(h, h_dev, rows_d * sizeof(float), hipMemcpyDeviceToDevice, dev->stream));
        stage_rows_with(dev, w, model, h, nq, out_n, out_dev, bb);
        return TAH_OK;
    });
}

// ---- fitting ---------------------------------------------------------------------------------------------------
extern "C" int tah_pack(tah_dev *dev, const float *c, int32_t d, int32_t rc, int32_t kv_format, uint8_t *out) {
    if (!c || !out) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (d <= 0 || rc <= 0 || kv_format < 0 || kv_format > 2) throw ArgError{"pack: bad size or format"};
        Loans loans(dev);
        const size_t n = 2 * (size_t)d * rc, bytes = tah_kv_record(kv_format, d, rc);
        float *cd = loans.take<float>(n);
        uint8_t *od = loans.take<uint8_t>(bytes);
        TAH_HIP(hipMemcpyAsync(cd, c, n * sizeof(float), hipMemcpyHostToDevice, dev->stream));
        if (kv_format == TAH_KV_F32)
            TAH_HIP(hipMemcpyAsync(od, cd, bytes, hipMemcpyDeviceToDevice, dev->stream));
        else
            pack(dev->stream, rc, d, rc, kv_format, cd, od);
        TAH_HIP(hipMemcpyAsync(out, od, bytes, hipMemcpyDeviceToHost, dev->stream));
        TAH_HIP(hipStreamSynchronize(dev->stream));
        return TAH_OK;
    });
}

extern "C" int tah_attend(tah_dev *dev, const float *q, const float *kv, int32_t rows, int32_t chunk, int32_t d,
                          int32_t heads, float *out) {
    if (!q || !kv || !out) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (rows <= 0 || chunk <= 0 || d <= 0 || heads <= 0 || d % heads) throw ArgError{"attend: bad shape"};
        Loans loans(dev);
        const size_t n = (size_t)rows * d;
        float *qd = loans.take<float>(n), *kvd = loans.take<float>(2 * n), *od = loans.take<float>(n);
        const AttnShape a{rows, rows, chunk, d, heads, TAH_KV_F32};
        void *work = loans.take<uint8_t>(attention_work_bytes(a));
        TAH_HIP(hipMemcpyAsync(qd, q, n * sizeof(float), hipMemcpyHostToDevice, dev->stream));
        TAH_HIP(hipMemcpyAsync(kvd, kv, 2 * n * sizeof(float), hipMemcpyHostToDevice, dev->stream));
        KvImages img;
        const KvImages *imgp = loan_images(dev->stream, loans, a, reinterpret_cast<const uint8_t *>(kvd), img);
        attention(dev->stream, a, qd, reinterpret_cast<const uint8_t *>(kvd), od, work, imgp);
        TAH_HIP(hipMemcpyAsync(out, od, n * sizeof(float), hipMemcpyDeviceToHost, dev->stream));
        TAH_HIP(hipStreamSynchronize(dev->stream));
        dev->stages++;
        return TAH_OK;
    });
}

// ---- the regression head --------------------------------------------------------------------------------------
static void check_quantiles(int rows, int n, const float *alphas, int na) {
    if (rows < 0 || n < 2 || n > 1024 || na < 0 || na > 64 || (na > 0 && !alphas))
        throw ArgError{"quantile_stats: 2 to 1024 quantiles a row and at most 64 levels"};
}

extern "C" int tah_quantile_stats_dev(tah_dev *dev, const float *q_dev, int32_t rows, int32_t n, const float *alphas,
                                      int32_t n_alphas, float *stats_dev) {
    if (!q_dev || !stats_dev) return TAH_E_ARG;
    return guarded(dev, [&] {
        check_quantiles(rows, n, alphas, n_alphas);
        if (rows == 0) return TAH_OK;
        Loans loans(dev);
        float *ad = loans.take<float>(std::max(n_alphas, 1));
        if (n_alphas)
            TAH_HIP(hipMemcpyAsync(ad, alphas, sizeof(float) * n_alphas, hipMemcpyHostToDevice, dev->stream));
        quantile_stats(dev->stream, rows, n, q_dev, n_alphas, ad, stats_dev);
        // the alphas' staging buffer goes back to the pool only once the copy from the caller's memory is done
        TAH_HIP(hipStreamSynchronize(dev->stream));
        return TAH_OK;
    });
}

extern "C" int tah_quantile_stats(tah_dev *dev, const float *q, int32_t rows, int32_t n, const float *alphas,
                                  int32_t n_alphas, float *stats) {
    if (!q || !stats) return TAH_E_ARG;
    return guarded(dev, [&] {
        check_quantiles(rows, n, alphas, n_alphas);
        if (rows == 0) return TAH_OK;
        Loans loans(dev);
        const size_t nin = (size_t)rows * n, nout = (size_t)rows * (3 + n_alphas);
        float *qd = loans.take<float>(nin), *sd = loans.take<float>(nout), *ad = loans.take<float>(std::max(n_alphas, 1));
        TAH_HIP(hipMemcpyAsync(qd, q, sizeof(float) * nin, hipMemcpyHostToDevice, dev->stream));
        if (n_alphas)
            TAH_HIP(hipMemcpyAsync(ad, alphas, sizeof(float) * n_alphas, hipMemcpyHostToDevice, dev->stream));
        quantile_stats(dev->stream, rows, n, qd, n_alphas, ad, sd);
        TAH_HIP(hipMemcpyAsync(stats, sd, sizeof(float) * nout, hipMemcpyDeviceToHost, dev->stream));
        TAH_HIP(hipStreamSynchronize(dev->stream));
        return TAH_OK;
    });
}

// The device's two pinned staging buffers for records on their way to a sink, at least `bytes` each.
static void staging(tah_dev *dev, size_t bytes) {
    for (int i = 0; i < 2; i++)
        if (!dev->copied[i]) TAH_HIP(hipEventCreateWithFlags(&dev->copied[i], hipEventDisableTiming));
    if (dev->pinned_bytes >= bytes) return;
    // a call that failed part-way may have left copies into them queued
    TAH_HIP(hipStreamSynchronize(dev->stream));
    for (int i = 0; i < 2; i++) {
        if (dev->pinned[i]) TAH_HIP(hipHostFree(dev->pinned[i]));
        dev->pinned[i] = nullptr;
    }
    dev->pinned_bytes = 0;
    for (int i = 0; i < 2; i++) TAH_HIP(hipHostMalloc(&dev->pinned[i], bytes, hipHostMallocDefault));
    dev->pinned_bytes = bytes;
}

extern "C" int tah_in_context(tah_dev *dev, const tah_weights *w, const float *h_host, int32_t rows, const float *scales,
                              int32_t kv_format, int32_t chunk, tah_layer_sink sink, void *ctx) {
    if (!w || !h_host || !scales || !sink) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (rows <= 0 || chunk <= 0 || kv_format < 0 || kv_format > 2) throw ArgError{"in_context: bad rows, chunk or format"};
        const int d = w->d, L = w->icl_layers;
        const int ff = icl_mid(w);
        const size_t n = (size_t)rows * d;
        const size_t lbytes = layer_bytes(kv_format, rows, chunk, d);
        hipStream_t s = dev->stream;
        Loans loans(dev);
        float *h = loans.take<float>(n), *t = loans.take<float>(n), *q = loans.take<float>(n);
        float *att = loans.take<float>(n), *kv = loans.take<float>(2 * n), *rec32 = loans.take<float>(2 * n);
        float *mid = loans.take<float>((size_t)rows * ff), *sc = loans.take<float>((size_t)L * d);
        uint8_t *recq = kv_format == TAH_KV_F32 ? nullptr : loans.take<uint8_t>(lbytes);
        const AttnShape a{rows, rows, chunk, d, w->icl_heads, TAH_KV_F32};
        void *work = loans.take<uint8_t>(attention_work_bytes(a));
        KvImages img;
        const bool use_img = rows >= TAH_SPLIT16_MIN_Q && kv_images_apply(TAH_KV_F32, d, w->icl_heads);
        if (use_img)
            img = kv_images_at(loans.take<uint8_t>(kv_images_bytes(rows, chunk, w->icl_heads, TAH_KV_F32)), rows, chunk,
                               w->icl_heads, TAH_KV_F32);
        staging(dev, lbytes);
        TAH_HIP(hipMemcpyAsync(h, h_host, n * sizeof(float), hipMemcpyHostToDevice, s));
        TAH_HIP(hipMemcpyAsync(sc, scales, sizeof(float) * L * d, hipMemcpyHostToDevice, s));
        for (int l = 0; l < L; l++) {
            const DevBlock &b = w->icl[l];
            // keys and values of every row, stored (src/fit.rs:627-663); the layer norms inside the products' kernels
            // where they take them (the split-K kernels from 1,025 rows), else into t first
            dense(s, rows, 2 * d, d, h, d, b.in_w + (size_t)d * d, b.in_s.rows(d), b.in_b + d, kv, 2 * d, EPI_NONE,
                  nullptr, 0, b.n1w, b.n1b, t);
            to_records(s, rows, d, chunk, kv, rec32);
            const uint8_t *stored = reinterpret_cast<const uint8_t *>(rec32);
            if (kv_format != TAH_KV_F32) {
                pack(s, rows, d, chunk, kv_format, rec32, recq);
                stored = recq;
            }
            // layer l's records into staging buffer l % 2 (the sink read layer l - 2's there before this was queued)
            TAH_HIP(hipMemcpyAsync(dev->pinned[l & 1], stored, lbytes, hipMemcpyDeviceToHost, s));
            TAH_HIP(hipEventRecord(dev->copied[l & 1], s));
            const bool last = l + 1 == L;
            if (!last) {
                // every row attends to all rows over the exact keys and values, then the rest of the block
                // (src/fit.rs:667-744)
                dense(s, rows, d, d, h, d, b.in_w, b.in_s.rows(0), b.in_b, q, d, EPI_NONE, nullptr, 0, b.n1w, b.n1b, t);
                query_modulate(s, rows, b, sc + (size_t)l * d, q, mid);
                if (use_img)
                    kv_images(s, rows, chunk, d, w->icl_heads, TAH_KV_F32, reinterpret_cast<const uint8_t *>(rec32), img);
                attention(s, a, q, reinterpret_cast<const uint8_t *>(rec32), att, work, use_img ? &img : nullptr);
                dense(s, rows, d, d, att, d, b.out_w, b.out_s, b.out_b, h, d, EPI_RESID, h, d);
                dense(s, rows, b.ff, d, h, d, b.l1w, b.l1_s, b.l1b, mid, b.ff, EPI_GELU, nullptr, 0, b.n2w, b.n2b, t);
                dense(s, rows, d, b.ff, mid, b.ff, b.l2w, b.l2_s, b.l2b, h, d, EPI_RESID, h, d);
            }
            // the card works on layer l (queued above) while the sink takes layer l - 1's records; on the stream the
            // copy of layer l's records runs before layer l + 1's keys overwrite rec32
            if (l > 0) {
                TAH_HIP(hipEventSynchronize(dev->copied[(l - 1) & 1]));
                const int rc = sink(ctx, l - 1, static_cast<const uint8_t *>(dev->pinned[(l - 1) & 1]), lbytes);
                if (rc != 0) {
                    TAH_HIP(hipStreamSynchronize(s));  // nothing queued is left touching the staging buffers
                    throw SinkError{rc};
                }
            }
        }
        TAH_HIP(hipEventSynchronize(dev->copied[(L - 1) & 1]));
        const int rc = sink(ctx, L - 1, static_cast<const uint8_t *>(dev->pinned[(L - 1) & 1]), lbytes);
        TAH_HIP(hipStreamSynchronize(s));
        if (rc != 0) throw SinkError{rc};
        dev->stages++;
        return TAH_OK;
    });
}

// ---- the column and row stages, and whole prediction from feature rows ------------------------------------------
extern "C" size_t tah_columns_bytes(const tah_weights *w, int32_t features, int32_t digits) {
    if (!w || features <= 0 || digits <= 0 || w->col_a2.empty()) return 0;
    const size_t n = (size_t)features * digits * w->col_blocks * 2 * w->e * w->inds;
    return align256(n * sizeof(float)) + align256(column_images_bytes(w, features, digits));
}

extern "C" size_t tah_model_held_bytes(const tah_model *m) { return m ? m->bytes : 0; }

extern "C" int tah_model_set_columns(tah_dev *dev, tah_model *model, const tah_weights *w, const float *col_kv,
                                     int32_t features, int32_t digits) {
    if (!model || !w || !col_kv) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (features <= 0 || digits <= 0 || w->col_a2.empty()) throw ArgError{"columns: bad features or digits"};
        const size_t n = (size_t)features * digits * w->col_blocks * 2 * w->e * w->inds;
        if (model->col_kv) {
            (void)hipFree(model->col_kv);
            model->bytes -= align256((size_t)model->features * model->digits * w->col_blocks * 2 * w->e * w->inds *
                                     sizeof(float));
            model->col_kv = nullptr;
        }
        if (model->col_img) {
            (void)hipFree(model->col_img);
            model->bytes -= align256(column_images_bytes(w, model->features, model->digits));
            model->col_img = nullptr;
        }
        model->features = model->digits = 0;
        TAH_HIP(hipMalloc(&model->col_kv, n * sizeof(float)));
        TAH_HIP(hipMemcpy(model->col_kv, col_kv, n * sizeof(float), hipMemcpyHostToDevice));
        model->bytes += align256(n * sizeof(float));
        // the column blocks' key/value images, made once here instead of at every prediction
        const size_t ib = column_images_bytes(w, features, digits);
        if (ib) {
            TAH_HIP(hipMalloc(&model->col_img, ib));
            column_images(dev->stream, w, model->col_kv, features, digits, model->col_img);
            TAH_HIP(hipStreamSynchronize(dev->stream));
            model->bytes += align256(ib);
        }
        model->features = features;
        model->digits = digits;
        return TAH_OK;
    });
}

// The rotary tables of a row of T tokens (Rope::new, src/nn.rs:304-321): a prefix of the ones made at upload.
struct RopeTabs {
    const float *cos, *sin;
};
static RopeTabs rope_tables(const tah_weights *w, int T) {
    if (!w->rope_tab) throw ArgError{"weights lack the rotary frequencies"};
    if (T > ROPE_POSITIONS) throw ArgError{"row stage: more tokens than the rotary tables cover"};
    return RopeTabs{w->rope_tab, w->rope_tab + (size_t)ROPE_POSITIONS * w->rope_half};
}

static void check_columns(const tah_weights *w, const tah_model *model) {
    if (!model->col_kv) throw ArgError{"the model holds no column cache (tah_model_set_columns)"};
    if (w->col_a2.empty() || w->row.empty() || !w->col_scale) throw ArgError{"weights lack the column or row stage"};
}

// Device work for n rows x (on the card): tokens [n][T][e] after the column stage.
static void embed_rows(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x, int n, float *tok,
                       Loans &loans) {
    const int features = model->features;
    float *cells = loans.take<float>((size_t)n * features * w->e);
    float *scratch = loans.take<float>(column_stage_floats(w, n, features, model->digits));
    column_stage(dev->stream, w, model->col_kv, model->digits, x, n, features, cells, scratch, model->col_img);
    assemble_tokens(dev->stream, w, cells, n, features, tok);
}

extern "C" int tah_embed(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x, int32_t n,
                         float *tok) {
    if (!w || !model || !x || !tok) return TAH_E_ARG;
    return guarded(dev, [&] {
        check_columns(w, model);
        if (n <= 0) return TAH_OK;
        const int F = model->features, T = w->cls + F;
        const size_t per_tok = (size_t)T * w->e;
        const int batch = batch_rows(dev, n, [&](int k) {
            const size_t kk = (size_t)k;
            return loan_bytes({kk * F, kk * per_tok, kk * F * w->e, column_stage_floats(w, k, F, model->digits)});
        });
        for (int r0 = 0; r0 < n; r0 += batch) {
            const int k = std::min(batch, n - r0);
            Loans loans(dev);
            float *xd = loans.take<float>((size_t)k * F);
            float *td = loans.take<float>((size_t)k * per_tok);
            TAH_HIP(hipMemcpyAsync(xd, x + (size_t)r0 * F, sizeof(float) * k * F, hipMemcpyHostToDevice, dev->stream));
            embed_rows(dev, w, model, xd, k, td, loans);
            TAH_HIP(hipMemcpyAsync(tok + (size_t)r0 * per_tok, td, sizeof(float) * k * per_tok, hipMemcpyDeviceToHost,
                                   dev->stream));
            TAH_HIP(hipStreamSynchronize(dev->stream));
        }
        return TAH_OK;
    });
}

extern "C" int tah_represent(tah_dev *dev, const tah_weights *w, const float *tok, int32_t n, int32_t tokens,
                             float *rep) {
    if (!w || !tok || !rep) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (w->row.empty()) throw ArgError{"weights lack the row stage"};
        if (n <= 0) return TAH_OK;
        if (tokens <= w->cls) throw ArgError{"represent: too few tokens"};
        const size_t per_tok = (size_t)tokens * w->e;
        const RopeTabs tabs = rope_tables(w, tokens);
        const int batch = batch_rows(dev, n, [&](int k) {
            return loan_bytes({(size_t)k * per_tok, (size_t)k * w->d, row_stage_floats(w, k, tokens)});
        });
        for (int r0 = 0; r0 < n; r0 += batch) {
            const int k = std::min(batch, n - r0);
            Loans loans(dev);
            float *td = loans.take<float>((size_t)k * per_tok), *rd = loans.take<float>((size_t)k * w->d);
            float *scratch = loans.take<float>(row_stage_floats(w, k, tokens));
            TAH_HIP(hipMemcpyAsync(td, tok + (size_t)r0 * per_tok, sizeof(float) * k * per_tok, hipMemcpyHostToDevice,
                                   dev->stream));
            row_stage(dev->stream, w, td, k, tokens, tabs.cos, tabs.sin, rd, scratch);
            TAH_HIP(hipMemcpyAsync(rep + (size_t)r0 * w->d, rd, sizeof(float) * k * w->d, hipMemcpyDeviceToHost,
                                   dev->stream));
            TAH_HIP(hipStreamSynchronize(dev->stream));
        }
        return TAH_OK;
    });
}

// From this many rows a batch's column and row stages run as two halves, the second on the device's side stream:
// each half's kernels then fill the other's last round of workgroups (a column block's 1,600 workgroups at 2,048 rows
// are 3.125 rounds of the 512 the card runs at once). The halves' rows are independent and their outputs the same.
// Measured per batch size: 768 rows 2.005 -> 1.955 ms as halves; 512 and 640 rows slower (1.478 -> 1.552, 1.802 ->
// 1.851 ms), 896 unchanged.
constexpr int TWO_HALVES_ROWS = 768;
static bool two_halves(const tah_weights *w, const tah_model *model, int k) {
    return k >= TWO_HALVES_ROWS && model->col_img && column_tokens_fits(w, k / 2, model->features, model->digits) &&
           column_tokens_fits(w, k - k / 2, model->features, model->digits);
}

// Joins the side stream back into the main one when it leaves scope (before the loans declared ahead of it go back
// to the pool), also when a launch threw.
struct SideJoin {
    tah_dev *dev;
    ~SideJoin() {
        (void)hipEventRecord(dev->join_ev, dev->side);
        (void)hipStreamWaitEvent(dev->stream, dev->join_ev, 0);
    }
};

// Working bytes of predict_rows for k rows, as it borrows them: the tokens and representations; the column stage's
// cells and scratch (none when it writes the tokens itself over the model's column images); the row stage's scratch
// (row_stage_floats: compact where only the fused kernels run; one for each half when they run apart); the
// in-context stage's buffers.
static size_t predict_batch_bytes(const tah_weights *w, const tah_model *model, int k) {
    const int T = w->cls + model->features;
    const size_t kk = (size_t)k;
    const size_t in_context = loan_bytes({kk * w->d, kk * w->d, kk * w->d, kk * std::max(icl_mid(w), w->dec_hidden)}) +
                              loan_raw(attention_work_bytes(shape_of(model, model->heads, k)));
    if (two_halves(w, model, k))
        return loan_bytes({kk * T * w->e, kk * w->d, row_stage_floats(w, k / 2, T), row_stage_floats(w, k - k / 2, T)}) +
               in_context;
    const bool direct = column_tokens_fits(w, k, model->features, model->digits);
    const size_t cells = direct ? 0 : kk * model->features * w->e;
    const size_t col = direct && model->col_img ? 0 : column_stage_floats(w, k, model->features, model->digits);
    return loan_bytes({kk * T * w->e, kk * w->d, cells, col, row_stage_floats(w, k, T)}) + in_context;
}

// All three stages for n rows x (on the card) into out [n][out_n] (on the card), in sub-batches that fit the
// working-memory budget (the reference's chain, src/gpu.rs:2171-2224); rows are independent.
static void predict_rows(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x, int n, int out_n,
                         float *out) {
    check_columns(w, model);
    check_stage(w, model, n, out_n);
    const int T = w->cls + model->features;
    const RopeTabs tabs = rope_tables(w, T);
    const int batch = batch_rows(dev, n, [&](int k) { return predict_batch_bytes(w, model, k); });
    for (int r0 = 0; r0 < n; r0 += batch) {
        const int k = std::min(batch, n - r0);
        Loans loans(dev);
        float *tok = loans.take<float>((size_t)k * T * w->e);
        float *rep = loans.take<float>((size_t)k * w->d);
        const float *xr = x + (size_t)r0 * model->features;
        if (two_halves(w, model, k)) {
            // the first half on the main stream, the second on the side stream after what the main stream holds so
            // far; the main stream then waits for the side stream's half (SideJoin, also on an error)
            TAH_HIP(hipEventRecord(dev->fork_ev, dev->stream));
            TAH_HIP(hipStreamWaitEvent(dev->side, dev->fork_ev, 0));
            {
                const SideJoin join{dev};
                const int half[2] = {k / 2, k - k / 2};
                for (int hf = 0; hf < 2; hf++) {
                    const hipStream_t s = hf ? dev->side : dev->stream;
                    const int r = hf ? half[0] : 0, m = half[hf];
                    float *sc = loans.take<float>(row_stage_floats(w, m, T));
                    const bool kv = row_stage_takes_kv(w, m, T);
                    float *tk = tok + (size_t)r * T * w->e;
                    column_stage_tokens(s, w, model->col_kv, xr + (size_t)r * model->features, m, model->features, tk,
                                        kv ? row_stage_kv(w, m, T, sc) : nullptr, kv ? w->cls_kv : nullptr, nullptr,
                                        model->col_img);
                    row_stage(s, w, tk, m, T, tabs.cos, tabs.sin, rep + (size_t)r * w->d, sc, kv);
                }
            }
            stage_rows(dev, w, model, rep, k, out_n, out + (size_t)r0 * out_n, loans);
            continue;
        }
        float *scratch = nullptr;
        bool kv_ready = false;
        if (column_tokens_fits(w, k, model->features, model->digits)) {
            // the column stage straight into the tokens, and the first row block's keys and values from its last
            // block's kernel where the row stage takes them
            float *cs = model->col_img ? nullptr : loans.take<float>(column_stage_floats(w, k, model->features, model->digits));
            scratch = loans.take<float>(row_stage_floats(w, k, T));
            kv_ready = row_stage_takes_kv(w, k, T);
            column_stage_tokens(dev->stream, w, model->col_kv, xr, k, model->features, tok,
                                kv_ready ? row_stage_kv(w, k, T, scratch) : nullptr,
                                kv_ready ? w->cls_kv : nullptr, cs, model->col_img);
        } else {
            embed_rows(dev, w, model, xr, k, tok, loans);
            scratch = loans.take<float>(row_stage_floats(w, k, T));
        }
        row_stage(dev->stream, w, tok, k, T, tabs.cos, tabs.sin, rep, scratch, kv_ready);
        stage_rows(dev, w, model, rep, k, out_n, out + (size_t)r0 * out_n, loans);
    }
}

extern "C" int tah_predict_rows_dev(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x_dev,
                                    int32_t n, int32_t out_n, float *out_dev) {
    if (!w || !model || !x_dev || !out_dev) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (n < 0) throw ArgError{"predict: bad row count"};
        if (n > 0) predict_rows(dev, w, model, x_dev, n, out_n, out_dev);
        return TAH_OK;
    });
}

extern "C" int tah_predict_rows(tah_dev *dev, const tah_weights *w, const tah_model *model, const float *x, int32_t n,
                                int32_t out_n, float *out) {
    if (!w || !model || !x || !out) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (n < 0) throw ArgError{"predict: bad row count"};
        if (n == 0) return TAH_OK;
        check_columns(w, model);
        Loans io(dev);
        float *xd = io.take<float>((size_t)n * model->features), *od = io.take<float>((size_t)n * out_n);
        TAH_HIP(hipMemcpyAsync(xd, x, sizeof(float) * n * model->features, hipMemcpyHostToDevice, dev->stream));
        predict_rows(dev, w, model, xd, n, out_n, od);
        TAH_HIP(hipMemcpyAsync(out, od, sizeof(float) * n * out_n, hipMemcpyDeviceToHost, dev->stream));
        TAH_HIP(hipStreamSynchronize(dev->stream));
        return TAH_OK;
    });
}

// ---- the column and row stages of a fit (Attend::columns + Attend::rows, cells kept on the card) -----------------

// Widest hidden layer of the column blocks' feed-forwards.
static int column_ff(const tah_weights *w) {
    int ff = 0;
    for (auto &b : w->col_a1) ff = std::max(ff, b.ff);
    for (auto &b : w->col_a2) ff = std::max(ff, b.ff);
    return ff;
}

// Working buffers of the column blocks for a batch of g feature groups of `rows` cells each.
struct ColumnBufs {
    float *t, *q, *att, *mid, *acc, *hid, *ht, *hmid, *kv2;
    void *work;
};

static size_t column_bufs_bytes(const tah_weights *w, int rows, int g) {
    const size_t M = (size_t)g * rows, I = (size_t)g * w->inds, e = w->e, ff = column_ff(w);
    return loan_bytes({M * e, M * e, M * e, M * std::max<size_t>(ff, 2 * e), I * e, I * e, I * e, I * ff, I * 2 * e}) +
           loan_raw(ind_attention_work_bytes(w, rows, g));
}

static ColumnBufs column_bufs(const tah_weights *w, int rows, int g, Loans &loans) {
    const size_t M = (size_t)g * rows, I = (size_t)g * w->inds, e = w->e, ff = column_ff(w);
    ColumnBufs b;
    b.t = loans.take<float>(M * e);
    b.q = loans.take<float>(M * e);
    b.att = loans.take<float>(M * e);
    b.mid = loans.take<float>(M * std::max<size_t>(ff, 2 * e));
    b.acc = loans.take<float>(I * e);
    b.hid = loans.take<float>(I * e);
    b.ht = loans.take<float>(I * e);
    b.hmid = loans.take<float>(I * ff);
    b.kv2 = loans.take<float>(I * 2 * e);
    b.work = loans.take<uint8_t>(ind_attention_work_bytes(w, rows, g));
    return b;
}

// Every column block for g feature groups whose cells (group-major [g][rows][e], through the input layer with the
// target's embedding added) are in `cells`, in place (src/fit.rs:366-406): per block, the inducing points' queries
// indq [blocks][inds][e] attend to the cells, the inducing points' output projection and feed-forward, their keys
// and values for the second attention written to the column cache (col_kv + g0 * gstride + off + block's place),
// then every cell through the block against them.
static void column_blocks(hipStream_t s, const tah_weights *w, float *cells, int rows, int g, const float *indq,
                          float *col_kv, size_t gstride, size_t off, int g0, const ColumnBufs &b) {
    const int e = w->e, inds = w->inds, nb = w->col_blocks;
    const size_t per = 2 * (size_t)e * inds, M = (size_t)g * rows, I = (size_t)g * inds;
    for (int bi = 0; bi < nb; bi++) {
        const DevBlock &a1 = w->col_a1[bi], &a2 = w->col_a2[bi];
        // the inducing points look at this batch's cells (src/fit.rs:366-392): the cells' keys and values, their
        // layer norm inside the projection's kernel where the block has its weight image (1,000,000 cells: 1.4 ms
        // as a norm and a product apart, each row read and written once more)
        if (a1.inimg && e == 128) {
            rows128(s, (int)M, 2 * e, cells, e, a1.inimg + (size_t)128 * e * 4, a1.ins, a1.in_b + e, b.mid, 2 * e,
                    EPI_NONE, nullptr, 0, nullptr, a1.n1w, a1.n1b);
        } else {
            layer_norm(s, (int)M, e, cells, e, a1.n1w, a1.n1b, b.t, e);
            gemm(s, (int)M, 2 * e, e, b.t, e, a1.in_w + (size_t)e * e, a1.in_b + e, b.mid, 2 * e, EPI_NONE, nullptr, 0);
        }
        ind_attention(s, w, rows, g, indq + (size_t)bi * inds * e, b.mid, b.acc, b.work);
        gemm(s, (int)I, e, e, b.acc, e, a1.out_w, a1.out_b, b.hid, e, EPI_NONE, nullptr, 0);
        add_ind(s, I * e, inds, e, w->col_ind + (size_t)bi * inds * e, b.hid);
        layer_norm(s, (int)I, e, b.hid, e, a1.n2w, a1.n2b, b.ht, e);
        gemm(s, (int)I, a1.ff, e, b.ht, e, a1.l1w, a1.l1b, b.hmid, a1.ff, EPI_GELU, nullptr, 0);
        gemm(s, (int)I, e, a1.ff, b.hmid, a1.ff, a1.l2w, a1.l2b, b.hid, e, EPI_RESID, b.hid, e);
        // their keys and values for the second attention: what prediction reuses (src/fit.rs:393-403)
        layer_norm(s, (int)I, e, b.hid, e, a2.n1w, a2.n1b, b.ht, e);
        gemm(s, (int)I, 2 * e, e, b.ht, e, a2.in_w + (size_t)e * e, a2.in_b + e, b.kv2, 2 * e, EPI_NONE, nullptr, 0);
        const size_t at = off + (size_t)bi * per;
        col_records(s, g, inds, e, b.kv2, col_kv, gstride, at, g0);
        // every cell against them (src/fit.rs:404-406)
        column_block(s, w, a2, cells, rows, g, 1, rows, col_kv + (size_t)g0 * gstride + at, gstride, b.t, b.q, b.att,
                     M * e * sizeof(float), b.mid);
    }
}

static void check_fit_weights(const tah_weights *w) {
    if (w->col_a1.empty() || w->col_a2.empty() || w->row.empty() || !w->col_ind || !w->col_scale)
        throw ArgError{"fit: the weights lack the column or row stage (upload them with the fitting blocks)"};
}

extern "C" int tah_fit_represent(tah_dev *dev, const tah_weights *w, const float *x, const float *y, int32_t rows,
                                 int32_t features, const int32_t *bases, int32_t digits, const float *ind_scales,
                                 float *col_kv_out, float *reps_out) {
    if (!w || !x || !y || !bases || !ind_scales || !col_kv_out || !reps_out) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (rows <= 0 || features <= 0 || digits <= 0) throw ArgError{"fit: bad rows, features or digits"};
        check_fit_weights(w);
        for (int i = 0; i < digits; i++)
            if (bases[i] <= 0) throw ArgError{"fit: label digit bases must be positive"};
        const int e = w->e, inds = w->inds, nb = w->col_blocks, d = w->d;
        const int T = w->cls + features;
        const size_t per = 2 * (size_t)e * inds, gstride = (size_t)digits * nb * per;
        hipStream_t s = dev->stream;
        Loans keep(dev);
        float *xd = keep.take<float>((size_t)rows * features), *yd = keep.take<float>(rows);
        float *sc = keep.take<float>((size_t)nb * e), *indq = keep.take<float>((size_t)nb * inds * e);
        float *it = keep.take<float>((size_t)inds * e);
        float *col_kv = keep.take<float>((size_t)features * gstride);
        float *emb = keep.take<float>((size_t)features * rows * e);
        float *reps = keep.take<float>((size_t)rows * d);
        TAH_HIP(hipMemcpyAsync(xd, x, sizeof(float) * rows * features, hipMemcpyHostToDevice, s));
        TAH_HIP(hipMemcpyAsync(yd, y, sizeof(float) * rows, hipMemcpyHostToDevice, s));
        TAH_HIP(hipMemcpyAsync(sc, ind_scales, sizeof(float) * nb * e, hipMemcpyHostToDevice, s));
        // the inducing points' queries, once per block, scaled for all rows (src/fit.rs:300-313)
        size_t qfloats = 0;
        for (auto &b : w->col_a1) qfloats = std::max(qfloats, query_scratch_floats(inds, b));
        Loans qloan(dev);
        float *qscr = qloan.take<float>(std::max<size_t>(qfloats, 1));
        for (int bi = 0; bi < nb; bi++) {
            const DevBlock &a1 = w->col_a1[bi];
            float *qb = indq + (size_t)bi * inds * e;
            layer_norm(s, inds, e, w->col_ind + (size_t)bi * inds * e, e, a1.n1w, a1.n1b, it, e);
            gemm(s, inds, e, e, it, e, a1.in_w, a1.in_b, qb, e, EPI_NONE, nullptr, 0);
            query_modulate(s, inds, a1, sc + (size_t)bi * e, qb, qscr);
        }
        // feature groups in batches that fit the working memory
        const int gb = batch_rows(dev, features, [&](int g) {
            const size_t M = (size_t)g * rows;
            return column_bufs_bytes(w, rows, g) + (digits > 1 ? loan_bytes({M * e, M * e}) : 0);
        });
        for (int g0 = 0; g0 < features; g0 += gb) {
            const int g = std::min(gb, features - g0);
            const size_t M = (size_t)g * rows;
            Loans loans(dev);
            float *cells = emb + (size_t)g0 * rows * e;
            const ColumnBufs cb = column_bufs(w, rows, g, loans);
            float *plain = digits > 1 ? loans.take<float>(M * e) : nullptr;
            float *sum = digits > 1 ? loans.take<float>(M * e) : nullptr;
            fit_cells(s, w, xd, rows, features, g0, g, cells);
            if (digits > 1) {
                TAH_HIP(hipMemcpyAsync(plain, cells, M * e * sizeof(float), hipMemcpyDeviceToDevice, s));
                TAH_HIP(hipMemsetAsync(sum, 0, M * e * sizeof(float), s));
            }
            for (int dg = 0; dg < digits; dg++) {
                if (dg > 0) TAH_HIP(hipMemcpyAsync(cells, plain, M * e * sizeof(float), hipMemcpyDeviceToDevice, s));
                int divisor = 1;
                for (int k = dg + 1; k < digits; k++) divisor *= bases[k];
                add_y_cells(s, w, yd, rows, g, digits, divisor, bases[dg], cells);
                column_blocks(s, w, cells, rows, g, indq, col_kv, gstride, (size_t)dg * nb * per, g0, cb);
                if (digits > 1) add_to(s, M * e, cells, sum);
            }
            if (digits > 1) scale_by(s, M * e, sum, 1.0f / (float)digits, cells);
        }
        // the row stage in batches of rows (src/fit.rs:516-539)
        const RopeTabs tabs = rope_tables(w, T);
        const int rb = batch_rows(dev, rows, [&](int k) {
            return loan_bytes({(size_t)k * T * e, row_stage_floats(w, k, T)});
        });
        for (int r0 = 0; r0 < rows; r0 += rb) {
            const int k = std::min(rb, rows - r0);
            Loans loans(dev);
            float *tok = loans.take<float>((size_t)k * T * e);
            float *scratch = loans.take<float>(row_stage_floats(w, k, T));
            tokens_gmajor(s, w, k, r0, rows, features, emb, tok);
            row_stage(s, w, tok, k, T, tabs.cos, tabs.sin, reps + (size_t)r0 * d, scratch);
        }
        TAH_HIP(hipMemcpyAsync(col_kv_out, col_kv, sizeof(float) * features * gstride, hipMemcpyDeviceToHost, s));
        TAH_HIP(hipMemcpyAsync(reps_out, reps, sizeof(float) * rows * d, hipMemcpyDeviceToHost, s));
        TAH_HIP(hipStreamSynchronize(s));
        dev->stages += 2;  // the column and the row stage
        return TAH_OK;
    });
}

// ---- the fit hooks one at a time, as fit::Attend offers them (src/fit.rs:45-74) ----------------------------------

// Bytes a tah_columns call borrows for g groups of `rows` cells.
static size_t columns_call_bytes(const tah_weights *w, int rows, int g) {
    const size_t M = (size_t)g * rows, e = w->e, nb = w->col_blocks;
    return column_bufs_bytes(w, rows, g) + loan_bytes({M * e, M * e, (size_t)g * nb * 2 * e * w->inds, nb * w->inds * e});
}

// Bytes a tah_rows call borrows for n rows of `features` cells.
static size_t rows_call_bytes(const tah_weights *w, int n, int features) {
    const size_t T = (size_t)w->cls + features, k = n;
    return loan_bytes({k * features * w->e, k * T * w->e, k * w->d, row_stage_floats(w, n, (int)T)});
}

// The room the budget leaves now, read under the device's lock.
static size_t room_of(const tah_dev *dev_) {
    auto *dev = const_cast<tah_dev *>(dev_);
    std::lock_guard<std::mutex> g(dev->lock);
    const size_t used = busy_bytes(dev->pool);
    return dev->pool.budget > used ? dev->pool.budget - used : 0;
}

// The largest count up to cap whose bytes (growing with the count) fit the room; 0 if not even one does.
template <class F>
static size_t largest_fitting(size_t room, int cap, F bytes_of) {
    int lo = 0, hi = std::max(cap, 1);  // lo fits (or is 0), everything above hi is out of reach
    while (lo < hi) {
        const int mid = lo + (hi - lo + 1) / 2;
        if (bytes_of(mid) <= room)
            lo = mid;
        else
            hi = mid - 1;
    }
    return (size_t)lo;
}

extern "C" size_t tah_column_batch(const tah_dev *dev, const tah_weights *w, int32_t rows) {
    if (!dev || !w || rows <= 0 || w->col_a1.empty() || w->col_a2.empty() || !w->col_ind || !w->col_scale) return 0;
    // a batch's cells are one launch's rows at most
    const int cap = (int)std::min<long>(4096, std::max<long>(1, 0x7FFFFFFFL / ((long)rows * w->e)));
    return largest_fitting(room_of(dev), cap, [&](int g) { return columns_call_bytes(w, rows, g); });
}

extern "C" int tah_columns(tah_dev *dev, const tah_weights *w, float *cells, int32_t rows, int32_t groups,
                           const float *ind_q, float *rec) {
    if (!w || !cells || !ind_q || !rec) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (rows <= 0 || groups <= 0) throw ArgError{"columns: bad rows or groups"};
        check_fit_weights(w);
        const size_t room = dev->pool.budget > busy_bytes(dev->pool) ? dev->pool.budget - busy_bytes(dev->pool) : 0;
        if (columns_call_bytes(w, rows, groups) > room)
            throw BudgetError{"graphics card: these feature groups do not fit the working-memory budget "
                              "(tah_column_batch says how many do)"};
        const int e = w->e, inds = w->inds, nb = w->col_blocks;
        const size_t M = (size_t)groups * rows, per = 2 * (size_t)e * inds, gstride = (size_t)nb * per;
        hipStream_t s = dev->stream;
        Loans loans(dev);
        float *by_row = loans.take<float>(M * e), *by_group = loans.take<float>(M * e);
        float *rec_d = loans.take<float>((size_t)groups * gstride), *indq = loans.take<float>((size_t)nb * inds * e);
        const ColumnBufs cb = column_bufs(w, rows, groups, loans);
        TAH_HIP(hipMemcpyAsync(by_row, cells, M * e * sizeof(float), hipMemcpyHostToDevice, s));
        TAH_HIP(hipMemcpyAsync(indq, ind_q, (size_t)nb * inds * e * sizeof(float), hipMemcpyHostToDevice, s));
        regroup(s, rows, groups, e, by_row, by_group, true);
        column_blocks(s, w, by_group, rows, groups, indq, rec_d, gstride, 0, 0, cb);
        regroup(s, rows, groups, e, by_group, by_row, false);
        TAH_HIP(hipMemcpyAsync(cells, by_row, M * e * sizeof(float), hipMemcpyDeviceToHost, s));
        TAH_HIP(hipMemcpyAsync(rec, rec_d, (size_t)groups * gstride * sizeof(float), hipMemcpyDeviceToHost, s));
        TAH_HIP(hipStreamSynchronize(s));
        dev->stages++;
        return TAH_OK;
    });
}

extern "C" size_t tah_row_batch(const tah_dev *dev, const tah_weights *w, int32_t features) {
    if (!dev || !w || features <= 0 || w->row.empty() || !w->cls_tokens) return 0;
    return largest_fitting(room_of(dev), 32768, [&](int n) { return rows_call_bytes(w, n, features); });
}

extern "C" int tah_rows(tah_dev *dev, const tah_weights *w, const float *cells, int32_t n, int32_t features,
                        float *reps) {
    if (!w || !cells || !reps) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (n <= 0 || features <= 0) throw ArgError{"rows: bad row or feature count"};
        if (w->row.empty() || !w->cls_tokens) throw ArgError{"weights lack the row stage"};
        const size_t room = dev->pool.budget > busy_bytes(dev->pool) ? dev->pool.budget - busy_bytes(dev->pool) : 0;
        if (rows_call_bytes(w, n, features) > room)
            throw BudgetError{"graphics card: these rows do not fit the working-memory budget (tah_row_batch says how "
                              "many do)"};
        const int T = w->cls + features, e = w->e;
        hipStream_t s = dev->stream;
        const RopeTabs tabs = rope_tables(w, T);
        Loans loans(dev);
        float *cd = loans.take<float>((size_t)n * features * e), *tok = loans.take<float>((size_t)n * T * e);
        float *rd = loans.take<float>((size_t)n * w->d), *scratch = loans.take<float>(row_stage_floats(w, n, T));
        TAH_HIP(hipMemcpyAsync(cd, cells, sizeof(float) * n * features * e, hipMemcpyHostToDevice, s));
        assemble_tokens(s, w, cd, n, features, tok);
        row_stage(s, w, tok, n, T, tabs.cos, tabs.sin, rd, scratch);
        TAH_HIP(hipMemcpyAsync(reps, rd, sizeof(float) * n * w->d, hipMemcpyDeviceToHost, s));
        TAH_HIP(hipStreamSynchronize(s));
        dev->stages++;
        return TAH_OK;
    });
}

// Bytes tah_attend (or tah_attend_rows with nq queries) borrows for keys and values of `rows` rows.
static size_t attend_call_bytes(int nq, int rows, int d, int heads) {
    const AttnShape a{nq, rows, 256, d, heads, TAH_KV_F32};
    size_t b = loan_bytes({(size_t)nq * d, 2 * (size_t)rows * d, 2 * (size_t)rows * d, (size_t)nq * d}) +
               loan_raw(attention_work_bytes(a));
    if (nq >= TAH_SPLIT16_MIN_Q && kv_images_apply(TAH_KV_F32, d, heads)) b += loan_raw(kv_images_bytes(rows, 256, heads, TAH_KV_F32));
    return b;
}

extern "C" int tah_attend_fits(const tah_dev *dev, int32_t rows, int32_t d) {
    if (!dev || rows <= 0 || d <= 0) return 0;
    const int heads = std::max(1, d / 64);  // head width 64 or less: what the attention kernels take
    if (d % heads != 0 || d / heads > 64) return 0;
    return attend_call_bytes(rows, rows, d, heads) <= dev->pool.budget ? 1 : 0;
}

// Attention outputs [nq][d] of queries q over row-major keys k and values v [n][d], all on the host.
static void attend_rows_on(tah_dev *dev, const float *q, const float *k, const float *v, int nq, int n, int d, int heads,
                           float *out) {
    hipStream_t s = dev->stream;
    Loans loans(dev);
    const int chunk = 256;
    float *qd = loans.take<float>((size_t)nq * d), *kv = loans.take<float>(2 * (size_t)n * d);
    float *rec = loans.take<float>(2 * (size_t)n * d), *od = loans.take<float>((size_t)nq * d);
    const AttnShape a{nq, n, chunk, d, heads, TAH_KV_F32};
    void *work = loans.take<uint8_t>(attention_work_bytes(a));
    TAH_HIP(hipMemcpyAsync(qd, q, sizeof(float) * nq * d, hipMemcpyHostToDevice, s));
    // keys and values each in one contiguous upload (rec as staging), then side by side on the card, [n][2d], as the
    // projection leaves them at fit
    TAH_HIP(hipMemcpyAsync(rec, k, sizeof(float) * n * d, hipMemcpyHostToDevice, s));
    TAH_HIP(hipMemcpyAsync(rec + (size_t)n * d, v, sizeof(float) * n * d, hipMemcpyHostToDevice, s));
    TAH_HIP(hipMemcpy2DAsync(kv, 2 * d * sizeof(float), rec, d * sizeof(float), d * sizeof(float), n,
                             hipMemcpyDeviceToDevice, s));
    TAH_HIP(hipMemcpy2DAsync(kv + d, 2 * d * sizeof(float), rec + (size_t)n * d, d * sizeof(float), d * sizeof(float), n,
                             hipMemcpyDeviceToDevice, s));
    to_records(s, n, d, chunk, kv, rec);
    KvImages img;
    const KvImages *imgp = loan_images(s, loans, a, reinterpret_cast<const uint8_t *>(rec), img);
    attention(s, a, qd, reinterpret_cast<const uint8_t *>(rec), od, work, imgp);
    TAH_HIP(hipMemcpyAsync(out, od, sizeof(float) * nq * d, hipMemcpyDeviceToHost, s));
    TAH_HIP(hipStreamSynchronize(s));
}

extern "C" int tah_attend_rows(tah_dev *dev, const float *q, const float *k, const float *v, int32_t nq, int32_t n,
                               int32_t d, int32_t heads, float *out) {
    if (!q || !k || !v || !out) return TAH_E_ARG;
    return guarded(dev, [&] {
        if (nq < 0 || n <= 0 || d <= 0 || heads <= 0 || d % heads) throw ArgError{"attend_rows: bad shape"};
        if (nq > 0) attend_rows_on(dev, q, k, v, nq, n, d, heads, out);
        return TAH_OK;
    });
}

extern "C" int tah_calibrate(tah_dev *dev, double ms, double *rate) {
    if (!rate) return TAH_E_ARG;
    return guarded(dev, [&] {
        const int nq = 256, n = 2048, d = 512, heads = 8;
        // fixed pseudo-random inputs in [-0.5, 0.5): a 64-bit linear congruential sequence, top 24 bits
        std::vector<float> q((size_t)nq * d), k((size_t)n * d), v((size_t)n * d), out((size_t)nq * d);
        uint64_t st = 0x9E3779B97F4A7C15ull;
        auto next = [&] {
            st = st * 6364136223846793005ull + 1442695040888963407ull;
            return (float)(st >> 40) / (float)(1u << 24) - 0.5f;
        };
        for (auto *vec : {&q, &k, &v})
            for (float &x : *vec) x = next();
        double best = 0.0, spent = 0.0;
        for (int i = 0;; i++) {
            const auto t0 = std::chrono::steady_clock::now();
            attend_rows_on(dev, q.data(), k.data(), v.data(), nq, n, d, heads, out.data());
            const double secs = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            spent += secs;
            // multiply-adds of the scores and of the weighted values
            best = std::max(best, 2.0 * nq * n * d / std::max(secs, 1e-9));
            if (i >= 2 && spent * 1e3 > ms) break;
        }
        *rate = best;
        return TAH_OK;
    });
}

extern "C" uint64_t tah_stages(const tah_dev *dev) { return dev ? dev->stages.load() : 0; }

extern "C" int tah_probe_attention(tah_dev *dev, int32_t launches) {
    return guarded(dev, [&] {
        probe_arm(dev->stream, launches);
        return TAH_OK;
    });
}

extern "C" int tah_probe_read(tah_dev *dev, double *ms, int32_t *launches) {
    if (!ms || !launches) return TAH_E_ARG;
    return guarded(dev, [&] {
        *launches = probe_read(dev->stream, ms);
        return TAH_OK;
    });
}
