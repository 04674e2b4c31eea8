// vocalarc_hip.h: the shape-generic device path (isolated kernels, model
// upload, STFT -> band split -> axial stack -> mask -> iSTFT, chunked
// separation).
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "dsp.hpp"
#include "elementwise.hpp"
#include "runtime.hpp"

using namespace vh;

// Physical activation layout of the device pipeline: [chunk][T][B][D] (one
// row per (frame, band) token).  The time axis reads it with pos_stride B, the
// band axis with pos_stride 1, so neither axis needs a transpose.
static AttnLayout time_axis_layout(int chunks, int T, int B) {
    return {chunks * B, T, B, T * B, 1, B};
}
static AttnLayout band_axis_layout(int chunks, int T, int B) {
    return {chunks * T, B, 1, B, 0, 1};
}
static AttnLayout contiguous_layout(int S, int L) { return {S, L, 1, L, 0, 1}; }

struct vh_model;

struct vh_context {
    hipStream_t stream = nullptr;
    std::vector<vh_model *> models;  // live models (vh_destroy frees those left)
    int device = 0;
    char name[256] = "";
    KernelTimer timer;
    RopeCache rope;
    BlockScratch scratch;
    DeviceBuffer staging;
    // vh_gemm_h2's computed A bound (float 0), vh_transformer's stream bound
    // (float 8) and the absmax scratch (from float 64)
    DeviceBuffer bounds;
};

struct vh_model {
    vh_context *ctx = nullptr;
    Dims d;
    DeviceBuffer weights;
    std::vector<LayerWeights> layers;  // [depth][2]
    std::vector<float *> band_gamma, band_w, band_b;
    float *final_gamma = nullptr;
    std::vector<float *> mask_w1, mask_b1, mask_w2, mask_b2;
    std::vector<int> first_freq;
    // bf16 copies of every matrix (built on the first switch to bf16)
    int precision = PREC_FP32;
    DeviceBuffer weights_h;
    // fp16 two-piece planes of the transformer and mask-estimator matrices and
    // the bounds of their A operands (built at load): per layer 4 floats
    // (layer_bounds), then the mask estimator's feature bound, then absmax
    // scratch
    DeviceBuffer weights_s, bounds;
    std::vector<void *> mask_w1_s, mask_w2_s;
    std::vector<void *> band_w_h, mask_w1_h, mask_w2_h;
    // DSP constants
    DeviceBuffer window, twiddle;
    // pipeline scratch (grown on demand)
    DeviceBuffer source, x, normed, mask, bandin, mhidden, proj, frames, chunk_out, starts, tables;
    int64_t band_in_total = 0;   // sum over bands of 4w (floats per spectrogram row)
    int64_t proj_total = 0;      // sum over bands of 8w
};

// ------------------------------------------------------------------ context
// ------------------------------------------------- no-allocation scratch
// Device scratch of vh_attention_noalloc: float 0 the operand bound,
// [64, 64 + ABSMAX_PARTIALS) the absmax partials, then the interleaved rotary
// table of VH_NOALLOC_MAX_LENGTH positions (1.05 MB in all).  Each device
// holds its own copy for the life of the process.  Host code never uses the
// array's name as an address: noalloc_scratch[device] holds the device
// address from hipGetSymbolAddress, resolved by vh_create with the device
// current, which also writes the rotary table there once: an entry depends
// only on its position and pair, so every length's table is its prefix.
constexpr size_t NOALLOC_ROPE_OFFSET = 64 + ABSMAX_PARTIALS;
constexpr size_t NOALLOC_FLOATS = NOALLOC_ROPE_OFFSET + (size_t)VH_NOALLOC_MAX_LENGTH * 64;
static __device__ __align__(256) float scratch[NOALLOC_FLOATS];

constexpr int NOALLOC_MAX_DEVICES = 64;
static std::mutex noalloc_mutex;  // guards noalloc_scratch
static float *noalloc_scratch[NOALLOC_MAX_DEVICES] = {};

// With `device` current: its scratch address and rotary table (once per
// device).
static bool resolve_noalloc_scratch(int device) {
    if (device < 0 || device >= NOALLOC_MAX_DEVICES) {
        set_error("no-allocation scratch: device %d beyond %d", device, NOALLOC_MAX_DEVICES);
        return false;
    }
    std::lock_guard<std::mutex> lock(noalloc_mutex);
    if (noalloc_scratch[device]) return true;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        set_error("hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        return false;
    }
    std::vector<float> rope((size_t)VH_NOALLOC_MAX_LENGTH * 64);
    rope_table_host(VH_NOALLOC_MAX_LENGTH, 64, nullptr, nullptr, rope.data());
    if (!check(hipMemcpy(static_cast<float *>(p) + NOALLOC_ROPE_OFFSET, rope.data(), rope.size() * sizeof(float),
                         hipMemcpyHostToDevice),
               "hipMemcpy(no-allocation rotary table)"))
        return false;
    noalloc_scratch[device] = static_cast<float *>(p);
    return true;
}

extern "C" vh_context *vh_create(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        set_error("no HIP device");
        return nullptr;
    }
    vh_context *ctx = new vh_context();
    if (!check(hipSetDevice(0), "hipSetDevice") || !resolve_noalloc_scratch(0)) {
        delete ctx;
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) == hipSuccess) snprintf(ctx->name, sizeof(ctx->name), "%s (%s)", prop.name, prop.gcnArchName);
    return ctx;
}

extern "C" void vh_destroy(vh_context *ctx) {
    if (!ctx) return;
    (void)hipStreamSynchronize(ctx->stream);
    for (vh_model *m : ctx->models) delete m;  // models not freed by their owner
    ctx->models.clear();
    ctx->timer.reset();
    delete ctx;
}

extern "C" int vh_set_stream(vh_context *ctx, void *s) {
    if (!ctx) return 0;
    ctx->stream = (hipStream_t)s;
    return 1;
}

extern "C" int vh_synchronize(vh_context *ctx) {
    if (!ctx) return 0;
    bool ok = check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    ctx->timer.collect();
    return ok ? 1 : 0;
}

extern "C" const char *vh_last_error(void) { return last_error(); }
extern "C" const char *vh_device_name(vh_context *ctx) { return ctx ? ctx->name : ""; }

// --------------------------------------------------------- isolated kernels
extern "C" int vh_rmsnorm(vh_context *ctx, int64_t rows, int dim, const float *x, const float *gamma, float *y) {
    if (!ctx) return 0;
    return rmsnorm(ctx->stream, x, dim, gamma, y, dim, rows, dim, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_rmsnorm_bf16(vh_context *ctx, int64_t rows, int dim, const float *x, const float *gamma, void *y) {
    if (!ctx) return 0;
    return rmsnorm_bf16(ctx->stream, x, dim, gamma, y, dim, rows, dim, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_rmsnorm_h2(vh_context *ctx, int64_t rows, int dim, const float *x, const float *gamma,
                             const float *bound, float *y) {
    if (!ctx) return 0;
    return rmsnorm_h2(ctx->stream, x, dim, gamma, y, dim, rows, dim, bound, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_softmax_rows(vh_context *ctx, int64_t rows, int len, const float *in, float *out) {
    if (!ctx) return 0;
    return softmax_rows(ctx->stream, in, out, rows, len, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_rope_bhld(vh_context *ctx, int64_t bh, int len, int dim_head, float *x) {
    if (!ctx || dim_head != 64) {
        set_error("vh_rope_bhld: dim_head must be 64");
        return 0;
    }
    const float *cs, *sn;
    if (!ctx->rope.get(len, dim_head, ctx->stream, &cs, &sn)) return 0;
    return rope_bhld(ctx->stream, x, cs, sn, bh, len, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_geglu(vh_context *ctx, int64_t rows, int width, const float *in, float *out) {
    if (!ctx) return 0;
    return geglu(ctx->stream, in, out, rows, width, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_residual_add(vh_context *ctx, int64_t n, float *x, const float *r) {
    if (!ctx) return 0;
    return residual_add(ctx->stream, x, r, n, &ctx->timer) ? 1 : 0;
}

extern "C" int vh_gemm(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, const float *W, int ldw,
                       const float *bias, float *C, int ldc, int epilogue) {
    if (!ctx) return 0;
    return gemm(ctx->stream, {A, lda, W, ldw, bias, C, ldc, M, N, K}, epilogue, &ctx->timer, "gemm") ? 1 : 0;
}

extern "C" int vh_gemm_bf16(vh_context *ctx, int64_t M, int N, int K, const void *A, int lda, const void *Wh, int ldw,
                            const float *bias, void *C, int ldc, int epilogue, int flags) {
    if (!ctx || (flags & ~(VH_BF16_A | VH_BF16_C | VH_BF16_STAGED))) return 0;
    GemmArgsBF16 g{A, lda, Wh, ldw, bias, C, ldc, M, N, K};
    g.a_bf16 = (flags & VH_BF16_A) != 0;
    g.c_bf16 = (flags & VH_BF16_C) != 0;
    g.staged = (flags & VH_BF16_STAGED) != 0;
    return gemm_bf16(ctx->stream, g, epilogue, &ctx->timer, "gemm_bf16") ? 1 : 0;
}

extern "C" int vh_gemm_split(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, const void *Ws,
                             const float *bias, float *C, int ldc, int epilogue) {
    if (!ctx) return 0;
    GemmArgsSplit g{A, lda, Ws, bias, C, ldc, M, N, K};
    return gemm_split(ctx->stream, g, epilogue, &ctx->timer, "gemm_split") ? 1 : 0;
}

extern "C" size_t vh_split_bytes(int N, int K) { return N > 0 && K > 0 ? split_bytes(N, K) : 0; }

extern "C" int vh_split_weights(vh_context *ctx, int N, int K, const float *W, int ldw_in, void *Ws) {
    if (!ctx || !W || !Ws) {
        set_error("vh_split_weights: null argument");
        return 0;
    }
    return split_weights(ctx->stream, W, N, K, ldw_in, Ws) ? 1 : 0;
}

extern "C" int vh_gemm_h2(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, float a_bound,
                          const void *Wp, const float *bias, float *C, int ldc, int epilogue, int flags) {
    if (!ctx || (flags & ~VH_H2_A_ROWS)) return 0;
    GemmArgsH2 g{A, lda, Wp, bias, C, ldc, M, N, K};
    g.a_h2 = (flags & VH_H2_A_ROWS) != 0;
    OperandBound b{nullptr, a_bound};
    if (g.a_h2 && !(a_bound > 0.0f)) {
        set_error("vh_gemm_h2: h2 rows need the bound they were split with");
        return 0;
    }
    if (!(a_bound > 0.0f)) {
        // the caller gave no bound: A's own maximum
        if (M <= 0 || K <= 0 || lda < K || !A) {
            set_error("vh_gemm_h2: bad shape M=%lld K=%d lda=%d", (long long)M, K, lda);
            return 0;
        }
        if (!ctx->bounds.ensure((64 + ABSMAX_PARTIALS) * sizeof(float), "hipMalloc(operand bound)") ||
            !absmax(ctx->stream, A, (M - 1) * lda + K, ctx->bounds.f() + 64, ctx->bounds.f()))
            return 0;
        b.dev = ctx->bounds.f();
    }
    return gemm_h2(ctx->stream, g, b, epilogue, &ctx->timer, "gemm_h2") ? 1 : 0;
}

extern "C" int vh_gemm_h2_ex(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda,
                             const float *a_bound_dev, const void *Wp, const float *bias, float *C, int ldc,
                             int epilogue, int flags, float *zero_slot, float *amax) {
    if (!ctx || !a_bound_dev || (flags & ~VH_H2_ROW_NORM)) {
        set_error("vh_gemm_h2_ex: null context or bound, or unknown flags %d", flags);
        return 0;
    }
    GemmArgsH2 g{A, lda, Wp, bias, C, ldc, M, N, K};
    g.row_norm = (flags & VH_H2_ROW_NORM) != 0;
    g.zero_slot = zero_slot;
    g.amax = amax;
    return gemm_h2(ctx->stream, g, OperandBound{a_bound_dev, 0.0f}, epilogue, &ctx->timer, "gemm_h2") ? 1 : 0;
}

extern "C" size_t vh_h2_bytes(int N, int K) { return N > 0 && K > 0 ? h2_bytes(N, K) : 0; }

extern "C" int vh_split_weights_h2(vh_context *ctx, int N, int K, const float *W, int ldw_in, void *Wp) {
    if (!ctx || !W || !Wp) {
        set_error("vh_split_weights_h2: null argument");
        return 0;
    }
    return split_weights_h2(ctx->stream, W, N, K, ldw_in, Wp) ? 1 : 0;
}

extern "C" int vh_operand_bounds(vh_context *ctx, const float *gamma, int D, const float *W, int N, const float *b,
                                 int square, float *out) {
    if (!ctx) return 0;
    return operand_bounds(ctx->stream, gamma, D, W, N, b, square != 0, out) ? 1 : 0;
}

extern "C" int vh_to_bf16(vh_context *ctx, int64_t rows, int cols, const float *src, void *dst, int ld) {
    if (!ctx || rows <= 0 || cols <= 0 || ld < cols || rows * (int64_t)cols > INT32_MAX) return 0;
    return to_bf16_rows(ctx->stream, src, (int)rows, cols, dst, ld) ? 1 : 0;
}

extern "C" int vh_attention(vh_context *ctx, int sequences, int length, int heads, const void *qkv, void *out,
                            int apply_rotary, int flags) {
    if (!ctx || (flags & ~(VH_ATT_OUT_BF16 | VH_ATT_BF16 | VH_ATT_SPLIT | VH_ATT_H2 | VH_ATT_OUT_H2))) return 0;
    const float *rt = nullptr;
    if (apply_rotary && !ctx->rope.get_interleaved(length, 64, ctx->stream, &rt)) return 0;
    const int inner = heads * 64;
    const bool h2 = (flags & VH_ATT_H2) && !(flags & VH_ATT_BF16);
    bool h2_ok = false;
    if (h2) {  // the operands' own maximum bounds them
        if (sequences <= 0 || length <= 0 || heads <= 0 || !qkv ||
            !ctx->bounds.ensure((64 + ABSMAX_PARTIALS) * sizeof(float), "hipMalloc(operand bound)") ||
            !absmax(ctx->stream, static_cast<const float *>(qkv), (int64_t)sequences * length * 3 * inner,
                    ctx->bounds.f() + 64, ctx->bounds.f()))
            return 0;
        // outside the two-piece attention's scale range (or not finite): the
        // products run on the kernels without piece scales
        float b = 0.0f;
        if (bounds_usable(ctx->stream, ctx->bounds.f(), 1, &b) < 0) return 0;
        h2_ok = h2_attention_bound_ok(b);
    }
    const bool out_h2 = (flags & VH_ATT_OUT_H2) != 0;
    if (out_h2 && !h2_ok) {
        set_error("vh_attention: VH_ATT_OUT_H2 needs the two-piece kernel (VH_ATT_H2, fp32, max|qkv| in its range)");
        return 0;
    }
    return attention(ctx->stream, qkv, 3 * inner, out, inner, rt, contiguous_layout(sequences, length), heads, -1,
                     &ctx->timer, (flags & VH_ATT_OUT_BF16) != 0, (flags & VH_ATT_BF16) != 0,
                     (flags & (VH_ATT_SPLIT | VH_ATT_H2)) != 0, h2_ok ? ctx->bounds.f() : nullptr, out_h2)
               ? 1
               : 0;
}

extern "C" int vh_attention_noalloc(vh_context *ctx, int sequences, int length, int heads, const void *qkv, void *out,
                                    int apply_rotary, int flags) {
    if (!ctx || (flags & ~(VH_ATT_OUT_BF16 | VH_ATT_BF16 | VH_ATT_SPLIT | VH_ATT_H2))) {
        set_error("vh_attention_noalloc: bad context or flags");
        return 0;
    }
    if (sequences <= 0 || length <= 0 || heads <= 0 || !qkv || !out) {
        set_error("vh_attention_noalloc: bad shape S=%d L=%d H=%d", sequences, length, heads);
        return 0;
    }
    if (length > VH_NOALLOC_MAX_LENGTH) {
        set_error("vh_attention_noalloc: length %d exceeds the %d positions of the no-allocation scratch", length,
                  VH_NOALLOC_MAX_LENGTH);
        return 0;
    }
    float *scr = nullptr;
    {
        std::lock_guard<std::mutex> lock(noalloc_mutex);
        scr = ctx->device >= 0 && ctx->device < NOALLOC_MAX_DEVICES ? noalloc_scratch[ctx->device] : nullptr;
    }
    if (!scr) {
        set_error("vh_attention_noalloc: scratch of device %d not resolved", ctx->device);
        return 0;
    }
    // the table vh_create wrote (bit for bit vh_attention's, whose length-L
    // table is a prefix of it); no copy and no synchronisation here
    const float *rt = apply_rotary ? scr + NOALLOC_ROPE_OFFSET : nullptr;
    const int inner = heads * 64;
    const bool h2 = (flags & VH_ATT_H2) && !(flags & VH_ATT_BF16);
    if (h2) {
        // as vh_attention: the operands' own maximum bounds them (every
        // partial written before it is read); the kernels choose between the
        // two-piece products and those without piece scales on the device
        if (!absmax(ctx->stream, static_cast<const float *>(qkv), (int64_t)sequences * length * 3 * inner, scr + 64,
                    scr))
            return 0;
    }
    return attention(ctx->stream, qkv, 3 * inner, out, inner, rt, contiguous_layout(sequences, length), heads, -1,
                     nullptr, (flags & VH_ATT_OUT_BF16) != 0, (flags & VH_ATT_BF16) != 0,
                     (flags & (VH_ATT_SPLIT | VH_ATT_H2)) != 0, h2 ? scr : nullptr, false, false, h2)
               ? 1
               : 0;
}

// -------------------------------------------------------------------- model
namespace {

struct PackReader {
    const unsigned char *cur, *end;
    const float *next(uint64_t expect) {
        if ((size_t)(end - cur) < 8) return nullptr;
        uint64_t n;
        memcpy(&n, cur, 8);
        cur += 8;
        if (n != expect || (size_t)(end - cur) < n * sizeof(float)) return nullptr;
        const float *r = reinterpret_cast<const float *>(cur);
        cur += n * sizeof(float);
        return r;
    }
};

// Bump allocator over the model's single weight allocation (256-byte aligned).
struct Arena {
    size_t used = 0;
    char *base = nullptr;
    float *take(size_t floats) {
        float *p = reinterpret_cast<float *>(base + used);
        used += (floats * sizeof(float) + 255) & ~(size_t)255;
        return p;
    }
};

size_t model_weight_bytes(const Dims &d) {
    auto r = [](size_t floats) { return (floats * sizeof(float) + 255) & ~(size_t)255; };
    size_t b = 0;
    const size_t D = d.dim;
    for (int l = 0; l < d.depth * 2; l++) {
        b += 2 * r(D);
        b += r((size_t)d.qkvg_dim() * D) + r(d.qkvg_dim());
        b += r(D * d.inner());
        b += r((size_t)d.ff1_out() * D) + r(d.ff1_out());
        b += r(D * d.ff_dim) + r(D);
    }
    for (int k = 0; k < d.bands; k++) b += r(d.in_dim(k)) + r(D * d.in_dim(k)) + r(D);
    b += r(D);
    for (int k = 0; k < d.bands; k++)
        b += r((size_t)d.mask_hidden * D) + r(d.mask_hidden) + r((size_t)2 * d.in_dim(k) * d.mask_hidden) +
             r(2 * d.in_dim(k));
    return b;
}

bool upload_pack(vh_model *m, const void *pack, size_t bytes) {
    const Dims &d = m->d;
    hipStream_t s = m->ctx->stream;
    if (bytes < 64 || memcmp(pack, "VSCNAT01", 8) != 0) {
        set_error("pack: bad magic");
        return false;
    }
    uint32_t f[14];
    memcpy(f, (const char *)pack + 8, sizeof(f));
    if (f[0] != 1 || f[1] != (uint32_t)d.dim || f[2] != (uint32_t)d.depth || f[3] != (uint32_t)d.bands ||
        f[4] != (uint32_t)d.heads || f[5] != (uint32_t)d.dim_head || f[6] != (uint32_t)d.freq_bins() ||
        f[7] != (uint32_t)d.channels || f[8] != (uint32_t)d.n_fft || f[9] != (uint32_t)d.hop) {
        set_error("pack: header does not match the model shape");
        return false;
    }
    if (!m->weights.ensure(model_weight_bytes(d), "hipMalloc(model weights)")) return false;
    if (!check(hipMemsetAsync(m->weights.ptr, 0, m->weights.bytes, s), "hipMemset(model weights)")) return false;
    Arena ar;
    ar.base = static_cast<char *>(m->weights.ptr);
    PackReader rd{(const unsigned char *)pack + 64, (const unsigned char *)pack + bytes};
    const int D = d.dim, H = d.heads, inner = d.inner(), nq = d.qkvg_dim();
    DeviceBuffer &stg = m->ctx->staging;
    std::vector<float> zeros;
    m->layers.resize((size_t)d.depth * 2);
    for (int l = 0; l < d.depth * 2; l++) {
        LayerWeights &w = m->layers[l];
        w.gamma = ar.take(D);
        w.wqkvg = ar.take((size_t)nq * D);
        w.bqkvg = ar.take(nq);
        w.wout = ar.take((size_t)D * inner);
        w.ff_gamma = ar.take(D);
        w.w1 = ar.take((size_t)d.ff1_out() * D);
        w.b1 = ar.take(d.ff1_out());
        w.w2 = ar.take((size_t)D * d.ff_dim);
        w.b2 = ar.take(D);
        const float *gamma = rd.next(D), *qkv = rd.next((uint64_t)3 * inner * D), *gw = rd.next((uint64_t)H * D),
                    *gb = rd.next(H), *wo = rd.next((uint64_t)D * inner), *fg = rd.next(D),
                    *w1 = rd.next((uint64_t)d.ff1_out() * D), *b1 = rd.next(d.ff1_out()),
                    *w2 = rd.next((uint64_t)D * d.ff_dim), *b2 = rd.next(D);
        if (!gamma || !qkv || !gw || !gb || !wo || !fg || !w1 || !b1 || !w2 || !b2) {
            set_error("pack: truncated or mis-sized transformer tensor (layer %d axis %d)", l / 2, l % 2);
            return false;
        }
        if (!upload_vector(s, gamma, D, w.gamma) || !upload_vector(s, fg, D, w.ff_gamma)) return false;
        if (!upload_weight(s, qkv, D, 3 * inner, w.wqkvg, D, 0, 0, stg)) return false;
        if (d.gated) {
            if (!upload_weight(s, gw, D, H, w.wqkvg, D, 3 * inner, 0, stg)) return false;
            if (!upload_vector(s, gb, H, w.bqkvg + 3 * inner)) return false;
        }
        if (!upload_weight(s, wo, inner, D, w.wout, inner, 0, 0, stg)) return false;
        if (!upload_weight(s, w1, D, d.ff1_out(), w.w1, D, 0, d.ffn_glu ? 1 : 0, stg)) return false;
        if (d.ffn_glu) {
            if (!stg.ensure((size_t)d.ff1_out() * sizeof(float), "hipMalloc(staging)")) return false;
            if (!upload_vector(s, b1, d.ff1_out(), stg.f())) return false;
            if (!interleave_glu_bias(s, stg.f(), w.b1, d.ff1_out())) return false;
            if (!check(hipStreamSynchronize(s), "sync")) return false;
        } else if (!upload_vector(s, b1, d.ff1_out(), w.b1)) {
            return false;
        }
        if (!upload_weight(s, w2, d.ff_dim, D, w.w2, d.ff_dim, 0, 0, stg)) return false;
        if (!upload_vector(s, b2, D, w.b2)) return false;
    }
    for (int k = 0; k < d.bands; k++) {
        const int in = d.in_dim(k);
        const float *g = rd.next(in), *w = rd.next((uint64_t)D * in), *b = rd.next(D);
        if (!g || !w || !b) {
            set_error("pack: truncated band-split tensor (band %d)", k);
            return false;
        }
        m->band_gamma.push_back(ar.take(in));
        m->band_w.push_back(ar.take((size_t)D * in));
        m->band_b.push_back(ar.take(D));
        if (!upload_vector(s, g, in, m->band_gamma.back()) || !upload_weight(s, w, in, D, m->band_w.back(), in, 0, 0, stg) ||
            !upload_vector(s, b, D, m->band_b.back()))
            return false;
    }
    const float *fg = rd.next(D);
    if (!fg) {
        set_error("pack: missing final gamma");
        return false;
    }
    m->final_gamma = ar.take(D);
    if (!upload_vector(s, fg, D, m->final_gamma)) return false;
    for (int k = 0; k < d.bands; k++) {
        const int in = d.in_dim(k), Hm = d.mask_hidden;
        const float *w1 = rd.next((uint64_t)Hm * D), *b1 = rd.next(Hm), *w2 = rd.next((uint64_t)2 * in * Hm),
                    *b2 = rd.next((uint64_t)2 * in);
        if (!w1 || !b1 || !w2 || !b2) {
            set_error("pack: truncated mask tensor (band %d)", k);
            return false;
        }
        m->mask_w1.push_back(ar.take((size_t)Hm * D));
        m->mask_b1.push_back(ar.take(Hm));
        m->mask_w2.push_back(ar.take((size_t)2 * in * Hm));
        m->mask_b2.push_back(ar.take(2 * in));
        if (!upload_weight(s, w1, D, Hm, m->mask_w1.back(), D, 0, 0, stg) || !upload_vector(s, b1, Hm, m->mask_b1.back()) ||
            !upload_weight(s, w2, Hm, 2 * in, m->mask_w2.back(), Hm, 0, 0, stg) ||
            !upload_vector(s, b2, 2 * in, m->mask_b2.back()))
            return false;
    }
    if (rd.cur != rd.end) {
        set_error("pack: %zu trailing bytes", (size_t)(rd.end - rd.cur));
        return false;
    }
    // DSP constants: the reference's float window expression and an exact
    // double twiddle table.
    const int N = d.n_fft;
    std::vector<float> win(N);
    for (int i = 0; i < N; i++) win[i] = 0.5f - 0.5f * cosf((float)(2.0 * 3.141592653589793238462643383279502884 * i / N));
    std::vector<double2_t> tw(N / 2);
    for (int j = 0; j < N / 2; j++) {
        const double a = -2.0 * 3.141592653589793238462643383279502884 * j / N;
        tw[j] = {cos(a), sin(a)};
    }
    if (!m->window.ensure(N * sizeof(float), "hipMalloc(window)") ||
        !m->twiddle.ensure(tw.size() * sizeof(double2_t), "hipMalloc(twiddles)"))
        return false;
    if (!check(hipMemcpyAsync(m->window.ptr, win.data(), N * sizeof(float), hipMemcpyHostToDevice, s), "hipMemcpy(window)") ||
        !check(hipMemcpyAsync(m->twiddle.ptr, tw.data(), tw.size() * sizeof(double2_t), hipMemcpyHostToDevice, s),
               "hipMemcpy(twiddles)"))
        return false;
    int f0 = 0;
    for (int k = 0; k < d.bands; k++) {
        m->first_freq.push_back(f0);
        f0 += d.band_widths[k];
        m->band_in_total += d.in_dim(k);
        m->proj_total += 2 * d.in_dim(k);
    }
    return check(hipStreamSynchronize(s), "hipStreamSynchronize(model upload)");
}

// bf16 copies of all matrices, rows padded to a multiple of 8 with zeros.
bool prepare_bf16(vh_model *m) {
    if (m->weights_h.ptr) return true;
    const Dims &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int D = d.dim, Hm = d.mask_hidden;
    auto bytes = [](int64_t rows, int cols) { return ((size_t)rows * bf16_pitch(cols) * 2 + 255) & ~(size_t)255; };
    size_t total = 0;
    const size_t per_layer = bytes(d.qkvg_dim(), D) + bytes(D, d.inner()) + bytes(d.ff1_out(), D) + bytes(D, d.ff_dim);
    total += per_layer * m->layers.size();
    for (int b = 0; b < d.bands; b++)
        total += bytes(D, d.in_dim(b)) + bytes(Hm, D) + bytes(2 * d.in_dim(b), Hm);
    if (!m->weights_h.ensure(total, "hipMalloc(bf16 weights)")) return false;
    if (!check(hipMemsetAsync(m->weights_h.ptr, 0, total, s), "hipMemset(bf16 weights)")) return false;
    char *cur = static_cast<char *>(m->weights_h.ptr);
    auto conv = [&](const float *src, int rows, int cols, void **dst) {
        *dst = cur;
        cur += bytes(rows, cols);
        return to_bf16_rows(s, src, rows, cols, *dst, bf16_pitch(cols));
    };
    for (LayerWeights &w : m->layers) {
        if (!conv(w.wqkvg, d.qkvg_dim(), D, &w.wqkvg_h) || !conv(w.wout, D, d.inner(), &w.wout_h) ||
            !conv(w.w1, d.ff1_out(), D, &w.w1_h) || !conv(w.w2, D, d.ff_dim, &w.w2_h))
            return false;
    }
    m->band_w_h.assign(d.bands, nullptr);
    m->mask_w1_h.assign(d.bands, nullptr);
    m->mask_w2_h.assign(d.bands, nullptr);
    for (int b = 0; b < d.bands; b++) {
        const int in = d.in_dim(b);
        if (!conv(m->band_w[b], D, in, &m->band_w_h[b]) || !conv(m->mask_w1[b], Hm, D, &m->mask_w1_h[b]) ||
            !conv(m->mask_w2[b], 2 * in, Hm, &m->mask_w2_h[b]))
            return false;
    }
    return check(hipStreamSynchronize(s), "hipStreamSynchronize(bf16 weights)");
}

// fp16 two-piece planes of the transformer and mask-estimator matrices whose
// K is a multiple of 16 (the fp32 path's linears on the matrix cores), and
// the bounds of their A operands.
static float *mask_feature_bound(vh_model *m) { return m->bounds.f() + 4 * m->layers.size(); }
static float *absmax_scratch(vh_model *m) { return m->bounds.f() + 4 * m->layers.size() + 64; }
// the residual stream's bound slot (XBound) of the layer stack
static float *stream_bound(vh_model *m) { return m->bounds.f() + 4 * m->layers.size() + 8; }

bool prepare_split(vh_model *m) {
    if (m->weights_s.ptr) return true;
    const Dims &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int D = d.dim, Hm = d.mask_hidden;
    auto bytes = [](int N, int K) { return K % SPLIT_K_MULTIPLE ? 0 : (h2_bytes(N, K) + 255) & ~(size_t)255; };
    // per layer: the four matrices, and the QKV one again with its RMSNorm
    // gain folded in (the attention's pre-norm fused into the QKV GEMM)
    // (and that matrix's gate rows in fp32 for the fused band-axis attention)
    const size_t gate_bytes = d.gated ? ((size_t)d.heads * D * sizeof(float) + 255) & ~(size_t)255 : 0;
    const size_t per_layer = 2 * bytes(d.qkvg_dim(), D) + bytes(D, d.inner()) + bytes(d.ff1_out(), D) +
                             bytes(D, d.ff_dim) + gate_bytes;
    size_t total = per_layer * m->layers.size();
    for (int b = 0; b < d.bands; b++) total += bytes(Hm, D) + bytes(2 * d.in_dim(b), Hm);
    m->mask_w1_s.assign(d.bands, nullptr);
    m->mask_w2_s.assign(d.bands, nullptr);
    if (!m->bounds.ensure((4 * m->layers.size() + 64 + ABSMAX_PARTIALS) * sizeof(float), "hipMalloc(operand bounds)"))
        return false;
    if (!operand_bounds(s, m->final_gamma, D, nullptr, 0, nullptr, false, mask_feature_bound(m))) return false;
    const int mask_ok = bounds_usable(s, mask_feature_bound(m), 1);
    if (mask_ok < 0) return false;
    if (total == 0) return true;
    if (!m->weights_s.ensure(total, "hipMalloc(split weights)")) return false;
    char *cur = static_cast<char *>(m->weights_s.ptr);
    auto split = [&](const float *src, int N, int K, void **dst) {
        if (K % SPLIT_K_MULTIPLE) return true;  // the fp32 MFMA GEMM serves this matrix
        *dst = cur;
        cur += bytes(N, K);
        return split_weights_h2(s, src, N, K, K, *dst);
    };
    DeviceBuffer fold_tmp;  // a gain-folded fp32 matrix on its way to its pieces
    auto split_folded = [&](const float *src, int N, const float *gamma, void **dst) {
        if (D % SPLIT_K_MULTIPLE) return true;
        if (!fold_tmp.ensure((size_t)N * D * sizeof(float), "hipMalloc(folded weight)")) return false;
        *dst = cur;
        cur += bytes(N, D);
        return fold_gain_split_h2(s, src, N, D, D, gamma, fold_tmp.f(), *dst);
    };
    for (size_t i = 0; i < m->layers.size(); i++) {
        LayerWeights &w = m->layers[i];
        if (!split(w.wqkvg, d.qkvg_dim(), D, &w.wqkvg_p) || !split(w.wout, D, d.inner(), &w.wout_p) ||
            !split(w.w1, d.ff1_out(), D, &w.w1_p) || !split(w.w2, D, d.ff_dim, &w.w2_p))
            return false;
        w.bounds = m->bounds.f() + 4 * i;
        if (!layer_bounds(s, d, w, w.bounds)) return false;
        float hb[4];
        const int ok = bounds_usable(s, w.bounds, 4, hb);
        if (ok < 0) return false;
        if (ok == 0) w.bounds = nullptr;  // weights beyond the scale range: this layer's linears on fp32 MFMA
        w.att_h2 = w.bounds && h2_attention_bound_ok(hb[1]);
        if (w.bounds && !split_folded(w.wqkvg, d.qkvg_dim(), w.gamma, &w.wqkvg_pg)) return false;
        if (w.wqkvg_pg && gate_bytes) {
            // fold_tmp still holds the gain-folded matrix (stream order)
            w.wgate_g = reinterpret_cast<float *>(cur);
            cur += gate_bytes;
            if (!check(hipMemcpyAsync(w.wgate_g, fold_tmp.f() + (size_t)d.qkv_dim() * D,
                                      (size_t)d.heads * D * sizeof(float), hipMemcpyDeviceToDevice, s),
                       "hipMemcpy(gate rows)"))
                return false;
        }
    }
    for (int b = 0; b < d.bands && mask_ok; b++)  // no pieces: the mask estimator stays on fp32 MFMA
        if (!split(m->mask_w1[b], Hm, D, &m->mask_w1_s[b]) || !split(m->mask_w2[b], 2 * d.in_dim(b), Hm, &m->mask_w2_s[b]))
            return false;
    return check(hipStreamSynchronize(s), "hipStreamSynchronize(split weights)");
}

// Batched token-wise linears of one pipeline stage in the model's precision
// (fp32 activations; the bf16 variant rounds them as they are staged).
bool stage_gemms(vh_model *m, const std::vector<GemmArgs> &gs, const std::vector<void *> &wh, int epi,
                 const char *name) {
    if (m->precision != PREC_BF16) return gemm_batched(m->ctx->stream, gs, epi, &m->ctx->timer, name);
    std::vector<GemmArgsBF16> hs;
    hs.reserve(gs.size());
    for (size_t i = 0; i < gs.size(); i++) {
        const GemmArgs &g = gs[i];
        hs.push_back({g.A, g.lda, wh[i], bf16_pitch(g.K), g.bias, g.C, g.ldc, g.M, g.N, g.K});
    }
    return gemm_bf16_batched(m->ctx->stream, hs, epi, &m->ctx->timer, name);
}

// ---- pipeline stages on `chunks` windows at once --------------------------

int log2i(int n) {
    int l = 0;
    while ((1 << l) < n) l++;
    return l;
}

bool stage_stft(vh_model *m, const float *audio, int64_t audio_len, const int64_t *starts_dev, int sig_len, int chunks,
                int T, float *source, const SpecLayout &lay) {
    const Dims &d = m->d;
    StftArgs a;
    a.audio = audio; a.audio_len = audio_len; a.starts = starts_dev; a.sig_len = sig_len;
    a.C = d.channels; a.T = T; a.F = d.freq_bins(); a.n_fft = d.n_fft; a.log2n = log2i(d.n_fft); a.hop = d.hop;
    a.window = m->window.f(); a.tw = static_cast<const double2_t *>(m->twiddle.ptr); a.source = source; a.out = lay;
    Scope sc(&m->ctx->timer, m->ctx->stream, "stft");
    hipLaunchKernelGGL(stft_kernel, dim3(T, chunks * d.channels), dim3(256), fft_lds_bytes(d.n_fft), m->ctx->stream, a);
    return sync_debug(m->ctx->stream, "stft_kernel");
}

// source bins (layout lay) -> rows of out: band-major (time_sequences, row
// b*M + m) or frame-major (row m*B + b).
bool stage_band_split(vh_model *m, const float *source, const SpecLayout &lay, int chunks, int T, float *out,
                      bool frame_major) {
    const Dims &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int M = chunks * T, B = d.bands, D = d.dim;
    if (!m->bandin.ensure((size_t)M * m->band_in_total * sizeof(float), "hipMalloc(band input)") ||
        !m->tables.ensure(sizeof(BandTable) + sizeof(MaskTable), "hipMalloc(tables)"))
        return false;
    BandTable tab;
    memset(&tab, 0, sizeof(tab));
    int64_t off = 0;
    std::vector<GemmArgs> gs;
    for (int b = 0; b < B; b++) {
        tab.first_freq[b] = m->first_freq[b];
        tab.width[b] = d.band_widths[b];
        tab.in_offset[b] = off;
        tab.gamma[b] = m->band_gamma[b];
        const int in = d.in_dim(b);
        float *C = frame_major ? out + (size_t)b * D : out + (size_t)b * M * D;
        gs.push_back({m->bandin.f() + off, in, m->band_w[b], in, m->band_b[b], C, frame_major ? B * D : D, M, D, in});
        off += (int64_t)M * in;
    }
    if (!check(hipMemcpyAsync(m->tables.ptr, &tab, sizeof(tab), hipMemcpyHostToDevice, s), "hipMemcpy(band table)"))
        return false;
    {
        Scope sc(&m->ctx->timer, s, "band_gather");
        hipLaunchKernelGGL(band_gather_norm_kernel, dim3((M + 3) / 4, B), dim3(256), 0, s, source, lay,
                           (const BandTable *)m->tables.ptr, m->bandin.f(), M, T, d.channels);
        if (!sync_debug(s, "band_gather_norm_kernel")) return false;
    }
    // The table must stay intact until the gather has read it.
    if (!check(hipStreamSynchronize(s), "hipStreamSynchronize(band table)")) return false;
    return stage_gemms(m, gs, m->band_w_h, EPI_STORE, "gemm_band_split");
}

// final-normed features (frame-major rows m*B + b; fp32, or bf16 when
// normed_bf16) -> mask bins (layout lay)
bool stage_mask(vh_model *m, const void *normed, bool normed_bf16, int chunks, int T, float *mask,
                const SpecLayout &lay, bool final_normed) {
    const Dims &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int M = chunks * T, B = d.bands, D = d.dim, Hm = d.mask_hidden;
    const bool h = m->precision == PREC_BF16;
    if (normed_bf16 && !h) {
        set_error("mask estimator: bf16 features need the bf16 variant");
        return false;
    }
    const size_t hid_elem = h ? 2 : 4, feat_elem = normed_bf16 ? 2 : 4;  // the bf16 hidden layer feeds layer 2 as is
    if (!m->mhidden.ensure((size_t)B * M * Hm * hid_elem, "hipMalloc(mask hidden)") ||
        !m->proj.ensure((size_t)M * m->proj_total * sizeof(float), "hipMalloc(mask projection)") ||
        !m->tables.ensure(sizeof(BandTable) + sizeof(MaskTable), "hipMalloc(tables)"))
        return false;
    std::vector<GemmArgs> g1, g2;
    std::vector<GemmArgsBF16> h1, h2;
    std::vector<GemmArgsH2> s1, s2;
    // fp32 path: both layers on the fp16 two-piece GEMM when every band's pieces exist
    bool sp = m->precision == PREC_FP32 && !normed_bf16;
    for (int b = 0; b < B && sp; b++) sp = m->mask_w1_s.size() == (size_t)B && m->mask_w1_s[b] && m->mask_w2_s[b];
    MaskTable tab;
    memset(&tab, 0, sizeof(tab));
    int64_t off = 0;
    for (int b = 0; b < B; b++) {
        char *hid = static_cast<char *>(m->mhidden.ptr) + (size_t)b * M * Hm * hid_elem;
        const char *feat = static_cast<const char *>(normed) + (size_t)b * D * feat_elem;
        const int out = 2 * d.in_dim(b);
        float *proj = m->proj.f() + off;
        if (h) {
            GemmArgsBF16 a{feat, B * D, m->mask_w1_h[b], bf16_pitch(D), m->mask_b1[b], hid, Hm, M, Hm, D};
            a.a_bf16 = normed_bf16;
            a.c_bf16 = true;
            GemmArgsBF16 c{hid, Hm, m->mask_w2_h[b], bf16_pitch(Hm), m->mask_b2[b], proj, out, M, out, Hm};
            c.a_bf16 = true;
            h1.push_back(a);
            h2.push_back(c);
        } else if (sp) {
            s1.push_back({reinterpret_cast<const float *>(feat), B * D, m->mask_w1_s[b], m->mask_b1[b],
                          reinterpret_cast<float *>(hid), Hm, M, Hm, D});
            s2.push_back({reinterpret_cast<const float *>(hid), Hm, m->mask_w2_s[b], m->mask_b2[b], proj, out, M, out,
                          Hm});
        } else {
            g1.push_back({reinterpret_cast<const float *>(feat), B * D, m->mask_w1[b], D, m->mask_b1[b],
                          reinterpret_cast<float *>(hid), Hm, M, Hm, D});
            g2.push_back({reinterpret_cast<const float *>(hid), Hm, m->mask_w2[b], Hm, m->mask_b2[b], proj, out, M, out,
                          Hm});
        }
        tab.first_freq[b] = m->first_freq[b];
        tab.dim[b] = d.in_dim(b);
        tab.proj_offset[b] = off;
        off += (int64_t)M * out;
    }
    KernelTimer *t = &m->ctx->timer;
    if (h) {
        if (!gemm_bf16_batched(s, h1, EPI_TANH, t, "gemm_mask1") || !gemm_bf16_batched(s, h2, EPI_STORE, t, "gemm_mask2"))
            return false;
    } else if (sp) {
        // layer 1's A: the final RMSNorm's bound, or for features from a caller
        // their maximum; layer 2's A: tanh, within [-1, 1]
        OperandBound b1{mask_feature_bound(m), 0.0f};
        if (!final_normed) {
            float *fb = mask_feature_bound(m) + 1;
            if (!absmax(s, static_cast<const float *>(normed), (int64_t)M * B * D, absmax_scratch(m), fb)) return false;
            b1.dev = fb;
        }
        if (!gemm_h2_batched(s, s1, b1, EPI_TANH, t, "gemm_mask1") ||
            !gemm_h2_batched(s, s2, OperandBound{nullptr, 1.0f}, EPI_STORE, t, "gemm_mask2"))
            return false;
    } else if (!gemm_batched(s, g1, EPI_TANH, t, "gemm_mask1") || !gemm_batched(s, g2, EPI_STORE, t, "gemm_mask2")) {
        return false;
    }
    MaskTable *dtab = reinterpret_cast<MaskTable *>(static_cast<char *>(m->tables.ptr) + sizeof(BandTable));
    if (!check(hipMemcpyAsync(dtab, &tab, sizeof(tab), hipMemcpyHostToDevice, s), "hipMemcpy(mask table)")) return false;
    int maxdim = 0;
    for (int b = 0; b < B; b++) maxdim = std::max(maxdim, d.in_dim(b));
    {
        Scope sc(&m->ctx->timer, s, "mask_glu");
        hipLaunchKernelGGL(mask_glu_scatter_kernel, dim3((unsigned)(((int64_t)M * maxdim + 255) / 256), B), dim3(256), 0, s,
                           m->proj.f(), dtab, mask, lay, M, T, d.channels);
        if (!sync_debug(s, "mask_glu_scatter_kernel")) return false;
    }
    return check(hipStreamSynchronize(s), "hipStreamSynchronize(mask table)");
}

// source, mask (layout lay) -> out[chunks*C][pitch] (first `length` samples of each)
bool stage_istft(vh_model *m, const float *source, const float *mask, const SpecLayout &lay, int chunks, int T,
                 int length, float *out, int64_t pitch) {
    const Dims &d = m->d;
    hipStream_t s = m->ctx->stream;
    const int sigs = chunks * d.channels;
    if (!m->frames.ensure((size_t)sigs * T * d.n_fft * sizeof(float), "hipMalloc(istft frames)")) return false;
    IstftArgs a;
    a.source = source; a.mask = mask; a.in = lay; a.C = d.channels; a.T = T; a.F = d.freq_bins(); a.n_fft = d.n_fft;
    a.log2n = log2i(d.n_fft); a.window = m->window.f(); a.tw = static_cast<const double2_t *>(m->twiddle.ptr);
    a.frames = m->frames.f();
    Scope sc(&m->ctx->timer, s, "istft");
    hipLaunchKernelGGL(istft_frames_kernel, dim3(T, sigs), dim3(256), fft_lds_bytes(d.n_fft), s, a);
    if (!sync_debug(s, "istft_frames_kernel")) return false;
    OlaArgs o;
    o.frames = m->frames.f(); o.window = m->window.f(); o.T = T; o.n_fft = d.n_fft; o.hop = d.hop; o.length = length;
    o.out = out; o.out_pitch = pitch;
    hipLaunchKernelGGL(ola_kernel, dim3((length + 255) / 256, sigs), dim3(256), 0, s, o);
    return sync_debug(s, "ola_kernel");
}

bool stage_stack(vh_model *m, float *x, int chunks, int T) {
    const Dims &d = m->d;
    const int64_t tokens = (int64_t)chunks * T * d.bands;
    vh_context *ctx = m->ctx;
    // attention pre-norms fused into the QKV GEMMs: the stream's bound is
    // found once, then carried from block to block by the FFN-down epilogues
    XBound xb;
    xb.dev = stream_bound(m);
    xb.scratch = absmax_scratch(m);
    for (int l = 0; l < d.depth; l++) {
        if (!transformer_block(ctx->stream, d, m->layers[2 * l], x, tokens, time_axis_layout(chunks, T, d.bands),
                               ctx->scratch, ctx->rope, &ctx->timer, m->precision, &xb))
            return false;
        if (!transformer_block(ctx->stream, d, m->layers[2 * l + 1], x, tokens, band_axis_layout(chunks, T, d.bands),
                               ctx->scratch, ctx->rope, &ctx->timer, m->precision, &xb))
            return false;
    }
    return true;
}

// Windows of `sig_len` samples (chunk k starts at starts[k]) -> separated
// windows out[chunks*C][pitch].
bool run_windows(vh_model *m, const float *audio, int64_t audio_len, const int64_t *starts_dev, int sig_len, int chunks,
                 float *out, int64_t pitch) {
    const Dims &d = m->d;
    const int T = d.frames(sig_len);
    const int64_t tokens = (int64_t)chunks * T * d.bands;
    const size_t spec = (size_t)chunks * d.freq_bins() * d.channels * T * 2;
    if (!m->source.ensure(spec * sizeof(float), "hipMalloc(source)") ||
        !m->mask.ensure(spec * sizeof(float), "hipMalloc(mask)") ||
        !m->x.ensure((size_t)tokens * d.dim * sizeof(float), "hipMalloc(features)") ||
        !m->normed.ensure((size_t)tokens * d.dim * sizeof(float), "hipMalloc(normed features)"))
        return false;
    // spectra stay frame-major on the device: each frame's bins contiguous
    const SpecLayout lay = spec_frame_major_layout(d.freq_bins(), d.channels, T);
    if (!stage_stft(m, audio, audio_len, starts_dev, sig_len, chunks, T, m->source.f(), lay)) return false;
    if (!stage_band_split(m, m->source.f(), lay, chunks, T, m->x.f(), true)) return false;
    if (!stage_stack(m, m->x.f(), chunks, T)) return false;
    const bool h = m->precision == PREC_BF16;
    if (h ? !rmsnorm_bf16(m->ctx->stream, m->x.f(), d.dim, m->final_gamma, m->normed.ptr, d.dim, tokens, d.dim,
                          &m->ctx->timer)
          : !rmsnorm(m->ctx->stream, m->x.f(), d.dim, m->final_gamma, m->normed.f(), d.dim, tokens, d.dim,
                     &m->ctx->timer))
        return false;
    if (!stage_mask(m, m->normed.ptr, h, chunks, T, m->mask.f(), lay, true)) return false;
    return stage_istft(m, m->source.f(), m->mask.f(), lay, chunks, T, sig_len, out, pitch);
}

}  // namespace

extern "C" vh_model *vh_model_load(vh_context *ctx, const vh_dims *dims, const void *pack, size_t bytes) {
    if (!ctx || !dims || !pack) return nullptr;
    vh_model *m = new vh_model();
    m->ctx = ctx;
    m->d = dims_from(*dims);
    char why[256];
    if (!m->d.valid(why, sizeof(why))) {
        set_error("model shape: %s", why);
        delete m;
        return nullptr;
    }
    if (!upload_pack(m, pack, bytes) || !prepare_split(m)) {
        delete m;
        return nullptr;
    }
    ctx->models.push_back(m);
    return m;
}

extern "C" int vh_model_set_precision(vh_model *m, int precision) {
    if (!m || (precision != VH_PRECISION_FP32 && precision != VH_PRECISION_BF16 &&
               precision != VH_PRECISION_FP32_MFMA)) {
        set_error("vh_model_set_precision: unknown precision %d", precision);
        return 0;
    }
    if (precision == VH_PRECISION_BF16 && !prepare_bf16(m)) return 0;
    m->precision = precision == VH_PRECISION_BF16 ? PREC_BF16 : precision == VH_PRECISION_FP32_MFMA ? PREC_FP32_MFMA
                                                                                                     : PREC_FP32;
    return 1;
}

extern "C" void vh_model_free(vh_model *m) {
    if (!m) return;
    vh_context *ctx = m->ctx;
    (void)hipStreamSynchronize(ctx->stream);
    auto it = std::find(ctx->models.begin(), ctx->models.end(), m);
    if (it != ctx->models.end()) ctx->models.erase(it);
    delete m;
}

extern "C" int vh_transformer(vh_context *ctx, vh_model *m, int layer, int axis, float *x, int S, int L) {
    if (!ctx || !m || layer < 0 || layer >= m->d.depth || axis < 0 || axis > 1 || S <= 0 || L <= 0) return 0;
    // the attention's pre-norm fused into the QKV GEMM as in the layer stack,
    // the stream's bound found by an absmax pass (float 8 of the context's bounds)
    if (!ctx->bounds.ensure((64 + ABSMAX_PARTIALS) * sizeof(float), "hipMalloc(operand bounds)")) return 0;
    XBound xb;
    xb.dev = ctx->bounds.f() + 8;
    xb.scratch = ctx->bounds.f() + 64;
    return transformer_block(ctx->stream, m->d, m->layers[2 * layer + axis], x, (int64_t)S * L, contiguous_layout(S, L),
                             ctx->scratch, ctx->rope, &ctx->timer, m->precision, &xb)
               ? 1
               : 0;
}

static bool spec_layout_of(int layout, const Dims &d, int T, SpecLayout *out) {
    if (layout == VH_SPEC_REFERENCE) *out = spec_reference_layout(d.freq_bins(), d.channels, T);
    else if (layout == VH_SPEC_FRAME_MAJOR) *out = spec_frame_major_layout(d.freq_bins(), d.channels, T);
    else {
        set_error("unknown spectrum layout %d", layout);
        return false;
    }
    return true;
}

extern "C" int vh_stft(vh_context *ctx, vh_model *m, const float *audio, int length, float *source, int layout) {
    if (!ctx || !m || length <= 0) return 0;
    const int T = m->d.frames(length);
    SpecLayout lay;
    if (!spec_layout_of(layout, m->d, T, &lay)) return 0;
    return stage_stft(m, audio, length, nullptr, length, 1, T, source, lay) ? 1 : 0;
}

extern "C" int vh_istft(vh_context *ctx, vh_model *m, const float *source, const float *mask, int length, float *audio,
                        int layout) {
    if (!ctx || !m || length <= 0) return 0;
    const int T = m->d.frames(length);
    SpecLayout lay;
    if (!spec_layout_of(layout, m->d, T, &lay)) return 0;
    return stage_istft(m, source, mask, lay, 1, T, length, audio, length) ? 1 : 0;
}

extern "C" int vh_band_split(vh_context *ctx, vh_model *m, const float *source, int frames, float *time_sequences,
                             int layout) {
    if (!ctx || !m || frames <= 0) return 0;
    SpecLayout lay;
    if (!spec_layout_of(layout, m->d, frames, &lay)) return 0;
    return stage_band_split(m, source, lay, 1, frames, time_sequences, false) ? 1 : 0;
}

extern "C" int vh_mask_estimate(vh_context *ctx, vh_model *m, const float *features, int frames, float *mask,
                                int layout) {
    if (!ctx || !m || frames <= 0) return 0;
    SpecLayout lay;
    if (!spec_layout_of(layout, m->d, frames, &lay)) return 0;
    return stage_mask(m, features, false, 1, frames, mask, lay, false) ? 1 : 0;
}

extern "C" int vh_forward(vh_context *ctx, vh_model *m, const float *audio, int length, float *vocals,
                          float *instrumental) {
    if (!ctx || !m || length <= 0) return 0;
    if (!run_windows(m, audio, length, nullptr, length, 1, vocals, length)) return 0;
    if (instrumental) {
        const int64_t n = (int64_t)m->d.channels * length;
        hipLaunchKernelGGL(subtract_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream, audio, vocals,
                           instrumental, n);
        if (!sync_debug(ctx->stream, "subtract_kernel")) return 0;
    }
    return 1;
}

extern "C" int vh_separate(vh_context *ctx, vh_model *m, const float *audio, int length, int chunk, int step, int batch,
                           float *vocals, float *instrumental) {
    if (!ctx || !m || length <= 0 || chunk <= 0 || step <= 0 || step > chunk || batch <= 0) {
        set_error("vh_separate: bad arguments");
        return 0;
    }
    const Dims &d = m->d;
    const int count = length <= chunk ? 1 : 1 + (length - chunk + step - 1) / step;
    hipStream_t s = ctx->stream;
    std::vector<int64_t> starts(count);
    for (int k = 0; k < count; k++) starts[k] = (int64_t)k * step;
    if (!m->starts.ensure(count * sizeof(int64_t), "hipMalloc(chunk starts)") ||
        !m->chunk_out.ensure((size_t)count * d.channels * chunk * sizeof(float), "hipMalloc(chunk outputs)"))
        return 0;
    if (!check(hipMemcpyAsync(m->starts.ptr, starts.data(), count * sizeof(int64_t), hipMemcpyHostToDevice, s),
               "hipMemcpy(chunk starts)") ||
        !check(hipStreamSynchronize(s), "hipStreamSynchronize(starts)"))
        return 0;
    for (int k0 = 0; k0 < count; k0 += batch) {
        const int n = std::min(batch, count - k0);
        if (!run_windows(m, audio, length, static_cast<const int64_t *>(m->starts.ptr) + k0, chunk, n,
                         m->chunk_out.f() + (size_t)k0 * d.channels * chunk, chunk))
            return 0;
    }
    FadeArgs a;
    a.chunks = m->chunk_out.f(); a.count = count; a.chunk = chunk; a.step = step; a.C = d.channels; a.length = length;
    a.out = vocals;
    a.mix = audio;
    a.instrumental = instrumental;
    Scope sc(&ctx->timer, s, "crossfade");
    hipLaunchKernelGGL(crossfade_kernel, dim3((unsigned)((length + 255) / 256), d.channels), dim3(256), 0, s, a);
    return sync_debug(s, "crossfade_kernel") ? 1 : 0;
}

// ---------------------------------------------------------------- timing
extern "C" int vh_timing_enable(vh_context *ctx, const char *classes) {
    if (!ctx) return 0;
    KernelTimer &t = ctx->timer;
    t.only.clear();
    t.all = classes && strcmp(classes, "*") == 0;
    t.enabled = classes && classes[0];
    if (t.enabled && !t.all) {
        const char *p = classes;
        while (*p) {
            const char *e = strchr(p, ',');
            const size_t n = e ? (size_t)(e - p) : strlen(p);
            if (n) t.only.emplace_back(p, n);
            p += n + (e ? 1 : 0);
        }
    }
    return 1;
}

extern "C" int vh_timing_reset(vh_context *ctx) {
    if (!ctx) return 0;
    (void)hipStreamSynchronize(ctx->stream);
    ctx->timer.reset();
    return 1;
}

extern "C" int vh_timing_get(vh_context *ctx, const char *name, double *total_ms, int64_t *count) {
    if (!ctx || !name) return 0;
    ctx->timer.collect();
    auto it = ctx->timer.totals.find(name);
    if (it == ctx->timer.totals.end()) return 0;
    if (total_ms) *total_ms = it->second.first;
    if (count) *count = it->second.second;
    return 1;
}
