// native_gpu_hip.cpp -- MI355X (gfx950) provider for the VocalArc host's GPU
// C-ABI (native_gpu.h).  Drop-in replacement of native/native_gpu_cuda.cu:
// same 12 entry points, same return/fallback contract, no vendor BLAS.
//
// Design:
//  * Weights are uploaded on first use from the host's packed layout
//    (native/vocalarc_separation.c:428-457) and unpacked on the device into
//    [out][in] rows.  The QKV and gate projections are fused into one matrix
//    (gates in 8 extra rows, padded to a 32-row tile) so one GEMM produces both.
//    Cache entries are keyed by host pointer and shape and carry a sampled
//    content fingerprint, so a pack reloaded at the same address is noticed.
//  * The resident tensor is kept in ONE physical layout.  A transpose
//    (native/native_gpu_cuda.cu:714-726 moves the whole tensor) only flips
//    which axis is the sequence axis; the attention kernel reads either axis
//    with strides.  A physical transpose happens only if the host reinterprets
//    the tensor with a different factorisation, or at resident_end.
//  * Errors print once and disable the provider (native/native_gpu_cuda.cu:88-102
//    behaviour): every later call returns 0 and the host recomputes on the CPU.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <vector>

#include "../../include/native_gpu.h"
#include "elementwise.hpp"
#include "runtime.hpp"

using namespace vh;

namespace {

// The host's compile-time shape (native/vocalarc_separation.c:33-57).
Dims host_dims() {
    Dims d;
    memset(&d, 0, sizeof(d));
    d.dim = 256; d.depth = 16; d.heads = 8; d.dim_head = 64; d.ff_dim = 1024; d.ffn_glu = 0; d.gated = 1;
    d.mask_hidden = 1024; d.n_fft = 2048; d.hop = 512; d.channels = 2;
    static const int widths[] = {2, 4, 12, 24, 48, 128, 129};
    static const int counts[] = {24, 36, 16, 8, 4, 1, 1};
    int b = 0;
    for (int i = 0; i < 7; i++)
        for (int k = 0; k < counts[i]; k++) d.band_widths[b++] = widths[i];
    d.bands = b;
    return d;
}

uint64_t fingerprint(const float *p, size_t n) {
    // FNV-1a over up to 64 evenly spaced samples plus the last element.
    uint64_t h = 1469598103934665603ull;
    auto mix = [&](uint32_t v) {
        for (int i = 0; i < 4; i++) {
            h ^= (v >> (8 * i)) & 0xffu;
            h *= 1099511628211ull;
        }
    };
    if (n == 0) return h;
    const size_t step = n > 64 ? n / 64 : 1;
    for (size_t i = 0; i < n; i += step) {
        uint32_t v;
        memcpy(&v, p + i, 4);
        mix(v);
    }
    uint32_t last;
    memcpy(&last, p + n - 1, 4);
    mix(last);
    return h;
}

struct CacheEntry {
    const void *key;   // host pointer (first tensor of a fused entry)
    const void *key2;  // second host tensor of a fused entry, or null
    int in, out, mode;
    uint64_t fp;
    float *dev;
    float *dev_bias;   // fused QKV+gate bias
    void *dev_split = nullptr;  // fp16 two-piece planes of dev (made on first use)
};

}  // namespace

struct native_gpu {
    int enabled = 0;
    char device_name[256] = "none";
    hipStream_t stream = nullptr;
    Dims d;
    std::vector<CacheEntry> cache;
    DeviceBuffer staging;
    BlockScratch scratch;
    RopeCache rope;
    // resident state
    DeviceBuffer x, x_alt;
    int active = 0;
    int64_t tokens = 0;
    int ls = 0, ll = 0;        // logical [ls][ll]
    bool transposed = false;   // physical [ll][ls]
    // mask + matmul scratch
    DeviceBuffer normed, hidden, proj, mask, io_in, io_out, tables;
    // A-operand bounds of the fp16 two-piece GEMMs outside the layers: [4..5]
    // the mask features, [6] a matmul input, then absmax scratch
    DeviceBuffer bounds;
    float *bound(int i) { return bounds.f() + i; }
    bool ensure_bounds() {
        return bounds.ensure((64 + ABSMAX_PARTIALS) * sizeof(float), "hipMalloc(operand bounds)");
    }
    // Layer bounds per set of cached device tensors they derive from (gains,
    // fused projection and its bias, FFN up matrix and its bias): computed
    // once, dropped whenever a cached tensor is replaced.
    struct LayerBounds {
        const void *keys[6];
        float *dev;
        bool att_h2;  // the fused projection's bound in the two-piece attention's range
    };
    std::vector<LayerBounds> layer_bounds_cache;
    void drop_layer_bounds() {
        for (auto &b : layer_bounds_cache)
            if (b.dev) (void)hipFree(b.dev);
        layer_bounds_cache.clear();
    }
    float *bounds_of(const LayerWeights &L, bool *ok, bool *att_h2) {
        const void *keys[6] = {L.gamma, L.wqkvg, L.bqkvg, L.ff_gamma, L.w1, L.b1};
        for (auto &b : layer_bounds_cache)
            if (memcmp(b.keys, keys, sizeof(keys)) == 0) {
                *att_h2 = b.att_h2;
                return b.dev;
            }
        float *dev = nullptr;
        *ok = false;
        *att_h2 = false;
        if (!check(hipMalloc((void **)&dev, 4 * sizeof(float)), "hipMalloc(layer bounds)")) return nullptr;
        if (!layer_bounds(stream, d, L, dev)) {
            (void)hipFree(dev);
            return nullptr;
        }
        float hb[4];
        const int usable = bounds_usable(stream, dev, 4, hb);
        if (usable <= 0) {  // beyond the scale range: the layer's linears run on fp32 MFMA
            (void)hipFree(dev);
            if (usable < 0) return nullptr;
            dev = nullptr;
        }
        *ok = true;
        LayerBounds e;
        memcpy(e.keys, keys, sizeof(keys));
        e.dev = dev;  // null: recorded as unusable, so the check is not repeated
        e.att_h2 = dev && h2_attention_bound_ok(hb[1]);
        *att_h2 = e.att_h2;
        layer_bounds_cache.push_back(e);
        return dev;
    }

    // Report, disable for the rest of the process, and tell the host to
    // compute this step itself.
    int fail(const char *what) {
        fprintf(stderr, "native HIP %s failed: %s; falling back to CPU\n", what, last_error());
        enabled = 0;
        return 0;
    }

    // ---- weight cache -----------------------------------------------------
    CacheEntry *find(const void *k, const void *k2, int in, int out, int mode, uint64_t fp) {
        for (auto &e : cache)
            if (e.key == k && e.key2 == k2 && e.in == in && e.out == out && e.mode == mode) {
                if (e.fp == fp) return &e;
                // same address, different contents: a reloaded pack
                drop_layer_bounds();
                (void)hipFree(e.dev);
                if (e.dev_bias) (void)hipFree(e.dev_bias);
                if (e.dev_split) (void)hipFree(e.dev_split);
                e = cache.back();
                cache.pop_back();
                return nullptr;
            }
        return nullptr;
    }

    const float *matrix(const float *host, int in, int out, int mode = 0) {
        const uint64_t fp = fingerprint(host, (size_t)in * out);
        if (CacheEntry *e = find(host, nullptr, in, out, mode, fp)) return e->dev;
        float *dev = nullptr;
        if (!check(hipMalloc((void **)&dev, (size_t)in * out * sizeof(float)), "hipMalloc(weight)")) return nullptr;
        if (!upload_weight(stream, host, in, out, dev, in, 0, mode, staging)) {
            (void)hipFree(dev);
            return nullptr;
        }
        cache.push_back({host, nullptr, in, out, mode, fp, dev, nullptr});
        return dev;
    }

    // fp16 two-piece planes (gemm_h2) of a cached device matrix [out][in];
    // null when `in` is not a multiple of 16 (the fp32 MFMA GEMM serves it).
    // VOCALARC_GPU_SPLIT=0 keeps every product on the fp32 MFMA instruction.
    static bool split_off() {
        static const bool off = [] {
            const char *v = getenv("VOCALARC_GPU_SPLIT");
            return v && strcmp(v, "0") == 0;
        }();
        return off;
    }
    const void *split(const float *dev, int in, int out) {
        if (split_off() || !dev || in % SPLIT_K_MULTIPLE) return nullptr;
        for (auto &e : cache) {
            if (e.dev != dev) continue;
            if (e.dev_split) return e.dev_split;
            void *p = nullptr;
            if (!check(hipMalloc(&p, h2_bytes(out, in)), "hipMalloc(split weight)")) return nullptr;
            if (!split_weights_h2(stream, dev, out, in, in, p)) {
                (void)hipFree(p);
                return nullptr;
            }
            e.dev_split = p;
            return p;
        }
        return nullptr;
    }

    const float *vector(const float *host, int n) {
        const uint64_t fp = fingerprint(host, (size_t)n);
        if (CacheEntry *e = find(host, nullptr, 0, n, 9, fp)) return e->dev;
        float *dev = nullptr;
        if (!check(hipMalloc((void **)&dev, (size_t)n * sizeof(float)), "hipMalloc(vector)")) return nullptr;
        if (!upload_vector(stream, host, n, dev)) {
            (void)hipFree(dev);
            return nullptr;
        }
        cache.push_back({host, nullptr, 0, n, 9, fp, dev, nullptr});
        return dev;
    }

    // Fused [qkv | gates | 0] matrix and its bias [0 | gate bias | 0].
    bool qkvg(const native_gpu_transformer_weights *w, const float **W, const float **B) {
        const int D = d.dim, inner = d.inner(), nq = d.qkvg_dim();
        const uint64_t fp = fingerprint(w->qkv, (size_t)3 * inner * D) ^ (fingerprint(w->gate_weight, (size_t)d.heads * D) * 3) ^
                            (fingerprint(w->gate_bias, d.heads) * 7);
        if (CacheEntry *e = find(w->qkv, w->gate_weight, D, nq, 10, fp)) {
            *W = e->dev;
            *B = e->dev_bias;
            return true;
        }
        float *dw = nullptr, *db = nullptr;
        if (!check(hipMalloc((void **)&dw, (size_t)nq * D * sizeof(float)), "hipMalloc(qkv weight)")) return false;
        if (!check(hipMalloc((void **)&db, (size_t)nq * sizeof(float)), "hipMalloc(qkv bias)")) {
            (void)hipFree(dw);
            return false;
        }
        bool ok = check(hipMemsetAsync(dw, 0, (size_t)nq * D * sizeof(float), stream), "hipMemset(qkv weight)") &&
                  check(hipMemsetAsync(db, 0, (size_t)nq * sizeof(float), stream), "hipMemset(qkv bias)") &&
                  upload_weight(stream, w->qkv, D, 3 * inner, dw, D, 0, 0, staging) &&
                  upload_weight(stream, w->gate_weight, D, d.heads, dw, D, 3 * inner, 0, staging) &&
                  upload_vector(stream, w->gate_bias, d.heads, db + 3 * inner);
        if (!ok) {
            (void)hipFree(dw);
            (void)hipFree(db);
            return false;
        }
        cache.push_back({w->qkv, w->gate_weight, D, nq, 10, fp, dw, db});
        *W = dw;
        *B = db;
        return true;
    }

    bool layer(const native_gpu_transformer_weights *w, LayerWeights &L) {
        const int D = d.dim;
        const float *W = nullptr, *B = nullptr;
        if (!qkvg(w, &W, &B)) return false;
        L.wqkvg = const_cast<float *>(W);
        L.bqkvg = const_cast<float *>(B);
        L.gamma = const_cast<float *>(vector(w->gamma, D));
        L.ff_gamma = const_cast<float *>(vector(w->ff_gamma, D));
        L.wout = const_cast<float *>(matrix(w->out_weight, d.inner(), D));
        L.w1 = const_cast<float *>(matrix(w->ff1_weight, D, d.ff_dim));
        L.b1 = const_cast<float *>(vector(w->ff1_bias, d.ff_dim));
        L.w2 = const_cast<float *>(matrix(w->ff2_weight, d.ff_dim, D));
        L.b2 = const_cast<float *>(vector(w->ff2_bias, D));
        if (!(L.gamma && L.ff_gamma && L.wout && L.w1 && L.b1 && L.w2 && L.b2)) return false;
        L.wqkvg_p = const_cast<void *>(split(L.wqkvg, D, d.qkvg_dim()));
        L.wout_p = const_cast<void *>(split(L.wout, d.inner(), D));
        L.w1_p = const_cast<void *>(split(L.w1, D, d.ff1_out()));
        L.w2_p = const_cast<void *>(split(L.w2, d.ff_dim, D));
        // the bounds of this layer's gains and matrices (computed on the
        // first call that uses them; none when they are beyond the fp16
        // two-piece scale range, and the fp32 MFMA GEMM runs)
        bool ok = true;
        L.bounds = bounds_of(L, &ok, &L.att_h2);
        return ok;
    }

    // ---- resident layout ----------------------------------------------------
    AttnLayout layout() const {
        if (transposed) return {ls, ll, ls, 0, 1, ls};  // physical [ll][ls]
        return {ls, ll, 1, ll, 0, 1};                   // physical [ls][ll]
    }

    bool materialize() {
        if (!transposed) return true;
        if (!x_alt.ensure(x.bytes, "hipMalloc(resident alt)")) return false;
        // physical [ll][ls] -> [ls][ll]
        if (!transpose_rows(stream, x.f(), x_alt.f(), 1, ll, ls, d.dim)) return false;
        std::swap(x.ptr, x_alt.ptr);
        std::swap(x.bytes, x_alt.bytes);
        transposed = false;
        return true;
    }

    bool view_as(int S, int L) {
        if (S == ls && L == ll) return true;
        if (!materialize()) return false;
        ls = S;
        ll = L;
        return true;
    }
};

// ------------------------------------------------------------------- ABI

extern "C" native_gpu *native_gpu_create(void) {
    const char *mode = getenv("VOCALARC_GPU");
    if (mode && (strcmp(mode, "off") == 0 || strcmp(mode, "cpu") == 0)) return nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return nullptr;
    native_gpu *gpu = new native_gpu();
    gpu->d = host_dims();
    if (!check(hipSetDevice(0), "hipSetDevice") || !check(hipStreamCreate(&gpu->stream), "hipStreamCreate")) {
        fprintf(stderr, "native HIP initialisation failed: %s\n", last_error());
        delete gpu;
        return nullptr;
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) == hipSuccess) {
        // the marketing name can be empty where the driver's name table is
        // missing: the architecture then names the device alone
        if (prop.name[0]) snprintf(gpu->device_name, sizeof(gpu->device_name), "%s (%s)", prop.name, prop.gcnArchName);
        else snprintf(gpu->device_name, sizeof(gpu->device_name), "HIP device %s", prop.gcnArchName);
        // printed raw inside JSON by the host: keep it free of quotes/backslashes
        for (char *c = gpu->device_name; *c; c++)
            if (*c == '"' || *c == '\\' || (unsigned char)*c < 0x20) *c = ' ';
    } else {
        snprintf(gpu->device_name, sizeof(gpu->device_name), "HIP device 0");
    }
    gpu->enabled = 1;
    return gpu;
}

extern "C" void native_gpu_destroy(native_gpu *gpu) {
    if (!gpu) return;
    if (gpu->stream) (void)hipStreamSynchronize(gpu->stream);
    for (auto &e : gpu->cache) {
        (void)hipFree(e.dev);
        if (e.dev_bias) (void)hipFree(e.dev_bias);
        if (e.dev_split) (void)hipFree(e.dev_split);
    }
    gpu->cache.clear();
    gpu->drop_layer_bounds();
    hipStream_t s = gpu->stream;
    delete gpu;  // buffers release themselves
    if (s) (void)hipStreamDestroy(s);
}

extern "C" const char *native_gpu_backend(const native_gpu *gpu) {
    return gpu && gpu->enabled ? "native-hip-fused" : "native-cpu";
}

extern "C" const char *native_gpu_device(const native_gpu *gpu) {
    return gpu && gpu->enabled ? gpu->device_name : "none";
}

extern "C" int native_gpu_uses_full_batches(const native_gpu *gpu) { return gpu && gpu->enabled ? 1 : 0; }

extern "C" int native_gpu_can_use_full_batches(const native_gpu *gpu, int frames) {
    if (!gpu || !gpu->enabled || frames <= 0) return 0;
    const char *o = getenv("VOCALARC_GPU_FULL_BATCHES");
    if (o && (strcmp(o, "0") == 0 || strcmp(o, "false") == 0 || strcmp(o, "off") == 0)) return 0;
    const Dims &d = gpu->d;
    const double tokens = (double)d.bands * frames;
    // device working set of the resident path
    double dev = tokens * (3.0 * d.dim + d.qkvg_dim() + d.inner() + d.ff_dim) * 4.0;
    dev += tokens * (double)d.mask_hidden * 4.0 + (double)frames * d.freq_bins() * d.channels * 6.0 * 4.0;
    dev += 512.0 * 1024 * 1024;  // weights (267 MB) + allocator reserve
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) != hipSuccess || free_b == 0) return 0;
    if (dev >= (double)free_b * 0.6) return 0;
    // With full batches the host sizes its CPU scratch for
    // max(bands, frames)^2 tokens (native/vocalarc_separation.c:1262-1272,
    // 1576-1582).  Decline when that would not fit in host memory, so long
    // inputs stay on bounded groups (and still reach native_gpu_transformer).
    const double side = (double)std::max(d.bands, frames);
    const double host = side * side * (d.dim + d.qkv_dim() + d.inner() + d.heads) * 4.0;
    const long pages = sysconf(_SC_PHYS_PAGES), page = sysconf(_SC_PAGE_SIZE);
    if (pages > 0 && page > 0 && host > 0.5 * (double)pages * (double)page) return 0;
    return 1;
}

extern "C" int native_gpu_matmul(native_gpu *gpu, int64_t rows, int in, int out, const float *input,
                                 const float *packed_weight, const float *bias, float *output) {
    if (!gpu || !gpu->enabled || rows <= 0 || in <= 0 || out <= 0 || !input || !packed_weight || !output) return 0;
    // Offload only when the work amortises the two PCIe transfers
    // (the dlopen provider uses the same knob, native/native_gpu.c:234-239).
    double min_work = 67108864.0;
    if (const char *v = getenv("VOCALARC_GPU_MIN_WORK")) min_work = atof(v);
    if ((double)rows * in * out < min_work) return 0;
    if (in % 4) return 0;
    const float *W = gpu->matrix(packed_weight, in, out);
    const float *B = bias ? gpu->vector(bias, out) : nullptr;
    if (!W || (bias && !B)) return gpu->fail("weight upload");
    const void *Ws = gpu->split(W, in, out);
    const size_t ib = (size_t)rows * in * sizeof(float), ob = (size_t)rows * out * sizeof(float);
    hipStream_t s = gpu->stream;
    auto product = [&]() {
        if (Ws) {  // the input's own maximum bounds it (beyond the scale range: fp32 MFMA)
            if (!gpu->ensure_bounds() || !absmax(s, gpu->io_in.f(), rows * in, gpu->bound(64), gpu->bound(6)))
                return false;
            const int usable = bounds_usable(s, gpu->bound(6), 1);
            if (usable < 0) return false;
            if (usable)
                return gemm_h2(s, {gpu->io_in.f(), in, Ws, B, gpu->io_out.f(), out, rows, out, in},
                               OperandBound{gpu->bound(6), 0.0f}, EPI_STORE);
        }
        return gemm(s, {gpu->io_in.f(), in, W, in, B, gpu->io_out.f(), out, rows, out, in}, EPI_STORE);
    };
    bool ok = gpu->io_in.ensure(ib, "hipMalloc(matmul input)") && gpu->io_out.ensure(ob, "hipMalloc(matmul output)") &&
              check(hipMemcpyAsync(gpu->io_in.ptr, input, ib, hipMemcpyHostToDevice, s), "hipMemcpy(matmul input)") &&
              product() &&
              check(hipMemcpyAsync(output, gpu->io_out.ptr, ob, hipMemcpyDeviceToHost, s), "hipMemcpy(matmul output)") &&
              check(hipStreamSynchronize(s), "hipStreamSynchronize(matmul)");
    if (!ok) return gpu->fail("matmul");
    return 1;
}

static int run_block(native_gpu *gpu, float *x, int64_t tokens, const AttnLayout &lay,
                     const native_gpu_transformer_weights *w) {
    LayerWeights L;
    if (!gpu->layer(w, L)) return gpu->fail("weight upload");
    // VOCALARC_GPU_SPLIT=0: every product (the attention's too) on the fp32 MFMA instruction
    if (!transformer_block(gpu->stream, gpu->d, L, x, tokens, lay, gpu->scratch, gpu->rope, nullptr,
                           native_gpu::split_off() ? PREC_FP32_MFMA : PREC_FP32))
        return gpu->fail("transformer");
    return 1;
}

extern "C" int native_gpu_transformer(native_gpu *gpu, int sequences, int length, float *data, float *normed,
                                      float *qkv, float *attention_output, float *gates,
                                      const native_gpu_transformer_weights *weights) {
    (void)normed; (void)qkv; (void)attention_output; (void)gates;
    if (!gpu || !gpu->enabled || sequences <= 0 || length <= 0 || !data || !weights) return 0;
    const int64_t tokens = (int64_t)sequences * length;
    const size_t bytes = (size_t)tokens * gpu->d.dim * sizeof(float);
    hipStream_t s = gpu->stream;
    if (!gpu->io_in.ensure(bytes, "hipMalloc(transformer data)") ||
        !check(hipMemcpyAsync(gpu->io_in.ptr, data, bytes, hipMemcpyHostToDevice, s), "hipMemcpy(transformer data)"))
        return gpu->fail("transformer upload");
    if (!run_block(gpu, gpu->io_in.f(), tokens, {sequences, length, 1, length, 0, 1}, weights)) return 0;
    if (!check(hipMemcpyAsync(data, gpu->io_in.ptr, bytes, hipMemcpyDeviceToHost, s), "hipMemcpy(transformer)") ||
        !check(hipStreamSynchronize(s), "hipStreamSynchronize(transformer)"))
        return gpu->fail("transformer download");
    return 1;
}

extern "C" int native_gpu_resident_begin(native_gpu *gpu, int sequences, int length, const float *data) {
    if (!gpu || !gpu->enabled || sequences <= 0 || length <= 0 || !data) return 0;
    // A residency left open by an aborted host loop is discarded here; the
    // reference provider would refuse every later begin instead.
    gpu->active = 0;
    const int64_t tokens = (int64_t)sequences * length;
    const size_t bytes = (size_t)tokens * gpu->d.dim * sizeof(float);
    if (!gpu->x.ensure(bytes, "hipMalloc(resident)") ||
        !check(hipMemcpyAsync(gpu->x.ptr, data, bytes, hipMemcpyHostToDevice, gpu->stream), "hipMemcpy(resident begin)") ||
        !check(hipStreamSynchronize(gpu->stream), "hipStreamSynchronize(resident begin)"))
        return gpu->fail("resident begin");
    gpu->tokens = tokens;
    gpu->ls = sequences;
    gpu->ll = length;
    gpu->transposed = false;
    gpu->active = 1;
    return 1;
}

extern "C" int native_gpu_resident_transformer(native_gpu *gpu, int sequences, int length,
                                               const native_gpu_transformer_weights *weights) {
    if (!gpu || !gpu->enabled || !gpu->active || !weights || (int64_t)sequences * length != gpu->tokens) return 0;
    if (!gpu->view_as(sequences, length)) return gpu->fail("resident layout");
    return run_block(gpu, gpu->x.f(), gpu->tokens, gpu->layout(), weights);
}

extern "C" int native_gpu_resident_transpose(native_gpu *gpu, int sequences, int length) {
    if (!gpu || !gpu->enabled || !gpu->active || (int64_t)sequences * length != gpu->tokens) return 0;
    if (!gpu->view_as(sequences, length)) return gpu->fail("resident layout");
    // logical [S][L] -> [L][S]: flip the view, move no data
    std::swap(gpu->ls, gpu->ll);
    gpu->transposed = !gpu->transposed;
    return 1;
}

extern "C" int native_gpu_resident_end(native_gpu *gpu, float *data) {
    if (!gpu || !gpu->enabled || !gpu->active || !data) return 0;
    gpu->active = 0;
    const size_t bytes = (size_t)gpu->tokens * gpu->d.dim * sizeof(float);
    if (!gpu->materialize() ||
        !check(hipMemcpyAsync(data, gpu->x.ptr, bytes, hipMemcpyDeviceToHost, gpu->stream), "hipMemcpy(resident end)") ||
        !check(hipStreamSynchronize(gpu->stream), "hipStreamSynchronize(resident end)"))
        return gpu->fail("resident end");
    return 1;
}

extern "C" int native_gpu_resident_mask(native_gpu *gpu, int frames, const float *final_gamma, float *mask,
                                        const native_gpu_mask_band *bands, int band_count) {
    if (!gpu || !gpu->enabled || !gpu->active || frames <= 0 || !final_gamma || !mask || !bands || band_count <= 0 ||
        band_count > VH_MAX_BANDS || (int64_t)frames * band_count != gpu->tokens)
        return 0;
    Dims &d = gpu->d;
    // The band table comes from the call; check it tiles the spectrum.
    int f0 = 0;
    for (int b = 0; b < band_count; b++) {
        const int in = bands[b].input_dim;
        if (in <= 0 || in % (2 * d.channels) || bands[b].first_frequency != f0 || !bands[b].first_weight ||
            !bands[b].first_bias || !bands[b].second_weight || !bands[b].second_bias)
            return 0;
        f0 += in / (2 * d.channels);
    }
    if (f0 != d.freq_bins()) return 0;
    if (!gpu->view_as(frames, band_count) || !gpu->materialize()) return gpu->fail("resident layout");
    hipStream_t s = gpu->stream;
    const int B = band_count, D = d.dim, Hm = d.mask_hidden, M = frames;
    int64_t proj_total = 0;
    for (int b = 0; b < B; b++) proj_total += 2 * bands[b].input_dim;
    const size_t mask_floats = (size_t)d.freq_bins() * d.channels * frames * 2;
    const float *gamma = gpu->vector(final_gamma, D);
    if (!gamma) return gpu->fail("weight upload");
    bool ok = gpu->normed.ensure((size_t)gpu->tokens * D * sizeof(float), "hipMalloc(mask features)") &&
              gpu->hidden.ensure((size_t)B * M * Hm * sizeof(float), "hipMalloc(mask hidden)") &&
              gpu->proj.ensure((size_t)M * proj_total * sizeof(float), "hipMalloc(mask projection)") &&
              gpu->mask.ensure(mask_floats * sizeof(float), "hipMalloc(mask)") &&
              gpu->tables.ensure(sizeof(MaskTable), "hipMalloc(mask table)");
    if (!ok) return gpu->fail("mask buffers");
    std::vector<GemmArgs> g1, g2;
    std::vector<GemmArgsH2> s1, s2;  // the same products on the fp16 two-piece GEMM
    // layer 1's A is the final RMSNorm's output: its bound from the gain
    // (beyond the fp16 two-piece scale range: fp32 MFMA instead)
    bool sp = gpu->ensure_bounds() && operand_bounds(s, gamma, D, nullptr, 0, nullptr, false, gpu->bound(4));
    if (!sp) return gpu->fail("mask bounds");
    const int usable = bounds_usable(s, gpu->bound(4), 1);
    if (usable < 0) return gpu->fail("mask bounds");
    sp = usable == 1;
    MaskTable tab;
    memset(&tab, 0, sizeof(tab));
    int64_t off = 0;
    int maxdim = 0;
    for (int b = 0; b < B; b++) {
        const int dim = bands[b].input_dim;
        const float *w1 = gpu->matrix(bands[b].first_weight, D, Hm);
        const float *b1 = gpu->vector(bands[b].first_bias, Hm);
        const float *w2 = gpu->matrix(bands[b].second_weight, Hm, 2 * dim);
        const float *b2 = gpu->vector(bands[b].second_bias, 2 * dim);
        if (!w1 || !b1 || !w2 || !b2) return gpu->fail("mask weight upload");
        float *hid = gpu->hidden.f() + (size_t)b * M * Hm;
        g1.push_back({gpu->normed.f() + (size_t)b * D, B * D, w1, D, b1, hid, Hm, M, Hm, D});
        g2.push_back({hid, Hm, w2, Hm, b2, gpu->proj.f() + off, 2 * dim, M, 2 * dim, Hm});
        const void *w1s = sp ? gpu->split(w1, D, Hm) : nullptr;
        const void *w2s = sp ? gpu->split(w2, Hm, 2 * dim) : nullptr;
        sp = sp && w1s && w2s;
        s1.push_back({gpu->normed.f() + (size_t)b * D, B * D, w1s, b1, hid, Hm, M, Hm, D});
        s2.push_back({hid, Hm, w2s, b2, gpu->proj.f() + off, 2 * dim, M, 2 * dim, Hm});
        tab.first_freq[b] = bands[b].first_frequency;
        tab.dim[b] = dim;
        tab.proj_offset[b] = off;
        off += (int64_t)M * 2 * dim;
        maxdim = std::max(maxdim, dim);
    }
    // layer 1's A bounded by bound(4); layer 2's A: tanh, within [-1, 1]
    ok = rmsnorm(s, gpu->x.f(), D, gamma, gpu->normed.f(), D, gpu->tokens, D) &&
         (sp ? gemm_h2_batched(s, s1, OperandBound{gpu->bound(4), 0.0f}, EPI_TANH) &&
                   gemm_h2_batched(s, s2, OperandBound{nullptr, 1.0f}, EPI_STORE)
             : gemm_batched(s, g1, EPI_TANH) && gemm_batched(s, g2, EPI_STORE)) &&
         check(hipMemcpyAsync(gpu->tables.ptr, &tab, sizeof(tab), hipMemcpyHostToDevice, s), "hipMemcpy(mask table)");
    if (ok) {
        hipLaunchKernelGGL(mask_glu_scatter_kernel, dim3((unsigned)(((int64_t)M * maxdim + 255) / 256), B), dim3(256), 0,
                           s, gpu->proj.f(), (const MaskTable *)gpu->tables.ptr, gpu->mask.f(),
                           spec_reference_layout(d.freq_bins(), d.channels, frames), M, frames, d.channels);
        ok = sync_debug(s, "mask_glu_scatter_kernel") &&
             check(hipMemcpyAsync(mask, gpu->mask.ptr, mask_floats * sizeof(float), hipMemcpyDeviceToHost, s),
                   "hipMemcpy(mask)") &&
             check(hipStreamSynchronize(s), "hipStreamSynchronize(mask)");
    }
    gpu->active = 0;
    if (!ok) return gpu->fail("resident mask");
    return 1;
}
