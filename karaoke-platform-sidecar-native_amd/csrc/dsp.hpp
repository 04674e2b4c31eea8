// STFT / iSTFT for the separation front and back end.
//
// Numerics follow native/vocalarc_separation.c:993-1136: float samples times
// the float periodic Hann window, a radix-2 FFT in double precision, results
// rounded to float; the inverse applies the complex mask in float, fills the
// Hermitian half, inverse-FFTs in double, and the overlap-add accumulates
// (float)(x * w) in frame order and divides by the float sum of w^2.
//
// One workgroup transforms one frame in LDS (n_fft complex doubles).  The FFT
// is the reference's radix-2 decimation in time with its butterflies grouped
// three stages at a time: a thread loads the 8 points {base + k + j*h} that
// stages h, 2h and 4h combine only among themselves, applies those 12
// butterflies in registers and writes them back -- the same operations on
// every point as stage-by-stage radix-2, in 4 LDS passes (and 4 barriers)
// instead of 11 for n = 2048, with points skewed in LDS (fft_slot) so their
// accesses do not collide on banks.  The overlap-add
// is a gather (each output sample sums the frames that cover it in ascending
// frame order), so no atomics are needed and the summation order is the
// reference's.
#pragma once

#include "common.hpp"

namespace vh {

struct double2_t {
    double x, y;
};

VH_DEVICE int reflect_index_dev(int index, int length) {
    if (length <= 1) return 0;
    while (index < 0 || index >= length) {
        if (index < 0) index = -index;
        else index = 2 * length - 2 - index;
    }
    return index;
}

// LDS slot of point i.  A 16-byte point covers 4 of the 64 banks, so point
// slot q uses bank quad q % 16; the skews i/8 and i/256 give 8 consecutive
// lanes distinct quads in every access pattern of the transform: the
// bit-reversed scatter (points 256 apart), the first pass (8 apart), the
// second (stride-1 within 8-lane groups) and the stride-1 passes.
VH_DEVICE int fft_slot(int i) { return i + (i >> 3) + (i >> 8); }
// Radix-2 butterfly of the decimation-in-time FFT: (a, b) -> (a + w b, a - w b).
VH_DEVICE void fft_bfly(double2_t &a, double2_t &b, double2_t w) {
    const double rr = b.x * w.x - b.y * w.y;
    const double ri = b.x * w.y + b.y * w.x;
    b = {a.x - rr, a.y - ri};
    a = {a.x + rr, a.y + ri};
}

// W_M^x, M = 2^lm, from tw[j] = exp(-2*pi*i*j/n) (conjugated for the inverse).
VH_DEVICE double2_t fft_tw(const double2_t *__restrict__ tw, int x, int lm, int log2n, bool inverse) {
    double2_t w = tw[x << (log2n - lm)];
    if (inverse) w.y = -w.y;
    return w;
}

// In-place FFT of buf (n = 2^log2n points, slot fft_slot(i), input in
// bit-reversed order); every thread of the block takes part.
VH_DEVICE void fft_lds(double2_t *buf, const double2_t *__restrict__ tw, int log2n, bool inverse) {
    const int n = 1 << log2n;
    const int tid = (int)threadIdx.x, nt = (int)blockDim.x;
    for (int s = 0; s < log2n;) {
        const int r = min(3, log2n - s);  // stages merged in this pass
        const int h = 1 << s;
        for (int g = tid; g < (n >> r); g += nt) {
            const int k = g & (h - 1);
            const int base = (g >> s) << (s + r);
            if (r == 3) {
                double2_t p[8];
#pragma unroll
                for (int j = 0; j < 8; j++) p[j] = buf[fft_slot(base + k + j * h)];
                const double2_t w1 = fft_tw(tw, k, s + 1, log2n, inverse);
                const double2_t w2a = fft_tw(tw, k, s + 2, log2n, inverse);
                const double2_t w2b = fft_tw(tw, k + h, s + 2, log2n, inverse);
                fft_bfly(p[0], p[1], w1);
                fft_bfly(p[2], p[3], w1);
                fft_bfly(p[4], p[5], w1);
                fft_bfly(p[6], p[7], w1);
                fft_bfly(p[0], p[2], w2a);
                fft_bfly(p[1], p[3], w2b);
                fft_bfly(p[4], p[6], w2a);
                fft_bfly(p[5], p[7], w2b);
#pragma unroll
                for (int j = 0; j < 4; j++) fft_bfly(p[j], p[j + 4], fft_tw(tw, k + j * h, s + 3, log2n, inverse));
#pragma unroll
                for (int j = 0; j < 8; j++) buf[fft_slot(base + k + j * h)] = p[j];
            } else if (r == 2) {
                double2_t p[4];
#pragma unroll
                for (int j = 0; j < 4; j++) p[j] = buf[fft_slot(base + k + j * h)];
                const double2_t w1 = fft_tw(tw, k, s + 1, log2n, inverse);
                fft_bfly(p[0], p[1], w1);
                fft_bfly(p[2], p[3], w1);
                fft_bfly(p[0], p[2], fft_tw(tw, k, s + 2, log2n, inverse));
                fft_bfly(p[1], p[3], fft_tw(tw, k + h, s + 2, log2n, inverse));
#pragma unroll
                for (int j = 0; j < 4; j++) buf[fft_slot(base + k + j * h)] = p[j];
            } else {
                double2_t a = buf[fft_slot(base + k)], b = buf[fft_slot(base + k + h)];
                fft_bfly(a, b, fft_tw(tw, k, s + 1, log2n, inverse));
                buf[fft_slot(base + k)] = a;
                buf[fft_slot(base + k + h)] = b;
            }
        }
        __syncthreads();
        s += r;
    }
}

// LDS bytes of one padded n-point transform (slots up to fft_slot(n - 1)).
inline size_t fft_lds_bytes(int n) { return (size_t)(n + n / 8 + n / 256 + 1) * sizeof(double2_t); }

VH_DEVICE int bitrev_dev(int i, int log2n) { return (int)(__brev((unsigned)i) >> (32 - log2n)); }

// The STFT / iSTFT kernels run 256 threads per frame; their global loads are
// issued DSP_UNROLL per thread at a time so a frame waits on memory once per
// 2048 elements rather than once per element.
constexpr int DSP_THREADS = 256, DSP_UNROLL = 8;

// One frame of the STFT of one signal.  Signal `sig` = chunk * C + c reads
// samples audio[c][start_k + j] (zero beyond `audio_len`), j in
// [0, sig_len), with centre reflect padding inside the window of the chunk.
// Output: bins (chunk, f, c, t) of `source` in layout `out`.
struct StftArgs {
    const float *audio;
    int64_t audio_len;       // samples per channel of the audio buffer
    const int64_t *starts;   // chunk start sample per chunk (device), or null = 0
    int sig_len;             // window (chunk) length
    int C, T, F, n_fft, log2n, hop;
    const float *window;     // [n_fft]
    const double2_t *tw;     // [n_fft/2]
    float *source;
    SpecLayout out;
};

static __global__ __launch_bounds__(256) void stft_kernel(StftArgs a) {
    extern __shared__ double2_t sbuf[];
    const int t = (int)blockIdx.x;
    const int sig = (int)blockIdx.y;
    const int chunk = sig / a.C, c = sig % a.C;
    const int64_t start = a.starts ? a.starts[chunk] : 0;
    const float *src = a.audio + (size_t)c * a.audio_len;
    const int base = t * a.hop - a.n_fft / 2;
    const int tid = (int)threadIdx.x;
    for (int i0 = 0; i0 < a.n_fft; i0 += DSP_THREADS * DSP_UNROLL) {
        float xv[DSP_UNROLL], wv[DSP_UNROLL];
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int i = i0 + tid + DSP_THREADS * u;
            xv[u] = 0.0f;
            wv[u] = 0.0f;
            if (i < a.n_fft) {
                const int64_t g = start + reflect_index_dev(base + i, a.sig_len);
                xv[u] = g < a.audio_len ? src[g] : 0.0f;
                wv[u] = a.window[i];
            }
        }
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int i = i0 + tid + DSP_THREADS * u;
            if (i < a.n_fft) sbuf[fft_slot(bitrev_dev(i, a.log2n))] = {(double)(xv[u] * wv[u]), 0.0};
        }
    }
    __syncthreads();
    fft_lds(sbuf, a.tw, a.log2n, false);
    for (int f = (int)threadIdx.x; f < a.F; f += (int)blockDim.x) {
        const double2_t z = sbuf[fft_slot(f)];
        *reinterpret_cast<float2 *>(a.source + 2 * spec_at(a.out, chunk, f, c, t)) = float2{(float)z.x, (float)z.y};
    }
}

// Complex mask multiply + Hermitian fill + inverse FFT + window for one
// frame; frames[sig][T][n_fft] = (float)(x * w).
struct IstftArgs {
    const float *source;  // bins (chunk, f, c, t) in layout `in`
    const float *mask;    // same layout
    SpecLayout in;
    int C, T, F, n_fft, log2n;
    const float *window;
    const double2_t *tw;
    float *frames;        // [sig][T][n_fft]
};

static __global__ __launch_bounds__(256) void istft_frames_kernel(IstftArgs a) {
    extern __shared__ double2_t sbuf[];
    const int t = (int)blockIdx.x;
    const int sig = (int)blockIdx.y;
    const int chunk = sig / a.C, c = sig % a.C;
    const int n = a.n_fft;
    const int tid = (int)threadIdx.x;
    for (int f0 = 0; f0 < a.F; f0 += DSP_THREADS * DSP_UNROLL) {
        float2 sv[DSP_UNROLL], mv[DSP_UNROLL];
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int f = f0 + tid + DSP_THREADS * u;
            if (f < a.F) {
                const int64_t e = 2 * spec_at(a.in, chunk, f, c, t);
                sv[u] = *reinterpret_cast<const float2 *>(a.source + e);
                mv[u] = *reinterpret_cast<const float2 *>(a.mask + e);
            }
        }
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int f = f0 + tid + DSP_THREADS * u;
            if (f < a.F) {
                const float re = sv[u].x * mv[u].x - sv[u].y * mv[u].y;
                const float im = sv[u].x * mv[u].y + sv[u].y * mv[u].x;
                sbuf[fft_slot(bitrev_dev(f, a.log2n))] = {(double)re, (double)im};
                if (f >= 1 && f < a.F - 1) sbuf[fft_slot(bitrev_dev(n - f, a.log2n))] = {(double)re, -(double)im};
            }
        }
    }
    __syncthreads();
    fft_lds(sbuf, a.tw, a.log2n, true);
    const double scale = 1.0 / n;
    float *dst = a.frames + ((size_t)sig * a.T + t) * n;
    for (int i0 = 0; i0 < n; i0 += DSP_THREADS * DSP_UNROLL) {
        float wv[DSP_UNROLL];
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int i = i0 + tid + DSP_THREADS * u;
            wv[u] = i < n ? a.window[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int i = i0 + tid + DSP_THREADS * u;
            if (i < n) dst[i] = (float)((sbuf[fft_slot(i)].x * scale) * (double)wv[u]);
        }
    }
}

// Gather overlap-add: out[sig][s] = sum_t frames[sig][t][s - t*hop + n/2] /
// sum_t w^2, ascending t; 0 where the envelope is <= 1e-12.
struct OlaArgs {
    const float *frames;
    const float *window;
    int T, n_fft, hop, length;
    float *out;            // [sig][out_pitch]
    int64_t out_pitch;
};

static __global__ __launch_bounds__(256) void ola_kernel(OlaArgs a) {
    const int sig = (int)blockIdx.y;
    const int s = (int)(blockIdx.x * 256 + threadIdx.x);
    if (s >= a.length) return;
    const int half = a.n_fft / 2;
    // frames t with 0 <= s - (t*hop - half) < n_fft
    int t_lo = s + half - a.n_fft + 1;
    t_lo = t_lo <= 0 ? 0 : (t_lo + a.hop - 1) / a.hop;
    int t_hi = (s + half) / a.hop;
    if (t_hi > a.T - 1) t_hi = a.T - 1;
    float acc = 0.0f, norm = 0.0f;
    const float *fr = a.frames + (size_t)sig * a.T * a.n_fft;
    for (int t0 = t_lo; t0 <= t_hi; t0 += DSP_UNROLL) {
        float fv[DSP_UNROLL], wv[DSP_UNROLL];
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++) {
            const int t = t0 + u, i = s - t * a.hop + half;
            fv[u] = t <= t_hi ? fr[(size_t)t * a.n_fft + i] : 0.0f;
            wv[u] = t <= t_hi ? a.window[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < DSP_UNROLL; u++)  // ascending frame order, as the reference
            if (t0 + u <= t_hi) {
                acc += fv[u];
                norm += wv[u] * wv[u];
            }
    }
    a.out[(size_t)sig * a.out_pitch + s] = norm > 1.0e-12f ? acc / norm : 0.0f;
}

// Cross-fade of chunk outputs: chunks[k][C][chunk] -> out[C][length],
// out = sum_k w_k * y_k / sum_k w_k over the chunks covering each sample, in
// ascending k.  Fade-in over the first (chunk-step) samples of every chunk
// but the first, fade-out over the last (chunk-step) of every chunk but the
// last: w = (i + 0.5)/overlap and ((chunk - i) - 0.5)/overlap.
struct FadeArgs {
    const float *chunks;
    int count, chunk, step, C;
    int64_t length;
    float *out;
    const float *mix;    // input audio [C][length] (for the instrumental)
    float *instrumental; // may be null
};

VH_DEVICE float fade_weight(int i, int k, int count, int chunk, int step) {
    const int overlap = chunk - step;
    float v = 1.0f;
    if (k > 0 && i < overlap) v = ((float)i + 0.5f) / (float)overlap;
    if (k + 1 < count && i >= chunk - overlap) v = ((float)(chunk - i) - 0.5f) / (float)overlap;
    return v;
}

static __global__ __launch_bounds__(256) void crossfade_kernel(FadeArgs a) {
    const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int c = (int)blockIdx.y;
    if (s >= a.length) return;
    int k_hi = (int)(s / a.step);
    if (k_hi > a.count - 1) k_hi = a.count - 1;
    int64_t lo = s - a.chunk + 1;
    int k_lo = lo <= 0 ? 0 : (int)((lo + a.step - 1) / a.step);
    float acc = 0.0f, ws = 0.0f;
    for (int k = k_lo; k <= k_hi; k++) {
        const int i = (int)(s - (int64_t)k * a.step);
        const float w = fade_weight(i, k, a.count, a.chunk, a.step);
        acc += w * a.chunks[((size_t)k * a.C + c) * a.chunk + i];
        ws += w;
    }
    const float v = acc / ws;
    a.out[(size_t)c * a.length + s] = v;
    if (a.instrumental) a.instrumental[(size_t)c * a.length + s] = a.mix[(size_t)c * a.length + s] - v;
}

// instrumental = mix - vocals (native/vocalarc_separation.c:1589-1591)
static __global__ __launch_bounds__(256) void subtract_kernel(const float *__restrict__ mix,
                                                              const float *__restrict__ vocals,
                                                              float *__restrict__ inst, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < n) inst[e] = mix[e] - vocals[e];
}

}  // namespace vh
