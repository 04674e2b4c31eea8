// STFT / iSTFT for the separation front and back end.
//
// Numerics follow native/vocalarc_separation.c:993-1136: float samples times
// the float periodic Hann window, a radix-2 FFT in double precision, results
// rounded to float; the inverse applies the complex mask in float, fills the
// Hermitian half, inverse-FFTs in double, and the overlap-add accumulates
// (float)(x * w) in frame order and divides by the float sum of w^2.
//
// One workgroup transforms one frame in LDS (n_fft complex doubles).  The
// overlap-add is a gather (each output sample sums the frames that cover it
// in ascending frame order), so no atomics are needed and the summation
// order is the reference's.
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

// In-place radix-2 decimation-in-time FFT of buf[n] (already in bit-reversed
// order).  tw[j] = exp(-2*pi*i*j/n), j < n/2; inverse uses the conjugate.
VH_DEVICE void fft_lds(double2_t *buf, const double2_t *__restrict__ tw, int n, bool inverse) {
    const int tid = (int)threadIdx.x, nt = (int)blockDim.x;
    for (int half = 1; half < n; half <<= 1) {
        const int stride = n / (2 * half);
        for (int j = tid; j < n / 2; j += nt) {
            const int k = j & (half - 1);
            const int i0 = (j - k) * 2 + k;
            const int i1 = i0 + half;
            double2_t w = tw[k * stride];
            if (inverse) w.y = -w.y;
            const double2_t a = buf[i0], b = buf[i1];
            const double rr = b.x * w.x - b.y * w.y;
            const double ri = b.x * w.y + b.y * w.x;
            buf[i0] = {a.x + rr, a.y + ri};
            buf[i1] = {a.x - rr, a.y - ri};
        }
        __syncthreads();
    }
}

VH_DEVICE int bitrev_dev(int i, int log2n) { return (int)(__brev((unsigned)i) >> (32 - log2n)); }

// One frame of the STFT of one signal.  Signal `sig` = chunk * C + c reads
// samples audio[c][start_k + j] (zero beyond `audio_len`), j in
// [0, sig_len), with centre reflect padding inside the window of the chunk.
// Output source[chunk][F][C][T][2].
struct StftArgs {
    const float *audio;
    int64_t audio_len;       // samples per channel of the audio buffer
    const int64_t *starts;   // chunk start sample per chunk (device), or null = 0
    int sig_len;             // window (chunk) length
    int C, T, F, n_fft, log2n, hop;
    const float *window;     // [n_fft]
    const double2_t *tw;     // [n_fft/2]
    float *source;
};

static __global__ __launch_bounds__(256) void stft_kernel(StftArgs a) {
    extern __shared__ double2_t sbuf[];
    const int t = (int)blockIdx.x;
    const int sig = (int)blockIdx.y;
    const int chunk = sig / a.C, c = sig % a.C;
    const int64_t start = a.starts ? a.starts[chunk] : 0;
    const float *src = a.audio + (size_t)c * a.audio_len;
    const int base = t * a.hop - a.n_fft / 2;
    for (int i = (int)threadIdx.x; i < a.n_fft; i += (int)blockDim.x) {
        const int j = reflect_index_dev(base + i, a.sig_len);
        const int64_t g = start + j;
        const float x = g < a.audio_len ? src[g] : 0.0f;
        sbuf[bitrev_dev(i, a.log2n)] = {(double)(x * a.window[i]), 0.0};
    }
    __syncthreads();
    fft_lds(sbuf, a.tw, a.n_fft, false);
    float *dst = a.source + (size_t)chunk * a.F * a.C * a.T * 2;
    for (int f = (int)threadIdx.x; f < a.F; f += (int)blockDim.x) {
        float2 v;
        v.x = (float)sbuf[f].x;
        v.y = (float)sbuf[f].y;
        *reinterpret_cast<float2 *>(dst + (((size_t)f * a.C + c) * a.T + t) * 2) = v;
    }
}

// Complex mask multiply + Hermitian fill + inverse FFT + window for one
// frame; frames[sig][T][n_fft] = (float)(x * w).
struct IstftArgs {
    const float *source;  // [chunk][F][C][T][2]
    const float *mask;    // same layout
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
    const size_t off = (size_t)chunk * a.F * a.C * a.T * 2;
    const int n = a.n_fft;
    for (int f = (int)threadIdx.x; f < a.F; f += (int)blockDim.x) {
        const size_t e = off + (((size_t)f * a.C + c) * a.T + t) * 2;
        const float2 s = *reinterpret_cast<const float2 *>(a.source + e);
        const float2 m = *reinterpret_cast<const float2 *>(a.mask + e);
        const float re = s.x * m.x - s.y * m.y;
        const float im = s.x * m.y + s.y * m.x;
        sbuf[bitrev_dev(f, a.log2n)] = {(double)re, (double)im};
        if (f >= 1 && f < a.F - 1) sbuf[bitrev_dev(n - f, a.log2n)] = {(double)re, -(double)im};
    }
    __syncthreads();
    fft_lds(sbuf, a.tw, n, true);
    const double scale = 1.0 / n;
    float *dst = a.frames + ((size_t)sig * a.T + t) * n;
    for (int i = (int)threadIdx.x; i < n; i += (int)blockDim.x)
        dst[i] = (float)((sbuf[i].x * scale) * (double)a.window[i]);
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
    for (int t = t_lo; t <= t_hi; t++) {
        const int i = s - t * a.hop + half;
        const float w = a.window[i];
        acc += fr[(size_t)t * a.n_fft + i];
        norm += w * w;
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
