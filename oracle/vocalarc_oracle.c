/*
 * CPU oracle for the VocalArc BS-RoFormer separation path -- TEST
 * INFRASTRUCTURE ONLY (see vocalarc_oracle.h).  Each function names the
 * reference lines it restates.  Reference paths are relative to the
 * reference repository root.
 *
 * Build: oracle/Makefile (gcc -O2 -mavx2 -mfma -ffp-contract=off -fopenmp).
 * -ffp-contract=off keeps every a*b+c that the reference evaluates with two
 * roundings as two roundings; the places where the reference uses FMA
 * intrinsics call fmaf() explicitly.
 */
#include "vocalarc_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define OR_PI 3.141592653589793238462643383279502884

void or_set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* ------------------------------------------------------------------------ */
/* shape helpers                                                             */

int or_freq_bins(const or_dims *d) { return d->n_fft / 2 + 1; }
int or_inner(const or_dims *d) { return d->heads * d->dim_head; }
int or_qkv_dim(const or_dims *d) { return 3 * or_inner(d); }
int or_ff1_out(const or_dims *d) { return d->ffn_glu ? 2 * d->ff_dim : d->ff_dim; }
int or_frames(const or_dims *d, int length) { return length / d->hop + 1; }

/* ------------------------------------------------------------------------ */
/* AVX2 kernel restatements: native/native_simd.c                            */

/* Horizontal reduction of an 8-lane accumulator in the order the AVX2 code
   performs it: 128-bit halves added lane-wise, then two hadd steps
   (native/native_simd.c:31-36). */
static float reduce8(const float acc[8]) {
    float l0 = acc[0] + acc[4], l1 = acc[1] + acc[5];
    float l2 = acc[2] + acc[6], l3 = acc[3] + acc[7];
    float h0 = l0 + l1, h1 = l2 + l3;
    return h0 + h1;
}

/* native/native_simd.c:24-39 (vocalarc_dot_avx2) */
float or_dot(const float *a, const float *b, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= n; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = fmaf(a[i + j], b[i + j], acc[j]);
    float sum = reduce8(acc);
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* native/native_simd.c:42-49 */
void or_axpy(float *dst, const float *src, float scale, int n) {
    for (int i = 0; i < n; i++) dst[i] = fmaf(src[i], scale, dst[i]);
}

/* native/native_simd.c:52-58 */
void or_scale(float *dst, float scale, int n) {
    for (int i = 0; i < n; i++) dst[i] *= scale;
}

/* Packed weight layout (native/vocalarc_separation.c:428-457,
   native/native_simd.c:61-95): full 32-wide output tiles stored [in][32],
   then the out%32 tail stored [in][tail].  Each output is a single FMA
   chain over the inputs, seeded with the bias. */
void or_matmul_row(const float *x, const float *w, const float *bias, float *y,
                   int in, int out) {
    int full = (out / 32) * 32;
    for (int ob = 0; ob < full; ob += 32) {
        float acc[32];
        for (int l = 0; l < 32; l++) acc[l] = bias ? bias[ob + l] : 0.0f;
        const float *tile = w + (size_t)(ob / 32) * in * 32;
        for (int i = 0; i < in; i++) {
            const float v = x[i];
            const float *row = tile + (size_t)i * 32;
            for (int l = 0; l < 32; l++) acc[l] = fmaf(v, row[l], acc[l]);
        }
        memcpy(y + ob, acc, sizeof(acc));
    }
    int tail = out - full;
    if (tail > 0) {
        const float *tw = w + (size_t)(out / 32) * in * 32;
        float acc[32];
        for (int l = 0; l < tail; l++) acc[l] = bias ? bias[full + l] : 0.0f;
        for (int i = 0; i < in; i++) {
            const float v = x[i];
            const float *row = tw + (size_t)i * tail;
            for (int l = 0; l < tail; l++) acc[l] = fmaf(v, row[l], acc[l]);
        }
        memcpy(y + full, acc, (size_t)tail * sizeof(float));
    }
}

/* native/native_simd.c:98-121 (vocalarc_rms_norm_row_avx2); also the
   scalar formula at native/vocalarc_separation.c:419-424.  Safe in place. */
void or_rms_norm_row(const float *x, const float *gamma, float *y, int dim) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 8 <= dim; i += 8)
        for (int j = 0; j < 8; j++) acc[j] = fmaf(x[i + j], x[i + j], acc[j]);
    float sum = reduce8(acc);
    for (; i < dim; i++) sum += x[i] * x[i];
    float inverse = sqrtf((float)dim) / sqrtf(sum + 1.0e-12f);
    for (i = 0; i < dim; i++) y[i] = (x[i] * inverse) * gamma[i];
}

/* native/vocalarc_separation.c:383-398: range reduction to 2^n and the
   degree-8 Taylor polynomial of e^r on [-ln2/2, ln2/2]. */
float or_fast_exp(float value) {
    if (value < -88.0f) return 0.0f;
    if (value > 88.0f) value = 88.0f;
    float scaled = value * 1.4426950408889634f;
    float n = floorf(scaled + 0.5f);
    float r = value - n * 0.6931471805599453f;
    float p = 1.0f + r * (1.0f + r * (0.5f + r * (0.1666666666666667f + r *
              (0.0416666666666667f + r * (0.0083333333333333f + r *
              (0.0013888888888889f + r * (0.0001984126984127f + r * 0.0000248015873016f)))))));
    return ldexpf(p, (int)n);
}

/* ------------------------------------------------------------------------ */
/* tensor ops                                                                */

/* native/vocalarc_separation.c:639-664 */
void or_rms_norm(int64_t rows, int dim, const float *x, const float *gamma, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        or_rms_norm_row(x + r * dim, gamma, y + r * dim, dim);
}

/* native/vocalarc_separation.c:612-636 (the CPU path of matmul) */
void or_matmul(int64_t rows, int in, int out, const float *x, const float *w,
               const float *bias, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        or_matmul_row(x + r * in, w, bias, y + r * out, in, out);
}

/* Inverse of the packed layout: W[out][in] row-major (the layout
   native/native_gpu_cuda.cu:104-124 produces for cuBLAS). */
void or_unpack_weight(const float *packed, int in, int out, float *unpacked) {
    int full = (out / 32) * 32, tail = out - full;
    for (int ob = 0; ob < full; ob += 32) {
        const float *tile = packed + (size_t)(ob / 32) * in * 32;
        for (int i = 0; i < in; i++)
            for (int l = 0; l < 32; l++) unpacked[(size_t)(ob + l) * in + i] = tile[(size_t)i * 32 + l];
    }
    const float *tw = packed + (size_t)(out / 32) * in * 32;
    for (int i = 0; i < in; i++)
        for (int l = 0; l < tail; l++) unpacked[(size_t)(full + l) * in + i] = tw[(size_t)i * tail + l];
}

void or_pack_weight(const float *unpacked, int in, int out, float *packed) {
    int full = (out / 32) * 32, tail = out - full;
    for (int ob = 0; ob < full; ob += 32) {
        float *tile = packed + (size_t)(ob / 32) * in * 32;
        for (int i = 0; i < in; i++)
            for (int l = 0; l < 32; l++) tile[(size_t)i * 32 + l] = unpacked[(size_t)(ob + l) * in + i];
    }
    float *tw = packed + (size_t)(out / 32) * in * 32;
    for (int i = 0; i < in; i++)
        for (int l = 0; l < tail; l++) tw[(size_t)i * tail + l] = unpacked[(size_t)(full + l) * in + i];
}

/* native/vocalarc_separation.c:1312-1314 */
void or_rope_frequencies(int dim_head, float *freq) {
    for (int i = 0; i < dim_head / 2; i++)
        freq[i] = 1.0f / powf(10000.0f, (float)(2 * i) / (float)dim_head);
}

/* native/vocalarc_separation.c:726-731: table[position][pair] */
void or_rope_table(int length, int dim_head, float *cosines, float *sines) {
    int pairs = dim_head / 2;
    float *freq = (float *)malloc((size_t)pairs * sizeof(float));
    or_rope_frequencies(dim_head, freq);
    for (int p = 0; p < length; p++)
        for (int k = 0; k < pairs; k++) {
            float angle = (float)p * freq[k];
            cosines[(size_t)p * pairs + k] = cosf(angle);
            sines[(size_t)p * pairs + k] = sinf(angle);
        }
    free(freq);
}

/* native/vocalarc_separation.c:666-672 */
static float gelu1(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f)); }

void or_gelu(int64_t n, float *x) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) x[i] = gelu1(x[i]);
}

/* GELU-GLU: in[rows][2*width] = [value | gate]; out = value * gelu(gate).
   No reference counterpart (the reference FFN is plain GELU); this is the
   GEGLU form of the BS-RoFormer FFN the benchmark configurations name. */
void or_geglu(int64_t rows, int width, const float *in, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *v = in + r * 2 * width;
        const float *g = v + width;
        for (int i = 0; i < width; i++) out[r * width + i] = v[i] * gelu1(g[i]);
    }
}

/* native/vocalarc_separation.c:820-834 */
void or_residual_add(int64_t n, float *dst, const float *src) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) dst[i] += src[i];
}

/* Materialised row softmax (max -> exp -> sum -> divide), the decomposition
   of native/native_gpu_cuda.cu:357-381, with libm expf. */
void or_softmax_rows(int64_t rows, int length, const float *in, float *out) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *x = in + r * length;
        float *y = out + r * length;
        float m = -FLT_MAX;
        for (int i = 0; i < length; i++) m = x[i] > m ? x[i] : m;
        float s = 0.0f;
        for (int i = 0; i < length; i++) { y[i] = expf(x[i] - m); s += y[i]; }
        for (int i = 0; i < length; i++) y[i] = y[i] / s;
    }
}

/* Rotary embedding of interleaved pairs on an [B*H][L][Dh] tensor, with the
   rotation of native/vocalarc_separation.c:692-711. */
void or_rope_bhld(int64_t bh, int length, int dim_head, float *x,
                  const float *cosines, const float *sines) {
    int pairs = dim_head / 2;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < bh; b++)
        for (int p = 0; p < length; p++) {
            float *v = x + ((size_t)b * length + p) * dim_head;
            for (int k = 0; k < pairs; k++) {
                float c = cosines[(size_t)p * pairs + k], s = sines[(size_t)p * pairs + k];
                float a = v[2 * k], bb = v[2 * k + 1];
                v[2 * k] = a * c - bb * s;
                v[2 * k + 1] = a * s + bb * c;
            }
        }
}

/* native/vocalarc_separation.c:692-711 on qkv[S*L][3*H*Dh] (q and k only) */
static void rotary_qkv(const or_dims *d, float *qkv, int64_t tokens, int length,
                       const float *cosines, const float *sines) {
    int inner = or_inner(d), qkv_dim = or_qkv_dim(d), pairs = d->dim_head / 2;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < tokens; t++) {
        int position = (int)(t % length);
        float *row = qkv + t * qkv_dim;
        for (int which = 0; which < 2; which++)
            for (int h = 0; h < d->heads; h++) {
                float *v = row + which * inner + h * d->dim_head;
                for (int k = 0; k < pairs; k++) {
                    float c = cosines[(size_t)position * pairs + k];
                    float s = sines[(size_t)position * pairs + k];
                    float a = v[2 * k], b = v[2 * k + 1];
                    v[2 * k] = a * c - b * s;
                    v[2 * k + 1] = a * s + b * c;
                }
            }
    }
}

/* native/vocalarc_separation.c:753-793: one pass of online softmax per query
   with the reference's fast_exp and its max-update rule. */
void or_attention(const or_dims *d, const float *qkv, float *out, int sequences, int length) {
    const int H = d->heads, Dh = d->dim_head, inner = or_inner(d), qkv_dim = or_qkv_dim(d);
    const float scale = 1.0f / sqrtf((float)Dh);
#pragma omp parallel for schedule(dynamic)
    for (int64_t task = 0; task < (int64_t)sequences * H; task++) {
        int seq = (int)(task / H), head = (int)(task % H);
        const float *sq = qkv + (size_t)seq * length * qkv_dim;
        float *so = out + (size_t)seq * length * inner;
        float *acc = (float *)malloc((size_t)Dh * sizeof(float));
        for (int q = 0; q < length; q++) {
            const float *qv = sq + (size_t)q * qkv_dim + head * Dh;
            for (int i = 0; i < Dh; i++) acc[i] = 0.0f;
            float maximum = -FLT_MAX, denominator = 0.0f;
            for (int k = 0; k < length; k++) {
                const float *kv = sq + (size_t)k * qkv_dim + inner + head * Dh;
                const float *vv = sq + (size_t)k * qkv_dim + 2 * inner + head * Dh;
                float score = or_dot(qv, kv, Dh) * scale;
                if (score > maximum) {
                    float rescale = maximum == -FLT_MAX ? 0.0f : or_fast_exp(maximum - score);
                    or_scale(acc, rescale, Dh);
                    denominator *= rescale;
                    maximum = score;
                    denominator += 1.0f;
                    or_axpy(acc, vv, 1.0f, Dh);
                } else {
                    float weight = or_fast_exp(score - maximum);
                    denominator += weight;
                    or_axpy(acc, vv, weight, Dh);
                }
            }
            float inverse = 1.0f / denominator;
            float *o = so + (size_t)q * inner + head * Dh;
            for (int i = 0; i < Dh; i++) o[i] = acc[i] * inverse;
        }
        free(acc);
    }
}

/* native/vocalarc_separation.c:836-873 (transformer_forward).  The FFN
   activation is GELU (reference) or GELU-GLU (d->ffn_glu). */
void or_transformer(const or_dims *d, const or_layer *w, float *data, int sequences, int length) {
    const int D = d->dim, H = d->heads, inner = or_inner(d), qkv_dim = or_qkv_dim(d);
    const int64_t tokens = (int64_t)sequences * length;
    const int f1 = or_ff1_out(d);
    float *normed = (float *)malloc((size_t)tokens * D * sizeof(float));
    float *qkv = (float *)malloc((size_t)tokens * (qkv_dim > f1 ? qkv_dim : f1) * sizeof(float));
    float *att = (float *)malloc((size_t)tokens * (inner > d->ff_dim ? inner : d->ff_dim) * sizeof(float));
    float *gates = (float *)malloc((size_t)tokens * H * sizeof(float));
    float *proj = (float *)malloc((size_t)tokens * D * sizeof(float));
    float *cosines = (float *)malloc((size_t)length * (d->dim_head / 2) * sizeof(float));
    float *sines = (float *)malloc((size_t)length * (d->dim_head / 2) * sizeof(float));
    or_rope_table(length, d->dim_head, cosines, sines);

    or_rms_norm(tokens, D, data, w->gamma, normed);
    or_matmul(tokens, D, qkv_dim, normed, w->qkv, NULL, qkv);
    if (d->gated) or_matmul(tokens, D, H, normed, w->gate_weight, w->gate_bias, gates);
    rotary_qkv(d, qkv, tokens, length, cosines, sines);
    or_attention(d, qkv, att, sequences, length);
    if (d->gated) {
        /* native/vocalarc_separation.c:808-818 */
#pragma omp parallel for schedule(static)
        for (int64_t t = 0; t < tokens; t++)
            for (int h = 0; h < H; h++) {
                float gate = 1.0f / (1.0f + or_fast_exp(-gates[t * H + h]));
                float *v = att + t * inner + h * d->dim_head;
                for (int i = 0; i < d->dim_head; i++) v[i] *= gate;
            }
    }
    or_matmul(tokens, inner, D, att, w->out_weight, NULL, proj);
    or_residual_add(tokens * D, data, proj);

    or_rms_norm(tokens, D, data, w->ff_gamma, normed);
    or_matmul(tokens, D, f1, normed, w->ff1_weight, w->ff1_bias, qkv);
    if (d->ffn_glu) {
        or_geglu(tokens, d->ff_dim, qkv, att);
    } else {
        or_gelu(tokens * d->ff_dim, qkv);
        memcpy(att, qkv, (size_t)tokens * d->ff_dim * sizeof(float));
    }
    or_matmul(tokens, d->ff_dim, D, att, w->ff2_weight, w->ff2_bias, proj);
    or_residual_add(tokens * D, data, proj);

    free(normed); free(qkv); free(att); free(gates); free(proj); free(cosines); free(sines);
}

/* ------------------------------------------------------------------------ */
/* DSP                                                                       */

typedef struct { double re, im; } cpx;

/* native/vocalarc_separation.c:993-1025: in-place radix-2 decimation in
   time with a bit-reversal permutation and per-stage twiddle recurrence, in
   double precision. */
static void fft_inplace(cpx *v, int n, int inverse) {
    for (int i = 1, j = 0; i < n; i++) {
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) { cpx t = v[i]; v[i] = v[j]; v[j] = t; }
    }
    for (int block = 2; block <= n; block <<= 1) {
        double angle = (2.0 * OR_PI / block) * (inverse ? 1.0 : -1.0);
        double wr_step = cos(angle), wi_step = sin(angle);
        int half = block >> 1;
        for (int start = 0; start < n; start += block) {
            double wr = 1.0, wi = 0.0;
            for (int i = 0; i < half; i++) {
                cpx a = v[start + i], b = v[start + i + half];
                double rr = b.re * wr - b.im * wi;
                double ri = b.re * wi + b.im * wr;
                v[start + i].re = a.re + rr;
                v[start + i].im = a.im + ri;
                v[start + i + half].re = a.re - rr;
                v[start + i + half].im = a.im - ri;
                double next = wr * wr_step - wi * wi_step;
                wi = wr * wi_step + wi * wr_step;
                wr = next;
            }
        }
    }
    if (inverse) {
        double s = 1.0 / n;
        for (int i = 0; i < n; i++) { v[i].re *= s; v[i].im *= s; }
    }
}

/* native/vocalarc_separation.c:1027-1034 */
static int reflect_index(int index, int length) {
    if (length <= 1) return 0;
    while (index < 0 || index >= length) {
        if (index < 0) index = -index;
        else index = 2 * length - 2 - index;
    }
    return index;
}

/* Periodic Hann as the reference evaluates it (native/vocalarc_separation.c:1052) */
void or_hann(int n_fft, float *window) {
    for (int i = 0; i < n_fft; i++)
        window[i] = 0.5f - 0.5f * cosf((float)(2.0 * OR_PI * i / n_fft));
}

/* native/vocalarc_separation.c:1044-1072 */
void or_stft(const or_dims *d, const float *audio, int length, int frames, float *source) {
    const int N = d->n_fft, F = or_freq_bins(d), C = d->channels, hop = d->hop;
    float *window = (float *)malloc((size_t)N * sizeof(float));
    or_hann(N, window);
#pragma omp parallel for schedule(static)
    for (int64_t task = 0; task < (int64_t)C * frames; task++) {
        int c = (int)(task / frames), t = (int)(task % frames);
        cpx *buf = (cpx *)malloc((size_t)N * sizeof(cpx));
        int start = t * hop - N / 2;
        for (int i = 0; i < N; i++) {
            int s = reflect_index(start + i, length);
            buf[i].re = audio[(size_t)c * length + s] * window[i];
            buf[i].im = 0.0;
        }
        fft_inplace(buf, N, 0);
        for (int f = 0; f < F; f++) {
            float *dst = source + (((size_t)f * C + c) * frames + t) * 2;
            dst[0] = (float)buf[f].re;
            dst[1] = (float)buf[f].im;
        }
        free(buf);
    }
    free(window);
}

/* native/vocalarc_separation.c:1084-1136.  The per-frame inverse FFTs are
   independent; the overlap-add runs in frame order exactly as the
   reference's serial loop does. */
void or_istft(const or_dims *d, const float *source, const float *mask, int length,
              int frames, float *audio) {
    const int N = d->n_fft, F = or_freq_bins(d), C = d->channels, hop = d->hop;
    float *window = (float *)malloc((size_t)N * sizeof(float));
    or_hann(N, window);
    double *time = (double *)malloc((size_t)C * frames * N * sizeof(double));
#pragma omp parallel for schedule(static)
    for (int64_t task = 0; task < (int64_t)C * frames; task++) {
        int c = (int)(task / frames), t = (int)(task % frames);
        cpx *buf = (cpx *)calloc((size_t)N, sizeof(cpx));
        for (int f = 0; f < F; f++) {
            const float *s = source + (((size_t)f * C + c) * frames + t) * 2;
            const float *m = mask + (((size_t)f * C + c) * frames + t) * 2;
            buf[f].re = s[0] * m[0] - s[1] * m[1];
            buf[f].im = s[0] * m[1] + s[1] * m[0];
        }
        for (int f = 1; f < F - 1; f++) { buf[N - f].re = buf[f].re; buf[N - f].im = -buf[f].im; }
        fft_inplace(buf, N, 1);
        double *dst = time + ((size_t)c * frames + t) * N;
        for (int i = 0; i < N; i++) dst[i] = buf[i].re;
        free(buf);
    }
    float *norm = (float *)calloc((size_t)length, sizeof(float));
    memset(audio, 0, (size_t)C * length * sizeof(float));
    for (int c = 0; c < C; c++) {
        float *out = audio + (size_t)c * length;
        for (int t = 0; t < frames; t++) {
            const double *src = time + ((size_t)c * frames + t) * N;
            int start = t * hop - N / 2;
            for (int i = 0; i < N; i++) {
                int s = start + i;
                if (s >= 0 && s < length) {
                    out[s] += (float)(src[i] * window[i]);
                    if (c == 0) norm[s] += window[i] * window[i];
                }
            }
        }
    }
    for (int c = 0; c < C; c++) {
        float *out = audio + (size_t)c * length;
        for (int s = 0; s < length; s++) out[s] = norm[s] > 1.0e-12f ? out[s] / norm[s] : 0.0f;
    }
    free(norm); free(time); free(window);
}

/* native/vocalarc_separation.c:887-926 */
void or_band_split(const or_model *m, const float *source, int frames, float *time_sequences) {
    const or_dims *d = &m->d;
    const int C = d->channels, D = d->dim;
    int first[OR_MAX_BANDS];
    for (int b = 0, f = 0; b < d->bands; b++) { first[b] = f; f += d->band_widths[b]; }
#pragma omp parallel for schedule(dynamic)
    for (int b = 0; b < d->bands; b++) {
        int in = m->bands[b].input_dim;
        float *input = (float *)malloc((size_t)frames * in * sizeof(float));
        for (int t = 0; t < frames; t++) {
            float *row = input + (size_t)t * in;
            int o = 0;
            for (int f = 0; f < d->band_widths[b]; f++)
                for (int c = 0; c < C; c++) {
                    const float *s = source + (((size_t)(first[b] + f) * C + c) * frames + t) * 2;
                    row[o++] = s[0];
                    row[o++] = s[1];
                }
            or_rms_norm_row(row, m->bands[b].gamma, row, in);
        }
        for (int t = 0; t < frames; t++)
            or_matmul_row(input + (size_t)t * in, m->bands[b].weight, m->bands[b].bias,
                          time_sequences + ((size_t)b * frames + t) * D, in, D);
        free(input);
    }
}

/* native/vocalarc_separation.c:1316-1340 (mask_band) for every band. */
void or_mask_estimate(const or_model *m, const float *features, int frames, float *mask) {
    const or_dims *d = &m->d;
    const int C = d->channels, D = d->dim, B = d->bands, Hm = d->mask_hidden, F = or_freq_bins(d);
    int first[OR_MAX_BANDS];
    for (int b = 0, f = 0; b < B; b++) { first[b] = f; f += d->band_widths[b]; }
    memset(mask, 0, (size_t)F * C * frames * 2 * sizeof(float));
#pragma omp parallel for schedule(dynamic)
    for (int64_t task = 0; task < (int64_t)B * frames; task++) {
        int b = (int)(task / frames), t = (int)(task % frames);
        const or_mask *w = &m->masks[b];
        int dim = w->output_dim;
        float *hidden = (float *)malloc((size_t)Hm * sizeof(float));
        float *proj = (float *)malloc((size_t)2 * dim * sizeof(float));
        or_matmul_row(features + ((size_t)t * B + b) * D, w->first_weight, w->first_bias, hidden, D, Hm);
        for (int i = 0; i < Hm; i++) hidden[i] = tanhf(hidden[i]);
        or_matmul_row(hidden, w->second_weight, w->second_bias, proj, Hm, 2 * dim);
        for (int i = 0; i < dim; i++) {
            int f = i / (C * 2), c = (i / 2) % C, comp = i % 2;
            mask[(((size_t)(first[b] + f) * C + c) * frames + t) * 2 + comp] =
                proj[i] * (1.0f / (1.0f + or_fast_exp(-proj[dim + i])));
        }
        free(hidden); free(proj);
    }
}

/* [B][T][D] <-> [T][B][D]: native/vocalarc_separation.c:935-965 */
static void transpose_rows(const float *src, float *dst, int a, int b, int D) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < a; i++)
        for (int j = 0; j < b; j++)
            memcpy(dst + ((size_t)j * a + i) * D, src + ((size_t)i * b + j) * D, (size_t)D * sizeof(float));
}

static int forward_impl(const or_model *m, const float *audio, int length, int max_layers,
                        float *vocals, float *features_out, const or_dumps *dumps) {
    const or_dims *d = &m->d;
    const int C = d->channels, D = d->dim, B = d->bands, F = or_freq_bins(d);
    const int T = or_frames(d, length);
    size_t spec = (size_t)F * C * T * 2, feat = (size_t)T * B * D;
    float *source = (float *)malloc(spec * sizeof(float));
    float *seq = (float *)malloc(feat * sizeof(float));
    float *features = (float *)malloc(feat * sizeof(float));
    if (!source || !seq || !features) { free(source); free(seq); free(features); return 0; }
    or_stft(d, audio, length, T, source);
    if (dumps && dumps->source) memcpy(dumps->source, source, spec * sizeof(float));
    or_band_split(m, source, T, seq);
    if (dumps && dumps->band) memcpy(dumps->band, seq, feat * sizeof(float));
    transpose_rows(seq, features, B, T, D);
    if (dumps && dumps->features0) memcpy(dumps->features0, features, feat * sizeof(float));
    int layers = max_layers < d->depth ? max_layers : d->depth;
    for (int l = 0; l < layers; l++) {
        or_transformer(d, &m->layers[2 * l + 0], seq, B, T);
        transpose_rows(seq, features, B, T, D);
        or_transformer(d, &m->layers[2 * l + 1], features, T, B);
        if (l + 1 < d->depth) transpose_rows(features, seq, T, B, D);
        if (dumps && l == 0 && dumps->features1) memcpy(dumps->features1, features, feat * sizeof(float));
        if (dumps && l == d->depth - 1 && dumps->features_last)
            memcpy(dumps->features_last, features, feat * sizeof(float));
    }
    if (features_out) memcpy(features_out, features, feat * sizeof(float));
    if (vocals) {
        or_rms_norm((int64_t)T * B, D, features, m->final_gamma, features);
        float *mask = (float *)malloc(spec * sizeof(float));
        or_mask_estimate(m, features, T, mask);
        if (dumps && dumps->mask) memcpy(dumps->mask, mask, spec * sizeof(float));
        or_istft(d, source, mask, length, T, vocals);
        free(mask);
    }
    free(source); free(seq); free(features);
    return 1;
}

int or_forward(const or_model *m, const float *audio, int length, float *vocals,
               const or_dumps *dumps) {
    return forward_impl(m, audio, length, m->d.depth, vocals, NULL, dumps);
}

int or_forward_layers(const or_model *m, const float *audio, int length, int layers,
                      float *features_out) {
    return forward_impl(m, audio, length, layers, NULL, features_out, NULL);
}

/* ------------------------------------------------------------------------ */
/* chunked separation (no reference counterpart: the reference host runs the
   whole file as one window, native/vocalarc_separation.c:1344)              */

int or_chunk_count(int length, int chunk, int step) {
    if (length <= chunk) return 1;
    return 1 + (length - chunk + step - 1) / step;
}

void or_chunk_weights(int chunk, int step, int index, int count, float *w) {
    int overlap = chunk - step;
    for (int i = 0; i < chunk; i++) {
        float v = 1.0f;
        if (index > 0 && i < overlap) v = ((float)i + 0.5f) / (float)overlap;
        if (index + 1 < count && i >= chunk - overlap) v = ((float)(chunk - i) - 0.5f) / (float)overlap;
        w[i] = v;
    }
}

int or_separate_chunked(const or_model *m, const float *audio, int length, int chunk,
                        int step, float *vocals) {
    const int C = m->d.channels;
    int count = or_chunk_count(length, chunk, step);
    float *in = (float *)malloc((size_t)C * chunk * sizeof(float));
    float *out = (float *)malloc((size_t)C * chunk * sizeof(float));
    float *w = (float *)malloc((size_t)chunk * sizeof(float));
    float *wsum = (float *)calloc((size_t)length, sizeof(float));
    memset(vocals, 0, (size_t)C * length * sizeof(float));
    for (int k = 0; k < count; k++) {
        int start = k * step;
        for (int c = 0; c < C; c++)
            for (int i = 0; i < chunk; i++) {
                int s = start + i;
                in[(size_t)c * chunk + i] = s < length ? audio[(size_t)c * length + s] : 0.0f;
            }
        if (!or_forward(m, in, chunk, out, NULL)) { free(in); free(out); free(w); free(wsum); return 0; }
        or_chunk_weights(chunk, step, k, count, w);
        for (int i = 0; i < chunk; i++) {
            int s = start + i;
            if (s >= length) break;
            for (int c = 0; c < C; c++) vocals[(size_t)c * length + s] += w[i] * out[(size_t)c * chunk + i];
            wsum[s] += w[i];
        }
    }
    for (int c = 0; c < C; c++)
        for (int s = 0; s < length; s++) vocals[(size_t)c * length + s] /= wsum[s];
    free(in); free(out); free(w); free(wsum);
    return 1;
}

/* ------------------------------------------------------------------------ */
/* pack (native/vocalarc_separation.c:489-589)                              */

static const float *next_tensor(const unsigned char **cur, const unsigned char *end, uint64_t expect) {
    if ((size_t)(end - *cur) < sizeof(uint64_t)) return NULL;
    uint64_t count;
    memcpy(&count, *cur, sizeof(count));
    *cur += sizeof(count);
    if (count != expect || (size_t)(end - *cur) < count * sizeof(float)) return NULL;
    const float *r = (const float *)*cur;
    *cur += count * sizeof(float);
    return r;
}

int or_model_parse(or_model *m, const or_dims *d, const void *blob, size_t bytes) {
    memset(m, 0, sizeof(*m));
    m->d = *d;
    if (bytes < 64 || memcmp(blob, "VSCNAT01", 8) != 0) return 0;
    uint32_t fields[14];
    memcpy(fields, (const unsigned char *)blob + 8, sizeof(fields));
    if (fields[0] != 1 || fields[1] != (uint32_t)d->dim || fields[2] != (uint32_t)d->depth ||
        fields[3] != (uint32_t)d->bands || fields[4] != (uint32_t)d->heads ||
        fields[5] != (uint32_t)d->dim_head || fields[6] != (uint32_t)or_freq_bins(d) ||
        fields[7] != (uint32_t)d->channels || fields[8] != (uint32_t)d->n_fft ||
        fields[9] != (uint32_t)d->hop)
        return 0;
    const unsigned char *cur = (const unsigned char *)blob + 64;
    const unsigned char *end = (const unsigned char *)blob + bytes;
    const int D = d->dim, H = d->heads, inner = or_inner(d), f1 = or_ff1_out(d);
    m->layers = (or_layer *)calloc((size_t)d->depth * 2, sizeof(or_layer));
    m->bands = (or_band *)calloc((size_t)d->bands, sizeof(or_band));
    m->masks = (or_mask *)calloc((size_t)d->bands, sizeof(or_mask));
    for (int l = 0; l < d->depth; l++)
        for (int a = 0; a < 2; a++) {
            or_layer *w = &m->layers[2 * l + a];
            if (!(w->gamma = next_tensor(&cur, end, D))) goto fail;
            if (!(w->qkv = next_tensor(&cur, end, (uint64_t)3 * inner * D))) goto fail;
            if (!(w->gate_weight = next_tensor(&cur, end, (uint64_t)H * D))) goto fail;
            if (!(w->gate_bias = next_tensor(&cur, end, H))) goto fail;
            if (!(w->out_weight = next_tensor(&cur, end, (uint64_t)D * inner))) goto fail;
            if (!(w->ff_gamma = next_tensor(&cur, end, D))) goto fail;
            if (!(w->ff1_weight = next_tensor(&cur, end, (uint64_t)f1 * D))) goto fail;
            if (!(w->ff1_bias = next_tensor(&cur, end, f1))) goto fail;
            if (!(w->ff2_weight = next_tensor(&cur, end, (uint64_t)D * d->ff_dim))) goto fail;
            if (!(w->ff2_bias = next_tensor(&cur, end, D))) goto fail;
        }
    for (int b = 0; b < d->bands; b++) {
        int in = d->band_widths[b] * d->channels * 2;
        m->bands[b].input_dim = in;
        if (!(m->bands[b].gamma = next_tensor(&cur, end, in))) goto fail;
        if (!(m->bands[b].weight = next_tensor(&cur, end, (uint64_t)D * in))) goto fail;
        if (!(m->bands[b].bias = next_tensor(&cur, end, D))) goto fail;
    }
    if (!(m->final_gamma = next_tensor(&cur, end, D))) goto fail;
    for (int b = 0; b < d->bands; b++) {
        int in = m->bands[b].input_dim;
        m->masks[b].output_dim = in;
        if (!(m->masks[b].first_weight = next_tensor(&cur, end, (uint64_t)d->mask_hidden * D))) goto fail;
        if (!(m->masks[b].first_bias = next_tensor(&cur, end, d->mask_hidden))) goto fail;
        if (!(m->masks[b].second_weight = next_tensor(&cur, end, (uint64_t)2 * in * d->mask_hidden))) goto fail;
        if (!(m->masks[b].second_bias = next_tensor(&cur, end, (uint64_t)2 * in))) goto fail;
    }
    if (cur != end) goto fail;
    return 1;
fail:
    or_model_free(m);
    return 0;
}

void or_model_free(or_model *m) {
    free(m->layers); free(m->bands); free(m->masks);
    m->layers = NULL; m->bands = NULL; m->masks = NULL;
}
