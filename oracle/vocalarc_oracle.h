/*
 * CPU oracle for the VocalArc BS-RoFormer separation path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * CPU path (native/vocalarc_separation.c + native/native_simd.c) with the
 * model dimensions turned into run-time parameters.  It exists to check the
 * HIP provider; the shipped library never links or calls it.  Only tests/,
 * the smoke entry point and the bench's cpu_baseline leg may use it.
 *
 * Accumulation orders follow the reference's AVX2/FMA kernels
 * (native/native_simd.c:24-121) so that at the reference dimensions the
 * oracle reproduces the reference executable to the last few ulps.
 */
#ifndef VOCALARC_ORACLE_H
#define VOCALARC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_MAX_BANDS 256

/* Model shape.  The reference fixes these at compile time
 * (native/vocalarc_separation.c:33-48); here they are data. */
typedef struct {
    int dim;          /* feature width D                          */
    int depth;        /* axial layers                             */
    int bands;        /* band count                               */
    int heads;        /* attention heads                          */
    int dim_head;     /* per-head width                           */
    int ff_dim;       /* FFN inner width (after GLU when ffn_glu) */
    int ffn_glu;      /* 0: Linear->GELU (reference); 1: GELU-GLU */
    int gated;        /* 1: per-head sigmoid gates (reference)    */
    int mask_hidden;  /* mask-estimator hidden width              */
    int n_fft;
    int hop;
    int channels;
    int band_widths[OR_MAX_BANDS]; /* frequency bins per band      */
} or_dims;

typedef struct {
    const float *gamma, *qkv, *gate_weight, *gate_bias, *out_weight;
    const float *ff_gamma, *ff1_weight, *ff1_bias, *ff2_weight, *ff2_bias;
} or_layer;

typedef struct {
    const float *gamma, *weight, *bias;
    int input_dim;
} or_band;

typedef struct {
    const float *first_weight, *first_bias, *second_weight, *second_bias;
    int output_dim;
} or_mask;

typedef struct {
    or_dims d;
    or_layer *layers;     /* [depth][2] : axis 0 = time, 1 = band */
    or_band *bands;       /* [bands]                              */
    const float *final_gamma;
    or_mask *masks;       /* [bands]                              */
} or_model;

/* ---- pack --------------------------------------------------------------- */
int or_freq_bins(const or_dims *d);
int or_qkv_dim(const or_dims *d);
int or_inner(const or_dims *d);
int or_ff1_out(const or_dims *d);
/* Parse a VSCNAT01 pack (native/vocalarc_separation.c:528-589) laid out for
   `d`.  Returns 1 on success; the model points into `blob`. */
int or_model_parse(or_model *m, const or_dims *d, const void *blob, size_t bytes);
void or_model_free(or_model *m);

/* ---- per-row kernels (native/native_simd.c) ----------------------------- */
float or_dot(const float *a, const float *b, int n);
void or_axpy(float *dst, const float *src, float scale, int n);
void or_scale(float *dst, float scale, int n);
void or_matmul_row(const float *x, const float *packed_w, const float *bias,
                   float *y, int in, int out);
void or_rms_norm_row(const float *x, const float *gamma, float *y, int dim);
float or_fast_exp(float v);

/* ---- tensor ops --------------------------------------------------------- */
void or_rms_norm(int64_t rows, int dim, const float *x, const float *gamma, float *y);
void or_matmul(int64_t rows, int in, int out, const float *x, const float *packed_w,
               const float *bias, float *y);
void or_unpack_weight(const float *packed, int in, int out, float *unpacked);
void or_pack_weight(const float *unpacked, int in, int out, float *packed);
void or_rope_frequencies(int dim_head, float *freq);
void or_rope_table(int length, int dim_head, float *cosines, float *sines);
void or_gelu(int64_t n, float *x);
void or_geglu(int64_t rows, int width, const float *in, float *out);
void or_residual_add(int64_t n, float *dst, const float *src);
void or_softmax_rows(int64_t rows, int length, const float *in, float *out);
void or_rope_bhld(int64_t bh, int length, int dim_head, float *x,
                  const float *cosines, const float *sines);

/* One axial transformer block over data[S][L][D] (in place).
   native/vocalarc_separation.c:836-873. */
void or_transformer(const or_dims *d, const or_layer *w, float *data, int sequences, int length);
/* Attention core only: qkv[S*L][3*H*Dh] (rotary already applied) -> out[S*L][H*Dh]. */
void or_attention(const or_dims *d, const float *qkv, float *out, int sequences, int length);

/* ---- DSP ---------------------------------------------------------------- */
void or_hann(int n_fft, float *window);
/* source[F][C][T][2]; audio[C][length] */
void or_stft(const or_dims *d, const float *audio, int length, int frames, float *source);
void or_istft(const or_dims *d, const float *source, const float *mask, int length,
              int frames, float *audio);
/* time_sequences[B][T][D] */
void or_band_split(const or_model *m, const float *source, int frames, float *time_sequences);
/* features[T][B][D] (already final-normed) -> mask[F][C][T][2] */
void or_mask_estimate(const or_model *m, const float *features, int frames, float *mask);

/* Full forward (native/vocalarc_separation.c:1342-1445): audio[C][length]
   -> vocals[C][length].  Any of the dump pointers may be NULL. */
typedef struct {
    float *source;      /* [F][C][T][2]  */
    float *band;        /* [B][T][D]     */
    float *features0;   /* [T][B][D]     */
    float *features1;   /* after layer 0 */
    float *features_last;
    float *mask;        /* [F][C][T][2]  */
} or_dumps;
int or_frames(const or_dims *d, int length);
int or_forward(const or_model *m, const float *audio, int length, float *vocals,
               const or_dumps *dumps);
/* Forward stopping after `layers` axial layers: used to time a bounded
   sample of the full model on the CPU. */
int or_forward_layers(const or_model *m, const float *audio, int length, int layers,
                      float *features_out);

/* Chunked separation: windows of `chunk` samples every `step` samples,
   linear cross-fade over the overlap, normalised by the summed fade weights. */
int or_chunk_count(int length, int chunk, int step);
void or_chunk_weights(int chunk, int step, int index, int count, float *weights);
int or_separate_chunked(const or_model *m, const float *audio, int length, int chunk,
                        int step, float *vocals);

void or_set_threads(int threads);

#ifdef __cplusplus
}
#endif

#endif
