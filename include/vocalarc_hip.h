/*
 * vocalarc_hip.h -- harness C-ABI of the MI355X (gfx950) VocalArc provider.
 *
 * The reference host reaches the GPU only through native_gpu.h (declared in
 * this directory as well).  That ABI is bound to the host's compile-time
 * shape (dim 256, 90 bands, hop 512, GELU) and never sees the STFT, iSTFT or
 * band split.  These entry points expose the same device path with the shape
 * as data, so the benchmark configurations (dim 384, 62 bands, hop 441,
 * GELU-GLU, chunked 5-minute input) run through the same kernels.  Each
 * function names the reference function whose computation it performs.
 *
 * Conventions: plain pointers and sizes only.  Pointers documented as
 * "device" are device memory owned by the caller; the library allocates its
 * own scratch.  Work is issued on the context's stream (default: the null
 * stream; see vh_set_stream) and is complete when vh_synchronize returns.
 * Functions return 1 on success and 0 on failure (message: vh_last_error).
 */
#ifndef VOCALARC_HIP_H
#define VOCALARC_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VH_MAX_BANDS 256

/* Model shape; the reference fixes these at compile time
   (native/vocalarc_separation.c:33-57).  Same field order as the oracle's. */
typedef struct {
    int dim, depth, bands, heads, dim_head, ff_dim;
    int ffn_glu;      /* 0: Linear->GELU (reference FFN), 1: GELU-GLU   */
    int gated;        /* 1: per-head sigmoid gates (reference)           */
    int mask_hidden;  /* mask-estimator hidden width (reference: FF_DIM) */
    int n_fft, hop, channels;
    int band_widths[VH_MAX_BANDS];
} vh_dims;

typedef struct vh_context vh_context;
typedef struct vh_model vh_model;

/* ---- context ----------------------------------------------------------- */
vh_context *vh_create(void);
/* Also frees every model loaded in ctx that vh_model_free has not freed. */
void vh_destroy(vh_context *ctx);
int vh_set_stream(vh_context *ctx, void *hip_stream);
int vh_synchronize(vh_context *ctx);
const char *vh_last_error(void);
const char *vh_device_name(vh_context *ctx);

/* ---- isolated kernels on device buffers --------------------------------- */
/* RMSNorm rows: y = x * sqrt(dim)/sqrt(sum x^2 + 1e-12) * gamma
   (native/vocalarc_separation.c:419-424, native/native_simd.c:98-121). */
int vh_rmsnorm(vh_context *ctx, int64_t rows, int dim, const float *x, const float *gamma, float *y);
/* Same, y written as bf16 (round to nearest even): the bf16 variant's GEMM operand. */
int vh_rmsnorm_bf16(vh_context *ctx, int64_t rows, int dim, const float *x, const float *gamma, void *y);
/* Same, y written as h2 rows for vh_gemm_h2 with VH_H2_A_ROWS: the values
   times 2^e (e: the largest with bound * 2^e < 2^14, bound the device float
   *bound, e.g. vh_operand_bounds' out[0]) split into fp16 pieces h, m; every
   16 k of a row take the row's 64 fp32 bytes: h of k 0-3, 8-11 | h of k 4-7,
   12-15 | m of k 0-3, 8-11 | m of k 4-7, 12-15 (dim a multiple of 16). */
int vh_rmsnorm_h2(vh_context *ctx, int64_t rows, int dim, const float *x, const float *gamma, const float *bound,
                  float *y);
/* Row softmax over [rows][len] (native/native_gpu_cuda.cu:357-381). */
int vh_softmax_rows(vh_context *ctx, int64_t rows, int len, const float *in, float *out);
/* Rotary embedding in place on [bh][len][dim_head] with base 10000
   (native/vocalarc_separation.c:692-744). dim_head must be 64. */
int vh_rope_bhld(vh_context *ctx, int64_t bh, int len, int dim_head, float *x);
/* GELU-GLU: in[rows][2*width] = [value|gate] -> out[rows][width]. */
int vh_geglu(vh_context *ctx, int64_t rows, int width, const float *in, float *out);
/* x[n] += r[n] (native/vocalarc_separation.c:820-834). */
int vh_residual_add(vh_context *ctx, int64_t n, float *x, const float *r);
/* C[M][N] (op)= A[M][K] * W[N][K]^T (+bias): the token-wise linear
   (native/vocalarc_separation.c:631-636).  epilogue: 0 store, 1 GELU,
   2 tanh, 3 residual (C +=), 4 GELU-GLU on interleaved columns. */
int vh_gemm(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, const float *W, int ldw,
            const float *bias, float *C, int ldc, int epilogue);
/* bf16-MFMA variant of vh_gemm: Wh a bf16 weight copy [N][ldw] (ldw a
   multiple of 8, >= K, zero padded), fp32 accumulation and epilogue.
   A is fp32, rounded to bf16 (nearest even) as it is staged, or bf16 with
   VH_BF16_A (then K and lda multiples of 8); C is fp32, or bf16 with
   VH_BF16_C (not with the residual epilogue).  K and lda multiples of 4,
   ldc at most 2^21, A and Wh 16-byte aligned.  bf16 A with K a multiple of 32 runs the
   pipelined kernel (direct global->LDS loads); VH_BF16_STAGED forces the
   register-staged kernel instead (same results, bit for bit). */
#define VH_BF16_A 1
#define VH_BF16_C 2
#define VH_BF16_STAGED 4
int vh_gemm_bf16(vh_context *ctx, int64_t M, int N, int K, const void *A, int lda, const void *Wh, int ldw,
                 const float *bias, void *C, int ldc, int epilogue, int flags);
/* vh_gemm in fp32 accuracy on bf16 matrix cores: every fp32 value is the
   exact sum of three bf16 pieces (h = bf16(x), m = bf16(x - h),
   l = x - h - m) and the six piece products that reach 2^-24 of a product
   are accumulated in fp32.  Ws: the weight's pieces from vh_split_weights.
   K a multiple of 16, lda a multiple of 4 and at most 2^21, ldc at most
   2^21, A and Ws 16-byte aligned.  The token-wise linear of
   native/vocalarc_separation.c:631-636, as vh_gemm. */
int vh_gemm_split(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, const void *Ws,
                  const float *bias, float *C, int ldc, int epilogue);
/* Bytes of the pieces of an N x K weight (N rounded up to 128 rows). */
size_t vh_split_bytes(int N, int K);
/* fp32 W[N][ldw_in] (K a multiple of 16) -> its bf16 pieces for
   vh_gemm_split, vh_split_bytes(N, K) bytes, tile-major: piece p (h, m, l)
   of W[n][k] at bf16 index
     ((n/128 * K/16 + k/16) * 3 + p) * 2048 + (n%128) * 16 + 8 * (s ^ (n/8)%2) + e
   where within every group of 16 k the (slot s, element e) order is
   k 0-3, 8-11 (s = 0), 4-7, 12-15 (s = 1); rows past N are zero. */
int vh_split_weights(vh_context *ctx, int N, int K, const float *W, int ldw_in, void *Ws);
/* vh_gemm in fp32 accuracy on fp16 matrix cores: A and W are scaled by
   powers of two (A's from a_bound, which every |A| element must respect;
   a_bound <= 0 computes max|A| on the device first; W's from its maximum)
   and every scaled value is split into two fp16 pieces (h = fp16(y),
   m = fp16(y - h)); the products hh, hm, mh are accumulated in fp32 and the
   result scaled back.  Wp: the weight's pieces from vh_split_weights_h2.
   K a multiple of 16, lda a multiple of 4 and at most 2^21, ldc at most
   2^21, A 16-byte aligned.  The token-wise linear of native/vocalarc_separation.c:631-636,
   as vh_gemm; the default fp32 path's linears. */
#define VH_H2_A_ROWS 1 /* flags of vh_gemm_h2: A given as h2 rows (vh_rmsnorm_h2), scaled from a_bound */
int vh_gemm_h2(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, float a_bound, const void *Wp,
               const float *bias, float *C, int ldc, int epilogue, int flags);
/* vh_gemm_h2 as the fused transformer block runs it: the bound is the device
   float a_bound_dev; with VH_H2_ROW_NORM (fp32 A, epilogue VH_EPI_STORE, GELU
   or GELU_GLU, K the row length) the GEMM of an RMSNorm of A's rows -- each
   output row is multiplied by sqrt(K) / sqrt(sum_k A^2 + 1e-12) before bias
   and activation, Wp holding the norm's gain folded in (the pieces of
   W[n][k] gamma[k]) -- so the normalised rows are never written; zero_slot
   (may be null) is set to 0 by the kernel; amax (epilogue VH_EPI_RESIDUAL,
   may be null) is raised to max |C| over the elements written, the bound of
   the next row-norm GEMM's A. */
#define VH_H2_ROW_NORM 2 /* flags of vh_gemm_h2_ex */
int vh_gemm_h2_ex(vh_context *ctx, int64_t M, int N, int K, const float *A, int lda, const float *a_bound_dev,
                  const void *Wp, const float *bias, float *C, int ldc, int epilogue, int flags, float *zero_slot,
                  float *amax);
/* Bytes of the fp16 pieces of an N x K weight: a 256-byte header, then two
   planes (N rounded up to 128 rows). */
size_t vh_h2_bytes(int N, int K);
/* fp32 W[N][ldw_in] (K a multiple of 16) -> max|W| in the header (float 0)
   and the fp16 pieces of W * 2^e (e: the largest with max|W| * 2^e < 2^14),
   tile-major as vh_split_weights with two planes: piece p (h, m) of W[n][k]
   at fp16 index 128 + ((n/128 * K/16 + k/16) * 2 + p) * 2048 + (n%128) * 16
   + 8 * (s ^ (n/8)%2) + e.  Wp 256-byte aligned, vh_h2_bytes(N, K) bytes. */
int vh_split_weights_h2(vh_context *ctx, int N, int K, const float *W, int ldw_in, void *Wp);
/* Bounds the model gives vh_gemm_h2 for A operands downstream of an RMSNorm
   with device gain gamma[D] (|y_i| <= ||y||_2 <= sqrt(D) max|gamma|):
   out[0] = sqrt(D) max|gamma| (1 + 2^-10); with W [N][D] (and bias b, may be
   null) out[1] = t, or t^2 when square (a GELU-GLU of two outputs), where
   t = (out[0] max_n ||W_n||_2 + max_n |b_n|)(1 + 2^-10) bounds every output
   of W y + b; 0 without W.  out: 2 device floats. */
int vh_operand_bounds(vh_context *ctx, const float *gamma, int D, const float *W, int N, const float *b, int square,
                      float *out);
/* fp32 src[rows][cols] -> bf16 dst[rows][ld] (round to nearest even). */
int vh_to_bf16(vh_context *ctx, int64_t rows, int cols, const float *src, void *dst, int ld);
/* Fused attention core over qkv[S*L][3*H*64] (rotary applied here):
   native/vocalarc_separation.c:692-793.  out[S*L][H*64].  flags:
   VH_ATT_OUT_BF16 writes out as bf16 (round to nearest even); VH_ATT_BF16
   takes qkv as bf16 and runs the bf16-MFMA kernel (q, k, v and the
   probabilities as bf16 operands, fp32 softmax statistics); VH_ATT_SPLIT
   (fp32 qkv, length > 64) runs the products in fp32 accuracy as exact
   three-piece bf16 splits on the bf16 matrix cores; VH_ATT_H2 (fp32 qkv,
   any length) runs them in fp32 accuracy as two-piece fp16 splits of
   power-of-two-scaled operands, the scales from max|qkv| computed on the
   device (the default fp32 path's attention on both axes, which takes its
   bound from the projection's weights instead); with VH_ATT_H2,
   VH_ATT_OUT_H2 writes out as h2 rows (vh_rmsnorm_h2's layout) scaled from
   that same bound, max|qkv| -- the A operand of a vh_gemm_h2 with
   VH_H2_A_ROWS and a_bound = max|qkv|, as the model's out projection takes
   it (vh_attention_noalloc does not take it). */
#define VH_ATT_OUT_BF16 1
#define VH_ATT_BF16 2
#define VH_ATT_SPLIT 4
#define VH_ATT_H2 8
#define VH_ATT_OUT_H2 16
int vh_attention(vh_context *ctx, int sequences, int length, int heads, const void *qkv, void *out,
                 int apply_rotary, int flags);
/* vh_attention without any device allocation, for callers that cannot
   allocate (code under HIP graph capture, tight serving loops, harnesses that
   forbid hipMalloc).  No counterpart in the reference.  Same arguments,
   kernels and results (bit for bit) as vh_attention; its scratch -- the
   rotary table, the operand bound and its absmax partials -- lives in one
   fixed device array per GPU (1.05 MB, held until the process ends), so
   length is at most VH_NOALLOC_MAX_LENGTH (a longer one fails with an
   error).  The rotary table is written there once, by vh_create; with
   VH_ATT_H2 the bound is computed into the array and the kernels themselves
   choose, on the device, between the two-piece products and those without
   piece scales (vh_attention reads the bound back to choose), so the call
   issues kernels only: no copy, no synchronisation, no allocation, and it
   can be captured in a HIP graph and replayed.  Every call on a GPU shares
   that array: calls that overlap on one GPU (other threads, or other
   streams before this one's work has finished) race. */
#define VH_NOALLOC_MAX_LENGTH 4096
int vh_attention_noalloc(vh_context *ctx, int sequences, int length, int heads, const void *qkv, void *out,
                         int apply_rotary, int flags);

/* ---- model -------------------------------------------------------------- */
/* Upload a VSCNAT01 pack (native/vocalarc_separation.c:528-589) laid out for
   `dims` from host memory.  Returns NULL on a malformed pack. */
vh_model *vh_model_load(vh_context *ctx, const vh_dims *dims, const void *pack, size_t bytes);
/* Before vh_destroy of its context (which frees the models left). */
void vh_model_free(vh_model *model);
/* Arithmetic of the model's matrix products (every linear of the transformer
   stack, band split and mask estimator):
   VH_PRECISION_FP32 (default, the parity path): fp32 accuracy.  The
     transformer and mask-estimator linears run on fp16 matrix cores by
     two-piece operand splitting (vh_gemm_h2; pieces and operand bounds made
     at load), and so does the attention on both axes (the two-piece
     kernels of VH_ATT_H2, scaled from the fused projection's weight bound;
     a layer whose bound lies outside their scale range runs its attention
     on the kernels without piece scales); the band split runs on the fp32
     MFMA instruction.
   VH_PRECISION_FP32_MFMA: every product on the fp32 MFMA instruction.
   VH_PRECISION_BF16: activations rounded to bf16 as they enter the matrix
     cores, bf16 weight copies made on the first switch, fp32 accumulation,
     normalisation, softmax and DSP (separately reported variant).
   The reference CUDA provider's counterpart is its TF32 switch
   (native/native_gpu_cuda.cu:566-570). */
#define VH_PRECISION_FP32 0
#define VH_PRECISION_BF16 1
#define VH_PRECISION_FP32_MFMA 2
int vh_model_set_precision(vh_model *model, int precision);
/* One axial transformer (native/vocalarc_separation.c:836-873) in place on
   device x[S][L][dim]; axis 0 = time weights, 1 = band weights. */
int vh_transformer(vh_context *ctx, vh_model *model, int layer, int axis, float *x, int sequences, int length);
/* Spectrum layouts (float (re, im) pairs): VH_SPEC_REFERENCE is the
   reference's source/mask[F][C][T][2] (native/vocalarc_separation.c:1058,
   1336); VH_SPEC_FRAME_MAJOR is [C][T][F][2], every frame's bins contiguous
   (what the device pipeline uses internally). */
#define VH_SPEC_REFERENCE 0
#define VH_SPEC_FRAME_MAJOR 1
/* STFT (native/vocalarc_separation.c:1044-1072): device audio[C][length] ->
   device source (layout), T = length/hop + 1. */
int vh_stft(vh_context *ctx, vh_model *model, const float *audio, int length, float *source, int layout);
/* Complex mask multiply + iSTFT + overlap-add
   (native/vocalarc_separation.c:1084-1136) -> device audio[C][length]. */
int vh_istft(vh_context *ctx, vh_model *model, const float *source, const float *mask, int length, float *audio,
             int layout);
/* Band split (native/vocalarc_separation.c:887-926): device source (layout)
   -> device time_sequences[B][T][dim]. */
int vh_band_split(vh_context *ctx, vh_model *model, const float *source, int frames, float *time_sequences,
                  int layout);
/* Mask estimator (native/vocalarc_separation.c:1316-1340, all bands) on
   final-normed device features[T][B][dim] -> device mask (layout). */
int vh_mask_estimate(vh_context *ctx, vh_model *model, const float *features, int frames, float *mask, int layout);
/* Whole forward of one window (native/vocalarc_separation.c:1342-1445):
   device audio[C][length] -> device vocals[C][length]; when `instrumental`
   is not NULL it receives audio - vocals (native/vocalarc_separation.c:1589-1591). */
int vh_forward(vh_context *ctx, vh_model *model, const float *audio, int length, float *vocals,
               float *instrumental);
/* Chunked separation of a long device audio[C][length]: windows of `chunk`
   samples every `step` samples (zero-padded at the end), `batch` windows per
   device pass, linear cross-fade over the overlap normalised by the summed
   fade weights; `instrumental` (nullable) as for vh_forward.  No reference counterpart (the reference host runs the whole
   file as one window, native/vocalarc_separation.c:1344). */
int vh_separate(vh_context *ctx, vh_model *model, const float *audio, int length, int chunk, int step, int batch,
                float *vocals, float *instrumental);

/* ---- measurement --------------------------------------------------------- */
/* Per-kernel-class timing with HIP events recorded on the context stream
   around each launch of the selected classes: a comma-separated list of
   class names (e.g. "gemm_ff1,attention_long"), "*" for all, NULL or ""
   to stop timing. */
int vh_timing_enable(vh_context *ctx, const char *classes);
int vh_timing_reset(vh_context *ctx);
/* Total milliseconds and launch count of a kernel class since the last reset
   (after vh_synchronize).  Returns 0 if the class never ran. */
int vh_timing_get(vh_context *ctx, const char *name, double *total_ms, int64_t *count);

#ifdef __cplusplus
}
#endif

#endif
