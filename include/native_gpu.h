/*
 * native_gpu.h -- the drop-in boundary: the GPU-provider C-ABI that the
 * unchanged VocalArc C11 host (native/vocalarc_separation.c) calls.
 *
 * Every declaration below is the interface of native/native_gpu.h in the
 * reference, kept binary-compatible (same names, argument order, struct
 * layouts) so that the HIP provider links into the host in place of
 * native/native_gpu_cuda.cu.  Line citations are into the reference's
 * native/native_gpu.h (h:) and native/vocalarc_separation.c (c:).
 *
 * Return convention (h:12-13, h:43-45): 1 = handled on the device, 0 = the
 * host must compute the step itself on the CPU.  A provider that hits a
 * runtime error reports it on stderr and disables itself for the rest of the
 * process, so every later call returns 0.
 */
#ifndef VOCALARC_NATIVE_GPU_H
#define VOCALARC_NATIVE_GPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct native_gpu native_gpu; /* h:10 */

/* h:14. Called once at host start-up (c:1522).  NULL when no usable GPU is
   present or VOCALARC_GPU is "off"/"cpu". */
native_gpu *native_gpu_create(void);
/* h:15. NULL-safe; releases every device allocation (c:1607). */
void native_gpu_destroy(native_gpu *gpu);

/* h:17-19. output[rows][out] = input[rows][in] * W^T (+ bias) with W in the
   host's packed layout (c:428-457).  Host pointers.  Called for every
   host-side linear (c:633); returns 0 below a minimum amount of work. */
int native_gpu_matmul(native_gpu *gpu, int64_t rows, int in, int out,
                      const float *input, const float *packed_weight,
                      const float *bias, float *output);

/* h:21-22. Printed raw inside the host's JSON (c:1516-1517): no quotes or
   backslashes.  "native-cpu" / "none" when NULL or disabled. */
const char *native_gpu_backend(const native_gpu *gpu);
const char *native_gpu_device(const native_gpu *gpu);

/* h:27-28. Whether the resident full-batch path is available, and whether
   `frames` frames fit the device (c:1358, c:1575). */
int native_gpu_uses_full_batches(const native_gpu *gpu);
int native_gpu_can_use_full_batches(const native_gpu *gpu, int frames);

/* h:30-41. Host pointers into the model pack, packed layout. */
typedef struct {
    const float *gamma;
    const float *qkv;
    const float *gate_weight;
    const float *gate_bias;
    const float *out_weight;
    const float *ff_gamma;
    const float *ff1_weight;
    const float *ff1_bias;
    const float *ff2_weight;
    const float *ff2_bias;
} native_gpu_transformer_weights;

/* h:46-49. One axial transformer block on host data[S][L][dim], updated in
   place (c:846).  The four scratch pointers are the host's and may be
   ignored. */
int native_gpu_transformer(native_gpu *gpu, int sequences, int length,
                           float *data, float *normed, float *qkv,
                           float *attention_output, float *gates,
                           const native_gpu_transformer_weights *weights);

/* h:53-58. Resident graph: begin copies data[S][L][dim] in (c:1359); each
   transformer runs on the resident tensor viewed as [S][L] (c:1376-1379);
   transpose turns [S][L] into [L][S]; end copies the current tensor out and
   ends residency (c:1399). */
int native_gpu_resident_begin(native_gpu *gpu, int sequences, int length,
                              const float *data);
int native_gpu_resident_transformer(native_gpu *gpu, int sequences, int length,
                                    const native_gpu_transformer_weights *weights);
int native_gpu_resident_transpose(native_gpu *gpu, int sequences, int length);
int native_gpu_resident_end(native_gpu *gpu, float *data);

/* h:60-67. One band of the mask estimator (c:1385-1395). */
typedef struct {
    const float *first_weight;
    const float *first_bias;
    const float *second_weight;
    const float *second_bias;
    int input_dim;
    int first_frequency;
} native_gpu_mask_band;

/* h:71-73. Final RMSNorm of the resident [frames][bands][dim] tensor, the
   per-band mask MLP + GLU, scattered into the host mask[F][C][frames][2]
   (c:1396-1397).  Ends residency. */
int native_gpu_resident_mask(native_gpu *gpu, int frames, const float *final_gamma,
                             float *mask, const native_gpu_mask_band *bands,
                             int band_count);

#ifdef __cplusplus
}
#endif

#endif
