// fp32 GEMM on CDNA4 matrix cores: C[M][N] (op)= A[M][K] * B[N][K]^T.
//
// A is the activation matrix (row-major, lda), B the weight matrix in
// [out][in] row-major order (ldb).  This is the token-wise linear of the
// reference (native/vocalarc_separation.c:631-636; cuBLAS at
// native/native_gpu_cuda.cu:540-552) with the bias and the following
// elementwise op fused into the store.
//
// Tiling: 128x128 block tile, 4 wavefronts in a 2x2 grid, each owning a 64x64
// sub-tile = 2x2 v_mfma_f32_32x32x2f32 accumulators (64 acc registers).  K is
// staged through LDS in chunks of 16 with one register-staged prefetch
// (double-buffered LDS, one barrier per chunk); 40 KB of LDS per workgroup
// lets four workgroups share a CU, so global-load latency of one is hidden
// behind the matrix work of the others.  Operand reads are ds_read_b128:
// lane (i, h) of a 32x32x2 MFMA feeds element k = 8g + 4h + r at step (g, r),
// so one 16-byte read per operand serves four MFMAs.  The LDS row pitch of 20
// floats puts the 16 rows of each read phase on disjoint banks.
#pragma once

#include "common.hpp"

namespace vh {

struct GemmDesc {
    const float *A;
    const float *B;
    const float *bias;  // may be null
    float *C;
    int M, N, K;
    int lda, ldb, ldc;
};

constexpr int GEMM_BM = 128, GEMM_BN = 128, GEMM_BK = 16, GEMM_PITCH = GEMM_BK + 4;
constexpr int GEMM_THREADS = 256;
static_assert(GEMM_BM == 128 && GEMM_BN == 128 && GEMM_THREADS == 256, "the product tile is 2 x 2 waves");
constexpr int GEMM_GROUP_M = 16;
constexpr size_t GEMM_L2_RESIDENT_BYTES = 3u << 20;
// Descriptors of a ragged batch travel in the kernel arguments (<= 4 KiB).
constexpr int GEMM_MAX_BATCH = 64;
struct GemmBatch {
    GemmDesc d[GEMM_MAX_BATCH];
};

// WM x WN wavefronts of 64x64 each (block tile 64*WM x 64*WN); the product
// uses 2 x 2 (GEMM_BM x GEMM_BN).
template <int EPI, int WM = 2, int WN = 2>
__device__ __forceinline__ void gemm_f32_body(const GemmDesc &d, int tile) {
    constexpr int GEMM_BM = 64 * WM, GEMM_BN = 64 * WN, GEMM_THREADS = 64 * WM * WN;
    __shared__ __attribute__((aligned(16))) float As[2][GEMM_BM][GEMM_PITCH];
    __shared__ __attribute__((aligned(16))) float Bs[2][GEMM_BN][GEMM_PITCH];

    const int tiles_n = (d.N + GEMM_BN - 1) / GEMM_BN;
    const int tiles_m = (d.M + GEMM_BM - 1) / GEMM_BM;
    if (tile >= tiles_m * tiles_n) return;
    // Grouped order: GEMM_GROUP_M row tiles x all column tiles, row fastest.
    // Consecutive workgroups share one weight tile (read once into L2 for
    // GEMM_GROUP_M of them) while the group's activation rows stay resident;
    // with column-fastest order a K=384 fp32 weight matrix wider than ~2000
    // rows no longer fits an XCD's 4 MB L2 and is re-fetched per row tile.
    // A weight matrix that fits comfortably in L2 is kept resident by plain
    // column-fastest order (group of one row tile), which reads each
    // activation row tile exactly once.
    const int gsz = (size_t)d.N * d.K * sizeof(float) <= GEMM_L2_RESIDENT_BYTES ? 1 : GEMM_GROUP_M;
    const int group = tile / (gsz * tiles_n);
    const int in_group = tile % (gsz * tiles_n);
    const int group_rows = min(gsz, tiles_m - group * gsz);
    const int m0 = (group * gsz + in_group % group_rows) * GEMM_BM;
    const int n0 = (in_group / group_rows) * GEMM_BN;

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 31, lh = lane >> 5;

    // global -> register staging: a k-chunk row holds GEMM_BK/4 float4s;
    // thread covers rows ld_row + RSTEP*q and float4 ld_c4 of the chunk.
    constexpr int C4 = GEMM_BK / 4;                  // float4s per tile row
    constexpr int RSTEP = GEMM_THREADS / C4;         // rows covered per pass
    constexpr int NQA = GEMM_BM / RSTEP, NQB = GEMM_BN / RSTEP;  // passes
    static_assert(GEMM_BM % RSTEP == 0 && GEMM_BN % RSTEP == 0, "staging must tile the block");
    const int ld_row = tid / C4, ld_c4 = tid % C4;
    floatx4 ra[NQA], rb[NQB];
    auto load = [&](int k0) {
        const int kk = k0 + 4 * ld_c4;
        const bool kin = kk < d.K;
#pragma unroll
        for (int q = 0; q < NQA; q++) {
            int gm = min(m0 + ld_row + RSTEP * q, d.M - 1);
            ra[q] = kin ? ld4(d.A + (size_t)gm * d.lda + kk) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int q = 0; q < NQB; q++) {
            int gn = min(n0 + ld_row + RSTEP * q, d.N - 1);
            rb[q] = kin ? ld4(d.B + (size_t)gn * d.ldb + kk) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < NQA; q++) st4(&As[buf][ld_row + RSTEP * q][4 * ld_c4], ra[q]);
#pragma unroll
        for (int q = 0; q < NQB; q++) st4(&Bs[buf][ld_row + RSTEP * q][4 * ld_c4], rb[q]);
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int nk = (d.K + GEMM_BK - 1) / GEMM_BK;
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * GEMM_BK);
#pragma unroll
        for (int g = 0; g < GEMM_BK / 8; g++) {
            floatx4 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = ld4(&As[buf][wm * 64 + i * 32 + li][8 * g + 4 * lh]);
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = ld4(&Bs[buf][wn * 64 + j * 32 + li][8 * g + 4 * lh]);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < 2; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][r], b[j][r], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    // Accumulator layout of a 32x32 MFMA tile: lane (li, lh), register r holds
    // row 8*(r/4) + 4*lh + r%4, column li.
    if constexpr (EPI == EPI_GEGLU) {
        const int nv = n0 + wn * 64 + li;  // value column in the interleaved weight
        const int ng = nv + 32;            // matching gate column
        const int oc = (n0 + wn * 64) / 2 + li;
        if (ng < d.N) {
            const float bv = d.bias ? d.bias[nv] : 0.0f;
            const float bg = d.bias ? d.bias[ng] : 0.0f;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (row < d.M) {
                        float v = acc[i][0][r] + bv;
                        float gt = acc[i][1][r] + bg;
                        d.C[(size_t)row * d.ldc + oc] = v * gelu_dev(gt);
                    }
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 64 + j * 32 + li;
            if (col >= d.N) continue;
            const float bc = d.bias ? d.bias[col] : 0.0f;
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    int row = m0 + wm * 64 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (row >= d.M) continue;
                    float v = acc[i][j][r] + bc;
                    float *p = d.C + (size_t)row * d.ldc + col;
                    if constexpr (EPI == EPI_STORE) *p = v;
                    else if constexpr (EPI == EPI_GELU) *p = gelu_dev(v);
                    else if constexpr (EPI == EPI_TANH) *p = tanhf(v);
                    else if constexpr (EPI == EPI_RESIDUAL) *p = *p + v;
                }
        }
    }
}

template <int EPI>
__global__ __launch_bounds__(GEMM_THREADS, 4) void gemm_f32_kernel(GemmDesc d) {
    gemm_f32_body<EPI>(d, xcd_swizzle((int)blockIdx.x, (int)gridDim.x));
}

template <int EPI>
__global__ __launch_bounds__(GEMM_THREADS, 4) void gemm_f32_batched_kernel(GemmBatch b) {
    gemm_f32_body<EPI>(b.d[blockIdx.z], (int)blockIdx.x);
}

}  // namespace vh
