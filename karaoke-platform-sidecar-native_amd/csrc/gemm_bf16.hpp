// bf16-MFMA variant of the token-wise linear: C[M][N] (op)= A[M][K] * B[N][K]^T
// with A read as fp32 and rounded to bf16 while it is staged into LDS, B a
// bf16 copy of the weight matrix, fp32 accumulation and the same fused fp32
// epilogues as the fp32 GEMM.  This is the separately reported reduced
// precision path; the fp32 GEMM (gemm.hpp) is the parity path.
//
// Tiling: 256x128 block tile, 4 wavefronts in a 2x2 grid, each owning a
// 128x64 sub-tile = 4x2 v_mfma_f32_32x32x16_bf16 accumulators.  K is staged in
// chunks of 32 (two MFMA steps); per step a wave reads 4 A and 2 B operands of
// 8 bf16 (ds_read_b128) for 8 MFMAs.  LDS rows are padded to 40 bf16 (80 B)
// so the 16 rows of each read phase fall on disjoint banks.
#pragma once

#include "common.hpp"

namespace vh {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

struct GemmDescBF16 {
    const float *A;     // fp32 activations
    const bf16 *B;      // bf16 weights [N][K]
    const float *bias;  // fp32, may be null
    float *C;
    int M, N, K;
    int lda, ldb, ldc;
};

constexpr int GB_BM = 256, GB_BN = 128, GB_BK = 32, GB_PITCH = GB_BK + 8;
constexpr int GB_THREADS = 256;
constexpr int GB_MAX_BATCH = 64;
struct GemmBatchBF16 {
    GemmDescBF16 d[GB_MAX_BATCH];
};

VH_DEVICE bf16x4 to_bf16x4(floatx4 v) {
    bf16x4 r;
    r[0] = (bf16)v[0];
    r[1] = (bf16)v[1];
    r[2] = (bf16)v[2];
    r[3] = (bf16)v[3];
    return r;
}

template <int EPI>
__device__ __forceinline__ void gemm_bf16_body(const GemmDescBF16 &d, int tile) {
    __shared__ __attribute__((aligned(16))) bf16 As[2][GB_BM][GB_PITCH];
    __shared__ __attribute__((aligned(16))) bf16 Bs[2][GB_BN][GB_PITCH];

    const int tiles_n = (d.N + GB_BN - 1) / GB_BN;
    const int tiles_m = (d.M + GB_BM - 1) / GB_BM;
    if (tile >= tiles_m * tiles_n) return;
    // column-fastest order within groups of row tiles (see gemm.hpp)
    const int gsz = (size_t)d.N * d.K * sizeof(bf16) <= (3u << 20) ? 1 : 8;
    const int group = tile / (gsz * tiles_n);
    const int in_group = tile % (gsz * tiles_n);
    const int group_rows = min(gsz, tiles_m - group * gsz);
    const int m0 = (group * gsz + in_group % group_rows) * GB_BM;
    const int n0 = (in_group / group_rows) * GB_BN;

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int li = lane & 31, lh = lane >> 5;

    // A: 256 rows x 8 float4 per chunk -> 8 float4 per thread (row tid/8 + 32q, quad tid%8)
    // B: 128 rows x 4 x 16 B (8 bf16) per chunk -> 2 per thread (row tid/4 + 64q, part tid%4)
    const int a_row = tid >> 3, a_c4 = tid & 7;
    const int b_row = tid >> 2, b_c8 = tid & 3;
    floatx4 ra[8];
    bf16x8 rb[2];
    auto load = [&](int k0) {
        const int ka = k0 + 4 * a_c4;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int gm = min(m0 + a_row + 32 * q, d.M - 1);
            ra[q] = ka < d.K ? ld4(d.A + (size_t)gm * d.lda + ka) : floatx4{0.f, 0.f, 0.f, 0.f};
        }
        const int kb = k0 + 8 * b_c8;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int gn = min(n0 + b_row + 64 * q, d.N - 1);
            if (kb < d.K) {
                rb[q] = *reinterpret_cast<const bf16x8 *>(d.B + (size_t)gn * d.ldb + kb);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) rb[q][e] = (bf16)0.0f;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int q = 0; q < 8; q++)
            *reinterpret_cast<bf16x4 *>(&As[buf][a_row + 32 * q][4 * a_c4]) = to_bf16x4(ra[q]);
#pragma unroll
        for (int q = 0; q < 2; q++) *reinterpret_cast<bf16x8 *>(&Bs[buf][b_row + 64 * q][8 * b_c8]) = rb[q];
    };

    floatx16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int nk = (d.K + GB_BK - 1) / GB_BK;
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * GB_BK);
#pragma unroll
        for (int st = 0; st < GB_BK / 16; st++) {
            bf16x8 a[4], b[2];
#pragma unroll
            for (int i = 0; i < 4; i++)
                a[i] = *reinterpret_cast<const bf16x8 *>(&As[buf][wm * 128 + 32 * i + li][16 * st + 8 * lh]);
#pragma unroll
            for (int j = 0; j < 2; j++)
                b[j] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][wn * 64 + 32 * j + li][16 * st + 8 * lh]);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    // Accumulator layout as for the fp32 32x32 MFMA: lane (li, lh), register r
    // holds row 8*(r/4) + 4*lh + r%4, column li.
    if constexpr (EPI == EPI_GEGLU) {
        const int nv = n0 + wn * 64 + li;
        const int ng = nv + 32;
        const int oc = (n0 + wn * 64) / 2 + li;
        if (ng < d.N) {
            const float bv = d.bias ? d.bias[nv] : 0.0f;
            const float bg = d.bias ? d.bias[ng] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (row < d.M) d.C[(size_t)row * d.ldc + oc] = (acc[i][0][r] + bv) * gelu_dev(acc[i][1][r] + bg);
                }
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int col = n0 + wn * 64 + j * 32 + li;
            if (col >= d.N) continue;
            const float bc = d.bias ? d.bias[col] : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int row = m0 + wm * 128 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (row >= d.M) continue;
                    const float v = acc[i][j][r] + bc;
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
__global__ __launch_bounds__(GB_THREADS, 2) void gemm_bf16_kernel(GemmDescBF16 d) {
    gemm_bf16_body<EPI>(d, xcd_swizzle((int)blockIdx.x, (int)gridDim.x));
}

template <int EPI>
__global__ __launch_bounds__(GB_THREADS, 2) void gemm_bf16_batched_kernel(GemmBatchBF16 b) {
    gemm_bf16_body<EPI>(b.d[blockIdx.z], (int)blockIdx.x);
}

// fp32 [rows][cols] -> bf16 [rows][ld] (weights at upload; padding untouched)
static __global__ __launch_bounds__(256) void to_bf16_kernel(const float *__restrict__ src, bf16 *__restrict__ dst,
                                                             int64_t rows, int cols, int ld) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= rows * cols) return;
    const int64_t r = e / cols;
    const int c = (int)(e - r * cols);
    dst[r * ld + c] = (bf16)src[e];
}

}  // namespace vh
