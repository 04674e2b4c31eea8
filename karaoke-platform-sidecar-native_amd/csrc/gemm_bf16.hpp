// bf16-MFMA variant of the token-wise linear: C[M][N] (op)= A[M][K] * B[N][K]^T
// with bf16 matrix-core operands, fp32 accumulation and the same fused fp32
// epilogues as the fp32 GEMM.  This is the separately reported reduced
// precision path; the fp32 GEMM (gemm.hpp) is the parity path.
//
// A is either fp32 (rounded to bf16, nearest-even, as it is staged into LDS)
// or already bf16 (written that way by its producer: the normalisation, the
// attention store or a preceding GEMM's epilogue).  The output is fp32 or
// bf16 (the residual epilogue is always fp32).
//
// Tiling (template parameters): WM x WN wavefronts, each owning FM x FN
// 32x32 accumulators of v_mfma_f32_32x32x16_bf16, i.e. a block tile of
// (32*WM*FM) x (32*WN*FN).  K is staged in chunks of BK (BK/16 MFMA steps);
// per step a wave reads FM A and FN B operands of 8 bf16 (ds_read_b128) for
// FM*FN MFMAs.  LDS rows are padded by 8 bf16 so the 16 rows of each read
// phase fall on disjoint banks.  Staging is register-prefetched one chunk
// ahead with double-buffered LDS.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace vh {

struct GemmDescBF16 {
    const void *A;      // fp32 or bf16 activations [M][lda]
    const bf16 *B;      // bf16 weights [N][ldb]
    const float *bias;  // fp32, may be null
    void *C;            // fp32 or bf16 [M][ldc]
    int M, N, K;
    int lda, ldb, ldc;
};

constexpr int GB_MAX_BATCH = 64;
struct GemmBatchBF16 {
    GemmDescBF16 d[GB_MAX_BATCH];
};

// One output element; fp32 outputs are written non-temporally (no kernel
// reads them back, and they would only displace the operands' lines in L2:
// -1.5 to -3% on the fp16 two-piece GEMMs).
template <typename T>
VH_DEVICE void store_out(T *p, float v) {
    if constexpr (std::is_same<T, float>::value) __builtin_nontemporal_store(v, p);
    else *p = (bf16)v;
}
// The same through a global-address-space pointer (the saddr-form stores
// of gemm_bf16_epilogue).
template <typename T>
VH_DEVICE void store_out(__attribute__((address_space(1))) T *p, float v) {
    if constexpr (std::is_same<T, float>::value) __builtin_nontemporal_store(v, p);
    else *p = (bf16)v;
}

// Fused epilogue of a wave's FM x FN accumulators whose tile starts at
// (row0, col0).  Accumulator layout as for the fp32 32x32 MFMA: lane (li,
// lh), register r holds row 8*(r/4) + 4*lh + r%4, column li.  Tiles whose
// rows all lie inside M (all but the last row of tiles) take a path without
// per-element row checks, so the residual epilogue issues its 16 loads of C
// together instead of one load-wait-store per element.  mx_out (residual
// epilogue only; null for none): raised to the largest |C| this lane wrote.
// bpre (null for none): the bias of the lane's column in each of the FN
// column tiles (0 past N), loaded by the caller before its K loop so that
// the load's latency is not spent here.  rs (null for none): a scale per
// accumulator row (rs[16 i + r] for register r of acc[i][.]), applied with
// the bias in one fused multiply-add (the row norm of the fp16 two-piece
// GEMM).
template <int EPI, typename TC, int FM, int FN>
VH_DEVICE void gemm_bf16_epilogue(const GemmDescBF16 &d, const floatx16 (&acc)[FM][FN], int row0, int col0, int li,
                                  int lh, float *mx_out = nullptr, const float *bpre = nullptr,
                                  const float *rs = nullptr) {
    TC *C = static_cast<TC *>(d.C);
    auto bias_of = [&](int j, int col) { return bpre ? bpre[j] : (d.bias ? d.bias[col] : 0.0f); };
    auto pre = [&](int i, int j, int r, float b) { return rs ? fmaf(acc[i][j][r], rs[16 * i + r], b) : acc[i][j][r] + b; };
    const bool rows_full = row0 + 32 * FM <= d.M;
    auto row_of = [&](int i, int r) { return row0 + i * 32 + 8 * (r >> 2) + 4 * lh + (r & 3); };
    // Full tiles address element (i, r) as a row pointer that is the same for
    // the whole wave (row0 is wave-uniform in every caller, so it lives in
    // SGPRs) plus the lane's 32-bit byte offset: the loads and stores take
    // the saddr form, with no 64-bit address arithmetic per element.
    // (ldc <= 2^21 by the callers' checks, so row offsets within a wave's
    // 32 * FM rows fit 32 bits)
    typedef __attribute__((address_space(1))) char gchar;
    typedef __attribute__((address_space(1))) TC gTC;
    const uint32_t pitch = (uint32_t)d.ldc * (uint32_t)sizeof(TC);
    const uint32_t lh_off = (uint32_t)(4 * lh) * pitch;
    const gchar *const rbase = (const gchar *)(reinterpret_cast<char *>(C) + (size_t)row0 * (size_t)pitch);
    auto at = [&](int i, int r, uint32_t off) {
        const gchar *rp = rbase + (uint32_t)(i * 32 + 8 * (r >> 2) + (r & 3)) * pitch;
        asm("" : "+s"(rp));  // opaque: the lane offset is not folded into it
        return (gTC *)(rp + off);
    };
    if constexpr (EPI == EPI_GEGLU) {
        // accumulator pair (2p, 2p+1) = value and gate columns of one 64-wide group
#pragma unroll
        for (int p = 0; p < FN / 2; p++) {
            const int nv = col0 + 64 * p + li;
            const int ng = nv + 32;
            const int oc = (col0 + 64 * p) / 2 + li;
            if (ng >= d.N) continue;
            const float bv = bias_of(2 * p, nv);
            const float bg = bias_of(2 * p + 1, ng);
            const uint32_t off = lh_off + (uint32_t)oc * (uint32_t)sizeof(TC);
#pragma unroll
            for (int i = 0; i < FM; i++) {
                auto value = [&](int r) { return pre(i, 2 * p, r, bv) * gelu_dev(pre(i, 2 * p + 1, r, bg)); };
                if (rows_full) {
#pragma unroll
                    for (int r = 0; r < 16; r++) store_out(at(i, r, off), value(r));
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = row_of(i, r);
                        if (row < d.M) store_out(C + (size_t)row * d.ldc + oc, value(r));
                    }
                }
            }
        }
    } else {
        static_assert(EPI != EPI_RESIDUAL || std::is_same<TC, float>::value, "residual output is fp32");
        float mx = 0.0f;  // largest |C| written (residual epilogue)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            const int col = col0 + j * 32 + li;
            if (col >= d.N) continue;
            const float bc = bias_of(j, col);
            const uint32_t off = lh_off + (uint32_t)col * (uint32_t)sizeof(TC);
#pragma unroll
            for (int i = 0; i < FM; i++) {
                auto value = [&](int r) {
                    const float v = pre(i, j, r, bc);
                    if constexpr (EPI == EPI_GELU) return gelu_dev(v);
                    else if constexpr (EPI == EPI_TANH) return tanhf(v);
                    else return v;
                };
                if (rows_full) {
                    if constexpr (EPI == EPI_RESIDUAL) {
                        float old[16];
#pragma unroll
                        for (int r = 0; r < 16; r++) old[r] = *at(i, r, off);
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const float v = old[r] + value(r);
                            mx = fmaxf(mx, fabsf(v));
                            store_out(at(i, r, off), v);
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 16; r++) store_out(at(i, r, off), value(r));
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = row_of(i, r);
                        if (row >= d.M) continue;
                        TC *p = C + (size_t)row * d.ldc + col;
                        const float v = EPI == EPI_RESIDUAL ? *p + value(r) : value(r);
                        if constexpr (EPI == EPI_RESIDUAL) mx = fmaxf(mx, fabsf(v));
                        store_out(p, v);
                    }
                }
            }
        }
        if constexpr (EPI == EPI_RESIDUAL) {
            if (mx_out) *mx_out = fmaxf(*mx_out, mx);
        }
    }
}

template <int WM, int WN, int FM, int FN>
struct BF16Tile {
    static constexpr int BM = 32 * WM * FM, BN = 32 * WN * FN, THREADS = 64 * WM * WN;
};

template <int EPI, typename TA, typename TC, int BK, int WM, int WN, int FM, int FN>
__device__ __forceinline__ void gemm_bf16_body(const GemmDescBF16 &d, int tile) {
    constexpr int GB_BM = BF16Tile<WM, WN, FM, FN>::BM, GB_BN = BF16Tile<WM, WN, FM, FN>::BN;
    constexpr int GB_THREADS = BF16Tile<WM, WN, FM, FN>::THREADS;
    static_assert(FN % 2 == 0 || EPI != EPI_GEGLU, "GELU-GLU needs value/gate column pairs per wave");
    constexpr int PITCH = BK + 8;
    constexpr bool A32 = std::is_same<TA, float>::value;
    constexpr int A_VEC = A32 ? 4 : 8;                      // elements per 16-byte load
    constexpr int A_CPR = BK / A_VEC;                       // chunks per row
    constexpr int A_RPP = GB_THREADS / A_CPR;               // rows per pass
    constexpr int A_PASSES = GB_BM / A_RPP;
    constexpr int B_CPR = BK / 8;
    constexpr int B_RPP = GB_THREADS / B_CPR;
    constexpr int B_PASSES = GB_BN / B_RPP;
    static_assert(GB_BM % A_RPP == 0 && GB_BN % B_RPP == 0, "staging must tile the block");
    __shared__ __attribute__((aligned(16))) bf16 As[2][GB_BM][PITCH];
    __shared__ __attribute__((aligned(16))) bf16 Bs[2][GB_BN][PITCH];

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
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave / WN, wn = wave % WN;
    const int li = lane & 31, lh = lane >> 5;

    const int a_row = tid / A_CPR, a_c = tid % A_CPR;
    const int b_row = tid / B_CPR, b_c = tid % B_CPR;
    const TA *Ag = static_cast<const TA *>(d.A);
    floatx4 ra32[A32 ? A_PASSES : 1];
    bf16x8 ra16[A32 ? 1 : A_PASSES];
    bf16x8 rb[B_PASSES];
    auto load = [&](int k0) {
        const int ka = k0 + A_VEC * a_c;
#pragma unroll
        for (int q = 0; q < A_PASSES; q++) {
            const int gm = min(m0 + a_row + A_RPP * q, d.M - 1);
            if constexpr (A32) {
                ra32[q] = ka < d.K ? ld4(reinterpret_cast<const float *>(Ag) + (size_t)gm * d.lda + ka)
                                   : floatx4{0.f, 0.f, 0.f, 0.f};
            } else {
                if (ka < d.K) {
                    ra16[q] = *reinterpret_cast<const bf16x8 *>(Ag + (size_t)gm * d.lda + ka);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; e++) ra16[q][e] = (bf16)0.0f;
                }
            }
        }
        const int kb = k0 + 8 * b_c;
#pragma unroll
        for (int q = 0; q < B_PASSES; q++) {
            const int gn = min(n0 + b_row + B_RPP * q, d.N - 1);
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
        for (int q = 0; q < A_PASSES; q++) {
            if constexpr (A32)
                *reinterpret_cast<bf16x4 *>(&As[buf][a_row + A_RPP * q][4 * a_c]) = to_bf16x4(ra32[q]);
            else
                *reinterpret_cast<bf16x8 *>(&As[buf][a_row + A_RPP * q][8 * a_c]) = ra16[q];
        }
#pragma unroll
        for (int q = 0; q < B_PASSES; q++) *reinterpret_cast<bf16x8 *>(&Bs[buf][b_row + B_RPP * q][8 * b_c]) = rb[q];
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    const int nk = (d.K + BK - 1) / BK;
    load(0);
    store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load((kt + 1) * BK);
#pragma unroll
        for (int st = 0; st < BK / 16; st++) {
            bf16x8 a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                a[i] = *reinterpret_cast<const bf16x8 *>(&As[buf][wm * 32 * FM + 32 * i + li][16 * st + 8 * lh]);
#pragma unroll
            for (int j = 0; j < FN; j++)
                b[j] = *reinterpret_cast<const bf16x8 *>(&Bs[buf][wn * 32 * FN + 32 * j + li][16 * st + 8 * lh]);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
    }

    gemm_bf16_epilogue<EPI, TC, FM, FN>(d, acc, m0 + wm * 32 * FM, n0 + wn * 32 * FN, li, lh);
}

template <int EPI, typename TA, typename TC, int BK, int WM, int WN, int FM, int FN, int OCC>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_bf16_kernel(GemmDescBF16 d) {
    gemm_bf16_body<EPI, TA, TC, BK, WM, WN, FM, FN>(d, xcd_swizzle((int)blockIdx.x, (int)gridDim.x));
}

template <int EPI, typename TA, typename TC, int BK, int WM, int WN, int FM, int FN, int OCC>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_bf16_batched_kernel(GemmBatchBF16 b) {
    gemm_bf16_body<EPI, TA, TC, BK, WM, WN, FM, FN>(b.d[blockIdx.z], (int)blockIdx.x);
}

// The bias of columns c .. c+3 (c a multiple of 4), clamped to N (columns
// past N are never stored): one 16-byte load where all four lie inside N and
// the bias is 16-byte aligned.
VH_DEVICE floatx4 bias_quad(const float *bias, int c, int N) {
    floatx4 b = {0.f, 0.f, 0.f, 0.f};
    if (!bias) return b;
    if (c + 4 <= N && !((uintptr_t)bias & 15)) return ld4(bias + c);
#pragma unroll
    for (int e = 0; e < 4; e++) b[e] = bias[min(c + e, N - 1)];
    return b;
}

// The eight bias quads a lane of gemm_bf16_epilogue_staged applies, for the
// wave's block starting at column col0: GELU-GLU value quads q (columns
// col0 + 8q + 4lh ..) in bq[q] and their gates 32 further in bq[4 + q];
// otherwise column tile j's quads in bq[4j + q].  Loaded before the K loop.
template <int EPI>
VH_DEVICE void bias_quads_staged(const GemmDescBF16 &d, int col0, int lh, floatx4 (&bq)[8]) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if constexpr (EPI == EPI_GEGLU) {
            bq[q] = bias_quad(d.bias, col0 + 8 * q + 4 * lh, d.N);
            bq[4 + q] = bias_quad(d.bias, col0 + 8 * q + 4 * lh + 32, d.N);
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++) bq[4 * j + q] = bias_quad(d.bias, col0 + 32 * j + 8 * q + 4 * lh, d.N);
        }
    }
}

// bf16-output epilogue of a wave's 64 x 64 block through LDS, for MFMAs that
// take the B tile as their first operand: the accumulators then hold C
// transposed -- lane (li, lh), register r of acc[i][j] is row 32 i + li,
// column 32 j + 8 (r / 4) + 4 lh + r % 4 of the block -- so each lane has
// four consecutive columns per register quad.  The lane writes each quad,
// finished (bias, activation or GELU-GLU) and rounded, as 8 bytes into the
// wave's own LDS block of 64 rows (`stage`, 64 x (OC + 8) bf16, OC the
// block's output columns), then every lane stores 16 bytes of a row, so a
// store instruction covers whole 64- or 128-byte row segments instead of
// 2-byte scatters (bf16 QKV -7%, FFN up -9% against the per-element store).
template <int EPI>
VH_DEVICE void gemm_bf16_epilogue_staged(const GemmDescBF16 &d, const floatx16 (&acc)[2][2], bf16 *stage, int row0,
                                         int col0, int lane, const floatx4 (&bq)[8]) {
    constexpr int OC = EPI == EPI_GEGLU ? 32 : 64;
    constexpr int PITCH = OC + 8;  // 16-byte aligned rows
    const int li = lane & 31, lh = lane >> 5;
    auto quad = [](const floatx16 &v, int q) { return floatx4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]}; };
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if constexpr (EPI == EPI_GEGLU) {
            // value columns 8q + 4lh .. +3 of the 64-wide group, gates 32 further
            const floatx4 bv = bq[q], bg = bq[4 + q];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const floatx4 v = quad(acc[i][0], q), g = quad(acc[i][1], q);
                floatx4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = (v[e] + bv[e]) * gelu_dev(g[e] + bg[e]);
                *reinterpret_cast<bf16x4 *>(&stage[(32 * i + li) * PITCH + 8 * q + 4 * lh]) = to_bf16x4(o);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int c = 32 * j + 8 * q + 4 * lh;
                const floatx4 b = bq[4 * j + q];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const floatx4 v = quad(acc[i][j], q);
                    floatx4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        o[e] = v[e] + b[e];
                        if constexpr (EPI == EPI_GELU) o[e] = gelu_dev(o[e]);
                        else if constexpr (EPI == EPI_TANH) o[e] = tanhf(o[e]);
                    }
                    *reinterpret_cast<bf16x4 *>(&stage[(32 * i + li) * PITCH + c]) = to_bf16x4(o);
                }
            }
        }
    }
    constexpr int LPR = OC / 8;  // lanes per row, 16 bytes each
    constexpr int RPI = 64 / LPR;  // rows per store instruction
    const int oc0 = EPI == EPI_GEGLU ? col0 / 2 : col0;
    const int ncols = EPI == EPI_GEGLU ? d.N / 2 : d.N;
    bf16 *C = static_cast<bf16 *>(d.C);
    if (row0 + 64 <= d.M && oc0 + OC <= ncols) {
        // whole block inside C: the store of rows RPI t .. from a row pointer
        // the wave shares (SGPRs, kept opaque as in gemm_bf16_epilogue) plus
        // the lane's 32-bit byte offset
        typedef __attribute__((address_space(1))) char gchar;
        const uint32_t pitch = (uint32_t)d.ldc * 2u;
        const uint32_t off = (uint32_t)(lane / LPR) * pitch + (uint32_t)(oc0 + 8 * (lane % LPR)) * 2u;
        const gchar *rbase = (const gchar *)(reinterpret_cast<char *>(C) + (size_t)row0 * (size_t)pitch);
#pragma unroll
        for (int t = 0; t < 64 / RPI; t++) {
            const bf16x8 v = *reinterpret_cast<const bf16x8 *>(&stage[(RPI * t + lane / LPR) * PITCH + 8 * (lane % LPR)]);
            const gchar *rp = rbase + (uint32_t)(RPI * t) * pitch;
            asm("" : "+s"(rp));
            *(__attribute__((address_space(1))) bf16x8 *)(rp + off) = v;
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < 64 / RPI; t++) {
        const int rr = RPI * t + lane / LPR, c8 = 8 * (lane % LPR);
        const bf16x8 v = *reinterpret_cast<const bf16x8 *>(&stage[rr * PITCH + c8]);
        const int row = row0 + rr, col = oc0 + c8;
        if (row < d.M) {
            bf16 *dst = C + (size_t)row * d.ldc + col;
            if (col + 8 <= ncols) {
                *reinterpret_cast<bf16x8 *>(dst) = v;
            } else {
                for (int e = 0; e < 8 && col + e < ncols; e++) dst[e] = v[e];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Pipelined variant for bf16 A with K % 32 == 0 (every bf16-variant GEMM but
// the band split): the same 256x128 block of 8 waves x (64x64), but operands
// reach LDS by direct global->LDS loads (global_load_lds_dwordx4) into a ring
// of 3 K-chunks, two chunks in flight while the third is multiplied -- about
// twice the bytes in flight of the register-staged kernel, with no registers
// spent on staging.  Each wave's load instruction fills 1 KB of LDS: 16 rows
// of 64 B, lane l carrying row l/4, 16-byte position l%4.  Position p of row
// r holds K-chunk p ^ ((r / 4) % 4), so the 16-byte operand reads (32 rows,
// one chunk) fall on distinct banks.  Identical operands and MFMA order to
// the register-staged kernel, so results are bit-identical (for bf16 outputs
// each MFMA takes its two operands the other way round, which gives the
// transposed block with the same bits: checked against the register-staged
// kernel by the boundary tests).
//
// The loads are issued from inline assembly and waited for with explicit
// s_waitcnt vmcnt(N) + barrier: the compiler's own wait insertion treats any
// LDS read after an LDS DMA as dependent on all of them (vmcnt(0)), which
// would serialise the ring.  The asm sets m0 (the LDS base of the DMA) right
// before each load; these kernels make no other use of m0 (checked on the
// built library by the boundary tests).  The load takes its address as a
// wave-uniform 64-bit base in SGPRs plus a 32-bit per-lane byte offset (the
// instruction's saddr form): one VGPR per load stream instead of a 64-bit
// address pair, and no per-lane address arithmetic when the base advances.
VH_DEVICE void lds_dma16s(uint32_t voffset, const void *sbase, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voffset), "s"(sbase), "s"(lds_base)
                 : "memory");
}

template <int N>
VH_DEVICE void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

constexpr int GBD_BM = 256, GBD_BN = 128, GBD_BK = 32, GBD_STAGES = 3, GBD_THREADS = 512;

template <int EPI, typename TC>
__device__ __forceinline__ void gemm_bf16_dma_body(const GemmDescBF16 &d, int tile) {
    // bf16 outputs leave through LDS in row order (gemm_bf16_epilogue_staged):
    // their MFMAs take the B tile first
    constexpr bool ROWS = std::is_same<TC, bf16>::value;
    constexpr int BM = GBD_BM, BN = GBD_BN, BK = GBD_BK, STAGES = GBD_STAGES, W = GBD_THREADS / 64;
    constexpr int A_BYTES = BM * BK * 2, STAGE_BYTES = A_BYTES + BN * BK * 2;
    constexpr int NA = BM / 16 / W, NB = BN / 16 / W;  // load instructions per wave per chunk
    static_assert(NA * 16 * W == BM && NB * 16 * W == BN, "loads must tile the chunk");
    __shared__ __attribute__((aligned(1024))) unsigned char ring[STAGES * STAGE_BYTES];

    const int tiles_n = (d.N + BN - 1) / BN;
    const int tiles_m = (d.M + BM - 1) / BM;
    if (tile >= tiles_m * tiles_n) return;
    const int gsz = (size_t)d.N * d.K * sizeof(bf16) <= (3u << 20) ? 1 : 8;
    const int group = tile / (gsz * tiles_n);
    const int in_group = tile % (gsz * tiles_n);
    const int group_rows = min(gsz, tiles_m - group * gsz);
    const int m0 = (group * gsz + in_group % group_rows) * BM;
    const int n0 = (in_group / group_rows) * BN;

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave >> 1, wn = wave & 1;  // 4 x 2 waves of 64 x 64
    const int li = lane & 31, lh = lane >> 5;
    const uint32_t ring_base = (uint32_t)(uintptr_t)ring;
    auto swz = [](int r) { return (r >> 2) & 3; };

    // load sources: the tile's first row (wave-uniform base) plus a 32-bit
    // lane byte offset (below 2^32: at most 256 rows of lda, ldb <= 2^21)
    const int dr = lane >> 2, dp = lane & 3;
    const bf16 *a_base = static_cast<const bf16 *>(d.A) + (size_t)m0 * d.lda;
    const bf16 *b_base = d.B + (size_t)n0 * d.ldb;
    uint32_t a_voff[NA], b_voff[NB];
#pragma unroll
    for (int j = 0; j < NA; j++) {
        const int r = 16 * (NA * wave + j) + dr;
        a_voff[j] = (uint32_t)(min(m0 + r, d.M - 1) - m0) * (uint32_t)d.lda * 2u + 16u * (dp ^ swz(r));
    }
#pragma unroll
    for (int j = 0; j < NB; j++) {
        const int r = 16 * (NB * wave + j) + dr;
        b_voff[j] = (uint32_t)(min(n0 + r, d.N - 1) - n0) * (uint32_t)d.ldb * 2u + 16u * (dp ^ swz(r));
    }
    auto issue = [&](int kt) {
        const uint32_t sb = ring_base + (kt % STAGES) * STAGE_BYTES;
        const int k0 = kt * BK;
#pragma unroll
        for (int j = 0; j < NA; j++) lds_dma16s(a_voff[j], a_base + k0, sb + (NA * wave + j) * 1024);
#pragma unroll
        for (int j = 0; j < NB; j++) lds_dma16s(b_voff[j], b_base + k0, sb + A_BYTES + (NB * wave + j) * 1024);
    };

    // bf16 outputs: the epilogue's bias quads, loaded before the K loop so
    // that their latency is spent there (they precede every DMA load, so the
    // loop's in-order vmcnt waits cover them)
    floatx4 bq[8];
    if constexpr (ROWS) bias_quads_staged<EPI>(d, n0 + wn * 64, lh, bq);

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.0f;

    // chunk kt lives in slot kt % 3; chunks kt+1 and kt+2 are in flight while
    // kt is multiplied.  Slot (kt+2) % 3 was last read in iteration kt-1,
    // which every wave finished before the barrier that ends it.
    const int nk = d.K / BK;
    issue(0);
    if (nk > 1) {
        issue(1);
        wait_vmcnt<NA + NB>();
    } else {
        wait_vmcnt<0>();
    }
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 2 < nk) issue(kt + 2);
        const unsigned char *sbuf = ring + (kt % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int st = 0; st < BK / 16; st++) {
            bf16x8 a[2], b[2];
            const int c = 2 * st + lh;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int r = wm * 64 + 32 * i + li;
                a[i] = *reinterpret_cast<const bf16x8 *>(sbuf + r * 64 + 16 * (c ^ swz(r)));
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int r = wn * 64 + 32 * j + li;
                b[j] = *reinterpret_cast<const bf16x8 *>(sbuf + A_BYTES + r * 64 + 16 * (c ^ swz(r)));
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = ROWS ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[i], acc[i][j], 0, 0, 0)
                                     : __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 2 < nk) wait_vmcnt<NA + NB>();  // chunk kt+1 has landed; kt+2 may still fly
        else wait_vmcnt<0>();
        __syncthreads();
    }
    if constexpr (ROWS) {
        // the ring is free: every wave finished its reads before the last
        // barrier and no load is in flight; wave w stages in its own ninth
        static_assert(GBD_THREADS / 64 * 64 * (64 + 8) * 2 <= STAGES * STAGE_BYTES, "staging fits the ring");
        gemm_bf16_epilogue_staged<EPI>(d, acc, reinterpret_cast<bf16 *>(ring) + wave * 64 * (64 + 8), m0 + wm * 64,
                                       n0 + wn * 64, lane, bq);
    } else {
        gemm_bf16_epilogue<EPI, TC, 2, 2>(d, acc, m0 + wm * 64, n0 + wn * 64, li, lh);
    }
}

template <int EPI, typename TC>
__global__ __launch_bounds__(GBD_THREADS, 2) void gemm_bf16_dma_kernel(GemmDescBF16 d) {
    gemm_bf16_dma_body<EPI, TC>(d, xcd_swizzle((int)blockIdx.x, (int)gridDim.x));
}

template <int EPI, typename TC>
__global__ __launch_bounds__(GBD_THREADS, 2) void gemm_bf16_dma_batched_kernel(GemmBatchBF16 b) {
    gemm_bf16_dma_body<EPI, TC>(b.d[blockIdx.z], (int)blockIdx.x);
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
