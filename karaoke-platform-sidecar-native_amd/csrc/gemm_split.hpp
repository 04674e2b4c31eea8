// fp32 token-wise linear on bf16 matrix cores by exact operand splitting:
// C[M][N] (op)= A[M][K] * W[N][K]^T with fp32 inputs, fp32 accumulation and
// the fused epilogues of the fp32 GEMM (gemm.hpp).
//
// Splitting.  Every fp32 x is the exact sum of three bf16 values
//   h = bf16(x),  m = bf16(x - h),  l = x - h - m
// (round to nearest even at each step; x - h and x - h - m are exact in fp32
// by Sterbenz, and the last remainder has at most 8 significant bits, so l
// holds it exactly: 3 x 8 bits cover fp32's 24).  With |m| <= 2^-8 |x| and
// |l| <= 2^-16 |x|, the product a*w = sum of nine bf16 x bf16 products, each
// exact in fp32.  The kernel accumulates the six that can reach 2^-24 |a||w|
// (hh, hm, mh, mm, hl, lh) in fp32 and drops ml, lm and ll (together at most
// 2^-23 |a||w|, below the rounding of the fp32 accumulation itself).  Six
// v_mfma_f32_32x32x16_bf16 products per 16 k-values cost 6/16 of a bf16 MFMA
// each, i.e. 2.67x the fp32 MFMA rate (v_mfma_f32_32x32x2f32) per fp32 MAC;
// measured error against fp64 is at or below the fp32 MFMA GEMM's.
//
// Operands.  W is split once, at upload, into its three bf16 pieces, stored
// tile-major: for every 128-row tile of W and every 16-wide K chunk, one
// 12 KB block that is exactly the LDS image of that chunk's W part --
// [piece][128 rows][2 slots][8], k permuted inside every group of 16
// (logical slot 0 holds k 0-3 and 8-11, slot 1 holds k 4-7 and 12-15, so a
// lane's eight k-values for the MFMA are one 16-byte read) and slot s of row
// r stored at s ^ (r/8)%2 (conflict-free operand reads); rows past N are
// zero.  Each W load instruction then reads 1 KB contiguous.  A stays fp32
// in memory (no producer changes); each wave splits the A values it reads
// from LDS in registers.
//
// Pipeline.  256x128 block, 8 waves of 32x128 (four 32x32 accumulators in a
// row), K in chunks of 16: each wave splits the eight A values per lane of
// its 32 rows (every A element is split once per block) and reads all four
// W column tiles.  Operands go straight from global memory to LDS
// (global_load_lds_dwordx4, as gemm_bf16_dma_kernel) into a 2-chunk ring: A
// as fp32 rows of 64 B (4 slots, slot c of row r at c ^ (r/4)%4), each W
// plane as rows of 32 B (2 slots, slot s of row r at s ^ (r/8)%2), so the
// operand reads are conflict-free.  56 KB of LDS, two workgroups per CU.
// The loads take a wave-uniform base and a 32-bit lane offset (the saddr
// form), which keeps the kernel within 120 VGPRs and its address arithmetic
// scalar; the branch on live accumulator columns is taken once per tile,
// outside the K loop.
#pragma once

#include "gemm_bf16.hpp"

namespace vh {

struct GemmDescSplit {
    const float *A;     // fp32 [M][lda]
    const bf16 *W;      // pieces, tile-major (split_weight_kernel)
    const float *bias;  // fp32, may be null
    float *C;           // fp32 [M][ldc]
    int M, N, K;
    int lda, ldc;
};

constexpr int GS_BM = 256, GS_BN = 128, GS_BK = 16, GS_THREADS = 512;
constexpr int GS_WBLOCK = 3 * GS_BN * GS_BK;  // bf16 per (row tile, K chunk) block of W pieces

// Index of k inside its W plane row (the 16-group permutation above).
VH_HOST_DEVICE inline int split_k_slot(int k) {
    const int r = k & 15;
    return (k & ~15) + 8 * ((r >> 2) & 1) + (r & 3) + 4 * (r >> 3);
}

VH_DEVICE void split3(float x, bf16 &h, bf16 &m, bf16 &l) {
    h = (bf16)x;
    const float r1 = x - (float)h;
    m = (bf16)r1;
    l = (bf16)(r1 - (float)m);
}

// Two fp32 -> two bf16 (nearest even) in one dword: one v_cvt_pk_bf16_f32.
VH_DEVICE uint32_t pack_bf16x2(float a, float b) {
    typedef float floatx2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){a, b}, bf16x2));
}

// Eight fp32 values (two float4) -> their h, m, l bf16 pieces.  Each piece
// pair is converted once, packed as the MFMA operand wants it, and read back
// as fp32 from the packed dword (low half << 16, high half masked): 5.5 VALU
// instructions per value.
VH_DEVICE void split8(floatx4 lo, floatx4 hi, bf16x8 &h, bf16x8 &m, bf16x8 &l) {
    const float x[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    uint32_t ph[4], pm[4], pl[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float a = x[2 * e], b = x[2 * e + 1];
        ph[e] = pack_bf16x2(a, b);
        const float ra = a - __uint_as_float(ph[e] << 16), rb = b - __uint_as_float(ph[e] & 0xffff0000u);
        pm[e] = pack_bf16x2(ra, rb);
        const float sa = ra - __uint_as_float(pm[e] << 16), sb = rb - __uint_as_float(pm[e] & 0xffff0000u);
        pl[e] = pack_bf16x2(sa, sb);
    }
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    h = __builtin_bit_cast(bf16x8, (u32x4){ph[0], ph[1], ph[2], ph[3]});
    m = __builtin_bit_cast(bf16x8, (u32x4){pm[0], pm[1], pm[2], pm[3]});
    l = __builtin_bit_cast(bf16x8, (u32x4){pl[0], pl[1], pl[2], pl[3]});
}

template <int EPI>
__device__ __forceinline__ void gemm_split_body(const GemmDescSplit &d, int tile) {
    constexpr int A_BYTES = GS_BM * GS_BK * 4;  // 16 KB: fp32 rows of 64 B
    constexpr int P_BYTES = GS_BN * GS_BK * 2;  // 4 KB per W plane: bf16 rows of 32 B
    constexpr int STAGE_BYTES = A_BYTES + 3 * P_BYTES;
    __shared__ __attribute__((aligned(1024))) unsigned char ring[2 * STAGE_BYTES];

    const int tiles_n = (d.N + GS_BN - 1) / GS_BN;
    const int tiles_m = (d.M + GS_BM - 1) / GS_BM;
    if (tile >= tiles_m * tiles_n) return;
    // column-fastest order within groups of row tiles (see gemm.hpp)
    const int gsz = (size_t)d.N * d.K * 6 <= (3u << 20) ? 1 : 8;
    const int group = tile / (gsz * tiles_n);
    const int in_group = tile % (gsz * tiles_n);
    const int group_rows = min(gsz, tiles_m - group * gsz);
    const int m0 = (group * gsz + in_group % group_rows) * GS_BM;
    const int n0 = (in_group / group_rows) * GS_BN;

    const int tid = (int)threadIdx.x;
    // wave-uniform: the per-wave choices below are scalar branches and the
    // load bases live in SGPRs
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const uint32_t ring_base = (uint32_t)(uintptr_t)ring;
    auto swz_a = [](int r) { return (r >> 2) & 3; };
    auto swz_w = [](int r) { return (r >> 3) & 1; };

    // Each load instruction fills 1 KB of the stage.  A: 16 blocks of 16 rows
    // (lane -> row l/4, slot l%4); wave w loads blocks w and w+8, each lane
    // from the tile's first row (scalar base) plus its own byte offset (below
    // 2^32: 256 rows of lda <= 2^21 floats).  W: the 12 1 KB blocks of the chunk's
    // tile-major image, lane l the l-th 16 bytes; wave w loads block w, and
    // waves 0-3 also block w+8.
    const float *a_base = d.A + (size_t)m0 * d.lda;
    uint32_t a_voff[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = 16 * (wave + 8 * j) + (lane >> 2);
        a_voff[j] = (uint32_t)(min(m0 + r, d.M - 1) - m0) * (uint32_t)d.lda * 4u + 16u * ((lane & 3) ^ swz_a(r));
    }
    const bf16 *w_base = d.W + (size_t)(n0 / GS_BN) * (d.K / GS_BK) * GS_WBLOCK;
    const uint32_t w_voff = 16 * lane;
    const int wb1 = min(wave + 8, 11);
    const bool two_w = wave < 4;
    auto issue = [&](int kt) {
        const uint32_t sb = ring_base + (kt & 1) * STAGE_BYTES;
        const float *ab = a_base + kt * GS_BK;
        lds_dma16s(a_voff[0], ab, sb + wave * 1024);
        lds_dma16s(a_voff[1], ab, sb + (wave + 8) * 1024);
        const bf16 *wb = w_base + (size_t)kt * GS_WBLOCK;
        lds_dma16s(w_voff, wb + wave * 512, sb + A_BYTES + wave * 1024);
        if (two_w) lds_dma16s(w_voff, wb + wb1 * 512, sb + A_BYTES + wb1 * 1024);
    };

    floatx16 acc[1][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[0][j][r] = 0.0f;

    const int nk = d.K / GS_BK;
    issue(0);
    wait_vmcnt<0>();
    __syncthreads();
    // The K loop for NJ live 32-column accumulators (4; 2 or 1 in a ragged
    // last column tile, whose columns past N are skipped, or computed from
    // the zero rows of the pieces when N - n0 is 65..96): chosen once per
    // tile, so the loop body is one basic block the compiler can schedule as
    // a whole.
    auto k_loop = [&](auto nj_c) {
        constexpr int NJ = decltype(nj_c)::value;
        for (int kt = 0; kt < nk; kt++) {
            // chunk kt+1 goes to the slot chunk kt-1 used: every wave finished
            // reading it before the barrier that ended the previous iteration
            if (kt + 1 < nk) issue(kt + 1);
            const unsigned char *sbuf = ring + (kt & 1) * STAGE_BYTES;
            const int r = wave * 32 + li;
            const floatx4 lo = *reinterpret_cast<const floatx4 *>(sbuf + r * 64 + 16 * (lh ^ swz_a(r)));
            const floatx4 hi = *reinterpret_cast<const floatx4 *>(sbuf + r * 64 + 16 * ((2 + lh) ^ swz_a(r)));
            bf16x8 ah, am, al;
            split8(lo, hi, ah, am, al);
            // small products first: (l,h) (h,l) (m,m) (m,h) (h,m) (h,h)
            const bf16x8 pa[6] = {al, ah, am, am, ah, ah};
            // W column tiles two at a time: their 6 pieces, then 12 products
#pragma unroll
            for (int jp = 0; jp < (NJ + 1) / 2; jp++) {
                constexpr int NJJ = NJ == 1 ? 1 : 2;
                bf16x8 wh[NJJ], wmd[NJJ], wl[NJJ];
#pragma unroll
                for (int jj = 0; jj < NJJ; jj++) {
                    const int rw = 32 * (2 * jp + jj) + li;
                    const unsigned char *wp = sbuf + A_BYTES + rw * 32 + 16 * (lh ^ swz_w(rw));
                    wh[jj] = *reinterpret_cast<const bf16x8 *>(wp);
                    wmd[jj] = *reinterpret_cast<const bf16x8 *>(wp + P_BYTES);
                    wl[jj] = *reinterpret_cast<const bf16x8 *>(wp + 2 * P_BYTES);
                }
                const bf16x8 *pw[6] = {wh, wl, wmd, wh, wmd, wh};
#pragma unroll
                for (int t = 0; t < 6; t++)
#pragma unroll
                    for (int jj = 0; jj < NJJ; jj++)
                        acc[0][2 * jp + jj] =
                            __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[t], pw[t][jj], acc[0][2 * jp + jj], 0, 0, 0);
            }
            wait_vmcnt<0>();  // chunk kt+1 has landed
            __syncthreads();
        }
    };
    const int live = d.N - n0;
    if (live > 64) k_loop(std::integral_constant<int, 4>());
    else if (live > 32) k_loop(std::integral_constant<int, 2>());
    else k_loop(std::integral_constant<int, 1>());
    GemmDescBF16 e{};
    e.bias = d.bias; e.C = d.C; e.M = d.M; e.N = d.N; e.K = d.K; e.ldc = d.ldc;
    gemm_bf16_epilogue<EPI, float, 1, 4>(e, acc, m0 + wave * 32, n0, li, lh);
}

template <int EPI>
__global__ __launch_bounds__(GS_THREADS, 2) void gemm_split_kernel(GemmDescSplit d) {
    gemm_split_body<EPI>(d, xcd_swizzle((int)blockIdx.x, (int)gridDim.x));
}

// Problems per launch of the ragged batched GEMMs (the mask estimator's
// per-band linears): descriptors in the kernel arguments, problem blockIdx.z,
// blocks past a problem's tiles return.
constexpr int GS_MAX_BATCH = 64;

// fp32 W [N][ldw_in] (K a multiple of 16) -> its h, m, l pieces, tile-major:
// element (n, k) of piece p at
//   ((n/128 * K/16 + k/16) * 3 + p) * 2048 + (n%128) * 16 + 8 * (s ^ (n/8)%2) + e
// where slot s and element e come from split_k_slot(k) % 16 = 8 s + e.  One
// thread per (padded row, k); rows past N are written as zero.
static __global__ __launch_bounds__(256) void split_weight_kernel(const float *__restrict__ W, int N, int K, int ldw_in,
                                                                 bf16 *__restrict__ tiles) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int rows = (N + GS_BN - 1) / GS_BN * GS_BN;
    if (idx >= (int64_t)rows * K) return;
    const int n = (int)(idx / K), k = (int)(idx % K);
    bf16 h = (bf16)0.0f, m = (bf16)0.0f, l = (bf16)0.0f;
    if (n < N) split3(W[(size_t)n * ldw_in + k], h, m, l);
    const int r = n % GS_BN, pos = split_k_slot(k) & 15;
    const int phys = (pos >> 3) ^ ((r >> 3) & 1);
    const size_t o = ((size_t)(n / GS_BN) * (K / GS_BK) + k / GS_BK) * GS_WBLOCK + (size_t)r * GS_BK + 8 * phys + (pos & 7);
    tiles[o] = h;
    tiles[o + GS_BN * GS_BK] = m;
    tiles[o + 2 * GS_BN * GS_BK] = l;
}

}  // namespace vh
