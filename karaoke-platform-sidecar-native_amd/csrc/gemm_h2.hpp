// fp32 token-wise linear on fp16 matrix cores by two-piece operand splitting:
// C[M][N] (op)= A[M][K] * W[N][K]^T with fp32 inputs, fp32 accumulation and
// the fused epilogues of the fp32 GEMM (gemm.hpp).  The default fp32 path's
// transformer and mask-estimator linears.
//
// Splitting.  Each operand is first scaled by a power of two 2^e (exact), so
// that everything it can hold lies below 2^14; then every scaled value y is
// split into two fp16 values (round to nearest even)
//   h = fp16(y),  m = fp16(y - h)
// y - h is exact in fp32 (Sterbenz) and |m| <= 2^-11 |y|, so h + m carries 22
// significant bits; where m is an fp16 subnormal (|y| < 2^-3, i.e. below
// 2^-17 of the operand's bound) the pair is exact to 2^-25 absolute.  The
// kernel accumulates the three products hh, hm, mh -- each exact in fp32
// (11 x 11 bits) -- and drops mm (<= 2^-22 |a||w|) and the pieces' rounding
// (<= 2^-22 each): per product term about 2^-21 relative, which the fp32
// accumulation over K (16 terms per MFMA, K/16 x 3 roundings) already
// exceeds.  Measured against fp64 on the transformer shapes, the result is
// 1.5-2 dB more accurate than the three-piece bf16 split (gemm_split.hpp,
// six products) and as accurate as a sequential fp32 FMA chain, at half its
// matrix-core work.
//
// Scales.  W's exponent comes from its absolute maximum, found on the device
// when the pieces are made and kept in their 256-byte header.  A's comes
// from a bound the caller supplies -- a value or a device float -- that every
// |A| element respects; the model derives exact bounds from the producers'
// weights (operand_bounds_kernel): an RMSNorm output obeys
// |y_i| <= ||y||_2 <= sqrt(D) max|gamma|, a linear of it obeys
// |W y + b|_n <= sqrt(D) max|gamma| ||W_n||_2 + |b_n|, an attention output
// (a convex combination of value rows times a gate in (0, 1)) obeys the
// value bound, a GELU-GLU output the square of its pre-activation bound
// (|gelu(g)| <= |g|), a tanh output 1.  The bound only has to hold: a loose
// one costs precision only for elements more than 2^17 below it.
//
// Operands and pipeline as gemm_split.hpp (256x128 block, 8 waves of 32x128,
// K chunks of 16 in a global->LDS DMA ring, A fp32 in LDS split by each wave
// in registers, or h2 rows read as they are): W's pieces are two fp16 planes
// per tile-major block (8 KB per 128 rows x 16 k, the same row/slot
// permutation), one 1 KB load per wave per chunk; a 3-chunk ring (two chunks
// in flight while one is multiplied: 72 KB of LDS, two workgroups per CU;
// 0-2.4% faster than two chunks, bit-identical); per wave and chunk 12 MFMAs
// (v_mfma_f32_32x32x16_f16) and, for fp32 A, 4 VALU per A value for the scale
// and split.
#pragma once

#include "attention.hpp"
#include "gemm_split.hpp"
#include "h2.hpp"

namespace vh {

struct GemmDescH2 {
    const float *A;  // fp32 [M][lda]
    const void *W;   // pieces (split_weight_h2_kernel): 256-byte header, then the planes
    const float *bias;
    float *C;
    int M, N, K;
    int lda, ldc;
    // Null for none.  zero_slot: a device float the kernel sets to 0 (the bound
    // slot a later residual GEMM raises); amax: raised to max |C| by the
    // residual epilogue (gemm_bf16_epilogue).
    float *zero_slot;
    float *amax;
    // kv_inner > 0: C holds a fused q|k|v|gates projection with k in columns
    // [kv_inner, 2 kv_inner) and v in [2 kv_inner, 3 kv_inner); those are
    // written times 2^ek and 2^ev (att_h2_exponents of *kv_bound), the scales
    // the fp16 two-piece attention would otherwise apply as it stages them
    const float *kv_bound;
    int kv_inner;
    // kv_pieces (with kv_inner): k, rotated, and v are written as the fp16
    // pieces of those scaled values (kv_pieces_epilogue), the rotary position
    // of row r being the frame (r / rope_period) % rope_len of rows ordered
    // [chunk][frame][band] (rope_period bands per frame), its (cos, sin) at
    // rope[(frame * 32 + pair) * 2]
    int kv_pieces;
    const float *rope;
    int rope_period, rope_len;
};

// The fused projection's k or v column tile (32 x 128 per wave, n0 inside
// [kv_inner, 3 kv_inner)) written as fp16 pieces instead of fp32: the head's
// 64 columns of a row occupy its 256 bytes of the region -- 64 h halves, then
// 64 m halves, dim order -- where h + m is the value y scaled by 2^ek (2^ev),
// h = fp16(y), m = fp16(y - h) (exact difference): the pieces the two-piece
// attention's staging forms, so the attention copies them into LDS as they
// are.  k is rotated first (rope_own: each lane swaps its value with the
// lane of the pair's other dimension), by the (cos, sin) of the row's frame;
// a wave's 32 consecutive rows span at most two frames.  Each value is first
// formed as the plain epilogue forms it: acc times the row's norm scale plus
// the bias in one fused multiply-add.
// tv: the rotary table entry (cos, sin) of frame f0 (lanes 0-31) or f1
// (lanes 32-63) and pair lane % 32, loaded before the K loop (k tiles only).
VH_DEVICE void kv_pieces_epilogue(const GemmDescH2 &d, int row0, int n0, int li, int lh, float2 tv,
                                  const floatx16 (&acc)[1][4], floatx16 rs, floatx4 bpre) {
    const bool is_k = n0 < 2 * d.kv_inner;
    const int region = is_k ? d.kv_inner : 2 * d.kv_inner;  // first column of the k (v) region
    const int B = d.rope_period;
    // first row (within the wave's 32) of the second frame the rows span: its
    // table entries are those tv holds in lanes 32-63
    const int off_b = B - row0 % B;
    const bool even = (li & 1) == 0;
    typedef __attribute__((address_space(1))) char gchar;
    typedef __attribute__((address_space(1))) uint16_t gu16;
    const uint32_t pitch = (uint32_t)d.ldc * 4u;
    const gchar *const rbase = (const gchar *)(reinterpret_cast<char *>(d.C) + (size_t)row0 * (size_t)pitch);
    // one straight-line body per (k or v, whole or ragged row tile, frame
    // boundary inside the wave's rows or not)
    auto body = [&](auto k_c, auto full_c, auto split_c) {
        constexpr bool IS_K = decltype(k_c)::value, FULL = decltype(full_c)::value;
        constexpr bool SPLIT = decltype(split_c)::value;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // one column tile at a time: nothing of the next is hoisted into
            // this one (the registers the K loop needs bound the epilogue's)
            __builtin_amdgcn_sched_barrier(0);
            const int kc = n0 + 32 * j + li - region;
            const uint32_t off_h = 4u * (uint32_t)region + 256u * (uint32_t)(kc >> 6) + 2u * (uint32_t)(kc & 63) +
                                   (uint32_t)(4 * lh) * pitch;
            float c0 = 1.0f, s0 = 0.0f, c1 = 1.0f, s1 = 0.0f;
            if constexpr (IS_K) {
                // the lane's pair: its entries from the lanes holding them
                const int pr = (kc & 63) >> 1;
                c0 = __shfl(tv.x, pr, 64);
                s0 = __shfl(tv.y, pr, 64);
                if (even) s0 = -s0;
                if constexpr (SPLIT) {
                    c1 = __shfl(tv.x, 32 + pr, 64);
                    s1 = __shfl(tv.y, 32 + pr, 64);
                    if (even) s1 = -s1;
                }
            }
            // rows in pairs (registers r, r + 1: consecutive rows of one
            // column): one v_cvt_pk_f16_f32 makes both h, one v_fma_mix_f32
            // per value and one v_cvt_pk_f16_f32 both m (m_pair_f16); the
            // halves leave by 2-byte stores of each half of the packed dwords
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                float y[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    y[e] = fmaf(acc[0][j][r + e], rs[r + e], bpre[j]);
                    if constexpr (IS_K) {
                        const float other =
                            __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(y[e]), 0xB1, 0xF, 0xF, false));
                        bool nxt = false;
                        if constexpr (SPLIT) nxt = 8 * ((r + e) >> 2) + 4 * lh + ((r + e) & 3) >= off_b;
                        y[e] = rope_own(y[e], other, nxt ? c1 : c0, nxt ? s1 : s0);
                    }
                }
                const uint32_t hp = pack_f16x2(y[0], y[1]);
                const uint32_t mp = m_pair_f16(y[0], y[1], opaque_one(), hp);
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const uint16_t hb = (uint16_t)(hp >> (16 * e)), mb = (uint16_t)(mp >> (16 * e));
                    const int rr = 8 * ((r + e) >> 2) + ((r + e) & 3);  // the row of register r + e, less 4 lh
                    if constexpr (FULL) {
                        // wave-uniform row pointer (SGPRs) + the lane's 32-bit
                        // offset; the high halves by the d16_hi form of the
                        // same store, which the compiler would otherwise
                        // address with a 64-bit VGPR pair per store
                        const gchar *rp = rbase + (uint32_t)rr * pitch;
                        asm("" : "+s"(rp));
                        if (e == 0) {
                            __builtin_nontemporal_store(hb, (gu16 *)(rp + off_h));
                            __builtin_nontemporal_store(mb, (gu16 *)(rp + off_h + 128u));
                        } else {
                            asm volatile("global_store_short_d16_hi %0, %1, %2 nt\n\t"
                                         "global_store_short_d16_hi %0, %3, %2 offset:128 nt"
                                         :
                                         : "v"(off_h), "v"(hp), "s"(rp), "v"(mp)
                                         : "memory");
                        }
                    } else if (row0 + rr + 4 * lh < d.M) {
                        char *rp = reinterpret_cast<char *>(d.C) + (size_t)(row0 + rr) * pitch + off_h;
                        __builtin_nontemporal_store(hb, reinterpret_cast<uint16_t *>(rp));
                        __builtin_nontemporal_store(mb, reinterpret_cast<uint16_t *>(rp + 128));
                    }
                }
            }
        }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    if (row0 + 32 <= d.M) {
        if (!is_k) body(F_(), T_(), F_());
        else if (off_b >= 32) body(T_(), T_(), F_());
        else body(T_(), T_(), T_());
    } else {
        if (!is_k) body(F_(), F_(), F_());
        else body(T_(), F_(), T_());
    }
}
// Bound on |A|: *ptr when ptr is set (a device float), else value.
struct H2Bound {
    const float *ptr;
    float value;
};

constexpr int H2_HEADER = 256;                // bytes before the planes: float max|W|
constexpr int H2_WBLOCK = 2 * GS_BN * GS_BK;  // fp16 per (row tile, K chunk) block of W pieces

// A_H2: A arrives as h2 rows (h2.hpp) scaled by 2^h2_exponent(a_bound) -- its
// producer split it -- and the K loop only reads the pieces.
// RING: K chunks held in LDS, RING - 1 of them in flight while one is multiplied.
// NORM (fp32 A): the GEMM of an RMSNorm of A's rows, W holding the norm's gain
// folded in (W[n][k] gamma[k]): each accumulator row is multiplied by its row's
// sqrt(K) / sqrt(sum_k A^2 + 1e-12) (the RMSNorm kernels' expression), the
// sum taken from the fp32 values the K loop splits anyway, before bias and
// activation.  So the normalised rows are never written: the RMSNorm pass and
// its 2 x 4 bytes per element of traffic go, and A is the residual stream
// itself, bounded by the max |x| its producer's epilogue recorded.
// KVS: the k and v columns scaled (GemmDescH2::kv_inner), compiled only into
// the fused projection's instantiations, and with kv_pieces written as their
// fp16 pieces (k rotated).
template <int EPI, bool A_H2, int RING = 3, bool NORM = false, bool KVS = false>
__device__ __forceinline__ void gemm_h2_body(const GemmDescH2 &d, float a_bound, int tile) {
    static_assert(!(NORM && A_H2), "the row norm needs the fp32 rows");
    constexpr int A_BYTES = GS_BM * GS_BK * 4;  // 16 KB: fp32 rows of 64 B
    constexpr int P_BYTES = GS_BN * GS_BK * 2;  // 4 KB per W plane: fp16 rows of 32 B
    constexpr int STAGE_BYTES = A_BYTES + 2 * P_BYTES;
    __shared__ __attribute__((aligned(1024))) unsigned char ring[RING * STAGE_BYTES];

    const int tiles_n = (d.N + GS_BN - 1) / GS_BN;
    const int tiles_m = (d.M + GS_BM - 1) / GS_BM;
    if (d.zero_slot && tile == 0 && threadIdx.x == 0) *d.zero_slot = 0.0f;
    if (tile >= tiles_m * tiles_n) return;
    // column-fastest order within groups of row tiles (see gemm.hpp)
    // groups of 4 row tiles for the wide GEMMs (measured against 1, 2, 8, 16:
    // best by 0.3-1.3% on N = 1568 and 3072), one for N = 384
    const int gsz = d.N >= 1024 ? 4 : 1;
    const int group = tile / (gsz * tiles_n);
    const int in_group = tile % (gsz * tiles_n);
    const int group_rows = min(gsz, tiles_m - group * gsz);
    const int m0 = (group * gsz + in_group % group_rows) * GS_BM;
    const int n0 = (in_group / group_rows) * GS_BN;

    const int ea = h2_exponent(a_bound);
    const int ew = h2_exponent(*static_cast<const float *>(d.W));
    const float a_scale = ldexpf(1.0f, ea);

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int li = lane & 31, lh = lane >> 5;
    const uint32_t ring_base = (uint32_t)(uintptr_t)ring;
    auto swz_a = [](int r) { return (r >> 2) & 3; };
    auto swz_w = [](int r) { return (r >> 3) & 1; };

    // the bias of the lane's column in each 32-column tile (0 past N), loaded
    // before the K loop so that its latency is spent there, not in the
    // epilogue
    float bpre[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int col = n0 + 32 * j + li;
        bpre[j] = d.bias && col < d.N ? d.bias[col] : 0.0f;
    }
    // each 32-column tile's extra power of two: ek for k columns, ev for v
    // (kv_inner is a multiple of 32, so a tile is all q, k, v or gates)
    int ekv[4] = {0, 0, 0, 0};
    if (KVS && d.kv_inner > 0) {
        int ek, eq, ev;
        att_h2_exponents(*d.kv_bound, 1.0f, ek, eq, ev);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = n0 + 32 * j;
            ekv[j] = c < d.kv_inner ? 0 : c < 2 * d.kv_inner ? ek : c < 3 * d.kv_inner ? ev : 0;
        }
    }

    // A: 16 loads of 1 KB (16 rows each), wave w loads blocks w and w+8 from
    // the tile's first row (scalar base) plus its lane offset (below 2^32:
    // 256 rows of lda <= 2^21 floats).  W: the 8 1 KB blocks of the chunk's
    // tile-major image, wave w the w-th.
    const float *a_base = d.A + (size_t)m0 * d.lda;
    uint32_t a_voff[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int r = 16 * (wave + 8 * j) + (lane >> 2);
        a_voff[j] = (uint32_t)(min(m0 + r, d.M - 1) - m0) * (uint32_t)d.lda * 4u + 16u * ((lane & 3) ^ swz_a(r));
    }
    const _Float16 *w_base = reinterpret_cast<const _Float16 *>(static_cast<const char *>(d.W) + H2_HEADER) +
                             (size_t)(n0 / GS_BN) * (d.K / GS_BK) * H2_WBLOCK;
    const uint32_t w_voff = 16 * lane;
    auto issue = [&](int kt) {
        const uint32_t sb = ring_base + (kt % RING) * STAGE_BYTES;
        const float *ab = a_base + kt * GS_BK;
        lds_dma16s(a_voff[0], ab, sb + wave * 1024);
        lds_dma16s(a_voff[1], ab, sb + (wave + 8) * 1024);
        lds_dma16s(w_voff, w_base + (size_t)kt * H2_WBLOCK + wave * 512, sb + A_BYTES + wave * 1024);
    };

    floatx16 acc[1][4];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[0][j][r] = 0.0f;

    // k/v pieces: the rotary table entries the epilogue of a k tile needs,
    // loaded now so that their latency is spent in the K loop (two registers)
    float2 tv = make_float2(1.0f, 0.0f);
    if constexpr (KVS && NORM && EPI == EPI_STORE) {
        if (d.kv_pieces && n0 >= d.kv_inner && n0 < 2 * d.kv_inner) {
            const int row0 = m0 + wave * 32;
            const int f0 = (row0 / d.rope_period) % d.rope_len;
            const int f = lane < 32 ? f0 : (f0 + 1 == d.rope_len ? 0 : f0 + 1);
            tv = *reinterpret_cast<const float2 *>(d.rope + 2 * (f * 32 + (lane & 31)));
        }
    }
    const int nk = d.K / GS_BK;
    float ss = 0.0f;  // NORM: sum of squares of this lane's half of row wave*32 + li
#pragma unroll
    for (int i = 0; i < RING - 1; i++)
        if (i < nk) issue(i);
    if constexpr (RING > 2) {
        if (nk > 1) wait_vmcnt<3 * (RING - 2)>();  // chunk 0 has landed
        else wait_vmcnt<0>();
    } else {
        wait_vmcnt<0>();
    }
    __syncthreads();
    // NJ live 32-column accumulators, chosen once per tile (as gemm_split_body)
    auto k_loop = [&](auto nj_c) {
        constexpr int NJ = decltype(nj_c)::value;
        for (int kt = 0; kt < nk; kt++) {
            // chunk kt+RING-1 goes to the slot chunk kt-1 used: every wave
            // finished reading it before the barrier that ended the previous
            // iteration
            if (kt + RING - 1 < nk) issue(kt + RING - 1);
            const unsigned char *sbuf = ring + (kt % RING) * STAGE_BYTES;
            const int r = wave * 32 + li;
            const unsigned char *ar = sbuf + r * 64;
            halfx8 ah, am;
            if constexpr (A_H2) {
                ah = *reinterpret_cast<const halfx8 *>(ar + 16 * (lh ^ swz_a(r)));
                am = *reinterpret_cast<const halfx8 *>(ar + 16 * ((2 + lh) ^ swz_a(r)));
            } else {
                const floatx4 lo = *reinterpret_cast<const floatx4 *>(ar + 16 * (lh ^ swz_a(r)));
                const floatx4 hi = *reinterpret_cast<const floatx4 *>(ar + 16 * ((2 + lh) ^ swz_a(r)));
                split8_h2(lo, hi, a_scale, ah, am);
                if constexpr (NORM) {
#pragma unroll
                    for (int e = 0; e < 4; e++) ss = fmaf(hi[e], hi[e], fmaf(lo[e], lo[e], ss));
                }
            }
            // W column tiles two at a time: their pieces, then (m,h) (h,m) (h,h)
#pragma unroll
            for (int jp = 0; jp < (NJ + 1) / 2; jp++) {
                constexpr int NJJ = NJ == 1 ? 1 : 2;
                halfx8 wh[NJJ], wm[NJJ];
#pragma unroll
                for (int jj = 0; jj < NJJ; jj++) {
                    const int rw = 32 * (2 * jp + jj) + li;
                    const unsigned char *wp = sbuf + A_BYTES + rw * 32 + 16 * (lh ^ swz_w(rw));
                    wh[jj] = *reinterpret_cast<const halfx8 *>(wp);
                    wm[jj] = *reinterpret_cast<const halfx8 *>(wp + P_BYTES);
                }
#pragma unroll
                for (int jj = 0; jj < NJJ; jj++)
                    acc[0][2 * jp + jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, wh[jj], acc[0][2 * jp + jj], 0, 0, 0);
#pragma unroll
                for (int jj = 0; jj < NJJ; jj++)
                    acc[0][2 * jp + jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wm[jj], acc[0][2 * jp + jj], 0, 0, 0);
#pragma unroll
                for (int jj = 0; jj < NJJ; jj++)
                    acc[0][2 * jp + jj] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, wh[jj], acc[0][2 * jp + jj], 0, 0, 0);
            }
            // chunk kt+1 has landed (3 loads per wave and chunk; later chunks may fly)
            if constexpr (RING > 2) {
                if (kt + RING - 1 < nk) wait_vmcnt<3 * (RING - 2)>();
                else wait_vmcnt<0>();
            } else {
                wait_vmcnt<0>();
            }
            __syncthreads();
        }
    };
    const int live = d.N - n0;
    if (live > 64) k_loop(std::integral_constant<int, 4>());
    else if (live > 32) k_loop(std::integral_constant<int, 2>());
    else k_loop(std::integral_constant<int, 1>());
    // both scales undone at once: acc 2^-(ea+ew) by one v_ldexp_f32 (exact, as
    // the two power-of-two multiplies it replaces were where their product
    // is a normal float, and correctly rounded where it is not)
    const int eu = -(ea + ew);
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int r = 0; r < 16; r++) acc[0][j][r] = ldexpf(acc[0][j][r], eu + ekv[j]);
        bpre[j] = ldexpf(bpre[j], ekv[j]);  // (acc + b) 2^e exactly, with the row norm too
    }
    float rs[16];  // NORM: the scale of each accumulator row, applied with the bias
    if constexpr (NORM) {
        // lanes li and li + 32 summed the two halves of row wave*32 + li;
        // register 4q + e of a lane holds row 8q + 4lh + e of the wave's 32
        __shared__ float rscale[GS_THREADS / 64][32];
        const float tot = ss + __shfl_xor(ss, 32, 64);
        if (lh == 0) rscale[wave][li] = sqrtf((float)d.K) / sqrtf(tot + 1.0e-12f);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const floatx4 r4 = *reinterpret_cast<const floatx4 *>(&rscale[wave][8 * q + 4 * lh]);
#pragma unroll
            for (int e = 0; e < 4; e++) rs[4 * q + e] = r4[e];
        }
    }
    if constexpr (KVS && NORM && EPI == EPI_STORE) {
        if (d.kv_pieces && n0 >= d.kv_inner && n0 < 3 * d.kv_inner) {
            // the plain epilogue's value of each element (bias and row norm in
            // one fused multiply-add), formed in place first so the row
            // scales and biases are dead before the rotation and the split
            // the row scales and biases as vector values (not arrays), which
            // keeps them in registers across the epilogue's variants
            floatx16 rsv;
#pragma unroll
            for (int r = 0; r < 16; r++) rsv[r] = rs[r];
            kv_pieces_epilogue(d, m0 + wave * 32, n0, li, lh, tv, acc, rsv,
                               floatx4{bpre[0], bpre[1], bpre[2], bpre[3]});
            return;
        }
    }
    GemmDescBF16 e{};
    e.bias = d.bias; e.C = d.C; e.M = d.M; e.N = d.N; e.K = d.K; e.ldc = d.ldc;
    float mx = 0.0f;
    gemm_bf16_epilogue<EPI, float, 1, 4>(e, acc, m0 + wave * 32, n0, li, lh, &mx, bpre, NORM ? rs : nullptr);
    if constexpr (EPI == EPI_RESIDUAL) {
        if (d.amax) {
            // one atomic per workgroup (one per wave, all on one address,
            // cost 17 us per launch of 4656 tiles); non-negative floats
            // order as their bit patterns
            __shared__ float wmax[GS_THREADS / 64];
            mx = wave_max(mx);
            if (lane == 0) wmax[wave] = mx;
            __syncthreads();
            if (tid == 0) {
#pragma unroll
                for (int w = 1; w < GS_THREADS / 64; w++) mx = fmaxf(mx, wmax[w]);
                atomicMax(reinterpret_cast<unsigned int *>(d.amax), __float_as_uint(mx));
            }
        }
    }
}

template <int EPI, bool A_H2, bool NORM = false, bool KVS = false>
__global__ __launch_bounds__(GS_THREADS, 2) void gemm_h2_kernel(GemmDescH2 d, H2Bound b) {
    gemm_h2_body<EPI, A_H2, 3, NORM, KVS>(d, b.ptr ? *b.ptr : b.value, xcd_swizzle((int)blockIdx.x, (int)gridDim.x));
}

// Ragged batch (the mask estimator's per-band linears): problem blockIdx.z,
// one bound for all problems.
struct GemmBatchH2 {
    GemmDescH2 d[GS_MAX_BATCH];
    H2Bound b;
};

template <int EPI>
__global__ __launch_bounds__(GS_THREADS, 2) void gemm_h2_batched_kernel(GemmBatchH2 b) {
    gemm_h2_body<EPI, false>(b.d[blockIdx.z], b.b.ptr ? *b.b.ptr : b.b.value, (int)blockIdx.x);
}

// max |W| over W [N][ldw] (first K columns) into out[0]; one workgroup of
// 1024 threads, no atomics.
static __global__ __launch_bounds__(1024) void absmax_kernel(const float *__restrict__ W, int N, int K, int ldw,
                                                            float *__restrict__ out) {
    __shared__ float red[16];
    float mx = 0.0f;
    const int64_t n = (int64_t)N * K;
    for (int64_t i = threadIdx.x; i < n; i += 1024) mx = fmaxf(mx, fabsf(W[(i / K) * ldw + i % K]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; w++) mx = fmaxf(mx, red[w]);
        out[0] = mx;
    }
}

// max |W| over W [N][ldw] (first K columns) raised into *out, which the
// stream zeroed before (zero_float_kernel): grid-stride over the matrix, one
// atomic max per workgroup (non-negative floats order as their bit
// patterns).  The weights' maxima at model load: one workgroup per matrix
// took 83 us each, 25 ms for a 16-layer model's 309 matrices.
static __global__ __launch_bounds__(256) void absmax_rows_kernel(const float *__restrict__ W, int N, int K, int ldw,
                                                                 float *__restrict__ out) {
    __shared__ float red[4];
    float mx = 0.0f;
    const int64_t n = (int64_t)N * K;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        mx = fmaxf(mx, fabsf(W[(i / K) * ldw + i % K]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0)
        atomicMax(reinterpret_cast<unsigned int *>(out),
                  __float_as_uint(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]))));
}

static __global__ void zero_float_kernel(float *out) { *out = 0.0f; }

// Per-workgroup max |x| over x[n] (grid-stride, 256 threads) into
// partial[blockIdx.x]; absmax_kernel over the partials finishes the reduction.
static __global__ __launch_bounds__(256) void absmax_partial_kernel(const float *__restrict__ x, int64_t n,
                                                                   float *__restrict__ partial) {
    __shared__ float red[4];
    float mx = 0.0f;
    const int64_t n4 = ((uintptr_t)x & 15) ? 0 : n / 4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const floatx4 v = ld4(x + 4 * i);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
    for (int64_t i = 4 * n4 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        mx = fmaxf(mx, fabsf(x[i]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// fp32 W [N][ldw_in] (K a multiple of 16) scaled by 2^h2_exponent(max|W|)
// (max|W| read from the header) -> its h, m fp16 pieces, tile-major: element
// (n, k) of piece p at H2_HEADER bytes plus, in fp16 units,
//   ((n/128 * K/16 + k/16) * 2 + p) * 2048 + (n%128) * 16 + 8 * (s ^ (n/8)%2) + e
// with slot s and element e from split_k_slot(k) % 16 = 8 s + e (the layout
// of split_weight_kernel with two planes).  Rows past N are zero.
static __global__ __launch_bounds__(256) void split_weight_h2_kernel(const float *__restrict__ W, int N, int K,
                                                                    int ldw_in, void *__restrict__ pieces) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int rows = (N + GS_BN - 1) / GS_BN * GS_BN;
    if (idx >= (int64_t)rows * K) return;
    const float s = ldexpf(1.0f, h2_exponent(*static_cast<const float *>(pieces)));
    const int n = (int)(idx / K), k = (int)(idx % K);
    _Float16 h = (_Float16)0.0f, m = (_Float16)0.0f;
    if (n < N) {
        const float y = W[(size_t)n * ldw_in + k] * s;
        h = (_Float16)y;
        m = (_Float16)(y - (float)h);
    }
    const int r = n % GS_BN, pos = split_k_slot(k) & 15;
    const int phys = (pos >> 3) ^ ((r >> 3) & 1);
    const size_t o = ((size_t)(n / GS_BN) * (K / GS_BK) + k / GS_BK) * H2_WBLOCK + (size_t)r * GS_BK + 8 * phys + (pos & 7);
    _Float16 *planes = reinterpret_cast<_Float16 *>(static_cast<char *>(pieces) + H2_HEADER);
    planes[o] = h;
    planes[o + GS_BN * GS_BK] = m;
}

// Bounds on the operands downstream of an RMSNorm with gain gamma[D]:
//   out[0] = sqrt(D) max|gamma|                  (|y_i| <= ||y||_2 <= out[0])
//   out[1] = t or t^2 (square), t = out[0] max_n ||W_n||_2 + max_n |b_n|
//            (a bound on every output of the linear W y + b, W [N][D]; its
//            square bounds a GELU-GLU of two such outputs); 0 without W.
// One workgroup of 1024 threads: one wave per row of W at a time.
static __global__ __launch_bounds__(1024) void operand_bounds_kernel(const float *__restrict__ gamma, int D,
                                                                    const float *__restrict__ W, int N,
                                                                    const float *__restrict__ b, int square,
                                                                    float *__restrict__ out) {
    __shared__ float red[2][16];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float g = 0.0f, nrm = 0.0f, bm = 0.0f;
    for (int i = tid; i < D; i += 1024) g = fmaxf(g, fabsf(gamma[i]));
    if (W) {
        for (int n = wave; n < N; n += 16) {
            float ss = 0.0f;
            for (int k = lane; k < D; k += 64) ss = fmaf(W[(size_t)n * D + k], W[(size_t)n * D + k], ss);
            nrm = fmaxf(nrm, sqrtf(wave_sum(ss)));
        }
        if (b)
            for (int n = tid; n < N; n += 1024) bm = fmaxf(bm, fabsf(b[n]));
    }
    g = wave_max(g);
    bm = wave_max(bm);
    if (lane == 0) {
        red[0][wave] = fmaxf(g, 0.0f);
        red[1][wave] = bm;
    }
    __shared__ float red_n[16];
    if (lane == 0) red_n[wave] = nrm;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++) {
            red[0][0] = fmaxf(red[0][0], red[0][w]);
            red[1][0] = fmaxf(red[1][0], red[1][w]);
            red_n[0] = fmaxf(red_n[0], red_n[w]);
        }
        // 1 + 2^-10 covers the rounding of the sums above
        const float in = sqrtf((float)D) * red[0][0] * (1.0f + 0x1p-10f);
        out[0] = in;
        float t = W ? (in * red_n[0] + red[1][0]) * (1.0f + 0x1p-10f) : 0.0f;
        out[1] = square ? t * t : t;
    }
}

}  // namespace vh
