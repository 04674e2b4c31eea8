// Fused axial attention in fp32 accuracy on fp16 matrix cores: the
// time-axis attention of the default fp32 path.  Same task decomposition,
// layout, rotary, online softmax, gate and software pipeline as
// attention_split_kernel (attention_split.hpp); every operand is instead
// scaled by a power of two and split into two fp16 pieces (gemm_h2.hpp):
//   S^T = K * Q^T: k (rotated) times 2^ek and q (rotated, times the softmax
//     scale and log2 e) times 2^eq, so both stay below 2^14; three
//     v_mfma_f32_32x32x16_f16 per 32-key block and 16 head dims (km.qh,
//     kh.qm, kh.qh); the block's scores are scaled back by 2^-(ek+eq).
//   O^T += V^T * P^T: v times 2^ev, the probabilities (at most 2^8: the
//     running maximum is raised lazily) times 2^5; three products per 16
//     keys and 32 dims.  Both power-of-two scales ride in the exponent's
//     one FMA, p = exp2(s * 2^-(ek+eq) + 5 - m); the row sums carry the 2^5
//     as well, so normalising cancels it and the output is scaled back by
//     2^-ev only.
// The exponents come from one bound B on |q|, |k| and |v| before rotation
// (a.bound, a device float; a rotated pair keeps its 2-norm, so rotated
// values stay below sqrt(2) B).  The probabilities, statistics,
// normalisation and gate are fp32 as in the fp32 kernel.  LDS holds two
// pieces per operand (38 KB), so three workgroups share a CU: three waves per
// SIMD within 168 VGPRs (a few spilled outside the key loop; 5% faster than
// two waves per SIMD without spills).
#pragma once

#include "attention.hpp"
#include "attention_bf16.hpp"
#include "gemm_h2.hpp"

namespace vh {

// OFF32 as attention_split_kernel.  KVS: k and v arrive already scaled
// (AttnArgs::kv_scaled); rotation commutes with the power of two, so the
// pieces are the same bits.
template <int WAVES, typename TO, bool ROPE, bool OFF32, bool KVS = false>
__global__ __launch_bounds__(64 * WAVES, 3) void attention_h2_kernel(AttnArgs a) {
    if (attn_guard_skip(a)) return;
    constexpr int NT = 64 * WAVES;
    constexpr int CHUNKS = ATT_KB * ATT_DH / 8;  // 8-element chunks per K (or V) tile: 256
    constexpr int PER_T = CHUNKS / NT;
    static_assert(CHUNKS % NT == 0, "tile must divide evenly");
    __shared__ __attribute__((aligned(16))) _Float16 Ks[2][2][ATT_KB][ATB_KPITCH];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[2][2][ATT_DH][ATB_VPITCH];

    const float *qkv = static_cast<const float *>(a.qkv);
    const int qgroups = (a.L + 32 * WAVES - 1) / (32 * WAVES);
    const int task = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);  // neighbouring tasks share K/V rows: same XCD
    const int qg = task % qgroups;
    const int sh = task / qgroups;
    const int h = sh % a.H;
    const int s = sh / a.H;

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int li = lane & 31, lh = lane >> 5;
    const int q0 = (qg * WAVES + wave) * 32;

    const int kcol = a.inner + h * ATT_DH;
    const int vcol = 2 * a.inner + h * ATT_DH;

    // power-of-two scales from the bound on |q|, |k|, |v|
    const float qs = a.scale * 1.4426950408889634f;
    const float bnd = *a.bound;
    int ek, eq, ev;
    att_h2_exponents(bnd, qs, ek, eq, ev);
    constexpr int EP = 5;  // probabilities <= 2^8: 2^8 * 2^5 < 2^14
    const float k_scale = ldexpf(1.0f, ek), v_scale = ldexpf(1.0f, ev);
    const float s_unscale = ldexpf(1.0f, -(ek + eq)), o_unscale = ldexpf(1.0f, -ev);

    // Q of query q0+li, dims 16g + 8lh .. +7, rotated, scaled (log2 domain), split.
    halfx8 qh[4], qm[4];
    {
        const int q = min(q0 + li, a.L - 1);
        const float *qp = qkv + (size_t)attn_row(a, s, q) * a.ld + h * ATT_DH;
        const float q_scale = qs * ldexpf(1.0f, eq);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 16 * g + 8 * lh;
            floatx4 lo = ld4(qp + d0), hi = ld4(qp + d0 + 4);
            if constexpr (ROPE) {
                lo = rope4_table(lo, a.rope, q, d0);
                hi = rope4_table(hi, a.rope, q, d0 + 4);
            }
            split8_h2(lo, hi, q_scale, qh[g], qm[g]);
        }
    }

    // Staging.  The stage holds one K block and one V block in registers as
    // loaded (K runs one block ahead of V, below); rotation and the split
    // happen when it is written to LDS, an iteration after its loads were
    // issued, so no wait on them falls inside the iteration's MFMA work.
    // Chunk c of the K tile is key c/8, dims 8*(c%8); chunk c of the V tile
    // is keys 2*(c%16) and 2*(c%16)+1, dims 4*(c/16) .. +3.  Keys past L (and
    // blocks past the last) load the row of key L-1: no branch around the
    // loads, and nothing to zero -- their scores are masked to -inf, so their
    // probabilities are exactly 0 and their (finite) V rows add nothing.
    struct Stage {
        floatx4 k[PER_T][2], kr[PER_T][2], v[PER_T][2];
    };
    const char *qkv_b = reinterpret_cast<const char *>(qkv);
    const uint32_t row_s_bytes = (uint32_t)attn_row(a, s, 0) * (uint32_t)a.ld * 4u;  // used when OFF32
    const uint32_t pos_bytes = (uint32_t)a.pos_stride * (uint32_t)a.ld * 4u;
    auto row_ptr = [&](int p, int col) -> const float * {
        if constexpr (OFF32)
            return reinterpret_cast<const float *>(qkv_b + (__umul24((uint32_t)p, pos_bytes) + row_s_bytes + 4u * col));
        else
            return qkv + (size_t)attn_row(a, s, p) * a.ld + col;
    };
    auto load = [&](Stage &st, int kbk, int kbv) {
#pragma unroll
        for (int i = 0; i < PER_T; i++) {
            const int c = tid + NT * i;
            const int kk = c >> 3, kd = 8 * (c & 7);
            const int pkc = min(kbk * ATT_KB + kk, a.L - 1);
            const float *kp = row_ptr(pkc, kcol + kd);
            st.k[i][0] = ld4(kp);
            st.k[i][1] = ld4(kp + 4);
            if constexpr (ROPE) {
                const float *tp = reinterpret_cast<const float *>(reinterpret_cast<const char *>(a.rope) +
                                                                  (__umul24((uint32_t)pkc, 4u * ATT_DH) + 4u * kd));
                st.kr[i][0] = ld4(tp);
                st.kr[i][1] = ld4(tp + 4);
            }
            const int vk = 2 * (c & 15), vd = 4 * (c >> 4);
#pragma unroll
            for (int e = 0; e < 2; e++) st.v[i][e] = ld4(row_ptr(min(kbv * ATT_KB + vk + e, a.L - 1), vcol + vd));
        }
    };
    // rotate and split: K block kbk into Ks[kbk%2], and (with_v) V block kbv
    // transposed into Vt[kbv%2]
    auto store = [&](const Stage &st, int kbk, int kbv, bool with_v) {
#pragma unroll
        for (int i = 0; i < PER_T; i++) {
            const int c = tid + NT * i;
            floatx4 k0 = st.k[i][0], k1 = st.k[i][1];
            if constexpr (ROPE) {
                k0 = rope_pairs(k0, st.kr[i][0]);
                k1 = rope_pairs(k1, st.kr[i][1]);
            }
            halfx8 p[2];
            if constexpr (KVS) split8_h2_unit(k0, k1, p[0], p[1]);
            else split8_h2(k0, k1, k_scale, p[0], p[1]);
#pragma unroll
            for (int k = 0; k < 2; k++) *reinterpret_cast<halfx8 *>(&Ks[kbk & 1][k][c >> 3][8 * (c & 7)]) = p[k];
            if (with_v) {
                // the two keys' values interleaved, so dword e of each piece is
                // the (key vk, key vk+1) pair of dim vd+e: one 32-bit write each
                const floatx4 &v0 = st.v[i][0], &v1 = st.v[i][1];
                if constexpr (KVS)
                    split8_h2_unit(floatx4{v0[0], v1[0], v0[1], v1[1]}, floatx4{v0[2], v1[2], v0[3], v1[3]}, p[0], p[1]);
                else
                    split8_h2(floatx4{v0[0], v1[0], v0[1], v1[1]}, floatx4{v0[2], v1[2], v0[3], v1[3]}, v_scale, p[0],
                              p[1]);
                const int vk = 2 * (c & 15), vd = 4 * (c >> 4);
                const int pos = (vk & 16) | split_k_slot(vk & 15);  // even: the pair stays adjacent
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const u32x4 w = __builtin_bit_cast(u32x4, p[k]);
#pragma unroll
                    for (int e = 0; e < 4; e++) *reinterpret_cast<uint32_t *>(&Vt[kbv & 1][k][vd + e][pos]) = w[e];
                }
            }
        }
    };
    // S^T block of 32 keys x 32 queries from Ks[kbuf], still scaled by
    // 2^(ek+eq); each 16-dim group's K pieces are read while the previous
    // group's products run
    auto qk = [&](int kbuf) {
        floatx16 sc;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = 0.0f;
        halfx8 kp[2][2];
        auto read = [&](int g, halfx8 (&k)[2]) {
#pragma unroll
            for (int p = 0; p < 2; p++) k[p] = *reinterpret_cast<const halfx8 *>(&Ks[kbuf][p][li][16 * g + 8 * lh]);
        };
        read(0, kp[0]);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            if (g < 3) read(g + 1, kp[(g + 1) & 1]);
            const halfx8 &kh = kp[g & 1][0], &km = kp[g & 1][1];
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(km, qh[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qm[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[g], sc, 0, 0, 0);
        }
        return sc;
    };

    floatx16 o[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[t][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    // First half of the online softmax of block kb (its scores just
    // computed, still scaled): mask keys past L, raise the running maximum
    // (and rescale o and l) as online_softmax_block does.  The maximum is
    // taken over the scaled scores and then scaled back: exact, the scale
    // being a positive power of two.
    auto soft_max = [&](floatx16 &sc, int kb) {
        const int valid = a.L - kb * ATT_KB;
        if (valid < ATT_KB) {
            const int vl = valid - 4 * lh;  // register r holds key 8(r/4) + 4lh + r%4
#pragma unroll
            for (int r = 0; r < 16; r++)
                if (8 * (r >> 2) + (r & 3) >= vl) sc[r] = -INFINITY;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) mb = fmaxf(mb, sc[r]);
        {
            // the other half-wave's maximum (lanes l and l^32 hold one query):
            // one v_permlane32_swap instead of an LDS permute round trip
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
            mb = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * s_unscale;
        }
        const bool grow = mb > m_run + 8.0f;
        if (__ballot(grow)) {
            const float m_new = grow ? mb : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
            o[0] *= alpha;
            o[1] *= alpha;
            m_run = m_new;
        }
    };
    // Second half (probabilities, row sum) and O^T += V^T P^T from Vt[vbuf].
    auto soft_pv = [&](floatx16 &sc, int vbuf) {
        float ls = 0.0f;
        const float c = (float)EP - m_run;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            sc[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], s_unscale, c));  // 2^5 times the probability
            ls += sc[r];
        }
        l_run += ls;
        // the lane's probabilities of keys 16st + {4lh..4lh+3, 8+4lh..8+4lh+3}
        // (registers 8st..8st+7) as pieces; V^T pieces for (st, t) read one
        // step ahead of their products
        halfx8 pp[2][2];
#pragma unroll
        for (int st = 0; st < 2; st++)
            split8_h2_unit(floatx4{sc[8 * st], sc[8 * st + 1], sc[8 * st + 2], sc[8 * st + 3]},
                           floatx4{sc[8 * st + 4], sc[8 * st + 5], sc[8 * st + 6], sc[8 * st + 7]}, pp[st][0],
                           pp[st][1]);
        halfx8 vp[2][2];
        auto read = [&](int step, halfx8 (&v)[2]) {
            const int st = step >> 1, t = step & 1;
#pragma unroll
            for (int k = 0; k < 2; k++)
                v[k] = *reinterpret_cast<const halfx8 *>(&Vt[vbuf][k][32 * t + li][16 * st + 8 * lh]);
        };
        read(0, vp[0]);
#pragma unroll
        for (int step = 0; step < 4; step++) {
            if (step < 3) read(step + 1, vp[(step + 1) & 1]);
            const int st = step >> 1, t = step & 1;
            const halfx8(&v)[2] = vp[step & 1];
            const halfx8 &ph = pp[st][0], &pm = pp[st][1];
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v[1], ph, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v[0], pm, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v[0], ph, o[t], 0, 0, 0);
        }
    };

    // Pipeline over key blocks kb = 0 .. nkb-1.  Entering iteration kb:
    // Ks[(kb+1)%2] holds K(kb+1), Vt[kb%2] holds V(kb), the stage registers
    // hold the loads of K(kb+2) and V(kb+1), and S holds block kb's scores
    // with its maximum applied.  The iteration computes block kb+1's scores
    // (their MFMAs run beside block kb's exponentials), accumulates block
    // kb's P V, stages K(kb+2) into Ks[kb%2] and V(kb+1) into Vt[(kb+1)%2]
    // (read last in iteration kb-1), issues the loads of K(kb+3) and
    // V(kb+2), and after the barrier applies block kb+1's maximum.  Blocks
    // past the last are computed from staged zeros and never used.
    const int nkb = (a.L + ATT_KB - 1) / ATT_KB;
    Stage st;
    load(st, 0, 0);
    store(st, 0, 0, true);
    load(st, 1, 1);
    store(st, 1, 0, false);
    load(st, 2, 1);
    __syncthreads();
    auto run = [&](auto active_c) {
        constexpr bool ACTIVE = decltype(active_c)::value;
        floatx16 s0, s1;
        if constexpr (ACTIVE) {
            s0 = qk(0);
            soft_max(s0, 0);
        }
        __syncthreads();  // every wave has read K(0): iteration 0 restages Ks[0]
        auto iteration = [&](int kb, floatx16 &sc, floatx16 &sn) {
            if constexpr (ACTIVE) {
                sn = qk((kb + 1) & 1);
                soft_pv(sc, kb & 1);
            }
            store(st, kb + 2, kb + 1, true);
            load(st, kb + 3, kb + 2);
            if constexpr (ACTIVE) {
                // interleave the iteration's 24 MFMAs with its VALU work (block
                // kb's exponentials and splits, the staging's rotation and
                // splits): five VALU instructions after each MFMA, so the wave
                // issues them while the matrix core runs instead of after a
                // burst of MFMAs (-2.2%; four: -0.5%, six spills)
#pragma unroll
                for (int i = 0; i < 24; i++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
                }
            }
            __syncthreads();
            if constexpr (ACTIVE) {
                if (kb + 1 < nkb) soft_max(sn, kb + 1);
            }
        };
        for (int kb = 0; kb < nkb; kb += 2) {
            iteration(kb, s0, s1);
            if (kb + 1 < nkb) iteration(kb + 1, s1, s0);
        }
    };
    if (q0 < a.L) run(std::true_type());
    else {
        run(std::false_type());
        return;
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const int q = q0 + li;
    if (q >= a.L) return;
    const float inv = (1.0f / l_tot) * o_unscale;
    const int row = attn_row(a, s, q);
    // the gate logit, loaded here rather than held through the key loop
    const float gate = a.gate_col >= 0 ? sigmoid_dev(qkv[(size_t)row * a.ld + a.gate_col + h]) : 1.0f;
    TO *op = static_cast<TO *>(a.out) + (size_t)row * a.ld_out + h * ATT_DH;
    if constexpr (std::is_same<TO, float>::value) {
        if (a.out_h2) {
            // chunk c of the head's 64 dims: this lane holds dims 4lh..4lh+3
            // and 8+4lh..8+4lh+3 of it (o[c/2] quads 2(c%2), 2(c%2)+1), the
            // chunk's MFMA operand half lh: h slot lh, m slot 2+lh
            const float so = ldexpf(1.0f, h2_exponent(bnd));
            unsigned char *rowp = reinterpret_cast<unsigned char *>(op);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                floatx4 lo, hi;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    lo[r] = (o[c >> 1][8 * (c & 1) + r] * inv) * gate;
                    hi[r] = (o[c >> 1][8 * (c & 1) + 4 + r] * inv) * gate;
                }
                store8_h2_half(rowp + 64 * c, lh, lo, hi, so);
            }
            return;
        }
    }
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            floatx4 v;
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = (o[t][4 * rq + r] * inv) * gate;
            st4(op + 32 * t + 8 * rq + 4 * lh, v);
        }
}

// attention_h2_kernel on k and v that the fused projection has already
// written as fp16 pieces (GemmDescH2::kv_pieces: k rotated, both scaled by
// their attention exponents; per head 256 bytes of the row's k and v regions,
// 64 h then 64 m halves).  Nothing is computed while staging: a 32-key block
// of K (or V) is 8 KB -- two pieces of 32 rows of 128 bytes -- copied global
// -> LDS by eight 1 KB global_load_lds_dwordx4 (two per wave), with no
// registers in between.  The 16-byte chunks of an LDS row are XOR-swizzled by
// its key so the reads below touch distinct banks: K chunk c of key r at
// slot c ^ ((r >> 1) & 7) (the QK^T operand reads: 16 lanes = 16 keys, one
// chunk), V chunk c at c ^ (4 ((r >> 1) & 1)).  V stays key-major: the PV
// product's V^T operand (32 dims x 8 keys per lane) comes from
// ds_read_b64_tr_b16, which hands each lane of a 16-lane group one column of
// the 4 x 16 block (4 keys x 16 dims) the group addresses -- two reads per
// piece give the 8 keys of a lane's operand in the probabilities' key order.
// The key blocks' pipeline, softmax and output are those of
// attention_h2_kernel (same bits); only the time axis with 32-bit staging
// offsets takes this path (OFF32).
constexpr int KVP_ROW = 128;                 // bytes of one piece of one key (64 halves)
constexpr int KVP_PIECE = ATT_KB * KVP_ROW;  // 4 KB: one piece of a 32-key block
VH_DEVICE int kvp_swz_k(int r) { return (r >> 1) & 7; }
VH_DEVICE int kvp_swz_v(int r) { return 4 * ((r >> 1) & 1); }

template <int WAVES>
__global__ __launch_bounds__(64 * WAVES, 3) void attention_h2_kvp_kernel(AttnArgs a) {
    static_assert(WAVES == 4, "two DMA loads per wave and operand");
    __shared__ __attribute__((aligned(1024))) unsigned char Ks[2][2][KVP_PIECE];
    __shared__ __attribute__((aligned(1024))) unsigned char Vs[2][2][KVP_PIECE];

    const float *qkv = static_cast<const float *>(a.qkv);
    const int qgroups = (a.L + 32 * WAVES - 1) / (32 * WAVES);
    const int task = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);  // neighbouring tasks share K/V rows: same XCD
    const int qg = task % qgroups;
    const int sh = task / qgroups;
    const int h = sh % a.H;
    const int s = sh / a.H;

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int li = lane & 31, lh = lane >> 5;
    const int q0 = (qg * WAVES + wave) * 32;

    const float qs = a.scale * 1.4426950408889634f;
    const float bnd = *a.bound;
    int ek, eq, ev;
    att_h2_exponents(bnd, qs, ek, eq, ev);
    constexpr int EP = 5;
    const float s_unscale = ldexpf(1.0f, -(ek + eq)), o_unscale = ldexpf(1.0f, -ev);

    halfx8 qh[4], qm[4];
    {
        const int q = min(q0 + li, a.L - 1);
        const float *qp = qkv + (size_t)attn_row(a, s, q) * a.ld + h * ATT_DH;
        const float q_scale = qs * ldexpf(1.0f, eq);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 16 * g + 8 * lh;
            floatx4 lo = ld4(qp + d0), hi = ld4(qp + d0 + 4);
            lo = rope4_table(lo, a.rope, q, d0);
            hi = rope4_table(hi, a.rope, q, d0 + 4);
            split8_h2(lo, hi, q_scale, qh[g], qm[g]);
        }
    }

    // DMA staging.  Load i (0..7) of a block copies piece i / 4, keys
    // 8 (i % 4) .. +7 of the block: lane l writes LDS bytes 16 l of the 1 KB,
    // i.e. key 8 (i % 4) + l / 8, slot l % 8, and reads that key's chunk
    // (l % 8) ^ swz from global memory.  Wave w issues loads w and w + 4 of K
    // and of V.  Keys past L load the row of key L-1 (their scores are masked,
    // their probabilities exactly 0).  32-bit offsets from the sequence's
    // first row (the launcher checks they fit).
    const char *seq_base = reinterpret_cast<const char *>(qkv) + (size_t)attn_row(a, s, 0) * a.ld * 4u;
    const uint32_t pos_bytes = (uint32_t)a.pos_stride * (uint32_t)a.ld * 4u;
    const int kr = 8 * (wave & 3) + (lane >> 3);  // the lane's key within the block (both of its loads)
    const uint32_t k_off = 4u * (uint32_t)a.inner + 256u * (uint32_t)h + 16u * (uint32_t)((lane & 7) ^ kvp_swz_k(kr));
    const uint32_t v_off = 8u * (uint32_t)a.inner + 256u * (uint32_t)h + 16u * (uint32_t)((lane & 7) ^ kvp_swz_v(kr));
    const uint32_t ks_base = (uint32_t)(uintptr_t)&Ks[0][0][0], vs_base = (uint32_t)(uintptr_t)&Vs[0][0][0];
    auto issue_k = [&](int kb) {
        const uint32_t row = (uint32_t)min(kb * ATT_KB + kr, a.L - 1) * pos_bytes;
#pragma unroll
        for (int p = 0; p < 2; p++)
            lds_dma16s(row + k_off + KVP_ROW * p, seq_base,
                       ks_base + (uint32_t)(((kb & 1) * 2 + p) * KVP_PIECE + 1024 * (wave & 3)));
    };
    auto issue_v = [&](int kb) {
        const uint32_t row = (uint32_t)min(kb * ATT_KB + kr, a.L - 1) * pos_bytes;
#pragma unroll
        for (int p = 0; p < 2; p++)
            lds_dma16s(row + v_off + KVP_ROW * p, seq_base,
                       vs_base + (uint32_t)(((kb & 1) * 2 + p) * KVP_PIECE + 1024 * (wave & 3)));
    };

    // S^T block from Ks[kbuf], still scaled by 2^(ek+eq)
    auto qk = [&](int kbuf) {
        floatx16 sc;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = 0.0f;
        const unsigned char *kb0 = &Ks[kbuf][0][0] + li * KVP_ROW;
        halfx8 kp[2][2];
        auto read = [&](int g, halfx8 (&k)[2]) {
            const int slot = (2 * g + lh) ^ kvp_swz_k(li);
#pragma unroll
            for (int p = 0; p < 2; p++) k[p] = *reinterpret_cast<const halfx8 *>(kb0 + p * KVP_PIECE + 16 * slot);
        };
        read(0, kp[0]);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            if (g < 3) read(g + 1, kp[(g + 1) & 1]);
            const halfx8 &kh = kp[g & 1][0], &km = kp[g & 1][1];
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(km, qh[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qm[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kh, qh[g], sc, 0, 0, 0);
        }
        return sc;
    };

    floatx16 o[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[t][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    auto soft_max = [&](floatx16 &sc, int kb) {
        const int valid = a.L - kb * ATT_KB;
        if (valid < ATT_KB) {
            const int vl = valid - 4 * lh;
#pragma unroll
            for (int r = 0; r < 16; r++)
                if (8 * (r >> 2) + (r & 3) >= vl) sc[r] = -INFINITY;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) mb = fmaxf(mb, sc[r]);
        {
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
            mb = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])) * s_unscale;
        }
        const bool grow = mb > m_run + 8.0f;
        if (__ballot(grow)) {
            const float m_new = grow ? mb : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
            o[0] *= alpha;
            o[1] *= alpha;
            m_run = m_new;
        }
    };
    // V^T operand rows: lane (group g = lane / 16, j = lane % 16) addresses
    // key 4 lh + j / 4 (+ 8 for the second read) of the step's 16 keys, dims
    // 16 (g % 2) + 4 (j % 4) .. +3 of the 32 of tile t
    typedef __fp16 fp16x4 __attribute__((ext_vector_type(4)));
    const int tr_j = lane & 15, tr_dhalf = (lane >> 4) & 1;
    auto soft_pv = [&](floatx16 &sc, int vbuf) {
        float ls = 0.0f;
        const float c = (float)EP - m_run;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            sc[r] = __builtin_amdgcn_exp2f(fmaf(sc[r], s_unscale, c));
            ls += sc[r];
        }
        l_run += ls;
        halfx8 pp[2][2];
#pragma unroll
        for (int st = 0; st < 2; st++)
            split8_h2_unit(floatx4{sc[8 * st], sc[8 * st + 1], sc[8 * st + 2], sc[8 * st + 3]},
                           floatx4{sc[8 * st + 4], sc[8 * st + 5], sc[8 * st + 6], sc[8 * st + 7]}, pp[st][0],
                           pp[st][1]);
        halfx8 vp[2][2];
        auto read = [&](int step, halfx8 (&v)[2]) {
            const int st = step >> 1, t = step & 1;
            const int key = 16 * st + 4 * lh + (tr_j >> 2);
            const int chunk = 4 * t + 2 * tr_dhalf + ((tr_j & 3) >> 1);
            const int byte = 8 * (tr_j & 1);
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const unsigned char *base = &Vs[vbuf][p][0];
                const unsigned char *a0 = base + key * KVP_ROW + 16 * (chunk ^ kvp_swz_v(key)) + byte;
                const unsigned char *a1 = base + (key + 8) * KVP_ROW + 16 * (chunk ^ kvp_swz_v(key + 8)) + byte;
                const fp16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (__attribute__((address_space(3))) fp16x4 *)(a0));
                const fp16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
                    (__attribute__((address_space(3))) fp16x4 *)(a1));
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
                const u32x2 w0 = __builtin_bit_cast(u32x2, r0), w1 = __builtin_bit_cast(u32x2, r1);
                v[p] = __builtin_bit_cast(halfx8, u32x4{w0[0], w0[1], w1[0], w1[1]});
            }
        };
        read(0, vp[0]);
#pragma unroll
        for (int step = 0; step < 4; step++) {
            if (step < 3) read(step + 1, vp[(step + 1) & 1]);
            const int st = step >> 1, t = step & 1;
            const halfx8(&v)[2] = vp[step & 1];
            const halfx8 &ph = pp[st][0], &pm = pp[st][1];
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v[1], ph, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v[0], pm, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(v[0], ph, o[t], 0, 0, 0);
        }
    };

    // Pipeline as attention_h2_kernel: entering iteration kb, Ks[(kb+1)%2]
    // holds K(kb+1) and Vs[kb%2] holds V(kb); the iteration issues K(kb+2)
    // into Ks[kb%2] (read last by block kb's scores, before the barrier that
    // ended the previous iteration) and V(kb+1) into Vs[(kb+1)%2], computes
    // block kb+1's scores and block kb's P V, and waits for its copies before
    // the barrier that ends it.
    const int nkb = (a.L + ATT_KB - 1) / ATT_KB;
    issue_k(0);
    issue_v(0);
    issue_k(1);
    wait_vmcnt<0>();
    __syncthreads();
    auto run = [&](auto active_c) {
        constexpr bool ACTIVE = decltype(active_c)::value;
        floatx16 s0, s1;
        if constexpr (ACTIVE) {
            s0 = qk(0);
            soft_max(s0, 0);
        }
        __syncthreads();  // every wave has read K(0): iteration 0 copies K(2) there
        auto iteration = [&](int kb, floatx16 &sc, floatx16 &sn) {
            issue_k(kb + 2);
            issue_v(kb + 1);
            if constexpr (ACTIVE) {
                sn = qk((kb + 1) & 1);
                soft_pv(sc, kb & 1);
            }
            wait_vmcnt<0>();
            __syncthreads();
            if constexpr (ACTIVE) {
                if (kb + 1 < nkb) soft_max(sn, kb + 1);
            }
        };
        for (int kb = 0; kb < nkb; kb += 2) {
            iteration(kb, s0, s1);
            if (kb + 1 < nkb) iteration(kb + 1, s1, s0);
        }
    };
    if (q0 < a.L) run(std::true_type());
    else {
        run(std::false_type());
        return;
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32, 64);
    const int q = q0 + li;
    if (q >= a.L) return;
    const float inv = (1.0f / l_tot) * o_unscale;
    const int row = attn_row(a, s, q);
    const float gate = a.gate_col >= 0 ? sigmoid_dev(qkv[(size_t)row * a.ld + a.gate_col + h]) : 1.0f;
    float *op = static_cast<float *>(a.out) + (size_t)row * a.ld_out + h * ATT_DH;
    if (a.out_h2) {
        const float so = ldexpf(1.0f, h2_exponent(bnd));
        unsigned char *rowp = reinterpret_cast<unsigned char *>(op);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            floatx4 lo, hi;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                lo[r] = (o[c >> 1][8 * (c & 1) + r] * inv) * gate;
                hi[r] = (o[c >> 1][8 * (c & 1) + 4 + r] * inv) * gate;
            }
            store8_h2_half(rowp + 64 * c, lh, lo, hi, so);
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            floatx4 v;
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = (o[t][4 * rq + r] * inv) * gate;
            st4(op + 32 * t + 8 * rq + 4 * lh, v);
        }
}

// Short sequences (L <= 64: the band axis) in fp32 accuracy on the fp16
// matrix cores: the persistent task loop, prefetch, query layout and
// single-pass softmax of attention_short_kernel (attention.hpp), with every
// product as three v_mfma_f32_16x16x32_f16 on two-piece operands scaled as in
// attention_h2_kernel (the probabilities are at most 1 here: scale 2^13).  A
// lane of a 16x16x32 MFMA supplies eight k-values, assigned to (lane group,
// slot) the same way for both operands, so the summed index may be relabelled
// freely as long as both operands agree:
//   S^T tile kt = K * Q^T, step s (head dims 32s..32s+31): slot 4c + e of
//     lane group g is dim 32s + 16c + 4g + e -- the lane's own rotated q
//     registers j = 2s + c -- and LDS holds each key's pieces in that order
//     (position 8(4s + g) + 4c + e), so a lane reads 16 bytes per piece.
//   O^T tile dt += V^T * P^T, step u (keys 32u..32u+31): slot 4c + r of lane
//     group g is key 32u + 16c + 4g + r -- the lane's own probabilities
//     sc[2u + c][r] -- and LDS holds V transposed, keys in that order; tile
//     row m is dim m + 16 dt, so lane (n, g) ends with dims 16 dt + 4g + r
//     (one 16-byte store per tile).
// LDS rows are 72 halves (36 dwords): the 16 rows one read touches fall on
// distinct 4-bank groups.  Two pieces of K and of V^T: 36 KB, four
// workgroups per CU.
VH_DEVICE void split4_h2(floatx4 v, float s, uint32_t &h01, uint32_t &h23, uint32_t &m01, uint32_t &m23) {
    h01 = pack_f16x2(v[0] * s, v[1] * s);
    h23 = pack_f16x2(v[2] * s, v[3] * s);
    m01 = m_pair_f16(v[0], v[1], s, h01);
    m23 = m_pair_f16(v[2], v[3], s, h23);
}
// The same for values already scaled (one: opaque_one()).
VH_DEVICE void split4_h2_unit(floatx4 v, float one, uint32_t &h01, uint32_t &h23, uint32_t &m01, uint32_t &m23) {
    h01 = pack_f16x2(v[0], v[1]);
    h23 = pack_f16x2(v[2], v[3]);
    m01 = m_pair_f16(v[0], v[1], one, h01);
    m23 = m_pair_f16(v[2], v[3], one, h23);
}

// KVS as attention_h2_kernel.
template <typename TO, bool KVS = false>
__global__ __launch_bounds__(256, 4) void attention_short_h2_kernel(AttnArgs a) {
    if (attn_guard_skip(a)) return;
    constexpr int KEYS = 64;
    constexpr int PITCH = ATT_DH + 8;
    __shared__ __attribute__((aligned(16))) _Float16 Kp[2][KEYS][PITCH];
    __shared__ __attribute__((aligned(16))) _Float16 Vp[2][ATT_DH][PITCH];
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

    const float *qkv = static_cast<const float *>(a.qkv);
    const int tasks = a.S * a.H;
    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int q = 16 * wave + n;
    const int qc = min(q, a.L - 1);
    // staging: K keys tid/16 + 16i with dims d_st..d_st+3; V keys vk, vk + 1
    // with dims vd..vd+3 and vd+32..vd+35
    const int d_st = 4 * (tid & 15);
    const int k_pos = 8 * (4 * (d_st >> 5) + ((d_st >> 2) & 3)) + 4 * ((d_st >> 4) & 1);
    const int vk = 2 * (tid & 31), vd = 4 * (tid >> 5);
    const int v_pos = 8 * (4 * (vk >> 5) + ((vk >> 2) & 3)) + 4 * ((vk >> 4) & 1) + (vk & 3);

    // power-of-two scales from the bound on |q|, |k|, |v|
    const float qs = a.scale * 1.4426950408889634f;
    const float bnd = *a.bound;
    const int ek = h2_exponent(1.4142135f * 1.0001f * bnd);
    const int eq = h2_exponent(1.4142135f * 1.0001f * bnd * qs);
    const int ev = h2_exponent(bnd);
    constexpr int EP = 13;  // probabilities <= 1: 2^13 < 2^14
    const float k_scale = ldexpf(1.0f, ek), v_scale = ldexpf(1.0f, ev), q_scale = qs * ldexpf(1.0f, eq);
    const float s_unscale = ldexpf(1.0f, -(ek + eq)), o_unscale = ldexpf(1.0f, -(ev + EP)), p_scale = ldexpf(1.0f, EP);
    const float one = opaque_one();  // KVS: the unit scale of the m pieces

    floatx4 kpre[4], vpre[4], qpre[4];
    float gpre = 0.0f;
    auto prefetch = [&](int task) {
        const int h = task % a.H, s = task / a.H;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = (tid >> 4) + 16 * i;
            kpre[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (key < a.L) kpre[i] = ld4(qkv + (size_t)attn_row(a, s, key) * a.ld + a.inner + h * ATT_DH + d_st);
            const int vkey = vk + (i & 1);
            vpre[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (vkey < a.L)
                vpre[i] = ld4(qkv + (size_t)attn_row(a, s, vkey) * a.ld + 2 * a.inner + h * ATT_DH + vd + 32 * (i >> 1));
        }
        const size_t qrow = (size_t)attn_row(a, s, qc) * a.ld;
#pragma unroll
        for (int j = 0; j < 4; j++) qpre[j] = ld4(qkv + qrow + h * ATT_DH + 16 * j + 4 * g);
        if (a.gate_col >= 0) gpre = qkv[qrow + a.gate_col + h];
    };

    const int per = (tasks + (int)gridDim.x - 1) / (int)gridDim.x;
    const int t_end = min(tasks, ((int)blockIdx.x + 1) * per);
    int task = (int)blockIdx.x * per;
    if (task < t_end) prefetch(task);
    for (; task < t_end; task++) {
        const int h = task % a.H, s = task / a.H;
        // keys past L are zeros, rotated with the table's last row
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = (tid >> 4) + 16 * i;
            uint32_t h01, h23, m01, m23;
            if constexpr (KVS) split4_h2_unit(rope4(kpre[i], a.rope, min(key, a.L - 1), d_st), one, h01, h23, m01, m23);
            else split4_h2(rope4(kpre[i], a.rope, min(key, a.L - 1), d_st), k_scale, h01, h23, m01, m23);
            *reinterpret_cast<u32x2 *>(&Kp[0][key][k_pos]) = u32x2{h01, h23};
            *reinterpret_cast<u32x2 *>(&Kp[1][key][k_pos]) = u32x2{m01, m23};
        }
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float x0 = vpre[2 * c][e], x1 = vpre[2 * c + 1][e];
                const uint32_t hp = KVS ? pack_f16x2(x0, x1) : pack_f16x2(x0 * v_scale, x1 * v_scale);
                const uint32_t mp = m_pair_f16(x0, x1, KVS ? one : v_scale, hp);
                const int dim = vd + 32 * c + e;
                *reinterpret_cast<uint32_t *>(&Vp[0][dim][v_pos]) = hp;
                *reinterpret_cast<uint32_t *>(&Vp[1][dim][v_pos]) = mp;
            }
        halfx8 qh[2], qm[2];
#pragma unroll
        for (int st = 0; st < 2; st++)
            split8_h2(rope4(qpre[2 * st], a.rope, qc, 32 * st + 4 * g),
                      rope4(qpre[2 * st + 1], a.rope, qc, 32 * st + 16 + 4 * g), q_scale, qh[st], qm[st]);
        const float gate_logit = gpre;
        __syncthreads();
        if (task + 1 < t_end) prefetch(task + 1);

        floatx4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            sc[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const halfx8 kh = *reinterpret_cast<const halfx8 *>(&Kp[0][16 * kt + n][8 * (4 * st + g)]);
                const halfx8 km = *reinterpret_cast<const halfx8 *>(&Kp[1][16 * kt + n][8 * (4 * st + g)]);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(km, qh[st], sc[kt], 0, 0, 0);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qm[st], sc[kt], 0, 0, 0);
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kh, qh[st], sc[kt], 0, 0, 0);
            }
            sc[kt] = sc[kt] * s_unscale;  // exact: a power of two
        }
        float m = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (16 * kt + 4 * g + r >= a.L) sc[kt][r] = -INFINITY;
                m = fmaxf(m, sc[kt][r]);
            }
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float l = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                sc[kt][r] = __builtin_amdgcn_exp2f(sc[kt][r] - m);
                l += sc[kt][r];
            }
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);

        floatx4 o[4];
#pragma unroll
        for (int dt = 0; dt < 4; dt++) o[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 2; u++) {
            halfx8 ph, pm;
            split8_h2(sc[2 * u], sc[2 * u + 1], p_scale, ph, pm);
#pragma unroll
            for (int dt = 0; dt < 4; dt++) {
                const halfx8 vh = *reinterpret_cast<const halfx8 *>(&Vp[0][n + 16 * dt][8 * (4 * u + g)]);
                const halfx8 vm = *reinterpret_cast<const halfx8 *>(&Vp[1][n + 16 * dt][8 * (4 * u + g)]);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vm, ph, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, pm, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vh, ph, o[dt], 0, 0, 0);
            }
        }

        if (q < a.L) {
            const float f = (1.0f / l) * (a.gate_col >= 0 ? sigmoid_dev(gate_logit) : 1.0f) * o_unscale;
            TO *op = static_cast<TO *>(a.out) + (size_t)attn_row(a, s, q) * a.ld_out + h * ATT_DH + 4 * g;
            bool done = false;
            if constexpr (std::is_same<TO, float>::value) {
                if (a.out_h2) {
                    // dims 16dt + 4g .. +3: group g of chunk dt, whose groups
                    // g^2 lies in lane ^ 32 (the same query)
                    const float so = ldexpf(1.0f, h2_exponent(bnd));
                    unsigned char *rowp = reinterpret_cast<unsigned char *>(op - 4 * g);
#pragma unroll
                    for (int dt = 0; dt < 4; dt++) store4_h2_swap<32>(rowp + 64 * dt, g, o[dt] * f, so);
                    done = true;
                }
            }
            if (!done) {
#pragma unroll
                for (int dt = 0; dt < 4; dt++) st4(op + 16 * dt, o[dt] * f);
            }
        }
        __syncthreads();  // LDS is refilled for the next task
    }
}

}  // namespace vh
