// Fused axial attention in fp32 accuracy on bf16 matrix cores: the time-axis
// attention of the default fp32 path.  Same task decomposition, layout,
// rotary, online softmax and gate as attention_kernel (attention.hpp); the
// two products run as exact three-piece bf16 splits (gemm_split.hpp):
//   S^T = K * Q^T: q (rotated, scaled to the log2 domain) is split once per
//     task in registers; k (rotated) and v are split as they are staged, so
//     LDS holds their h, m, l pieces as three planes.  Per 32-key block and
//     16 head dims: six v_mfma_f32_32x32x16_bf16 (kl.qh, kh.ql, km.qm,
//     km.qh, kh.qm, kh.qh), small products first.
//   O^T += V^T * P^T: the lane's fp32 probabilities of keys
//     {16st + 4lh + 0..3, 16st + 8 + 4lh + 0..3} (registers 8st..8st+7, the
//     bf16 kernel's key order) are split in registers; six products per 16
//     keys and 32 dims.  Each V^T row stores its keys permuted inside groups
//     of 16 (keys 0-3, 8-11, 4-7, 12-15), so those eight keys are one
//     16-byte read per piece, and each thread stages two adjacent keys so the
//     transposed writes are 32-bit pairs.
// The probabilities, statistics, normalisation and gate are fp32 as in the
// fp32 kernel; the dropped piece products are below 2^-23 of each term.
#pragma once

#include "attention.hpp"
#include "attention_bf16.hpp"
#include "gemm_split.hpp"

namespace vh {

// OFF32: every row of qkv lies below 4 GB and a position step of the sequence
// is below 16 MB (the launcher checks), so the staging addresses are one
// 24-bit multiply-add from a per-lane byte offset and the SGPR base.
template <int WAVES, typename TO, bool ROPE, bool OFF32>
__global__ __launch_bounds__(64 * WAVES, 2) void attention_split_kernel(AttnArgs a) {
    if (attn_guard_skip(a)) return;
    constexpr int NT = 64 * WAVES;
    constexpr int CHUNKS = ATT_KB * ATT_DH / 8;  // 8-element chunks per K (or V) tile: 256
    constexpr int PER_T = CHUNKS / NT;
    static_assert(CHUNKS % NT == 0, "tile must divide evenly");
    __shared__ __attribute__((aligned(16))) bf16 Ks[2][3][ATT_KB][ATB_KPITCH];
    __shared__ __attribute__((aligned(16))) bf16 Vt[2][3][ATT_DH][ATB_VPITCH];

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

    // Q of query q0+li, dims 16g + 8lh .. +7, rotated, scaled (log2 domain), split.
    bf16x8 qh[4], qm[4], ql[4];
    float gate_logit = 0.0f;  // loaded with Q so the store does not wait on it
    {
        const int q = min(q0 + li, a.L - 1);
        const float *qp = qkv + (size_t)attn_row(a, s, q) * a.ld + h * ATT_DH;
        if (a.gate_col >= 0) gate_logit = qkv[(size_t)attn_row(a, s, q) * a.ld + a.gate_col + h];
        const float qs = a.scale * 1.4426950408889634f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 16 * g + 8 * lh;
            floatx4 lo = ld4(qp + d0), hi = ld4(qp + d0 + 4);
            if constexpr (ROPE) {
                lo = rope4_table(lo, a.rope, q, d0);
                hi = rope4_table(hi, a.rope, q, d0 + 4);
            }
            split8(lo * qs, hi * qs, qh[g], qm[g], ql[g]);
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
            bf16x8 p[3];
            split8(k0, k1, p[0], p[1], p[2]);
#pragma unroll
            for (int k = 0; k < 3; k++) *reinterpret_cast<bf16x8 *>(&Ks[kbk & 1][k][c >> 3][8 * (c & 7)]) = p[k];
            if (with_v) {
                // the two keys' values interleaved, so dword e of each piece is
                // the (key vk, key vk+1) pair of dim vd+e: one 32-bit write each
                const floatx4 &v0 = st.v[i][0], &v1 = st.v[i][1];
                split8(floatx4{v0[0], v1[0], v0[1], v1[1]}, floatx4{v0[2], v1[2], v0[3], v1[3]}, p[0], p[1], p[2]);
                const int vk = 2 * (c & 15), vd = 4 * (c >> 4);
                const int pos = (vk & 16) | split_k_slot(vk & 15);  // even: the pair stays adjacent
                typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
                for (int k = 0; k < 3; k++) {
                    const u32x4 w = __builtin_bit_cast(u32x4, p[k]);
#pragma unroll
                    for (int e = 0; e < 4; e++) *reinterpret_cast<uint32_t *>(&Vt[kbv & 1][k][vd + e][pos]) = w[e];
                }
            }
        }
    };
    // S^T block of 32 keys x 32 queries from Ks[kbuf]; each 16-dim group's
    // K pieces are read while the previous group's products run
    auto qk = [&](int kbuf) {
        floatx16 sc;
#pragma unroll
        for (int r = 0; r < 16; r++) sc[r] = 0.0f;
        bf16x8 kp[2][3];
        auto read = [&](int g, bf16x8 (&k)[3]) {
#pragma unroll
            for (int p = 0; p < 3; p++) k[p] = *reinterpret_cast<const bf16x8 *>(&Ks[kbuf][p][li][16 * g + 8 * lh]);
        };
        read(0, kp[0]);
#pragma unroll
        for (int g = 0; g < 4; g++) {
            if (g < 3) read(g + 1, kp[(g + 1) & 1]);
            const bf16x8 &kh = kp[g & 1][0], &km = kp[g & 1][1], &kl = kp[g & 1][2];
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(km, qm[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(km, qh[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qm[g], sc, 0, 0, 0);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[g], sc, 0, 0, 0);
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
    // computed): mask keys past L, raise the running maximum (and rescale o
    // and l) as online_softmax_block does.
    auto soft_max = [&](floatx16 &sc, int kb) {
        const int valid = a.L - kb * ATT_KB;
        if (valid < ATT_KB) {
#pragma unroll
            for (int r = 0; r < 16; r++)
                if (8 * (r >> 2) + 4 * lh + (r & 3) >= valid) sc[r] = -INFINITY;
        }
        float mb = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; r++) mb = fmaxf(mb, sc[r]);
        {
            // the other half-wave's maximum (lanes l and l^32 hold one query):
            // one v_permlane32_swap instead of an LDS permute round trip
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
            mb = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
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
#pragma unroll
        for (int r = 0; r < 16; r++) {
            sc[r] = __builtin_amdgcn_exp2f(sc[r] - m_run);
            ls += sc[r];
        }
        l_run += ls;
        // the lane's probabilities of keys 16st + {4lh..4lh+3, 8+4lh..8+4lh+3}
        // (registers 8st..8st+7) as pieces; V^T pieces for (st, t) read one
        // step ahead of their products
        bf16x8 pp[2][3];
#pragma unroll
        for (int st = 0; st < 2; st++)
            split8(floatx4{sc[8 * st], sc[8 * st + 1], sc[8 * st + 2], sc[8 * st + 3]},
                   floatx4{sc[8 * st + 4], sc[8 * st + 5], sc[8 * st + 6], sc[8 * st + 7]}, pp[st][0], pp[st][1],
                   pp[st][2]);
        bf16x8 vp[2][3];
        auto read = [&](int step, bf16x8 (&v)[3]) {
            const int st = step >> 1, t = step & 1;
#pragma unroll
            for (int k = 0; k < 3; k++)
                v[k] = *reinterpret_cast<const bf16x8 *>(&Vt[vbuf][k][32 * t + li][16 * st + 8 * lh]);
        };
        read(0, vp[0]);
#pragma unroll
        for (int step = 0; step < 4; step++) {
            if (step < 3) read(step + 1, vp[(step + 1) & 1]);
            const int st = step >> 1, t = step & 1;
            const bf16x8(&v)[3] = vp[step & 1];
            const bf16x8 &ph = pp[st][0], &pm = pp[st][1], &pl = pp[st][2];
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[2], ph, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[0], pl, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[1], pm, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[1], ph, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[0], pm, o[t], 0, 0, 0);
            o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v[0], ph, o[t], 0, 0, 0);
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
    const float inv = 1.0f / l_tot;
    const int row = attn_row(a, s, q);
    const float gate = a.gate_col >= 0 ? sigmoid_dev(gate_logit) : 1.0f;
    TO *op = static_cast<TO *>(a.out) + (size_t)row * a.ld_out + h * ATT_DH;
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

}  // namespace vh
