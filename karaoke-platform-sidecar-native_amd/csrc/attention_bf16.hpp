// Fused axial attention on bf16 matrix cores: the bf16 variant of
// attention_kernel (attention.hpp), same task decomposition, layout and
// online softmax, with q, k, v and the probabilities as bf16 MFMA operands
// and fp32 accumulation, statistics and normalisation.
//
// q/k/v/gates come from the bf16 fused projection (rows as in attention.hpp).
// q and k are rotated in fp32 (host-built cos/sin table) and rounded to bf16;
// q is also scaled by scale*log2(e) before rounding.
//
// Per wavefront: 32 queries.  Per block of 32 keys:
//   S^T = K * Q^T: 4 x v_mfma_f32_32x32x16_bf16 over the 64 head dims (A = K
//     rows from LDS, B = the wave's Q held in registers).  Lane (li, lh)
//     receives the scores of query li for keys 8*(r/4) + 4*lh + r%4.
//   O^T += V^T * P^T: per 16-key step st the lane's own registers
//     8st .. 8st+7 are the probabilities of keys {16st + 4lh + 0..3,
//     16st + 8 + 4lh + 0..3}: converted to bf16 they are the B operand as
//     they stand, and the A operand (V^T rows from LDS) is read in the same
//     key order (two 8-byte reads).
#pragma once

#include "attention.hpp"
#include "common.hpp"

namespace vh {

constexpr int ATB_KPITCH = ATT_DH + 8;  // K tile row pitch (bf16): 144 B, conflict-free 16-byte reads
constexpr int ATB_VPITCH = ATT_KB + 8;  // V^T tile row pitch (bf16)

VH_DEVICE floatx4 lo4(bf16x8 v) { return floatx4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]}; }
VH_DEVICE floatx4 hi4(bf16x8 v) { return floatx4{(float)v[4], (float)v[5], (float)v[6], (float)v[7]}; }

// Rotate the four interleaved pairs of 8 dims starting at d0 (fp32), scale,
// round to bf16.
VH_DEVICE bf16x8 rope8_bf16(bf16x8 v, const float *tab, int pos, int d0, float scale) {
    floatx4 a = rope4(lo4(v), tab, pos, d0) * scale;
    floatx4 b = rope4(hi4(v), tab, pos, d0 + 4) * scale;
    bf16x8 r;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        r[e] = (bf16)a[e];
        r[4 + e] = (bf16)b[e];
    }
    return r;
}

template <int WAVES, typename TO>
__global__ __launch_bounds__(64 * WAVES, 4) void attention_bf16_kernel(AttnArgs a) {
    constexpr int NT = 64 * WAVES;
    constexpr int CHUNKS = ATT_KB * ATT_DH / 8;  // 16-byte chunks per K (or V) tile: 256
    constexpr int PER_T = CHUNKS / NT;
    static_assert(CHUNKS % NT == 0, "tile must divide evenly");
    __shared__ __attribute__((aligned(16))) bf16 Ks[2][ATT_KB][ATB_KPITCH];
    __shared__ __attribute__((aligned(16))) bf16 Vt[2][ATT_DH][ATB_VPITCH];

    const bf16 *qkv = static_cast<const bf16 *>(a.qkv);
    const int qgroups = (a.L + 32 * WAVES - 1) / (32 * WAVES);
    const int task = xcd_swizzle((int)blockIdx.x, (int)gridDim.x);  // neighbouring tasks share K/V rows: same XCD
    const int qg = task % qgroups;
    const int sh = task / qgroups;
    const int h = sh % a.H;
    const int s = sh / a.H;

    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int li = lane & 31, lh = lane >> 5;
    const int q0 = (qg * WAVES + wave) * 32;
    const bool wave_active = q0 < a.L;

    const int kcol = a.inner + h * ATT_DH;
    const int vcol = 2 * a.inner + h * ATT_DH;

    // Q of query q0+li, dims 16g + 8lh .. +7, rotated and scaled (log2 domain).
    bf16x8 qb[4];
    float gate_logit = 0.0f;  // loaded with Q so the store does not wait on it
    {
        const int q = min(q0 + li, a.L - 1);
        const bf16 *qp = qkv + (size_t)attn_row(a, s, q) * a.ld + h * ATT_DH;
        if (a.gate_col >= 0) gate_logit = (float)qkv[(size_t)attn_row(a, s, q) * a.ld + a.gate_col + h];
        const float qs = a.scale * 1.4426950408889634f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = 16 * g + 8 * lh;
            qb[g] = rope8_bf16(*reinterpret_cast<const bf16x8 *>(qp + d0), a.rope, q, d0, qs);
        }
    }

    // Staging: chunk c of the K tile is key c/8, dims 8*(c%8) (8 threads read
    // one key's 128 contiguous bytes); chunk c of the V tile is key c%32, dims
    // 8*(c/32), so a wave's V^T column writes spread over the banks.
    bf16x8 kreg[PER_T], vreg[PER_T];
    auto load = [&](int kb) {
#pragma unroll
        for (int i = 0; i < PER_T; i++) {
            const int c = tid + NT * i;
            const int kk = c >> 3, kd = 8 * (c & 7);
            const int vk = c & 31, vd = 8 * (c >> 5);
            const int pk = kb * ATT_KB + kk, pv = kb * ATT_KB + vk;
            if (pk < a.L) {
                const bf16 *kp = qkv + (size_t)attn_row(a, s, pk) * a.ld + kcol + kd;
                kreg[i] = rope8_bf16(*reinterpret_cast<const bf16x8 *>(kp), a.rope, pk, kd, 1.0f);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) kreg[i][e] = (bf16)0.0f;
            }
            if (pv < a.L) {
                vreg[i] = *reinterpret_cast<const bf16x8 *>(qkv + (size_t)attn_row(a, s, pv) * a.ld + vcol + vd);
            } else {
#pragma unroll
                for (int e = 0; e < 8; e++) vreg[i][e] = (bf16)0.0f;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER_T; i++) {
            const int c = tid + NT * i;
            *reinterpret_cast<bf16x8 *>(&Ks[buf][c >> 3][8 * (c & 7)]) = kreg[i];
            const int vk = c & 31, vd = 8 * (c >> 5);
#pragma unroll
            for (int e = 0; e < 8; e++) Vt[buf][vd + e][vk] = vreg[i][e];
        }
    };

    floatx16 o[2];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[t][r] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;

    const int nkb = (a.L + ATT_KB - 1) / ATT_KB;
    load(0);
    store(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; kb++) {
        const int buf = kb & 1;
        if (kb + 1 < nkb) load(kb + 1);
        if (wave_active) {
            floatx16 sc;
#pragma unroll
            for (int r = 0; r < 16; r++) sc[r] = 0.0f;
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const bf16x8 kf = *reinterpret_cast<const bf16x8 *>(&Ks[buf][li][16 * g + 8 * lh]);
                sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qb[g], sc, 0, 0, 0);
            }
            const int valid = a.L - kb * ATT_KB;
            if (valid < ATT_KB) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (8 * (r >> 2) + 4 * lh + (r & 3) >= valid) sc[r] = -INFINITY;
            }
            online_softmax_block(sc, m_run, l_run, o);
#pragma unroll
            for (int st = 0; st < 2; st++) {
                bf16x8 pb;
#pragma unroll
                for (int e = 0; e < 8; e++) pb[e] = (bf16)sc[8 * st + e];
#pragma unroll
                for (int t = 0; t < 2; t++) {
                    const bf16 *vr = &Vt[buf][32 * t + li][16 * st + 4 * lh];
                    const bf16x4 v0 = *reinterpret_cast<const bf16x4 *>(vr);
                    const bf16x4 v1 = *reinterpret_cast<const bf16x4 *>(vr + 8);
                    const bf16x8 va = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
                    o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, o[t], 0, 0, 0);
                }
            }
        }
        if (kb + 1 < nkb) store(buf ^ 1);
        __syncthreads();
    }

    if (!wave_active) return;
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
