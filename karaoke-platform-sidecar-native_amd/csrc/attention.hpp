// Fused axial attention on CDNA4 fp32 matrix cores.
//
// Computes, for every (sequence, head, query), the softmax-weighted sum over
// all keys of one axial sequence, with the rotary embedding applied to q and
// k as they are loaded and the per-head sigmoid gate applied at the store.
// This is the whole of native/vocalarc_separation.c:692-818 (rotary,
// attention_heads, apply_gates) for one transformer in one launch; the
// reference CUDA provider spends 5 launches and a materialised score matrix
// on it (native/native_gpu_cuda.cu:497-538).
//
// Layout: q, k, v and the gate logits live in one row per token of the fused
// QKV(+gate) projection (q at column 0, k at `inner`, v at 2*inner, gates at
// `gate_col`).  A token of sequence s at position p sits in row
//   (s / group) * group_stride + (s % group) * seq_stride + p * pos_stride,
// so the same kernel reads the time axis and the band axis of one physical
// [frames][bands] activation tensor without a transpose.
//
// Per wavefront: 32 queries.  For each block of 32 keys the wave computes
// S^T = K * Q^T with v_mfma_f32_32x32x2f32, which leaves every lane holding
// 16 scores of ONE query (rows = keys).  The online-softmax statistics are
// therefore lane-local plus one exchange with the partner half-wave, and the
// probabilities are already in the B-operand layout of O^T += V^T * P^T: step
// s of that MFMA consumes register s.  V is staged transposed in LDS so its
// A operand is one ds_read_b128 per four MFMAs.
#pragma once

#include "common.hpp"
#include "h2.hpp"

namespace vh {

struct AttnArgs {
    const void *qkv;   // fused projection rows (fp32, or bf16 for the bf16 kernel)
    int ld;            // row pitch of qkv (floats)
    void *out;         // [rows][ld_out] fp32 or bf16, head h at column h*64
    int ld_out;
    const float *rope;  // [L][32][2] (cos, sin) pairs, may be null (no rotary)
    int S, L, H;
    int group, group_stride, seq_stride, pos_stride;
    int inner;      // H * 64
    int gate_col;   // < 0: no gates
    float scale;    // 1/sqrt(64)
    const float *bound;  // device bound on |q|, |k|, |v| (attention_h2_kernel only)
    // fp32 out written as h2 rows (h2.hpp) scaled by 2^h2_exponent(*bound):
    // the out projection's A operand, split here once instead of in each of
    // its column tiles (the fp16 two-piece kernels only)
    int out_h2;
    // the k and v columns of qkv arrive multiplied by 2^ek and 2^ev
    // (att_h2_exponents of *bound), as the fused projection writes them: the
    // staging splits them without scaling (the fp16 two-piece kernels only)
    int kv_scaled;
    // Range choice on the device (null: none).  The kernel runs only when
    // h2_attention_bound_ok(*guard) equals guard_h2 and otherwise returns at
    // once: the two-piece kernel launched with guard_h2 = 1 and the kernel
    // without piece scales with guard_h2 = 0 on the same bound compute the
    // attention once between them, with no read-back of the bound.
    const float *guard;
    int guard_h2;
    // k and v arrive as the fused projection's fp16 pieces
    // (GemmDescH2::kv_pieces; attention_h2_kvp_kernel)
    int kv_pieces;
};

constexpr int ATT_DH = 64;
constexpr int ATT_KB = 32;             // keys per iteration
constexpr int ATT_KPITCH = ATT_DH + 4; // K tile row pitch (floats)
constexpr int ATT_VPITCH = ATT_KB + 4; // V^T tile row pitch (floats)

// Whether a guarded launch (AttnArgs::guard) has nothing to do.
VH_DEVICE bool attn_guard_skip(const AttnArgs &a) {
    return a.guard && h2_attention_bound_ok(*a.guard) != (a.guard_h2 != 0);
}

VH_DEVICE int attn_row(const AttnArgs &a, int s, int p) {
    return (s / a.group) * a.group_stride + (s % a.group) * a.seq_stride + p * a.pos_stride;
}

// Rotate the two interleaved pairs of a float4 by t = (cos, sin) of each
// pair; rope4_table reads t for the float4 at dimension d0 of position pos
// from the table (one 16-byte load).  Explicit fused forms, the same in every
// kernel that rotates and symmetric in the pair: element e of a pair is
// fma(x_e, cos, x_other * (e ? sin : -sin)) (the reference's
// first*c - second*s, first*s + second*c, native/vocalarc_separation.c:
// 705-706, with the product of the element itself fused), so a lane holding
// one element and its partner's (rope_own) rounds as a lane holding both.
VH_DEVICE float rope_own(float own, float other, float c, float s_signed) {
    return __builtin_fmaf(own, c, other * s_signed);
}
VH_DEVICE floatx4 rope_pairs(floatx4 v, floatx4 t) {
    const float c0 = t[0], s0 = t[1], c1 = t[2], s1 = t[3];
    floatx4 r;
    r[0] = rope_own(v[0], v[1], c0, -s0);
    r[1] = rope_own(v[1], v[0], c0, s0);
    r[2] = rope_own(v[2], v[3], c1, -s1);
    r[3] = rope_own(v[3], v[2], c1, s1);
    return r;
}
VH_DEVICE floatx4 rope4_table(floatx4 v, const float *tab, int pos, int d0) {
    return rope_pairs(v, ld4(tab + pos * ATT_DH + d0));
}
VH_DEVICE floatx4 rope4(floatx4 v, const float *tab, int pos, int d0) {
    return tab == nullptr ? v : rope4_table(v, tab, pos, d0);
}

// Workgroup: WAVES wavefronts x 32 queries of one (sequence, head).  Each
// iteration stages 32 keys (K rows and V transposed) in LDS, double
// buffered (35 KB, so several workgroups share a CU).  Staging map: thread e
// loads key e%16 (+16 for e >= 256) and 16-byte chunk (e/16)%16 of that key's
// 64 dims, which makes both the K row writes and the V column writes
// bank-conflict free.
// One 32-key block of the online softmax for the lane's query: sc holds its
// scores (log2 domain) on entry and the unnormalised probabilities on exit.
// The running maximum is raised only when a block exceeds it by more than
// 2^8 (a factor the fp32 sums absorb exactly), so the rescale of the
// accumulators -- 34 multiplies -- runs on a few blocks per row instead of
// every one; o / l is unchanged.  The branch is taken by the whole wave.
VH_DEVICE void online_softmax_block(floatx16 &sc, float &m_run, float &l_run, floatx16 (&o)[2]) {
    float mb = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; r++) mb = fmaxf(mb, sc[r]);
    mb = fmaxf(mb, __shfl_xor(mb, 32, 64));
    const bool grow = mb > m_run + 8.0f;
    if (__ballot(grow)) {
        const float m_new = grow ? mb : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        o[0] *= alpha;
        o[1] *= alpha;
        m_run = m_new;
    }
    float ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; r++) {
        sc[r] = __builtin_amdgcn_exp2f(sc[r] - m_run);
        ls += sc[r];
    }
    l_run += ls;
}

template <int WAVES, typename TO>
__global__ __launch_bounds__(64 * WAVES, 4) void attention_kernel(AttnArgs a) {
    constexpr int NT = 64 * WAVES;
    constexpr int KV_F4 = ATT_KB * ATT_DH / 4;   // float4s per K (or V) tile
    constexpr int PER_T = KV_F4 / NT;            // per thread
    static_assert(KV_F4 % NT == 0, "tile must divide evenly");
    __shared__ __attribute__((aligned(16))) float Ks[2][ATT_KB][ATT_KPITCH];
    __shared__ __attribute__((aligned(16))) float Vt[2][ATT_DH][ATT_VPITCH];

    const float *qkv = static_cast<const float *>(a.qkv);
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

    // Q for query q0+li, dims 8g + 4lh .. +3, rotated, then scaled by
    // scale*log2(e) so the scores come out in the base-2 exponent domain.
    floatx4 qr[8];
    float gate_logit = 0.0f;  // loaded with Q so the store does not wait on it
    {
        const int q = min(q0 + li, a.L - 1);
        const float *qp = qkv + (size_t)attn_row(a, s, q) * a.ld + h * ATT_DH;
        if (a.gate_col >= 0) gate_logit = qkv[(size_t)attn_row(a, s, q) * a.ld + a.gate_col + h];
        const float qs = a.scale * 1.4426950408889634f;
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int d0 = 8 * g + 4 * lh;
            qr[g] = rope4(ld4(qp + d0), a.rope, q, d0) * qs;
        }
    }

    floatx4 kreg[PER_T], vreg[PER_T];
    auto slot = [&](int i, int &kk, int &d0) {
        const int e = tid + NT * i;
        kk = (e & 15) + 16 * (e >> 8);  // key within the tile
        d0 = 4 * ((e >> 4) & 15);       // first dim of the chunk
    };
    auto load = [&](int kb) {
#pragma unroll
        for (int i = 0; i < PER_T; i++) {
            int kk, d0;
            slot(i, kk, d0);
            const int p = kb * ATT_KB + kk;
            if (p < a.L) {
                const size_t row = (size_t)attn_row(a, s, p) * a.ld;
                kreg[i] = rope4(ld4(qkv + row + kcol + d0), a.rope, p, d0);
                vreg[i] = ld4(qkv + row + vcol + d0);
            } else {
                kreg[i] = floatx4{0.f, 0.f, 0.f, 0.f};
                vreg[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < PER_T; i++) {
            int kk, d0;
            slot(i, kk, d0);
            st4(&Ks[buf][kk][d0], kreg[i]);
#pragma unroll
            for (int c = 0; c < 4; c++) Vt[buf][d0 + c][kk] = vreg[i][c];
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
            for (int g = 0; g < 8; g++) {
                const floatx4 kf = ld4(&Ks[buf][li][8 * g + 4 * lh]);
#pragma unroll
                for (int r = 0; r < 4; r++) sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[r], qr[g][r], sc, 0, 0, 0);
            }
            // sc[r]: score (log2 domain) of key kb*32 + 8*(r/4) + 4*lh + r%4 for
            // query q0 + li.
            const int valid = a.L - kb * ATT_KB;
            if (valid < ATT_KB) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    if (8 * (r >> 2) + 4 * lh + (r & 3) >= valid) sc[r] = -INFINITY;
            }
            online_softmax_block(sc, m_run, l_run, o);
            // O^T += V^T * P^T: step (qq, r) consumes keys 8qq + 4lh + r, which
            // is register 4qq + r of the lane's own half.
#pragma unroll
            for (int qq = 0; qq < 4; qq++) {
                const floatx4 v0 = ld4(&Vt[buf][li][8 * qq + 4 * lh]);
                const floatx4 v1 = ld4(&Vt[buf][32 + li][8 * qq + 4 * lh]);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    o[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(v0[r], sc[4 * qq + r], o[0], 0, 0, 0);
                    o[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(v1[r], sc[4 * qq + r], o[1], 0, 0, 0);
                }
            }
        }
        if (kb + 1 < nkb) store(buf ^ 1);
        __syncthreads();
    }

    if (!wave_active) return;
    // Both half-waves hold partial row sums of the same query; combine them
    // while every lane of the wave is still active.
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

// Short sequences (L <= 64: the band axis).  A persistent workgroup loops
// over (sequence, head) tasks; each task has all of its keys staged in LDS
// at once, and the next task's q/k/v loads are in flight while the current
// one computes.  Four wavefronts of 16 queries run v_mfma_f32_16x16x4f32
// (operand lane (i, k) = element [i = lane%16][k = lane/16]; result lane
// (j, g), register r = row 4g + r, column j) and a single-pass softmax.
//   S^T tile kt (16 keys x 16 queries) = K * Q^T over 16 steps: k-slot g of
//     step 4j + e is head dim 16j + 4g + e, so one 16-byte read gives lane
//     (m, g) the next four steps of key row 16kt + m, and the wave's q
//     loads read 64 contiguous bytes per 4 lanes.  Lane (n, g) receives
//     query n, keys 16kt + 4g + r.
//   O^T tile dt (16 dims x 16 queries) += V^T * P^T: step (kt, r) uses k-slot
//     g = key 16kt + 4g + r, the lane's own probability register; tile row m
//     is dim 4*sigma(m) + dt with sigma(4a + b) = 4b + a, so one 16-byte read
//     of V row 16kt + 4g + r feeds all four tiles, and lane (n, g) ends with
//     dims 16r + 4g + dt: its four 16-byte stores line up with its neighbours'.
// K and V keep their natural row layout in LDS (pitch 68 floats: the rows
// or columns of each 8-lane read phase fall on distinct banks).
VH_DEVICE int short_sigma(int m) { return 4 * (m & 3) + (m >> 2); }

template <typename TO>
__global__ __launch_bounds__(256, 4) void attention_short_kernel(AttnArgs a) {
    if (attn_guard_skip(a)) return;
    constexpr int PITCH = ATT_DH + 4;
    constexpr int KEYS = 64;
    __shared__ __attribute__((aligned(16))) float Ks[KEYS][PITCH];
    __shared__ __attribute__((aligned(16))) float Vs[KEYS][PITCH];

    const float *qkv = static_cast<const float *>(a.qkv);
    const int tasks = a.S * a.H;
    const int tid = (int)threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int q = 16 * wave + n;
    const int qc = min(q, a.L - 1);
    const int d_st = 4 * (tid & 15);  // staging: keys tid/16 + 16i, dims d_st..d_st+3

    floatx4 kpre[4], vpre[4], qpre[4];
    float gpre = 0.0f;
    auto prefetch = [&](int task) {
        const int h = task % a.H, s = task / a.H;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = (tid >> 4) + 16 * i;
            kpre[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            vpre[i] = floatx4{0.f, 0.f, 0.f, 0.f};
            if (key < a.L) {
                const size_t row = (size_t)attn_row(a, s, key) * a.ld;
                kpre[i] = ld4(qkv + row + a.inner + h * ATT_DH + d_st);
                vpre[i] = ld4(qkv + row + 2 * a.inner + h * ATT_DH + d_st);
            }
        }
        const size_t qrow = (size_t)attn_row(a, s, qc) * a.ld;
#pragma unroll
        for (int j = 0; j < 4; j++) qpre[j] = ld4(qkv + qrow + h * ATT_DH + 16 * j + 4 * g);
        if (a.gate_col >= 0) gpre = qkv[qrow + a.gate_col + h];
    };

    // a contiguous run of tasks per workgroup: the heads of one sequence in
    // turn, so the block reads its rows' q/k/v slices back to back
    const int per = (tasks + (int)gridDim.x - 1) / (int)gridDim.x;
    const int t_end = min(tasks, ((int)blockIdx.x + 1) * per);
    int task = (int)blockIdx.x * per;
    if (task < t_end) prefetch(task);
    for (; task < t_end; task++) {
        const int h = task % a.H, s = task / a.H;
        // this task's keys into LDS (K rotated), its queries into registers;
        // keys past L are zeros, rotated with the table's last row (the table
        // has L rows)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = (tid >> 4) + 16 * i;
            st4(&Ks[key][d_st], rope4(kpre[i], a.rope, min(key, a.L - 1), d_st));
            st4(&Vs[key][d_st], vpre[i]);
        }
        floatx4 qr[4];
        {
            const float qs = a.scale * 1.4426950408889634f;
#pragma unroll
            for (int j = 0; j < 4; j++) qr[j] = rope4(qpre[j], a.rope, qc, 16 * j + 4 * g) * qs;
        }
        const float gate_logit = gpre;
        __syncthreads();
        if (task + 1 < t_end) prefetch(task + 1);

        floatx4 sc[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            const float *kr = &Ks[16 * kt + n][4 * g];
            floatx4 k4[4];
#pragma unroll
            for (int j = 0; j < 4; j++) k4[j] = ld4(kr + 16 * j);
            sc[kt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ds = 0; ds < 16; ds++)
                sc[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(k4[ds >> 2][ds & 3], qr[ds >> 2][ds & 3], sc[kt], 0, 0, 0);
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
        const int vcol = 4 * short_sigma(n);
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const floatx4 vv = ld4(&Vs[16 * kt + 4 * g + r][vcol]);
#pragma unroll
                for (int dt = 0; dt < 4; dt++)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[dt], sc[kt][r], o[dt], 0, 0, 0);
            }

        if (q < a.L) {
            const float f = (1.0f / l) * (a.gate_col >= 0 ? sigmoid_dev(gate_logit) : 1.0f);
            TO *op = static_cast<TO *>(a.out) + (size_t)attn_row(a, s, q) * a.ld_out + h * ATT_DH + 4 * g;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                floatx4 v;
#pragma unroll
                for (int dt = 0; dt < 4; dt++) v[dt] = o[dt][r] * f;
                st4(op + 16 * r, v);
            }
        }
        __syncthreads();  // LDS is refilled for the next task
    }
}

}  // namespace vh
