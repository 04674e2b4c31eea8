// Bandwidth-bound kernels: one pass over HBM each, 16-byte accesses,
// wave64 shuffle reductions (no LDS round trips for row statistics).
#pragma once

#include "common.hpp"
#include "h2.hpp"

namespace vh {

// ---------------------------------------------------------------- RMSNorm
// y = x * (sqrt(d) / sqrt(sum(x^2) + 1e-12)) * gamma
// (native/vocalarc_separation.c:419-424, native/native_simd.c:98-121).
// One wavefront per pair of rows: rows 2p and 2p+1 lie back to back (the
// row pitch is dim), so the pair is one contiguous span of 2*dim/4 float4s
// and lane l loads span float4s l, l+64, ... -- every lane busy and twice
// the bytes in flight of a wave per row (non-temporal: each byte is touched
// once).  Each lane adds its float4s' squares into the sum of the row they
// belong to; the pair is held in registers between the two passes.
// TY: fp32, or bf16 when the output feeds a bf16-operand GEMM.
template <typename TY>
VH_DEVICE void st4_once(TY *p, floatx4 v) { st4(p, v); }
template <>
VH_DEVICE void st4_once<float>(float *p, floatx4 v) { st4_stream(p, v); }

template <int MAXV>
VH_DEVICE void rmsnorm_pair_load(const float *xs, int nv, int total, int lane, floatx4 (&v)[MAXV], float &s0,
                                 float &s1) {
    s0 = 0.0f;
    s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = lane + 64 * i;
        if (c < total) {
            v[i] = ld4_stream(xs + 4 * c);
            const float q = v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
            if (c < nv) s0 += q;
            else s1 += q;
        }
    }
    s0 = wave_sum(s0);
    s1 = wave_sum(s1);
}

template <int MAXV, typename TY>
static __global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x,
                                                             const float *__restrict__ gamma, TY *__restrict__ y,
                                                             int rows, int dim) {
    const int row0 = 2 * ((int)blockIdx.x * 4 + ((int)threadIdx.x >> 6));
    const int lane = (int)threadIdx.x & 63;
    if (row0 >= rows) return;
    const int nv = dim >> 2;
    const int total = (row0 + 1 < rows ? 2 : 1) * nv;
    floatx4 v[MAXV];
    float s0, s1;
    rmsnorm_pair_load<MAXV>(x + (size_t)row0 * dim, nv, total, lane, v, s0, s1);
    const float inv0 = sqrtf((float)dim) / sqrtf(s0 + 1.0e-12f);
    const float inv1 = sqrtf((float)dim) / sqrtf(s1 + 1.0e-12f);
    TY *ys = y + (size_t)row0 * dim;
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = lane + 64 * i;
        if (c < total) {
            const bool second = c >= nv;
            st4_once(ys + 4 * c, (v[i] * (second ? inv1 : inv0)) * ld4(gamma + 4 * (second ? c - nv : c)));
        }
    }
}

// The same RMSNorm writing y as h2 rows (h2.hpp) scaled by
// 2^h2_exponent(*bound): the A operand of the fp16 two-piece GEMMs, split
// once here instead of in every column tile of the GEMM.  dim a multiple of
// 16 (so the quads of lanes that share a chunk are whole, in either row of
// the pair: nv is a multiple of 4); an h2 row takes the bytes of its fp32 row.
template <int MAXV>
static __global__ __launch_bounds__(256) void rmsnorm_h2_kernel(const float *__restrict__ x,
                                                               const float *__restrict__ gamma,
                                                               float *__restrict__ y, int rows, int dim,
                                                               const float *__restrict__ bound) {
    const int row0 = 2 * ((int)blockIdx.x * 4 + ((int)threadIdx.x >> 6));
    const int lane = (int)threadIdx.x & 63;
    if (row0 >= rows) return;
    const float s = ldexpf(1.0f, h2_exponent(*bound));
    const int nv = dim >> 2;
    const int total = (row0 + 1 < rows ? 2 : 1) * nv;
    floatx4 v[MAXV];
    float s0, s1;
    rmsnorm_pair_load<MAXV>(x + (size_t)row0 * dim, nv, total, lane, v, s0, s1);
    const float inv0 = sqrtf((float)dim) / sqrtf(s0 + 1.0e-12f);
    const float inv1 = sqrtf((float)dim) / sqrtf(s1 + 1.0e-12f);
    unsigned char *ys = reinterpret_cast<unsigned char *>(y + (size_t)row0 * dim);
#pragma unroll
    for (int i = 0; i < MAXV; i++) {
        const int c = lane + 64 * i;
        if (c < total) {
            const bool second = c >= nv;
            store4_h2_quad(ys + 64 * (c >> 2), c & 3, (v[i] * (second ? inv1 : inv0)) * ld4(gamma + 4 * (second ? c - nv : c)),
                           s);
        }
    }
}

// ------------------------------------------------------------ row softmax
// Materialised softmax of score rows (max, exp, sum, divide), the
// decomposition of native/native_gpu_cuda.cu:357-381.  A workgroup takes 4
// consecutive rows: their 4*len floats start 16-byte aligned whatever len is
// (the first row index is a multiple of 4), so the block moves them between
// HBM and LDS as whole aligned float4s (non-temporal) and never splits a
// chunk with a neighbouring block; wave w then reduces row w from LDS (lane
// l holds elements l, l+64, ...) and writes the result back for the block's
// aligned store.  Rows up to 64*MAXV long.
template <int MAXV>
static __global__ __launch_bounds__(256) void softmax_rows_kernel(const float *__restrict__ in,
                                                                  float *__restrict__ out, int64_t rows, int len) {
    extern __shared__ float srow[];  // [4][len]
    const int tid = (int)threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int64_t row0 = (int64_t)blockIdx.x * 4;
    const int nrows = (int)min<int64_t>(4, rows - row0);
    const int64_t e0 = row0 * len;
    const int ne = nrows * len, n4 = ne >> 2;
    for (int c = tid; c < n4; c += 256) *reinterpret_cast<floatx4 *>(&srow[4 * c]) = ld4_stream(in + e0 + 4 * c);
    for (int e = 4 * n4 + tid; e < ne; e += 256) srow[e] = in[e0 + e];  // the last block's partial chunk
    __syncthreads();
    if (w < nrows) {
        float *r = srow + w * len;
        float v[MAXV];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < MAXV; i++) {
            const int e = lane + 64 * i;
            v[i] = e < len ? r[e] : -INFINITY;
            m = fmaxf(m, v[i]);
        }
        m = wave_max(m);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXV; i++) {
            v[i] = fast_exp_dev(v[i] - m);  // exp(-inf) = 0 past the row's end
            sum += v[i];
        }
        const float inv = 1.0f / wave_sum(sum);
#pragma unroll
        for (int i = 0; i < MAXV; i++) {
            const int e = lane + 64 * i;
            if (e < len) r[e] = v[i] * inv;
        }
    }
    __syncthreads();
    for (int c = tid; c < n4; c += 256) st4_stream(out + e0 + 4 * c, *reinterpret_cast<const floatx4 *>(&srow[4 * c]));
    for (int e = 4 * n4 + tid; e < ne; e += 256) out[e0 + e] = srow[e];
}

// --------------------------------------------------------- rotary [BH][L][64]
// Interleaved-pair rotation (native/vocalarc_separation.c:692-711) with the
// host-built cos/sin table [L][32] (native/vocalarc_separation.c:726-731).
// One float4 (two pairs) per thread, x streamed (non-temporal: each byte is
// touched once).
static __global__ __launch_bounds__(256) void rope_bhld_kernel(float *__restrict__ x, const float *__restrict__ cs,
                                                               const float *__restrict__ sn, int64_t n4, int len) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n4) return;
    const int c4 = (int)(e & 15);           // float4 within the 64-wide head row
    const int pos = (int)((e >> 4) % len);  // position
    float *p = x + 4 * e;
    const floatx4 v = ld4_stream(p);
    const int pi = pos * 32 + 2 * c4;
    const float c0 = cs[pi], s0 = sn[pi], c1 = cs[pi + 1], s1 = sn[pi + 1];
    floatx4 r;
    r[0] = v[0] * c0 - v[1] * s0;
    r[1] = v[0] * s0 + v[1] * c0;
    r[2] = v[2] * c1 - v[3] * s1;
    r[3] = v[2] * s1 + v[3] * c1;
    st4_stream(p, r);
}

// ------------------------------------------------------------- GELU-GLU
// in[rows][2w] = [value | gate] -> out[rows][w] = value * gelu(gate)
static __global__ __launch_bounds__(256) void geglu_kernel(const float *__restrict__ in, float *__restrict__ out,
                                                    int64_t rows, int width) {
    const int w4 = width >> 2;
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= rows * w4) return;
    const int64_t r = e / w4;
    const int c = (int)(e % w4);
    const float *ir = in + r * 2 * width;
    floatx4 v = ld4_stream(ir + 4 * c);
    floatx4 g = ld4_stream(ir + width + 4 * c);
    floatx4 o;
#pragma unroll
    for (int k = 0; k < 4; k++) o[k] = v[k] * gelu_dev(g[k]);
    st4_stream(out + r * width + 4 * c, o);
}

// ----------------------------------------------------------- residual add
// x += r (native/vocalarc_separation.c:820-834)
static __global__ __launch_bounds__(256) void residual_add_kernel(float *__restrict__ x, const float *__restrict__ r,
                                                           int64_t n4) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= n4) return;
    st4_stream(x + 4 * e, ld4_stream(x + 4 * e) + ld4_stream(r + 4 * e));
}

// ------------------------------------------------------------ GELU (in place)
static __global__ __launch_bounds__(256) void gelu_kernel(float *__restrict__ x, int64_t n) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e < n) x[e] = gelu_dev(x[e]);
}

// --------------------------------------------------------- weight unpack
// Packed layout (native/vocalarc_separation.c:428-457: full 32-wide output
// tiles [in][32], then the out%32 tail [in][tail]) -> [row][in] rows of the
// destination.  mode 0: row = dst_row0 + o.  mode 1 (GELU-GLU interleave):
// value output c (o < out/2) and gate output c (o >= out/2) go to rows
// (c/32)*64 + c%32 and (c/32)*64 + 32 + c%32, so a 64-column GEMM tile holds
// 32 values and their 32 gates.
static __global__ __launch_bounds__(256) void unpack_weight_kernel(const float *__restrict__ packed, int in, int out,
                                                            float *__restrict__ dst, int ldd, int dst_row0,
                                                            int mode) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)in * out) return;
    const int i = (int)(e % in);
    const int o = (int)(e / in);
    const int full = (out / 32) * 32;
    float v;
    if (o < full) v = packed[(size_t)(o / 32) * in * 32 + (size_t)i * 32 + (o % 32)];
    else v = packed[(size_t)full * in + (size_t)i * (out - full) + (o - full)];
    int row = o;
    if (mode == 1) {
        const int half = out / 2;
        const int g = o >= half ? 1 : 0;
        const int c = o - g * half;
        row = (c / 32) * 64 + 32 * g + (c % 32);
    }
    dst[(size_t)(dst_row0 + row) * ldd + i] = v;
}

// Vector permutation matching mode 1 of unpack_weight_kernel.
static __global__ __launch_bounds__(256) void interleave_glu_bias_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                                  int out) {
    const int o = (int)(blockIdx.x * 256 + threadIdx.x);
    if (o >= out) return;
    const int half = out / 2;
    const int g = o >= half ? 1 : 0;
    const int c = o - g * half;
    dst[(c / 32) * 64 + 32 * g + (c % 32)] = src[o];
}

// W [N][ldw] with column k multiplied by g[k] -> out [N][K]: an RMSNorm's gain
// folded into the matrix that consumes its output (gemm_h2 row_norm).
static __global__ __launch_bounds__(256) void scale_columns_kernel(const float *__restrict__ W, int N, int K, int ldw,
                                                                  const float *__restrict__ g,
                                                                  float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)N * K) return;
    const int n = (int)(i / K), k = (int)(i % K);
    out[i] = W[(size_t)n * ldw + k] * g[k];
}

// ------------------------------------------------- token-row transposes
// [outer][a][b][D] -> [outer][b][a][D]: whole D-float rows move, so reads and
// writes are both contiguous 16-byte streams.
static __global__ __launch_bounds__(256) void transpose_rows_kernel(const float *__restrict__ src, float *__restrict__ dst,
                                                             int outer, int a, int b, int d4) {
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t total = (int64_t)outer * a * b * d4;
    if (e >= total) return;
    const int c = (int)(e % d4);
    const int64_t tok = e / d4;            // source token index within outer: (i, j)
    const int j = (int)(tok % b);
    const int64_t t2 = tok / b;
    const int i = (int)(t2 % a);
    const int64_t ot = t2 / a;
    const int64_t dt = (ot * b + j) * a + i;
    st4(dst + dt * 4 * d4 + 4 * c, ld4(src + tok * 4 * d4 + 4 * c));
}

// --------------------------------------------------------- band split gather
// For band b and spectrogram row m (= chunk*T + t) gather the band's bins from
// source bins (layout lay) in (frequency, channel, re/im) order, RMS-normalise
// with the band gamma and write row m of the band's input matrix
// (native/vocalarc_separation.c:887-912).
struct BandTable {
    int first_freq[256];
    int width[256];
    int64_t in_offset[256];  // float offset of the band's [M][4w] input matrix
    const float *gamma[256];
};

static __global__ __launch_bounds__(256) void band_gather_norm_kernel(const float *__restrict__ source,
                                                               SpecLayout lay, const BandTable *__restrict__ tab,
                                                               float *__restrict__ bandin, int M, int T, int C) {
    const int b = (int)blockIdx.y;
    const int m = (int)blockIdx.x * 4 + ((int)threadIdx.x >> 6);
    const int lane = (int)threadIdx.x & 63;
    if (m >= M) return;
    const int chunk = m / T, t = m % T;
    const int w = tab->width[b], ff = tab->first_freq[b];
    const int in_dim = w * C * 2;
    const int pairs = w * C;
    float *dst = bandin + tab->in_offset[b] + (size_t)m * in_dim;
    const float *gamma = tab->gamma[b];
    constexpr int MAXP = 5;  // up to 320 (frequency, channel) pairs per band
    float2 v[MAXP];
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXP; k++) {
        const int j = lane + 64 * k;
        if (j < pairs) {
            const int f = j / C, c = j % C;
            v[k] = *reinterpret_cast<const float2 *>(source + 2 * spec_at(lay, chunk, ff + f, c, t));
            ss += v[k].x * v[k].x + v[k].y * v[k].y;
        }
    }
    ss = wave_sum(ss);
    const float inv = sqrtf((float)in_dim) / sqrtf(ss + 1.0e-12f);
#pragma unroll
    for (int k = 0; k < MAXP; k++) {
        const int j = lane + 64 * k;
        if (j < pairs) {
            float2 o;
            o.x = (v[k].x * inv) * gamma[2 * j];
            o.y = (v[k].y * inv) * gamma[2 * j + 1];
            *reinterpret_cast<float2 *>(dst + 2 * j) = o;
        }
    }
}

// ------------------------------------------------------ mask GLU + scatter
// proj_b[m][2*dim] (bias included) -> mask bins (layout lay):
// m_i = p_i * sigmoid(p_{dim+i}), i -> (frequency i/(2C), channel (i/2)%C,
// component i%2) (native/vocalarc_separation.c:1330-1338).
struct MaskTable {
    int first_freq[256];
    int dim[256];            // 4w
    int64_t proj_offset[256];
};

static __global__ __launch_bounds__(256) void mask_glu_scatter_kernel(const float *__restrict__ proj,
                                                               const MaskTable *__restrict__ tab,
                                                               float *__restrict__ mask, SpecLayout lay, int M, int T,
                                                               int C) {
    const int b = (int)blockIdx.y;
    const int dim = tab->dim[b];
    const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (e >= (int64_t)M * dim) return;
    const int m = (int)(e / dim), i = (int)(e % dim);
    const int chunk = m / T, t = m % T;
    const float *p = proj + tab->proj_offset[b] + (size_t)m * 2 * dim;
    const float val = p[i] * (1.0f / (1.0f + __expf(-p[dim + i])));
    const int f = tab->first_freq[b] + i / (2 * C);
    const int c = (i / 2) % C, comp = i & 1;
    mask[2 * spec_at(lay, chunk, f, c, t) + comp] = val;
}

}  // namespace vh
