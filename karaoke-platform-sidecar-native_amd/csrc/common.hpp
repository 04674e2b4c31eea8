// Shared device helpers for the gfx950 kernels of the VocalArc HIP provider.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

#define VH_DEVICE __device__ __forceinline__
#define VH_HOST_DEVICE __host__ __device__

// 64-lane wavefront reductions through cross-lane permutes.
VH_DEVICE float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

VH_DEVICE float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// exp(x) through the hardware base-2 exponential.
VH_DEVICE float fast_exp_dev(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

VH_DEVICE float sigmoid_dev(float x) { return 1.0f / (1.0f + __expf(-x)); }

// GELU(x) = 0.5 x (1 + erf(x / sqrt 2)) (native/vocalarc_separation.c:666-672).
// erf(z) = 1 - exp(-z^2) P(t), t = 1 / (1 + p |z|), with P a degree-7
// polynomial without constant term: the form of Abramowitz & Stegun 7.1.26,
// refitted (least squares toward minimax on z in [0, 4.5]) to an absolute
// erf error of 2.3e-9 before rounding.  Evaluated in fp32 the GELU error is
// within 1.3e-7 * max(|x|, 1) over [-8, 8], the same as a GELU built on a
// correctly rounded fp32 erf, in 16 VALU instructions (two of them
// transcendental) instead of the general erff's branches.
VH_DEVICE float gelu_dev(float x) {
    const float z = x * 0.7071067811865475f;
    const float az = fabsf(z);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.445f, az, 1.0f));
    float q = 0.09287256f;
    q = fmaf(q, t, -0.51063324f);
    q = fmaf(q, t, 0.92279828f);
    q = fmaf(q, t, -0.44809147f);
    q = fmaf(q, t, 0.49923836f);
    q = fmaf(q, t, 0.18621909f);
    q = fmaf(q, t, 0.25759641f);
    q *= t;
    const float e = __builtin_amdgcn_exp2f(az * (az * -1.4426950408889634f));
    const float erf_abs = fmaf(-q, e, 1.0f);
    const float erf = __builtin_copysignf(erf_abs, z);
    const float h = 0.5f * x;
    return fmaf(h, erf, h);
}

VH_DEVICE floatx4 ld4(const float *p) { return *reinterpret_cast<const floatx4 *>(p); }
VH_DEVICE void st4(float *p, floatx4 v) { *reinterpret_cast<floatx4 *>(p) = v; }

// Complex spectrum element (chunk, frequency f, channel c, frame t) of a
// float array of (re, im) pairs, at pair index
// chunk*chunk_s + f*f_s + c*c_s + t*t_s.  The reference's layout is
// [chunk][F][C][T] (native/vocalarc_separation.c:1058, 1336); the device
// pipeline keeps spectra frame-major, [chunk][C][T][F], so every frame's bins
// are contiguous for the FFTs, the band gather and the mask scatter.
struct SpecLayout {
    int64_t chunk_s, f_s, c_s, t_s;
};
inline SpecLayout spec_reference_layout(int F, int C, int T) {
    return {(int64_t)F * C * T, (int64_t)C * T, (int64_t)T, 1};
}
inline SpecLayout spec_frame_major_layout(int F, int C, int T) {
    return {(int64_t)C * T * F, 1, (int64_t)T * F, (int64_t)F};
}
VH_DEVICE int64_t spec_at(const SpecLayout &l, int chunk, int f, int c, int t) {
    return chunk * l.chunk_s + f * l.f_s + c * l.c_s + t * l.t_s;
}

// bf16 storage (round to nearest even on conversion: v_cvt_pk_bf16_f32)
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

VH_DEVICE bf16x4 to_bf16x4(floatx4 v) {
    bf16x4 r;
    r[0] = (bf16)v[0];
    r[1] = (bf16)v[1];
    r[2] = (bf16)v[2];
    r[3] = (bf16)v[3];
    return r;
}

// Four consecutive outputs, fp32 or bf16.
VH_DEVICE void st4(bf16 *p, floatx4 v) { *reinterpret_cast<bf16x4 *>(p) = to_bf16x4(v); }

// Non-temporal streaming variants for data touched exactly once.
VH_DEVICE floatx4 ld4_stream(const float *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(p));
}
VH_DEVICE void st4_stream(float *p, floatx4 v) {
    __builtin_nontemporal_store(v, reinterpret_cast<floatx4 *>(p));
}

// Workgroups are dispatched round-robin over the 8 XCDs of an MI355X
// (workgroup i runs on XCD i % 8).  Remapping the linear id so that each XCD
// owns a contiguous range of tiles keeps neighbouring tiles (which share
// operand rows) in the same L2.
VH_DEVICE int xcd_swizzle(int id, int count) {
    const int xcds = 8;
    int per = count / xcds;
    int rem = count % xcds;
    int xcd = id % xcds;
    int local = id / xcds;
    // XCDs [0, rem) own per+1 tiles, the rest own per tiles.
    int base = xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per;
    int mine = xcd < rem ? per + 1 : per;
    return local < mine ? base + local : id;  // tail ids (never produced when count % 8 == 0) keep their id
}
