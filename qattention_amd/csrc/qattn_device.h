// qattn_device.h -- gfx950 device helpers shared by the tree and prefix kernels.
//
// Element types are fp16 and bf16 only (the reference accepts exactly these,
// src/ragged_attn.py:1113-1116).  All arithmetic is fp32.  A 16-byte vector
// (8 elements) per lane is the unit of every global/LDS access: a D-element
// head row is covered by D/8 consecutive lanes ("a row group").
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qattn {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef __bf16 b2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef __bf16 b8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

struct alignas(16) Vec16 {
    uint32_t w[4];
};

struct F16 {
    static constexpr int kCode = 0;
};
struct BF16 {
    static constexpr int kCode = 1;
};

__device__ __forceinline__ Vec16 ld16(const void* p) {
    uint4 x = *reinterpret_cast<const uint4*>(p);
    Vec16 r;
    r.w[0] = x.x; r.w[1] = x.y; r.w[2] = x.z; r.w[3] = x.w;
    return r;
}

__device__ __forceinline__ void st16(void* p, const Vec16& v) {
    *reinterpret_cast<uint4*>(p) = make_uint4(v.w[0], v.w[1], v.w[2], v.w[3]);
}

// Packed 2-element dot product with fp32 accumulation (v_dot2_f32_{f16,bf16}).
template <typename T>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c);

template <>
__device__ __forceinline__ float dot2<F16>(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2_t, a), __builtin_bit_cast(h2_t, b), c, false);
}
template <>
__device__ __forceinline__ float dot2<BF16>(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2_t, a), __builtin_bit_cast(b2_t, b), c, false);
}

// 8-element partial dot product of two 16-byte vectors.
template <typename T>
__device__ __forceinline__ float dot8(const Vec16& a, const Vec16& b) {
    float s = dot2<T>(a.w[0], b.w[0], 0.f);
    s = dot2<T>(a.w[1], b.w[1], s);
    s = dot2<T>(a.w[2], b.w[2], s);
    s = dot2<T>(a.w[3], b.w[3], s);
    return s;
}

// Element j (0..7) of a 16-byte vector as fp32.
template <typename T>
__device__ __forceinline__ float elem(const Vec16& v, int j);

template <>
__device__ __forceinline__ float elem<F16>(const Vec16& v, int j) {
    h2_t p = __builtin_bit_cast(h2_t, v.w[j >> 1]);
    return (float)p[j & 1];
}
template <>
__device__ __forceinline__ float elem<BF16>(const Vec16& v, int j) {
    uint32_t w = v.w[j >> 1];
    uint32_t bits = (j & 1) ? (w & 0xffff0000u) : (w << 16);
    return __builtin_bit_cast(float, bits);
}

// acc[j] = acc[j] * alpha + p * v[j]   (alpha rescale folded in)
template <typename T>
__device__ __forceinline__ void axpy8(float* acc, float p, const Vec16& v) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(p, elem<T>(v, j), acc[j]);
}

// Round 8 fp32 values to one 16-byte vector of T (round to nearest even).
template <typename T>
__device__ __forceinline__ Vec16 pack8(const float* x);

template <>
__device__ __forceinline__ Vec16 pack8<F16>(const float* x) {
    Vec16 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2_t p;
        p[0] = (_Float16)x[2 * i];
        p[1] = (_Float16)x[2 * i + 1];
        r.w[i] = __builtin_bit_cast(uint32_t, p);
    }
    return r;
}
template <>
__device__ __forceinline__ Vec16 pack8<BF16>(const float* x) {
    Vec16 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        b2_t p;
        p[0] = (__bf16)x[2 * i];
        p[1] = (__bf16)x[2 * i + 1];
        r.w[i] = __builtin_bit_cast(uint32_t, p);
    }
    return r;
}

// DPP lane exchange within a 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over a group of LPR consecutive lanes (LPR in {4, 8, 16}); every lane
// of the group receives the total.  quad_perm [1,0,3,2] and [2,3,0,1] form
// the quad sum, row_half_mirror folds quads within 8 lanes, row_mirror folds
// the two halves of a 16-lane row.
template <int LPR>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(LPR == 4 || LPR == 8 || LPR == 16, "group size");
    x += dpp<0xB1>(x);
    x += dpp<0x4E>(x);
    if constexpr (LPR >= 8) x += dpp<0x141>(x);
    if constexpr (LPR >= 16) x += dpp<0x140>(x);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace qattn
