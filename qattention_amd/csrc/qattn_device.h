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

// ---------------------------------------------------------------------------
// v_mfma_f32_16x16x32_{f16,bf16} and the operand layouts the kernels rely on
// (one wave, lane l, i = l / 16, c = l % 16):
//   A (16 x 32): lane holds A[c][8i .. 8i+7]      (one 16-byte vector)
//   B (32 x 16): lane holds B[8i .. 8i+7][c]
//   D (16 x 16): lane holds D[4i + r][c], r = 0..3
// ---------------------------------------------------------------------------
template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<F16> {
    static __device__ __forceinline__ f4_t mma(const Vec16& a, const Vec16& b, f4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0,
                                                     0, 0);
    }
    // 16x16x16: lane (c, i) feeds A[c][4i..4i+3] and B[4i..4i+3][c]
    static __device__ __forceinline__ f4_t mma16(uint2 a, uint2 b, f4_t c) {
        typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4_t, a), __builtin_bit_cast(h4_t, b), c, 0, 0,
                                                    0);
    }
    static __device__ __forceinline__ uint32_t pack2(float x, float y) {
        h2_t h;
        h[0] = (_Float16)x;
        h[1] = (_Float16)y;
        return __builtin_bit_cast(uint32_t, h);
    }
    // the two elements of a packed pair back as fp32
    static __device__ __forceinline__ float lo(uint32_t w) { return (float)__builtin_bit_cast(h2_t, w)[0]; }
    static __device__ __forceinline__ float hi(uint32_t w) { return (float)__builtin_bit_cast(h2_t, w)[1]; }
};

template <>
struct MfmaOps<BF16> {
    static __device__ __forceinline__ f4_t mma(const Vec16& a, const Vec16& b, f4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0,
                                                      0, 0);
    }
    static __device__ __forceinline__ f4_t mma16(uint2 a, uint2 b, f4_t c) {
        typedef short s4_t __attribute__((ext_vector_type(4)));
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s4_t, a), __builtin_bit_cast(s4_t, b), c, 0,
                                                        0, 0);
    }
    static __device__ __forceinline__ uint32_t pack2(float x, float y) {
        b2_t h;
        h[0] = (__bf16)x;
        h[1] = (__bf16)y;
        return __builtin_bit_cast(uint32_t, h);
    }
    static __device__ __forceinline__ float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
    static __device__ __forceinline__ float hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
};

// ---------------------------------------------------------------------------
// v_mfma_f32_32x32x16_{f16,bf16} (gfx950; lane l, h = l / 32, c = l % 32;
// checked element by element on the GPU with exact small integers):
//   A (32 x 16): lane holds A[c][8h .. 8h+7]      (one 16-byte vector)
//   B (16 x 32): lane holds B[8h .. 8h+7][c]
//   D (32 x 32): lane holds D[8(r/4) + 4h + r%4][c] in element r, r = 0..15
// One 32x32x16 product is twice the FLOPs of a 16x16x32 one; a stream of
// them with this prefix kernel's softmax mix and LDS operand reads sustained
// 66% of the fp16 peak at 2 waves per SIMD, against 33% for 16x16x32.
// ---------------------------------------------------------------------------
typedef float f16v_t __attribute__((ext_vector_type(16)));

template <typename T>
__device__ __forceinline__ f16v_t mma32(const Vec16& a, const Vec16& b, f16v_t c);
template <>
__device__ __forceinline__ f16v_t mma32<F16>(const Vec16& a, const Vec16& b, f16v_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(h8_t, a), __builtin_bit_cast(h8_t, b), c, 0, 0,
                                                  0);
}
template <>
__device__ __forceinline__ f16v_t mma32<BF16>(const Vec16& a, const Vec16& b, f16v_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(b8_t, a), __builtin_bit_cast(b8_t, b), c, 0, 0,
                                                   0);
}

// Reductions over the lane pair l, l ^ 32 (one column of a 32x32 MFMA output).
__device__ __forceinline__ float xor32_max(float x) {
    auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}
__device__ __forceinline__ float xor32_sum(float x) {
    auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
}

// Prefix split states store each query's numerator / l, a convex
// combination of V rows: in fp16 for fp16 inputs (it fits fp16's range, and
// half the bytes of fp32 is half of what the split merge reads), in fp32 for
// bf16 inputs (bf16's 8-bit mantissa would add a second rounding the size of
// the output's own).
template <typename T>
constexpr bool kPartHalf = T::kCode == F16::kCode;

__device__ __forceinline__ float xor_max(float x, int m) { return fmaxf(x, __shfl_xor(x, m)); }

// Reductions over the 4 lanes l, l^16, l^32, l^48 (one MFMA output column)
// with gfx950's v_permlane16_swap / v_permlane32_swap: swap(x, x) returns the
// pair (x[l], x[l ^ 16]) (resp. ^ 32) in some order, so op(first, second) is
// the xor-16 (xor-32) reduction, entirely in VALU.
__device__ __forceinline__ float col4_max(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    x = fmaxf(__builtin_bit_cast(float, (uint32_t)a[0]), __builtin_bit_cast(float, (uint32_t)a[1]));
    auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    return fmaxf(__builtin_bit_cast(float, (uint32_t)b[0]), __builtin_bit_cast(float, (uint32_t)b[1]));
}
__device__ __forceinline__ float col4_sum(float x) {
    auto a = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    x = __builtin_bit_cast(float, (uint32_t)a[0]) + __builtin_bit_cast(float, (uint32_t)a[1]);
    auto b = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, x),
                                              false, false);
    return __builtin_bit_cast(float, (uint32_t)b[0]) + __builtin_bit_cast(float, (uint32_t)b[1]);
}

// Column of key k (0..63) of a block in the LDS copy of V^T: within each 32-key
// half, key 16u + 4g + j sits at 8g + 4u + j, so the 8 keys a lane feeds to
// one PV MFMA (4 from each of two S^T tiles) are contiguous.
__device__ __forceinline__ int vt_col(int k) {
    const int half = k >> 5, r = k & 31;
    const int u = r >> 4, g = (r >> 2) & 3, j = r & 3;
    return 32 * half + 8 * g + 4 * u + j;
}


__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

}  // namespace qattn
