// Shared device helpers for the gfx950 kernels behind include/mi_qmm.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mi_qmm.h"

namespace mi {

typedef __bf16 bf16;
typedef _Float16 f16;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Error reporting (mi_abi.hip). fail() records the message and returns code.
int fail(int code, const char *fmt, ...);
int launch_status(const char *what);  // MI_OK or MI_ERR_LAUNCH after a launch

// 8 lanes of T packed in 16 bytes, and 4 lanes in 8 bytes.
template <typename T> struct Vec;
template <> struct Vec<bf16> { typedef bf16x8 x8; typedef bf16x4 x4; };
template <> struct Vec<f16> { typedef f16x8 x8; typedef f16x4 x4; };

template <typename T> __device__ __forceinline__ float f32(T v) { return (float)v; }
// float -> T with one round-to-nearest-even conversion (v_cvt_pk_bf16_f32 /
// v_cvt_f16_f32 on gfx950).
template <typename T> __device__ __forceinline__ T cvt(float v) { return (T)v; }

// An fp32 result held as fp32 before a conversion to T, as the source writes
// it. For fp16 the compiler otherwise folds the product or fma that makes v
// into one mixed-precision instruction (v_fma_mixlo_f16) that rounds once,
// straight to fp16: a different value in a few last places, chosen or not
// depending on the surrounding code -- so two kernels that share an
// expression could disagree. (bf16 has no such instruction.)
template <typename T> __device__ __forceinline__ float pin32(float v) {
    if constexpr (sizeof(T) == 2 && !__is_same(T, bf16)) asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ uint4 ld16(const void *p) { return *(const uint4 *)p; }
// A 16-byte load marked non-temporal (streamed data read once: quantized
// weights in the GEMV). Measured on MI355X over a 2 GiB read: 7.0-7.1 TB/s
// against 6.2 TB/s with ordinary loads.
__device__ __forceinline__ uint4 ld16_nt(const void *p) {
    typedef unsigned U4 __attribute__((ext_vector_type(4)));
    const U4 v = __builtin_nontemporal_load((const U4 *)p);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 ld8(const void *p) { return *(const uint2 *)p; }
__device__ __forceinline__ void st16(void *p, uint4 v) { *(uint4 *)p = v; }
__device__ __forceinline__ void st8(void *p, uint2 v) { *(uint2 *)p = v; }

// Unpack the 8 values of a 16-byte group of T into floats.
template <typename T> __device__ __forceinline__ void unpack8(uint4 raw, float (&f)[8]) {
    typedef typename Vec<T>::x8 V;
    V v = __builtin_bit_cast(V, raw);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)v[i];
}

template <typename T> __device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
    typedef typename Vec<T>::x8 V;
    V v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (T)f[i];
    return __builtin_bit_cast(uint4, v);
}

// Two floats to the two T lanes of one dword (a low, b high), each rounded to
// nearest even; bf16 pairs take one v_cvt_pk_bf16_f32.
template <typename T> __device__ __forceinline__ uint32_t pk2(float a, float b) {
    typedef float F2 __attribute__((ext_vector_type(2)));
    typedef T T2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((F2){a, b}, T2));
}

// Unpack the 4 values of an 8-byte group of T into floats.
template <typename T> __device__ __forceinline__ void unpack4(uint2 raw, float (&f)[4]) {
    typedef typename Vec<T>::x4 V;
    V v = __builtin_bit_cast(V, raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = (float)v[i];
}

template <typename T> __device__ __forceinline__ uint2 pack4(const float (&f)[4]) {
    typedef typename Vec<T>::x4 V;
    V v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (T)f[i];
    return __builtin_bit_cast(uint2, v);
}

// Affine dequant of 8 consecutive packed values: T(fma(s, q, b)), one
// rounding (the reference's dequant form). For 4 bits the 8 values are the 8
// nibbles of word w0; for 8 bits they are the 4 bytes of w0 followed by the 4
// bytes of w1. init() prepares the words once; pair(k) converts values 2k and
// 2k + 1 into one packed register, so a caller can spread the four pairs
// between other instructions; launder() pins the prepared words in registers.
//
// 4 bits: each nibble reaches the fma as an fp16 denormal, q * 2^-24, the
// 16-bit half of a word (w >> 4j) & 0x000F000F holding nibbles j and j + 4;
// v_fma_mix_f32 reads that half as its f16 operand, so
// fma(s * 2^24, q * 2^-24, b) = fma(s, q, b) exactly (s * 2^24 is exact for
// every fp16 scale and every bf16 scale of magnitude below 2^104, and the
// kernels run with fp16 denormals preserved): 19 VALU per 8 values where a
// byte conversion per value took 23. Checked on MI355X against
// fmaf(s, q, b) over every finite bf16 scale below 2^104, all 16 nibbles and
// 256 biases: no difference in 484 million values. A bf16 scale of 2^104 or
// more overflows s * 2^24 (inf, or NaN for q = 0); no quantizer produces one
// short of weights near 3e32, and the plain dequant entry has no such limit.
template <typename T, int BITS> struct Dequant8 {
    uint32_t r[4];  // 4 bits: the f16-denormal pairs (nibbles j, j + 4); 8 bits: w0, w1
    float s, bias;

    __device__ __forceinline__ void init(uint32_t w0, uint32_t w1, float s_, float b_) {
        bias = b_;
        if constexpr (BITS == 4) {
            s = __builtin_ldexpf(s_, 24);
#pragma unroll
            for (int j = 0; j < 4; ++j) r[j] = (w0 >> (4 * j)) & 0x000F000Fu;
            // (kept as words: the masks would otherwise be folded into each
            // value's conversion again)
            asm("" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
        } else {
            s = s_;
            r[0] = w0;
            r[1] = w1;
        }
    }
    __device__ __forceinline__ void launder() {
        if constexpr (BITS == 4)
            asm volatile("" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
        else
            asm volatile("" : "+v"(r[0]), "+v"(r[1]));
    }
    // Values 2k and 2k + 1 are converted together (pk2): converted one by
    // one, the compiler packed mismatched pairs and re-shuffled them.
    __device__ __forceinline__ uint32_t pair(int k) const {
        if constexpr (BITS == 4) {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            const int n0 = 2 * k, n1 = 2 * k + 1;  // nibble n sits in r[n % 4], half n / 4
            const h2 v0 = __builtin_bit_cast(h2, r[n0 & 3]), v1 = __builtin_bit_cast(h2, r[n1 & 3]);
            return pk2<T>(__builtin_fmaf(s, (float)v0[n0 >> 2], bias),
                          __builtin_fmaf(s, (float)v1[n1 >> 2], bias));
        } else {
            const uint32_t w = k < 2 ? r[0] : r[1];
            const int sh = 16 * (k & 1);
            return pk2<T>(__builtin_fmaf(s, (float)((w >> sh) & 255u), bias),
                          __builtin_fmaf(s, (float)((w >> (sh + 8)) & 255u), bias));
        }
    }
};

template <typename T, int BITS>
__device__ __forceinline__ typename Vec<T>::x8 dequant8(uint32_t w0, uint32_t w1, float s,
                                                       float b) {
    Dequant8<T, BITS> d;
    d.init(w0, w1, s, b);
    return __builtin_bit_cast(typename Vec<T>::x8, (uint4){d.pair(0), d.pair(1), d.pair(2), d.pair(3)});
}

// Register "launder": an empty asm that claims to rewrite the value. Placed
// where a prefetched register buffer is handed to the next pipeline step, it
// stops the compiler from folding the two loads feeding that hand-off into one
// load at the top of the loop (which would serialize load and use); the wait
// for the prefetched data then lands at the hand-off, after the compute.
__device__ __forceinline__ void launder(uint4 &v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}
__device__ __forceinline__ void launder(uint32_t &v) { asm volatile("" : "+v"(v)); }

// The rotation of a pair (a, c) by an angle of cosine cs and sine sn, each
// output one fma over a rounded product: a cs - c sn and a sn + c cs
// (norm_rope_kernel and the q/k/v GEMM's head epilogue share them).
__device__ __forceinline__ float rope_first(float a, float c, float cs, float sn) {
    return __builtin_fmaf(a, cs, -(c * sn));
}
__device__ __forceinline__ float rope_second(float a, float c, float cs, float sn) {
    return __builtin_fmaf(a, sn, c * cs);
}

// One DPP-moved copy of v (CTRL: the gfx9 DPP control; every lane active).
template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, 0xF, false));
}
// The sum over each 16-lane row, the same bits in every lane of the row:
// pairs within quads, then quad sums across a half-row and half-row sums
// across the row (mirrors), each step adding two values the lanes of its
// group hold alike. Four DPP adds, where an xor-shuffle tree takes four
// dependent ds_bpermute trips through the LDS unit.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1, 0, 3, 2]: lane ^ 1
    v += dpp_f32<0x4E>(v);   // quad_perm [2, 3, 0, 1]: lane ^ 2
    v += dpp_f32<0x141>(v);  // row_half_mirror: lane 7 - i of each 8
    v += dpp_f32<0x140>(v);  // row_mirror: lane 15 - i of each 16
    return v;
}

__host__ __device__ constexpr int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline int ilog2(int v) {
    int r = 0;
    while ((1 << (r + 1)) <= v) ++r;
    return r;
}

inline hipStream_t as_stream(void *s) { return (hipStream_t)s; }

inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

inline bool valid_dtype(int d) { return d == MI_F32 || d == MI_F16 || d == MI_BF16; }

// Checks shared by the quantized entries (scaffold/stitch.py:103-123).
int check_quant(int64_t N, int64_t K, int group_size, int bits, int dtype);

}  // namespace mi
