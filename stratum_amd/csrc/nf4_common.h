// Shared device/host definitions of the gfx950 NF4 library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/stratum_nf4.h"

namespace stm {

// The 16 NF4 levels (QLoRA, arXiv 2305.14314 App. E), as fp32. They are the
// values bitsandbytes returns in QuantState.code and the reference stores in
// NF4Payload.code (stratum/upload.py:78,372).
#define STM_NF4_LEVELS                                                                                     \
    {-1.0f, -0.6961928009986877f, -0.5250730514526367f, -0.39491748809814453f, -0.28444138169288635f,       \
     -0.18477343022823334f, -0.09105003625154495f, 0.0f, 0.07958029955625534f, 0.16093020141124725f,        \
     0.24611230194568634f, 0.33791524171829224f, 0.44070982933044434f, 0.5626170039176941f,                 \
     0.7229568362236023f, 1.0f}

__device__ static constexpr float kLevelsDev[16] = STM_NF4_LEVELS;
static constexpr float kLevelsHost[16] = STM_NF4_LEVELS;

// 65-cell lookup table used by the quantize kernel (see nf4_tables.cpp).
struct CellTable {
    float bound[65];
    uint32_t base[65];
};

// Error reporting (thread-local, host side).
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

int build_cell_table(int rounding, CellTable* out);
int decision_boundaries(int rounding, float out[15]);

// Materialise an fp32 value in a VGPR so that the following conversion to a
// 16-bit type stays a separate rounding. Without it the backend may fold
// "fp32 multiply, then convert to f16" into one v_fma_mixlo_f16 with a +0
// addend, which rounds once and turns a -0.0 product into +0.0; the dequantize
// contract is one fp32 product followed by one round-to-nearest-even conversion.
__device__ __forceinline__ float opaque(float v) {
    __asm__("" : "+v"(v));
    return v;
}

// ------------------------------------------------------------ 16-bit types
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct BF16 {
    typedef bf16x8_t vec8;
    static constexpr int tag = STM_BF16;
    // two fp32 -> packed bf16 pair, round to nearest even (one v_cvt_pk_bf16_f32)
    __device__ static inline uint32_t pack2(float lo, float hi) {
        const f32x2_t v = {lo, hi};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    }
    __device__ static inline float to_f32(uint16_t bits) { return __uint_as_float((uint32_t)bits << 16); }
    __device__ static inline uint16_t from_f32(float v) {
        __bf16 a = (__bf16)v;
        return __builtin_bit_cast(uint16_t, a);
    }
};

struct F16 {
    typedef f16x8_t vec8;
    static constexpr int tag = STM_F16;
    // two fp32 -> packed fp16 pair, round to nearest even (one v_cvt_pk_f16_f32)
    __device__ static inline uint32_t pack2(float lo, float hi) {
        const f32x2_t v = {lo, hi};
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
    }
    __device__ static inline float to_f32(uint16_t bits) { return (float)__builtin_bit_cast(_Float16, bits); }
    __device__ static inline uint16_t from_f32(float v) {
        _Float16 a = (_Float16)v;
        return __builtin_bit_cast(uint16_t, a);
    }
};

__host__ __device__ inline int ilog2(int64_t v) {
    int r = 0;
    while ((int64_t(1) << (r + 1)) <= v) ++r;
    return r;
}

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

}  // namespace stm
