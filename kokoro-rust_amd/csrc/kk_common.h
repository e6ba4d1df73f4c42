// kk_common.h -- shared definitions of the gfx950 decoder + generator engine.
//
// Activations live in HBM time-major: a domain buffer is [L rows][ld channels] with channels
// contiguous, so a tap shift of a convolution is a row offset and an MFMA B-fragment (8 input
// channels of one time column) is one 16-byte load.  Items of a ragged batch are packed along the
// rows with zero gaps; col_item[row] is the owning item or -1 (the reference's Dom,
// src/gpu_batch.rs:31-59).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdint>

namespace kk {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kStyleDim = 128;
constexpr int kHarmonics = 9;

// One time domain of the packed layout (device view).
struct DomDev {
    int64_t l;                // rows
    const int32_t* col_item;  // [l]
    const int64_t* start;     // [nb]
    const int64_t* len;       // [nb]
    int nb;
};

// Per-(item, channel) AdaIN coefficients: v = x * sc + sh (InstanceNorm + affine + style folded).
struct Coef {
    float sc, sh;
};

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    // round to nearest even; quiet NaNs
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u;
        return (uint16_t)(u >> 16);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__host__ __device__ inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace kk
