// Device-side helpers shared by the gfx950 kernels: exact f16 decode, GGUF
// block decode (bit-exact with internal/gguf/dequant.go), wavefront
// reductions, and the reference's fast exp (internal/ml/attention.go:34-61).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wh {

__device__ __forceinline__ float u2f(uint32_t b) { return __uint_as_float(b); }

// Exact IEEE half -> float by bit manipulation (internal/gguf/dequant.go:15-44):
// subnormals are normalised, Inf/NaN keep their payload bits.
__device__ __forceinline__ float h2f(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) return u2f(s);
        uint32_t k = (uint32_t)__clz((int)m) - 21u;  // shifts that bring the leading 1 to bit 10
        m = (m << k) & 0x3FFu;
        return u2f(s | ((113u - k) << 23) | (m << 13));
    }
    if (e == 31) return u2f(s | 0x7F800000u | (m << 13));
    return u2f(s | ((e + 112u) << 23) | (m << 13));
}

// d*q + m without contraction: the reference computes it as two rounded
// float32 operations (internal/gguf/dequant.go:123,176).
__device__ __forceinline__ float mul_add_nofma(float d, float q, float m) {
#pragma clang fp contract(off)
    float t = d * q;
    return t + m;
}

// Wavefront (64-lane) butterfly sum over groups of G lanes (G power of 2 <= 64).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// internal/ml/attention.go:34-61 — restated operation by operation so the
// device and the reference evaluate the same float32 polynomial.
__device__ __forceinline__ float fast_exp(float x) {
#pragma clang fp contract(off)
    const float inv_ln2 = 1.4426950408889634f, ln2 = 0.6931471805599453f;
    if (x <= -20.0f) return 0.0f;
    float y = x * inv_ln2;
    int k = (int)y;
    if ((float)k > y) k--;
    float r = x - (float)k * ln2;
    float r2 = r * r, r3 = r2 * r, r4 = r3 * r;
    float poly = 1.0f + r + 0.5f * r2 + (float)(1.0 / 6.0) * r3 + (float)(1.0 / 24.0) * r4;
    if (k < -126) return 0.0f;
    if (k > 127) return 3.40282346638528859811704183484516925440e+38f;
    return poly * u2f((uint32_t)(k + 127) << 23);
}

// tanh-form GELU with tanh in float64 (internal/ml/ops.go:102-122).
__device__ __forceinline__ float gelu_ref(float x) {
#pragma clang fp contract(off)
    const float k = 0.7978845608028654f;
    float inner = k * (x + 0.044715f * x * x * x);
    return x * 0.5f * (float)(1.0 + tanh((double)inner));
}

// Bit-exact dequantisation of element j (0..31) of block b of row r.
struct MatView {
    const uint8_t *qs;
    const void *sc;
    const uint32_t *qh;
    int32_t rows, cols, nb;
};

template <int TYPE>
__device__ __forceinline__ float dequant_elem(const MatView &m, int r, int b, int j) {
#pragma clang fp contract(off)
    size_t blk = (size_t)r * m.nb + b;
    if constexpr (TYPE == 0) {
        return ((const float *)m.qs)[blk * 32 + j];
    } else if constexpr (TYPE == 8) {
        float d = h2f(((const uint16_t *)m.sc)[blk]);
        return d * (float)(int)((const int8_t *)m.qs)[blk * 32 + j];
    } else {
        uint8_t byte = m.qs[blk * 16 + (j >> 1)];
        uint32_t nib = (j & 1) ? (uint32_t)(byte >> 4) : (uint32_t)(byte & 0xF);
        if constexpr (TYPE == 2) {
            float d = h2f(((const uint16_t *)m.sc)[blk]);
            return d * (float)((int32_t)nib - 8);
        } else if constexpr (TYPE == 3) {
            uint32_t w = ((const uint32_t *)m.sc)[blk];
            return mul_add_nofma(h2f(w & 0xFFFFu), (float)nib, h2f(w >> 16));
        } else if constexpr (TYPE == 6) {
            float d = h2f(((const uint16_t *)m.sc)[blk]);
            uint32_t hi = (m.qh[blk] >> j) & 1u;
            return d * (float)((int32_t)(nib | (hi << 4)) - 16);
        } else {  // TYPE == 7
            uint32_t w = ((const uint32_t *)m.sc)[blk];
            uint32_t hi = (m.qh[blk] >> j) & 1u;
            return mul_add_nofma(h2f(w & 0xFFFFu), (float)(nib | (hi << 4)), h2f(w >> 16));
        }
    }
}

}  // namespace wh
