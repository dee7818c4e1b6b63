// Base-Offset PE fake quantization of one token row (peco/quantization.py:97-150), the
// arithmetic shared by every kernel that applies it (the quantizer and pack kernels, the
// attention's query load and the k-means update's packing pass).
//
// Per token, over all D channels, in this fp32 order (one rounding per line):
//   r = x - C[label]; low = min r; high = max r
//   scale = (high - low) / (2^bits - 1), or 1 when not positive
//   code  = clamp(rint((r - low) / scale), 0, 2^bits - 1)      (rint = half-to-even)
//   xhat  = C[label] + (low + scale * code), cast to the input dtype (RNE)
// Translation units are built with -ffp-contract=off and correctly rounded division, so
// every line is one IEEE operation, as in the torch reference. The row's low/high are
// reduced by the caller (fminf/fmaxf: the order does not change the value, and the sign of
// a zero bound cannot change a code or a reconstruction).
#pragma once

#include <type_traits>

#include "common.hpp"

namespace peco {

struct BaseOffsetRow {
    float low, scale, inv, tol, levels;
};

__device__ __forceinline__ BaseOffsetRow base_offset_row(float low, float high, float levels) {
    BaseOffsetRow p;
    const float span = high - low;
    const float raw = span / levels;
    p.low = low;
    p.scale = raw > 0.0f ? raw : 1.0f;
    p.levels = levels;
    // code = rint(RN(shifted / scale)) with the division done once per row: qa = shifted * inv
    // (inv = RN(1 / scale)) and Q = shifted / scale satisfy |qa - Q| <= Q * (2^-23 + 2^-48),
    // and |RN(Q) - Q| <= Q * 2^-24 with Q <= levels, so rint(qa) == rint(RN(Q)) unless qa lies
    // within levels * 1.8e-7 of a half-integer. There (tol = levels * 2^-21 with margin; the
    // distance qa - rint(qa) is computed exactly) the correctly rounded division decides.
    p.inv = 1.0f / p.scale;
    p.tol = levels * 4.76837158203125e-7f;
    return p;
}

// Reconstruction from a rounded quotient q: the code clamped to [0, levels] (v_med3, equal to
// the two-sided clamp for every finite q) and C + (low + scale * code).
__device__ __forceinline__ float base_offset_rebuild(float q, float c, const BaseOffsetRow& p, uint32_t& code) {
    q = __builtin_amdgcn_fmed3f(q, 0.0f, p.levels);
    code = static_cast<uint32_t>(q);
    const float step = p.scale * q;
    const float resid = p.low + step;
    return c + resid;
}

// Code and reconstruction of one residual r = x - c.
__device__ __forceinline__ float base_offset_value(float r, float c, const BaseOffsetRow& p, uint32_t& code) {
    const float shifted = r - p.low;
    const float qa = shifted * p.inv;
    float q = __builtin_rintf(qa);
    if (fabsf(qa - q) >= 0.5f - p.tol) q = __builtin_rintf(shifted / p.scale);
    return base_offset_rebuild(q, c, p, code);
}

// Eight consecutive elements of a row: loads as fp32, stores with RNE, bit copies.
template <int DT> struct Row8 {
    // Loads 8 consecutive elements (starting at element offset e) as fp32.
    __device__ __forceinline__ static void load(const void* base, int64_t e, float (&v)[8]) {
        if constexpr (DT == kF32) {
            const f32x4* p = reinterpret_cast<const f32x4*>(static_cast<const float*>(base) + e);
            const f32x4 a = p[0], b = p[1];
#pragma unroll
            for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
        } else {
            const u16x8 u = *reinterpret_cast<const u16x8*>(static_cast<const uint16_t*>(base) + e);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = half_to_f32<DT>(u[i]);
        }
    }
    __device__ __forceinline__ static void store(void* base, int64_t e, const float (&v)[8]) {
        if constexpr (DT == kF32) {
            f32x4* p = reinterpret_cast<f32x4*>(static_cast<float*>(base) + e);
            p[0] = f32x4{v[0], v[1], v[2], v[3]};
            p[1] = f32x4{v[4], v[5], v[6], v[7]};
        } else {
            u16x8 u;
#pragma unroll
            for (int i = 0; i < 8; ++i) u[i] = f32_to_half<DT>(v[i]);
            *reinterpret_cast<u16x8*>(static_cast<uint16_t*>(base) + e) = u;
        }
    }
    // Bit-exact copy of 8 elements.
    __device__ __forceinline__ static void copy(const void* src, int64_t es, void* dst, int64_t ed) {
        if constexpr (DT == kF32) {
            const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(src) + es);
            u32x4* q = reinterpret_cast<u32x4*>(static_cast<float*>(dst) + ed);
            q[0] = p[0];
            q[1] = p[1];
        } else {
            *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(dst) + ed) =
                *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(src) + es);
        }
    }
};

__device__ __forceinline__ void load_centroid8(const float* c, float (&v)[8]) {
    const f32x4 a = reinterpret_cast<const f32x4*>(c)[0];
    const f32x4 b = reinterpret_cast<const f32x4*>(c)[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = a[i]; v[4 + i] = b[i]; }
}

// Minimum and maximum over an aligned group of G lanes (8 or 16, inside one 16-lane DPP row):
// DPP moves (swaps within quads, then the half-row and row mirrors) instead of LDS permutes.
template <int G>
__device__ __forceinline__ void group_min_max(float& lo, float& hi) {
    static_assert(G == 8 || G == 16, "lane groups of 8 or 16");
    auto step = [&](auto ctrl) __attribute__((always_inline)) {
        constexpr int C = decltype(ctrl)::value;
        lo = fminf(lo, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(lo), C, 0xf, 0xf, false)));
        hi = fmaxf(hi, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(hi), C, 0xf, 0xf, false)));
    };
    step(std::integral_constant<int, 0xb1>{});   // quad_perm [1, 0, 3, 2]: lane ^ 1
    step(std::integral_constant<int, 0x4e>{});   // quad_perm [2, 3, 0, 1]: lane ^ 2
    step(std::integral_constant<int, 0x141>{});  // row_half_mirror: quads 0-1 and 2-3 meet
    if constexpr (G == 16) step(std::integral_constant<int, 0x140>{});  // row_mirror: the two halves meet
}

// Quantize 8 residual channels of one token held by this lane; the lane group of G lanes
// together holds the whole token. Returns codes, writes xhat, low and scale.
template <int G>
__device__ __forceinline__ void base_offset_lane(const float (&x)[8], const float (&c)[8], float levels,
                                                 float (&xhat)[8], uint8_t (&code)[8], float& low_out,
                                                 float& scale_out) {
    float r[8];
    float lo = INFINITY, hi = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        r[i] = x[i] - c[i];
        lo = fminf(lo, r[i]);
        hi = fmaxf(hi, r[i]);
    }
    group_min_max<G>(lo, hi);
    const BaseOffsetRow p = base_offset_row(lo, hi, levels);
    // base_offset_value for the 8 channels, with one branch for the rare near-half quotients
    // of the lane instead of one per channel.
    float shifted[8], q[8];
    float near = 0.0f;  // largest |qa - rint(qa)| of the lane
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        shifted[i] = r[i] - p.low;
        const float qa = shifted[i] * p.inv;
        q[i] = __builtin_rintf(qa);
        near = __builtin_fmaxf(near, fabsf(qa - q[i]));
    }
    if (near >= 0.5f - p.tol) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float qa = shifted[i] * p.inv;
            if (fabsf(qa - q[i]) >= 0.5f - p.tol) q[i] = __builtin_rintf(shifted[i] / p.scale);
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t k;
        xhat[i] = base_offset_rebuild(q[i], c[i], p, k);
        code[i] = static_cast<uint8_t>(k);
    }
    low_out = p.low;
    scale_out = p.scale;
}

}  // namespace peco
