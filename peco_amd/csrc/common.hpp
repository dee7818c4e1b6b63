// Shared device helpers for the PECO gfx950 kernels.
//
// All kernels are written for CDNA4 (gfx950): 64-lane wavefronts, MFMA matrix cores,
// 160 KB LDS per CU. Exact fp32 arithmetic matters for the k-means labels and the
// Base-Offset codes, so every translation unit is compiled with -ffp-contract=off and
// correctly rounded fp32 division; fused multiply-adds are written explicitly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#define PECO_API extern "C" __attribute__((visibility("default")))

namespace peco {

constexpr int kWave = 64;

// PECO-specific status codes live above the hipError_t range.
enum Status : int {
    kOk = 0,
    kInvalidValue = 1,          // == hipErrorInvalidValue
    kWorkspaceTooSmall = 20001,
    kUnsupportedShape = 20002,
    kUnsupportedDtype = 20003,
    kScratchExceeded = 20004,   // larger than the static scratch of an allocation-free entry
};

enum DType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16 with round-to-nearest-even (NaN kept quiet).
// Round to nearest even; a NaN stays a (quiet) NaN. Written without branches so that
// unrolled conversions stay straight-line code.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t quiet = (u >> 16) | 0x40u;
    return static_cast<uint16_t>(f != f ? quiet : rounded);
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t b) {
    return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT> __device__ __forceinline__ float load_elem(const void* p, int64_t i);
template <> __device__ __forceinline__ float load_elem<kBF16>(const void* p, int64_t i) {
    return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <> __device__ __forceinline__ float load_elem<kF16>(const void* p, int64_t i) {
    return f16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
}
template <> __device__ __forceinline__ float load_elem<kF32>(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
}

// Unpack 16-bit payloads (bf16 or fp16, chosen at compile time) to fp32.
template <int DT> __device__ __forceinline__ float half_to_f32(uint16_t b) {
    if constexpr (DT == kBF16) return bf16_bits_to_f32(b);
    else return f16_bits_to_f32(b);
}
template <int DT> __device__ __forceinline__ uint16_t f32_to_half(float f) {
    if constexpr (DT == kBF16) return f32_to_bf16_bits(f);
    else return f32_to_f16_bits(f);
}

// Order-preserving map of fp32 onto uint32 (for packed (value, index) min keys).
__device__ __forceinline__ uint32_t orderable(float f) {
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

template <typename T> __device__ __forceinline__ T wave_shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, kWave);
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Compute units of the current device (cached per device; 256 if the query fails).
inline int device_compute_units() {
    static std::mutex m;
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lock(m);
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// One 16-byte-per-lane direct load from global memory into the LDS span starting at byte
// address lds (M0). Written as inline assembly so that the compiler's wait-count pass does not
// see an LDS write in flight: it cannot tell the buffer being filled from the one being read
// by the fragment reads and would otherwise wait for the whole prefetch in the middle of
// every tile. The caller waits for vmcnt(0) before the barrier that publishes the tile.
__device__ __forceinline__ void dma16(const uint16_t* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

// The same with a wave-uniform base address in SGPRs and a 32-bit byte offset per lane (one
// VALU operation per load for the offset instead of 64-bit address arithmetic).
__device__ __forceinline__ void dma16_off(const void* base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory", "m0");
}

// The same with 4 bytes per lane: lane i writes lds + 4i.
__device__ __forceinline__ void dma4(const void* src, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds) : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}

// XCDs of an MI355X: workgroup i of a launch is dispatched to XCD i % kXcdCount, each with
// its own L2.
constexpr int kXcdCount = 8;

}  // namespace peco
