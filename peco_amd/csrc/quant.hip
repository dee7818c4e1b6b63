// Stage 2: Base-Offset PE centroid-residual quantizer (peco/quantization.py:97-150),
// plus the fused "pack" kernel that applies it while gathering Q/K/V into cluster order
// and appending the unsorted text rows (peco/processor.py:141-149).
//
// The per-token arithmetic (base_offset.hpp) is one IEEE operation per step, in the torch
// reference's order.
//
// Layout: a token row of D elements is handled by G = D/8 lanes (8 elements per lane,
// 16-byte loads for 16-bit inputs), so one wavefront covers 64/G rows and min/max are
// reduced with log2(G) xor-shuffles inside the lane group. HBM-bound streaming kernel.
#include "base_offset.hpp"
#include "common.hpp"

#include <algorithm>

namespace peco {
namespace {

template <int DT, int G>
__global__ __launch_bounds__(256) void base_offset_kernel(const void* __restrict__ x, const int32_t* __restrict__ labels,
                                                          const float* __restrict__ centroids, int64_t rows,
                                                          int tokens, int clusters, int bits,
                                                          uint8_t* __restrict__ codes, float* __restrict__ low,
                                                          float* __restrict__ scale, void* __restrict__ xhat) {
    constexpr int D = G * 8;
    const int sub = threadIdx.x % G;
    const float levels = static_cast<float>((1 << bits) - 1);
    for (int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / G; row < rows;
         row += static_cast<int64_t>(gridDim.x) * blockDim.x / G) {
        const int64_t b = row / tokens;
        const int lab = labels[row];
        float xv[8], cv[8], out[8], lo, sc;
        uint8_t q[8];
        Row8<DT>::load(x, row * D + sub * 8, xv);
        load_centroid8(centroids + (b * clusters + lab) * D + sub * 8, cv);
        base_offset_lane<G>(xv, cv, levels, out, q, lo, sc);
        if (codes) {
            u32x2 packed;
            packed[0] = q[0] | (q[1] << 8) | (q[2] << 16) | (static_cast<uint32_t>(q[3]) << 24);
            packed[1] = q[4] | (q[5] << 8) | (q[6] << 16) | (static_cast<uint32_t>(q[7]) << 24);
            *reinterpret_cast<u32x2*>(codes + row * D + sub * 8) = packed;
        }
        if (sub == 0) {
            if (low) low[row] = lo;
            if (scale) scale[row] = sc;
        }
        if (xhat) Row8<DT>::store(xhat, row * D + sub * 8, out);
    }
}

template <int DT, int G>
__global__ __launch_bounds__(256) void base_offset_decode_kernel(const uint8_t* __restrict__ codes,
                                                                 const float* __restrict__ low,
                                                                 const float* __restrict__ scale,
                                                                 const int32_t* __restrict__ labels,
                                                                 const float* __restrict__ centroids, int64_t rows,
                                                                 int tokens, int clusters, void* __restrict__ xhat) {
    constexpr int D = G * 8;
    const int sub = threadIdx.x % G;
    for (int64_t row = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / G; row < rows;
         row += static_cast<int64_t>(gridDim.x) * blockDim.x / G) {
        const int64_t b = row / tokens;
        float cv[8], out[8];
        load_centroid8(centroids + (b * clusters + labels[row]) * D + sub * 8, cv);
        const u32x2 packed = *reinterpret_cast<const u32x2*>(codes + row * D + sub * 8);
        const float lo = low[row], sc = scale[row];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t code = (packed[i / 4] >> (8 * (i % 4))) & 0xffu;
            const float step = sc * static_cast<float>(code);
            const float resid = lo + step;
            out[i] = cv[i] + resid;
        }
        Row8<DT>::store(xhat, row * D + sub * 8, out);
    }
}

}  // namespace

struct PackTensor {
    const void* input;        // [batch, length, dims]
    void* output;             // [batch, length, dims]
    const int32_t* indices;   // [batch, video]: original video token at each packed position
    const int32_t* labels;    // [batch, video] (read only when bits != 0)
    const float* centroids;   // [batch, clusters, dims] (read only when bits != 0)
    int clusters;
    int bits;                 // 0 = plain gather, 4 or 8 = fake-quantize while gathering
};

struct PackArgs {
    PackTensor t[3];
    int num, batch, length, video;
};

namespace {

template <int DT, int G>
// Grid (row tiles, batch, tensor): 16-lane groups (G lanes) own one output row each, so no
// thread divides a linear index.
__global__ __launch_bounds__(256) void pack_kernel(PackArgs a) {
    constexpr int D = G * 8;
    const int sub = threadIdx.x % G;
    const int j = static_cast<int>(blockIdx.x) * (256 / G) + static_cast<int>(threadIdx.x) / G;
    if (j >= a.length) return;
    const int64_t b = blockIdx.y;
    const PackTensor& T = a.t[blockIdx.z];
    const int64_t row = b * a.length + j;
    const int64_t dst = row * D + sub * 8;
    if (j >= a.video) {
        Row8<DT>::copy(T.input, dst, T.output, dst);
        return;
    }
    const int tok = T.indices[b * a.video + j];
    const int64_t src = (b * a.length + tok) * D + sub * 8;
    if (T.bits == 0) {
        Row8<DT>::copy(T.input, src, T.output, dst);
        return;
    }
    const int lab = T.labels[b * a.video + tok];
    float xv[8], cv[8], out[8], lo, sc;
    uint8_t q[8];
    Row8<DT>::load(T.input, src, xv);
    load_centroid8(T.centroids + (b * T.clusters + lab) * D + sub * 8, cv);
    base_offset_lane<G>(xv, cv, static_cast<float>((1 << T.bits) - 1), out, q, lo, sc);
    Row8<DT>::store(T.output, dst, out);
}

int grid_for_rows(int64_t rows, int G) {
    const int64_t threads = rows * G;
    return static_cast<int>(std::min<int64_t>(ceil_div(threads, 256), 1 << 20));
}

template <template <int, int> class K, typename... Args>
bool dispatch_dt_g(int dtype, int dims, int64_t rows, hipStream_t s, Args... args) {
#define PECO_LAUNCH(DT_, G_)                                                                             \
    hipLaunchKernelGGL((K<DT_, G_>::kernel), dim3(grid_for_rows(rows, G_)), dim3(256), 0, s, args...); \
    return true;
    const int G = dims / 8;
    if (dtype == kBF16) {
        if (G == 16) { PECO_LAUNCH(kBF16, 16) }
        if (G == 8) { PECO_LAUNCH(kBF16, 8) }
    } else if (dtype == kF16) {
        if (G == 16) { PECO_LAUNCH(kF16, 16) }
        if (G == 8) { PECO_LAUNCH(kF16, 8) }
    } else if (dtype == kF32) {
        if (G == 16) { PECO_LAUNCH(kF32, 16) }
        if (G == 8) { PECO_LAUNCH(kF32, 8) }
    }
#undef PECO_LAUNCH
    return false;
}

template <int DT, int G> struct EncodeK { static constexpr auto kernel = base_offset_kernel<DT, G>; };
template <int DT, int G> struct DecodeK { static constexpr auto kernel = base_offset_decode_kernel<DT, G>; };

bool valid_quant_args(int batch, int tokens, int clusters, int dims) {
    return batch >= 1 && tokens >= 1 && clusters >= 1 && (dims == 64 || dims == 128);
}

}  // namespace
}  // namespace peco

using namespace peco;

PECO_API int peco_base_offset_encode(const void* x, int dtype, const int32_t* labels, const float* centroids,
                                     int batch, int tokens, int clusters, int dims, int bits, uint8_t* codes,
                                     float* low, float* scale, void* stream) {
    if (!x || !labels || !centroids || !valid_quant_args(batch, tokens, clusters, dims) || (bits != 4 && bits != 8))
        return kInvalidValue;
    const int64_t rows = static_cast<int64_t>(batch) * tokens;
    if (!dispatch_dt_g<EncodeK>(dtype, dims, rows, static_cast<hipStream_t>(stream), x, labels, centroids, rows,
                                tokens, clusters, bits, codes, low, scale, static_cast<void*>(nullptr)))
        return kUnsupportedDtype;
    return hipGetLastError();
}

PECO_API int peco_base_offset_decode(const uint8_t* codes, const float* low, const float* scale,
                                     const int32_t* labels, const float* centroids, int batch, int tokens,
                                     int clusters, int dims, int dtype, void* out, void* stream) {
    if (!codes || !low || !scale || !labels || !centroids || !out || !valid_quant_args(batch, tokens, clusters, dims))
        return kInvalidValue;
    const int64_t rows = static_cast<int64_t>(batch) * tokens;
    if (!dispatch_dt_g<DecodeK>(dtype, dims, rows, static_cast<hipStream_t>(stream), codes, low, scale, labels,
                                centroids, rows, tokens, clusters, out))
        return kUnsupportedDtype;
    return hipGetLastError();
}

PECO_API int peco_base_offset_fake_quant(const void* x, int dtype, const int32_t* labels, const float* centroids,
                                         int batch, int tokens, int clusters, int dims, int bits, void* out,
                                         void* stream) {
    if (!x || !labels || !centroids || !out || !valid_quant_args(batch, tokens, clusters, dims) ||
        (bits != 4 && bits != 8))
        return kInvalidValue;
    const int64_t rows = static_cast<int64_t>(batch) * tokens;
    if (!dispatch_dt_g<EncodeK>(dtype, dims, rows, static_cast<hipStream_t>(stream), x, labels, centroids, rows,
                                tokens, clusters, bits, static_cast<uint8_t*>(nullptr), static_cast<float*>(nullptr),
                                static_cast<float*>(nullptr), out))
        return kUnsupportedDtype;
    return hipGetLastError();
}

// One launch packs up to three tensors (Q, K, V) of shape [batch, length, dims]:
// rows [0, video) are gathered in cluster order (optionally fake-quantized),
// rows [video, length) (text) are copied in place.
PECO_API int peco_pack_clustered(const void* const* inputs, void* const* outputs, const int32_t* const* indices,
                                 const int32_t* const* labels, const float* const* centroids, const int* clusters,
                                 const int* bits, int num_tensors, int batch, int length, int video, int dims,
                                 int dtype, void* stream) {
    if (num_tensors < 1 || num_tensors > 3 || batch < 1 || length < 1 || video < 0 || video > length ||
        (dims != 64 && dims != 128))
        return kInvalidValue;
    PackArgs a{};
    a.num = num_tensors;
    a.batch = batch;
    a.length = length;
    a.video = video;
    for (int i = 0; i < num_tensors; ++i) {
        if (!inputs[i] || !outputs[i] || (video > 0 && !indices[i])) return kInvalidValue;
        if (bits[i] != 0 && bits[i] != 4 && bits[i] != 8) return kInvalidValue;
        if (bits[i] != 0 && (!labels[i] || !centroids[i] || clusters[i] < 1)) return kInvalidValue;
        a.t[i] = PackTensor{inputs[i], outputs[i], indices[i], labels[i], centroids[i], clusters[i], bits[i]};
    }
    if (batch > 65535) return kUnsupportedShape;
    const int G = dims / 8;
    const dim3 grid(static_cast<unsigned>(ceil_div(length, 256 / G)), static_cast<unsigned>(batch),
                    static_cast<unsigned>(num_tensors));
    const hipStream_t s = static_cast<hipStream_t>(stream);
#define PECO_PACK(DT_)                                                                   \
    do {                                                                                 \
        if (G == 16) hipLaunchKernelGGL((pack_kernel<DT_, 16>), grid, dim3(256), 0, s, a); \
        else hipLaunchKernelGGL((pack_kernel<DT_, 8>), grid, dim3(256), 0, s, a);          \
    } while (0)
    if (dtype == kBF16) PECO_PACK(kBF16);
    else if (dtype == kF16) PECO_PACK(kF16);
    else if (dtype == kF32) PECO_PACK(kF32);
    else return kUnsupportedDtype;
#undef PECO_PACK
    return hipGetLastError();
}
