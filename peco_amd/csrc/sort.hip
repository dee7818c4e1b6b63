// Stage 3: stable cluster sort of token labels, and row gather/scatter by permutation.
//
// The permutation is the stable argsort of labels per batch entry
// (peco/clustering.py:105, torch.argsort(..., stable=True)), computed as a counting sort:
//   1. sort_hist:  per 256-token tile, a label histogram (LDS atomics; counts only).
//   2. sort_scan_groups + sort_scan: reduce-then-scan of the tile counts -> per (tile,
//                  cluster) run its exclusive prefix within a group of kScanTiles tiles,
//                  per (group, cluster) its absolute start, counts and offsets.
//   3. sort_place: per tile, one wavefront ranks 64 tokens per step. Lanes holding the
//                  same label are found with one ballot per label bit (no serial match
//                  loop); the rank among equal labels is a popcount of lower lanes, so
//                  original order is kept within each cluster.
// Reordering copies rows of dims*item_size bytes with 16-byte lanes where alignment
// allows (peco/kernels/kmeans.cu:92-107 is the reference's 2/4-byte-per-thread copy).
#include "sort.hpp"

#include <algorithm>

namespace peco {
namespace {

__device__ __forceinline__ int find_problem_by_block(const SortArgs& a, int block) {
    int p = 0;
    while (p + 1 < a.num && block >= a.p[p + 1].block_begin) ++p;
    return p;
}

__device__ __forceinline__ int find_problem_by_batch(const SortArgs& a, int b) {
    int p = 0;
    while (p + 1 < a.num && b >= a.p[p + 1].batch_begin) ++p;
    return p;
}

__device__ __forceinline__ int find_problem_by_scan_group(const SortArgs& a, int g) {
    int p = 0;
    while (p + 1 < a.num && g >= a.p[p + 1].scan_group_begin) ++p;
    return p;
}

// [batch, scan groups, clusters] area behind the tile histograms.
__device__ __forceinline__ int32_t* scan_group_area(const SortProblem& P) {
    return P.tile_hist + static_cast<int64_t>(P.batch) * P.tiles * P.clusters;
}

__global__ __launch_bounds__(256) void sort_hist_kernel(SortArgs args) {
    extern __shared__ int hist[];
    const int pi = find_problem_by_block(args, blockIdx.x);
    const SortProblem& P = args.p[pi];
    const int local = blockIdx.x - P.block_begin;
    const int b = local / P.tiles;
    const int tile = local % P.tiles;
    for (int k = threadIdx.x; k < P.clusters; k += blockDim.x) hist[k] = 0;
    __syncthreads();
    const int32_t* lab = P.labels + static_cast<int64_t>(b) * P.tokens;
    const int begin = tile * kSortTile;
    const int end = min(P.tokens, begin + kSortTile);
    for (int t = begin + threadIdx.x; t < end; t += blockDim.x) {
        const int L = lab[t];
        if (static_cast<unsigned>(L) < static_cast<unsigned>(P.clusters)) atomicAdd(&hist[L], 1);
    }
    __syncthreads();
    int32_t* out = P.tile_hist + (static_cast<int64_t>(b) * P.tiles + tile) * P.clusters;
    for (int k = threadIdx.x; k < P.clusters; k += blockDim.x) out[k] = hist[k];
}

// Phase 1 of the scan: per group of kScanTiles tiles, each (tile, cluster) count becomes its
// exclusive prefix within the group (in place) and the group's cluster totals go to the
// group area. A cluster's whole group column is loaded before any of it is written.
__global__ __launch_bounds__(256) void sort_scan_groups_kernel(SortArgs args) {
    const int pi = find_problem_by_scan_group(args, blockIdx.x);
    const SortProblem& P = args.p[pi];
    const int local = blockIdx.x - P.scan_group_begin;
    const int b = local / P.scan_groups;
    const int g = local % P.scan_groups;
    const int K = P.clusters;
    const int t0 = g * kScanTiles;
    const int nt = min(kScanTiles, P.tiles - t0);
    int32_t* th = P.tile_hist + (static_cast<int64_t>(b) * P.tiles + t0) * K;
    int32_t* gt = scan_group_area(P) + (static_cast<int64_t>(b) * P.scan_groups + g) * K;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        int c[kScanTiles];
#pragma unroll
        for (int u = 0; u < kScanTiles; ++u) {
            // Clamped unconditional loads (masked after) stay in flight together.
            const int v = th[static_cast<int64_t>(min(u, nt - 1)) * K + k];
            c[u] = u < nt ? v : 0;
        }
        int run = 0;
#pragma unroll
        for (int u = 0; u < kScanTiles; ++u) {
            if (u < nt) th[static_cast<int64_t>(u) * K + k] = run;
            run += c[u];
        }
        gt[k] = run;
    }
}

// Phase 2, per batch entry: cluster totals from the group totals, their exclusive scan
// (offsets, counts), and each (group, cluster) total replaced by the group's absolute start.
__global__ __launch_bounds__(256) void sort_scan_kernel(SortArgs args) {
    extern __shared__ int cnt[];
    __shared__ int tmp[4];
    const int pi = find_problem_by_batch(args, blockIdx.x);
    const SortProblem& P = args.p[pi];
    const int b = blockIdx.x - P.batch_begin;
    const int K = P.clusters;
    const int groups = P.scan_groups;
    int32_t* gt = scan_group_area(P) + static_cast<int64_t>(b) * groups * K;
    constexpr int kBatch = 8;  // group totals in flight per thread
    // Pass 1 (loads only): total count of each cluster.
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        int run = 0;
        for (int g0 = 0; g0 < groups; g0 += kBatch) {
            int c[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int v = gt[static_cast<int64_t>(min(g0 + u, groups - 1)) * K + k];
                c[u] = g0 + u < groups ? v : 0;
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) run += c[u];
        }
        cnt[k] = run;
    }
    __syncthreads();
    // Exclusive scan over clusters: each thread owns a contiguous chunk.
    const int per = static_cast<int>(ceil_div(K, blockDim.x));
    const int k0 = threadIdx.x * per;
    const int k1 = min(K, k0 + per);
    int local = 0;
    for (int k = k0; k < k1; ++k) local += cnt[k];
    int total = 0;
    int run = block_exclusive_scan256(local, tmp, &total);
    int32_t* off = P.offsets + static_cast<int64_t>(b) * (K + 1);
    int32_t* counts = P.counts ? P.counts + static_cast<int64_t>(b) * K : nullptr;
    for (int k = k0; k < k1; ++k) {
        const int c = cnt[k];
        off[k] = run;
        if (counts) counts[k] = c;
        cnt[k] = run;  // becomes the cluster's first sorted position
        run += c;
    }
    if (threadIdx.x == 0) off[K] = total;
    __syncthreads();
    // Pass 2: each (group, cluster) total becomes the absolute start of that group's runs. A
    // batch of totals is read before any of it is overwritten.
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        int pos = cnt[k];
        for (int g0 = 0; g0 < groups; g0 += kBatch) {
            int c[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int v = gt[static_cast<int64_t>(min(g0 + u, groups - 1)) * K + k];
                c[u] = g0 + u < groups ? v : 0;
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                if (g0 + u < groups) gt[static_cast<int64_t>(g0 + u) * K + k] = pos;
                pos += c[u];
            }
        }
    }
}

__global__ __launch_bounds__(64) void sort_place_kernel(SortArgs args) {
    extern __shared__ int base[];
    const int pi = find_problem_by_block(args, blockIdx.x);
    const SortProblem& P = args.p[pi];
    const int local = blockIdx.x - P.block_begin;
    const int b = local / P.tiles;
    const int tile = local % P.tiles;
    const int K = P.clusters;
    const int lane = threadIdx.x;
    const int32_t* th = P.tile_hist + (static_cast<int64_t>(b) * P.tiles + tile) * K;
    int32_t* th_mut = P.tile_hist + (static_cast<int64_t>(b) * P.tiles + tile) * K;
    const int32_t* gs = scan_group_area(P) + (static_cast<int64_t>(b) * P.scan_groups + tile / kScanTiles) * K;
    // Run starts of this tile: the in-group prefix plus the group's start (four of each in
    // flight per lane before any store).
    for (int k0 = 0; k0 < K; k0 += 4 * kWave) {
        int v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int e = min(k0 + u * kWave + lane, K - 1);
            const int x = th[e] + gs[e];
            v[u] = k0 + u * kWave + lane < K ? x : 0;
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int k = k0 + u * kWave + lane;
            if (k < K) {
                base[k] = v[u];
                if (args.zero_hist) th_mut[k] = 0;
            }
        }
    }
    __syncthreads();
    const int bits = K > 1 ? 32 - __builtin_clz(static_cast<unsigned>(K - 1)) : 0;
    const int32_t* lab = P.labels + static_cast<int64_t>(b) * P.tokens;
    int32_t* idx = P.indices + static_cast<int64_t>(b) * P.tokens;
    int32_t* ranks = P.ranks ? P.ranks + static_cast<int64_t>(b) * P.tokens : nullptr;
    const int begin = tile * kSortTile;
    const int end = min(P.tokens, begin + kSortTile);
    // All labels of the tile are loaded before ranking starts (16 independent loads per lane).
    constexpr int kSteps = kSortTile / kWave;
    int labs[kSteps];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int t = begin + st * kWave + lane;
        const int raw = lab[min(t, end - 1)];  // clamped, unconditional: all loads in flight
        labs[st] = t < end ? raw : -1;
    }
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int t = begin + st * kWave + lane;
        const int pos = place_step(labs[st], t < end, K, bits, base);
        if (pos >= 0) {
            idx[pos] = t;
            if (ranks) ranks[t] = pos;
        }
    }
}

__device__ __forceinline__ int find_problem_by_group(const SortArgs& a, int group) {
    int p = 0;
    while (p + 1 < a.num && group >= a.p[p + 1].group_begin) ++p;
    return p;
}

// Scan and place in one launch for small batch entries (sort_fusable). Workgroup (b, g)
// ranks tiles kFusedTiles*g .. +3, one per wavefront. Every workgroup of entry b loads the
// whole tile histogram of b (at most kFusedMaxTiles rows, all in flight per cluster) and
// computes the cluster totals, their exclusive scan and its own tiles' run starts, so the
// result equals sort_scan followed by sort_place. The histogram is left unchanged (other
// workgroups still read it); next_hist, when given, is cleared for the next producer.
__global__ __launch_bounds__(256) void sort_fused_kernel(SortArgs args) {
    extern __shared__ int lds[];  // [kFusedTiles][K] run starts, then [K] cluster offsets
    __shared__ int tmp[4];
    const int pi = find_problem_by_group(args, blockIdx.x);
    const SortProblem& P = args.p[pi];
    const int groups = static_cast<int>(ceil_div(P.tiles, kFusedTiles));
    const int local = blockIdx.x - P.group_begin;
    const int b = local / groups;
    const int g = local % groups;
    const int K = P.clusters;
    const int tiles = P.tiles;
    const int wave = threadIdx.x / kWave;
    const int lane = lane_id();
    const int tile = g * kFusedTiles + wave;
    const int begin = tile * kSortTile;
    const int end = min(P.tokens, begin + kSortTile);
    const int32_t* lab = P.labels + static_cast<int64_t>(b) * P.tokens;
    // This wavefront's labels first, so their loads overlap the histogram loads below.
    constexpr int kSteps = kSortTile / kWave;
    int labs[kSteps];
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int t = begin + st * kWave + lane;
        const int raw = lab[min(t, P.tokens - 1)];  // clamped, unconditional: all loads in flight
        labs[st] = t < end ? raw : -1;
    }
    int* starts = lds;
    int* offs = lds + kFusedTiles * K;
    const int32_t* th = P.tile_hist + static_cast<int64_t>(b) * tiles * K;
    const int first = g * kFusedTiles;
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        int c[kFusedMaxTiles];
#pragma unroll
        for (int t = 0; t < kFusedMaxTiles; ++t) {
            const int v = th[static_cast<int64_t>(min(t, tiles - 1)) * K + k];
            c[t] = t < tiles ? v : 0;
        }
        int run = 0;  // tokens of cluster k in tiles before t
#pragma unroll
        for (int t = 0; t < kFusedMaxTiles; ++t) {
            const int w = t - first;
            if (w >= 0 && w < kFusedTiles) starts[w * K + k] = run;
            run += c[t];
        }
        offs[k] = run;  // the cluster's total for now
    }
    __syncthreads();
    // Exclusive scan of the totals over clusters (each thread owns a contiguous chunk).
    const int per = static_cast<int>(ceil_div(K, blockDim.x));
    const int k0 = min(K, static_cast<int>(threadIdx.x) * per);
    const int k1 = min(K, k0 + per);
    int chunk = 0;
    for (int k = k0; k < k1; ++k) chunk += offs[k];
    int total = 0;
    int run = block_exclusive_scan256(chunk, tmp, &total);
    int32_t* off = P.offsets + static_cast<int64_t>(b) * (K + 1);
    int32_t* counts = P.counts ? P.counts + static_cast<int64_t>(b) * K : nullptr;
    for (int k = k0; k < k1; ++k) {
        const int c = offs[k];
        if (g == 0) {
            off[k] = run;
            if (counts) counts[k] = c;
        }
        offs[k] = run;
        run += c;
    }
    if (g == 0 && threadIdx.x == 0) off[K] = total;
    __syncthreads();
    if (P.next_hist) {
        // Clear this workgroup's tiles in the histogram the next producer accumulates into.
        const int rows = min(kFusedTiles, tiles - first);
        int32_t* nh = P.next_hist + (static_cast<int64_t>(b) * tiles + first) * K;
        for (int i = threadIdx.x; i < rows * K; i += blockDim.x) nh[i] = 0;
    }
    if (tile >= tiles) return;
    // Rank this wavefront's tile as sort_place does, from its own run starts.
    int* base = starts + wave * K;
    for (int k = lane; k < K; k += kWave) base[k] += offs[k];
    __builtin_amdgcn_wave_barrier();
    const int bits = K > 1 ? 32 - __builtin_clz(static_cast<unsigned>(K - 1)) : 0;
    int32_t* idx = P.indices + static_cast<int64_t>(b) * P.tokens;
    int32_t* ranks = P.ranks ? P.ranks + static_cast<int64_t>(b) * P.tokens : nullptr;
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
        const int t = begin + st * kWave + lane;
        const int pos = place_step(labs[st], t < end, K, bits, base);
        if (pos >= 0) {
            idx[pos] = t;
            if (ranks) ranks[t] = pos;
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void reorder_rows_kernel(const T* __restrict__ in, const int32_t* __restrict__ idx,
                                                           T* __restrict__ out, int tokens, int chunks,
                                                           int64_t total, int inverse) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = i / chunks;
        const int c = static_cast<int>(i - row * chunks);
        const int64_t head = row / tokens;
        const int tok = idx[row];
        if (static_cast<unsigned>(tok) >= static_cast<unsigned>(tokens)) continue;
        const int64_t mapped = (head * tokens + tok) * chunks + c;
        if (inverse) out[mapped] = in[i];
        else out[i] = in[mapped];
    }
}

}  // namespace

void sort_args_finalize(SortArgs& a) {
    int blocks = 0, batches = 0, groups = 0, scan_groups = 0;
    for (int i = 0; i < a.num; ++i) {
        a.p[i].tiles = sort_tiles(a.p[i].tokens);
        a.p[i].scan_groups = sort_scan_groups(a.p[i].tokens);
        a.p[i].block_begin = blocks;
        a.p[i].batch_begin = batches;
        a.p[i].group_begin = groups;
        a.p[i].scan_group_begin = scan_groups;
        blocks += a.p[i].batch * a.p[i].tiles;
        batches += a.p[i].batch;
        groups += a.p[i].batch * static_cast<int>(ceil_div(a.p[i].tiles, kFusedTiles));
        scan_groups += a.p[i].batch * a.p[i].scan_groups;
    }
    a.total_blocks = blocks;
    a.total_batches = batches;
    a.total_groups = groups;
    a.total_scan_groups = scan_groups;
}

hipError_t launch_cluster_sort(const SortArgs& args, hipStream_t stream, bool with_hist) {
    int kmax = 1;
    for (int i = 0; i < args.num; ++i) kmax = max(kmax, args.p[i].clusters);
    const size_t lds = sizeof(int) * static_cast<size_t>(kmax);
    if (args.fused && !with_hist) {
        for (int i = 0; i < args.num; ++i)
            if (!sort_fusable(args.p[i].tokens, args.p[i].clusters)) return hipErrorInvalidValue;
        hipLaunchKernelGGL(sort_fused_kernel, dim3(args.total_groups), dim3(256), (kFusedTiles + 1) * lds, stream,
                           args);
        return hipGetLastError();
    }
    if (with_hist) hipLaunchKernelGGL(sort_hist_kernel, dim3(args.total_blocks), dim3(256), lds, stream, args);
    hipLaunchKernelGGL(sort_scan_groups_kernel, dim3(args.total_scan_groups), dim3(256), 0, stream, args);
    hipLaunchKernelGGL(sort_scan_kernel, dim3(args.total_batches), dim3(256), lds, stream, args);
    hipLaunchKernelGGL(sort_place_kernel, dim3(args.total_blocks), dim3(64), lds, stream, args);
    return hipGetLastError();
}

}  // namespace peco

using namespace peco;

PECO_API size_t peco_cluster_sort_workspace_size(int batch, int tokens, int clusters) {
    if (batch < 1 || tokens < 1 || clusters < 1) return 0;
    return sizeof(int32_t) * (sort_workspace_ints(batch, tokens, clusters) + static_cast<size_t>(batch) * (clusters + 1));
}

PECO_API int peco_cluster_sort(const int32_t* labels, int batch, int tokens, int clusters, int32_t* indices,
                               int32_t* ranks, int32_t* counts, int32_t* offsets, void* workspace,
                               size_t workspace_bytes, void* stream) {
    if (!labels || !indices || batch < 1 || tokens < 1 || clusters < 1 || clusters > kMaxSortClusters)
        return kInvalidValue;
    if (workspace_bytes < peco_cluster_sort_workspace_size(batch, tokens, clusters) || !workspace)
        return kWorkspaceTooSmall;
    SortArgs a{};
    a.num = 1;
    SortProblem& p = a.p[0];
    p.labels = labels;
    p.indices = indices;
    p.ranks = ranks;
    p.counts = counts;
    p.tile_hist = static_cast<int32_t*>(workspace);
    p.offsets = offsets ? offsets : p.tile_hist + sort_workspace_ints(batch, tokens, clusters);
    p.batch = batch;
    p.tokens = tokens;
    p.clusters = clusters;
    sort_args_finalize(a);
    return launch_cluster_sort(a, static_cast<hipStream_t>(stream), true);
}

PECO_API int peco_reorder_token_features(const void* input, const int32_t* indices, void* output, int batch_heads,
                                         int tokens, int dims, int item_size, int inverse, void* stream) {
    if (!input || !indices || !output || batch_heads < 1 || tokens < 0 || dims < 1 ||
        (item_size != 2 && item_size != 4))
        return kInvalidValue;
    if (tokens == 0) return kOk;
    const int64_t row_bytes = static_cast<int64_t>(dims) * item_size;
    const uintptr_t align = reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(output);
    const int64_t rows = static_cast<int64_t>(batch_heads) * tokens;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    auto launch = [&](auto tag, int width) {
        using T = decltype(tag);
        const int chunks = static_cast<int>(row_bytes / width);
        const int64_t total = rows * chunks;
        const int blocks = static_cast<int>(std::min<int64_t>(ceil_div(total, 256), 1 << 20));
        hipLaunchKernelGGL(reorder_rows_kernel<T>, dim3(blocks), dim3(256), 0, s, static_cast<const T*>(input),
                           indices, static_cast<T*>(output), tokens, chunks, total, inverse);
    };
    if (row_bytes % 16 == 0 && align % 16 == 0) launch(u32x4{}, 16);
    else if (row_bytes % 4 == 0 && align % 4 == 0) launch(uint32_t{}, 4);
    else launch(uint16_t{}, 2);
    return hipGetLastError();
}
