// Stable counting sort of cluster labels (host-side launch interface).
#pragma once

#include "common.hpp"

namespace peco {

// Tokens per sort tile: one tile is ranked by a single wavefront, 64 tokens per step. The
// k-means assign kernel adds its labels to these histograms with atomics.
constexpr int kSortTile = 256;
constexpr int kMaxSortClusters = 16384;

struct SortProblem {
    const int32_t* labels;  // [batch, tokens], values in [0, clusters)
    int32_t* indices;       // [batch, tokens]: original token at each sorted position
    int32_t* ranks;         // nullable [batch, tokens]: sorted position of each token
    int32_t* counts;        // nullable [batch, clusters]
    int32_t* offsets;       // [batch, clusters + 1]: first sorted position of each cluster
    int32_t* tile_hist;     // workspace [batch, tiles, clusters]
    int32_t* next_hist;     // nullable, fused sort only: histograms cleared for the next producer
    int batch, tokens, clusters, tiles;
    int block_begin;        // first linear (batch, tile) block of this problem
    int batch_begin;        // first linear batch entry of this problem (scan grid)
    int group_begin;        // first linear (batch, tile group) workgroup (fused grid)
    int scan_groups;        // groups of kScanTiles tiles per batch entry
    int scan_group_begin;   // first linear (batch, scan group) workgroup (group scan grid)
};

constexpr int kMaxSortProblems = 2;

struct SortArgs {
    SortProblem p[kMaxSortProblems];
    int num;
    int total_blocks;   // sum of batch * tiles
    int total_batches;  // sum of batch
    int zero_hist;      // sort_place clears each consumed tile histogram (for accumulating producers)
    int fused;          // one sort_fused launch instead of scan + place (sort_fusable problems only)
    int total_groups;   // sum of batch * ceil(tiles / kFusedTiles)
    int total_scan_groups;  // sum of batch * scan_groups
};

// Fused sort: a workgroup ranks kFusedTiles consecutive tiles (one per wavefront) and derives
// the cluster offsets of its batch entry from the tile histograms itself. Each workgroup reads
// the whole [tiles, clusters] histogram of its entry, so this is for small entries only.
constexpr int kFusedTiles = 4;
constexpr int kFusedMaxTiles = 32;
constexpr int kFusedMaxClusters = 1024;

inline bool sort_fusable(int tokens, int clusters) {
    return ceil_div(tokens, kSortTile) <= kFusedMaxTiles && clusters <= kFusedMaxClusters;
}

inline int sort_tiles(int tokens) { return static_cast<int>(ceil_div(tokens, kSortTile)); }

// The unfused scan is a reduce-then-scan over groups of kScanTiles tiles: per group, the
// (tile, cluster) counts become exclusive prefixes within the group and the group totals go
// to a second area; per batch entry, the group totals are scanned into cluster offsets and
// group starts; the place kernel adds its group's start to its in-group prefixes.
constexpr int kScanTiles = 32;

inline int sort_scan_groups(int tokens) { return static_cast<int>(ceil_div(sort_tiles(tokens), kScanTiles)); }

// [batch, tiles, clusters] tile histograms followed by [batch, scan groups, clusters] group
// totals.
inline size_t sort_workspace_ints(int batch, int tokens, int clusters) {
    return static_cast<size_t>(batch) * (sort_tiles(tokens) + sort_scan_groups(tokens)) * clusters;
}

__device__ __forceinline__ int wave_inclusive_scan(int v) {
    const int lane = __lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const int y = __shfl_up(v, d, kWave);
        if (lane >= d) v += y;
    }
    return v;
}

// Exclusive scan across a 256-thread block; returns the exclusive prefix and the total.
__device__ __forceinline__ int block_exclusive_scan256(int v, int* tmp, int* total) {
    const int lane = __lane_id();
    const int wave = threadIdx.x / kWave;
    const int inc = wave_inclusive_scan(v);
    if (lane == kWave - 1) tmp[wave] = inc;
    __syncthreads();
    int base = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int t = tmp[w];
        base += w < wave ? t : 0;
        sum += t;
    }
    __syncthreads();
    *total = sum;
    return base + inc - v;
}

// One step of a stable counting-sort placement by one wavefront: each lane holds one token
// (label raw, in_tile false past the entry's end; a label outside [0, K) places nothing).
// Lanes with the same label are found with one ballot per label bit (bits = ceil(log2 K)),
// the rank among them is a popcount of the lower lanes (token order kept), and base[L], this
// wavefront's LDS row of next positions, advances by their count. Returns the token's sorted
// position, or -1. The wavefront's LDS reads and writes execute in program order, so the
// read of base[L] precedes the update without a workgroup barrier (whose memory fence would
// also wait for the caller's scattered global stores every step).
__device__ __forceinline__ int place_step(int raw, bool in_tile, int K, int bits, int* base) {
    const int lane = __lane_id();
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (kWave - lane));
    const bool active = in_tile && static_cast<unsigned>(raw) < static_cast<unsigned>(K);
    const int L = active ? raw : 0;
    uint64_t eq = __ballot(active);
    for (int bit = 0; bit < bits; ++bit) {
        const bool on = active && ((L >> bit) & 1);
        const uint64_t m = __ballot(on);
        eq &= ((L >> bit) & 1) ? m : ~m;
    }
    const int rank = __popcll(eq & below);
    const int count = __popcll(eq);
    const bool last = active && ((eq >> lane) == 1ull);
    int pos = -1;
    if (active) pos = base[L] + rank;
    __builtin_amdgcn_wave_barrier();
    if (last) base[L] += count;
    __builtin_amdgcn_wave_barrier();
    return pos;
}

// Fills block_begin/batch_begin/totals for problems[0..num).
void sort_args_finalize(SortArgs& args);

// with_hist=false: tile_hist already holds the per-tile label counts (e.g. accumulated
// by the k-means assign kernel), so only the scan and place kernels run (or, with
// args.fused, the single fused kernel, which leaves tile_hist unchanged and clears
// next_hist instead).
hipError_t launch_cluster_sort(const SortArgs& args, hipStream_t stream, bool with_hist);

}  // namespace peco
